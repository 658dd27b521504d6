// repack.hip -- the aligned, size-neutral repacked PQ2_0 row layout (gfx950).
//
// Layout (reference src/pq2_0_repack.h:46-57): a row of nb blocks keeps its
// 34*nb bytes; d[nb] fp16 first, then unit u = plane*nb + block (8 code bytes,
// chunk `plane` of `block`) at byte 2*nb + 8u.  nb % 8 == 0 keeps the code
// region 16-byte aligned.
//   * repack_kernel      -- the one-time byte permutation
//                           (replaces gemv_repack_p40.cu:165-207);
//   * gemv_repack_kernel -- y = W_repacked . x for fp32 x, quantising x once
//                           per workgroup into LDS with the host rounding
//                           (replaces gemv_repack_p40.cu:57-162,209-220).
// In the repacked layout a lane's 8-byte unit is naturally aligned, so the
// GEMV needs no LDS staging of weights: 64 lanes read 512 contiguous bytes
// with one dwordx2 load, and the block scales of consecutive units are
// consecutive fp16 values.
#include "pq2_device.h"
#include "host_state.h"
#include "../../include/bonsai_p40.h"

using namespace pq2;

namespace {

constexpr int RP_WAVES = 4;
constexpr int RP_THREADS = 64 * RP_WAVES;

template <bool DST_ALIGNED8>
__global__ void __launch_bounds__(256)
repack_kernel(const uint8_t * __restrict__ src, uint8_t * __restrict__ dst, int64_t n_out, int nb) {
    const int64_t nunits = 4 * (int64_t)nb;
    const int64_t total = n_out * nunits;
    const size_t stride = (size_t)PQ2_BYTES * nb;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t row = i / nunits;
        const int u = (int)(i - row * nunits);
        const int p = u / nb, b = u - p * nb;
        const uint8_t * s = src + row * stride + (size_t)PQ2_BYTES * b;
        uint8_t * d = dst + row * stride;
        const uint16_t * sp = reinterpret_cast<const uint16_t *>(s + 2 + 8 * p);
        const uint32_t lo = (uint32_t)sp[0] | ((uint32_t)sp[1] << 16);
        const uint32_t hi = (uint32_t)sp[2] | ((uint32_t)sp[3] << 16);
        uint8_t * du = d + 2 * (size_t)nb + 8 * (size_t)u;
        if (DST_ALIGNED8) {
            *reinterpret_cast<uint2 *>(du) = make_uint2(lo, hi);
        } else {
            uint16_t * dp = reinterpret_cast<uint16_t *>(du);
            dp[0] = (uint16_t)lo; dp[1] = (uint16_t)(lo >> 16);
            dp[2] = (uint16_t)hi; dp[3] = (uint16_t)(hi >> 16);
        }
        if (p == 0) *reinterpret_cast<uint16_t *>(d + 2 * b) = *reinterpret_cast<const uint16_t *>(s);
    }
}

// Host-rounding Q8_1 quantisation of one chunk held by a lane pair (16
// elements per lane) into the LDS activation planes used by the GEMV:
// act_q[8c + k] = permuted word k, act_sc[c] = {decoded fp16 d, -s}.
__device__ __forceinline__ void quant_pair_lds(const float (&v)[16], uint32_t * act_q, int2 * act_sc,
                                               int c, int half) {
#pragma clang fp contract(off)
    float amax = 0.0f;
#pragma unroll
    for (int r = 0; r < 16; ++r) amax = fmaxf(amax, fabsf(v[r]));
    amax = fmaxf(amax, dpp_mov<DPP_QUAD_XOR1>(amax));
    const float d = amax / 127.0f;
    const float id = d > 0.0f ? 1.0f / d : 0.0f;
    int q[16];
    int sum = 0;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const float prod = v[r] * id;
        int t = (int)__builtin_roundf(prod);
        t = t < -127 ? -127 : (t > 127 ? 127 : t);
        q[r] = t;
        sum += t;
    }
    sum += dpp_mov_i<DPP_QUAD_XOR1>(sum);
    if (half == 0) act_sc[c] = make_int2(__float_as_int(f16_bits_to_f32(f32_to_f16_away(d))), -sum);
#pragma unroll
    for (int k = 0; k < 4; ++k)
        act_q[8 * c + 4 * half + k] = (uint32_t)(q[k] & 0xff) | ((uint32_t)(q[4 + k] & 0xff) << 8) |
                                      ((uint32_t)(q[8 + k] & 0xff) << 16) |
                                      ((uint32_t)(q[12 + k] & 0xff) << 24);
}

// Persistent grid: every workgroup quantises x into LDS once, then its waves
// take rows grid-stride.  Lane l handles units l, l+64, ... of the row.
__global__ void __launch_bounds__(RP_THREADS)
gemv_repack_kernel(const uint8_t * __restrict__ W, const float * __restrict__ x,
                   float * __restrict__ y, int n_out, int nb) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int nchunk = 4 * nb;
    uint32_t * act_q = reinterpret_cast<uint32_t *>(smem);
    int2 * act_sc = reinterpret_cast<int2 *>(smem + (size_t)nchunk * 32);

    for (int c0 = 0; c0 < nchunk; c0 += RP_THREADS / 2) {
        const int c = c0 + (threadIdx.x >> 1);
        const int half = threadIdx.x & 1;
        if (c < nchunk) {      // both lanes of a pair agree
            float v[16];
            const float * xp = x + (size_t)c * QK8 + 16 * half;
#pragma unroll
            for (int r = 0; r < 16; ++r) v[r] = xp[r];
            quant_pair_lds(v, act_q, act_sc, c, half);
        }
    }
    __syncthreads();

    const int lane = threadIdx.x & 63;
    const int nunits = 4 * nb;
    const size_t stride = (size_t)PQ2_BYTES * nb;
    const int nwaves = gridDim.x * RP_WAVES;
    for (int row = blockIdx.x * RP_WAVES + (threadIdx.x >> 6); row < n_out; row += nwaves) {
        const uint8_t * wr = W + (size_t)row * stride;
        const uint2 * units = reinterpret_cast<const uint2 *>(wr + 2 * (size_t)nb);
        const uint16_t * dws = reinterpret_cast<const uint16_t *>(wr);
        float acc = 0.0f;
        for (int u = lane; u < nunits; u += 64) {
            const uint2 w = units[u];
            const int p = u / nb, b = u - p * nb;
            const int c = 4 * b + p;
            const int4 a0 = *reinterpret_cast<const int4 *>(act_q + 8 * c);
            const int4 a1 = *reinterpret_cast<const int4 *>(act_q + 8 * c + 4);
            const int2 sc = act_sc[c];
            const int a[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
            const int s = chunk_dot_i32(w.x, w.y, a, sc.y);
            acc += f16_bits_to_f32(dws[b]) * (__int_as_float(sc.x) * (float)s);
        }
        acc = wave_sum_to_lane63(acc);
        if (lane == 63) y[row] = acc;
    }
}

int lds_limit() { return pq2host::device_info().max_lds; }

}  // namespace

namespace pq2 {
// gemv.hip: the streaming kernel on the repacked layout; -1 if not applicable
int gemv_repack_streaming(const void * W, const float * x, float * y, int64_t n_out, int64_t n_in,
                          bonsai_stream stream);
}

extern "C" {

int bonsai_p40_repack(const void * src, void * dst, int64_t n_out, int64_t n_in, bonsai_stream stream) {
    if (n_in % QK_PQ2 != 0 || n_out <= 0 || n_in <= 0) return 1;
    const int64_t nb = n_in / QK_PQ2;
    if (nb % 8 != 0 || nb > (1 << 24)) return 1;
    if ((((uintptr_t)src | (uintptr_t)dst) & 1u) != 0 || pq2host::any_null(src, dst)) return 1;
    const int64_t total = n_out * 4 * nb;
    int64_t blocks = (total + 255) / 256;
    if (blocks > 65535 * 8) blocks = 65535 * 8;
    const bool al8 = ((uintptr_t)dst & 7u) == 0;
    if (al8)
        hipLaunchKernelGGL(repack_kernel<true>, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream,
                           (const uint8_t *)src, (uint8_t *)dst, n_out, (int)nb);
    else
        hipLaunchKernelGGL(repack_kernel<false>, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream,
                           (const uint8_t *)src, (uint8_t *)dst, n_out, (int)nb);
    return (int)hipGetLastError();
}

int bonsai_p40_gemv_repack(const void * W, const float * x, float * y, int64_t n_out, int64_t n_in,
                           bonsai_stream stream) {
    if (n_in % QK_PQ2 != 0 || n_out <= 0 || n_in <= 0) return 1;
    const int64_t nb = n_in / QK_PQ2;
    if (nb % 8 != 0 || n_out > 0x7fffffff) return 1;
    if (((uintptr_t)W & 7u) != 0) return 1;            // 8-byte units must be aligned
    if (pq2host::any_null(W, x, y)) return 1;
    const int rc = pq2::gemv_repack_streaming(W, x, y, n_out, n_in, stream);
    if (rc >= 0) return rc;
    const size_t lds = (size_t)nb * 4 * 40;
    if (lds > (size_t)lds_limit()) return 1;
    static pq2host::PerDeviceOnce attr;
    pq2host::once_per_device(attr, [] {
        pq2host::set_max_dynamic_lds(reinterpret_cast<const void *>(gemv_repack_kernel), lds_limit());
    });
    int64_t blocks = (n_out + RP_WAVES - 1) / RP_WAVES;
    if (blocks > 256 * 4) blocks = 256 * 4;
    hipLaunchKernelGGL(gemv_repack_kernel, dim3((unsigned)blocks), dim3(RP_THREADS), lds,
                       (hipStream_t)stream, (const uint8_t *)W, x, y, (int)n_out, (int)nb);
    return (int)hipGetLastError();
}

}  // extern "C"
