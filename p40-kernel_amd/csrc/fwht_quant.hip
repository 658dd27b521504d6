// fwht_quant.hip -- activation pre-pass kernels for gfx950:
//   * FWHT-1024 (normalised Sylvester-Hadamard, optional +-1 signs),
//   * permuted Q8_1 quantisation with the reference host rounding,
//   * both fused into one LDS-resident butterfly kernel, optionally preceded
//     by SwiGLU (the FFN glue) and writing the GEMV (token-major) or the GEMM
//     (chunk-major) activation layout.
//
// Reference semantics: src/fwht.h:20-42 (transform, stage order, signs of
// length n), src/pq2_0.h:99-126 (quantiser), src/ops.h:27-31 (SwiGLU); device
// counterparts replaced: src/kernels/elementwise_p40.cu:17-41,75-80 and
// src/kernels/gemv_p40.cu:168-208.
//
// One wave (64 lanes) owns one 1024-element block; the transform and the
// quantiser are the register-resident device functions of fwht_device.h
// (lane l holds the 16 consecutive elements of row fwht_row(l)), so the
// rotated values are bit-identical to fwht_blocks() and the Q8_1 bytes to the
// host quantiser.
//
// No floating-point contraction anywhere in this file: the host computes the
// products x*id and x*sign as separately rounded fp32 multiplies.
#pragma clang fp contract(off)

#include "fwht_device.h"
#include "../../include/bonsai_p40.h"

using namespace pq2;

namespace {

enum : int {
    M_ROT = 1,        // apply the FWHT
    M_SIGNS = 2,      // multiply by signs first
    M_SWIGLU = 4,     // input = silu(gate) * up
    M_OUT_F32 = 8,    // write the rotated fp32 block back
    M_OUT_Q8 = 16,    // write permuted Q8_1
    M_CHUNK_MAJOR = 32,
    M_VEC = 64,       // 16-byte aligned fp32 pointers: dwordx4 loads/stores
};

__device__ __forceinline__ float silu(float g) { return g / (1.0f + expf(-g)); }

// Grid (n/1024, n_tok), 64 threads.  `x` (and `up` for SwiGLU) are [n_tok][n].
template <int MODE>
__global__ void __launch_bounds__(64)
rot_quant_kernel(const float * __restrict__ x, const float * __restrict__ up,
                 const float * __restrict__ signs, float * __restrict__ xout,
                 uint8_t * __restrict__ q, int n, int n_tok) {
    const int l = threadIdx.x;
    const int blk = blockIdx.x;
    const int tok = blockIdx.y;
    const bool vec = (MODE & M_VEC) != 0;
    const int row = fwht_row(l);
    const size_t base = (size_t)tok * n + (size_t)blk * HBLK + 16 * row;

    float v[16];
    load16(x + base, v, vec);
    if (MODE & M_SWIGLU) {
        float u[16];
        load16(up + base, u, vec);
#pragma unroll
        for (int r = 0; r < 16; ++r) v[r] = silu(v[r]) * u[r];
    }
    if (MODE & M_SIGNS) {
        float sg[16];
        load16(signs + (size_t)blk * HBLK + 16 * row, sg, vec);
#pragma unroll
        for (int r = 0; r < 16; ++r) v[r] *= sg[r];
    }

    if (MODE & M_ROT) fwht1024_regs(v, l);

    if (MODE & M_OUT_F32) store16(xout + base, v, vec);
    if (MODE & M_OUT_Q8) {
        const int nchunk = n / QK8;
        const int c = blk * (HBLK / QK8) + (row >> 1);
        const size_t bidx = (MODE & M_CHUNK_MAJOR) ? (size_t)c * n_tok + tok : (size_t)tok * nchunk + c;
        quant_pair_store(v, q + bidx * Q81_BYTES, row & 1);
    }
}

// Quantisation only (n % 32 == 0): 256 threads = 128 chunks per workgroup,
// lane pair per chunk.  Grid (ceil(nchunk/128), n_tok).
template <bool CHUNK_MAJOR, bool VEC>
__global__ void __launch_bounds__(256)
quant_kernel(const float * __restrict__ x, uint8_t * __restrict__ q, int nchunk, int n_tok) {
    const int c = blockIdx.x * 128 + (threadIdx.x >> 1);
    const int tok = blockIdx.y;
    const int half = threadIdx.x & 1;
    // both lanes of a pair are in or out together (c is shared)
    if (c >= nchunk) return;
    float v[16];
    load16(x + (size_t)tok * nchunk * QK8 + (size_t)c * QK8 + 16 * half, v, VEC);
    const size_t bidx = CHUNK_MAJOR ? (size_t)c * n_tok + tok : (size_t)tok * nchunk + c;
    quant_pair_store(v, q + bidx * Q81_BYTES, half);
}

inline bool al16(const void * p) { return p == nullptr || ((uintptr_t)p & 15u) == 0; }
inline bool al4(const void * p) { return ((uintptr_t)p & 3u) == 0; }

template <int MODE>
int launch_rot(const float * x, const float * up, const float * signs, float * xout, void * q,
               int64_t n, int64_t n_tok, hipStream_t st) {
    dim3 grid((unsigned)(n / HBLK), (unsigned)n_tok);
    const bool vec = al16(x) && al16(up) && al16(signs) && al16(xout);
    const bool sg = signs != nullptr;
#define PQ2_ROT_LAUNCH(M)                                                                         \
    hipLaunchKernelGGL(rot_quant_kernel<(M)>, grid, dim3(64), 0, st, x, up, signs, xout,         \
                       (uint8_t *)q, (int)n, (int)n_tok)
    if (vec && sg) PQ2_ROT_LAUNCH(MODE | M_VEC | M_SIGNS);
    else if (vec) PQ2_ROT_LAUNCH(MODE | M_VEC);
    else if (sg) PQ2_ROT_LAUNCH(MODE | M_SIGNS);
    else PQ2_ROT_LAUNCH(MODE);
#undef PQ2_ROT_LAUNCH
    return (int)hipGetLastError();
}

int launch_quant(const float * x, void * q, int64_t n, int64_t n_tok, bool chunk_major, hipStream_t st) {
    const int nchunk = (int)(n / QK8);
    dim3 grid((unsigned)cdiv(nchunk, 128), (unsigned)n_tok);
    const bool vec = al16(x);
    if (chunk_major) {
        if (vec) hipLaunchKernelGGL((quant_kernel<true, true>), grid, dim3(256), 0, st, x, (uint8_t *)q, nchunk, (int)n_tok);
        else hipLaunchKernelGGL((quant_kernel<true, false>), grid, dim3(256), 0, st, x, (uint8_t *)q, nchunk, (int)n_tok);
    } else {
        if (vec) hipLaunchKernelGGL((quant_kernel<false, true>), grid, dim3(256), 0, st, x, (uint8_t *)q, nchunk, (int)n_tok);
        else hipLaunchKernelGGL((quant_kernel<false, false>), grid, dim3(256), 0, st, x, (uint8_t *)q, nchunk, (int)n_tok);
    }
    return (int)hipGetLastError();
}

constexpr int64_t MAX_GRID_Y = 65535;

}  // namespace

extern "C" {

int bonsai_p40_fwht(float * x, const float * signs, int64_t n, bonsai_stream stream) {
    if (n <= 0 || n % HBLK != 0 || x == nullptr) return 1;
    if (n / HBLK > 0x7fffffff) return 1;
    return launch_rot<M_ROT | M_OUT_F32>(x, nullptr, signs, x, nullptr, n, 1, (hipStream_t)stream);
}

int bonsai_p40_quant_activations(const float * x, void * out, int64_t n, bonsai_stream stream) {
    if (n <= 0 || n % QK8 != 0 || !al4(out)) return 1;
    if (n / QK8 > 0x7fffffff - 128) return 1;
    return launch_quant(x, out, n, 1, false, (hipStream_t)stream);
}

int bonsai_p40_fwht_quant(const float * x, const float * signs, void * xq, int64_t n,
                          bonsai_stream stream) {
    if (n <= 0 || n % HBLK != 0 || !al4(xq)) return 1;
    return launch_rot<M_ROT | M_OUT_Q8>(x, nullptr, signs, nullptr, xq, n, 1, (hipStream_t)stream);
}

int bonsai_p40_quant_tokens(const float * X, const float * signs, void * Xq, int64_t n,
                            int64_t n_tok, int rotate, bonsai_stream stream) {
    if (n <= 0 || n_tok <= 0 || n_tok > MAX_GRID_Y || !al4(Xq)) return 1;
    if (n % (rotate ? HBLK : QK8) != 0) return 1;
    if (n * n_tok > ((int64_t)1 << 40)) return 1;
    if (rotate)
        return launch_rot<M_ROT | M_OUT_Q8 | M_CHUNK_MAJOR>(X, nullptr, signs, nullptr, Xq, n, n_tok,
                                                            (hipStream_t)stream);
    if (signs != nullptr) return 1;   // signs only apply with the rotation
    return launch_quant(X, Xq, n, n_tok, true, (hipStream_t)stream);
}

int bonsai_p40_swiglu_fwht_quant(const float * gate, const float * up, const float * signs,
                                 void * xq, int64_t n, bonsai_stream stream) {
    if (n <= 0 || n % HBLK != 0 || !al4(xq)) return 1;
    return launch_rot<M_ROT | M_OUT_Q8 | M_SWIGLU>(gate, up, signs, nullptr, xq, n, 1,
                                                   (hipStream_t)stream);
}

}  // extern "C"
