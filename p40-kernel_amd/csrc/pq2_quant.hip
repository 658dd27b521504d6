// pq2_quant.hip -- the reference ternary weight quantiser and dequantiser on
// gfx950 (src/pq2_0.h:62-90): fp32 rows -> block_pq2_0 and back.
//
// quantize: per 128 weights, d = amax (stored with the host's ties-away fp16
// encode), id = 1/d (IEEE division; 0 for an all-zero block), code =
// clamp(round_half_away(x * id) + 1, 0, 3) packed 4 per byte, element j at
// bits 2(j%4) of byte j/4.  The bytes equal quantize_row_pq2_0's for every
// finite input (NaN or infinite inputs reach lroundf(NaN) in the reference,
// whose result is unspecified).  dequantize: y = (code - 1) * d, exact.
//
// Load-time transforms, not on the per-token path: a block is 32 lanes (four
// weights, i.e. one code byte, per lane), two blocks per wave.
#include "pq2_device.h"
#include "../../include/bonsai_p40.h"

using namespace pq2;

namespace {

constexpr int QZ_THREADS = 256;                    // 8 blocks per workgroup
constexpr int QZ_BLOCKS = QZ_THREADS / 32;

// maximum over the 32 lanes of a half-wave (every lane gets it)
__device__ __forceinline__ float half_wave_max(float v) {
#pragma unroll
    for (int m = 1; m < 32; m <<= 1) v = fmaxf(v, __shfl_xor(v, m, 32));
    return v;
}

__global__ void __launch_bounds__(QZ_THREADS)
quantize_pq2_0_kernel(const float * __restrict__ x, uint8_t * __restrict__ w, int64_t nblk) {
    const int64_t b = (int64_t)blockIdx.x * QZ_BLOCKS + (threadIdx.x >> 5);
    const int l = threadIdx.x & 31;
    if (b >= nblk) return;                          // both halves of a wave exit per block
    const float * xb = x + b * QK_PQ2 + 4 * l;
    float v[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = xb[i];
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) amax = fmaxf(amax, fabsf(v[i]));
    amax = half_wave_max(amax);
    const float id = amax > 0.0f ? 1.0f / amax : 0.0f;
    uint32_t byte = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float p = v[i] * id;
        // round half away from zero: trunc(2p) - trunc(p) (2p is exact)
        int q = (int)truncf(2.0f * p) - (int)truncf(p) + 1;
        q = q < 0 ? 0 : (q > 3 ? 3 : q);
        byte |= (uint32_t)q << (2 * i);
    }
    uint8_t * wb = w + b * PQ2_BYTES;
    wb[2 + l] = (uint8_t)byte;
    if (l == 0) {
        const uint32_t h = f32_to_f16_away(amax);
        wb[0] = (uint8_t)h;
        wb[1] = (uint8_t)(h >> 8);
    }
}

__global__ void __launch_bounds__(QZ_THREADS)
dequantize_pq2_0_kernel(const uint8_t * __restrict__ w, float * __restrict__ y, int64_t nblk) {
    const int64_t b = (int64_t)blockIdx.x * QZ_BLOCKS + (threadIdx.x >> 5);
    const int l = threadIdx.x & 31;
    if (b >= nblk) return;
    const uint8_t * wb = w + b * PQ2_BYTES;
    const float d = f16_bits_to_f32((uint32_t)wb[0] | ((uint32_t)wb[1] << 8));
    const uint32_t byte = wb[2 + l];
    float * yb = y + b * QK_PQ2 + 4 * l;
#pragma unroll
    for (int i = 0; i < 4; ++i) yb[i] = (float)((int)((byte >> (2 * i)) & 3u) - 1) * d;
}

}  // namespace

extern "C" {

int bonsai_p40_quantize_pq2_0(const float * x, void * w, int64_t n, bonsai_stream stream) {
    if (n <= 0 || n % QK_PQ2 != 0 || x == nullptr || w == nullptr) return 1;
    if (((uintptr_t)x & 3u) != 0 || ((uintptr_t)w & 1u) != 0) return 1;
    const int64_t nblk = n / QK_PQ2;
    const int64_t grid = (nblk + QZ_BLOCKS - 1) / QZ_BLOCKS;
    if (grid > 0x7fffffff) return 1;
    hipLaunchKernelGGL(quantize_pq2_0_kernel, dim3((unsigned)grid), dim3(QZ_THREADS), 0, (hipStream_t)stream, x,
                       static_cast<uint8_t *>(w), nblk);
    return (int)hipGetLastError();
}

int bonsai_p40_dequantize_pq2_0(const void * w, float * y, int64_t n, bonsai_stream stream) {
    if (n <= 0 || n % QK_PQ2 != 0 || w == nullptr || y == nullptr) return 1;
    if (((uintptr_t)y & 3u) != 0 || ((uintptr_t)w & 1u) != 0) return 1;
    const int64_t nblk = n / QK_PQ2;
    const int64_t grid = (nblk + QZ_BLOCKS - 1) / QZ_BLOCKS;
    if (grid > 0x7fffffff) return 1;
    hipLaunchKernelGGL(dequantize_pq2_0_kernel, dim3((unsigned)grid), dim3(QZ_THREADS), 0, (hipStream_t)stream,
                       static_cast<const uint8_t *>(w), y, nblk);
    return (int)hipGetLastError();
}

}  // extern "C"
