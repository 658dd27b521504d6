// gemm.hip -- prefill PQ2_0 x Q8_1 GEMM on gfx950 int8 MFMA.
//
// Contract (reference tests/test_p40.cpp:449-470, src/kernels/gemm_p40.cu:44-154):
//   Y[r*n_tok + t] = sum_b sum_p f16(dw[r,b]) * f16(da[4b+p, t]) * S(r, b, p, t)
// with S the exact integer chunk dot sum (code-1)*q over the 32 weights of
// chunk p of block b, and X chunk-major (block (c, t) at c*n_tok + t).
//
// Tile design: a workgroup of 4 waves computes a (32*WM) x (32*WN) tile of
// (rows x tokens); each wave owns a 32 x 32 sub-tile.  Per PQ2_0 block
// (K = 128 = 4 chunks) the workgroup stages the block's codes and fp16 d of
// its rows and the 4 Q8_1 chunks of its tokens in LDS; each chunk is then one
// v_mfma_i32_32x32x32_i8 per wave (K = 32 = one chunk, so the int32 result is
// exactly S for every (row, token) of the sub-tile):
//   * A (rows x 32): codes unpacked to int8 (code - 1) in registers with SWAR
//     ((w >> 2k) & 0x03030303, then +0x7f7f7f7f ^ 0x80808080 per byte), so the
//     "- s" bias of the reference is folded into the product;
//   * B (32 x tokens): the permuted Q8_1 bytes as stored -- the code word
//     extraction order k, k+4, k+8, k+12 matches the activation permutation,
//     so A and B share the same K order without any shuffle;
//   * epilogue per chunk: inner += da[t] * float(S) (per token scale), per
//     block: acc += dw[r] * inner (per row scale) -- fp32, as the reference.
#include "pq2_device.h"
#include "../../include/bonsai_p40.h"

using namespace pq2;

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

__device__ __forceinline__ int codes_minus_one(uint32_t w, int k) {
    const uint32_t t = (w >> (2 * k)) & 0x03030303u;
    return (int)((t + 0x7f7f7f7fu) ^ 0x80808080u);
}

template <int WM, int WN>
__global__ void __launch_bounds__(256)
gemm_mfma_kernel(const uint8_t * __restrict__ W, const uint8_t * __restrict__ X,
                 float * __restrict__ Y, int n_out, int n_tok, int nb) {
    constexpr int BM = 32 * WM, BN = 32 * WN;
    __shared__ uint32_t sA[BM][9];                       // 8 code dwords per row (+1 pad)
    __shared__ __attribute__((aligned(16))) float sDw[BM];
    __shared__ __attribute__((aligned(16))) uint32_t sX[4][BN][8];
    __shared__ float sDa[4][BN];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave % WM, wn = wave / WM;
    const int row0 = blockIdx.x * BM, tok0 = blockIdx.y * BN;
    const int h = lane >> 5, l32 = lane & 31;
    const size_t wstride = (size_t)PQ2_BYTES * nb;

    float acc[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[i] = 0.0f;

    for (int b = 0; b < nb; ++b) {
        for (int i = tid; i < BM * 17; i += 256) {
            const int rr = i / 17, k = i - 17 * rr;
            const int row = row0 + rr;
            uint32_t v = 0x5555u;                         // all codes 1 -> value 0
            if (row < n_out)
                v = reinterpret_cast<const uint16_t *>(W + (size_t)row * wstride + (size_t)PQ2_BYTES * b)[k];
            else if (k == 0)
                v = 0;
            if (k == 0) sDw[rr] = f16_bits_to_f32(v);
            else reinterpret_cast<uint16_t *>(sA[rr])[k - 1] = (uint16_t)v;
        }
        for (int i = tid; i < 4 * BN * 9; i += 256) {
            const int k = i % 9, rest = i / 9;
            const int t = rest % BN, p = rest / BN;
            const int tok = tok0 + t;
            uint32_t v = 0;
            if (tok < n_tok)
                v = reinterpret_cast<const uint32_t *>(X + ((size_t)(4 * b + p) * n_tok + tok) * Q81_BYTES)[k];
            if (k == 0) sDa[p][t] = f16_bits_to_f32(v & 0xffffu);
            else sX[p][t][k - 1] = v;
        }
        __syncthreads();

        float inner[16];
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            const uint32_t w = sA[wm * 32 + l32][2 * p + h];
            v4i A;
            A.x = codes_minus_one(w, 0); A.y = codes_minus_one(w, 1);
            A.z = codes_minus_one(w, 2); A.w = codes_minus_one(w, 3);
            const v4i B = *reinterpret_cast<const v4i *>(&sX[p][wn * 32 + l32][4 * h]);
            v16i S = {};
            S = __builtin_amdgcn_mfma_i32_32x32x32_i8(A, B, S, 0, 0, 0);
            const float da = sDa[p][wn * 32 + l32];
#pragma unroll
            for (int i = 0; i < 16; ++i) inner[i] = (p == 0) ? da * (float)S[i] : fmaf(da, (float)S[i], inner[i]);
        }
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const float4 dw = *reinterpret_cast<const float4 *>(&sDw[wm * 32 + 8 * q + 4 * h]);
            acc[4 * q + 0] = fmaf(dw.x, inner[4 * q + 0], acc[4 * q + 0]);
            acc[4 * q + 1] = fmaf(dw.y, inner[4 * q + 1], acc[4 * q + 1]);
            acc[4 * q + 2] = fmaf(dw.z, inner[4 * q + 2], acc[4 * q + 2]);
            acc[4 * q + 3] = fmaf(dw.w, inner[4 * q + 3], acc[4 * q + 3]);
        }
        __syncthreads();
    }

    const int tok = tok0 + wn * 32 + l32;
    if (tok < n_tok) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int row = row0 + wm * 32 + 8 * (i >> 2) + 4 * h + (i & 3);
            if (row < n_out) Y[(size_t)row * n_tok + tok] = acc[i];
        }
    }
}

}  // namespace

extern "C" {

int bonsai_p40_gemm(const void * W, const void * Xq, float * Y, int64_t n_out, int64_t n_in,
                    int64_t n_tok, bonsai_stream stream) {
    if (n_in <= 0 || n_in % QK_PQ2 != 0) return 1;
    if (n_out <= 0 || n_tok <= 0) return 0;
    if (((uintptr_t)Xq & 3u) != 0 || ((uintptr_t)W & 1u) != 0) return 1;
    if (n_out > 0x7fffffff || n_tok > 0x7fffffff) return 1;
    const int nb = (int)(n_in / QK_PQ2);
    hipStream_t st = (hipStream_t)stream;
    if (n_tok <= 32) {
        dim3 grid((unsigned)cdiv(n_out, 128), (unsigned)cdiv(n_tok, 32));
        hipLaunchKernelGGL((gemm_mfma_kernel<4, 1>), grid, dim3(256), 0, st, (const uint8_t *)W,
                           (const uint8_t *)Xq, Y, (int)n_out, (int)n_tok, nb);
    } else {
        dim3 grid((unsigned)cdiv(n_out, 64), (unsigned)cdiv(n_tok, 64));
        hipLaunchKernelGGL((gemm_mfma_kernel<2, 2>), grid, dim3(256), 0, st, (const uint8_t *)W,
                           (const uint8_t *)Xq, Y, (int)n_out, (int)n_tok, nb);
    }
    return (int)hipGetLastError();
}

}  // extern "C"
