// fwht_quant.hip -- activation pre-pass kernels for gfx950:
//   * FWHT-1024 (normalised Sylvester-Hadamard, optional +-1 signs),
//   * permuted Q8_1 quantisation with the reference host rounding,
//   * both fused into one register-resident butterfly kernel, writing the
//     GEMV (token-major) or the GEMM (chunk-major) activation layout;
//   * SwiGLU (the FFN glue) -> FWHT -> Q8_1, the SwiGLU spread over 4 waves;
//   * RMSNorm -> FWHT -> Q8_1 of token rows in one launch (the step before
//     every projection of a layer).
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
#include "host_state.h"
#include "../../include/bonsai_p40.h"

using namespace pq2;

namespace {

enum : int {
    M_ROT = 1,        // apply the FWHT
    M_SIGNS = 2,      // multiply by signs first
    M_OUT_F32 = 8,    // write the rotated fp32 block back
    M_OUT_Q8 = 16,    // write permuted Q8_1
    M_CHUNK_MAJOR = 32,
    M_VEC = 64,       // 16-byte aligned fp32 pointers: dwordx4 loads/stores
};


// Grid (n/1024, n_tok), 64 threads.  `x` is [n_tok][n].  Block b reads its
// signs at signs + b * sign_stride: 1024 for a length-n vector (the host
// form), 0 for one 1024-entry vector reused by every block (the reference
// device kernel's form).
template <int MODE>
__global__ void __launch_bounds__(64)
rot_quant_kernel(const float * __restrict__ x, const float * __restrict__ signs, float * __restrict__ xout,
                 uint8_t * __restrict__ q, int n, int n_tok, int sign_stride) {
    const int l = threadIdx.x;
    const int blk = blockIdx.x;
    const int tok = blockIdx.y;
    const bool vec = (MODE & M_VEC) != 0;
    const int row = fwht_row(l);
    const size_t base = (size_t)tok * n + (size_t)blk * HBLK + 16 * row;

    float v[16];
    load16(x + base, v, vec);
    if (MODE & M_SIGNS) {
        float sg[16];
        load16(signs + (size_t)blk * sign_stride + 16 * row, sg, vec);
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

// RMSNorm -> FWHT -> Q8_1 of token rows (src/ops.h:13-22, then the pre-pass
// above).  Grid n_tok, one workgroup per token, nw = min(n / 1024, 16) waves;
// wave w owns the Hadamard blocks w, w + nw, ...  The sum of squares is
// accumulated in fp64 in the one order every normalising kernel uses
// (rms_sumsq: per-block lane sums, a wave tree, blocks in order), so every
// path computes the same s = 1 / sqrtf((float)(ss / n) + eps); the
// reference's sequential fp32 sum differs from it by that sum's own rounding.
// Then y = (x * s) * w, the signs, the register FWHT and the quantiser, as
// the pre-pass.  Output
// chunk-major (block (c, t) at c * n_tok + t; for one token the GEMV layout).
template <bool VEC, bool SIGNS>
__global__ void __launch_bounds__(1024)
rms_rot_quant_kernel(const float * __restrict__ x, const float * __restrict__ w,
                     const float * __restrict__ signs, uint8_t * __restrict__ q, int n, int n_tok,
                     float eps) {
    __shared__ double red[RMS_GROUP];
    const int l = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    const int tok = blockIdx.x;
    const int nhb = n / HBLK;
    const int row = fwht_row(l);
    const float * xt = x + (size_t)tok * n;

    const double tot = rms_sumsq(
        nhb, red, nw, wave, l, [&](int b, float (&v)[16]) { load16(xt + (size_t)HBLK * b + 16 * row, v, VEC); },
        [] { __syncthreads(); });
    const float s = 1.0f / sqrtf((float)(tot / (double)n) + eps);

    for (int b = wave; b < nhb; b += nw) {
        float v[16], wv[16];
        load16(xt + (size_t)HBLK * b + 16 * row, v, VEC);
        load16(w + (size_t)HBLK * b + 16 * row, wv, VEC);
#pragma unroll
        for (int r = 0; r < 16; ++r) v[r] = v[r] * s * wv[r];
        if constexpr (SIGNS) {
            float sg[16];
            load16(signs + (size_t)HBLK * b + 16 * row, sg, VEC);
#pragma unroll
            for (int r = 0; r < 16; ++r) v[r] *= sg[r];
        }
        fwht1024_regs(v, l);
        const size_t c = (size_t)b * (HBLK / QK8) + (row >> 1);
        quant_pair_store(v, q + (c * n_tok + tok) * Q81_BYTES, row & 1);
    }
}

// The same, one workgroup (4 waves) per (Hadamard block, token) for few
// tokens: every workgroup computes the token's sum of squares itself, in the
// order of rms_sumsq (so all blocks of a token, and every other normalising
// kernel, get a bit-identical scale), while wave 0's own block of x, w and
// signs is already in flight; wave 0 then normalises, rotates and quantises.
// The whole row is read once per block (an L2 hit after the first): the
// blocks spread over the CUs instead of queueing on one.
template <bool VEC, bool SIGNS>
__global__ void __launch_bounds__(256)
rms_rot_quant_block_kernel(const float * __restrict__ x, const float * __restrict__ w,
                           const float * __restrict__ signs, uint8_t * __restrict__ q, int n,
                           int n_tok, float eps) {
    __shared__ double red[RMS_GROUP];
    const int tid = threadIdx.x, l = tid & 63, wave = tid >> 6;
    const int b = blockIdx.x, tok = blockIdx.y;
    const int row = fwht_row(l);
    const float * xt = x + (size_t)tok * n;
    float v[16], wv[16], sg[16];
    if (wave == 0) {
        load16(xt + (size_t)HBLK * b + 16 * row, v, VEC);
        load16(w + (size_t)HBLK * b + 16 * row, wv, VEC);
        if constexpr (SIGNS) load16(signs + (size_t)HBLK * b + 16 * row, sg, VEC);
    }
    const double tot = rms_sumsq(
        n / HBLK, red, 4, wave, l,
        [&](int bb, float (&u)[16]) { load16(xt + (size_t)HBLK * bb + 16 * row, u, VEC); },
        [] { __syncthreads(); });
    if (wave != 0) return;
    const float s = 1.0f / sqrtf((float)(tot / (double)n) + eps);
#pragma unroll
    for (int r = 0; r < 16; ++r) v[r] = v[r] * s * wv[r];
    if constexpr (SIGNS) {
#pragma unroll
        for (int r = 0; r < 16; ++r) v[r] *= sg[r];
    }
    fwht1024_regs(v, l);
    const size_t c = (size_t)b * (HBLK / QK8) + (row >> 1);
    quant_pair_store(v, q + (c * n_tok + tok) * Q81_BYTES, row & 1);
}

// SwiGLU -> FWHT -> Q8_1 of one token, 4 waves per Hadamard block: the
// SwiGLU (an expf and an IEEE division per element, the bulk of the work) is
// spread over all 256 threads, 4 elements each, into LDS; wave 0 then loads
// the block in the FWHT lane layout, applies the signs, rotates and
// quantises.  Element values are swiglu1() of fwht_device.h.
template <bool VEC, bool SIGNS>
__global__ void __launch_bounds__(256)
swiglu_rot_quant_kernel(const float * __restrict__ gate, const float * __restrict__ up,
                        const float * __restrict__ signs, uint8_t * __restrict__ q) {
    __shared__ __attribute__((aligned(16))) float h[HBLK];
    const int tid = threadIdx.x, l = tid & 63;
    const size_t base = (size_t)blockIdx.x * HBLK;
    float g[4], u[4];
    if constexpr (VEC) {
        const float4 g4 = reinterpret_cast<const float4 *>(gate + base)[tid];
        const float4 u4 = reinterpret_cast<const float4 *>(up + base)[tid];
        g[0] = g4.x; g[1] = g4.y; g[2] = g4.z; g[3] = g4.w;
        u[0] = u4.x; u[1] = u4.y; u[2] = u4.z; u[3] = u4.w;
    } else {
#pragma unroll
        for (int k = 0; k < 4; ++k) { g[k] = gate[base + 4 * tid + k]; u[k] = up[base + 4 * tid + k]; }
    }
    float4 r;
    r.x = swiglu1(g[0], u[0]); r.y = swiglu1(g[1], u[1]); r.z = swiglu1(g[2], u[2]); r.w = swiglu1(g[3], u[3]);
    reinterpret_cast<float4 *>(h)[tid] = r;
    __syncthreads();
    if (tid >= 64) return;
    const int row = fwht_row(l);
    float v[16];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const float4 t = reinterpret_cast<const float4 *>(h + 16 * row)[k];
        v[4 * k] = t.x; v[4 * k + 1] = t.y; v[4 * k + 2] = t.z; v[4 * k + 3] = t.w;
    }
    if constexpr (SIGNS) {
        float sg[16];
        load16(signs + base + 16 * row, sg, VEC);
#pragma unroll
        for (int k = 0; k < 16; ++k) v[k] *= sg[k];
    }
    fwht1024_regs(v, l);
    quant_pair_store(v, q + ((size_t)blockIdx.x * (HBLK / QK8) + (row >> 1)) * Q81_BYTES, row & 1);
}

inline bool al16(const void * p) { return p == nullptr || ((uintptr_t)p & 15u) == 0; }
inline bool al4(const void * p) { return ((uintptr_t)p & 3u) == 0; }

template <int MODE>
int launch_rot(const float * x, const float * signs, float * xout, void * q,
               int64_t n, int64_t n_tok, hipStream_t st, int sign_stride = HBLK) {
    dim3 grid((unsigned)(n / HBLK), (unsigned)n_tok);
    const bool vec = al16(x) && al16(signs) && al16(xout);
    const bool sg = signs != nullptr;
#define PQ2_ROT_LAUNCH(M)                                                                         \
    hipLaunchKernelGGL(rot_quant_kernel<(M)>, grid, dim3(64), 0, st, x, signs, xout,         \
                       (uint8_t *)q, (int)n, (int)n_tok, sign_stride)
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
    // the reference device kernel's meaning: signs[0..1023] for every block
    // (elementwise_p40.cu:23), so no sign past the 1024th is ever read
    return launch_rot<M_ROT | M_OUT_F32>(x, signs, x, nullptr, n, 1, (hipStream_t)stream, 0);
}

int bonsai_p40_fwht_signs_n(float * x, const float * signs, int64_t n, bonsai_stream stream) {
    if (n <= 0 || n % HBLK != 0 || x == nullptr) return 1;
    if (n / HBLK > 0x7fffffff) return 1;
    return launch_rot<M_ROT | M_OUT_F32>(x, signs, x, nullptr, n, 1, (hipStream_t)stream, HBLK);
}

int bonsai_p40_quant_activations(const float * x, void * out, int64_t n, bonsai_stream stream) {
    if (n <= 0 || n % QK8 != 0 || !al4(out) || pq2host::any_null(x, out)) return 1;
    if (n / QK8 > 0x7fffffff - 128) return 1;
    return launch_quant(x, out, n, 1, false, (hipStream_t)stream);
}

int bonsai_p40_fwht_quant(const float * x, const float * signs, void * xq, int64_t n,
                          bonsai_stream stream) {
    if (n <= 0 || n % HBLK != 0 || !al4(xq) || pq2host::any_null(x, xq)) return 1;
    return launch_rot<M_ROT | M_OUT_Q8>(x, signs, nullptr, xq, n, 1, (hipStream_t)stream);
}

int bonsai_p40_quant_tokens(const float * X, const float * signs, void * Xq, int64_t n,
                            int64_t n_tok, int rotate, bonsai_stream stream) {
    if (n <= 0 || n_tok <= 0 || n_tok > MAX_GRID_Y || !al4(Xq) || pq2host::any_null(X, Xq)) return 1;
    if (n % (rotate ? HBLK : QK8) != 0) return 1;
    if (n * n_tok > ((int64_t)1 << 40)) return 1;
    if (rotate)
        return launch_rot<M_ROT | M_OUT_Q8 | M_CHUNK_MAJOR>(X, signs, nullptr, Xq, n, n_tok,
                                                            (hipStream_t)stream);
    if (signs != nullptr) return 1;   // signs only apply with the rotation
    return launch_quant(X, Xq, n, n_tok, true, (hipStream_t)stream);
}

int bonsai_p40_rmsnorm_fwht_quant(const float * x, const float * w, const float * signs, void * xq,
                                  int64_t n, int64_t n_tok, float eps, bonsai_stream stream) {
    if (n <= 0 || n % HBLK != 0 || pq2host::any_null(x, w, xq) || !al4(xq)) return 1;
    if (n_tok <= 0) return 0;
    if (n_tok > 0x7fffffff || n > 0x7fffffff) return 1;
    const int nw = (int)(n / HBLK < 16 ? n / HBLK : 16);
    const bool vec = al16(x) && al16(w) && al16(signs);
    hipStream_t st = (hipStream_t)stream;
    // few tokens: a workgroup per block (spread over the CUs); many: one per
    // token (each token row read once)
    const bool per_block = n_tok * (n / HBLK) <= 4096 && n_tok <= 65535 && n / HBLK <= 0x7fffffff;
#define PQ2_RMS_LAUNCH(V, S)                                                                        \
    if (per_block)                                                                                  \
        hipLaunchKernelGGL((rms_rot_quant_block_kernel<V, S>), dim3((unsigned)(n / HBLK), (unsigned)n_tok), \
                           dim3(256), 0, st, x, w, signs, (uint8_t *)xq, (int)n, (int)n_tok, eps);  \
    else                                                                                            \
        hipLaunchKernelGGL((rms_rot_quant_kernel<V, S>), dim3((unsigned)n_tok), dim3(64 * nw), 0, st, \
                           x, w, signs, (uint8_t *)xq, (int)n, (int)n_tok, eps)
    if (vec && signs) PQ2_RMS_LAUNCH(true, true);
    else if (vec) PQ2_RMS_LAUNCH(true, false);
    else if (signs) PQ2_RMS_LAUNCH(false, true);
    else PQ2_RMS_LAUNCH(false, false);
#undef PQ2_RMS_LAUNCH
    return (int)hipGetLastError();
}

int bonsai_p40_swiglu_fwht_quant(const float * gate, const float * up, const float * signs,
                                 void * xq, int64_t n, bonsai_stream stream) {
    if (n <= 0 || n % HBLK != 0 || !al4(xq) || pq2host::any_null(gate, up, xq)) return 1;
    if (n / HBLK > 0x7fffffff) return 1;
    const bool vec = al16(gate) && al16(up) && al16(signs);
    const dim3 grid((unsigned)(n / HBLK));
    hipStream_t st = (hipStream_t)stream;
    if (vec && signs) hipLaunchKernelGGL((swiglu_rot_quant_kernel<true, true>), grid, dim3(256), 0, st, gate, up, signs, (uint8_t *)xq);
    else if (vec) hipLaunchKernelGGL((swiglu_rot_quant_kernel<true, false>), grid, dim3(256), 0, st, gate, up, signs, (uint8_t *)xq);
    else if (signs) hipLaunchKernelGGL((swiglu_rot_quant_kernel<false, true>), grid, dim3(256), 0, st, gate, up, signs, (uint8_t *)xq);
    else hipLaunchKernelGGL((swiglu_rot_quant_kernel<false, false>), grid, dim3(256), 0, st, gate, up, signs, (uint8_t *)xq);
    return (int)hipGetLastError();
}

}  // extern "C"
