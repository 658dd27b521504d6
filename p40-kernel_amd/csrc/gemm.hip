// gemm.hip -- prefill PQ2_0 x Q8_1 GEMM on gfx950 int8 MFMA.
//
// Contract (reference tests/test_p40.cpp:449-470, src/kernels/gemm_p40.cu:44-154):
//   Y[r*n_tok + t] = sum_b sum_p f16(dw[r,b]) * f16(da[4b+p, t]) * S(r, b, p, t)
// with S the exact integer chunk dot sum (code-1)*q over the 32 weights of
// chunk p of block b, and X chunk-major (block (c, t) at c*n_tok + t).
//
// Design
// ------
// * One v_mfma_i32_32x32x32_i8 covers one Q8_1 chunk (K = 32) for a 32x32
//   (rows x tokens) tile, so its int32 result is exactly S for every element.
//   A = codes unpacked to int8 (code - 1) with SWAR ((w >> 2k) & 0x03030303,
//   then +0x7f7f7f7f ^ 0x80808080 per byte), which folds the reference's "- s"
//   bias into the product; B = the permuted Q8_1 bytes as stored: the code
//   word extraction order k, k+4, k+8, k+12 is the activation permutation, so
//   A and B share one K order without any shuffle.
// * Epilogue per chunk: inner += da[t] * float(S) (per-token scale); per block
//   acc += dw[r] * inner (per-row scale).  This fp32 rescale per (row, token,
//   chunk) -- about 2.25 VALU instructions per element per chunk against one
//   32-cycle MFMA per 1024 elements -- is what bounds the kernel.
// * Workgroup tile BM x BN = 128 x 128 (8 waves, 4 x 2, each 32 x 64 = 1 x 2
//   MFMA tiles sharing one unpacked A operand).  Per PQ2_0 block (K = 128) the workgroup stages the tile's
//   codes (realigned to dwords), block scales and the 4 Q8_1 chunks of its
//   tokens in LDS; the next block's global loads are issued into registers
//   before the current block is computed.
// * Small batches (n_tok <= 32) use a 128 x 32 tile (4 waves stacked on rows).
#include "pq2_device.h"
#include "host_state.h"
#include "../../include/bonsai_p40.h"

#include <stdlib.h>
#include <type_traits>

using namespace pq2;

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

// s_waitcnt vmcnt(N) with the other counters open (gfx9 encoding)
template <int N>
__device__ __forceinline__ void wait_vmcnt_sk() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x0F70);
}

__device__ __forceinline__ int codes_minus_one(uint32_t w, int k) {
    const uint32_t t = (w >> (2 * k)) & 0x03030303u;
    return (int)((t + 0x7f7f7f7fu) ^ 0x80808080u);
}

// WM x WN waves, each owning TM x TN MFMA tiles of 32 x 32.
template <int WM, int WN, int TM, int TN>
struct GemmCfg {
    static constexpr int BM = 32 * TM * WM;     // rows per workgroup
    static constexpr int BN = 32 * TN * WN;     // tokens per workgroup
    static constexpr int THREADS = 64 * WM * WN;
    // global loads per thread per block
    static constexpr int A_DW = BM * 9;                    // 9 dwords cover a 34-byte block
    static constexpr int A_PER = (A_DW + THREADS - 1) / THREADS;
    static constexpr int X_DW = 4 * BN * 9;                // 4 chunks x BN tokens x 36 bytes
    static constexpr int X_PER = (X_DW + THREADS - 1) / THREADS;
};

template <int WM, int WN, int TM, int TN>
__global__ void __launch_bounds__(64 * WM * WN)
gemm_mfma_kernel(const uint8_t * __restrict__ W, const uint8_t * __restrict__ X,
                 float * __restrict__ Y, int n_out, int n_tok, int nb) {
    using C = GemmCfg<WM, WN, TM, TN>;
    constexpr int BM = C::BM, BN = C::BN;
    __shared__ uint32_t sA[BM][10];                       // raw 9-dword window of each row's block (+1 pad)
    __shared__ __attribute__((aligned(16))) uint32_t sX[4][BN][8];
    __shared__ float sDa[4][BN];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave % WM, wn = wave / WM;
    const int row0 = blockIdx.x * BM, tok0 = blockIdx.y * BN;
    const int h = lane >> 5, l32 = lane & 31;
    const size_t wstride = (size_t)PQ2_BYTES * nb;          // bytes per weight row (even nb: 4-aligned)

    // ---- global -> register prefetch of one block ---------------------------
    // A: row rr, dword k (0..8) of the 9-dword window that starts at the
    // block's dword-aligned floor.  For even nb a block starts 4-aligned when
    // b is even and 2 bytes past a dword when b is odd.
    uint32_t ra[C::A_PER];
    uint32_t rx[C::X_PER];
    auto prefetch = [&](int b) {
#pragma unroll
        for (int j = 0; j < C::A_PER; ++j) {
            const int i = tid + j * C::THREADS;
            uint32_t v = 0x55555555u;                     // codes all 1 -> (code - 1) = 0
            if (i < C::A_DW) {
                const int rr = i / 9, k = i - 9 * rr;
                const int row = row0 + rr;
                if (row < n_out) {
                    const size_t boff = (size_t)row * wstride + (size_t)PQ2_BYTES * b;
                    // window [floor(block start), +36): for an even block it ends 2 bytes
                    // into the next block, for an odd one exactly at the block end, so
                    // it never leaves the row (the last block of a row is odd)
                    const size_t a0 = (boff & ~(size_t)3) + 4 * (size_t)k;
                    v = *reinterpret_cast<const uint32_t *>(W + a0);
                } else if (k == 0) {
                    v = 0;
                }
            }
            ra[j] = v;
        }
#pragma unroll
        for (int j = 0; j < C::X_PER; ++j) {
            const int i = tid + j * C::THREADS;
            uint32_t v = 0;
            if (i < C::X_DW) {
                const int k = i % 9, rest = i / 9;
                const int t = rest % BN, p = rest / BN;
                const int tok = tok0 + t;
                if (tok < n_tok)
                    v = reinterpret_cast<const uint32_t *>(X + ((size_t)(4 * b + p) * n_tok + tok) * Q81_BYTES)[k];
            }
            rx[j] = v;
        }
    };
    // ---- registers -> LDS ---------------------------------------------------
    auto commit = [&]() {
#pragma unroll
        for (int j = 0; j < C::A_PER; ++j) {
            const int i = tid + j * C::THREADS;
            if (i < C::A_DW) {
                const int rr = i / 9, k = i - 9 * rr;
                sA[rr][k] = ra[j];
            }
        }
#pragma unroll
        for (int j = 0; j < C::X_PER; ++j) {
            const int i = tid + j * C::THREADS;
            if (i < C::X_DW) {
                const int k = i % 9, rest = i / 9;
                const int t = rest % BN, p = rest / BN;
                if (k == 0) sDa[p][t] = f16_bits_to_f32(rx[j] & 0xffffu);
                else sX[p][t][k - 1] = rx[j];
            }
        }
    };

    float acc[TM][TN][16];
#pragma unroll
    for (int a = 0; a < TM; ++a)
#pragma unroll
        for (int c = 0; c < TN; ++c)
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[a][c][i] = 0.0f;

    prefetch(0);
    for (int b = 0; b < nb; ++b) {
        __syncthreads();                       // previous block's LDS reads are done
        commit();
        __syncthreads();
        if (b + 1 < nb) prefetch(b + 1);
        // The raw window of a row starts at the block's dword floor; the block
        // begins sh bytes into dword 0 (0 for even b, 2 for odd b: rows are
        // 4-byte aligned because nb is even).  fp16 d = block bytes [0, 2),
        // code dword c = block bytes [2 + 4c, 6 + 4c).
        const int sh = (int)(((size_t)PQ2_BYTES * b) & 3);

        float inner[TM][TN][16];
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            v4i A[TM];
#pragma unroll
            for (int a = 0; a < TM; ++a) {
                const int rr = (wm * TM + a) * 32 + l32;
                // code dword (2p + h) = block bytes [2 + 8p + 4h, 6 + 8p + 4h)
                const int byte = sh + 2 + 8 * p + 4 * h;
                const uint32_t lo = sA[rr][byte >> 2], hi = sA[rr][(byte >> 2) + 1];
                const uint32_t w = __builtin_amdgcn_alignbyte(hi, lo, byte & 3);
                A[a].x = codes_minus_one(w, 0); A[a].y = codes_minus_one(w, 1);
                A[a].z = codes_minus_one(w, 2); A[a].w = codes_minus_one(w, 3);
            }
#pragma unroll
            for (int c = 0; c < TN; ++c) {
                const int tt = (wn * TN + c) * 32 + l32;
                const v4i Bv = *reinterpret_cast<const v4i *>(&sX[p][tt][4 * h]);
                const float da = sDa[p][tt];
#pragma unroll
                for (int a = 0; a < TM; ++a) {
                    v16i S = {};
                    S = __builtin_amdgcn_mfma_i32_32x32x32_i8(A[a], Bv, S, 0, 0, 0);
#pragma unroll
                    for (int i = 0; i < 16; ++i)
                        inner[a][c][i] = (p == 0) ? da * (float)S[i] : fmaf(da, (float)S[i], inner[a][c][i]);
                }
            }
        }
        // per-row block scale: rows 8(i/4) + 4h + (i%4) of each 32-row tile
#pragma unroll
        for (int a = 0; a < TM; ++a) {
            const int rbase = (wm * TM + a) * 32;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int rr = rbase + 8 * q + 4 * h;
                float dw[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const uint32_t d0 = sA[rr + e][0];
                    dw[e] = f16_bits_to_f32(sh ? (d0 >> 16) : (d0 & 0xffffu));
                }
#pragma unroll
                for (int c = 0; c < TN; ++c)
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        acc[a][c][4 * q + e] = fmaf(dw[e], inner[a][c][4 * q + e], acc[a][c][4 * q + e]);
            }
        }
    }

#pragma unroll
    for (int c = 0; c < TN; ++c) {
        const int tok = tok0 + (wn * TN + c) * 32 + l32;
        if (tok >= n_tok) continue;
#pragma unroll
        for (int a = 0; a < TM; ++a) {
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int row = row0 + (wm * TM + a) * 32 + 8 * (i >> 2) + 4 * h + (i & 3);
                if (row < n_out) Y[(size_t)row * n_tok + tok] = acc[a][c][i];
            }
        }
    }
}

// Odd nb (n_in = 128 * odd): blocks are 2-byte aligned with a row-dependent
// phase, so this variant stages codes with 16-bit loads.
__global__ void __launch_bounds__(256)
gemm_mfma_kernel_u16(const uint8_t * __restrict__ W, const uint8_t * __restrict__ X,
                     float * __restrict__ Y, int n_out, int n_tok, int nb) {
    constexpr int BM = 64, BN = 64;
    __shared__ uint32_t sA[BM][9];
    __shared__ __attribute__((aligned(16))) float sDw[BM];
    __shared__ __attribute__((aligned(16))) uint32_t sX[4][BN][8];
    __shared__ float sDa[4][BN];
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave % 2, wn = wave / 2;
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
            uint32_t v = 0x5555u;
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
            const v4i Bv = *reinterpret_cast<const v4i *>(&sX[p][wn * 32 + l32][4 * h]);
            v16i S = {};
            S = __builtin_amdgcn_mfma_i32_32x32x32_i8(A, Bv, S, 0, 0, 0);
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

// ---------------------------------------------------------------------------
// Small batch (2 <= n_tok <= 16), bandwidth-bound: a workgroup owns 16 rows
// and its 4 waves split K into quarters on even-block boundaries (every model
// width has nb % 8 == 0).  Each wave DMAs its 16 row segments (34 * nb/4
// bytes each, dword aligned) into LDS with global_load_lds_dword, then per
// Q8_1 chunk issues one v_mfma_i32_16x16x32_i8: A = 16 rows x 32 weights as
// int8 (code - 1), B = 32 activations x 16 token columns read straight from
// the chunk-major X (columns past n_tok carry a duplicate token and are not
// stored).  Lane (r = l%16, g = l/16) supplies the 8 bytes of K-group g:
// activation words 2(g%2), 2(g%2)+1 of half g/2 -- the code words
// (w >> 2k) & 0x03030303 of the same half line up byte for byte.  The four
// K-quarter partials are summed through LDS.
typedef int v2i __attribute__((ext_vector_type(2), aligned(4)));
typedef int v4ia __attribute__((ext_vector_type(4)));
typedef int v4ia4 __attribute__((ext_vector_type(4), aligned(4)));   // 4-byte aligned (36-byte records)
typedef __attribute__((address_space(3))) void lds_void;

__global__ void __launch_bounds__(256)
gemm_skinny_kernel(const uint8_t * __restrict__ W, const uint8_t * __restrict__ X,
                   float * __restrict__ Y, int n_out, int n_tok, int nb) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int nbq = nb / 4;                       // blocks per K quarter (even)
    const int seg = PQ2_BYTES * nbq;              // bytes per row segment (multiple of 4)
    const int segdw = seg / 4;
    uint8_t * wl = smem + (size_t)wave * 16 * seg;
    float * red = reinterpret_cast<float *>(smem + (size_t)4 * 16 * seg);   // [4][16][16]
    const int row0 = blockIdx.x * 16;
    const size_t wstride = (size_t)PQ2_BYTES * nb;

    // 1. DMA the wave's 16 row segments: LDS dword idx = r * segdw + d
    const int ndw = 16 * segdw;
    for (int i = 0; i < ndw; i += 64) {
        const int idx = i + lane;
        if (idx < ndw) {                          // lanes past the segment write nothing
            const int r = idx / segdw, d = idx - r * segdw;
            const int row = min(row0 + r, n_out - 1);
            const uint8_t * src = W + (size_t)row * wstride + (size_t)seg * wave + 4 * (size_t)d;
            __builtin_amdgcn_global_load_lds(src, (lds_void *)(wl + 4 * i), 4, 0, 0);
        }
    }

    const int r = lane & 15, g = lane >> 4;
    const int t = min(lane & 15, n_tok - 1);      // B column (token)
    const int h = g >> 1, kk = 2 * (g & 1);       // half and first activation word of the K-group
    const int c0 = 4 * nbq * wave;                // first global chunk of this quarter
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};

    // X for two blocks (8 chunks) per register set, loaded two blocks ahead
    uint32_t nd[8], cd[8];
    v2i nx[8], cx[8];
    // per-lane byte offset inside a chunk's n_tok blocks; the chunk base is uniform
    const uint32_t xlane = (uint32_t)t * Q81_BYTES;
    const size_t cstride = (size_t)n_tok * Q81_BYTES;
    auto load_x = [&](int b) {
        const uint8_t * xc = X + (size_t)(c0 + 4 * min(b, nbq - 2)) * cstride;   // past the end: re-read the last pair
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            const uint8_t * xp = xc + (size_t)q * cstride + xlane;
            nd[q] = *reinterpret_cast<const uint32_t *>(xp);
            nx[q] = *reinterpret_cast<const v2i *>(xp + 4 + 8 * g);
        }
    };
    load_x(0);
    __builtin_amdgcn_s_waitcnt(0x0F70);           // vmcnt(0): the segments (and X pair 0) have landed
    __builtin_amdgcn_wave_barrier();

    for (int b = 0; b < nbq; b += 2) {
#pragma unroll
        for (int q = 0; q < 8; ++q) { cd[q] = nd[q]; cx[q] = nx[q]; }
        load_x(b + 2);
#pragma unroll
        for (int bb = 0; bb < 2; ++bb) {
            v4ia S[4];
#pragma unroll
            for (int p = 0; p < 4; ++p) {
                // code word h of chunk p of block b + bb, realigned from two LDS dwords
                const int off = r * seg + PQ2_BYTES * (b + bb) + 2 + 8 * p + 4 * h;
                const uint32_t lo = *reinterpret_cast<const uint32_t *>(wl + (off & ~3));
                const uint32_t hi = *reinterpret_cast<const uint32_t *>(wl + (off & ~3) + 4);
                const uint32_t w = __builtin_amdgcn_alignbyte(hi, lo, off & 3);
                v2i Av;
                Av.x = codes_minus_one(w, kk);
                Av.y = codes_minus_one(w, kk + 1);
                S[p] = __builtin_amdgcn_mfma_i32_16x16x32_i8(__builtin_bit_cast(long, Av),
                                                           __builtin_bit_cast(long, cx[4 * bb + p]),
                                                           (v4ia){0, 0, 0, 0}, 0, 0, 0);
            }
            float inner[4];
#pragma unroll
            for (int p = 0; p < 4; ++p) {
                const float da = f16_bits_to_f32(cd[4 * bb + p] & 0xffffu);
#pragma unroll
                for (int i = 0; i < 4; ++i) inner[i] = (p == 0) ? da * (float)S[p][i] : fmaf(da, (float)S[p][i], inner[i]);
            }
            // output rows 4g + i of the 16: their block scale
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t dwb = *reinterpret_cast<const uint16_t *>(wl + (4 * g + i) * seg + PQ2_BYTES * (b + bb));
                acc[i] = fmaf(f16_bits_to_f32(dwb), inner[i], acc[i]);
            }
        }
    }
    // 2. sum the four K quarters
#pragma unroll
    for (int i = 0; i < 4; ++i) red[(wave * 16 + 4 * g + i) * 16 + (lane & 15)] = acc[i];
    __syncthreads();
    if (wave == 0) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int rr = 4 * g + i, col = lane & 15;
            const float v = red[(0 * 16 + rr) * 16 + col] + red[(1 * 16 + rr) * 16 + col] +
                            red[(2 * 16 + rr) * 16 + col] + red[(3 * 16 + rr) * 16 + col];
            const int row = row0 + rr;
            if (row < n_out && col < n_tok) Y[(size_t)row * n_tok + col] = v;
        }
    }
}

// ---------------------------------------------------------------------------
// Small batch, streamed (2 <= n_tok <= 16).  A workgroup owns R = 16 * RT
// weight rows; its KS waves split K into contiguous ranges of pieces of 2
// PQ2_0 blocks (nb even, nb >= 2 KS) and each wave streams its range through a private
// LDS ring of two pieces: a piece is the R row segments of 68 bytes
// (17 dwords, dword DMA) plus the 8 Q8_1 chunks of all n_tok tokens
// (contiguous in the chunk-major X, dwordx4 DMA; NT >= n_tok bounds the
// instruction count, and MFMA columns past n_tok repeat the last token and
// are never stored).  All global reads are LDS DMA, so every wait is an
// explicit vmcnt on this wave's own pieces.
//
// Per chunk: one v_mfma_i32_16x16x32_i8 per 16-row tile with A = the raw
// codes (0..3) of 16 rows, B = the 32 permuted int8 of 16 token columns, and
// the accumulator input C = -s of the lane's token, so the result is exactly
// sum (code - 1) * q.  Lane l holds token l % 16 and rows 4(l/16) + i of the
// tile: the per-token scale is lane-uniform (inner = da * S per chunk), the
// per-row block scale is applied per block.  The KS partial sums meet in LDS.
constexpr int SK_D = 2;                                   // ring depth (pieces)

template <int RT, int KS, int NT>
struct SkinnyCfg {
    static constexpr int R = 16 * RT;
    static constexpr int W_DW = R * 17;                   // weight dwords per piece
    static constexpr int NIW = (W_DW + 63) / 64;
    static constexpr int A_PC = 8 * NT * 9 / 4;           // 16-byte pieces of activation per piece (NT tokens)
    static constexpr int NIA = (A_PC + 63) / 64;
    static constexpr int PER = NIW + NIA;                 // DMA instructions per piece
    static constexpr int W_BYTES = 64 * 4 * NIW;          // LDS bytes (every DMA lane has a slot)
    static constexpr int A_BYTES = 64 * 16 * NIA;
    static constexpr int SLOT = W_BYTES + A_BYTES;
    static constexpr int LDS = KS * SK_D * SLOT;
    static_assert(SK_D * PER < 64, "vmcnt range");
    static_assert(LDS >= KS * R * 16 * 4, "reduction buffer fits in the ring");
};

// DMA of one piece: NIW dword instructions of weights, NIA dwordx4
// instructions of activations.  (A free function: with the two DMA forms
// inside a kernel lambda the host pass drops the kernel's host symbol.)
template <int NIW, int NIA>
__device__ __forceinline__ void small_issue(const uint8_t * wb, const uint32_t * woff,
                                            const uint8_t * xb, const uint32_t * aoff,
                                            uint8_t * dst, int w_bytes) {
#pragma unroll
    for (int k = 0; k < NIW; ++k)
        __builtin_amdgcn_global_load_lds(wb + woff[k], (lds_void *)(dst + 256 * k), 4, 0, 0);
#pragma unroll
    for (int k = 0; k < NIA; ++k)
        __builtin_amdgcn_global_load_lds(xb + aoff[k], (lds_void *)(dst + w_bytes + 1024 * k), 16, 0, 0);
}

template <int RT, int KS, int NT>
__global__ void __launch_bounds__(64 * KS)
gemm_small_kernel(const uint8_t * __restrict__ W, const uint8_t * __restrict__ X,
                  float * __restrict__ Y, int n_out, int n_tok, int nb) {
    using C = SkinnyCfg<RT, KS, NT>;
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    uint8_t * ring = smem + (size_t)wave * SK_D * C::SLOT;
    const int row0 = blockIdx.x * C::R;
    const size_t rs = (size_t)PQ2_BYTES * nb;
    // the nb / 2 pieces of a row are dealt to the KS waves in contiguous
    // ranges that differ by at most one piece
    const int np_all = nb / 2;
    const int pbeg = wave * np_all / KS, pend = (wave + 1) * np_all / KS;
    const int np = pend - pbeg;                             // pieces of this wave (>= 1)
    const int blk0 = 2 * pbeg;

    // per-lane DMA sources of one piece, as offsets from the piece's block
    uint32_t woff[C::NIW];
#pragma unroll
    for (int k = 0; k < C::NIW; ++k) {
        const int idx = min(64 * k + lane, C::W_DW - 1);   // lanes past the piece re-read its last dword
        const int r = idx / 17, d = idx - 17 * r;
        woff[k] = (uint32_t)(min(row0 + r, n_out - 1) * rs + 4 * d);   // W < 4 GiB (host)
    }
    // the 8 chunks of a piece are 8 * n_tok contiguous Q8_1 blocks of the
    // chunk-major X (288 * n_tok bytes, 16-byte aligned): dwordx4 DMA
    const int a_pieces = 18 * n_tok;
    uint32_t aoff[C::NIA];
#pragma unroll
    for (int k = 0; k < C::NIA; ++k) aoff[k] = 16u * (uint32_t)min(64 * k + lane, a_pieces - 1);
    // piece j = blocks blk0 + 2j and blk0 + 2j + 1
#define PQ2_SMALL_ISSUE(j, slot)                                                                   \
    small_issue<C::NIW, C::NIA>(W + (size_t)PQ2_BYTES * (blk0 + 2 * (j)), woff,                      \
                                X + (size_t)4 * (blk0 + 2 * (j)) * n_tok * Q81_BYTES, aoff,          \
                                ring + (slot) * C::SLOT, C::W_BYTES)
#pragma unroll
    for (int i = 0; i < SK_D; ++i) PQ2_SMALL_ISSUE(min(i, np - 1), i);

    const int l16 = lane & 15, g = lane >> 4;
    const int h = g >> 1, pr = 2 * (g & 1);                // code word and first bit pair of K-group g
    float acc[RT][4];
#pragma unroll
    for (int mt = 0; mt < RT; ++mt)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[mt][i] = 0.0f;

    for (int j = 0; j < np; ++j) {
        const int slot = j % SK_D;
        if (j + 1 < np) wait_vmcnt_sk<C::PER>(); else wait_vmcnt_sk<0>();
        __builtin_amdgcn_wave_barrier();
        const uint8_t * wl = ring + slot * C::SLOT;
        const uint8_t * al = wl + C::W_BYTES;
#pragma unroll
        for (int bb = 0; bb < 2; ++bb) {
            // the block's four chunks: every MFMA first (four independent
            // products in flight, their operand reads ahead of them), then
            // the epilogues in chunk order -- one chunk at a time left each
            // MFMA's latency and the LDS round trip before it exposed
            v4ia S[4][RT];
            float da[4];
#pragma unroll
            for (int p = 0; p < 4; ++p) {
                // B: token column l16, K-group g of chunk 4bb + p; scale and -s of that token
                const uint8_t * ab = al + ((4 * bb + p) * n_tok + min(l16, n_tok - 1)) * Q81_BYTES;
                const uint32_t ds = *reinterpret_cast<const uint32_t *>(ab);
                const uint32_t b0 = *reinterpret_cast<const uint32_t *>(ab + 4 + 8 * g);
                const uint32_t b1 = *reinterpret_cast<const uint32_t *>(ab + 8 + 8 * g);
                const int ns = -(int)(int16_t)(ds >> 16);
                da[p] = f16_bits_to_f32(ds & 0xffffu);
                const long Bv = __builtin_bit_cast(long, (v2i){(int)b0, (int)b1});
#pragma unroll
                for (int mt = 0; mt < RT; ++mt) {
                    // code word h of chunk p of block bb for row 16 mt + l16 (2-byte aligned
                    // for bb = 0, dword aligned for bb = 1)
                    const int off = (16 * mt + l16) * 68 + 34 * bb + 2 + 8 * p + 4 * h;
                    uint32_t w;
                    if (bb == 0) {
                        const uint32_t lo = *reinterpret_cast<const uint32_t *>(wl + off - 2);
                        const uint32_t hi = *reinterpret_cast<const uint32_t *>(wl + off + 2);
                        w = __builtin_amdgcn_alignbyte(hi, lo, 2);
                    } else {
                        w = *reinterpret_cast<const uint32_t *>(wl + off);
                    }
                    const long Av = __builtin_bit_cast(long, (v2i){(int)((w >> (2 * pr)) & 0x03030303u),
                                                                  (int)((w >> (2 * pr + 2)) & 0x03030303u)});
                    S[p][mt] = __builtin_amdgcn_mfma_i32_16x16x32_i8(Av, Bv, (v4ia){ns, ns, ns, ns}, 0, 0, 0);
                }
            }
            float inner[RT][4];
#pragma unroll
            for (int p = 0; p < 4; ++p)
#pragma unroll
                for (int mt = 0; mt < RT; ++mt)
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        inner[mt][i] = p == 0 ? da[p] * (float)S[p][mt][i] : fmaf(da[p], (float)S[p][mt][i], inner[mt][i]);
            // pin the block's epilogue here (otherwise the MFMAs of both blocks
            // are hoisted together and converted at the end)
#pragma unroll
            for (int mt = 0; mt < RT; ++mt)
#pragma unroll
                for (int i = 0; i < 4; ++i) asm volatile("" : "+v"(inner[mt][i]));
            __builtin_amdgcn_sched_barrier(0);
            // block scale of output rows 16 mt + 4g + i
#pragma unroll
            for (int mt = 0; mt < RT; ++mt)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const uint32_t dwb = *reinterpret_cast<const uint16_t *>(wl + (16 * mt + 4 * g + i) * 68 + 34 * bb);
                    acc[mt][i] = fmaf(f16_bits_to_f32(dwb), inner[mt][i], acc[mt][i]);
                }
        }
        if (j + SK_D < np) {
            __builtin_amdgcn_s_waitcnt(0xC07F);             // lgkmcnt(0): this slot's reads are done
            __builtin_amdgcn_wave_barrier();
            PQ2_SMALL_ISSUE(j + SK_D, slot);
        }
    }
#undef PQ2_SMALL_ISSUE
    // sum the KS partials of every (row, token) through LDS (the ring is free now)
    __syncthreads();
    float * red = reinterpret_cast<float *>(smem);            // [KS][R][16]
#pragma unroll
    for (int mt = 0; mt < RT; ++mt)
#pragma unroll
        for (int i = 0; i < 4; ++i) red[(wave * C::R + 16 * mt + 4 * g + i) * 16 + l16] = acc[mt][i];
    __syncthreads();
    for (int e = threadIdx.x; e < C::R * 16; e += 64 * KS) {
        const int rr = e >> 4, t = e & 15;
        float v = 0.0f;
#pragma unroll
        for (int q = 0; q < KS; ++q) v += red[(q * C::R + rr) * 16 + t];
        const int row = row0 + rr;
        if (row < n_out && t < n_tok) Y[(size_t)row * n_tok + t] = v;
    }
}

template <int RT, int KS, int NT>
int launch_small_t(const uint8_t * W, const uint8_t * X, float * Y, int n_out, int n_tok, int nb,
                   hipStream_t st) {
    using C = SkinnyCfg<RT, KS, NT>;
    auto kern = gemm_small_kernel<RT, KS, NT>;
    static pq2host::PerDeviceOnce attr;
    pq2host::once_per_device(attr, [&] {
        pq2host::set_max_dynamic_lds(reinterpret_cast<const void *>(kern), C::LDS);
    });
    hipLaunchKernelGGL(kern, dim3((unsigned)cdiv(n_out, C::R)), dim3(64 * KS), C::LDS, st, W, X, Y,
                       n_out, n_tok, nb);
    return (int)hipGetLastError();
}

template <int RT, int KS>
int launch_small_nt(const uint8_t * W, const uint8_t * X, float * Y, int n_out, int n_tok, int nb,
                    hipStream_t st) {
    if (n_tok <= 2) return launch_small_t<RT, KS, 2>(W, X, Y, n_out, n_tok, nb, st);
    if (n_tok <= 4) return launch_small_t<RT, KS, 4>(W, X, Y, n_out, n_tok, nb, st);
    if (n_tok <= 8) return launch_small_t<RT, KS, 8>(W, X, Y, n_out, n_tok, nb, st);
    return launch_small_t<RT, KS, 16>(W, X, Y, n_out, n_tok, nb, st);
}

// ---------------------------------------------------------------------------
// Small batch (3 <= n_tok <= 8) on v_mfma_i32_16x16x64_i8 with a
// block-diagonal B.  The 16 MFMA columns are (token, chunk) pairs, not
// tokens: with NT tokens a 16 x 16 result tile holds CPD = 16 / NT (rounded
// down to 4 or 2) chunks of every token, so no column idles for want of
// tokens and the per-chunk fp32 rescale runs once per 16 x 16 tile instead
// of once per chunk.  One instruction has K = 64 = two chunks: K-group g of
// lane (x, g) carries half g & 1 of chunk 2m + (g >> 1) of the tile; the A
// lane (row x, g) holds those 16 codes (0..3, the code dword's bit pairs k
// = 0..3 as four int8 dwords, (w >> 2k) & 0x03030303), the B lane (column x,
// g) the 16 matching permuted activation bytes -- activation words 4h..4h+3
// of half h line up with the four bit pairs of code dword h byte for byte --
// when column x's chunk is that chunk, and 16 zero bytes otherwise.  A tile
// takes CPD / 2 instructions accumulating into one result, started at -s of
// each column's (token, chunk), so every element is exactly the chunk dot
// sum (code - 1) q.  Lane (x, g) of the result holds rows 4g + i of column
// x: inner += da(column) * S per tile, acc += dw(row, block) * inner per
// block; the CPD columns of a token and the KS K-ranges meet in LDS at the
// end.  Streaming as gemm_small_kernel: R = 16 RT rows per workgroup, K split
// over KS waves in pieces of two blocks, each wave's pieces DMA'd through a
// private two-slot LDS ring (weights and the pieces' NT-token activations).
template <int NT>
struct BdShape {
    static constexpr int CPD = NT <= 4 ? 4 : 2;          // chunks per result tile
    static constexpr int MPD = CPD / 2;                   // instructions per tile
    static constexpr int DPB = 4 / CPD;                   // tiles per block
    static constexpr int ZERO = 2048;                     // zero bytes behind the rings
    static_assert(NT >= 3 && NT <= 8, "token count");
    static_assert((8 - CPD) * NT * Q81_BYTES + 16 <= ZERO, "zero region covers every tile offset");
};

template <int RT, int KS, int NT>
__global__ void __launch_bounds__(64 * KS)
gemm_bd_kernel(const uint8_t * __restrict__ W, const uint8_t * __restrict__ X,
               float * __restrict__ Y, int n_out, int nb) {
    using C = SkinnyCfg<RT, KS, NT>;
    using S = BdShape<NT>;
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    uint8_t * ring = smem + (size_t)wave * SK_D * C::SLOT;
    uint8_t * zero = smem + C::LDS;
    for (int i = threadIdx.x; i < S::ZERO / 16; i += 64 * KS)
        reinterpret_cast<v4ia *>(zero)[i] = (v4ia){0, 0, 0, 0};
    const int row0 = blockIdx.x * C::R;
    const size_t rs = (size_t)PQ2_BYTES * nb;
    const int np_all = nb / 2;
    const int pbeg = wave * np_all / KS, pend = (wave + 1) * np_all / KS;
    const int np = pend - pbeg;                             // pieces of this wave (>= 1)
    const int blk0 = 2 * pbeg;

    uint32_t woff[C::NIW];
#pragma unroll
    for (int k = 0; k < C::NIW; ++k) {
        const int idx = min(64 * k + lane, C::W_DW - 1);   // lanes past the piece re-read its last dword
        const int r = idx / 17, d = idx - 17 * r;
        woff[k] = (uint32_t)(min(row0 + r, n_out - 1) * rs + 4 * d);   // W < 4 GiB (host)
    }
    uint32_t aoff[C::NIA];
#pragma unroll
    for (int k = 0; k < C::NIA; ++k) aoff[k] = 16u * (uint32_t)min(64 * k + lane, C::A_PC - 1);
#define PQ2_BD_ISSUE(j, slot)                                                                      \
    small_issue<C::NIW, C::NIA>(W + (size_t)PQ2_BYTES * (blk0 + 2 * (j)), woff,                      \
                                X + (size_t)4 * (blk0 + 2 * (j)) * NT * Q81_BYTES, aoff,             \
                                ring + (slot) * C::SLOT, C::W_BYTES)
#pragma unroll
    for (int i = 0; i < SK_D; ++i) PQ2_BD_ISSUE(min(i, np - 1), i);
    __syncthreads();                                        // the zero region is written

    const int x = lane & 15, g = lane >> 4;
    const int gq = g >> 1, hh = g & 1;
    const int cc = x / NT, t = x - NT * (x / NT);           // column x = chunk cc of token t
    const bool col_ok = cc < S::CPD;
    const int cce = col_ok ? cc : S::CPD - 1;               // idle columns read a live column's scale
    // slot-relative byte offsets of the lane's B operand (before the tile's
    // chunk offset) and of its column's Q8_1 scale word
    const int b_off = C::W_BYTES + (cc * NT + t) * Q81_BYTES + 4 + 16 * hh;
    const int ds_off = C::W_BYTES + (cce * NT + t) * Q81_BYTES;
    const int a_off = x * 68 + 2 + 8 * gq + 4 * hh;         // code dword of (row x, K-group g), block 0 of the piece
    float acc[RT][4];
#pragma unroll
    for (int mt = 0; mt < RT; ++mt)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[mt][i] = 0.0f;

    for (int j = 0; j < np; ++j) {
        const int slot = j % SK_D;
        if (j + 1 < np) wait_vmcnt_sk<C::PER>(); else wait_vmcnt_sk<0>();
        __builtin_amdgcn_wave_barrier();
        const uint8_t * wl = ring + slot * C::SLOT;
        // instruction m reads real activations only where column x's chunk is
        // the chunk its K-group carries, zeros elsewhere.  The choice is a
        // byte offset from the slot and the read is four dword loads: a
        // 16-byte load at 4-byte alignment, or one through a choice between
        // two pointers, reached the compiler without the alias information
        // that tells it which LDS the load reads, and it then waited for every
        // LDS-DMA in flight -- the next piece's included -- before the read,
        // so no piece streamed beside the arithmetic of the one before it
        const int zrel = (int)(zero - wl);
        int bsrc[S::MPD];
#pragma unroll
        for (int m = 0; m < S::MPD; ++m) bsrc[m] = (col_ok && cc == 2 * m + gq) ? b_off : zrel;
#pragma unroll
        for (int bb = 0; bb < 2; ++bb) {
            float inner[RT][4];
#pragma unroll
            for (int dt = 0; dt < S::DPB; ++dt) {
                const int c0 = 4 * bb + dt * S::CPD;        // first chunk of the tile within the piece
                const uint32_t dsw = *reinterpret_cast<const uint32_t *>(wl + ds_off + c0 * NT * Q81_BYTES);
                const int ns = -(int)(int16_t)(dsw >> 16);
                const float da = f16_bits_to_f32(dsw & 0xffffu);
                v4ia Dt[RT];
#pragma unroll
                for (int mt = 0; mt < RT; ++mt) Dt[mt] = (v4ia){ns, ns, ns, ns};
#pragma unroll
                for (int m = 0; m < S::MPD; ++m) {
                    const int * bp = reinterpret_cast<const int *>(wl + bsrc[m] + c0 * NT * Q81_BYTES);
                    const v4ia Bv = {bp[0], bp[1], bp[2], bp[3]};
#pragma unroll
                    for (int mt = 0; mt < RT; ++mt) {
                        // code dword: chunk c0 + 2m + gq, half hh, row 16 mt + x (2-byte aligned in block 0)
                        const int off = a_off + 16 * mt * 68 + 34 * bb + 8 * (dt * S::CPD + 2 * m);
                        uint32_t w;
                        if (bb == 0) {
                            const uint32_t lo = *reinterpret_cast<const uint32_t *>(wl + off - 2);
                            const uint32_t hi = *reinterpret_cast<const uint32_t *>(wl + off + 2);
                            w = __builtin_amdgcn_alignbyte(hi, lo, 2);
                        } else {
                            w = *reinterpret_cast<const uint32_t *>(wl + off);
                        }
                        const v4ia Av = {(int)(w & 0x03030303u), (int)((w >> 2) & 0x03030303u),
                                         (int)((w >> 4) & 0x03030303u), (int)((w >> 6) & 0x03030303u)};
                        Dt[mt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(Av, Bv, Dt[mt], 0, 0, 0);
                    }
                }
#pragma unroll
                for (int mt = 0; mt < RT; ++mt)
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        inner[mt][i] = dt == 0 ? da * (float)Dt[mt][i] : fmaf(da, (float)Dt[mt][i], inner[mt][i]);
            }
            // block scale of rows 16 mt + 4g + i
#pragma unroll
            for (int mt = 0; mt < RT; ++mt)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const uint32_t dwb = *reinterpret_cast<const uint16_t *>(wl + (16 * mt + 4 * g + i) * 68 + 34 * bb);
                    acc[mt][i] = fmaf(f16_bits_to_f32(dwb), inner[mt][i], acc[mt][i]);
                }
        }
        if (j + SK_D < np) {
            __builtin_amdgcn_s_waitcnt(0xC07F);             // lgkmcnt(0): this slot's reads are done
            __builtin_amdgcn_wave_barrier();
            PQ2_BD_ISSUE(j + SK_D, slot);
        }
    }
#undef PQ2_BD_ISSUE
    // sum the CPD columns of every token and the KS K-ranges through LDS
    __syncthreads();
    float * red = reinterpret_cast<float *>(smem);            // [KS][R][16]
#pragma unroll
    for (int mt = 0; mt < RT; ++mt)
#pragma unroll
        for (int i = 0; i < 4; ++i) red[(wave * C::R + 16 * mt + 4 * g + i) * 16 + x] = acc[mt][i];
    __syncthreads();
    for (int e = threadIdx.x; e < C::R * NT; e += 64 * KS) {
        const int rr = e / NT, tt = e - NT * (e / NT);
        float v = 0.0f;
#pragma unroll
        for (int q = 0; q < KS; ++q)
#pragma unroll
            for (int k = 0; k < S::CPD; ++k) v += red[(q * C::R + rr) * 16 + k * NT + tt];
        const int row = row0 + rr;
        if (row < n_out) Y[(size_t)row * NT + tt] = v;
    }
}

template <int RT, int KS, int NT>
int launch_bd_t(const uint8_t * W, const uint8_t * X, float * Y, int n_out, int nb, hipStream_t st) {
    using C = SkinnyCfg<RT, KS, NT>;
    constexpr int lds = C::LDS + BdShape<NT>::ZERO;
    auto kern = gemm_bd_kernel<RT, KS, NT>;
    static pq2host::PerDeviceOnce attr;
    pq2host::once_per_device(attr, [&] {
        pq2host::set_max_dynamic_lds(reinterpret_cast<const void *>(kern), lds);
    });
    hipLaunchKernelGGL(kern, dim3((unsigned)cdiv(n_out, C::R)), dim3(64 * KS), lds, st, W, X, Y, n_out, nb);
    return (int)hipGetLastError();
}

template <int RT, int KS>
int launch_bd_nt(const uint8_t * W, const uint8_t * X, float * Y, int n_out, int n_tok, int nb, hipStream_t st) {
    switch (n_tok) {
        case 3: return launch_bd_t<RT, KS, 3>(W, X, Y, n_out, nb, st);
        case 4: return launch_bd_t<RT, KS, 4>(W, X, Y, n_out, nb, st);
        case 5: return launch_bd_t<RT, KS, 5>(W, X, Y, n_out, nb, st);
        case 6: return launch_bd_t<RT, KS, 6>(W, X, Y, n_out, nb, st);
        case 7: return launch_bd_t<RT, KS, 7>(W, X, Y, n_out, nb, st);
        case 8: return launch_bd_t<RT, KS, 8>(W, X, Y, n_out, nb, st);
        default: return -1;
    }
}

// Workgroup shape of the block-diagonal kernel, 0 where another small-batch
// kernel is faster.  Measured on MI355X (us, HIP-graph replay; previous path
// = 4x4x4 MFMA kernel for 3..4 tokens on its widths, 16x16x32 kernel else):
//                 previous  16 rows/8 ways  16/4  32/4  32/8
//   17408x5120 B3   11.56     10.81        11.83 12.45 13.78
//              B4   10.92     13.78        11.82 12.63 14.00
//              B5   15.57     14.21        12.56 13.66 14.78
//              B8   15.86     15.51        14.87 14.42 19.68
//   5120x17408 B3   16.02     13.85        17.44 19.16 14.59
//              B4   17.16     14.48        17.39 19.21 14.54
//              B5   18.03     15.43        17.44 20.24 15.24
//              B8   18.78     17.15        18.64 20.11 15.74
//   6144x5120  B5    7.72      6.81         7.36  8.38  7.48
//              B8    8.16      7.31         7.93  8.50  7.93
//   5120x6144  B3    6.61      7.15         7.82  8.48  7.55
//              B4    6.76      7.49         7.95  8.67  7.72
//              B5    8.70      7.86         8.25  9.31  8.18
//              B8    8.94      8.48         8.62  9.20  8.37
// (1 = 16 rows / K in 8, 2 = 16 / 4, 3 = 32 / 4, 4 = 32 / 8, 5 = 16 / 2).
// 16 rows with K in 2 (about 19 KB of LDS: 8 workgroups per CU) wins where
// all its workgroups are resident at once, at 6..8 tokens (us, 32/4 or 16/4
// -> 16/2): 17408x5120 B8 14.12 -> 13.10, B6 13.55 -> 12.33, B5 12.34 ->
// 12.29; with 34816 rows (a second round) 20.92 -> 23.67; at 6144x5120 B8
// (7.28 -> 10.69) and 5120x17408 B8 (15.43 -> 30.60) the shapes above stay.
int bd_choice(int nb, int64_t n_out, int64_t n_tok, int cus) {
    if (n_tok < 3 || n_tok > 8) return 0;
    const bool mfma4_width = nb == 8 || nb == 40 || nb == 48;
    if (mfma4_width && (n_tok == 4 || (n_tok == 3 && nb != 40))) return 0;
    // the 17408-column rows: 16 rows, K in 8 (µs, with the pieces streaming
    // beside the arithmetic, 5120x17408, this choice / 32 rows, K in 8):
    // B5 14.87 / 15.43, B6 15.24 / 15.58, B7 15.61 / 15.89, B8 16.20 / 16.31
    if (nb >= 96) return 1;
    if (n_out >= 12288 && n_tok >= 6 && (n_out + 15) / 16 <= 8 * (int64_t)cus) return 5;
    if (n_out >= 12288 && n_tok >= 5) return n_tok >= 7 ? 3 : 2;
    return 1;
}

template <int WM, int WN, int TM, int TN>
void launch_gemm(const uint8_t * W, const uint8_t * X, float * Y, int n_out, int n_tok, int nb,
                 hipStream_t st) {
    using C = GemmCfg<WM, WN, TM, TN>;
    dim3 grid((unsigned)cdiv(n_out, C::BM), (unsigned)cdiv(n_tok, C::BN));
    hipLaunchKernelGGL((gemm_mfma_kernel<WM, WN, TM, TN>), grid, dim3(C::THREADS), 0, st, W, X, Y,
                       n_out, n_tok, nb);
}

using pq2host::knob;

int gemm_cu_count() { return pq2host::device_info().cus; }

// LDS limit of the skinny kernel on the current device (its dynamic-LDS
// attribute raised to the device maximum once per device)
int skinny_lds_limit() {
    const int v = pq2host::device_info().max_lds;
    static pq2host::PerDeviceOnce attr;
    pq2host::once_per_device(attr, [v] {
        pq2host::set_max_dynamic_lds(reinterpret_cast<const void *>(gemm_skinny_kernel), v);
    });
    return v;
}

// ---------------------------------------------------------------------------
// f16-MFMA prefill GEMM.  v_mfma_f32_16x16x32_f16 with A = (code - 1) * dw
// and B = q as f16: (code - 1) * dw is exact in f16 (code - 1 is -1, 0, 1 or
// 2), q is a small integer, every product is exact in fp32 and every partial
// sum is dw times an integer of at most 13 bits (|S| <= 8128), so each MFMA
// returns dw * S exactly.  The per-chunk activation scale then costs one FMA
// per output element (the int8 MFMA needs a convert and an FMA), and the
// weight scale nothing beyond one packed f16 multiply per two staged codes.
//
// Workgroup: tile 128 rows x 128 tokens, 1024 threads (16 waves as 4 x 4, 4
// per SIMD; a wave owns 32 rows x 32 tokens = 2 x 2 MFMA tiles of 16 x 16) or
// 512 (8 waves as 2 x 4, 64 x 32 each).  Per PQ2_0 block (K = 128) the
// workgroup converts the tile's codes and Q8_1 bytes to f16 once, into LDS
// laid out [chunk][row or token][32 positions] with the four 16-byte groups
// of a row swizzled by (row / 4) % 4 (conflict-free ds_read_b128 of the MFMA
// operands); the next block's raw bytes are loaded into registers while the
// current block is computed, and two LDS stages need one barrier per block.
//
// A block scale with |dw| >= 32768 would overflow f16 at code 3 (2 dw): such
// a block is staged as dw / 2 (exact there) and the workgroup repeats the
// main loop once with every other block's scale set to 0, adding the second
// half -- a second pass only for workgroups that meet such a scale.
//
// f16 conversions (exact):
//  * code c -> f16(c - 1): v_perm picks the high byte from the table
//    {0xBC, 0x00, 0x3C, 0x40} (f16 -1, 0, 1, 2 have zero low bytes), two more
//    v_perm spread 4 high bytes into 4 halves;
//  * q -> f16(q): v_perm builds the halves 0x6400 + (q + 128) (= 1024 + q +
//    128), a packed f16 add of -1152 leaves q.
constexpr int GF_BM = 128;
constexpr int GF_STAGE_A = 4 * GF_BM * 64;          // bytes: [4 chunks][BM rows][64 B]

typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 v2h __attribute__((ext_vector_type(2)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef uint32_t v4u __attribute__((ext_vector_type(4)));

__device__ __forceinline__ void codes4_to_f16(uint32_t c4, uint32_t & lo, uint32_t & hi) {
    const uint32_t hb = __builtin_amdgcn_perm(0u, 0x403C00BCu, c4);   // byte i = table[c_i]
    lo = __builtin_amdgcn_perm(hb, 0u, 0x050C040Cu);                   // {0, hb0, 0, hb1}
    hi = __builtin_amdgcn_perm(hb, 0u, 0x070C060Cu);                   // {0, hb2, 0, hb3}
}

__device__ __forceinline__ uint32_t sub1152_f16x2(uint32_t x) {
    const v2h r = __builtin_bit_cast(v2h, x) + (v2h){(_Float16)-1152.0f, (_Float16)-1152.0f};
    return __builtin_bit_cast(uint32_t, r);
}

__device__ __forceinline__ uint32_t mul_f16x2(uint32_t a, uint32_t b) {
    const v2h r = __builtin_bit_cast(v2h, a) * __builtin_bit_cast(v2h, b);
    return __builtin_bit_cast(uint32_t, r);
}

__device__ __forceinline__ void q4_to_f16(uint32_t q4, uint32_t & lo, uint32_t & hi) {
    const uint32_t x = q4 ^ 0x80808080u;                               // q + 128 per byte
    lo = sub1152_f16x2(__builtin_amdgcn_perm(x, 0x64646464u, 0x00050004u));
    hi = sub1152_f16x2(__builtin_amdgcn_perm(x, 0x64646464u, 0x00070006u));
}

// Byte offset of the 16-byte group g of row r in a [rows][64 B] tile.  The
// group is XOR-swizzled by ((r >> 1) ^ (r >> 2)) & 3 so that 16-byte accesses
// of consecutive rows at one g hit distinct banks both with 32 banks (8
// lanes per cycle) and with 64 banks (16 lanes per cycle).
__device__ __forceinline__ int gf_swz(int r, int g) { return r * 64 + ((g ^ ((r >> 1) ^ (r >> 2))) & 3) * 16; }

// WM x WN waves, each owning MI x NI MFMA tiles of 16 x 16; the workgroup
// tile is 128 rows x BN tokens (BN = 128, or 64 where the 128-token tiles
// leave CUs idle).  With 512 threads (BN = 128) every thread stages one A item
// and one B item per block; with 1024 threads (4 waves per SIMD, for latency
// hiding) waves 0-7 stage A items, the next BN / 16 waves B items, and the
// rest only compute.
template <int WM, int WN, int MI, int NI, int BN = 128>
__global__ void __launch_bounds__(64 * WM * WN)
gemm_f16_kernel(const uint8_t * __restrict__ W, const uint8_t * __restrict__ X,
                float * __restrict__ Y, int n_out, int n_tok, int nb) {
    constexpr int THREADS = 64 * WM * WN;
    constexpr int GF_BN = BN;
    constexpr int GF_STAGE_B = 4 * BN * 64;
    static_assert(16 * MI * WM == GF_BM && 16 * NI * WN == GF_BN, "workgroup tile");
    static_assert(THREADS == 512 || THREADS == 1024, "staging roles");
    static_assert(BN == 128 || (BN == 64 && THREADS == 1024), "token tile");
    constexpr bool SPLIT = THREADS == 1024;
    __shared__ __attribute__((aligned(16))) uint8_t sA[2][GF_STAGE_A];
    __shared__ __attribute__((aligned(16))) uint8_t sB[2][GF_STAGE_B];
    __shared__ __attribute__((aligned(16))) float sDa[2][4][GF_BN];
    // set when a staged block scale was halved (below): the workgroup then
    // runs a second pass over the halved blocks only
    __shared__ int sHasBig;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave % WM, wn = wave / WM;
    const int row0 = blockIdx.x * GF_BM, tok0 = blockIdx.y * GF_BN;
    const int l16 = lane & 15, g = lane >> 4;
    const size_t rs = (size_t)PQ2_BYTES * nb;                  // bytes per weight row
    const size_t w_bytes = rs * (size_t)n_out;

    // staging roles: A item (row ar, chunk ap), B item (token bt, chunk bp);
    // LDS writes of a wave cover consecutive rows / tokens of one chunk
    const int it = tid & 511;
    const int ar = it & 127, ap = it >> 7;                     // a wave stages 64 consecutive rows
    const int bp = it / BN, bt = it % BN;

    float acc[MI][NI][4];
#pragma unroll
    for (int mi = 0; mi < MI; ++mi)
#pragma unroll
        for (int ni = 0; ni < NI; ++ni)
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[mi][ni][i] = 0.0f;

    // the staging and main loop, specialised on the thread's staging roles
    // (runtime role branches around the raw registers make the compiler keep
    // them in scratch)
    auto main_loop = [&](auto role_a, auto role_b) __attribute__((always_inline)) {
    constexpr bool do_a = decltype(role_a)::value;
    constexpr bool do_b = decltype(role_b)::value;
    for (int pass = 0; pass < 2; ++pass) {
    if (pass == 1) {                                           // rare: some |dw| >= 32768
        __syncthreads();
        if (!sHasBig) break;
    }
    // raw bytes of one block held in registers between its global load and
    // its conversion into LDS; two sets, so a block's loads are issued two
    // block-steps before they are consumed.  A: words 0-2 = 3-dword window
    // over the 8 code bytes, word 3 = block scale; B: one Q8_1 block (9
    // words), after A's words unless a thread stages only one of them.
    constexpr int QB = do_a ? 4 : 0;
    struct Raw {
        uint32_t w[QB + 9];
        uint32_t sh;                                           // A: shift, bit 2 tail, bit 3 block in range
    };
    // byte offsets into W (kept as offsets so the loads stay global, not flat)
    const size_t w_align = (uintptr_t)W & 3;
    size_t a_off = (size_t)min(row0 + ar, n_out - 1) * rs + 2 + 8 * ap;   // chunk ap of block 0
    const uint8_t * b_ptr = X + ((size_t)bp * n_tok + min(tok0 + bt, n_tok - 1)) * Q81_BYTES;
    const size_t b_step = (size_t)4 * n_tok * Q81_BYTES;
    int pf_block = 0;                                          // block the next prefetch reads
    // Loads are unconditional (rows / tokens past the edge re-read the last
    // one, the conversion zeroes them) so the compiler can count them: the
    // wait before a conversion then leaves the younger block's loads in flight.
    auto prefetch = [&](Raw & r) {                             // the next block in order (the last block again past the end)
        if constexpr (do_a) {
            // dword-aligned window (in absolute address terms) over the 8 code bytes
            const size_t aa = ((a_off + w_align) & ~(size_t)3) - w_align;
            r.sh = (uint32_t)((a_off + w_align) & 3);
            r.w[0] = *reinterpret_cast<const uint32_t *>(W + aa);
            r.w[1] = *reinterpret_cast<const uint32_t *>(W + aa + 4);
            // the window may end past W when its last chunk is the matrix's last.
            // Shift 2: the code bytes end 2 bytes into the third dword, so read
            // the dword ending at W's end and shift (flag in sh bit 2).  Shift 0:
            // the third dword is not used (alignbyte by 0 keeps w[1]), so re-read
            // the second one.  Every dword read lies in [0, w_bytes).
            const bool tail = aa + 12 > w_bytes;
            r.w[2] = *reinterpret_cast<const uint32_t *>(W + (tail ? (r.sh ? aa + 6 : aa + 4) : aa + 8));
            r.sh |= (tail ? 4u : 0u) | (pf_block < nb ? 8u : 0u);
            r.w[3] = (uint32_t)*reinterpret_cast<const uint16_t *>(W + a_off - 2 - 8 * ap);   // block scale
        }
        if constexpr (!do_a) {
            r.sh = pf_block < nb ? 8u : 0u;
        }
        if constexpr (do_b) {
            const uint32_t * xb = reinterpret_cast<const uint32_t *>(b_ptr);
#pragma unroll
            for (int k = 0; k < 9; ++k) r.w[QB + k] = xb[k];
        }
        if (++pf_block < nb) {
            a_off += PQ2_BYTES;
            b_ptr += b_step;
        }
    };
    // Conversion of one block's raw bytes into LDS stage st, in four parts
    // (part q writes 16-byte group q of every A and B row) so that it can be
    // interleaved with the four chunk steps of the current block.
    uint32_t cw0 = 0, cw1 = 0;                                 // realigned code words
    uint32_t dw2 = 0;                                          // the row's block scale, f16 x 2
    auto commit_part = [&](const Raw & r, int st, int q) {
        // a block past the end (the padding step of an odd block count) gets
        // zero scales, so its products add exactly nothing
        const bool live = (r.sh & 8u) != 0;
        uint32_t o0, o1, o2, o3;
        if constexpr (do_a) {
            if (q == 0) {
                const uint32_t sh = r.sh & 3u;
                const uint32_t a2 = (r.sh & 4u) ? (r.w[2] >> 16) : r.w[2];
                // rows past n_out (re-reading the last row) only reach their
                // own outputs, which are not stored
                cw0 = __builtin_amdgcn_alignbyte(r.w[1], r.w[0], sh);
                cw1 = __builtin_amdgcn_alignbyte(a2, r.w[1], sh);
                // the weight scale rides in A: (code - 1) * dw is exact in f16
                // (code - 1 is -1, 0, 1 or 2); a dead row or block gets scale 0.
                // 2 * dw overflows f16 for |dw| >= 32768 (exponent field 30):
                // such a block is staged with dw / 2 (exact there), which adds
                // half of its
                // contributions, once in the first pass and once more in a
                // second pass that stages only those blocks (dw = 0 elsewhere)
                uint32_t dwh = live ? (r.w[3] & 0xffffu) : 0u;
                const bool big = (dwh & 0x7C00u) == 0x7800u;
                dwh -= big ? 0x400u : 0u;
                dwh = (pass == 0 || big) ? dwh : 0u;
                dw2 = dwh | (dwh << 16);
                if (big) sHasBig = 1;
            }
            const uint32_t w = q < 2 ? cw0 : cw1;
            const int k0 = 2 * (q & 1);                        // bit pair of position 8q
            codes4_to_f16((w >> (2 * k0)) & 0x03030303u, o0, o1);
            codes4_to_f16((w >> (2 * k0 + 2)) & 0x03030303u, o2, o3);
            o0 = mul_f16x2(o0, dw2); o1 = mul_f16x2(o1, dw2); o2 = mul_f16x2(o2, dw2); o3 = mul_f16x2(o3, dw2);
            *reinterpret_cast<v4u *>(&sA[st][ap * GF_BM * 64] + gf_swz(ar, q)) = (v4u){o0, o1, o2, o3};
        }
        if constexpr (do_b) {
            // tokens past n_tok (re-reading the last token) only reach their
            // own output columns, which are not stored
            if (q == 0) sDa[st][bp][bt] = live ? f16_bits_to_f32(r.w[QB] & 0xffffu) : 0.0f;
            q4_to_f16(r.w[QB + 1 + 2 * q], o0, o1);
            q4_to_f16(r.w[QB + 2 + 2 * q], o2, o3);
            *reinterpret_cast<v4u *>(&sB[st][bp * GF_BN * 64] + gf_swz(bt, q)) = (v4u){o0, o1, o2, o3};
        }
    };
    auto commit = [&](const Raw & r, int st) {
#pragma unroll
        for (int q = 0; q < 4; ++q) commit_part(r, st, q);
    };

    Raw raw0, raw1;
    prefetch(raw0);
    prefetch(raw1);
    commit(raw0, 0);
    __syncthreads();
    // step b: issue block b+2's loads into the set block b used, compute block
    // b from LDS stage b&1, convert block b+1 (loaded a step earlier) into the
    // other stage.  Every step issues and converts unconditionally (past the
    // end it re-reads the last block and fills the unused stage), so the
    // compiler's wait before the conversion leaves the younger loads in flight.
    auto step = [&](int b, Raw & mine, Raw & next) {
        const int st = b & 1;
        prefetch(mine);
        // chunk pipeline: the MFMAs of chunk p+1 are issued before the epilogue
        // of chunk p, and a quarter of the next block's conversion follows each
        // epilogue, so VALU work runs while the matrix core is busy
        v4f S[2][MI][NI];
        float da[2][NI];
        auto issue = [&](int p) {
            const uint8_t * a_src = &sA[st][p * GF_BM * 64];
            const uint8_t * b_src = &sB[st][p * GF_BN * 64];
            v8h A[MI], Bf[NI];
#pragma unroll
            for (int mi = 0; mi < MI; ++mi)
                A[mi] = *reinterpret_cast<const v8h *>(a_src + gf_swz(wm * 16 * MI + 16 * mi + l16, g));
#pragma unroll
            for (int ni = 0; ni < NI; ++ni) {
                const int tt = wn * 16 * NI + 16 * ni + l16;
                Bf[ni] = *reinterpret_cast<const v8h *>(b_src + gf_swz(tt, g));
                da[p & 1][ni] = sDa[st][p][tt];
            }
#pragma unroll
            for (int mi = 0; mi < MI; ++mi)
#pragma unroll
                for (int ni = 0; ni < NI; ++ni)
                    S[p & 1][mi][ni] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[mi], Bf[ni], (v4f){0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
        };
        auto epilogue = [&](int p) {
#pragma unroll
            for (int mi = 0; mi < MI; ++mi)
#pragma unroll
                for (int ni = 0; ni < NI; ++ni)
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        acc[mi][ni][i] = fmaf(da[p & 1][ni], S[p & 1][mi][ni][i], acc[mi][ni][i]);
            // pin the chunk's epilogue here: without it the compiler sinks all
            // the FMAs below the last MFMA and keeps every result live
#pragma unroll
            for (int mi = 0; mi < MI; ++mi)
#pragma unroll
                for (int ni = 0; ni < NI; ++ni)
#pragma unroll
                    for (int i = 0; i < 4; ++i) asm volatile("" : "+v"(acc[mi][ni][i]));
        };
        // the conversion of the next block runs at raised wave priority: the
        // barrier below waits for the last wave's conversion, so the arbiter
        // serves it ahead of other waves' MFMA and epilogue work (MI355X, one
        // process, min us, default -> raised: 17408x5120 M = 2048 545 -> 522,
        // 5120x17408 M = 2048 549 -> 534, M = 512 198 -> 180; priorities 1, 2
        // and 3 measured alike; raising the MFMA phase instead moved nothing)
        issue(0);
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            __builtin_amdgcn_s_setprio(0);
            if (p < 3) issue(p + 1);
            __builtin_amdgcn_sched_barrier(0);
            epilogue(p);
            __builtin_amdgcn_sched_barrier(0);
            __builtin_amdgcn_s_setprio(1);
            commit_part(next, st ^ 1, p);
            __builtin_amdgcn_sched_barrier(0);
        }
        __builtin_amdgcn_s_setprio(0);
        __syncthreads();
    };

    // register sets alternate; an odd block count runs one padding step whose
    // scales are zero
    for (int b = 0; b < nb; b += 2) {
        step(b, raw0, raw1);
        step(b + 1, raw1, raw0);
    }
    }
    };
    using yes = std::integral_constant<bool, true>;
    using no = std::integral_constant<bool, false>;
    if (tid == 0) sHasBig = 0;
    __syncthreads();
    if constexpr (!SPLIT) main_loop(yes{}, yes{});
    else if (wave < 8) main_loop(yes{}, no{});
    else if (wave < 8 + BN / 16) main_loop(no{}, yes{});
    else main_loop(no{}, no{});
#pragma unroll
    for (int mi = 0; mi < MI; ++mi)
#pragma unroll
        for (int ni = 0; ni < NI; ++ni) {
            const int tok = tok0 + wn * 16 * NI + 16 * ni + l16;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int row = row0 + wm * 16 * MI + 16 * mi + 4 * g + i;
                if (row < n_out && tok < n_tok) Y[(size_t)row * n_tok + tok] = acc[mi][ni][i];
            }
        }
}

// The 128-row f16 prefill kernel (gemm_f16_kernel) over rows [0, n_out) of w / Y.
int gemm_prefill_f16(const uint8_t * w, const uint8_t * x, float * Y, int64_t n_out, int64_t n_tok, int nb,
                     hipStream_t st) {
    // 16 waves (4 per SIMD, 32 x 32 wave tiles) measured 12-22 % faster than
    // 8 waves (2 per SIMD, 64 x 32) on every prefill shape: the latency of
    // the chunk pipeline and the per-block barrier is hidden by more waves.
    // One workgroup fits a CU: where even twice the 128-token tiles fit in
    // one round, 64-token tiles put twice the CUs to work (6144x5120 at
    // M = 256: 61 -> 42 us); past that the extra round costs more than the
    // idle CUs (5120x17408 at M = 512: 200 -> 256 us), so 128.
    const int64_t tiles128 = cdiv(n_out, GF_BM) * cdiv(n_tok, 128);
    int bn = knob(pq2host::K_GEMM_F16_BN, 0);
    if (bn != 64 && bn != 128) bn = 2 * tiles128 <= gemm_cu_count() ? 64 : 128;
    // A last round that only part-fills the CUs (17408 rows at M = 512:
    // 544 tiles = 2 rounds + 32 tiles) costs a whole round.  Where the
    // full rounds cover whole row tiles, they run as one launch and the
    // remaining rows as a second launch of 64-token tiles, which spreads
    // them over more CUs (twice the tiles, each about half the work).
    const int cus = gemm_cu_count();
    const int64_t ttok = cdiv(n_tok, 128), rounds = tiles128 / cus, rest = tiles128 - rounds * cus;
    if (bn == 128 && rounds >= 1 && rest > 0 && 2 * rest <= cus && (rounds * cus) % ttok == 0 &&
        knob(pq2host::K_GEMM_F16_SPLIT, 1) > 0 && knob(pq2host::K_GEMM_F16_WAVES, 16) != 8) {
        const int64_t rows_main = rounds * cus / ttok * GF_BM;
        const int64_t rows_tail = n_out - rows_main;
        if (rows_tail > 0 && cdiv(rows_tail, GF_BM) * cdiv(n_tok, 64) <= cus) {
            hipLaunchKernelGGL((gemm_f16_kernel<4, 4, 2, 2>), dim3((unsigned)(rows_main / GF_BM), (unsigned)ttok),
                               dim3(1024), 0, st, w, x, Y, (int)rows_main, (int)n_tok, nb);
            hipLaunchKernelGGL((gemm_f16_kernel<4, 4, 2, 1, 64>),
                               dim3((unsigned)cdiv(rows_tail, GF_BM), (unsigned)cdiv(n_tok, 64)), dim3(1024), 0,
                               st, w + (size_t)rows_main * PQ2_BYTES * nb, x, Y + (size_t)rows_main * n_tok,
                               (int)rows_tail, (int)n_tok, nb);
            return (int)hipGetLastError();
        }
    }
    const dim3 grid((unsigned)cdiv(n_out, GF_BM), (unsigned)cdiv(n_tok, bn));
    if (knob(pq2host::K_GEMM_F16_WAVES, 16) == 8)
        hipLaunchKernelGGL((gemm_f16_kernel<2, 4, 4, 2>), dim3(grid.x, (unsigned)cdiv(n_tok, 128)), dim3(512),
                           0, st, w, x, Y, (int)n_out, (int)n_tok, nb);
    else if (bn == 64)
        hipLaunchKernelGGL((gemm_f16_kernel<4, 4, 2, 1, 64>), grid, dim3(1024), 0, st, w, x, Y, (int)n_out,
                           (int)n_tok, nb);
    else
        hipLaunchKernelGGL((gemm_f16_kernel<4, 4, 2, 2>), grid, dim3(1024), 0, st, w, x, Y, (int)n_out, (int)n_tok, nb);
    return (int)hipGetLastError();
}

}  // namespace

namespace pq2 {
// gemv.hip: 2..4 tokens on the streaming kernels; -1 if not applicable
int gemv_small_batch(const void * W, const void * Xq, float * Y, int64_t n_out, int64_t n_in,
                     int64_t n_tok, bonsai_stream stream);
// gemm_wide.hip: rows [0, rows) that the wide kernel takes (0: none) and its launch
int64_t gemm_wide_rows(const void * W, const void * Xq, int64_t n_out, int64_t n_tok, int nb, int cus, bool force,
                       int * mi);
int gemm_wide_launch(const void * W, const void * Xq, float * Y, int64_t n_out, int64_t n_tok, int nb, int mi,
                     hipStream_t st);
int64_t gemm_wide_x16_bytes(int64_t n_tok, int nb);
int gemm_wide_launch_ws(const void * W, const void * Xq, float * Y, int64_t n_out, int64_t n_tok, int nb, int mi,
                        void * ws, hipStream_t st);
}

namespace {

// bonsai_p40_gemm's dispatch; ws (non-NULL: large enough and aligned, checked
// by the caller) lets the long-prompt kernel take the activation by DMA
int gemm_dispatch(const void * W, const void * Xq, float * Y, int64_t n_out, int64_t n_in, int64_t n_tok,
                  void * ws, bonsai_stream stream) {
    if (n_in <= 0 || n_in % QK_PQ2 != 0) return 1;
    if (n_out <= 0 || n_tok <= 0) return 0;
    if (((uintptr_t)Xq & 3u) != 0 || ((uintptr_t)W & 1u) != 0 || pq2host::any_null(W, Xq, Y)) return 1;
    if (n_out > 0x7fffffff || n_tok > 0x7fffffff || n_in / QK_PQ2 > (1 << 24)) return 1;
    const int nb = (int)(n_in / QK_PQ2);
    hipStream_t st = (hipStream_t)stream;
    const uint8_t * w = (const uint8_t *)W;
    const uint8_t * x = (const uint8_t *)Xq;
    if (n_tok == 1) return bonsai_p40_gemv(W, Xq, Y, n_out, n_in, stream);   // chunk-major == token-major
    // the block-diagonal and streamed small-batch kernels address W with
    // 32-bit per-lane offsets: a matrix of 4 GiB or more takes the kernels
    // below them, which use 64-bit offsets
    const bool off32 = (uint64_t)n_out * PQ2_BYTES * (uint64_t)nb < (1ull << 32);
    const int bd_cfg = knob(pq2host::K_GEMM_BD, -1) < 0 ? bd_choice(nb, n_out, n_tok, gemm_cu_count())
                                                              : knob(pq2host::K_GEMM_BD, 0);
    if (off32 && bd_cfg > 0 && n_tok >= 3 && n_tok <= 8 && nb % 2 == 0 && nb >= 16 && ((uintptr_t)W & 3u) == 0 &&
        ((uintptr_t)Xq & 15u) == 0) {
        switch (bd_cfg) {
            case 2: return launch_bd_nt<1, 4>(w, x, Y, (int)n_out, (int)n_tok, nb, st);
            case 3: return launch_bd_nt<2, 4>(w, x, Y, (int)n_out, (int)n_tok, nb, st);
            case 4: return launch_bd_nt<2, 8>(w, x, Y, (int)n_out, (int)n_tok, nb, st);
            case 5: return launch_bd_nt<1, 2>(w, x, Y, (int)n_out, (int)n_tok, nb, st);
            default: return launch_bd_nt<1, 8>(w, x, Y, (int)n_out, (int)n_tok, nb, st);
        }
    }
    if (n_tok <= 4) {
        const int rc = pq2::gemv_small_batch(W, Xq, Y, n_out, n_in, n_tok, stream);
        if (rc >= 0) return rc;
    }
    const size_t skinny_lds = (size_t)4 * 16 * PQ2_BYTES * (nb / 4) + 4096;
    const int small_sel = knob(pq2host::K_GEMM_SMALL, 0);   // 0 streamed, 1 previous kernel
    if (off32 && n_tok <= 16 && small_sel == 0 && nb % 2 == 0 && nb >= 8 && ((uintptr_t)W & 3u) == 0 &&
        ((uintptr_t)Xq & 15u) == 0) {
        switch (knob(pq2host::K_GEMM_SMALL_CFG, 0)) {
            case 1: return launch_small_nt<1, 4>(w, x, Y, (int)n_out, (int)n_tok, nb, st);
            case 2: return launch_small_nt<2, 4>(w, x, Y, (int)n_out, (int)n_tok, nb, st);
            case 3: return launch_small_nt<4, 4>(w, x, Y, (int)n_out, (int)n_tok, nb, st);
            case 4: return launch_small_nt<1, 2>(w, x, Y, (int)n_out, (int)n_tok, nb, st);
            case 5: return launch_small_nt<2, 2>(w, x, Y, (int)n_out, (int)n_tok, nb, st);
            case 6: return launch_small_nt<4, 2>(w, x, Y, (int)n_out, (int)n_tok, nb, st);
            case 7: return launch_small_nt<1, 8>(w, x, Y, (int)n_out, (int)n_tok, nb, st);
            case 8: return launch_small_nt<1, 16>(w, x, Y, (int)n_out, (int)n_tok, nb, st);
            default: break;
        }
        // measured on MI355X: 16-row workgroups; K split 8 ways up to 8 tokens
        // (more waves in flight), 4 ways for 9..16 tokens (the ring's LDS)
        if (n_tok <= 8 && nb >= 16) return launch_small_nt<1, 8>(w, x, Y, (int)n_out, (int)n_tok, nb, st);
        return launch_small_nt<1, 4>(w, x, Y, (int)n_out, (int)n_tok, nb, st);
    }
    if (n_tok <= 16 && nb % 8 == 0 && ((uintptr_t)W & 3u) == 0 && skinny_lds <= (size_t)skinny_lds_limit()) {
        hipLaunchKernelGGL(gemm_skinny_kernel, dim3((unsigned)cdiv(n_out, 16)), dim3(256), skinny_lds, st, w, x, Y,
                           (int)n_out, (int)n_tok, nb);
        return (int)hipGetLastError();
    }
    if (knob(pq2host::K_GEMM_KERNEL, 0) == 0) {
        // long prompts: the 256-row wide kernel (gemm_wide.hip) over the rows
        // whose tiles fill whole rounds of CUs, the 128-row kernel for the rest
        const int wide = knob(pq2host::K_GEMM_WIDE, 1);
        if (wide != 0 && n_tok > 16) {
            int mi = 8;
            const int64_t rows = pq2::gemm_wide_rows(W, Xq, n_out, n_tok, nb, gemm_cu_count(), wide == 2, &mi);
            if (rows > 0) {
                // with a workspace: the activation converted once (an extra
                // pass of 100 B per Q8_1 block), then the tiles DMA it -- worth
                // it where that pass is spread over enough rows (measured on
                // MI355X, M = 2048: 17408x5120 425 -> 414 us, 5120x17408 450 ->
                // 459 us, so 8192 rows and more)
                const bool via_ws = ws != nullptr && n_out >= 8192;
                const int rc = via_ws ? pq2::gemm_wide_launch_ws(W, Xq, Y, rows, n_tok, nb, mi, ws, st)
                                      : pq2::gemm_wide_launch(W, Xq, Y, rows, n_tok, nb, mi, st);
                if (rc != 0 || rows == n_out) return rc;
                return gemm_prefill_f16(w + (size_t)rows * PQ2_BYTES * nb, x, Y + (size_t)rows * n_tok,
                                        n_out - rows, n_tok, nb, st);
            }
        }
        return gemm_prefill_f16(w, x, Y, n_out, n_tok, nb, st);
    } else if ((nb & 1) || ((uintptr_t)W & 3u) != 0) {
        dim3 grid((unsigned)cdiv(n_out, 64), (unsigned)cdiv(n_tok, 64));
        hipLaunchKernelGGL(gemm_mfma_kernel_u16, grid, dim3(256), 0, st, w, x, Y, (int)n_out, (int)n_tok, nb);
    } else if (n_tok <= 32) {
        launch_gemm<4, 1, 1, 1>(w, x, Y, (int)n_out, (int)n_tok, nb, st);
    } else {
        launch_gemm<4, 2, 1, 2>(w, x, Y, (int)n_out, (int)n_tok, nb, st);
    }
    return (int)hipGetLastError();
}

}  // namespace

extern "C" {

int bonsai_p40_gemm(const void * W, const void * Xq, float * Y, int64_t n_out, int64_t n_in,
                    int64_t n_tok, bonsai_stream stream) {
    return gemm_dispatch(W, Xq, Y, n_out, n_in, n_tok, nullptr, stream);
}

int64_t bonsai_p40_gemm_workspace_bytes(int64_t n_in, int64_t n_tok) {
    if (n_in <= 0 || n_tok <= 0 || n_in % QK_PQ2 != 0 || n_in / QK_PQ2 > (1 << 24)) return 0;
    return pq2::gemm_wide_x16_bytes(n_tok, (int)(n_in / QK_PQ2));
}

int bonsai_p40_gemm_ws(const void * W, const void * Xq, float * Y, int64_t n_out, int64_t n_in,
                       int64_t n_tok, void * workspace, int64_t ws_bytes, bonsai_stream stream) {
    if (workspace == nullptr) return gemm_dispatch(W, Xq, Y, n_out, n_in, n_tok, nullptr, stream);
    if (((uintptr_t)workspace & 15u) != 0) return 1;
    const int64_t need = bonsai_p40_gemm_workspace_bytes(n_in, n_tok);
    if (ws_bytes < need) return 1;
    return gemm_dispatch(W, Xq, Y, n_out, n_in, n_tok, need > 0 ? workspace : nullptr, stream);
}

}  // extern "C"
