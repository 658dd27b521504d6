// gemm_wide.hip -- prefill PQ2_0 x Q8_1 GEMM for long prompts: 256 x 256
// (or 160 x 256) workgroup tiles on v_mfma_f32_16x16x32_f16.
//
// Contract (reference tests/test_p40.cpp:449-470, src/kernels/gemm_p40.cu:44-154):
//   Y[r*n_tok + t] = sum_b sum_p f16(dw[r,b]) * f16(da[4b+p, t]) * S(r, b, p, t)
// with S the exact integer chunk dot sum (code-1)*q over chunk p of block b,
// X chunk-major (Q8_1 block (c, t) at c*n_tok + t).
//
// Numerics (shared with gemm_f16_kernel in gemm.hip, and bit-identical to
// it): per Q8_1 chunk (K = 32) one f16 MFMA with A = (code - 1) * dw and
// B = q.  (code - 1) * dw is exact in f16, every product is exact in fp32 and
// every partial sum is dw times an integer of at most 13 bits (|S| <= 8128),
// so the MFMA returns dw * S exactly; one fp32 FMA per output element then
// adds da * (dw * S), chunk after chunk in K order.
//
// Why this tile.  Every instruction of the inner loop, the MFMA included,
// takes one of the SIMD's VALU issue slots, and the per-chunk FMA epilogue
// already costs 4 of them per 16 x 16 x 32 MFMA.  The operand conversion
// (codes -> f16 with the block scale, q -> f16) is paid once per workgroup
// tile: per chunk a BM x BN tile converts BM rows of codes and BN tokens of
// Q8_1 bytes for BM * BN / 256 MFMAs, ~1.5 VALU instructions per MFMA at
// 256 x 256 against ~5 at 128 x 128 (the 16-wave kernel in gemm.hip).  Each
// of the 8 waves owns MI x 4 MFMA tiles (128 x 64 at MI = 8), so a chunk's
// fragment reads are 12 KB per wave for 32 MFMAs (0.375 KB per MFMA against
// 1 KB for 32 x 32 wave tiles).
//
// Pipeline, one step per chunk c over RING LDS slots of one chunk each
// (RING = 2: a barrier after every chunk, chunk c+2 converted during chunk c;
// RING = 4: a barrier after every second chunk, chunk c+3 converted):
//   * the wave's MFMAs of chunk c run on fragments already in registers, two
//     MFMAs at a time, each pair followed by the FMAs of the pair before;
//     each fragment register is reloaded with chunk c+1's fragment from the
//     next slot right after its last use (the tile order makes that at least
//     2 MI - 2 tiles before it is needed);
//   * every thread converts its share of chunk c + LEAD (16 codes of one row
//     and 16 Q8_1 bytes of one token, loaded two steps earlier) in 8 pieces
//     between the MFMA pairs into a slot no wave reads in this interval;
//   * its raw registers then take chunk c + LEAD + 2's buffer loads;
//   * the barrier waits for LDS operations only: the global loads stay in
//     flight.
// The loop is unrolled over two PQ2_0 blocks (8 chunks), so the byte
// alignment of a block's codes (34-byte blocks: 2 bytes past a dword for an
// even block) and every register set are static.
//
// Code -> f16 with the block scale: per block each staging thread builds the
// 8-byte table {-dw, 0, dw, 2 dw} as a low-byte and a high-byte plane, and
// two v_perm per f16 pair look it up (the first builds the byte selector
// {c0, c0 + 4, c1, c1 + 4} from the codes).  q -> f16: v_perm to
// 0x6400 + (q + 128), a packed f16 add of -1152 (both exact).
//
// A block scale with |dw| >= 32768 would overflow f16 at code 3 (2 dw): such
// a block is staged as dw / 2 and the workgroup repeats its main loop with
// only those blocks (every other block's scale set to 0), adding the second
// half -- a second pass only for workgroups that meet such a scale.
//
// Requirements (checked by gemm_wide_rows): nb even, W and Xq 4-byte aligned,
// the matrix and Xq each below 2 GiB (buffer descriptors with 32-bit ranges).
#include "pq2_device.h"
#include "gemv_device.h"
#include "host_state.h"
#include "../../include/bonsai_p40.h"

#include <stdint.h>
#include <algorithm>
#include <type_traits>

using namespace pq2;

namespace {

typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 v2h __attribute__((ext_vector_type(2)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef uint32_t v4u __attribute__((ext_vector_type(4)));

// Workgroup tile: BM = 32 * MI rows x WB_N tokens, 8 waves as 2 (rows) x 4
// (tokens), a wave owning MI x 4 MFMA tiles of 16 x 16 (MI = 8: 256 rows;
// MI = 5: 160 rows, the tile that fills one round for 5120-row matrices).
constexpr int WB_N = 256, W_NI = 4;
template <int MI, bool BD = false>
struct WideCfg {
    static constexpr int BM = 32 * MI;
    static constexpr int ST_A = BM * 64;          // one chunk of f16 A: [row][32 positions]
    static constexpr int ST_B = WB_N * 64;        // one chunk of f16 B: [token][32 positions]
    static constexpr int ST_D = WB_N * 4;         // one chunk of fp32 activation scales
    static constexpr int ST = ST_A + ST_B + ST_D; // bytes per LDS slot
    // 2 slots for 256-row tiles (4 would spill registers), 4 for 160-row ones
    // (measured faster there: 5120x17408 at M = 2048 ~490 against ~510 us);
    // with the activation by DMA (BD) 2 A slots and a barrier after every
    // chunk, the B tiles and scales in RB slots of their own
    static constexpr int RING = (MI == 8 || BD) ? 2 : 4;
    static constexpr int SA = BD ? ST_A : ST;     // bytes per ring slot
    static constexpr int RB = 4;                  // BD: B slots (chunk c in slot c % 4)
    static constexpr int SB = ST_B + ST_D;        // BD: bytes per B slot
};

// Byte offset of 16-byte group g of row r in a [rows][64 B] tile, XOR-swizzled
// by ((r >> 1) ^ (r >> 2)) & 3: the fragment reads of 16 consecutive rows at
// one g and the staging writes hit distinct banks.  Adding 16 to r adds 1024.
__device__ __forceinline__ int wswz(int r, int g) { return r * 64 + ((g ^ ((r >> 1) ^ (r >> 2))) & 3) * 16; }

__device__ __forceinline__ uint32_t add_f16x2(uint32_t x, uint32_t c) {
    const v2h r = __builtin_bit_cast(v2h, x) + __builtin_bit_cast(v2h, c);
    return __builtin_bit_cast(uint32_t, r);
}

// four codes (bytes of x, values 0..3) -> four f16 of the block table
__device__ __forceinline__ void codes4_lookup(uint32_t x, uint32_t tl, uint32_t th, uint32_t & lo, uint32_t & hi) {
    const uint32_t x4 = x | 0x04040404u;
    lo = __builtin_amdgcn_perm(th, tl, __builtin_amdgcn_perm(x4, x, 0x05010400u));
    hi = __builtin_amdgcn_perm(th, tl, __builtin_amdgcn_perm(x4, x, 0x07030602u));
}

// four q bytes -> four f16
__device__ __forceinline__ void q4_f16(uint32_t q4, uint32_t & lo, uint32_t & hi) {
    const uint32_t x = q4 ^ 0x80808080u;                              // q + 128 per byte
    const uint32_t m1152 = 0xE480E480u;                               // f16 -1152, twice
    lo = add_f16x2(__builtin_amdgcn_perm(x, 0x64646464u, 0x00050004u), m1152);
    hi = add_f16x2(__builtin_amdgcn_perm(x, 0x64646464u, 0x00070006u), m1152);
}

// raw bytes of one chunk for one staging thread, loaded two steps before
// their conversion
struct WideRaw {
    uint32_t a0, a1;      // dword window over the row's 4 code bytes
    uint32_t d;           // the token's Q8_1 d (low half) and s
    v4u q;                // the token's 16 q bytes
};

// Buffer loads of chunk-in-block P of block b for one staging thread.  A:
// the row's code window; EVEN: block b is even, so its code bytes start 2
// bytes past a dword (rows are 4-byte aligned: 34 * nb with nb even).  B: the
// token's Q8_1 block.  Offsets: a_off = the row's byte offset + 4 * half,
// x_off = the token's Q8_1 block offset within a chunk, q_off = x_off + 4 +
// 16 * half; w_soff / x_soff are the workgroup-uniform byte offsets of block
// b in a row and of the chunk in X, and the per-chunk constant rides in the
// scalar offset as well (no VALU add).  (Free functions: the buffer builtins
// inside a kernel lambda drop the kernel's host stub.)
template <int P, bool EVEN>
__device__ __forceinline__ void wide_load_a(__amdgpu_buffer_rsrc_t rw, uint32_t a_off, uint32_t w_soff, WideRaw & r) {
    if constexpr (EVEN) {
        r.a0 = __builtin_amdgcn_raw_buffer_load_b32(rw, a_off, w_soff + 8 * P, 0);
        r.a1 = __builtin_amdgcn_raw_buffer_load_b32(rw, a_off, w_soff + 8 * P + 4, 0);
    } else {
        r.a0 = __builtin_amdgcn_raw_buffer_load_b32(rw, a_off, w_soff + 8 * P + 2, 0);
        r.a1 = r.a0;
    }
}

__device__ __forceinline__ void wide_load_b(__amdgpu_buffer_rsrc_t rx, uint32_t x_off, uint32_t q_off, uint32_t x_soff,
                                            WideRaw & r) {
    r.d = __builtin_amdgcn_raw_buffer_load_b32(rx, x_off, x_soff, 0);
    r.q = __builtin_amdgcn_raw_buffer_load_b128(rx, q_off, x_soff, 0);
}

// the dword holding block b's scale (low half for an even block, high half
// for an odd one); row_off = the row's byte offset
template <bool EVEN>
__device__ __forceinline__ uint32_t wide_load_dw(__amdgpu_buffer_rsrc_t rw, uint32_t row_off, uint32_t w_soff) {
    return __builtin_amdgcn_raw_buffer_load_b32(rw, row_off, EVEN ? w_soff : w_soff - 2, 0);
}

// BD: one chunk's f16 activation tile and fp32 scales by LDS-DMA into a B
// slot, three instructions per wave: the wave's two 1 KB pieces of the
// [token][64 B] tile (lane offsets b0, b1 carry the tile's group swizzle) and
// the scales of its 32 tokens (4 bytes per lane, lanes 0..31); soff_b /
// soff_d = the chunk's byte offset in X16 / XD.
__device__ __forceinline__ void wide_b_dma(__amdgpu_buffer_rsrc_t rxh, __amdgpu_buffer_rsrc_t rxd, uint8_t * slot,
                                           int wave, int lane, uint32_t b0, uint32_t b1, uint32_t dl, uint32_t soff_b,
                                           uint32_t soff_d, int d_at) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rxh, (lds_void *)(slot + 2048 * wave), 16, b0, soff_b, 0, 0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rxh, (lds_void *)(slot + 2048 * wave + 1024), 16, b1, soff_b, 0, 0);
    if (lane < 32)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rxd, (lds_void *)(slot + d_at + 128 * wave), 4, dl, soff_d, 0, 0);
}

// BD: A-side buffer loads issued at the step that loads chunk position j (the
// code window: 2 dwords for an even block, 1 for an odd one; the block scale
// dword with the block's first chunk), and the explicit wait at the end of
// step J for the B slot DMA'd two steps before: the wave's VMEM instructions
// younger than it are steps J - 1 and J, each A loads then 3 DMAs
constexpr int wide_na(int j) { return ((j & 7) < 4 ? 2 : 1) + ((j & 3) == 0 ? 1 : 0); }
template <int J, int LOAD>
constexpr int wide_bd_wait() { return wide_na(J - 1 + LOAD) + 3 + wide_na(J + LOAD) + 3; }

// The activation in the layout the BD kernel DMAs: block b of the chunk-major
// Q8_1 X (36 B at 36 b) becomes 64 B of f16 at X16 + 64 b (q byte e -> f16 e,
// exact) and its d as fp32 at XD[b] (exact); two threads per block.
__global__ void __launch_bounds__(256)
wide_x16_kernel(const uint8_t * __restrict__ Xq, uint8_t * __restrict__ X16, float * __restrict__ XD, int64_t blocks) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t b = i >> 1;
    const int h = (int)(i & 1);
    if (b >= blocks) return;
    const uint32_t * src = reinterpret_cast<const uint32_t *>(Xq + b * Q81_BYTES);
    uint32_t o[8];
#pragma unroll
    for (int k = 0; k < 4; ++k) q4_f16(src[1 + 4 * h + k], o[2 * k], o[2 * k + 1]);
    v4u * dst = reinterpret_cast<v4u *>(X16 + b * 64 + 32 * h);
    dst[0] = (v4u){o[0], o[1], o[2], o[3]};
    dst[1] = (v4u){o[4], o[5], o[6], o[7]};
    if (h == 0) XD[b] = f16_bits_to_f32(src[0] & 0xffffu);
}

template <int MI, bool BD>
__global__ void __launch_bounds__(512)
gemm_wide_kernel(const uint8_t * __restrict__ W, const uint8_t * __restrict__ X, float * __restrict__ Y,
                 int n_out, int n_tok, int nb, const uint8_t * __restrict__ X16, const float * __restrict__ XD) {
    using C = WideCfg<MI, BD>;
    constexpr int WB_M = C::BM, ST_A = C::ST_A, ST_B = C::ST_B, ST = C::ST, RING = C::RING, SA = C::SA;
    constexpr int LEAD = RING == 4 ? 3 : 2, LOAD = LEAD + 2;
    static_assert(!BD || (RING == 2 && LOAD == 4), "BD: the B DMA runs 4 chunks ahead");
    __shared__ __attribute__((aligned(16))) uint8_t smem[RING * SA];
    // BD: the B slots as separate LDS objects, so that reads of one slot are
    // not ordered behind the DMA into another
    __shared__ __attribute__((aligned(16))) uint8_t sb0[BD ? C::SB : 16], sb1[BD ? C::SB : 16],
        sb2[BD ? C::SB : 16], sb3[BD ? C::SB : 16];
    __shared__ int sBig;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave & 1, wn = wave >> 1;                  // 2 x 4 waves
    const int l16 = lane & 15, g = lane >> 4;
    const int row0 = blockIdx.x * WB_M, tok0 = blockIdx.y * WB_N;
    const int nc = 4 * nb;                                    // chunks

    // ---- staging roles: row (A) / token (B) sr, half sh of the chunk ----------
    // (with MI < 8 the threads past 2 * BM stage no A)
    const int sr = tid >> 1, sh = tid & 1;
    const bool stage_a = MI == 8 || sr < WB_M;                          // (tid < 512)
    const uint32_t rs = (uint32_t)PQ2_BYTES * (uint32_t)nb;
    const uint32_t a_row = (uint32_t)min(row0 + sr, n_out - 1) * rs;     // rows past n_out re-read the last
    const uint32_t b_tok = (uint32_t)min(tok0 + sr, n_tok - 1) * Q81_BYTES;
    const uint32_t a_off = a_row + 4 * sh, b_q = b_tok + 4 + 16 * sh;
    const uint32_t x_chunk = (uint32_t)n_tok * Q81_BYTES;                // bytes per chunk of X
    const __amdgpu_buffer_rsrc_t rw =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(W), (short)0, (int)(rs * (uint32_t)n_out), 0x00020000);
    const __amdgpu_buffer_rsrc_t rx =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(X), (short)0, (int)(x_chunk * (uint32_t)nc), 0x00020000);
    const int wa = wswz(sr, 2 * sh);                                     // group 2 sh; 2 sh + 1 at wa1
    const int wa1 = wswz(sr, 2 * sh + 1);
    const int wd = ST_B + 4 * sr;                                        // in the B slot
    // ---- fragment reads -------------------------------------------------------
    const int ra = wswz(wm * 16 * MI + l16, g);                          // + 1024 mi
    const int rb = wswz(wn * 64 + l16, g);                               // in the B slot, + 1024 ni
    const int rd = ST_B + 4 * (wn * 64 + l16);                           // in the B slot, + 64 ni
    // LDS slot bases: ring slot st of A; B slot s (tile, then scales)
    auto a_slot = [&](int st) __attribute__((always_inline)) { return smem + st * SA; };
    auto b_slot = [&](int s) __attribute__((always_inline)) -> uint8_t * {
        if constexpr (BD) return s == 0 ? sb0 : (s == 1 ? sb1 : (s == 2 ? sb2 : sb3));
        else return smem + s * ST + ST_A;
    };
    // ---- BD: the activation tile and scales by DMA from X16 / XD ---------------
    // (tokens past n_tok re-read the last token, as the staged path does)
    const uint32_t x16_chunk = (uint32_t)n_tok * 64u, xd_chunk = (uint32_t)n_tok * 4u;
    __amdgpu_buffer_rsrc_t rxh = rx, rxd = rx;
    uint32_t b_l0 = 0, b_l1 = 0, d_l = 0;
    if constexpr (BD) {
        rxh = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(X16), (short)0, (int)(x16_chunk * (uint32_t)nc),
                                                0x00020000);
        rxd = __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(XD), (short)0, (int)(xd_chunk * (uint32_t)nc),
                                                0x00020000);
        auto bsrc = [&](int r) {
            const int p = (lane & 3) ^ (((r >> 1) ^ (r >> 2)) & 3);      // logical group at physical lane & 3
            return (uint32_t)min(tok0 + r, n_tok - 1) * 64u + 16u * (uint32_t)p;
        };
        b_l0 = bsrc(32 * wave + (lane >> 2));
        b_l1 = bsrc(32 * wave + 16 + (lane >> 2));
        d_l = (uint32_t)min(tok0 + 32 * wave + lane, n_tok - 1) * 4u;
    }

    v4f acc[MI][W_NI];
#pragma unroll
    for (int mi = 0; mi < MI; ++mi)
#pragma unroll
        for (int ni = 0; ni < W_NI; ++ni) acc[mi][ni] = (v4f){0.0f, 0.0f, 0.0f, 0.0f};

    if (tid == 0) sBig = 0;
    __syncthreads();

    for (int pass = 0; pass < 2; ++pass) {
        if (pass == 1) {
            __syncthreads();
            if (!sBig) break;
        }
        WideRaw raw[2];
        uint32_t rdw = 0;         // dword holding the next block's scale
        uint32_t tl = 0, th = 0;  // block table planes

        // global loads of chunk c into r (jc = its position in the 8-chunk
        // iteration): the A part (code window, and for the first chunk of a
        // block the block scale) and the B part (the token's Q8_1 block)
        auto load_chunk_a = [&](int c, auto jc, WideRaw & r) __attribute__((always_inline)) {
            constexpr int j = decltype(jc)::value;
            constexpr int p = j & 3;
            constexpr bool even = (j >> 2) == 0;
            const int cc = c < nc ? c : c - 8;                            // past the end: two blocks back (same alignment)
            const uint32_t w_soff = 34u * (uint32_t)(cc >> 2);
            if (BD || stage_a) {                                          // (BD: every wave, for exact counts)
                wide_load_a<p, even>(rw, a_off, w_soff, r);
                if constexpr (p == 0) rdw = wide_load_dw<even>(rw, a_row, w_soff);
            }
        };
        auto load_chunk_b = [&](int c, WideRaw & r) __attribute__((always_inline)) {
            const int cc = c < nc ? c : c - 8;
            wide_load_b(rx, b_tok, b_q, (uint32_t)cc * x_chunk, r);
        };
        auto load_chunk = [&](int c, auto jc, WideRaw & r) __attribute__((always_inline)) {
            load_chunk_a(c, jc, r);
            if constexpr (!BD) load_chunk_b(c, r);
        };
        // BD: chunk c's tile and scales into B slot c % 4
        auto dma_chunk = [&](int c, int s) __attribute__((always_inline)) {
            const int cc = c < nc ? c : c - 8;
            wide_b_dma(rxh, rxd, b_slot(s), wave, lane, b_l0, b_l1, d_l, (uint32_t)cc * x16_chunk,
                       (uint32_t)cc * xd_chunk, ST_B);
        };
        // end-of-step barrier: BD waits for LDS only (a full fence would also
        // wait for the B DMAs still in flight), with a compiler memory barrier
        auto step_barrier = [&]() __attribute__((always_inline)) {
            if constexpr (BD) {
                __builtin_amdgcn_s_waitcnt(0xC07F);                      // lgkmcnt(0)
                __builtin_amdgcn_s_barrier();
                asm volatile("" ::: "memory");
            } else {
                __syncthreads();
            }
        };
        // block table from the loaded scale dword (odd: the block is odd, its
        // scale in the dword's high half)
        auto build_table = [&](int odd) __attribute__((always_inline)) {
            uint32_t dwb = (odd ? (rdw >> 16) : rdw) & 0xffffu;
            const bool big = (dwb & 0x7C00u) == 0x7800u;                  // |dw| >= 32768: 2 dw overflows
            if (big) sBig = 1;
            dwb -= big ? 0x400u : 0u;                                     // dw / 2, exact
            dwb = (pass == 0 || big) ? dwb : 0u;
            const _Float16 h = __builtin_bit_cast(_Float16, (uint16_t)dwb);
            const uint32_t v0 = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)(-h));
            const uint32_t v3 = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)(h + h));
            const uint32_t p01 = v0;                                      // code 0: -dw, code 1: 0
            const uint32_t p23 = dwb | (v3 << 16);                        // code 2: dw, code 3: 2 dw
            tl = __builtin_amdgcn_perm(p23, p01, 0x06040200u);
            th = __builtin_amdgcn_perm(p23, p01, 0x07050301u);
        };
        // Conversion of one chunk's raw bytes r into slot st, in 8 pieces:
        // piece k < 4 turns 4 codes, piece k >= 4 4 q bytes into f16; each odd
        // piece writes the 16-byte group it completes (the last one also the
        // token's scale).  EVEN: the chunk's block is even (its code bytes
        // start 2 bytes past the loaded dword window).
        uint32_t cw = 0;                                                  // the realigned code dword
        uint32_t plo = 0, phi = 0;                                        // the even piece, held for the write
        auto convert_piece = [&](const WideRaw & r, int k, bool even, int st) __attribute__((always_inline)) {
            uint32_t lo, hi;
            if (BD && k >= 4) return;                                     // BD: B arrives by DMA
            if (k < 4) {
                if (!stage_a) return;
                if (k == 0) cw = even ? __builtin_amdgcn_alignbyte(r.a1, r.a0, 2) : r.a0;
                codes4_lookup((cw >> (2 * k)) & 0x03030303u, tl, th, lo, hi);
                if (k & 1) *reinterpret_cast<v4u *>(a_slot(st) + ((k & 2) ? wa1 : wa)) = (v4u){plo, phi, lo, hi};
            } else {
                const uint32_t q4 = k == 4 ? r.q.x : k == 5 ? r.q.y : k == 6 ? r.q.z : r.q.w;
                q4_f16(q4, lo, hi);
                if (k & 1) *reinterpret_cast<v4u *>(b_slot(st) + ((k & 2) ? wa1 : wa)) = (v4u){plo, phi, lo, hi};
                if (k == 7 && sh == 0) *reinterpret_cast<float *>(b_slot(st) + wd) = f16_bits_to_f32(r.d & 0xffffu);
            }
            if (!(k & 1)) {
                plo = lo;
                phi = hi;
            }
        };
        auto convert = [&](const WideRaw & r, int j, int st) __attribute__((always_inline)) {
#pragma unroll
            for (int k = 0; k < 8; ++k) convert_piece(r, k, (j >> 2) == 0, st);
        };

        v8h A[MI];
        v8h Bf[W_NI];
        float dv[W_NI];
        auto load_frag_a = [&](int st, int mi) __attribute__((always_inline)) {
            A[mi] = *reinterpret_cast<const v8h *>(a_slot(st) + ra + 1024 * mi);
        };
        auto load_frag_b = [&](int s, int ni) __attribute__((always_inline)) {
            Bf[ni] = *reinterpret_cast<const v8h *>(b_slot(s) + rb + 1024 * ni);
        };
        auto load_scale = [&](int s, int ni) __attribute__((always_inline)) {
            dv[ni] = *reinterpret_cast<const float *>(b_slot(s) + rd + 64 * ni);
        };

        // ---- prologue: chunks 0 .. LEAD-1 converted, LEAD and LEAD+1 in flight -
        if constexpr (BD) {
            // every chunk's A loads, then its B DMA, in chunk order (the
            // order the step waits count on): chunks 0..3 in flight, 0 and 1
            // converted; chunk 1's B (and so chunk 0's) has landed before the
            // barrier
            load_chunk_a(0, std::integral_constant<int, 0>{}, raw[0]);
            dma_chunk(0, 0);
            load_chunk_a(1, std::integral_constant<int, 1>{}, raw[1]);
            dma_chunk(1, 1);
            build_table(0);
            convert(raw[0], 0, 0);
            convert(raw[1], 1, 1);
            load_chunk_a(2, std::integral_constant<int, 2>{}, raw[0]);
            dma_chunk(2, 2);
            load_chunk_a(3, std::integral_constant<int, 3>{}, raw[1]);
            dma_chunk(3, 3);
            wait_vmcnt<wide_bd_wait<-1, LOAD>()>();
        } else {
            load_chunk(0, std::integral_constant<int, 0>{}, raw[0]);
            load_chunk(1, std::integral_constant<int, 1>{}, raw[1]);
            build_table(0);
            convert(raw[0], 0, 0);
            convert(raw[1], 1, 1);
            load_chunk(2, std::integral_constant<int, 2>{}, raw[0]);
            if constexpr (RING == 4) {
                convert(raw[0], 2, 2);
                load_chunk(3, std::integral_constant<int, 3>{}, raw[1]);
                load_chunk(4, std::integral_constant<int, 4>{}, raw[0]);
            } else {
                load_chunk(3, std::integral_constant<int, 3>{}, raw[1]);
            }
        }
        step_barrier();
#pragma unroll
        for (int mi = 0; mi < MI; ++mi) load_frag_a(0, mi);
#pragma unroll
        for (int ni = 0; ni < W_NI; ++ni) {
            load_frag_b(0, ni);
            load_scale(0, ni);
        }
        // the first steps convert into the slots after: every wave's reads of
        // chunk 0 must be complete first
        step_barrier();

        // one chunk; J = the chunk's position in the 8-chunk iteration
        auto step = [&](int c0, auto jc) __attribute__((always_inline)) {
            constexpr int J = decltype(jc)::value;
            constexpr int st_next = (J + 1) % RING, st_conv = (J + LEAD) % RING;   // LDS slots
            constexpr int sb_next = BD ? (J + 1) % C::RB : st_next;       // B slot of chunk c + 1
            constexpr int rset = (J + LEAD) & 1;                          // raw set of chunk c + LEAD
            const int c = c0 + J;
            // the block table for chunk c + LEAD when it starts a block
            if constexpr (((J + LEAD) & 3) == 0) build_table(((J + LEAD) & 7) >> 2);
            __builtin_amdgcn_sched_barrier(0);
            // The MI x 4 MFMA tiles in two halves, each row-major over two token
            // fragments: half h covers (mi, 2h) and (mi, 2h + 1) for every mi.
            // MFMAs go in pairs; each pair is followed by the 4-FMA epilogues of
            // the pair before (their products have had two MFMAs of time).
            // Fragment registers are reloaded with chunk c+1's fragments right
            // after their last use (B[0], B[1] and their scales in the middle,
            // A[mi] after (mi, 3), B[2], B[3] at the end).
            constexpr int NT = MI * W_NI, NH = NT / 2;
            v4f S[4];
            auto tile_mi = [](int t) { return (t % NH) / 2; };
            auto tile_ni = [](int t) { return 2 * (t / NH) + (t & 1); };
            auto fma_tile = [&](int t) __attribute__((always_inline)) {
                const int mi = tile_mi(t), ni = tile_ni(t);
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[mi][ni][i] = fmaf(dv[ni], S[t & 3][i], acc[mi][ni][i]);
                // pin the FMAs here: otherwise they sink below the step's last
                // MFMA with every product kept live
                asm volatile("" : "+v"(acc[mi][ni]));
                if (mi == MI - 1) load_scale(sb_next, ni);
            };
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                const int mi = tile_mi(t), ni = tile_ni(t);
                S[t & 3] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[mi], Bf[ni], (v4f){0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
                // the MFMA issues before the epilogues that follow it: left
                // free, the scheduler puts it after them, and each epilogue then
                // reads a product only one MFMA old (hazard nops and a stall
                // on the matrix core instead of two MFMAs of cover)
                __builtin_amdgcn_sched_barrier(0);
                if ((t & 1) && t >= 3) {
                    fma_tile(t - 3);
                    fma_tile(t - 2);
                }
                if (ni == W_NI - 1) load_frag_a(st_next, mi);
                if (mi == MI - 1) load_frag_b(sb_next, ni);
#pragma unroll
                for (int k = 0; k < 8; ++k) {
                    if (t != k * NT / 8 + 1) continue;
                    // piece k of chunk c + LEAD into its slot; its raw registers
                    // then take chunk c + LOAD's loads
                    convert_piece(raw[rset], k, (((J + LEAD) & 7) >> 2) == 0, st_conv);
                    if (k == 1) load_chunk_a(c + LOAD, std::integral_constant<int, (J + LOAD) & 7>{}, raw[rset]);
                    if constexpr (BD) {
                        if (k == 4) dma_chunk(c + LOAD, J % C::RB);       // into chunk c's slot, read by now
                    } else {
                        if (k == 7) load_chunk_b(c + LOAD, raw[rset]);
                    }
                }
                __builtin_amdgcn_sched_barrier(0);
            }
            fma_tile(NT - 2);
            fma_tile(NT - 1);
            __builtin_amdgcn_sched_barrier(0);
            if constexpr (BD) wait_vmcnt<wide_bd_wait<J, LOAD>()>();        // chunk c + 2's B slot has landed
            if (RING == 2 || (J & 1)) step_barrier();
        };
        for (int c0 = 0; c0 < nc; c0 += 8) {                            // nc % 8 == 0 (nb even)
            step(c0, std::integral_constant<int, 0>{});
            step(c0, std::integral_constant<int, 1>{});
            step(c0, std::integral_constant<int, 2>{});
            step(c0, std::integral_constant<int, 3>{});
            step(c0, std::integral_constant<int, 4>{});
            step(c0, std::integral_constant<int, 5>{});
            step(c0, std::integral_constant<int, 6>{});
            step(c0, std::integral_constant<int, 7>{});
        }
        if constexpr (BD) wait_vmcnt<0>();          // the DMAs past the last chunk have landed
    }

    // ---- store: lane holds rows 4g + i of each 16-row tile, token l16 --------
#pragma unroll
    for (int mi = 0; mi < MI; ++mi)
#pragma unroll
        for (int ni = 0; ni < W_NI; ++ni) {
            const int tok = tok0 + wn * 64 + 16 * ni + l16;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int row = row0 + wm * 16 * MI + 16 * mi + 4 * g + i;
                if (row < n_out && tok < n_tok) Y[(size_t)row * n_tok + tok] = acc[mi][ni][i];
            }
        }
}

}  // namespace

namespace pq2 {

// Rows [0, rows) of the product that the wide kernel takes, and its tile
// height (*mi = 8: 256 rows, 5: 160 rows): the whole 256-row tiles whose
// 256 x 256 tiles fill whole rounds of the device's CUs (the caller runs the
// remaining rows on the 128-row kernel), or, short of one round, every row on
// 256- or 160-row tiles where one round of them holds at least 3/4 of a full
// round's outputs; 0 where the kernel's requirements do not hold or its tiles
// would fill too little of a round.  force: every row whenever the requirements
// hold (tests; the BONSAI_GEMM_WIDE_MI knob picks the tile height there).
int64_t gemm_wide_rows(const void * W, const void * Xq, int64_t n_out, int64_t n_tok, int nb, int cus, bool force,
                       int * mi) {
    *mi = 8;
    if (nb < 2 || nb % 2 != 0 || ((uintptr_t)W & 3u) != 0 || ((uintptr_t)Xq & 3u) != 0) return 0;
    if ((uint64_t)n_out * PQ2_BYTES * (uint64_t)nb >= (1ull << 31)) return 0;      // buffer ranges are int
    if ((uint64_t)n_tok * Q81_BYTES * 4ull * (uint64_t)nb >= (1ull << 31)) return 0;
    if (force) {
        *mi = pq2host::knob(pq2host::K_GEMM_WIDE_MI, 8) == 5 ? 5 : 8;
        return n_out;
    }
    const int64_t T = (n_tok + WB_N - 1) / WB_N;
    if (4 * n_tok < 3 * T * WB_N) return 0;                                       // token tiles mostly empty
    // 256-row tiles over the rows whose tiles fill whole rounds
    const int64_t R = n_out / 256, rounds = R * T / cus;
    if (rounds >= 1) return std::min<int64_t>(R, rounds * cus / T) * 256;
    // Less than one round: a round of wide tiles takes about the same time
    // however many CUs it fills, so one pays where at least 3/4 of a full
    // round's outputs are real (measured on MI355X, one process, us, LDS kernel
    // -> wide: 17408x5120 M = 768 225 -> 181 (256 rows), M = 512 165 -> 138
    // (160 rows), 6144x5120 M = 2048 189 -> 180 (256 rows); at 5/8 and below
    // the LDS kernel stays faster: 17408x5120 M = 384 116 against 137,
    // 5120x6144 M = 1024 126 against 160)
    const int64_t outputs = n_out * n_tok;
    if ((n_out + 255) / 256 * T <= cus && 4 * outputs >= 3 * (int64_t)cus * 256 * WB_N) return n_out;
    if ((n_out + 159) / 160 * T <= cus && 4 * outputs >= 3 * (int64_t)cus * 160 * WB_N) {
        *mi = 5;
        return n_out;
    }
    return 0;
}

// The wide kernel (mi = 8 or 5) over rows [0, n_out) of W / Y (the caller
// offsets both for a row range); requires what gemm_wide_rows checks.
int gemm_wide_launch(const void * W, const void * Xq, float * Y, int64_t n_out, int64_t n_tok, int nb, int mi,
                     hipStream_t st) {
    const unsigned gy = (unsigned)((n_tok + WB_N - 1) / WB_N);
    const uint8_t * w = (const uint8_t *)W, * x = (const uint8_t *)Xq;
    if (mi == 5)
        hipLaunchKernelGGL((gemm_wide_kernel<5, false>), dim3((unsigned)((n_out + 159) / 160), gy), dim3(512), 0, st,
                           w, x, Y, (int)n_out, (int)n_tok, nb, nullptr, nullptr);
    else
        hipLaunchKernelGGL((gemm_wide_kernel<8, false>), dim3((unsigned)((n_out + 255) / 256), gy), dim3(512), 0, st,
                           w, x, Y, (int)n_out, (int)n_tok, nb, nullptr, nullptr);
    return (int)hipGetLastError();
}

// Bytes of the activation in the layout the wide kernel DMAs (X16: f16 of
// every q byte, 64 B per Q8_1 block; XD: its d as fp32), 0 if the 32-bit
// buffer offsets cannot address it.
int64_t gemm_wide_x16_bytes(int64_t n_tok, int nb) {
    const int64_t blocks = n_tok * 4 * (int64_t)nb;
    if (blocks * 64 >= (1ll << 31)) return 0;
    return blocks * 68;
}

// The same product as gemm_wide_launch, with the activation converted once
// into ws (gemm_wide_x16_bytes, 16-byte aligned) and the kernel's B side
// arriving by LDS-DMA from there; bit-identical to gemm_wide_launch.
int gemm_wide_launch_ws(const void * W, const void * Xq, float * Y, int64_t n_out, int64_t n_tok, int nb, int mi,
                        void * ws, hipStream_t st) {
    const int64_t blocks = n_tok * 4 * (int64_t)nb;
    uint8_t * x16 = static_cast<uint8_t *>(ws);
    float * xd = reinterpret_cast<float *>(x16 + blocks * 64);
    hipLaunchKernelGGL(wide_x16_kernel, dim3((unsigned)((2 * blocks + 255) / 256)), dim3(256), 0, st,
                       (const uint8_t *)Xq, x16, xd, blocks);
    const unsigned gy = (unsigned)((n_tok + WB_N - 1) / WB_N);
    const uint8_t * w = (const uint8_t *)W, * x = (const uint8_t *)Xq;
    if (mi == 5)
        hipLaunchKernelGGL((gemm_wide_kernel<5, true>), dim3((unsigned)((n_out + 159) / 160), gy), dim3(512), 0, st,
                           w, x, Y, (int)n_out, (int)n_tok, nb, x16, xd);
    else
        hipLaunchKernelGGL((gemm_wide_kernel<8, true>), dim3((unsigned)((n_out + 255) / 256), gy), dim3(512), 0, st,
                           w, x, Y, (int)n_out, (int)n_tok, nb, x16, xd);
    return (int)hipGetLastError();
}

}  // namespace pq2
