// pq2_device.h -- gfx950 device helpers shared by the PQ2_0 kernels.
//
// Formats (reference src/pq2_0.h:45-54): block_pq2_0 is 34 bytes (fp16 d at
// byte 0, 32 code bytes at 2), block_q8_1 is 36 bytes (fp16 d at 0, raw int16
// activation sum s at 2, 32 permuted int8 at 4).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace pq2 {

constexpr int QK_PQ2 = 128;      // weights per PQ2_0 block
constexpr int QK8 = 32;          // elements per Q8_1 block
constexpr int PQ2_BYTES = 34;
constexpr int Q81_BYTES = 36;
constexpr int HBLK = 1024;       // Hadamard block

// ---- fp16 ----------------------------------------------------------------
__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

// fp32 -> fp16 bits with the reference HOST rounding (src/p40_common.h:82-114):
// the magnitude rounds half away from zero (hardware cvt rounds to nearest
// even, which differs on exact ties), overflow -> inf, NaN -> quiet NaN.
__device__ __forceinline__ uint32_t f32_to_f16_away(float f) {
    const uint32_t x = __float_as_uint(f);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t fe = (x >> 23) & 0xffu;
    const uint32_t mant = x & 0x7fffffu;
    int e = (int)fe - 112;
    if (fe == 0xffu) return sign | 0x7c00u | (mant ? 0x200u : 0u);
    if (e >= 31) return sign | 0x7c00u;
    if (e <= 0) {
        if (e < -10) return sign;
        const uint32_t full = mant | 0x800000u;
        const uint32_t sh = (uint32_t)(14 - e);
        uint32_t q = full >> sh;
        q += (full >> (sh - 1)) & 1u;
        return sign | q;
    }
    uint32_t q = mant >> 13;
    if (mant & 0x1000u) {
        ++q;
        if (q == 0x400u) { q = 0; ++e; if (e >= 31) return sign | 0x7c00u; }
    }
    return sign | ((uint32_t)e << 10) | q;
}

// ---- DPP cross-lane helpers (wave64) --------------------------------------
template <int CTRL, int ROW_MASK = 0xf, int BANK_MASK = 0xf>
__device__ __forceinline__ float dpp_mov(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROW_MASK,
                                                      BANK_MASK, false));
}

template <int CTRL>
__device__ __forceinline__ int dpp_mov_i(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xf, 0xf, false);
}

constexpr int DPP_QUAD_XOR1 = 0xB1;       // quad_perm [1,0,3,2]
constexpr int DPP_QUAD_XOR2 = 0x4E;       // quad_perm [2,3,0,1]
constexpr int DPP_ROW_HALF_MIRROR = 0x141;
constexpr int DPP_ROW_MIRROR = 0x140;
constexpr int DPP_ROW_BCAST15 = 0x142;
constexpr int DPP_ROW_BCAST31 = 0x143;

// Sum over the 64 lanes of a wave; the total lands in lane 63.
// Rows of 16 are reduced with quad/mirror DPP moves (every lane of a row then
// holds the row sum), then row_bcast:15 / row_bcast:31 fold the four rows
// into lane 63.
__device__ __forceinline__ float wave_sum_to_lane63(float v) {
    v += dpp_mov<DPP_QUAD_XOR1>(v);
    v += dpp_mov<DPP_QUAD_XOR2>(v);
    v += dpp_mov<DPP_ROW_HALF_MIRROR>(v);
    v += dpp_mov<DPP_ROW_MIRROR>(v);
    v += dpp_mov<DPP_ROW_BCAST15, 0xa>(v);
    v += dpp_mov<DPP_ROW_BCAST31, 0xc>(v);
    return v;
}

// fp64 moves and sum over the 64 lanes of a wave, the total in every lane:
// rows of 16 by quad/mirror DPP moves of both halves, then the four row sums
// (read from lanes 0, 16, 32, 48) added in a fixed order.  No LDS round trips
// (a __shfl_xor of a double is two ds_bpermute per step).
template <int CTRL>
__device__ __forceinline__ double dpp_mov_f64(double v) {
    const unsigned long long u = (unsigned long long)__double_as_longlong(v);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)u, CTRL, 0xf, 0xf, false);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)(uint32_t)(u >> 32), CTRL, 0xf, 0xf, false);
    return __longlong_as_double((long long)(((unsigned long long)hi << 32) | lo));
}

__device__ __forceinline__ double readlane_f64(double v, int lane) {
    const unsigned long long u = (unsigned long long)__double_as_longlong(v);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)u, lane);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(u >> 32), lane);
    return __longlong_as_double((long long)(((unsigned long long)hi << 32) | lo));
}

__device__ __forceinline__ double wave_sum_f64(double v) {
    v += dpp_mov_f64<DPP_QUAD_XOR1>(v);
    v += dpp_mov_f64<DPP_QUAD_XOR2>(v);
    v += dpp_mov_f64<DPP_ROW_HALF_MIRROR>(v);
    v += dpp_mov_f64<DPP_ROW_MIRROR>(v);
    return (readlane_f64(v, 0) + readlane_f64(v, 16)) + (readlane_f64(v, 32) + readlane_f64(v, 48));
}

// ---- integer chunk dot ------------------------------------------------------
// sumi = bias + sum_k dot4((w >> 2k) & 0x03030303, a_k) over the two 16-code
// words (w0, w1) of a 32-weight chunk against the 8 permuted activation words
// (src/pq2_0.h:149-172).  Codes are 0..3, so the signed v_dot4 equals the
// reference's unsigned-code x signed-activation product.
__device__ __forceinline__ int chunk_dot_i32(uint32_t w0, uint32_t w1, const int (&a)[8],
                                             int bias) {
    int s = bias;
    s = __builtin_amdgcn_sdot4((int)(w0 & 0x03030303u), a[0], s, false);
    s = __builtin_amdgcn_sdot4((int)((w0 >> 2) & 0x03030303u), a[1], s, false);
    s = __builtin_amdgcn_sdot4((int)((w0 >> 4) & 0x03030303u), a[2], s, false);
    s = __builtin_amdgcn_sdot4((int)((w0 >> 6) & 0x03030303u), a[3], s, false);
    s = __builtin_amdgcn_sdot4((int)(w1 & 0x03030303u), a[4], s, false);
    s = __builtin_amdgcn_sdot4((int)((w1 >> 2) & 0x03030303u), a[5], s, false);
    s = __builtin_amdgcn_sdot4((int)((w1 >> 4) & 0x03030303u), a[6], s, false);
    s = __builtin_amdgcn_sdot4((int)((w1 >> 6) & 0x03030303u), a[7], s, false);
    return s;
}

// Same chunk dot, scaled by 16 and with one extraction shift per word: bit
// pairs 0 and 1 of every code byte are taken with the mask 0x03030303 from w
// and w >> 2 (weight 1), bit pairs 2 and 3 with 0x30303030 from w and w >> 2,
// which leaves 16 * code in each byte (<= 48, still a positive int8).  The two
// partial sums combine as 16 * s1 + s16 with one v_lshl_add; `bias16` is
// -16 * s.  The result is exactly 16 * sumi.
__device__ __forceinline__ int chunk_dot_x16(uint32_t w0, uint32_t w1, const int (&a)[8],
                                             int bias16) {
    constexpr uint32_t M = 0x03030303u, M4 = 0x30303030u;
    const uint32_t v0 = w0 >> 2, v1 = w1 >> 2;
    int s1 = 0, s16 = bias16;
    s1 = __builtin_amdgcn_sdot4((int)(w0 & M), a[0], s1, false);
    s1 = __builtin_amdgcn_sdot4((int)(v0 & M), a[1], s1, false);
    s16 = __builtin_amdgcn_sdot4((int)(w0 & M4), a[2], s16, false);
    s16 = __builtin_amdgcn_sdot4((int)(v0 & M4), a[3], s16, false);
    s1 = __builtin_amdgcn_sdot4((int)(w1 & M), a[4], s1, false);
    s1 = __builtin_amdgcn_sdot4((int)(v1 & M), a[5], s1, false);
    s16 = __builtin_amdgcn_sdot4((int)(w1 & M4), a[6], s16, false);
    s16 = __builtin_amdgcn_sdot4((int)(v1 & M4), a[7], s16, false);
    return (s1 << 4) + s16;
}

// Nibble-plane form of the same chunk dot, for activations that are reused
// across many weight rows.  An int8 activation splits as a = 16*h + l with
// h = a >> 4 (signed, -8..7) and l = a & 15 (unsigned, 0..15); both are the
// two nibbles of the byte as stored.  A code word w gives two nibble words
// with one shift and two masks: w & 0x33333333 holds bit pairs 0 and 2 of
// every byte (nibbles 2j and 2j+1), (w >> 2) & 0x33333333 bit pairs 1 and 3.
// The matching activation planes interleave the nibbles of permuted words
// a_k and a_{k+2} the same way, so
//   sum code*a = 16 * sdot8(codes, h-plane) + udot8(codes, l-plane)
// with codes 0..3 valid both as signed and unsigned 4-bit values.
// nib_planes() builds the 4 h-words and 4 l-words of one chunk from its 8
// permuted activation words; chunk_dot_nib() returns sumi exactly.
__device__ __forceinline__ void nib_planes(const uint32_t (&a)[8], uint32_t (&h)[4], uint32_t (&l)[4]) {
    constexpr uint32_t LO = 0x0F0F0F0Fu;
#pragma unroll
    for (int q = 0; q < 2; ++q) {
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const uint32_t x = a[4 * q + k], z = a[4 * q + k + 2];
            h[2 * q + k] = ((x >> 4) & LO) | (z & ~LO);
            l[2 * q + k] = (x & LO) | ((z << 4) & ~LO);
        }
    }
}

// The four nibble words of a chunk's two code words.
__device__ __forceinline__ void code_nibbles(uint32_t w0, uint32_t w1, uint32_t (&n)[4]) {
    constexpr uint32_t M = 0x33333333u;
    n[0] = w0 & M; n[1] = (w0 >> 2) & M; n[2] = w1 & M; n[3] = (w1 >> 2) & M;
}

__device__ __forceinline__ int chunk_dot_nibw(const uint32_t (&n)[4], const uint32_t (&h)[4],
                                              const uint32_t (&l)[4], int bias) {
    // the first product in the three-operand form with a literal 0 accumulator
    // (the builtin becomes the tied-accumulator form plus a v_mov of the 0)
    int sh;
    asm("v_dot8_i32_i4 %0, %1, %2, 0" : "=v"(sh) : "v"(n[0]), "v"(h[0]));
    sh = __builtin_amdgcn_sdot8((int)n[1], (int)h[1], sh, false);
    sh = __builtin_amdgcn_sdot8((int)n[2], (int)h[2], sh, false);
    sh = __builtin_amdgcn_sdot8((int)n[3], (int)h[3], sh, false);
    uint32_t sl = __builtin_amdgcn_udot8(n[0], l[0], (uint32_t)bias, false);
    sl = __builtin_amdgcn_udot8(n[1], l[1], sl, false);
    sl = __builtin_amdgcn_udot8(n[2], l[2], sl, false);
    sl = __builtin_amdgcn_udot8(n[3], l[3], sl, false);
    return (int)(((uint32_t)sh << 4) + sl);   // modulo 2^32: exact for |sumi| < 2^31
}

__device__ __forceinline__ int chunk_dot_nib(uint32_t w0, uint32_t w1, const uint32_t (&h)[4],
                                             const uint32_t (&l)[4], int bias) {
    uint32_t n[4];
    code_nibbles(w0, w1, n);
    return chunk_dot_nibw(n, h, l, bias);
}

__host__ __device__ constexpr int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

}  // namespace pq2
