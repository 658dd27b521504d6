// fwht_device.h -- FWHT-1024 and permuted Q8_1 quantisation of one block by
// one wave, shared by the pre-pass kernels and the fused GEMV.
//
// Reference semantics: src/fwht.h:20-42 (transform, stage order h = 1..512,
// signs, 1/32 normalisation), src/pq2_0.h:99-126 (quantiser, host rounding).
//
// The whole transform runs in registers, without LDS.  Lane l holds the 16
// consecutive elements 16 row(l) .. 16 row(l) + 15 of the block, where the
// 6-bit row index maps the element bits 4..9 onto lane bits so that every
// cross-lane butterfly partner is one cheap move:
//   e4 = l0^l2, e5 = l1^l2, e6 = l2^l3, e7 = l3, e8 = l4, e9 = l5,
// i.e. flipping e4, e5, e6, e7 is lane ^1, ^2, ^7, ^15 -- the DPP quad_perm
// [1,0,3,2], quad_perm [2,3,0,1], row_half_mirror and row_mirror moves --
// and flipping e8, e9 is lane ^16, ^32 -- v_permlane16_swap and
// v_permlane32_swap.  Stages h = 1..8 are register butterflies.  Every stage
// produces the host's a+b (lane holding the lower element) or a-b (lane
// holding the upper element) with one correctly rounded operation, in the
// host's order h = 1, 2, ..., 512, so the rotated values are bit-identical to
// fwht_blocks().  A Q8_1 chunk (elements 32c..32c+31, bits 0..4) is the lane
// pair (l, l^1), so its amax and sum need a single DPP exchange, and each
// lane writes its 16-element half already transposed (activation word k =
// elements k, k+4, k+8, k+12).
//
// No floating-point contraction: the host computes x*sign, x*id and the
// butterfly sums as separately rounded fp32 operations, so every function
// here turns contraction off for its own body.
#pragma once

#include "pq2_device.h"

namespace pq2 {

template <int H>
__device__ __forceinline__ void butterfly(float (&v)[16]) {
#pragma clang fp contract(off)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        if (!(r & H)) {
            const float a = v[r], b = v[r | H];
            v[r] = a + b;
            v[r | H] = a - b;
        }
    }
}

__device__ __forceinline__ void load16(const float * p, float (&v)[16], bool vec) {
    if (vec) {
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const float4 t = reinterpret_cast<const float4 *>(p)[k];
            v[4 * k] = t.x; v[4 * k + 1] = t.y; v[4 * k + 2] = t.z; v[4 * k + 3] = t.w;
        }
    } else {
#pragma unroll
        for (int r = 0; r < 16; ++r) v[r] = p[r];
    }
}

__device__ __forceinline__ void store16(float * p, const float (&v)[16], bool vec) {
    if (vec) {
#pragma unroll
        for (int k = 0; k < 4; ++k)
            reinterpret_cast<float4 *>(p)[k] = make_float4(v[4 * k], v[4 * k + 1], v[4 * k + 2], v[4 * k + 3]);
    } else {
#pragma unroll
        for (int r = 0; r < 16; ++r) p[r] = v[r];
    }
}

// Row (element bits 4..9) held by lane l.
__device__ __forceinline__ int fwht_row(int l) {
    const int e4 = (l ^ (l >> 2)) & 1, e5 = ((l >> 1) ^ (l >> 2)) & 1, e6 = ((l >> 2) ^ (l >> 3)) & 1;
    return e4 | (e5 << 1) | (e6 << 2) | (l & 0x38);
}

// Butterfly across lanes for an element bit whose partner lane is one DPP
// move away, on sign-carrying values: a lane stores y = sigma v with sigma =
// +-1, and the two lanes of every pair store the same sigma.  y' = y + c p
// with p the partner's y and c = +1 on the lane holding the lower element,
// -1 on the other, is sigma (a + b) on the lower lane and -sigma (a - b) on
// the upper one: the host's sum and difference, correctly rounded (the
// product c p is exact and rounding is sign-symmetric), with the upper
// lane's sigma flipped.  One v_fmac with a DPP operand per element.
// The compiler does not fold a DPP move into the tied v_fmac, so the 16
// v_fmac_f32_dpp of a stage are written out: instruction k reads the
// partner's v[k] through DPP and writes v[k] (all lanes read before any
// writes), and no instruction reads a register written by the one before it.
// The leading s_nop 1 gives the 2 wait states a DPP read needs after a VALU
// write of its source, which the hazard recogniser cannot see into the asm.
#define PQ2_DPP_FMAC16(DPP)                                                                     \
    asm volatile("s_nop 1\n"                                                                   \
        "v_fmac_f32_dpp %0, %0, %16 " DPP " row_mask:0xf bank_mask:0xf\n"\
        "v_fmac_f32_dpp %1, %1, %16 " DPP " row_mask:0xf bank_mask:0xf\n"\
        "v_fmac_f32_dpp %2, %2, %16 " DPP " row_mask:0xf bank_mask:0xf\n"\
        "v_fmac_f32_dpp %3, %3, %16 " DPP " row_mask:0xf bank_mask:0xf\n"\
        "v_fmac_f32_dpp %4, %4, %16 " DPP " row_mask:0xf bank_mask:0xf\n"\
        "v_fmac_f32_dpp %5, %5, %16 " DPP " row_mask:0xf bank_mask:0xf\n"\
        "v_fmac_f32_dpp %6, %6, %16 " DPP " row_mask:0xf bank_mask:0xf\n"\
        "v_fmac_f32_dpp %7, %7, %16 " DPP " row_mask:0xf bank_mask:0xf\n"\
        "v_fmac_f32_dpp %8, %8, %16 " DPP " row_mask:0xf bank_mask:0xf\n"\
        "v_fmac_f32_dpp %9, %9, %16 " DPP " row_mask:0xf bank_mask:0xf\n"\
        "v_fmac_f32_dpp %10, %10, %16 " DPP " row_mask:0xf bank_mask:0xf\n"\
        "v_fmac_f32_dpp %11, %11, %16 " DPP " row_mask:0xf bank_mask:0xf\n"\
        "v_fmac_f32_dpp %12, %12, %16 " DPP " row_mask:0xf bank_mask:0xf\n"\
        "v_fmac_f32_dpp %13, %13, %16 " DPP " row_mask:0xf bank_mask:0xf\n"\
        "v_fmac_f32_dpp %14, %14, %16 " DPP " row_mask:0xf bank_mask:0xf\n"\
        "v_fmac_f32_dpp %15, %15, %16 " DPP " row_mask:0xf bank_mask:0xf\n"\
        : "+v"(v[0]), "+v"(v[1]), "+v"(v[2]), "+v"(v[3]), "+v"(v[4]), "+v"(v[5]),     \
                   "+v"(v[6]), "+v"(v[7]), "+v"(v[8]), "+v"(v[9]), "+v"(v[10]), "+v"(v[11]),    \
                   "+v"(v[12]), "+v"(v[13]), "+v"(v[14]), "+v"(v[15])                           \
                 : "v"(c))

template <int CTRL>
__device__ __forceinline__ void dpp_stage(float (&v)[16], float c) {
    if constexpr (CTRL == DPP_QUAD_XOR1) PQ2_DPP_FMAC16("quad_perm:[1,0,3,2]");
    else if constexpr (CTRL == DPP_QUAD_XOR2) PQ2_DPP_FMAC16("quad_perm:[2,3,0,1]");
    else if constexpr (CTRL == DPP_ROW_HALF_MIRROR) PQ2_DPP_FMAC16("row_half_mirror");
    else if constexpr (CTRL == DPP_ROW_MIRROR) PQ2_DPP_FMAC16("row_mirror");
    else static_assert(CTRL == DPP_QUAD_XOR1, "unsupported DPP pattern");
}
#undef PQ2_DPP_FMAC16

// Butterfly across lane halves (SWAP32) or across row pairs (16-lane rows),
// two registers at a time: the first swap gives every lane both operands of
// one element's butterfly (the lower-lane value first), every lane forms a+b
// and a-b, and the second swap sends each result to the lane owning it.
template <bool SWAP32>
__device__ __forceinline__ void swap_stage(float (&v)[16]) {
#pragma clang fp contract(off)
#pragma unroll
    for (int r = 0; r < 16; r += 2) {
        const auto s1 = SWAP32 ? __builtin_amdgcn_permlane32_swap(__float_as_uint(v[r]), __float_as_uint(v[r + 1]), false, false)
                               : __builtin_amdgcn_permlane16_swap(__float_as_uint(v[r]), __float_as_uint(v[r + 1]), false, false);
        const float a = __uint_as_float(s1[0]), b = __uint_as_float(s1[1]);
        const float sum = a + b, dif = a - b;
        const auto s2 = SWAP32 ? __builtin_amdgcn_permlane32_swap(__float_as_uint(sum), __float_as_uint(dif), false, false)
                               : __builtin_amdgcn_permlane16_swap(__float_as_uint(sum), __float_as_uint(dif), false, false);
        v[r] = __uint_as_float(s2[0]);
        v[r + 1] = __uint_as_float(s2[1]);
    }
}

// In-place normalised FWHT of the block held by the 64 lanes of one wave,
// lane l holding elements 16 fwht_row(l) + r in v[r].
__device__ __forceinline__ void fwht1024_regs(float (&v)[16], int l) {
#pragma clang fp contract(off)
    butterfly<1>(v); butterfly<2>(v); butterfly<4>(v); butterfly<8>(v);   // h = 1..8
    const int row = fwht_row(l);
    // after stage e_k the stored sign is (-1)^(e4 + ... + e_k); partners
    // differ only in e_k, so they always hold the same sign
    dpp_stage<DPP_QUAD_XOR1>(v, (row & 1) ? -1.0f : 1.0f);                 // h = 16
    dpp_stage<DPP_QUAD_XOR2>(v, (row & 2) ? -1.0f : 1.0f);                 // h = 32
    dpp_stage<DPP_ROW_HALF_MIRROR>(v, (row & 4) ? -1.0f : 1.0f);           // h = 64
    dpp_stage<DPP_ROW_MIRROR>(v, (row & 8) ? -1.0f : 1.0f);                // h = 128
    // lanes 16 and 32 apart share e4..e7, hence the sign: sum and difference
    // of two stored values carry it unchanged
    swap_stage<false>(v);                                                  // h = 256
    swap_stage<true>(v);                                                   // h = 512
    const float scale = (__builtin_popcount(row & 15) & 1) ? -1.0f / 32.0f : 1.0f / 32.0f;
#pragma unroll
    for (int r = 0; r < 16; ++r) v[r] = v[r] * scale;
}

// SwiGLU of one element, silu(g) * u with silu(g) = g / (1 + exp(-g))
// (src/ops.h:27-31): one rounded division and one rounded product, no
// contraction.  The FFN glue kernels all use this, so their values agree bit
// for bit.
__device__ __forceinline__ float swiglu1(float g, float u) {
#pragma clang fp contract(off)
    const float s = g / (1.0f + expf(-g));
    return s * u;
}

// Quantise the 32-element chunk held by the lane pair (l, l^1), 16 elements
// per lane, and store it as one block_q8_1 at `blk` (4-byte aligned, global or
// LDS).  d = amax/127 (IEEE division), id = 1/d or 0, q = round-half-away(x*id)
// clamped to +-127, s = sum q; d stored with the host's fp16 rounding.
__device__ __forceinline__ void quant_pair_store(const float (&v)[16], uint8_t * blk, int half) {
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
        // round half away from zero: with t = trunc(p) and f = p - t,
        // trunc(2p) = 2t + trunc(2f) (same signs), and trunc(2f) is sign(p)
        // exactly when |f| >= 1/2, so trunc(2p) - trunc(p) = lroundf(p)
        // (2p = p + p is exact; |p| <= 127.00002 here)
        const float prod = v[r] * id;
        int t = (int)(prod + prod) - (int)prod;
        t = t < -127 ? -127 : (t > 127 ? 127 : t);
        q[r] = t;
        sum += t;
    }
    sum += dpp_mov_i<DPP_QUAD_XOR1>(sum);
    uint32_t * out = reinterpret_cast<uint32_t *>(blk);
    if (half == 0) out[0] = f32_to_f16_away(d) | ((uint32_t)(sum & 0xffff) << 16);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        out[1 + 4 * half + k] = (uint32_t)(q[k] & 0xff) | ((uint32_t)(q[4 + k] & 0xff) << 8) |
                                ((uint32_t)(q[8 + k] & 0xff) << 16) |
                                ((uint32_t)(q[12 + k] & 0xff) << 24);
    }
}

// The one summation order of an RMSNorm sum of squares, shared by every
// kernel that normalises a row (the pre-pass kernels, the fused GEMVs, the
// chain), so that all of them compute the same fp64 total bit for bit:
//  * block b's partial: lane l adds the squares of its 16 elements
//    HBLK b + 16 fwht_row(l) + r, r = 0..15, in order (each square is exact in
//    fp64), then wave_sum_f64 adds the 64 lane sums as a balanced tree in lane
//    order;
//  * the total adds the block partials in block order 0, 1, ..., nhb - 1.
// nw waves call this together; wave w computes the partials of blocks w,
// w + nw, ... of each group of up to RMS_GROUP blocks into red (LDS,
// RMS_GROUP doubles), every thread then adds the group in block order.
// load(b, v) delivers the lane's 16 elements of block b; sync() is a
// workgroup barrier that also completes this thread's LDS stores.  Returns
// the total in every thread.
constexpr int RMS_GROUP = 64;
template <class Load, class Sync>
__device__ __forceinline__ double rms_sumsq(int nhb, double * red, int nw, int wave, int lane, Load load,
                                           Sync sync) {
    double tot = 0.0;
    for (int g = 0; g < nhb; g += RMS_GROUP) {
        const int nbg = nhb - g < RMS_GROUP ? nhb - g : RMS_GROUP;
        for (int b = wave; b < nbg; b += nw) {
            float v[16];
            load(g + b, v);
            double s = 0.0;
#pragma unroll
            for (int r = 0; r < 16; ++r) s += (double)v[r] * (double)v[r];
            s = wave_sum_f64(s);
            if (lane == 0) red[b] = s;
        }
        sync();
        for (int b = 0; b < nbg; ++b) tot += red[b];
        if (g + RMS_GROUP < nhb) sync();          // red is refilled by the next group
    }
    return tot;
}

}  // namespace pq2
