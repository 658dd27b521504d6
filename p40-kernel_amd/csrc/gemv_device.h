// gemv_device.h -- building blocks of the streaming decode GEMV shared by the
// per-launch kernels (gemv.hip) and the persistent chain kernel (chain.hip):
// the unit/slot geometry of a row width, explicit vmcnt waits, the buffer
// LDS-DMA of one unit, the two-row wave reduction and the branch-free matrix
// selection of a group.
#pragma once

#include "pq2_device.h"

namespace pq2 {

constexpr int SLOT_BYTES = 16 * PQ2_BYTES;   // 64 chunks = 16 blocks = 544 B

// Unit and slot geometry of the streaming kernels for rows of NB blocks.
template <int NB, int NT = 1>
struct NbSpec {
    static constexpr int NCH = 4 * NB;
    static constexpr int G = (NCH % 64 == 0 || NT >= 3) ? 1 : ((2 * NCH / 64) <= 8 ? 2 : 1);
    static constexpr int S = (G * NCH + 63) / 64;
    static constexpr int UB = G * PQ2_BYTES * NB;
    static constexpr int NPIECE = UB / 16;
    static constexpr int NPL = (NPIECE + 63) / 64;
    // LDS bytes per unit buffer: the slot windows (S * 544 + 16) and every
    // byte a full NPL-instruction DMA can write (1024 * NPL)
    static constexpr int LDSB = (S * SLOT_BYTES + 16 > 1024 * NPL) ? S * SLOT_BYTES + 16 : 1024 * NPL;
    static constexpr int SPLIT = (G == 2) ? NCH / 64 : -1;
    static constexpr bool PARTIAL = (G * NCH) % 64 != 0;   // last slot has idle lanes 32..63
    static_assert(UB % 16 == 0, "a unit is a whole number of 16-byte pieces");
};

// s_waitcnt vmcnt(N) with the other counters left open (gfx9 encoding:
// vmcnt[3:0] at bits 3:0, vmcnt[5:4] at 15:14, expcnt 6:4, lgkmcnt 11:8).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x0F70);
}

typedef __attribute__((address_space(3))) void lds_void;

// cache-policy operand of global_load_lds on gfx950: bit 1 = nt (non-temporal)
constexpr int CPOL_NT = 2;
// word 3 of a raw buffer descriptor on gfx9-family parts (32-bit data format,
// no swizzle): byte-addressed loads with the range check against num_records
constexpr int BUF_DW3 = 0x00020000;

// NPL 16-byte LDS-DMA pieces of one unit from a matrix of m_bytes bytes (the
// buffer range): piece k of lane l from byte unit_off + poff[k] into
// dst + 1024 k + 16 l; pieces past the range land as zeros.  (A free
// function: the buffer builtins inside a kernel lambda drop the kernel's
// host-side stub.)
template <int NPL>
__device__ __forceinline__ void unit_buffer_dma(const uint8_t * W, int m_bytes, uint32_t unit_off,
                                                const uint32_t * poff, uint8_t * dst) {
    const __amdgpu_buffer_rsrc_t rsrc =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(W), (short)0, m_bytes, BUF_DW3);
#pragma unroll
    for (int k = 0; k < NPL; ++k)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (lds_void *)(dst + 1024 * k), 16, unit_off + poff[k], 0, 0,
                                                 CPOL_NT);
}

// One 16-byte LDS-DMA piece per lane from byte `off` of a buffer of m_bytes
// bytes into dst + 16 lane; an offset at or past m_bytes lands zeros without
// a memory access.
__device__ __forceinline__ void tail_slot_dma(const uint8_t * W, uint32_t m_bytes, uint32_t off, uint8_t * dst) {
    const __amdgpu_buffer_rsrc_t rsrc =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(W), (short)0, (int)m_bytes, BUF_DW3);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (lds_void *)dst, 16, off, 0, 0, CPOL_NT);
}

// Reduce acc0 over lanes 0..63 and acc1 over lanes 0..63 at once:
// v_permlane32_swap folds the upper half of acc0 onto its lower half and the
// lower half of acc1 onto its upper half in one exchange, then one DPP tree
// sums each 32-lane half.  Row totals land in lanes 31 (acc0) and 63 (acc1).
__device__ __forceinline__ float wave_sum2_to_lanes31_63(float acc0, float acc1) {
    const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_int(acc0), __float_as_int(acc1), false, false);
    float v = __int_as_float(sw[0]) + __int_as_float(sw[1]);
    v += dpp_mov<DPP_QUAD_XOR1>(v);
    v += dpp_mov<DPP_QUAD_XOR2>(v);
    v += dpp_mov<DPP_ROW_HALF_MIRROR>(v);
    v += dpp_mov<DPP_ROW_MIRROR>(v);
    v += dpp_mov<DPP_ROW_BCAST15, 0xa>(v);
    return v;
}

// A group of up to MAX_GROUP matrices with the same n_in that multiply one
// activation: unit u of the group's unit space is unit u - u0[m] of matrix m,
// where m counts the starts u0[1..3] at or below u (entries past the last
// matrix hold the total, so no unit maps there).  A matrix's units are
// counted on their own (its last unit may hold fewer than G rows), so no
// unit straddles two matrices.
constexpr int MAX_GROUP = 4;

// Per-unit view of a group, without branches: the starts are monotone, so
// field F of the matrix owning unit u is F[0] + sum_k [u >= u0[k]] (F[k] -
// F[k-1]), k = 1..3, with the differences formed once at kernel start (a
// select between kernel-argument loads is turned into branches by the
// compiler).  GROUP = false: one matrix, no selection at all.
template <bool GROUP>
struct GroupSel {
    uint64_t w0, dw1, dw2, dw3;      // weight base and differences
    uint64_t y0, dy1, dy2, dy3;      // output base and differences
    int u1, u2, u3;                  // unit starts of matrices 1..3
    int n0, dn1, dn2, dn3;           // row counts and differences

    template <class M>
    __device__ __forceinline__ explicit GroupSel(const M & mg) {
        w0 = (uint64_t)mg.W[0];
        y0 = (uint64_t)mg.y[0];
        n0 = mg.n_out[0];
        if constexpr (GROUP) {
            dw1 = (uint64_t)mg.W[1] - w0; dw2 = (uint64_t)mg.W[2] - (uint64_t)mg.W[1];
            dw3 = (uint64_t)mg.W[3] - (uint64_t)mg.W[2];
            dy1 = (uint64_t)mg.y[1] - y0; dy2 = (uint64_t)mg.y[2] - (uint64_t)mg.y[1];
            dy3 = (uint64_t)mg.y[3] - (uint64_t)mg.y[2];
            u1 = mg.u0[1]; u2 = mg.u0[2]; u3 = mg.u0[3];
            dn1 = mg.n_out[1] - n0; dn2 = mg.n_out[2] - mg.n_out[1]; dn3 = mg.n_out[3] - mg.n_out[2];
        }
    }
    // fields of the matrix owning unit u; lu = u's index within it
    __device__ __forceinline__ void at(int u, const uint8_t *& W, float *& y, int & n_out, int & lu) const {
        if constexpr (!GROUP) {
            W = reinterpret_cast<const uint8_t *>(w0);
            y = reinterpret_cast<float *>(y0);
            n_out = n0;
            lu = u;
        } else {
            const uint64_t m1 = 0ull - (uint64_t)(u >= u1), m2 = 0ull - (uint64_t)(u >= u2),
                           m3 = 0ull - (uint64_t)(u >= u3);
            W = reinterpret_cast<const uint8_t *>(w0 + (dw1 & m1) + (dw2 & m2) + (dw3 & m3));
            y = reinterpret_cast<float *>(y0 + (dy1 & m1) + (dy2 & m2) + (dy3 & m3));
            const int k1 = (int)m1, k2 = (int)m2, k3 = (int)m3;
            n_out = n0 + (dn1 & k1) + (dn2 & k2) + (dn3 & k3);
            lu = u - ((u1 & k1) + ((u2 - u1) & k2) + ((u3 - u2) & k3));
        }
    }
};

}  // namespace pq2
