// chain.hip -- the decode chain as one persistent launch (gfx950).
//
// A decode token is a chain of dependent steps: grouped GEMVs whose input is
// the previous step's output (rotated and quantised, or RMS-normalised first)
// and the FFN glue.  Launched one by one, every step pays a launch boundary,
// a ramp (the first weight bytes arrive ~1 us after the workgroups start) and
// a tail.  Here one workgroup per CU runs all steps:
//   * between dependent phases every workgroup passes a grid-wide barrier: it
//     publishes its barrier count in its own flag word with an agent-scope
//     release store (no read-modify-write: a contended device-scope atomic is
//     serialised at the memory side, ~0.7 us per operation while HBM streams)
//     and wave 0 polls all flags, then acquires at agent scope; the number of
//     polls is bounded: a wait that gives up is counted in *status and sets
//     the workspace's abort word, which every later barrier and poll checks,
//     so every workgroup of a failed launch leaves within one wait bound;
//   * before it waits, every wave but wave 0 already issues the LDS-DMA of its
//     first weight units of the next GEMV step (the weights do not depend on
//     the barrier), so HBM keeps streaming through the barrier;
//   * wave 0 alone stores what other workgroups read (every wave's outputs
//     reach it through LDS), with device-coherent stores (cache policy sc1),
//     and never has weight DMAs in flight when it publishes its flag: one
//     vmcnt(0) then covers exactly the workgroup's stores, and the release's
//     L2 write-back finds none of them dirty;
//   * inputs written in the launch are read with device-scope loads (sc1)
//     after the barrier's acquire;
//   * a step's descriptor is copied into registers while the wave has no DMA
//     in flight (a descriptor load behind in-flight DMAs would wait for them).
// Each step computes exactly what its per-launch entry point computes: the
// unit/slot walk, chunk dots, row reductions, the fused RMSNorm / FWHT / Q8_1
// prologue and the SwiGLU glue are the same device code (gemv_device.h,
// fwht_device.h), with 8 waves per workgroup like the fused launches, so the
// results are bit-identical.
#include "fwht_device.h"
#include "gemv_device.h"
#include "host_state.h"
#include "../../include/bonsai_p40.h"

#include <cstring>
#include <vector>

using namespace pq2;

namespace {

constexpr int CW = 8;                // waves per workgroup
constexpr int CD = 2;                // units in flight per wave in the steady state
constexpr int CSL = CD + 1;          // ring slots per wave: also the prefetch depth
constexpr int CPOL_SC1 = 16;         // cache policy sc1: device-scope coherent access
constexpr int MAX_WG = BONSAI_P40_CHAIN_WORKSPACE_BYTES / 4 - 1;   // flag words
constexpr int ABORT_WORD = MAX_WG;   // the workspace's last word: set once a barrier wait gave up
constexpr int GLUE_ONLY = 4;         // device step kind: a glue phase and no GEMV
// polls of a barrier wait before it gives up (one device-coherent load round
// plus a short sleep each: some tens of milliseconds in all)
constexpr uint32_t CHAIN_SPIN_LIMIT = 1u << 16;

// Device form of the chain: a header, then one step per GEMV, each carrying
// the SwiGLU glue that precedes it (a glue step not followed by a GEMV step
// becomes a GLUE_ONLY step).
struct ChainHeader {
    int n_dev, n_public, pad0, pad1;
};
struct ChainStep {
    int kind, nb, n_units, glue;
    int n_out[MAX_GROUP];
    int u0[MAX_GROUP + 1];
    int gnblk;                       // glue: 1024-blocks
    const uint8_t * W[MAX_GROUP];
    float * y[MAX_GROUP];
    const void * x;
    const float * norm_w;
    const float * signs;
    const float * gg;                // glue: gate rows
    const float * gu;                // glue: up rows
    const float * gsigns;            // glue: signs (may be null)
    uint8_t * gq;                    // glue: Q8_1 output
    float eps;
    int pad[3];
};
static_assert(sizeof(ChainHeader) == 16 && sizeof(ChainStep) % 16 == 0, "plan layout");

// LDS arena layout of a GEMV step of NB-block rows: per-wave unit rings, the
// Q8_1 activation, and for the fused prologue the fp32 input, signs and norm
// weights of its 1024-blocks, then the RMS partial sums.
template <int NB>
struct Arena {
    using P = NbSpec<NB>;
    static constexpr int NHB = P::NCH / 32;
    static constexpr int RING = CW * CSL * P::LDSB;
    static constexpr int ACT = RING;
    static constexpr int ACT_BYTES = (Q81_BYTES * P::NCH + 1023) / 1024 * 1024;
    static constexpr int XS = ACT + ACT_BYTES;
    static constexpr int SS = XS + NHB * HBLK * 4;
    static constexpr int NS = SS + NHB * HBLK * 4;
    static constexpr int PART = NS + NHB * HBLK * 4;
    static constexpr int END_ROT = PART + 8 * NHB;      // with the fused prologue (one partial per block)
    static constexpr int END_Q8 = ACT + ACT_BYTES;      // Q8 input only
};
// every wave's outputs of a step pass through LDS to wave 0, and the glue's
// Q8_1 blocks are assembled there; the buffer lies past every ring, so the
// next step's prefetched units do not touch it
constexpr int OUT_OFF = Arena<136>::END_Q8;
constexpr int OUT_BYTES = CW * 64 * 4;
constexpr int ARENA_BYTES = OUT_OFF + OUT_BYTES;
static_assert(Arena<40>::END_ROT <= ARENA_BYTES && Arena<48>::END_ROT <= ARENA_BYTES, "arena");
static_assert(Arena<40>::RING <= OUT_OFF && Arena<48>::RING <= OUT_OFF, "output buffer past the rings");
static_assert((HBLK / QK8) * Q81_BYTES <= OUT_BYTES, "a glue block fits the output buffer");
static_assert(ARENA_BYTES <= 160 * 1024, "one workgroup per CU");

// Device-coherent store (written through to the point of coherence) that the
// compiler does not track: the only wave that issues these (wave 0) waits for
// them with an explicit vmcnt(0) before it publishes the workgroup's flag.
__device__ __forceinline__ void store_sc1(void * p, uint32_t v) {
    asm volatile("global_store_dword %0, %1, off sc1" : : "v"(p), "v"(v) : "memory");
}

// Grid-wide barrier number `target` (the flags count barriers passed, across
// launches), entered by all waves; wave 0 publishes and polls.  Returns false
// when the launch is being abandoned: this workgroup's wait gave up (counted
// in *status), or another workgroup's did (the abort word is set).
__device__ bool grid_barrier(uint32_t * flags, uint32_t target, uint32_t * status) {
    __shared__ uint32_t bar_ok;
    if (threadIdx.x < 64) {
        wait_vmcnt<0>();                           // this workgroup's stores are acknowledged
        uint32_t * abort_w = flags + ABORT_WORD;
        bool ok = __hip_atomic_load(abort_w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 0;
        if (ok) {
            // the release orders the step's outputs (written by this wave)
            // before the flag for every workgroup that acquires it
            if (threadIdx.x == 0)
                __hip_atomic_store(&flags[blockIdx.x], target, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
            const int nwg = gridDim.x;
            uint32_t polls = 0;
            while (true) {
                bool all = true;
                for (int i = threadIdx.x; i < nwg; i += 64) {
                    const uint32_t f = __hip_atomic_load(&flags[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    all = all && (int)(f - target) >= 0;
                }
                if (__builtin_amdgcn_ballot_w64(!all) == 0) break;
                if (__hip_atomic_load(abort_w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0) {
                    ok = false;
                    break;
                }
                if (++polls > CHAIN_SPIN_LIMIT) {
                    if (threadIdx.x == 0) {
                        if (status != nullptr)
                            __hip_atomic_fetch_add(status, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                        __hip_atomic_store(abort_w, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    }
                    ok = false;
                    break;
                }
                __builtin_amdgcn_s_sleep(1);
            }
            // pairs with the other workgroups' release stores: their outputs
            // are visible to every wave of this workgroup after the s_barrier
            if (ok) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
        }
        if (threadIdx.x == 0) bar_ok = ok ? 1u : 0u;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
    return bar_ok != 0;
}

// Unit numbering of the streaming GEMV (gemv_nb_kernel): grid-strided over
// all waves, groups of 8 consecutive units per XCD when the grid is a
// multiple of 8 workgroups.
__device__ __forceinline__ int chain_wave_index(int wave) {
    int gw = wave * gridDim.x + blockIdx.x;
    if ((gridDim.x & 7) == 0) {
        const int K = gridDim.x >> 3;
        const int t = wave * K + (blockIdx.x >> 3);
        gw = (((t >> 3) << 3) + (blockIdx.x & 7)) << 3 | (t & 7);
    }
    return gw;
}

__device__ __forceinline__ int units_of(int n_units, int gw, int NW) {
    return gw < n_units ? (n_units - 1 - gw) / NW + 1 : 0;
}

// Issue units [from, to) of this wave for a step of NB-block rows into its ring.
template <int NB>
__device__ __forceinline__ void issue_units(const GroupSel<true> & gs, uint8_t * arena, int gw, int NW, int wave,
                                            int lane, int from, int to) {
    using P = NbSpec<NB>;
    uint8_t * ring = arena + wave * CSL * P::LDSB;
    uint32_t poff[P::NPL];
#pragma unroll
    for (int k = 0; k < P::NPL; ++k) poff[k] = 16u * (uint32_t)min(lane + 64 * k, P::NPIECE - 1);
    for (int k = from; k < to; ++k) {
        const uint8_t * Wm;
        float * ym;
        int n_out_m, lu;
        gs.at(gw + k * NW, Wm, ym, n_out_m, lu);
        unit_buffer_dma<P::NPL>(Wm, n_out_m * (PQ2_BYTES * NB), (uint32_t)lu * (uint32_t)P::UB, poff,
                                ring + (k % CSL) * P::LDSB);
    }
}

// Prefetch of a GEMV step: this wave's first min(nu, CSL) units.  Returns
// how many were issued.
__device__ int prefetch_step(const ChainStep & nx, uint8_t * arena, int gw, int NW, int wave, int lane) {
    const int n = min(units_of(nx.n_units, gw, NW), CSL);
    const GroupSel<true> gs(nx);
    if (nx.nb == 40) issue_units<40>(gs, arena, gw, NW, wave, lane, 0, n);
    else if (nx.nb == 48) issue_units<48>(gs, arena, gw, NW, wave, lane, 0, n);
    else issue_units<136>(gs, arena, gw, NW, wave, lane, 0, n);
    return n;
}

template <int K>
__device__ __forceinline__ void wait_units(int younger) {
    // younger = unit DMAs of this wave issued after the one waited for
    if (younger >= 2) wait_vmcnt<2 * K>();
    else if (younger == 1) wait_vmcnt<K>();
    else wait_vmcnt<0>();
}

// Copy of device step d (or an empty step past the end) into registers.
__device__ __forceinline__ ChainStep load_step(const ChainStep * plan, int d, int n_dev) {
    ChainStep s{};
    if (d < n_dev) s = plan[d];
    else s.kind = -1;
    return s;
}

// LDS-DMA of device step d (a valid step: the caller clamps) into `dst`, by
// one wave: 48 dwords, one per lane (lanes past them re-read the last).
__device__ __forceinline__ void dma_step(const ChainStep * plan, int d, uint8_t * dst) {
    constexpr int NDW = (int)(sizeof(ChainStep) / 4);
    const int lane = threadIdx.x & 63;
    const uint32_t * src = reinterpret_cast<const uint32_t *>(plan + d) + min(lane, NDW - 1);
    __builtin_amdgcn_global_load_lds(src, (lds_void *)dst, 4, 0, 0);
}

// One GEMV step of NB-block rows.  `pf` units of this wave were issued before
// the step began (0 for the first step of the launch).  After its unit walk
// the wave copies device step d + 1 into `nx`; every wave but wave 0 then
// issues that step's first units and returns their count (0 for wave 0).
template <int NB, int KIND>
__device__ int gemv_step(const ChainStep & st, const ChainStep * plan, int d, int n_dev, ChainStep & nx,
                         uint8_t * arena, uint8_t * desc, int pf) {
    using P = NbSpec<NB>;
    using A = Arena<NB>;
    static_assert(KIND == BONSAI_P40_CHAIN_Q8 || A::END_ROT <= ARENA_BYTES, "arena");
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int gw = chain_wave_index(wave);
    const int NW = gridDim.x * CW;
    const int nu = units_of(st.n_units, gw, NW);
    const GroupSel<true> gs(st);
    uint8_t * ring = arena + wave * CSL * P::LDSB;
    uint8_t * act = arena + A::ACT;
    int issued = pf;

    // 1. the activation: DMA (device-coherent: it may be an earlier step's
    //    output); the first step of a launch issues it ahead of its first units
    if constexpr (KIND == BONSAI_P40_CHAIN_Q8) {
        const uint8_t * xq = static_cast<const uint8_t *>(st.x);
        constexpr int AB = Q81_BYTES * P::NCH;
        constexpr int NA = (AB + 1023) / 1024;
        for (int k = wave; k < NA; k += CW) {
            const int off = min(16 * (64 * k + lane), AB - 16);
            __builtin_amdgcn_global_load_lds(xq + off, (lds_void *)(act + 1024 * k), 16, 0, CPOL_SC1);
        }
    } else {
        const float * x = static_cast<const float *>(st.x);
        float * xst = reinterpret_cast<float *>(arena + A::XS);
        float * sst = reinterpret_cast<float *>(arena + A::SS);
        float * nst = reinterpret_cast<float *>(arena + A::NS);
        for (int b = wave; b < A::NHB; b += CW) {
#pragma unroll
            for (int j = 0; j < 4; ++j)
                __builtin_amdgcn_global_load_lds(x + HBLK * b + 256 * j + 4 * lane,
                                                 (lds_void *)(xst + HBLK * b + 256 * j), 16, 0, CPOL_SC1);
            if (st.signs != nullptr) {
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    __builtin_amdgcn_global_load_lds(st.signs + HBLK * b + 256 * j + 4 * lane,
                                                     (lds_void *)(sst + HBLK * b + 256 * j), 16, 0, 0);
            }
            if constexpr (KIND == BONSAI_P40_CHAIN_RMSNORM_FWHT) {
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    __builtin_amdgcn_global_load_lds(st.norm_w + HBLK * b + 256 * j + 4 * lane,
                                                     (lds_void *)(nst + HBLK * b + 256 * j), 16, 0, 0);
            }
        }
    }
    // the next step's descriptor, by LDS-DMA (read from LDS after the unit
    // walk: a register load now would wait for every DMA in flight)
    if (wave == 0) dma_step(plan, min(d + 1, n_dev - 1), desc);
    __builtin_amdgcn_sched_barrier(0);
    if (issued == 0) {
        const int n = min(nu, CD);
        issue_units<NB>(gs, arena, gw, NW, wave, lane, 0, n);
        issued = n;
        // the activation is older than these units: wait for it alone
        wait_units<P::NPL>(issued);
    } else {
        wait_vmcnt<0>();            // the prefetched units are older: everything
    }

    // 2. fused prologue: RMSNorm scale, signs, FWHT and Q8_1 of this wave's
    //    1024-blocks into the activation (the device code of the fused GEMV)
    if constexpr (KIND != BONSAI_P40_CHAIN_Q8) {
        const float * xst = reinterpret_cast<const float *>(arena + A::XS);
        const float * sst = reinterpret_cast<const float *>(arena + A::SS);
        const float * nst = reinterpret_cast<const float *>(arena + A::NS);
        const int row = fwht_row(lane);
        float rs = 1.0f;
        if constexpr (KIND == BONSAI_P40_CHAIN_RMSNORM_FWHT) {
            // the order of rms_sumsq, as the per-launch kernels
            static_assert(A::NHB <= RMS_GROUP, "one group of block partials");
            const double tot = rms_sumsq(
                A::NHB, reinterpret_cast<double *>(arena + A::PART), CW, wave, lane,
                [&](int b, float (&v)[16]) {
#pragma unroll
                    for (int r = 0; r < 16; ++r) v[r] = xst[HBLK * b + 16 * row + r];
                },
                [] {
                    __builtin_amdgcn_s_waitcnt(0xC07F);
                    __builtin_amdgcn_s_barrier();
                });
            rs = 1.0f / sqrtf((float)(tot / (double)(A::NHB * HBLK)) + st.eps);
        }
        for (int b = wave; b < A::NHB; b += CW) {
            float v[16];
#pragma unroll
            for (int r = 0; r < 16; ++r) v[r] = xst[HBLK * b + 16 * row + r];
            if constexpr (KIND == BONSAI_P40_CHAIN_RMSNORM_FWHT) {
#pragma clang fp contract(off)
#pragma unroll
                for (int r = 0; r < 16; ++r) v[r] = v[r] * rs * nst[HBLK * b + 16 * row + r];
            }
            if (st.signs != nullptr) {
#pragma clang fp contract(off)
#pragma unroll
                for (int r = 0; r < 16; ++r) v[r] *= sst[HBLK * b + 16 * row + r];
            }
            fwht1024_regs(v, lane);
            quant_pair_store(v, act + Q81_BYTES * (32 * b + (row >> 1)), row & 1);
        }
        __builtin_amdgcn_s_waitcnt(0xC07F);
    }
    __builtin_amdgcn_s_barrier();    // the whole activation is in LDS

    // 3. the lane's activation nibble planes, scale and bias per slot
    uint32_t ah[P::S][4], al[P::S][4];
    float da[P::S];
    int bias[P::S];
#pragma unroll
    for (int j = 0; j < P::S; ++j) {
        const int v = 64 * j + lane;
        const bool valid = v < P::G * P::NCH;
        int c = v >= P::NCH ? v - P::NCH : v;
        c = valid ? c : 0;
        const uint32_t * a = reinterpret_cast<const uint32_t *>(act + Q81_BYTES * c);
        const uint32_t ds = a[0];
        uint32_t aw[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) aw[k] = valid ? a[1 + k] : 0u;
        nib_planes(aw, ah[j], al[j]);
        da[j] = valid ? f16_bits_to_f32(ds & 0xffffu) : 0.0f;
        bias[j] = valid ? -(int)(int16_t)(ds >> 16) : 0;
    }
    const int cw = PQ2_BYTES * (lane >> 2) + 2 + 8 * (lane & 3);
    const int sh = cw & 3;
    const int cw_al = cw - sh;
    const int dwo = PQ2_BYTES * (lane >> 2);

    // 4. the unit walk of gemv_nb_kernel: wait for unit i, refill the ring,
    //    chunk dots, two-row reduction; outputs stay in lanes
    float ykeep = 0.0f;
    for (int i = 0; i < nu; ++i) {
        wait_units<P::NPL>(issued - 1 - i);
        __builtin_amdgcn_wave_barrier();
        // unit i + CD goes into the slot unit i - 1 used (consumed)
        if (issued < nu && issued <= i + CD) {
            issue_units<NB>(gs, arena, gw, NW, wave, lane, issued, issued + 1);
            ++issued;
        }
        const uint8_t * ub = ring + (i % CSL) * P::LDSB;
        float acc0 = 0.0f, acc1 = 0.0f;
#pragma unroll
        for (int j = 0; j < P::S; ++j) {
            const uint32_t * cpa = reinterpret_cast<const uint32_t *>(ub + cw_al + SLOT_BYTES * j);
            const uint32_t w0 = __builtin_amdgcn_alignbyte(cpa[1], cpa[0], sh);
            const uint32_t w1 = __builtin_amdgcn_alignbyte(cpa[2], cpa[1], sh);
            const uint32_t dwb = *reinterpret_cast<const uint16_t *>(ub + dwo + SLOT_BYTES * j);
            const int s = chunk_dot_nib(w0, w1, ah[j], al[j], bias[j]);
            const float ts = da[j] * (float)s;
            float dw = f16_bits_to_f32(dwb);
            if (P::PARTIAL && j == P::S - 1) dw = lane < 32 ? dw : 0.0f;
            if (P::G == 1 || j < P::SPLIT) acc0 = fmaf(dw, ts, acc0);
            else if (j > P::SPLIT) acc1 = fmaf(dw, ts, acc1);
            else if (lane < 32) acc0 = fmaf(dw, ts, acc0);
            else acc1 = fmaf(dw, ts, acc1);
        }
        if (P::G == 2) {
            const float v = wave_sum2_to_lanes31_63(acc0, acc1);
            const float t0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 31));
            const float t1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
            ykeep = (lane == 2 * i) ? t0 : ((lane == 2 * i + 1) ? t1 : ykeep);
        } else {
            const float t0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wave_sum_to_lane63(acc0)), 63));
            ykeep = (lane == i) ? t0 : ykeep;
        }
        __builtin_amdgcn_s_waitcnt(0xC07F);        // lgkmcnt(0): this slot's reads are done
        __builtin_amdgcn_wave_barrier();
    }
    // 5. outputs: every wave leaves its lanes' values in LDS; wave 0 stores
    //    them device-coherent (later steps of this launch read them) while
    //    the other waves issue the next step's first units
    wait_vmcnt<0>();                           // (wave 0: the descriptor DMA has landed)
    float * ost = reinterpret_cast<float *>(arena + OUT_OFF);
    ost[64 * wave + lane] = ykeep;
    __builtin_amdgcn_s_waitcnt(0xC07F);        // lgkmcnt(0)
    __builtin_amdgcn_s_barrier();              // also: every wave has left this step's ring
    // 6. the next step's descriptor from LDS
    nx = *reinterpret_cast<const ChainStep *>(desc);
    if (d + 1 >= n_dev) nx.kind = -1;
    if (wave == 0) {
        for (int w = 0; w < CW; ++w) {
            const int gww = chain_wave_index(w);
            const int nuw = units_of(st.n_units, gww, NW);
            if (lane < nuw * P::G) {
                const uint8_t * Wm;
                float * ym;
                int n_out_m, lu;
                gs.at(gww + (lane / P::G) * NW, Wm, ym, n_out_m, lu);
                const int row = lu * P::G + lane % P::G;
                if (row < n_out_m) store_sc1(ym + row, __float_as_uint(ost[64 * w + lane]));
            }
        }
        return 0;
    }
    if (nx.kind < 0 || nx.kind == GLUE_ONLY) return 0;
    return prefetch_step(nx, arena, gw, NW, wave, lane);
}

// The FFN glue phase: workgroup t finishes the 1024-blocks t, t + #wg, ...
// with wave 0 alone (the other waves may have the next step's units in
// flight): lane l loads the 16 gate and up values of its FWHT row with
// device-scope loads, forms SwiGLU, applies the signs, rotates and quantises
// -- bonsai_p40_swiglu_fwht_quant's arithmetic, element for element -- into
// LDS, and the block is copied out with device-coherent stores.
__device__ void glue_phase(const ChainStep & st, uint8_t * arena) {
    if (threadIdx.x >= 64) return;
    const int l = threadIdx.x, row = fwht_row(l);
    uint8_t * qb = arena + OUT_OFF;
    for (int b = blockIdx.x; b < st.gnblk; b += gridDim.x) {
        const float * g = st.gg + (size_t)HBLK * b + 16 * row;
        const float * u = st.gu + (size_t)HBLK * b + 16 * row;
        float v[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const float gv = __hip_atomic_load(g + r, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            const float uv = __hip_atomic_load(u + r, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            v[r] = swiglu1(gv, uv);
        }
        if (st.gsigns != nullptr) {
#pragma clang fp contract(off)
            const float * sg = st.gsigns + (size_t)HBLK * b + 16 * row;
#pragma unroll
            for (int r = 0; r < 16; ++r) v[r] *= sg[r];
        }
        fwht1024_regs(v, l);
        quant_pair_store(v, qb + (row >> 1) * Q81_BYTES, row & 1);
        __builtin_amdgcn_s_waitcnt(0xC07F);
        __builtin_amdgcn_wave_barrier();
        const uint32_t * src = reinterpret_cast<const uint32_t *>(qb);
        uint32_t * dst = reinterpret_cast<uint32_t *>(st.gq + (size_t)b * (HBLK / QK8) * Q81_BYTES);
        for (int i = l; i < (HBLK / QK8) * Q81_BYTES / 4; i += 64) store_sc1(dst + i, src[i]);
        __builtin_amdgcn_s_waitcnt(0xC07F);
        __builtin_amdgcn_wave_barrier();
    }
}

__global__ void __launch_bounds__(64 * CW)
chain_kernel(const ChainStep * __restrict__ plan, const ChainHeader * __restrict__ hdr, int n_public,
             uint32_t * __restrict__ flags, uint32_t * __restrict__ status) {
    __shared__ __attribute__((aligned(16))) uint8_t arena[ARENA_BYTES];
    __shared__ __attribute__((aligned(16))) uint8_t desc_lds[2][256];
    const int n_dev = hdr->n_dev;
    if (hdr->n_public != n_public) {               // the plan is not the one named
        if (blockIdx.x == 0 && threadIdx.x == 0 && status != nullptr)
            __hip_atomic_fetch_add(status, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return;
    }
    // a launch on a workspace whose abort word is set (an earlier launch gave
    // up and the workspace was not zero-filled again) does nothing
    if (__hip_atomic_load(flags + ABORT_WORD, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0) {
        if (blockIdx.x == 0 && threadIdx.x == 0 && status != nullptr)
            __hip_atomic_fetch_add(status, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return;
    }
    // every workgroup's flag equals the number of barriers the launches before
    // this one passed
    const uint32_t base = __hip_atomic_load(&flags[blockIdx.x], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    uint32_t nbar = 0;
    bool first = true;
    int pf = 0;
    ChainStep cur = load_step(plan, 0, n_dev);
    for (int d = 0; d < n_dev; ++d) {
        ChainStep nx;
        if (cur.glue) {
            if (!first && !grid_barrier(flags, base + (++nbar), status)) break;
            first = false;
            glue_phase(cur, arena);
        }
        if (cur.kind == GLUE_ONLY) {
            nx = load_step(plan, d + 1, n_dev);    // no prefetch into a glue-only step
            pf = 0;
        } else {
            if (!first && !grid_barrier(flags, base + (++nbar), status)) break;
            first = false;
            if (cur.nb == 40) {
                if (cur.kind == BONSAI_P40_CHAIN_Q8)
                    pf = gemv_step<40, BONSAI_P40_CHAIN_Q8>(cur, plan, d, n_dev, nx, arena, desc_lds[d & 1], pf);
                else if (cur.kind == BONSAI_P40_CHAIN_FWHT)
                    pf = gemv_step<40, BONSAI_P40_CHAIN_FWHT>(cur, plan, d, n_dev, nx, arena, desc_lds[d & 1], pf);
                else
                    pf = gemv_step<40, BONSAI_P40_CHAIN_RMSNORM_FWHT>(cur, plan, d, n_dev, nx, arena, desc_lds[d & 1], pf);
            } else if (cur.nb == 48) {
                if (cur.kind == BONSAI_P40_CHAIN_Q8)
                    pf = gemv_step<48, BONSAI_P40_CHAIN_Q8>(cur, plan, d, n_dev, nx, arena, desc_lds[d & 1], pf);
                else if (cur.kind == BONSAI_P40_CHAIN_FWHT)
                    pf = gemv_step<48, BONSAI_P40_CHAIN_FWHT>(cur, plan, d, n_dev, nx, arena, desc_lds[d & 1], pf);
                else
                    pf = gemv_step<48, BONSAI_P40_CHAIN_RMSNORM_FWHT>(cur, plan, d, n_dev, nx, arena, desc_lds[d & 1], pf);
            } else {
                pf = gemv_step<136, BONSAI_P40_CHAIN_Q8>(cur, plan, d, n_dev, nx, arena, desc_lds[d & 1], pf);
            }
        }
        cur = nx;
    }
    // the last phase's stores are acknowledged before the launch ends
    wait_vmcnt<0>();
}

bool aligned(const void * p, uintptr_t a) { return ((uintptr_t)p & (a - 1)) == 0; }

// Host check of one GEMV step into its device form; false if invalid.
bool make_gemv(const bonsai_p40_chain_step & s, ChainStep & d) {
    if (s.kind != BONSAI_P40_CHAIN_Q8 && s.kind != BONSAI_P40_CHAIN_FWHT && s.kind != BONSAI_P40_CHAIN_RMSNORM_FWHT)
        return false;
    if (s.n_in <= 0 || s.n_in % HBLK != 0) return false;
    d.kind = s.kind;
    d.x = s.x;
    d.norm_w = s.norm_w;
    d.signs = s.signs;
    d.eps = s.eps;
    d.nb = (int)(s.n_in / QK_PQ2);
    if (d.nb != 40 && d.nb != 48 && !(d.nb == 136 && s.kind == BONSAI_P40_CHAIN_Q8)) return false;
    if (s.x == nullptr || !aligned(s.x, s.kind == BONSAI_P40_CHAIN_Q8 ? 4 : 16)) return false;
    if (s.signs != nullptr && (s.kind == BONSAI_P40_CHAIN_Q8 || !aligned(s.signs, 16))) return false;
    if (s.kind == BONSAI_P40_CHAIN_RMSNORM_FWHT && (s.norm_w == nullptr || !aligned(s.norm_w, 16))) return false;
    if (s.n_mat < 1 || s.n_mat > MAX_GROUP) return false;
    const int G = d.nb == 40 ? NbSpec<40>::G : (d.nb == 48 ? NbSpec<48>::G : NbSpec<136>::G);
    int64_t u = 0;
    for (int m = 0; m < s.n_mat; ++m) {
        d.u0[m] = (int)u;
        if (s.W[m] == nullptr || s.y[m] == nullptr || !aligned(s.W[m], 16) || !aligned(s.y[m], 4)) return false;
        if (s.n_out[m] <= 0 || s.n_out[m] * PQ2_BYTES * d.nb >= ((int64_t)1 << 31)) return false;
        d.W[m] = static_cast<const uint8_t *>(s.W[m]);
        d.y[m] = s.y[m];
        d.n_out[m] = (int)s.n_out[m];
        u += (s.n_out[m] + G - 1) / G;
        if (u > (1 << 24)) return false;
    }
    // trailing entries repeat the last matrix (never selected: their units
    // start at the total)
    for (int m = s.n_mat; m < MAX_GROUP; ++m) {
        d.u0[m] = (int)u;
        d.W[m] = d.W[s.n_mat - 1];
        d.y[m] = d.y[s.n_mat - 1];
        d.n_out[m] = d.n_out[s.n_mat - 1];
    }
    d.u0[MAX_GROUP] = (int)u;
    d.n_units = (int)u;
    return true;
}

bool make_glue(const bonsai_p40_chain_step & s, ChainStep & d) {
    if (s.n_in <= 0 || s.n_in % HBLK != 0 || s.n_in > ((int64_t)HBLK << 20)) return false;
    if (s.x == nullptr || s.x2 == nullptr || s.q_out == nullptr) return false;
    if (!aligned(s.x, 4) || !aligned(s.x2, 4) || !aligned(s.q_out, 4)) return false;
    if (s.signs != nullptr && !aligned(s.signs, 16)) return false;
    d.glue = 1;
    d.gnblk = (int)(s.n_in / HBLK);
    d.gg = static_cast<const float *>(s.x);
    d.gu = s.x2;
    d.gsigns = s.signs;
    d.gq = static_cast<uint8_t *>(s.q_out);
    return true;
}

int rows_per_unit(int nb) { return nb == 40 ? NbSpec<40>::G : (nb == 48 ? NbSpec<48>::G : NbSpec<136>::G); }

int chain_grid() {
    const int cus = pq2host::device_info().cus;
    return cus < MAX_WG ? cus : MAX_WG;
}

}  // namespace

extern "C" {

int64_t bonsai_p40_chain_plan_bytes(int n_steps) {
    return n_steps <= 0 ? 0 : (int64_t)sizeof(ChainHeader) + (int64_t)n_steps * (int64_t)sizeof(ChainStep);
}

int bonsai_p40_chain_plan(const bonsai_p40_chain_step * steps, int n_steps, void * plan) {
    if (steps == nullptr || plan == nullptr || n_steps <= 0 || n_steps > (1 << 16)) return 1;
    if (!aligned(plan, 16)) return 1;
    // shapes and pointers first (no device needed): each glue step rides on
    // the GEMV step after it, or becomes a glue-only step
    std::vector<ChainStep> d;
    ChainStep pending{};
    bool has_pending = false;
    for (int i = 0; i < n_steps; ++i) {
        const bonsai_p40_chain_step & s = steps[i];
        if (s.kind == BONSAI_P40_CHAIN_SWIGLU) {
            if (has_pending) {                     // two glue steps in a row
                pending.kind = GLUE_ONLY;
                d.push_back(pending);
            }
            pending = ChainStep{};
            if (!make_glue(s, pending)) return 1;
            has_pending = true;
            continue;
        }
        ChainStep g = has_pending ? pending : ChainStep{};
        if (!make_gemv(s, g)) return 1;
        d.push_back(g);
        has_pending = false;
    }
    if (has_pending) {
        pending.kind = GLUE_ONLY;
        d.push_back(pending);
    }
    // each wave keeps its outputs of a step in its 64 lanes
    const int nw = chain_grid() * CW;
    if (nw <= 0) return 1;
    for (const ChainStep & c : d)
        if (c.kind != GLUE_ONLY && (int64_t)c.n_units > (int64_t)(64 / rows_per_unit(c.nb)) * nw) return 1;
    std::vector<uint8_t> img(sizeof(ChainHeader) + d.size() * sizeof(ChainStep));
    const ChainHeader h{(int)d.size(), n_steps, 0, 0};
    std::memcpy(img.data(), &h, sizeof h);
    std::memcpy(img.data() + sizeof h, d.data(), d.size() * sizeof(ChainStep));
    return (int)hipMemcpy(plan, img.data(), img.size(), hipMemcpyHostToDevice);
}

int bonsai_p40_chain_run(const void * plan, int n_steps, void * workspace, uint32_t * status,
                         bonsai_stream stream) {
    if (plan == nullptr || workspace == nullptr || n_steps <= 0 || n_steps > (1 << 16)) return 1;
    if (!aligned(plan, 16) || !aligned(workspace, 4)) return 1;
    const int grid = chain_grid();
    if (grid <= 0) return 1;
    const auto * h = static_cast<const ChainHeader *>(plan);
    hipLaunchKernelGGL(chain_kernel, dim3((unsigned)grid), dim3(64 * CW), 0, (hipStream_t)stream,
                       reinterpret_cast<const ChainStep *>(h + 1), h, n_steps, static_cast<uint32_t *>(workspace),
                       status);
    return (int)hipGetLastError();
}

}  // extern "C"
