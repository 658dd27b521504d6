// gemv.hip -- decode GEMV over the native 34-byte block_pq2_0 layout (gfx950).
//
// Contract: y[r] = sum_b sum_iqs (f16(d_w) * f16(d_a)) * sumi(r, b, iqs) where
// sumi = sum_k dot4((w >> 2k) & 0x03030303, a_k) - s is the integer chunk dot
// of src/pq2_0.h:149-191; replaces src/kernels/gemv_p40.cu:82-165,210-219.
// Integer chunk dots are exact; the fp32 sum is a lane-parallel tree instead
// of the host's sequential loop (compared within 1e-5 relative, normwise).
//
// Streaming design (fast path: n_in % 1024 == 0, W 16-byte aligned)
// ---------------------------------------------------------------------
// * Rows are contiguous runs of 34*nb bytes and nb % 8 == 0, so every row
//   starts 16-byte aligned.  A wave owns a "unit" of G consecutive rows
//   (G = 2 when 4*nb % 64 == 32, else 1) = G*34*nb contiguous bytes, and
//   streams it with fully coalesced 128-bit loads (64 lanes x 16 B = 1 KiB per
//   instruction) into registers, then into its private LDS buffer.  The next
//   unit's loads are in flight while the current unit is consumed.
// * In LDS the unit is read as a sequence of "slots" of 64 chunks (16 blocks,
//   544 bytes): lane l takes chunk 64j + l of slot j.  Since 4*nb*G is a
//   multiple of 64, every slot is full; with G = 2 one slot straddles the two
//   rows exactly at lane 32.  The lane's 8 code bytes start 2 bytes past a
//   dword boundary for even blocks, so it reads 3 aligned dwords and realigns
//   with v_alignbyte (a per-lane constant shift).
// * The permuted Q8_1 activation is staged once per workgroup into LDS as a
//   16-byte aligned plane of int8 words plus a {d_a as f32, -s} plane; each
//   slot reads its chunk's 8 words with two ds_read_b128.
// * The chunk dot is 8 v_dot4 with the -s bias as the accumulator seed; the
//   fp32 row partials are reduced across the wave with DPP (quad_perm,
//   row_half_mirror, row_mirror, row_bcast15/31) and lane 63 stores y.
// Any other shape or alignment takes a simple wave-per-row kernel.
#include "fwht_device.h"
#include "gemv_device.h"
#include "host_state.h"

#include <atomic>
#include <mutex>
#include "../../include/bonsai_p40.h"

#include <stdlib.h>

using namespace pq2;

namespace {

constexpr int GV_WAVES = 4;
constexpr int GV_THREADS = 64 * GV_WAVES;
constexpr int MAX_NPL = 17;                  // max 16-byte pieces per lane per unit

typedef uint32_t v4u __attribute__((ext_vector_type(4)));

struct StreamGeom {
    int nb, nchunk, G, unit_bytes, ubuf_pad, slots, npieces, npl;
    size_t lds_bytes;
};

inline StreamGeom stream_geom(int64_t n_in) {
    StreamGeom g{};
    g.nb = (int)(n_in / QK_PQ2);
    g.nchunk = 4 * g.nb;
    g.G = (g.nchunk % 64 == 0) ? 1 : 2;
    g.unit_bytes = g.G * PQ2_BYTES * g.nb;
    g.ubuf_pad = g.unit_bytes + 16;
    g.slots = g.G * g.nchunk / 64;
    g.npieces = g.unit_bytes / 16;
    g.npl = (g.npieces + 63) / 64;
    g.lds_bytes = (size_t)g.nchunk * 40 + (size_t)GV_WAVES * g.ubuf_pad;
    return g;
}

// Stage the permuted Q8_1 activation (36-byte blocks, 4-byte aligned) into
// LDS: act_q[c*8 + k] = activation word k of chunk c, act_sc[c] = {d_a, -s}.
__device__ __forceinline__ void stage_activation(const uint32_t * __restrict__ xw,
                                                 uint32_t * act_q, int2 * act_sc, int nchunk) {
    for (int m = threadIdx.x; m < nchunk * 9; m += blockDim.x) {
        const uint32_t v = xw[m];
        const int c = m / 9, k = m - 9 * c;
        if (k == 0)
            act_sc[c] = make_int2(__float_as_int(f16_bits_to_f32(v & 0xffffu)), -(int)(int16_t)(v >> 16));
        else
            act_q[8 * c + k - 1] = v;
    }
}

template <int G, int NPL, bool DUMP>
__global__ void __launch_bounds__(GV_THREADS)
gemv_stream_kernel(const uint8_t * __restrict__ W, const uint8_t * __restrict__ xq,
                   float * __restrict__ y, int32_t * __restrict__ dump, int n_out, int nb,
                   int units_per_wave) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    const int nchunk = 4 * nb;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    uint32_t * act_q = reinterpret_cast<uint32_t *>(smem);
    int2 * act_sc = reinterpret_cast<int2 *>(smem + (size_t)nchunk * 32);
    const int unit_bytes = G * PQ2_BYTES * nb;
    uint8_t * ubuf = smem + (size_t)nchunk * 40 + (size_t)wave * (unit_bytes + 16);

    stage_activation(reinterpret_cast<const uint32_t *>(xq), act_q, act_sc, nchunk);
    __syncthreads();

    const int n_units = (n_out + G - 1) / G;
    int u = (blockIdx.x * GV_WAVES + wave) * units_per_wave;
    const int u_end = min(u + units_per_wave, n_units);
    if (u >= u_end) return;   // no workgroup barrier below this point

    const size_t total_bytes = (size_t)n_out * PQ2_BYTES * nb;
    const int npieces = unit_bytes / 16;
    const int slots = G * nchunk / 64;

    // per-lane constants of the slot walk
    const int cw = PQ2_BYTES * (lane >> 2) + 2 + 8 * (lane & 3);   // code bytes of chunk `lane`
    const int sh = cw & 3;                                           // 2 (even block) or 0
    const int cw_al = cw - sh;
    const int dwo = PQ2_BYTES * (lane >> 2);                         // fp16 d of its block

    v4u r[NPL];
    auto load_unit = [&](int uu) {
        const uint8_t * src = W + (size_t)uu * unit_bytes;
        const size_t avail = total_bytes - (size_t)uu * unit_bytes;
#pragma unroll
        for (int k = 0; k < NPL; ++k) {
            const int p = lane + 64 * k;
            if (p < npieces && (size_t)16 * p < avail)
                r[k] = __builtin_nontemporal_load(reinterpret_cast<const v4u *>(src) + p);
        }
    };

    load_unit(u);
    for (; u < u_end; ++u) {
#pragma unroll
        for (int k = 0; k < NPL; ++k) {
            const int p = lane + 64 * k;
            if (p < npieces) *reinterpret_cast<v4u *>(ubuf + 16 * p) = r[k];
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        if (u + 1 < u_end) load_unit(u + 1);

        float acc0 = 0.0f, acc1 = 0.0f;
        for (int j = 0; j < slots; ++j) {
            const uint8_t * cp = ubuf + cw_al + SLOT_BYTES * j;
            const uint32_t d0 = *reinterpret_cast<const uint32_t *>(cp);
            const uint32_t d1 = *reinterpret_cast<const uint32_t *>(cp + 4);
            const uint32_t d2 = *reinterpret_cast<const uint32_t *>(cp + 8);
            const uint32_t w0 = __builtin_amdgcn_alignbyte(d1, d0, sh);
            const uint32_t w1 = __builtin_amdgcn_alignbyte(d2, d1, sh);
            const uint32_t dwb = *reinterpret_cast<const uint16_t *>(ubuf + dwo + SLOT_BYTES * j);
            const int v = 64 * j + lane;
            const bool second = (G == 2) && (v >= nchunk);
            const int c = second ? v - nchunk : v;
            const int4 a0 = *reinterpret_cast<const int4 *>(act_q + 8 * c);
            const int4 a1 = *reinterpret_cast<const int4 *>(act_q + 8 * c + 4);
            const int2 sc = act_sc[c];
            const int a[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
            const int s = chunk_dot_i32(w0, w1, a, sc.y);
            if (DUMP) {
                const int row = u * G + (second ? 1 : 0);
                if (row < n_out) dump[(size_t)row * nchunk + c] = s;
            } else {
                const float contrib = f16_bits_to_f32(dwb) * (__int_as_float(sc.x) * (float)s);
                if (second) acc1 += contrib; else acc0 += contrib;
            }
        }
        if (!DUMP) {
            const float t0 = wave_sum_to_lane63(acc0);
            const int row0 = u * G;
            if (lane == 63) y[row0] = t0;
            if (G == 2) {
                const float t1 = wave_sum_to_lane63(acc1);
                if (lane == 63 && row0 + 1 < n_out) y[row0 + 1] = t1;
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
}

// ---------------------------------------------------------------------------
// Shape-specialised streaming kernel (compile-time nb for the model's row
// widths).  Same unit/slot walk as gemv_stream_kernel, but
//   * one wave per workgroup, no workgroup barrier: each lane loads the Q8_1
//     blocks of exactly the chunks it multiplies into registers, once, and
//     keeps them for every unit (a unit's slot j always meets the same
//     activation chunk, (64j + lane) mod 4nb);
//   * the first unit's weight loads are issued before the activation loads;
//   * the slot loop is fully unrolled, so every LDS offset is an immediate
//     and the row of each slot is known at compile time;
//   * the chunk dot is the 16x-scaled form (one shift per code word), the
//   scale 1/16 folded into the activation scale.
// G = 1 when 4*nb % 64 == 0; otherwise G = 2 if that needs <= 8 slots, else
// G = 1 with a half-empty last slot whose idle lanes carry zero activations.
// With NT >= 3 tokens G = 1 (fewer slots, so the per-token activation planes
// fit in registers).

typedef int v4i_a4 __attribute__((ext_vector_type(4), aligned(4)));






// FFN epilogue of the gate/up group (EPI kernels only): hq = Q8_1(FWHT(h_signs
// .* swiglu(gate, up))) per 1024-block, each block as soon as its 1024 gate
// (y[0]) and 1024 up (y[1]) rows are stored.  The rows travel as the bitwise
// complement of their fp32 bits, so that a zero word means "not written in
// this launch" (no fp32 result of the GEMV has all bits set: a NaN it
// produces is quiet with a payload from an input or the default one); the
// block's finaliser clears them back to zero after reading them.  sync[1] is
// set to 1 when a finaliser gave up (the rows are then not all cleared and
// the workspace must be zero-filled again).  status (may be null) counts waits
// that gave up.
struct FfnEpilogue {
    uint32_t * sync;
    const float * h_signs;
    uint8_t * hq;
    uint32_t * status;
    int nblk;                   // 1024-blocks of the gate/up rows
};
struct MatGroup {
    const uint8_t * W[MAX_GROUP];
    float * y[MAX_GROUP];
    int n_out[MAX_GROUP];
    int u0[MAX_GROUP + 1];
    const float * norm_w;       // RMSNorm weights of the fused rotation (RMS kernels only)
    float eps;
    FfnEpilogue epi;
};

MatGroup single_group(const void * W, float * y, int64_t n_out) {
    MatGroup mg{};
    mg.W[0] = static_cast<const uint8_t *>(W);
    mg.y[0] = y;
    mg.n_out[0] = (int)n_out;
    return mg;
}


// LDS staging of the fp32 activation (and signs) for the fused rotation:
// block b at float 1024 b.  Function-scope LDS, so that only the kernels that
// use it allocate it.
template <int N>
__device__ __forceinline__ float * rot_x_stage() {
    __shared__ __attribute__((aligned(16))) float buf[N];
    return buf;
}
template <int N>
__device__ __forceinline__ float * rot_sign_stage() {
    __shared__ __attribute__((aligned(16))) float buf[N];
    return buf;
}
template <int N>
__device__ __forceinline__ float * rot_norm_stage() {
    __shared__ __attribute__((aligned(16))) float buf[N];
    return buf;
}
template <int N>
__device__ __forceinline__ double * rms_partials() {
    __shared__ double buf[N];
    return buf;
}

// Polls of an FFN block's wait before it gives up (each poll is 32
// device-coherent loads per lane plus a short sleep: some tens of
// milliseconds in all).
constexpr uint32_t EPI_SPIN_LIMIT = 1u << 16;

// One FFN block's glue by one wave: wait until the block's 1024 gate and 1024
// up rows are all written (a bounded poll of device-coherent loads), then
// SwiGLU, signs, FWHT and Q8_1 in registers, and clear the rows for the next
// launch.  The rows are single 32-bit atomic words, so a non-zero word read
// here is the writer's store itself and no further ordering is needed.  With
// `stage` (8 KiB of this wave's own LDS) the words are polled coalesced (lane
// l reads words 64 k + l) and reach the FWHT layout (lane l: the 16
// consecutive rows of its FWHT row) through LDS; without it each lane polls
// its 16 gate and 16 up rows directly.
__device__ __forceinline__ void ffn_finalise_block(const MatGroup & mg, int b, float * stage) {
    const FfnEpilogue & e = mg.epi;
    const int lane = threadIdx.x & 63;
    const int row = fwht_row(lane);
    uint32_t * g = reinterpret_cast<uint32_t *>(mg.y[0]) + (size_t)HBLK * b;
    uint32_t * u = reinterpret_cast<uint32_t *>(mg.y[1]) + (size_t)HBLK * b;
    // word k of this lane: index 64 k + lane (coalesced) or 16 row + k
    const int base = stage != nullptr ? lane : 16 * row;
    const int step = stage != nullptr ? 64 : 1;
    uint32_t gv[16], uv[16];
    uint32_t polls = 0;
    bool ok = false;
    for (;;) {
        bool have = true;
#pragma unroll
        for (int k = 0; k < 16; ++k) {
            gv[k] = __hip_atomic_load(g + base + step * k, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            uv[k] = __hip_atomic_load(u + base + step * k, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            have = have && gv[k] != 0u && uv[k] != 0u;
        }
        if (__builtin_amdgcn_ballot_w64(!have) == 0) {
            ok = true;
            break;
        }
        if (++polls > EPI_SPIN_LIMIT) break;
        __builtin_amdgcn_s_sleep(1);
    }
    if (!ok) {
        if (lane == 0) {
            if (e.status != nullptr) __hip_atomic_fetch_add(e.status, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(&e.sync[1], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        return;
    }
    float v[16];
    if (stage != nullptr) {
#pragma unroll
        for (int k = 0; k < 16; ++k) {
            stage[64 * k + lane] = __uint_as_float(~gv[k]);
            stage[HBLK + 64 * k + lane] = __uint_as_float(~uv[k]);
        }
        __builtin_amdgcn_s_waitcnt(0xC07F);        // lgkmcnt(0): the stores are done
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int r = 0; r < 16; ++r) v[r] = swiglu1(stage[16 * row + r], stage[HBLK + 16 * row + r]);
    } else {
#pragma unroll
        for (int r = 0; r < 16; ++r) v[r] = swiglu1(__uint_as_float(~gv[r]), __uint_as_float(~uv[r]));
    }
    if (e.h_signs != nullptr) {
        const float * sg = e.h_signs + (size_t)HBLK * b + 16 * row;
#pragma unroll
        for (int r = 0; r < 16; ++r) v[r] *= sg[r];
    }
    fwht1024_regs(v, lane);
    quant_pair_store(v, e.hq + ((size_t)b * (HBLK / QK8) + (row >> 1)) * Q81_BYTES, row & 1);
    // (the loads above are complete: their values were used)
#pragma unroll
    for (int k = 0; k < 16; ++k) {
        __hip_atomic_store(g + base + step * k, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(u + base + step * k, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// The finalising quad's LDS words: [0] quarters in LDS, [1] a quarter's
// wait gave up.  Function-scope LDS, so only the FFN-epilogue kernels
// allocate it.
__device__ __forceinline__ uint32_t * ffn_quad_words() {
    __shared__ uint32_t w[2];
    return w;
}

// One FFN block's glue by four waves of one workgroup (quarter h = 0..3 of
// the block, h = 3 also runs the rotation): each wave polls its quarter of
// the block's gate and up words (lane l: words 256 h + 64 k + l, k < 4),
// runs SwiGLU on them into its own LDS ring (1 KiB), clears the words and
// counts itself in the workgroup's quad counter; the h = 3 wave waits
// (bounded) for the four quarters, then reads the block in the FWHT layout
// from the four rings, applies the signs, rotates and quantises.  quarter_lds
// points at each wave's own 1 KiB; lds_of(q) at quarter q's.
template <class F>
__device__ __forceinline__ void ffn_finalise_quarter(const MatGroup & mg, int b, int h, float * quarter_lds,
                                                     F lds_of) {
    const FfnEpilogue & e = mg.epi;
    const int lane = threadIdx.x & 63;
    uint32_t * g = reinterpret_cast<uint32_t *>(mg.y[0]) + (size_t)HBLK * b + 256 * h + lane;
    uint32_t * u = reinterpret_cast<uint32_t *>(mg.y[1]) + (size_t)HBLK * b + 256 * h + lane;
    uint32_t * qw = ffn_quad_words();
    uint32_t gv[4], uv[4];
    uint32_t polls = 0;
    bool ok = false;
    for (;;) {
        bool have = true;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            gv[k] = __hip_atomic_load(g + 64 * k, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            uv[k] = __hip_atomic_load(u + 64 * k, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            have = have && gv[k] != 0u && uv[k] != 0u;
        }
        if (__builtin_amdgcn_ballot_w64(!have) == 0) {
            ok = true;
            break;
        }
        if (++polls > EPI_SPIN_LIMIT) break;
        __builtin_amdgcn_s_sleep(1);
    }
    if (ok) {
#pragma unroll
        for (int k = 0; k < 4; ++k) quarter_lds[64 * k + lane] = swiglu1(__uint_as_float(~gv[k]), __uint_as_float(~uv[k]));
        // (the loads above are complete: their values were used)
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            __hip_atomic_store(g + 64 * k, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(u + 64 * k, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    } else if (lane == 0) {
        if (e.status != nullptr) __hip_atomic_fetch_add(e.status, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(&e.sync[1], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(&qw[1], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
    // publish the quarter to the rotating wave: its LDS stores, then the count
    __builtin_amdgcn_s_waitcnt(0xC07F);            // lgkmcnt(0)
    if (lane == 0) __hip_atomic_fetch_add(&qw[0], 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
    if (h != 3) return;
    polls = 0;
    while (__hip_atomic_load(&qw[0], __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) < 4u) {
        if (++polls > EPI_SPIN_LIMIT) break;
        __builtin_amdgcn_s_sleep(1);
    }
    if (polls > EPI_SPIN_LIMIT || __hip_atomic_load(&qw[1], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) != 0u) {
        if (polls > EPI_SPIN_LIMIT && lane == 0) {
            if (e.status != nullptr) __hip_atomic_fetch_add(e.status, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(&e.sync[1], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        return;
    }
    const int row = fwht_row(lane);
    // the FWHT row's 16 elements lie in quarter (16 row) / 256
    const float * src = lds_of((16 * row) >> 8) + ((16 * row) & 255);
    float v[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) v[r] = src[r];
    if (e.h_signs != nullptr) {
        const float * sg = e.h_signs + (size_t)HBLK * b + 16 * row;
#pragma unroll
        for (int r = 0; r < 16; ++r) v[r] *= sg[r];
    }
    fwht1024_regs(v, lane);
    quant_pair_store(v, e.hq + ((size_t)b * (HBLK / QK8) + (row >> 1)) * Q81_BYTES, row & 1);
}

// Workgroup of WAVES waves.  Each wave owns up to `units_per_wave` units
// (grid-strided) and a private ring of D unit buffers in LDS; the workgroup shares one
// LDS copy of the Q8_1 activation.  Every weight read is an LDS DMA
// (global_load_lds_dwordx4), so the only waits are the explicit vmcnt waits
// below, and each unit is consumed as soon as its own bytes have landed.
//
// ROT = 0: `xin` is the permuted Q8_1 activation, DMA'd into LDS.
// ROT = 1 (2 with signs): `xin` is the fp32 activation; the workgroup itself
// computes Q8_1(FWHT(signs .* x)) into the same LDS block layout, wave w
// taking the Hadamard blocks w, w + WAVES, ..., while its first weight units
// are in flight.  x (and signs) reach LDS by DMA issued before any weight
// DMA, so one explicit vmcnt wait covers them and leaves the weights
// outstanding (a register load would make the compiler wait for everything
// issued after it).
//
// NT > 1 (small batch, n_tok <= NT tokens): xin is the chunk-major Q8_1 of
// the tokens (block (c, t) at c n_tok + t, the GEMM's X layout); every lane
// keeps the nibble planes of its chunk for each token, so a unit's code words
// are extracted once and dotted against NT activations.  Tokens past n_tok
// have zero planes; y is [n_out][n_tok].
//
// ROT = 3 quantises the fp32 activation without the rotation.  RP: the
// weights are in the aligned repacked layout (a row's fp16 scales first, then
// unit p*nb + b = the 8 code bytes of chunk p of block b): the DMA moves the
// same rows, only the lane's LDS offsets change (8-byte aligned code words,
// no realignment).
// whether a variant can run the shared tail (two 1 KiB DMA areas per ring
// slot, the plain single-token unit layout)
template <int NB, int NT, bool RP, bool DUMP, bool EPI>
constexpr bool nb_tail_ok() {
    return NT == 1 && !RP && !DUMP && !EPI && NbSpec<NB, NT>::LDSB >= 2048 && NbSpec<NB, NT>::S <= 16;
}

template <int NB, int D, int WAVES, bool DUMP, int ROT = 0, bool GROUP = false, int NT = 1, bool RP = false,
          bool RMS = false, bool OVL = false, bool EPI = false>
__global__ void __launch_bounds__(64 * WAVES)
gemv_nb_kernel(const MatGroup mg, const void * __restrict__ xin, const float * __restrict__ signs,
               int32_t * __restrict__ dump, int units_per_wave, int n_tok, int xcd_log2m, int tail) {
    using P = NbSpec<NB, NT>;
    static_assert(NT == 1 || (!DUMP && ROT == 0 && !GROUP), "small batch: plain GEMV only");
    static_assert(!RP || (NT == 1 && !GROUP && !DUMP), "repacked layout: single-token GEMV only");
    static_assert(D >= 1 && D <= 3, "ring depth");
    static_assert(D * P::NPL < 64, "vmcnt range");
    static_assert(ROT == 0 || P::NCH % 32 == 0, "the rotation needs whole 1024-element blocks");
    static_assert(!RMS || ROT == 1 || ROT == 2, "RMSNorm rides on the fused rotation");
    static_assert(!OVL || (ROT == 1 && !RMS && !RP && NT == 1), "ring-staged rotation: plain FWHT");
    static_assert(!EPI || (GROUP && NT == 1 && !DUMP && !RP), "FFN epilogue: the gate/up group");
    constexpr int ACT_BYTES = Q81_BYTES * P::NCH * NT;
    constexpr int NA = (ACT_BYTES + 1023) / 1024;          // activation DMA instructions
    constexpr int NHB = P::NCH / 32;                       // Hadamard blocks of the row
    __shared__ __attribute__((aligned(16))) uint8_t act_lds[NA * 1024];
    // D units in flight per wave, D + 1 ring slots: the next unit is issued as
    // soon as the current one has landed, before it is computed
    constexpr int SL = D + 1;
    __shared__ __attribute__((aligned(16))) uint8_t ring_all[WAVES][SL][P::LDSB];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    __builtin_assume(lane >= 0 && lane < 64);
    uint8_t (*ring)[P::LDSB] = ring_all[wave];
    const int n_units = mg.u0[MAX_GROUP];
    const GroupSel<GROUP> gs(mg);
    // units are dealt to waves grid-strided: wave gw owns units gw, gw + NW,
    // gw + 2 NW, ...  Every issue round then reads one contiguous stretch of
    // W across the whole grid; a contiguous per-wave span of 3 units
    // (8160 B at 17408x5120) measured 15 % slower (HBM channel camping).
    // slot-major wave numbering: the waves that carry one unit more than the
    // others are spread over all workgroups (hence all CUs) rather than packed
    // into the first ones
    // XCD-aware numbering (xcd_log2m > 0, grid a multiple of 8 workgroups,
    // which the dispatcher deals round-robin to the 8 XCDs): within a round
    // of NW units, groups of M = 2^xcd_log2m consecutive units go to one XCD
    // (its waves numbered wave-major), groups round-robin over the XCDs -- a
    // line shared by two neighbouring units is then fetched into one L2.
    auto wave_index = [&](int w) {
        if (xcd_log2m <= 0) return w * (int)gridDim.x + (int)blockIdx.x;
        const int K = gridDim.x >> 3;
        const int t = w * K + (blockIdx.x >> 3);
        const int m = (1 << xcd_log2m) - 1;
        return (((t >> xcd_log2m) << 3) + (int)(blockIdx.x & 7)) << xcd_log2m | (t & m);
    };
    const int gw = wave_index(wave);
    const int NW = gridDim.x * WAVES;
    int nu = gw < n_units ? min(units_per_wave, (n_units - 1 - gw) / NW + 1) : 0;
    // Shared tail (tail = T > 0, set by the dispatcher only when the last
    // round of units is exactly the last units of waves 0..T-1 of every
    // workgroup and every wave has at least D + 1 units): those T units leave
    // their waves' loops; their T * S slots are dealt over all the
    // workgroup's waves (slot q = k S + j of tail unit k to wave q % WAVES).
    // Each wave DMAs its slots (one 544-byte slot per instruction) ahead of
    // its first unit and computes their chunk dots while its first units
    // land, keeping the products (dw, da s) in registers; after the loops the
    // products meet in LDS and wave k folds unit k's slots in slot order with
    // the loop's own FMA sequence -- y is bit-identical to the
    // one-wave-per-unit schedule, and no wave carries a whole extra unit.
    const int T = nb_tail_ok<NB, NT, RP, DUMP, EPI>() ? tail : 0;
    if (T > 0 && wave < T) --nu;
    // EPI: tail != 0 means the launch's last round of units falls on waves
    // below WAVES / 2 of every workgroup, so waves WAVES / 2 .. WAVES - 1 have
    // the fewest units: those of workgroups 0 .. nblk - 1 finalise block
    // blockIdx.x as a quad
    const bool epi_quad = EPI && WAVES == 8 && tail != 0 && (int)blockIdx.x < mg.epi.nblk;
    if constexpr (EPI) {
        if (epi_quad && threadIdx.x == 0) {
            ffn_quad_words()[0] = 0u;
            ffn_quad_words()[1] = 0u;
        }
    }

    // OVL: the fp32 blocks are staged in the unit ring itself (the widest rows,
    // where a separate stage does not fit beside an 8-wave ring): slots k =
    // 0..NBW-1 of a wave hold blocks min(wave + WAVES k, NHB - 1) in registers
    constexpr int NBW = OVL ? (NHB + WAVES - 1) / WAVES : 1;
    float xr[NBW][16];

    // 1. activation: ROT = 0 -- this wave's share of the Q8_1 DMA
    //    (instructions k = wave, wave + WAVES, ...); ROT > 0 -- the fp32
    //    blocks (and signs) of this wave into its staging areas
    if constexpr (ROT == 0) {
        const uint8_t * xq = static_cast<const uint8_t *>(xin);
        const int act_bytes = NT == 1 ? ACT_BYTES : Q81_BYTES * P::NCH * n_tok;
        const int na = NT == 1 ? NA : (act_bytes + 1023) / 1024;
        for (int k = wave; k < na; k += WAVES) {
            const int off = min(16 * (64 * k + lane), act_bytes - 16);
            __builtin_amdgcn_global_load_lds(xq + off, (lds_void *)(&act_lds[1024 * k]), 16, 0, 0);
        }
    } else if constexpr (OVL) {
        // the blocks go through the ring before any unit: DMA, wait for all of
        // it (nothing else is in flight), copy the wave's blocks into
        // registers, and release the ring with a workgroup barrier
        static_assert(NHB * HBLK * 4 <= WAVES * SL * P::LDSB, "the staged blocks fit in the ring");
        const float * x = static_cast<const float *>(xin);
        float * xst = reinterpret_cast<float *>(&ring_all[0][0][0]);
        for (int b = wave; b < NHB; b += WAVES) {
#pragma unroll
            for (int j = 0; j < 4; ++j)
                __builtin_amdgcn_global_load_lds(x + HBLK * b + 256 * j + 4 * lane,
                                                 (lds_void *)(xst + HBLK * b + 256 * j), 16, 0, 0);
        }
        wait_vmcnt<0>();
        const int xrow = fwht_row(lane);
#pragma unroll
        for (int k = 0; k < NBW; ++k) {
            const float * xb = xst + HBLK * min(wave + WAVES * k, NHB - 1) + 16 * xrow;
#pragma unroll
            for (int r = 0; r < 16; ++r) xr[k][r] = xb[r];
        }
        __builtin_amdgcn_s_waitcnt(0xC07F);        // lgkmcnt(0): the wave's reads are done
        __builtin_amdgcn_s_barrier();
    } else {
        const float * x = static_cast<const float *>(xin);
        float * xst = rot_x_stage<NHB * HBLK>();
        for (int b = wave; b < NHB; b += WAVES) {
#pragma unroll
            for (int j = 0; j < 4; ++j)
                __builtin_amdgcn_global_load_lds(x + HBLK * b + 256 * j + 4 * lane,
                                                 (lds_void *)(xst + HBLK * b + 256 * j), 16, 0, 0);
            if constexpr (ROT == 2) {
                float * sst = rot_sign_stage<NHB * HBLK>();
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    __builtin_amdgcn_global_load_lds(signs + HBLK * b + 256 * j + 4 * lane,
                                                     (lds_void *)(sst + HBLK * b + 256 * j), 16, 0, 0);
            }
            if constexpr (RMS) {
                float * nst = rot_norm_stage<NHB * HBLK>();
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    __builtin_amdgcn_global_load_lds(mg.norm_w + HBLK * b + 256 * j + 4 * lane,
                                                     (lds_void *)(nst + HBLK * b + 256 * j), 16, 0, 0);
            }
        }
    }
    __builtin_amdgcn_sched_barrier(0);

    // 2. the first D units.  Unit i is exactly NPL instructions; lanes past
    //    the unit re-read its last piece (landing in LDS past the unit bytes).
    //    A full unit's pieces are a uniform base plus a per-lane 32-bit offset;
    //    only a trailing unit with fewer than G rows clamps to the end of W.
    uint32_t poff[P::NPL];
#pragma unroll
    for (int k = 0; k < P::NPL; ++k) poff[k] = 16u * (uint32_t)min(lane + 64 * k, P::NPIECE - 1);
    auto issue = [&](int uu, int slot) {
        const uint8_t * Wm;
        float * ym;
        int n_out_m, lu;
        gs.at(uu, Wm, ym, n_out_m, lu);
        const uint64_t m_bytes = (uint64_t)n_out_m * (PQ2_BYTES * NB);
        if (m_bytes < 0x80000000ull) {
            // buffer DMA with the matrix as the range: the unit offset is one
            // add per piece, and a piece past the end (a trailing unit with
            // fewer than G rows) reads zeros instead of memory
            unit_buffer_dma<P::NPL>(Wm, (int)m_bytes, (uint32_t)lu * (uint32_t)P::UB, poff, ring[slot]);
            return;
        }
        const uint8_t * base = Wm + (size_t)lu * P::UB;
        const bool full = lu < n_out_m / P::G;              // all G rows present
        const size_t last_piece = (size_t)n_out_m * PQ2_BYTES * NB / 16 - 1;
#pragma unroll
        for (int k = 0; k < P::NPL; ++k) {
            const uint8_t * src = base + poff[k];
            if (!full) {
                size_t p = (size_t)lu * (P::UB / 16) + poff[k] / 16;
                src = Wm + 16 * (p < last_piece ? p : last_piece);
            }
            // nt: weights stream through L2 without displacing the activation
            __builtin_amdgcn_global_load_lds(src, (lds_void *)(&ring[slot][1024 * k]), 16, 0, CPOL_NT);
        }
    };
    // shared tail: this wave's (up to two) tail slots, one DMA instruction
    // each into ring slot D (free until step 0 issues unit D into it), older
    // than every unit; an instruction without a slot reads past the buffer
    // range (zeros, no memory traffic)
    if (T > 0) {
#pragma unroll
        for (int r = 0; r < 2; ++r) {
            const int q = wave + WAVES * r;
            const int k = q < T * P::S ? q / P::S : 0;
            const uint8_t * Wm;
            float * ym;
            int n_out_m, lu;
            gs.at(wave_index(k) + (units_per_wave - 1) * NW, Wm, ym, n_out_m, lu);
            const uint32_t m_bytes = (uint32_t)n_out_m * (uint32_t)(PQ2_BYTES * NB);
            uint32_t off = m_bytes;
            if (q < T * P::S && lane < SLOT_BYTES / 16)
                off = (uint32_t)lu * (uint32_t)P::UB + (uint32_t)(SLOT_BYTES * (q - k * P::S) + 16 * lane);
            tail_slot_dma(Wm, m_bytes, off, &ring[D][1024 * r]);
        }
    }
    // issue rounds: every wave's activation share, then every wave's first
    // unit, then every second unit, ...  A CU serves its requests roughly in
    // issue order, so the barrier between rounds keeps each wave's first
    // bytes (and the shared activation) ahead of the other waves' later units
    // instead of queued behind them.
#pragma unroll
    for (int i = 0; i < D; ++i) {
        __builtin_amdgcn_s_barrier();
        if (nu > 0) issue(gw + min(i, nu - 1) * NW, i);
        __builtin_amdgcn_sched_barrier(0);
    }

    if constexpr (ROT == 0) {
        // 3. own activation share landed (all unit DMAs are younger), then the
        //    workgroup barrier makes every share visible
        if (nu > 0) wait_vmcnt<D * P::NPL>();
        else wait_vmcnt<0>();
        __builtin_amdgcn_s_barrier();
        if (nu <= 0 && !EPI) return;   // (EPI: every wave reaches the epilogue)
    } else if constexpr (OVL) {
        // 3. rotate and quantise the register blocks (a repeated one is rotated
        //    and not stored) while the first units stream in, then the barrier
        const int xrow = fwht_row(lane);
#pragma unroll
        for (int k = 0; k < NBW; ++k) {
            const int b = wave + WAVES * k;
            float v[16];
#pragma unroll
            for (int r = 0; r < 16; ++r) v[r] = xr[k][r];
            fwht1024_regs(v, lane);
            if (b < NHB) quant_pair_store(v, &act_lds[Q81_BYTES * (32 * b + (xrow >> 1))], xrow & 1);
        }
        __builtin_amdgcn_s_waitcnt(0xC07F);        // lgkmcnt(0): this wave's LDS stores are done
        __builtin_amdgcn_s_barrier();
        if (nu <= 0 && !EPI) return;   // (EPI: every wave reaches the epilogue)
    } else {
        // 3. own staged blocks landed (all unit DMAs are younger); rotate and
        //    quantise them into the LDS activation (chunk c of block b at byte
        //    36 (32 b + c)), then the workgroup barrier makes every block visible
        if (nu > 0) wait_vmcnt<D * P::NPL>();
        else wait_vmcnt<0>();
        const int row = fwht_row(lane);
        // RMSNorm scale: the fp64 sum of squares in the order of rms_sumsq
        // (block partials of the waves, added in block order), the same in
        // every workgroup and in every other normalising kernel
        float rs = 1.0f;
        if constexpr (RMS) {
            static_assert(NHB <= RMS_GROUP, "one group of block partials");
            const float * xst = rot_x_stage<NHB * HBLK>();
            const double tot = rms_sumsq(
                NHB, rms_partials<NHB>(), WAVES, wave, lane,
                [&](int b, float (&v)[16]) {
#pragma unroll
                    for (int r = 0; r < 16; ++r) v[r] = xst[HBLK * b + 16 * row + r];
                },
                [] {   // LDS only: the unit DMAs stay in flight
                    __builtin_amdgcn_s_waitcnt(0xC07F);
                    __builtin_amdgcn_s_barrier();
                });
            rs = 1.0f / sqrtf((float)(tot / (double)(NHB * HBLK)) + mg.eps);
        }
        for (int b = wave; b < NHB; b += WAVES) {
            const float * xb = rot_x_stage<NHB * HBLK>() + HBLK * b + 16 * row;
            float v[16];
#pragma unroll
            for (int r = 0; r < 16; ++r) v[r] = xb[r];
            if constexpr (RMS) {
#pragma clang fp contract(off)
                const float * nb_ = rot_norm_stage<NHB * HBLK>() + HBLK * b + 16 * row;
#pragma unroll
                for (int r = 0; r < 16; ++r) v[r] = v[r] * rs * nb_[r];
            }
            if constexpr (ROT == 2) {
#pragma clang fp contract(off)
                const float * sb = rot_sign_stage<NHB * HBLK>() + HBLK * b + 16 * row;
#pragma unroll
                for (int r = 0; r < 16; ++r) v[r] *= sb[r];
            }
            if constexpr (ROT != 3) fwht1024_regs(v, lane);
            quant_pair_store(v, &act_lds[Q81_BYTES * (32 * b + (row >> 1))], row & 1);
        }
        __builtin_amdgcn_s_waitcnt(0xC07F);        // lgkmcnt(0): this wave's LDS stores are done
        __builtin_amdgcn_s_barrier();
        if (nu <= 0 && !EPI) return;   // (EPI: every wave reaches the epilogue)
    }

    // the lane's chunk of slot j is the same in every unit: its activation
    // nibble planes, scale and -s bias stay in registers
    uint32_t ah[NT][P::S][4], al[NT][P::S][4];
    float da[NT][P::S];
    int bias[NT][P::S];
#pragma unroll
    for (int j = 0; j < P::S; ++j) {
        const int v = 64 * j + lane;
        const bool valid = v < P::G * P::NCH;
        int c = v >= P::NCH ? v - P::NCH : v;
        c = valid ? c : 0;
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const bool tv = valid && (NT == 1 || t < n_tok);
            const int blk = NT == 1 ? c : (tv ? c * n_tok + t : 0);
            const uint32_t * a = reinterpret_cast<const uint32_t *>(&act_lds[Q81_BYTES * blk]);
            const uint32_t ds = a[0];
            uint32_t aw[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) aw[k] = tv ? a[1 + k] : 0u;
            nib_planes(aw, ah[t][j], al[t][j]);
            da[t][j] = tv ? f16_bits_to_f32(ds & 0xffffu) : 0.0f;
            bias[t][j] = tv ? -(int)(int16_t)(ds >> 16) : 0;
        }
    }

    // code bytes of the lane's chunk: 8 bytes at a 2-byte aligned LDS offset,
    // read as 3 aligned dwords and realigned with v_alignbyte (a per-lane
    // constant shift; unaligned 8-byte DS reads measured slower); block scale
    // at the block start
    const int cw = PQ2_BYTES * (lane >> 2) + 2 + 8 * (lane & 3);
    const int sh = cw & 3;
    const int cw_al = cw - sh;
    const int dwo = PQ2_BYTES * (lane >> 2);
    // repacked layout: slot j, lane l -> chunk c of row r of the unit; code
    // unit at r*rowbytes + 2 nb + 8 ((c % 4) nb + c / 4), scale at
    // r*rowbytes + 2 (c / 4)
    int rp_code[RP ? P::S : 1], rp_dw[RP ? P::S : 1];
    if constexpr (RP) {
#pragma unroll
        for (int j = 0; j < P::S; ++j) {
            const int v = 64 * j + lane;
            const int r = (P::G == 2 && v >= P::NCH) ? 1 : 0;
            int c = v - r * P::NCH;
            c = c < P::NCH ? c : 0;                        // idle lanes of a partial slot
            rp_code[j] = r * PQ2_BYTES * NB + 2 * NB + 8 * ((c & 3) * NB + (c >> 2));
            rp_dw[j] = r * PQ2_BYTES * NB + 2 * (c >> 2);
        }
    }
    float ykeep = 0.0f;                       // lane (G i + r) NT + t keeps row r, token t of unit i

    float2 tail_e[2] = {{0.0f, 0.0f}, {0.0f, 0.0f}};
    if (T > 0) {
        // shared tail: chunk dots of this wave's tail slots (landed: every
        // unit DMA is younger); products (dw, da s) of slot r in tail_e[r]
        wait_vmcnt<D * P::NPL>();
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int r = 0; r < 2; ++r) {
            const int q = wave + WAVES * r;
            if (q < T * P::S) {
                const int j = q % P::S;
                const uint8_t * tb = &ring[D][1024 * r];
                const uint32_t * cpa = reinterpret_cast<const uint32_t *>(tb + cw_al);
                const uint32_t w0 = __builtin_amdgcn_alignbyte(cpa[1], cpa[0], sh);
                const uint32_t w1 = __builtin_amdgcn_alignbyte(cpa[2], cpa[1], sh);
                const uint32_t dwb = *reinterpret_cast<const uint16_t *>(tb + dwo);
                int s = 0;
                float daj = 0.0f;
#pragma unroll
                for (int jj = 0; jj < P::S; ++jj) {
                    if (jj == j) {
                        s = chunk_dot_nib(w0, w1, ah[0][jj], al[0][jj], bias[0][jj]);
                        daj = da[0][jj];
                    }
                }
                float dw = f16_bits_to_f32(dwb);
                if (P::PARTIAL && j == P::S - 1) dw = lane < 32 ? dw : 0.0f;
                tail_e[r].x = dw;
                tail_e[r].y = daj * (float)s;
            }
        }
        // ring slot D is read out before step 0 DMAs unit D into it
        __builtin_amdgcn_s_waitcnt(0xC07F);
        __builtin_amdgcn_wave_barrier();
    }

    int i = 0;
    if (nu > 0) do {
        const int slot = i % SL;
        const int newer = min(D - 1, nu - 1 - i);
        if (newer >= 2) wait_vmcnt<2 * P::NPL>();
        else if (newer == 1) wait_vmcnt<P::NPL>();
        else wait_vmcnt<0>();
        __builtin_amdgcn_wave_barrier();
        // unit i + D goes into the slot unit i - 1 used (its reads completed:
        // lgkmcnt(0) at the end of the previous step)
        if (i + D < nu) issue(gw + (i + D) * NW, (i + D) % SL);
        const uint8_t * ub = ring[slot];
        const int u = gw + i * NW;

        float acc0[NT], acc1[NT];
#pragma unroll
        for (int t = 0; t < NT; ++t) acc0[t] = acc1[t] = 0.0f;
        // the unit's LDS words.  Up to 5 slots (rows of up to 6144 columns)
        // every read is issued before any arithmetic, so the unit pays one
        // LDS round trip: left to itself the compiler waited three times per
        // unit (measured on MI355X, bit-identical, µs: 17408x5120 6.52-6.61
        // -> 6.45-6.51, gate+up grouped 11.45-11.79 -> 11.07-11.24, 2 tokens
        // 9.57-9.62 -> 9.28-9.37; 17408-column rows, 9 slots, measured no
        // better and keep the compiler's order)
        constexpr bool HOIST = !RP && P::S <= 5;
        uint32_t cwr[HOIST ? P::S : 1][3], dwr[HOIST ? P::S : 1];
        if constexpr (HOIST) {
#pragma unroll
            for (int j = 0; j < P::S; ++j) {
                const uint32_t * cpa = reinterpret_cast<const uint32_t *>(ub + cw_al + SLOT_BYTES * j);
                cwr[j][0] = cpa[0];
                cwr[j][1] = cpa[1];
                cwr[j][2] = cpa[2];
                dwr[j] = *reinterpret_cast<const uint16_t *>(ub + dwo + SLOT_BYTES * j);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int j = 0; j < P::S; ++j) {
            uint32_t w0, w1, dwb;
            if constexpr (HOIST) {
                w0 = __builtin_amdgcn_alignbyte(cwr[j][1], cwr[j][0], sh);
                w1 = __builtin_amdgcn_alignbyte(cwr[j][2], cwr[j][1], sh);
                dwb = dwr[j];
            } else if constexpr (RP) {
                const uint2 wv = *reinterpret_cast<const uint2 *>(ub + rp_code[j]);
                w0 = wv.x;
                w1 = wv.y;
                dwb = *reinterpret_cast<const uint16_t *>(ub + rp_dw[j]);
            } else {
                const uint32_t * cpa = reinterpret_cast<const uint32_t *>(ub + cw_al + SLOT_BYTES * j);
                w0 = __builtin_amdgcn_alignbyte(cpa[1], cpa[0], sh);
                w1 = __builtin_amdgcn_alignbyte(cpa[2], cpa[1], sh);
                dwb = *reinterpret_cast<const uint16_t *>(ub + dwo + SLOT_BYTES * j);
            }
            const bool second = (P::G == 2) && (j > P::SPLIT || (j == P::SPLIT && lane >= 32));
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                const int s = chunk_dot_nib(w0, w1, ah[t][j], al[t][j], bias[t][j]);
                if (DUMP) {
                    const int v = 64 * j + lane;
                    const int row = u * P::G + (second ? 1 : 0);
                    if (v < P::G * P::NCH && row < mg.n_out[0])     // single matrix
                        dump[(size_t)row * P::NCH + (second ? v - P::NCH : v)] = s;
                } else {
                    const float ts = da[t][j] * (float)s;
                    float dw = f16_bits_to_f32(dwb);
                    if (P::PARTIAL && j == P::S - 1) dw = lane < 32 ? dw : 0.0f;   // idle lanes: LDS past the unit
                    if (P::G == 1 || j < P::SPLIT) acc0[t] = fmaf(dw, ts, acc0[t]);
                    else if (j > P::SPLIT) acc1[t] = fmaf(dw, ts, acc1[t]);
                    else if (lane < 32) acc0[t] = fmaf(dw, ts, acc0[t]);
                    else acc1[t] = fmaf(dw, ts, acc1[t]);
                }
            }
        }
        if (!DUMP) {
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                if (P::G == 2) {
                    const float v = wave_sum2_to_lanes31_63(acc0[t], acc1[t]);
                    const float t0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 31));
                    const float t1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
                    ykeep = (lane == 2 * i * NT + t) ? t0 : ((lane == (2 * i + 1) * NT + t) ? t1 : ykeep);
                } else {
                    const float t0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wave_sum_to_lane63(acc0[t])), 63));
                    ykeep = (lane == i * NT + t) ? t0 : ykeep;
                }
            }
        }
        __builtin_amdgcn_s_waitcnt(0xC07F);        // lgkmcnt(0): this slot's reads are done
        __builtin_amdgcn_wave_barrier();
    } while (++i < nu);
    if (T > 0) {
        // the products of slot r to bytes 512 r + 8 lane of ring slot
        // (nu + 1) % SL (free: its last unit was nu - D or earlier)
        const int pslot = (nu + 1) % SL;
#pragma unroll
        for (int r = 0; r < 2; ++r)
            if (wave + WAVES * r < T * P::S)
                *reinterpret_cast<float2 *>(&ring[pslot][512 * r + 8 * lane]) = tail_e[r];
        __builtin_amdgcn_s_waitcnt(0xC07F);        // lgkmcnt(0): this wave's products are in LDS
        __builtin_amdgcn_s_barrier();
        if (wave < T) {
            // fold tail unit k = wave exactly as the loop folds a unit
            const int k = wave;
            float acc0 = 0.0f, acc1 = 0.0f;
#pragma unroll
            for (int j = 0; j < P::S; ++j) {
                const int q = k * P::S + j;
                const float2 e = *reinterpret_cast<const float2 *>(
                    &ring_all[q % WAVES][pslot][512 * (q / WAVES) + 8 * lane]);
                if (P::G == 1 || j < P::SPLIT) acc0 = fmaf(e.x, e.y, acc0);
                else if (j > P::SPLIT) acc1 = fmaf(e.x, e.y, acc1);
                else if (lane < 32) acc0 = fmaf(e.x, e.y, acc0);
                else acc1 = fmaf(e.x, e.y, acc1);
            }
            float t0, t1 = 0.0f;
            if (P::G == 2) {
                const float v = wave_sum2_to_lanes31_63(acc0, acc1);
                t0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 31));
                t1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
            } else {
                t0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wave_sum_to_lane63(acc0)), 63));
            }
            const uint8_t * Wm;
            float * ym;
            int n_out_m, lu;
            gs.at(gw + (units_per_wave - 1) * NW, Wm, ym, n_out_m, lu);
            const int row = lu * P::G + lane;
            if (lane < P::G && row < n_out_m) ym[row] = lane == 0 ? t0 : t1;
        }
    }
    if constexpr (EPI) {
        // every row of the wave in one store: the complement of its fp32 bits as
        // a device-coherent 32-bit atomic word (a finaliser polls for it)
        if (lane < nu * P::G) {
            const uint8_t * Wm;
            float * ym;
            int n_out_m, lu;
            gs.at(gw + (lane / P::G) * NW, Wm, ym, n_out_m, lu);
            const int row = lu * P::G + lane % P::G;
            if (row < n_out_m)
                __hip_atomic_store(reinterpret_cast<uint32_t *>(ym) + row, ~__float_as_uint(ykeep), __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
        }
        if (tail != 0) {
            if (epi_quad && wave >= WAVES / 2) {
                float * mine = reinterpret_cast<float *>(&ring[0][0]);
                ffn_finalise_quarter(mg, (int)blockIdx.x, wave - WAVES / 2, mine, [&](int q) {
                    return reinterpret_cast<const float *>(&ring_all[WAVES / 2 + q][0][0]);
                });
            }
            return;
        }
        // the last nblk waves of the numbering (those with the fewest units)
        // each finalise the blocks b = NW - 1 - gw, + NW, ...
        // this wave's own ring (its units are done) stages the block when it is
        // large enough: 8 KiB
        float * stage = nullptr;
        if constexpr (SL * P::LDSB >= 2 * HBLK * 4) stage = reinterpret_cast<float *>(&ring[0][0]);
        for (int b = NW - 1 - gw; b >= 0 && b < mg.epi.nblk; b += NW) ffn_finalise_block(mg, b, stage);
        return;
    }
    if (!DUMP && lane < nu * P::G * NT) {
        const uint8_t * Wm;
        float * ym;
        int n_out_m, lu;
        const int rt = lane / NT, t = lane - NT * rt;        // (G i + r), token
        gs.at(gw + (rt / P::G) * NW, Wm, ym, n_out_m, lu);
        const int row = lu * P::G + rt % P::G;
        if (NT == 1) {
            if (row < n_out_m) ym[row] = ykeep;
        } else if (row < n_out_m && t < n_tok) {
            ym[(size_t)row * n_tok + t] = ykeep;
        }
    }
}

// Generic path: one wave per row, lane-strided chunks, 2-byte weight loads
// (any n_in % 128 == 0, any 2-byte aligned W).
template <bool DUMP>
__global__ void __launch_bounds__(GV_THREADS)
gemv_rowwave_kernel(const uint8_t * __restrict__ W, const uint8_t * __restrict__ xq,
                    float * __restrict__ y, int32_t * __restrict__ dump, int n_out, int nb) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * GV_WAVES + (threadIdx.x >> 6);
    if (row >= n_out) return;
    const int nchunk = 4 * nb;
    const uint8_t * wr = W + (size_t)row * PQ2_BYTES * nb;
    float acc = 0.0f;
    for (int c = lane; c < nchunk; c += 64) {
        const uint8_t * blk = wr + (size_t)PQ2_BYTES * (c >> 2);
        const uint16_t * qp = reinterpret_cast<const uint16_t *>(blk + 2 + 8 * (c & 3));
        const uint32_t w0 = (uint32_t)qp[0] | ((uint32_t)qp[1] << 16);
        const uint32_t w1 = (uint32_t)qp[2] | ((uint32_t)qp[3] << 16);
        const uint32_t * ab = reinterpret_cast<const uint32_t *>(xq + (size_t)Q81_BYTES * c);
        const uint32_t ds = ab[0];
        const int a[8] = {(int)ab[1], (int)ab[2], (int)ab[3], (int)ab[4],
                          (int)ab[5], (int)ab[6], (int)ab[7], (int)ab[8]};
        const int s = chunk_dot_i32(w0, w1, a, -(int)(int16_t)(ds >> 16));
        if (DUMP) {
            dump[(size_t)row * nchunk + c] = s;
        } else {
            const float dw = f16_bits_to_f32(*reinterpret_cast<const uint16_t *>(blk));
            acc += dw * (f16_bits_to_f32(ds & 0xffffu) * (float)s);
        }
    }
    if (!DUMP) {
        acc = wave_sum_to_lane63(acc);
        if (lane == 63) y[row] = acc;
    }
}

using pq2host::knob;

int max_lds_per_block() { return pq2host::device_info().max_lds; }

template <int G, int NPL, bool DUMP>
int launch_stream_t(const uint8_t * W, const uint8_t * xq, float * y, int32_t * dump, int n_out,
                    const StreamGeom & g, hipStream_t st) {
    auto kern = gemv_stream_kernel<G, NPL, DUMP>;
    static pq2host::PerDeviceOnce attr;
    pq2host::once_per_device(attr, [&] {
        pq2host::set_max_dynamic_lds(reinterpret_cast<const void *>(kern), max_lds_per_block());
    });
    const int n_units = (n_out + G - 1) / G;
    int upw = knob(pq2host::K_GEMV_UNITS_PER_WAVE, 0);
    if (upw <= 0) {
        const int target_waves = 256 * 12;
        upw = (n_units + target_waves - 1) / target_waves;
        if (upw < 1) upw = 1;
    }
    const int waves = (n_units + upw - 1) / upw;
    const int blocks = (waves + GV_WAVES - 1) / GV_WAVES;
    hipLaunchKernelGGL(kern, dim3(blocks), dim3(GV_THREADS), g.lds_bytes, st, W, xq, y, dump,
                       n_out, g.nb, upw);
    return (int)hipGetLastError();
}

template <int G, bool DUMP>
int launch_stream_g(const uint8_t * W, const uint8_t * xq, float * y, int32_t * dump, int n_out,
                    const StreamGeom & g, hipStream_t st) {
    switch (g.npl) {
#define PQ2_NPL_CASE(N) case N: return launch_stream_t<G, N, DUMP>(W, xq, y, dump, n_out, g, st);
        PQ2_NPL_CASE(1) PQ2_NPL_CASE(2) PQ2_NPL_CASE(3) PQ2_NPL_CASE(4) PQ2_NPL_CASE(5)
        PQ2_NPL_CASE(6) PQ2_NPL_CASE(7) PQ2_NPL_CASE(8) PQ2_NPL_CASE(9) PQ2_NPL_CASE(10)
        PQ2_NPL_CASE(11) PQ2_NPL_CASE(12) PQ2_NPL_CASE(13) PQ2_NPL_CASE(14) PQ2_NPL_CASE(15)
        PQ2_NPL_CASE(16) PQ2_NPL_CASE(17)
#undef PQ2_NPL_CASE
        default: return -1;
    }
}

int cu_count() { return pq2host::device_info().cus; }

// Workgroups per CU for the decode GEMV, from sweeps on MI355X (HIP-graph
// replay, weights streamed from HBM): rows of <= 48 blocks want 3 workgroups
// per CU on the 24 MB matrices and 2 on the 7-8 MB ones; the widest rows
// (60 KB of LDS per workgroup) run best at one per CU.
int default_wg_per_cu(int nb, int64_t w_bytes) {
    if (nb >= 96) return 1;
    return w_bytes >= (16 << 20) ? 3 : 2;
}

// LDS bytes of one gemv_nb_kernel workgroup (all static allocations)
template <int NB, int D, int WAVES, int ROT, int NT = 1, bool RMS = false, bool OVL = false>
constexpr int nb_lds_bytes() {
    using P = NbSpec<NB, NT>;
    constexpr int act = (Q81_BYTES * P::NCH * NT + 1023) / 1024 * 1024;
    constexpr int ring = WAVES * (D + 1) * P::LDSB;
    constexpr int nhb = P::NCH / 32;
    constexpr int stage = OVL ? 0 : (ROT ? nhb * HBLK * 4 : 0) + (ROT == 2 ? nhb * HBLK * 4 : 0)   // ROT 3: x only
                          + (RMS ? nhb * HBLK * 4 + 8 * nhb : 0);
    return act + ring + stage;
}

constexpr int LDS_PER_CU = 160 * 1024;

// Unit starts of a group; false if the group's unit count overflows int.
template <int G>
bool group_units(MatGroup & mg, int n_mat) {
    int64_t u = 0;
    for (int m = 0; m < MAX_GROUP; ++m) {
        mg.u0[m] = (int)u;
        if (m < n_mat) u += (mg.n_out[m] + G - 1) / G;
        else { mg.W[m] = nullptr; mg.y[m] = nullptr; mg.n_out[m] = 0; }
    }
    for (int m = n_mat; m <= MAX_GROUP; ++m) mg.u0[m] = (int)u;
    return u < 0x40000000;
}

template <int NB, int D, int WAVES, bool DUMP, int ROT = 0, int NT = 1, bool RP = false, bool RMS = false,
          bool OVL = false, bool EPI = false>
int launch_nb_t(MatGroup mg, int n_mat, const void * xin, const float * signs, int32_t * dump,
                int per_cu, hipStream_t st, int n_tok = 1) {
    using P = NbSpec<NB, NT>;
    constexpr int lds = nb_lds_bytes<NB, D, WAVES, ROT, NT, RMS, OVL>();
    static_assert(lds <= LDS_PER_CU, "workgroup LDS");
    if (!group_units<P::G>(mg, n_mat)) return 1;
    const int n_units = mg.u0[MAX_GROUP];
    // a whole number of workgroups per CU (the dispatcher then places exactly
    // that many on every CU), fewer for small matrices
    if (per_cu > LDS_PER_CU / lds) per_cu = LDS_PER_CU / lds;
    int blocks = per_cu * cu_count();
    const int max_blocks = (n_units + WAVES - 1) / WAVES;
    if (blocks > max_blocks) blocks = max_blocks;
    const int NW = blocks * WAVES;
    int upw = (n_units + NW - 1) / NW;
    if (upw > 64 / (P::G * NT)) {               // one output per lane of a wave
        upw = 64 / (P::G * NT);
        blocks = (n_units + upw * WAVES - 1) / (upw * WAVES);
    }
    // groups of 2^xl consecutive units per XCD: 4 units cut HBM fetch by 3.4 % and time by
    // 3-5 % on the model's shapes against plain numbering; 8 units measured another ~1 %
    int xl = knob(pq2host::K_GEMV_XCD_LOG2M, 3);
    if (xl < 0 || xl > 3 || blocks % 8 != 0) xl = 0;
    while (xl > 0 && ((blocks / 8) * WAVES) % (1 << xl) != 0) --xl;
    // shared tail: the last round of L units must be exactly the last units of
    // waves 0..T-1 of every workgroup -- L = T * blocks, and with the XCD
    // numbering 2^xl must divide T * blocks / 8 (then unit index < L holds
    // exactly for waves < T) -- and every wave keeps D + 1 or more units
    int tail = 0;
    if constexpr (EPI) {
        // FFN epilogue: a four-wave quad per block (tail = 1) where waves
        // WAVES / 2 .. WAVES - 1 of every workgroup carry the fewest units: the
        // last round is complete, or is exactly the units of waves 0 .. T - 1,
        // T <= WAVES / 2, of every workgroup (the numbering condition above)
        const int nw = blocks * WAVES;
        const int L = n_units - (upw - 1) * nw;
        bool quad = WAVES == 8 && mg.epi.nblk <= blocks && knob(pq2host::K_FFN_QUAD, 1) != 0;
        if (quad && L != nw) {
            const int Tq = L / blocks;
            quad = L % blocks == 0 && Tq <= WAVES / 2 && (xl == 0 || (Tq * (blocks / 8)) % (1 << xl) == 0);
        }
        tail = quad ? 1 : 0;
    }
    if (nb_tail_ok<NB, NT, RP, DUMP, EPI>() && knob(pq2host::K_GEMV_TAIL, 0) != 0 && upw >= D + 1) {
        const int nw = blocks * WAVES;
        const int L = n_units - (upw - 1) * nw;
        bool small = true;
        for (int m = 0; m < n_mat; ++m) small = small && (int64_t)mg.n_out[m] * PQ2_BYTES * NB < 0x80000000ll;
        if (small && L > 0 && L < nw && L % blocks == 0) {
            const int T = L / blocks;
            if (T * P::S <= 2 * WAVES && (xl == 0 || (T * (blocks / 8)) % (1 << xl) == 0)) tail = T;
        }
    }
    if constexpr (EPI) {
        static_assert(!OVL && !RP && NT == 1 && !DUMP, "FFN epilogue: the fused gate/up group");
        if (n_mat != 2) return 1;
        hipLaunchKernelGGL((gemv_nb_kernel<NB, D, WAVES, false, ROT, true, 1, false, RMS, false, true>),
                           dim3(blocks), dim3(64 * WAVES), 0, st, mg, xin, signs, dump, upw, 1, xl, tail);
    } else if constexpr (OVL) {
        if (n_mat > 1)
            hipLaunchKernelGGL((gemv_nb_kernel<NB, D, WAVES, false, ROT, true, 1, false, false, true>), dim3(blocks),
                               dim3(64 * WAVES), 0, st, mg, xin, signs, dump, upw, 1, xl, tail);
        else
            hipLaunchKernelGGL((gemv_nb_kernel<NB, D, WAVES, false, ROT, false, 1, false, false, true>), dim3(blocks),
                               dim3(64 * WAVES), 0, st, mg, xin, signs, dump, upw, 1, xl, tail);
    } else if constexpr (RMS) {
        if (n_mat > 1)
            hipLaunchKernelGGL((gemv_nb_kernel<NB, D, WAVES, false, ROT, true, 1, false, true>), dim3(blocks),
                               dim3(64 * WAVES), 0, st, mg, xin, signs, dump, upw, 1, xl, tail);
        else
            hipLaunchKernelGGL((gemv_nb_kernel<NB, D, WAVES, false, ROT, false, 1, false, true>), dim3(blocks),
                               dim3(64 * WAVES), 0, st, mg, xin, signs, dump, upw, 1, xl, tail);
    } else if constexpr (RP)
        hipLaunchKernelGGL((gemv_nb_kernel<NB, D, WAVES, false, ROT, false, 1, true>), dim3(blocks),
                           dim3(64 * WAVES), 0, st, mg, xin, signs, dump, upw, 1, xl, tail);
    else if constexpr (NT > 1)
        hipLaunchKernelGGL((gemv_nb_kernel<NB, D, WAVES, false, 0, false, NT>), dim3(blocks), dim3(64 * WAVES),
                           0, st, mg, xin, signs, dump, upw, n_tok, xl, tail);
    else if (n_mat > 1)
        hipLaunchKernelGGL((gemv_nb_kernel<NB, D, WAVES, DUMP, ROT, true>), dim3(blocks), dim3(64 * WAVES), 0,
                           st, mg, xin, signs, dump, upw, 1, xl, tail);
    else
        hipLaunchKernelGGL((gemv_nb_kernel<NB, D, WAVES, DUMP, ROT, false>), dim3(blocks), dim3(64 * WAVES), 0,
                           st, mg, xin, signs, dump, upw, 1, xl, tail);
    return (int)hipGetLastError();
}

int64_t group_weight_bytes(const MatGroup & mg, int n_mat, int nb) {
    int64_t b = 0;
    for (int m = 0; m < n_mat; ++m) b += (int64_t)mg.n_out[m] * PQ2_BYTES * nb;
    return b;
}

template <int NB, bool DUMP>
int launch_nb(const MatGroup & mg, int n_mat, const uint8_t * xq, int32_t * dump, hipStream_t st) {
    // 4-wave workgroups with two unit buffers per wave measured best at every
    // model width (deeper rings queue more bytes ahead of the activation)
    int per_cu = knob(pq2host::K_GEMV_WG_PER_CU, 0);
    if (per_cu <= 0) {
        per_cu = default_wg_per_cu(NB, group_weight_bytes(mg, n_mat, NB));
        // a matrix below 16 MB whose units fill one 4-wave workgroup per CU
        // evenly, with at most 3 units per wave, runs best that way (6144x5120:
        // 3 units per wave, 4.41 -> 4.21 us, against 1.5 with two workgroups per
        // CU; at 4 units per wave (q/k/v grouped: 4.80 -> 5.11 us) and 5
        // (5120x6144) two workgroups per CU stay faster)
        int64_t units = 0;
        for (int m = 0; m < n_mat; ++m) units += (mg.n_out[m] + NbSpec<NB, 1>::G - 1) / NbSpec<NB, 1>::G;
        const int64_t waves1 = 4 * (int64_t)cu_count();
        if (per_cu == 2 && units % waves1 == 0 && units / waves1 <= 3) per_cu = 1;
        // rows of 5120 and 6144 columns (2-row units): other workgroup shapes
        // measured faster on MI355X (same process, alternating shapes, us):
        //   one 8-wave workgroup per CU: 17408x5120 6.95 -> 6.31, gate+up
        //     grouped 11.08 -> 9.95, 5120x6144 4.11 -> 4.00;
        //   one 6-wave workgroup per CU: q/k/v grouped (4096 units) 4.78 -> 4.62;
        //   ring depth 1, three per CU: 1024x5120 (512 units) 2.91 -> 2.79;
        //   6144x5120 (3 units per wave of one 4-wave workgroup per CU) and
        //   the 17408-wide rows keep the shape above.
        if constexpr (!DUMP && (NB == 40 || NB == 48)) {
            if (NB == 48 || group_weight_bytes(mg, n_mat, NB) >= (16 << 20))
                return launch_nb_t<NB, 2, 8, false>(mg, n_mat, xq, nullptr, dump, 1, st);
            if (NB == 40 && units <= waves1)
                return launch_nb_t<NB, 1, 4, false>(mg, n_mat, xq, nullptr, dump, 3, st);
            if (NB == 40 && units > 3 * waves1)
                return launch_nb_t<NB, 2, 6, false>(mg, n_mat, xq, nullptr, dump, 1, st);
        }
    }
    return launch_nb_t<NB, 2, 4, DUMP>(mg, n_mat, xq, nullptr, dump, per_cu, st);
}

// ---------------------------------------------------------------------------
// Small batch, 4..8 tokens: v_mfma_i32_4x4x4i8 on the streaming scheme.
// The instruction computes 16 independent 4x4 blocks; block b of lane group
// 4b..4b+3 takes A row i from lane 4b+i and B column j from lane 4b+j (4
// int8 along K in one dword each) and returns D(row i, column j) in register
// i of lane 4b+j.  Here a unit is 4 consecutive weight rows, a slot 16 chunks
// of it: block b = chunk 16s+b, its 4 rows = the unit's rows, its 4 columns =
// 4 tokens.  Eight instructions (K = 4 each) cover a chunk: instruction q
// takes the code bytes (w_{q/4} >> 2(q%4)) & 0x03030303 -- exactly the
// positions of permuted activation word q -- and the accumulator starts at
// -s, so D is the integer chunk dot sum (code-1) q with no idle columns.  The
// 16 chunk partial sums of a (row, token) meet at the end of the unit (row
// rotations, then permlane swaps).  The chunk-major X of all tokens sits in
// LDS; units stream through a 2-slot LDS ring by DMA.  NTG groups of 4
// tokens share the code words; the dispatcher uses one group (3..4 tokens):
// two groups measured no faster than the 16x16 MFMA kernel.
template <int NB>
struct Mfma4Spec {
    static constexpr int NCH = 4 * NB;
    static constexpr int NS = NCH / 16;                  // slots per unit
    static constexpr int RB = PQ2_BYTES * NB;            // bytes per row
    static constexpr int UB = 4 * RB;                    // bytes per unit
    static constexpr int NPIECE = UB / 16;
    static constexpr int NPL = (NPIECE + 63) / 64;
    static constexpr int LDSB = (UB + 16 > 1024 * NPL) ? UB + 16 : 1024 * NPL;
    static_assert(NCH % 16 == 0 && UB % 16 == 0 && RB % 4 == 0, "unit shape");
};

template <int NB, int NTG, int WAVES>
constexpr int mfma4_lds_bytes() {
    using P = Mfma4Spec<NB>;
    return (Q81_BYTES * P::NCH * 4 * NTG + 1023) / 1024 * 1024 + WAVES * 2 * P::LDSB;
}

constexpr int DPP_ROW_ROR4 = 0x124, DPP_ROW_ROR8 = 0x128;

template <int NB, int NTG, int WAVES>
__global__ void __launch_bounds__(64 * WAVES)
gemv_mfma4_kernel(const uint8_t * __restrict__ W, const uint8_t * __restrict__ X, float * __restrict__ Y,
                  int n_out, int n_tok, int units_per_wave) {
    using P = Mfma4Spec<NB>;
    typedef int v4i_t __attribute__((ext_vector_type(4)));
    constexpr int ACT_MAX = Q81_BYTES * P::NCH * 4 * NTG;
    __shared__ __attribute__((aligned(16))) uint8_t act_lds[(ACT_MAX + 1023) / 1024 * 1024];
    __shared__ __attribute__((aligned(16))) uint8_t ring_all[WAVES][2][P::LDSB];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    __builtin_assume(lane >= 0 && lane < 64);
    uint8_t (*ring)[P::LDSB] = ring_all[wave];
    const int n_units = (n_out + 3) / 4;
    const int n_full = n_out / 4;
    const int gw = wave * gridDim.x + blockIdx.x;
    const int NW = gridDim.x * WAVES;
    const int nu = gw < n_units ? min(units_per_wave, (n_units - 1 - gw) / NW + 1) : 0;

    // 1. this wave's share of the activation DMA
    const int act_bytes = Q81_BYTES * P::NCH * n_tok;
    const int na = (act_bytes + 1023) / 1024;
    for (int k = wave; k < na; k += WAVES) {
        const int off = min(16 * (64 * k + lane), act_bytes - 16);
        __builtin_amdgcn_global_load_lds(X + off, (lds_void *)(&act_lds[1024 * k]), 16, 0, 0);
    }
    __builtin_amdgcn_sched_barrier(0);

    // 2. unit DMA (a trailing unit with fewer than 4 rows clamps to the end of W)
    uint32_t poff[P::NPL];
#pragma unroll
    for (int k = 0; k < P::NPL; ++k) poff[k] = 16u * (uint32_t)min(lane + 64 * k, P::NPIECE - 1);
    const size_t last_piece = (size_t)n_out * P::RB / 16 - 1;
    auto issue = [&](int uu, int slot) {
        const uint8_t * base = W + (size_t)uu * P::UB;
        const bool full = uu < n_full;
#pragma unroll
        for (int k = 0; k < P::NPL; ++k) {
            const uint8_t * src = base + poff[k];
            if (!full) {
                size_t pc = (size_t)uu * (P::UB / 16) + poff[k] / 16;
                src = W + 16 * (pc < last_piece ? pc : last_piece);
            }
            __builtin_amdgcn_global_load_lds(src, (lds_void *)(&ring[slot][1024 * k]), 16, 0, CPOL_NT);
        }
    };
    __builtin_amdgcn_s_barrier();
    if (nu > 0) issue(gw, 0);
    __builtin_amdgcn_sched_barrier(0);
    if (nu > 0) wait_vmcnt<P::NPL>();
    else wait_vmcnt<0>();
    __builtin_amdgcn_s_barrier();
    if (nu <= 0) return;

    // per-lane roles: row i of the unit, chunk offset b in the slot, token j of a group
    const int i4 = lane & 3, b16 = lane >> 2;
    const int cbase = i4 * P::RB + PQ2_BYTES * (b16 >> 2) + 2 + 8 * (b16 & 3);   // code bytes, slot 0
    const int csh = cbase & 3;
    const int c_al = cbase - csh;
    const int dbase = i4 * P::RB + PQ2_BYTES * (b16 >> 2);                      // block scale, slot 0

    // outputs stay in lanes until the end (a global store inside the unit
    // loop makes the compiler wait for the next unit's DMA before the ring
    // reads): lane 16 it + 4 r + j keeps (row r, token j) of unit it
    float ykeep[NTG];
#pragma unroll
    for (int g = 0; g < NTG; ++g) ykeep[g] = 0.0f;
    // the lane's activation words (chunk 16 sl + b16 of its token) are the
    // same in every unit: up to 10 slots they are read once and kept in
    // registers (measured on MI355X, bit-identical, µs: 17408x5120 4 tokens
    // 10.79-10.95 -> 10.24-10.35, 6144x5120 4 tokens 6.20-6.26 ->
    // 6.14-6.19); the 12 slots of 6144-column rows measured slower so
    // (5120x6144 6.54-6.59 -> 6.70-6.76) and read them per unit
    constexpr bool KEEP = P::NS * NTG <= 10;
    uint32_t awk[KEEP ? P::NS : 1][NTG][9];
    if constexpr (KEEP) {
#pragma unroll
        for (int sl = 0; sl < P::NS; ++sl)
#pragma unroll
            for (int g = 0; g < NTG; ++g) {
                const int t = 4 * g + i4;
                const bool tv = t < n_tok;
                const uint32_t * ab =
                    reinterpret_cast<const uint32_t *>(&act_lds[Q81_BYTES * (tv ? (16 * sl + b16) * n_tok + t : 0)]);
#pragma unroll
                for (int k = 0; k < 9; ++k) awk[sl][g][k] = ab[k];
            }
    }
    for (int it = 0; it < nu; ++it) {
        const int slot = it & 1;
        wait_vmcnt<0>();
        __builtin_amdgcn_wave_barrier();
        if (it + 1 < nu) issue(gw + (it + 1) * NW, slot ^ 1);   // the other slot's reads are done
        const uint8_t * ub = ring[slot];
        float acc[NTG][4];
#pragma unroll
        for (int g = 0; g < NTG; ++g)
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[g][r] = 0.0f;
#pragma unroll
        for (int sl = 0; sl < P::NS; ++sl) {
            const uint32_t * cpa = reinterpret_cast<const uint32_t *>(ub + c_al + 136 * sl);
            const uint32_t w0 = __builtin_amdgcn_alignbyte(cpa[1], cpa[0], csh);
            const uint32_t w1 = __builtin_amdgcn_alignbyte(cpa[2], cpa[1], csh);
            // block scales of the 4 rows: each lane reads its own row's, the quad shares them
            const float dwi = f16_bits_to_f32(*reinterpret_cast<const uint16_t *>(ub + dbase + 136 * sl));
            float dwr[4];
            dwr[0] = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(dwi), 0x00, 0xf, 0xf, true));
            dwr[1] = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(dwi), 0x55, 0xf, 0xf, true));
            dwr[2] = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(dwi), 0xAA, 0xf, 0xf, true));
            dwr[3] = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(dwi), 0xFF, 0xf, 0xf, true));
            const int c = 16 * sl + b16;
#pragma unroll
            for (int g = 0; g < NTG; ++g) {
                const int t = 4 * g + i4;                      // this lane's token (column)
                const bool tv = t < n_tok;
                // unconditional reads (a missing token reads block 0 and is zeroed)
                uint32_t awl[9];
                const uint32_t * aw = awl;
                if constexpr (KEEP) {
                    aw = awk[sl][g];
                } else {
                    const uint32_t * ab = reinterpret_cast<const uint32_t *>(&act_lds[Q81_BYTES * (tv ? c * n_tok + t : 0)]);
#pragma unroll
                    for (int k = 0; k < 9; ++k) awl[k] = ab[k];
                }
                const uint32_t ds = tv ? aw[0] : 0u;
                const int ns = -(int)(int16_t)(ds >> 16);
                v4i_t d = {ns, ns, ns, ns};
#pragma unroll
                for (int q = 0; q < 8; ++q) {
                    const uint32_t wq = q < 4 ? w0 : w1;
                    const int a = (int)((wq >> (2 * (q & 3))) & 0x03030303u);
                    const int bq = tv ? (int)aw[1 + q] : 0;
                    d = __builtin_amdgcn_mfma_i32_4x4x4i8(a, bq, d, 0, 0, 0);
                }
                const float da = f16_bits_to_f32(ds & 0xffffu);
#pragma unroll
                for (int r = 0; r < 4; ++r) acc[g][r] = fmaf(dwr[r] * da, (float)d[r], acc[g][r]);
            }
        }
        // sum the 16 chunk blocks of every (row, token): within a 16-lane row
        // by rotations of 4 and 8 (they keep lane % 4, the token), then across
        // the four rows by permlane16 and permlane32 swaps
#pragma unroll
        for (int g = 0; g < NTG; ++g) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                float v = acc[g][r];
                v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), DPP_ROW_ROR8, 0xf, 0xf, true));
                v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), DPP_ROW_ROR4, 0xf, 0xf, true));
                const auto s16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
                v = __uint_as_float(s16[0]) + __uint_as_float(s16[1]);
                const auto s32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
                v = __uint_as_float(s32[0]) + __uint_as_float(s32[1]);
                ykeep[g] = (b16 == 4 * it + r) ? v : ykeep[g];  // every lane holds its token j's total
            }
        }
        __builtin_amdgcn_s_waitcnt(0xC07F);        // lgkmcnt(0): this slot's reads are done
        __builtin_amdgcn_wave_barrier();
    }
    if (lane < 16 * nu) {
        const int row = 4 * (gw + (lane >> 4) * NW) + ((lane >> 2) & 3);
#pragma unroll
        for (int g = 0; g < NTG; ++g) {
            const int t = 4 * g + i4;
            if (row < n_out && t < n_tok) Y[(size_t)row * n_tok + t] = ykeep[g];
        }
    }
}

template <int NB, int NTG, int WAVES>
int launch_mfma4(const uint8_t * W, const uint8_t * X, float * Y, int n_out, int n_tok, hipStream_t st) {
    constexpr int lds = mfma4_lds_bytes<NB, NTG, WAVES>();
    static_assert(lds <= LDS_PER_CU, "workgroup LDS");
    const int n_units = (n_out + 3) / 4;
    int per_cu = knob(pq2host::K_MFMA4_WG_PER_CU, LDS_PER_CU / lds);
    if (per_cu > LDS_PER_CU / lds) per_cu = LDS_PER_CU / lds;
    if (per_cu < 1) per_cu = 1;
    int blocks = per_cu * cu_count();
    const int max_blocks = (n_units + WAVES - 1) / WAVES;
    if (blocks > max_blocks) blocks = max_blocks;
    int upw = (n_units + blocks * WAVES - 1) / (blocks * WAVES);
    if (upw > 4) {                                  // 16 outputs per unit in the lanes of a wave
        upw = 4;
        blocks = (n_units + 4 * WAVES - 1) / (4 * WAVES);
    }
    hipLaunchKernelGGL((gemv_mfma4_kernel<NB, NTG, WAVES>), dim3(blocks), dim3(64 * WAVES), 0, st, W, X, Y,
                       n_out, n_tok, upw);
    return (int)hipGetLastError();
}

// 3..4 tokens: 8-wave workgroups for the large matrices, 4-wave ones (more
// workgroups) below 4096 rows -- measured on MI355X.
template <int NB>
int launch_mfma4_nt(const uint8_t * W, const uint8_t * X, float * Y, int n_out, int n_tok, hipStream_t st) {
    const int waves = knob(pq2host::K_MFMA4_WAVES, n_out >= 4096 ? 8 : 4);
    if (waves == 4) return launch_mfma4<NB, 1, 4>(W, X, Y, n_out, n_tok, st);
    return launch_mfma4<NB, 1, 8>(W, X, Y, n_out, n_tok, st);
}

// Small batch on the streaming kernel: n_tok <= NT tokens (2 or 3), chunk-major Xq.
// Instantiated where the per-token planes fit in registers: NT * S * 10
// registers of activation per lane, at most 120 where three waves share a
// SIMD, at most 400 for the widest rows (one workgroup, one wave per SIMD).
template <int NB, int NT>
constexpr bool nt_fits() { return NT * NbSpec<NB, NT>::S * 10 <= (NB >= 96 ? 400 : 120); }

template <int NB, int NT>
int launch_nb_small(const uint8_t * W, const uint8_t * X, float * Y, int n_out, int n_tok, hipStream_t st) {
    if constexpr (!nt_fits<NB, NT>()) {
        return -1;
    } else {
        MatGroup mg = single_group(W, Y, n_out);
        int per_cu = knob(pq2host::K_GEMV_WG_PER_CU, 0);
        // 2 tokens on 5120- and 6144-column rows: one 8-wave workgroup per CU
        // once the units fill its waves, ring depth 1 up to 2 units per wave
        // and 2 beyond (MI355X, us, three or two 4-wave workgroups per CU ->
        // this shape): 17408x5120 9.23 -> 9.02, 34816x5120 13.06 -> 12.89,
        // 6144x5120 6.32 -> 5.63, 4096x5120 5.41 -> 5.00, 5120x6144 5.40 ->
        // 4.73, 6144x6144 5.47 -> 5.14, 2048x6144 4.27 -> 3.73; 2048x5120 (fewer
        // units than waves) keeps the 4-wave shape (4.29 against 4.97)
        if constexpr (NT == 2 && (NB == 40 || NB == 48)) {
            const int64_t units = ((int64_t)n_out + NbSpec<NB, NT>::G - 1) / NbSpec<NB, NT>::G;
            const int64_t waves8 = 8 * (int64_t)cu_count();
            if (per_cu <= 0 && units > 2 * waves8)
                return launch_nb_t<NB, 2, 8, false, 0, NT>(mg, 1, X, nullptr, nullptr, 1, st, n_tok);
            if (per_cu <= 0 && units >= waves8)
                return launch_nb_t<NB, 1, 8, false, 0, NT>(mg, 1, X, nullptr, nullptr, 1, st, n_tok);
        }
        if (per_cu <= 0) per_cu = default_wg_per_cu(NB, (int64_t)n_out * PQ2_BYTES * NB);
        return launch_nb_t<NB, 2, 4, false, 0, NT>(mg, 1, X, nullptr, nullptr, per_cu, st, n_tok);
    }
}

template <int NB>
int launch_nb_small_nt(const uint8_t * W, const uint8_t * X, float * Y, int n_out, int n_tok, hipStream_t st) {
    switch (n_tok) {
        case 2: return launch_nb_small<NB, 2>(W, X, Y, n_out, n_tok, st);
        case 3: return launch_nb_small<NB, 3>(W, X, Y, n_out, n_tok, st);
        default: return -1;
    }
}

// Fused rotation: every workgroup rotates the whole activation, so the
// fused kernel wants few, wide workgroups: 8 waves and one workgroup per CU
// where the LDS allows (measured on MI355X: 7.7 us at 17408x5120, 5.5-5.6 us
// at 6144x5120 and 5120x6144, against 9.9 / 7.0 / 6.8 us for the pre-pass
// plus the GEMV; two workgroups per CU: 6.9 us at 5120x6144), else 4 waves
// with D = 2 or D = 1.  Returns -1 when no shape fits the LDS of a workgroup.
template <int NB, int ROT, bool RP = false, bool RMS = false, bool EPI = false>
int launch_nb_rot(const MatGroup & mg, int n_mat, const float * x, const float * signs, hipStream_t st) {
    const int waves = knob(pq2host::K_FGEMV_WAVES, 8);
    int per_cu = knob(pq2host::K_GEMV_WG_PER_CU, 0);
    if (per_cu <= 0) per_cu = 1;
    if constexpr (nb_lds_bytes<NB, 2, 8, ROT, 1, RMS>() <= LDS_PER_CU) {
        if (waves == 8)
            return launch_nb_t<NB, 2, 8, false, ROT, 1, RP, RMS, false, EPI>(mg, n_mat, x, signs, nullptr, per_cu, st);
    } else if constexpr (ROT == 1 && !RP && !RMS && !EPI && nb_lds_bytes<NB, 2, 8, 1, 1, false, true>() <= LDS_PER_CU) {
        // the separate stage does not fit beside an 8-wave ring: stage in the ring
        if (waves == 8 && knob(pq2host::K_FGEMV_OVL, 1) == 1)
            return launch_nb_t<NB, 2, 8, false, 1, 1, false, false, true>(mg, n_mat, x, signs, nullptr, per_cu, st);
    }
    if constexpr (nb_lds_bytes<NB, 2, 4, ROT, 1, RMS>() <= LDS_PER_CU)
        return launch_nb_t<NB, 2, 4, false, ROT, 1, RP, RMS, false, EPI>(mg, n_mat, x, signs, nullptr, per_cu, st);
    else if constexpr (nb_lds_bytes<NB, 1, 4, ROT, 1, RMS>() <= LDS_PER_CU)
        return launch_nb_t<NB, 1, 4, false, ROT, 1, RP, RMS, false, EPI>(mg, n_mat, x, signs, nullptr, per_cu, st);
    else
        return -1;
}

// Generic fused path (any n_in % 1024 == 0 whose Q8_1 activation fits in
// LDS): every workgroup rotates (unless rotate is false) and quantises the
// whole activation into LDS (one Hadamard block per wave at a time), then each
// wave computes one row
// with the lane-strided chunk walk of gemv_rowwave_kernel.  With norm_w, x is
// first RMS-normalised: the workgroup sums the squares of all of x in fp64 in
// the order of rms_sumsq (the same in every workgroup and every other
// normalising kernel).
__global__ void __launch_bounds__(GV_THREADS)
gemv_rot_generic_kernel(const uint8_t * __restrict__ W, const float * __restrict__ x,
                        const float * __restrict__ signs, float * __restrict__ y, int n_out, int nb,
                        bool vec, const float * __restrict__ norm_w, float eps, bool rotate) {
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    __shared__ double red[RMS_GROUP];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int nchunk = 4 * nb;
    uint8_t * act = smem;
    const int xrow = fwht_row(lane);
    float rs = 1.0f;
    if (norm_w != nullptr) {
        const double tot = rms_sumsq(
            nchunk / 32, red, GV_WAVES, wave, lane,
            [&](int b, float (&v)[16]) { load16(x + (size_t)HBLK * b + 16 * xrow, v, vec); },
            [] { __syncthreads(); });
        rs = 1.0f / sqrtf((float)(tot / (double)(32 * nchunk)) + eps);
    }
    for (int b = wave; b < nchunk / 32; b += GV_WAVES) {
        float v[16];
        load16(x + (size_t)HBLK * b + 16 * xrow, v, vec);
        if (norm_w != nullptr) {
#pragma clang fp contract(off)
            float wv[16];
            load16(norm_w + (size_t)HBLK * b + 16 * xrow, wv, vec);
#pragma unroll
            for (int r = 0; r < 16; ++r) v[r] = v[r] * rs * wv[r];
        }
        if (signs != nullptr) {
#pragma clang fp contract(off)
            float sg[16];
            load16(signs + (size_t)HBLK * b + 16 * xrow, sg, vec);
#pragma unroll
            for (int r = 0; r < 16; ++r) v[r] *= sg[r];
        }
        if (rotate) fwht1024_regs(v, lane);
        quant_pair_store(v, act + (size_t)Q81_BYTES * (32 * b + (xrow >> 1)), xrow & 1);
    }
    __syncthreads();
    const int row = blockIdx.x * GV_WAVES + wave;
    if (row >= n_out) return;
    const uint8_t * wr = W + (size_t)row * PQ2_BYTES * nb;
    float acc = 0.0f;
    for (int c = lane; c < nchunk; c += 64) {
        const uint8_t * blk = wr + (size_t)PQ2_BYTES * (c >> 2);
        const uint16_t * qp = reinterpret_cast<const uint16_t *>(blk + 2 + 8 * (c & 3));
        const uint32_t w0 = (uint32_t)qp[0] | ((uint32_t)qp[1] << 16);
        const uint32_t w1 = (uint32_t)qp[2] | ((uint32_t)qp[3] << 16);
        const uint32_t * ab = reinterpret_cast<const uint32_t *>(act + (size_t)Q81_BYTES * c);
        const uint32_t ds = ab[0];
        const int a[8] = {(int)ab[1], (int)ab[2], (int)ab[3], (int)ab[4],
                          (int)ab[5], (int)ab[6], (int)ab[7], (int)ab[8]};
        const int s = chunk_dot_i32(w0, w1, a, -(int)(int16_t)(ds >> 16));
        const float dw = f16_bits_to_f32(*reinterpret_cast<const uint16_t *>(blk));
        acc += dw * (f16_bits_to_f32(ds & 0xffffu) * (float)s);
    }
    acc = wave_sum_to_lane63(acc);
    if (lane == 63) y[row] = acc;
}

size_t rot_generic_lds(int64_t n_in) { return (size_t)(n_in / QK8) * Q81_BYTES; }

bool group_w_aligned(const MatGroup & mg, int n_mat) {
    for (int m = 0; m < n_mat; ++m)
        if (((uintptr_t)mg.W[m] & 15u) != 0) return false;
    return true;
}

// One generic fused launch per matrix of a group (rotate = false: Q8_1 of x
// itself); 1 when the activation does not fit in a workgroup's LDS.
int rot_generic_launch(const MatGroup & mg, int n_mat, const float * x, const float * signs, int64_t n_in,
                       bool rotate, hipStream_t st) {
    const size_t lds = rot_generic_lds(n_in);
    if (lds > (size_t)max_lds_per_block()) return 1;
    // the kernel's static LDS (its fp64 partial sums) comes off the maximum
    static pq2host::PerDeviceOnce attr;
    pq2host::once_per_device(attr, [] {
        pq2host::set_max_dynamic_lds(reinterpret_cast<const void *>(gemv_rot_generic_kernel),
                                     max_lds_per_block() - 1024);
    });
    if (lds > (size_t)max_lds_per_block() - 1024) return 1;
    const bool vec = ((uintptr_t)x & 15u) == 0 && ((uintptr_t)signs & 15u) == 0 &&
                     ((uintptr_t)mg.norm_w & 15u) == 0;
    for (int m = 0; m < n_mat; ++m) {
        if (mg.n_out[m] <= 0) continue;
        const unsigned blocks = (unsigned)((mg.n_out[m] + GV_WAVES - 1) / GV_WAVES);
        hipLaunchKernelGGL(gemv_rot_generic_kernel, dim3(blocks), dim3(GV_THREADS), lds, st, mg.W[m], x,
                           signs, mg.y[m], mg.n_out[m], (int)(n_in / QK_PQ2), vec, mg.norm_w, mg.eps, rotate);
        const int rc = (int)hipGetLastError();
        if (rc != 0) return rc;
    }
    return 0;
}

// Q8_1 (no rotation) + GEMV of one matrix in one launch: the streaming
// kernel on the model widths (the activation quantised into every
// workgroup's LDS, as the fused FWHT path without its butterflies), else the
// generic fused kernel.
int quant_gemv_dispatch(const MatGroup & mg, const float * x, int64_t n_in, hipStream_t st) {
    if (group_w_aligned(mg, 1) && ((uintptr_t)x & 15u) == 0 && knob(pq2host::K_GEMV_KERNEL, 0) == 0) {
        int rc = -1;
        switch (n_in / QK_PQ2) {
            case 8: rc = launch_nb_rot<8, 3>(mg, 1, x, nullptr, st); break;
            case 40: rc = launch_nb_rot<40, 3>(mg, 1, x, nullptr, st); break;
            case 48: rc = launch_nb_rot<48, 3>(mg, 1, x, nullptr, st); break;
            case 80: rc = launch_nb_rot<80, 3>(mg, 1, x, nullptr, st); break;
            case 96: rc = launch_nb_rot<96, 3>(mg, 1, x, nullptr, st); break;
            case 136: rc = launch_nb_rot<136, 3>(mg, 1, x, nullptr, st); break;
            default: break;
        }
        if (rc >= 0) return rc;
    }
    return rot_generic_launch(mg, 1, x, nullptr, n_in, false, st);
}

// Fused FWHT + Q8_1 + GEMV of a group: one streaming launch on the model
// widths, else one generic fused launch per matrix.
int fwht_gemv_group_dispatch(const MatGroup & mg, int n_mat, const float * x, const float * signs,
                             int64_t n_in, hipStream_t st) {
    const bool al = group_w_aligned(mg, n_mat) && ((uintptr_t)x & 15u) == 0 && ((uintptr_t)signs & 15u) == 0 &&
                    ((uintptr_t)mg.norm_w & 15u) == 0;
    if (al && knob(pq2host::K_GEMV_KERNEL, 0) == 0) {
        int rc = -1;
        if (mg.norm_w != nullptr) {
            // RMSNorm on the widths a layer input has (the model's 5120 and 6144,
            // and 1024); other widths take the generic kernel below
#define PQ2_RMS_CASE(N)                                                                         \
    case N: rc = signs ? launch_nb_rot<N, 2, false, true>(mg, n_mat, x, signs, st)              \
                       : launch_nb_rot<N, 1, false, true>(mg, n_mat, x, signs, st); break;
            switch (n_in / QK_PQ2) {
                PQ2_RMS_CASE(8) PQ2_RMS_CASE(40) PQ2_RMS_CASE(48)
                default: break;
            }
#undef PQ2_RMS_CASE
        } else {
#define PQ2_ROT_CASE(N)                                                                         \
    case N: rc = signs ? launch_nb_rot<N, 2>(mg, n_mat, x, signs, st)                           \
                       : launch_nb_rot<N, 1>(mg, n_mat, x, signs, st); break;
            switch (n_in / QK_PQ2) {
                PQ2_ROT_CASE(8) PQ2_ROT_CASE(40) PQ2_ROT_CASE(48) PQ2_ROT_CASE(80) PQ2_ROT_CASE(96)
                PQ2_ROT_CASE(136)
                default: break;
            }
#undef PQ2_ROT_CASE
        }
        if (rc >= 0) return rc;
    }
    return rot_generic_launch(mg, n_mat, x, signs, n_in, true, st);
}

// One matrix on the widths without a specialised kernel: the runtime-shaped
// streaming kernel, or the generic wave-per-row kernel.
template <bool DUMP>
int gemv_other(const uint8_t * w, const uint8_t * x, float * y, int32_t * dump, int n_out, int64_t n_in,
               int kernel_sel, hipStream_t st) {
    const StreamGeom g = stream_geom(n_in);
    const bool fast = (n_in % HBLK == 0) && (((uintptr_t)w & 15u) == 0) && g.npl <= MAX_NPL &&
                      g.lds_bytes <= (size_t)max_lds_per_block() &&
                      kernel_sel != 2;
    if (fast) {
        const int rc = (g.G == 1) ? launch_stream_g<1, DUMP>(w, x, y, dump, n_out, g, st)
                                  : launch_stream_g<2, DUMP>(w, x, y, dump, n_out, g, st);
        if (rc >= 0) return rc;
    }
    const unsigned blocks = (unsigned)((n_out + GV_WAVES - 1) / GV_WAVES);
    hipLaunchKernelGGL(gemv_rowwave_kernel<DUMP>, dim3(blocks), dim3(GV_THREADS), 0, st, w, x, y,
                       dump, n_out, g.nb);
    return (int)hipGetLastError();
}

template <bool DUMP>
int gemv_group_dispatch(const MatGroup & mg, int n_mat, const void * xq, int32_t * dump, int64_t n_in,
                        hipStream_t st) {
    const uint8_t * x = static_cast<const uint8_t *>(xq);
    const int kernel_sel = knob(pq2host::K_GEMV_KERNEL, 0);   // 0 auto, 1 stream, 2 generic
    if (group_w_aligned(mg, n_mat) && ((uintptr_t)x & 15u) == 0 && kernel_sel == 0) {
        switch (n_in / QK_PQ2) {
            case 8: return launch_nb<8, DUMP>(mg, n_mat, x, dump, st);
            case 40: return launch_nb<40, DUMP>(mg, n_mat, x, dump, st);
            case 48: return launch_nb<48, DUMP>(mg, n_mat, x, dump, st);
            case 80: return launch_nb<80, DUMP>(mg, n_mat, x, dump, st);
            case 96: return launch_nb<96, DUMP>(mg, n_mat, x, dump, st);
            case 136: return launch_nb<136, DUMP>(mg, n_mat, x, dump, st);
            default: break;
        }
    }
    for (int m = 0; m < n_mat; ++m) {
        if (mg.n_out[m] <= 0) continue;
        const int rc = gemv_other<DUMP>(mg.W[m], x, mg.y[m], dump, mg.n_out[m], n_in, kernel_sel, st);
        if (rc != 0) return rc;
    }
    return 0;
}

// Host arrays of a group -> MatGroup.  Returns 1 on bad arguments, 0 with
// *n_rows = 0 for an empty group, else 0.
int make_group(MatGroup & mg, const void * const * W, float * const * y, const int64_t * n_out, int n_mat,
               int64_t * n_rows) {
    *n_rows = 0;
    if (n_mat < 1 || n_mat > MAX_GROUP || W == nullptr || y == nullptr || n_out == nullptr) return 1;
    for (int m = 0; m < MAX_GROUP; ++m) {
        const int64_t r = m < n_mat ? n_out[m] : 0;
        if (r > 0x3fffffff) return 1;
        mg.W[m] = m < n_mat ? static_cast<const uint8_t *>(W[m]) : nullptr;
        mg.y[m] = m < n_mat ? y[m] : nullptr;
        mg.n_out[m] = r > 0 ? (int)r : 0;
        if (r > 0 && pq2host::any_null(mg.W[m], mg.y[m])) return 1;
        *n_rows += mg.n_out[m];
    }
    return 0;
}

}  // namespace

namespace pq2 {

// Small batch (2..4 tokens) on the streaming kernels, for the GEMM's
// dispatcher; -1 when the shape or alignment has neither (the caller then
// uses the MFMA small-batch kernel).  Measured on MI355X (us; per-token
// planes / 4x4x4 MFMA / the MFMA small-batch kernel of gemm.hip):
//   17408x5120  B=2 10.3 / 10.6 / 12.8   B=3 12.2 / 10.6 / 13.1   B=4 -- / 10.4 / 13.3
//   6144x5120   B=2  6.6 /  6.1 /  7.2   B=3  6.7 /  6.2 /  7.4   B=4 -- /  6.2 /  7.5
//   5120x6144   B=2  5.7 /  6.4 /  8.1   B=3  6.8 /  6.6 /  8.3   B=4 -- /  6.5 /  8.4
//   5120x17408  B=2 10.9 /  -- / 16.3   B=3 16.1 /  -- / 16.9
// so 2 tokens take the planes kernel, 3..4 the 4x4x4 kernel on its widths
// (8, 40, 48 blocks per row), 3 tokens the planes kernel elsewhere.
// BONSAI_GEMM_SMALL_GEMV = 1 turns both off.

int gemv_small_batch(const void * W, const void * Xq, float * Y, int64_t n_out, int64_t n_in,
                     int64_t n_tok, bonsai_stream stream) {
    if (n_tok < 2 || n_tok > 4 || n_out <= 0 || n_out > 0x3fffffff) return -1;
    if (((uintptr_t)W & 15u) != 0 || ((uintptr_t)Xq & 15u) != 0) return -1;
    if (n_tok > knob(pq2host::K_GEMM_SMALL_GEMV, 4)) return -1;
    const uint8_t * w = static_cast<const uint8_t *>(W);
    const uint8_t * x = static_cast<const uint8_t *>(Xq);
    hipStream_t st = (hipStream_t)stream;
    const int nb = (int)(n_in / QK_PQ2);
    if (n_tok >= knob(pq2host::K_MFMA4_MIN_TOK, 3) && (nb == 8 || nb == 40 || nb == 48)) {
        switch (nb) {
            case 8: return launch_mfma4_nt<8>(w, x, Y, (int)n_out, (int)n_tok, st);
            case 40: return launch_mfma4_nt<40>(w, x, Y, (int)n_out, (int)n_tok, st);
            default: return launch_mfma4_nt<48>(w, x, Y, (int)n_out, (int)n_tok, st);
        }
    }
    // 4 tokens on the other widths: the 16x16 MFMA kernel (per-token planes
    // for 4 tokens on the 17408-wide rows measured 21.1 us against 17.4)
    if (n_tok > 3) return -1;
    switch (n_in / QK_PQ2) {
        case 8: return launch_nb_small_nt<8>(w, x, Y, (int)n_out, (int)n_tok, st);
        case 40: return launch_nb_small_nt<40>(w, x, Y, (int)n_out, (int)n_tok, st);
        case 48: return launch_nb_small_nt<48>(w, x, Y, (int)n_out, (int)n_tok, st);
        case 80: return launch_nb_small_nt<80>(w, x, Y, (int)n_out, (int)n_tok, st);
        case 96: return launch_nb_small_nt<96>(w, x, Y, (int)n_out, (int)n_tok, st);
        case 136: return launch_nb_small_nt<136>(w, x, Y, (int)n_out, (int)n_tok, st);
        default: return -1;
    }
}

// Repacked-layout GEMV from fp32 x on the streaming kernel (quantised in
// every workgroup, no rotation), for bonsai_p40_gemv_repack; -1 when the
// width or alignment has no such kernel.
int gemv_repack_streaming(const void * W, const float * x, float * y, int64_t n_out, int64_t n_in,
                          bonsai_stream stream) {
    if (n_out <= 0 || n_out > 0x3fffffff) return -1;
    if (((uintptr_t)W & 15u) != 0 || ((uintptr_t)x & 15u) != 0) return -1;
    if (knob(pq2host::K_GEMV_KERNEL, 0) != 0) return -1;
    const MatGroup mg = single_group(W, y, n_out);
    hipStream_t st = (hipStream_t)stream;
    switch (n_in / QK_PQ2) {
        case 8: return launch_nb_rot<8, 3, true>(mg, 1, x, nullptr, st);
        case 40: return launch_nb_rot<40, 3, true>(mg, 1, x, nullptr, st);
        case 48: return launch_nb_rot<48, 3, true>(mg, 1, x, nullptr, st);
        case 80: return launch_nb_rot<80, 3, true>(mg, 1, x, nullptr, st);
        case 96: return launch_nb_rot<96, 3, true>(mg, 1, x, nullptr, st);
        case 136: return launch_nb_rot<136, 3, true>(mg, 1, x, nullptr, st);
        default: return -1;
    }
}

// FFN gate/up with the SwiGLU glue (bonsai_p40_ffn_gate_up_swiglu and its
// allocation-free form): sync = two zeroed counters, gu = gate rows then up
// rows (2 n_ff floats, 16-byte aligned).
bool ffn_args_ok(const void * Wg, const void * Wu, const float * x, const void * hq, int64_t n_ff,
                 int64_t n_embd) {
    if (Wg == nullptr || Wu == nullptr || x == nullptr || hq == nullptr) return false;
    if (n_ff <= 0 || n_ff % HBLK != 0 || n_ff > 0x3fffffff) return false;
    if (n_embd <= 0 || n_embd % HBLK != 0 || n_embd / QK_PQ2 > (1 << 24)) return false;
    return ((uintptr_t)hq & 3u) == 0;
}

int ffn_gate_up_swiglu(const void * Wg, const void * Wu, const float * x, const float * norm_w,
                       const float * x_signs, const float * h_signs, void * hq, int64_t n_ff, int64_t n_embd,
                       float eps, uint32_t * sync, float * gu, uint32_t * status, hipStream_t st) {
    MatGroup mg{};
    const void * Ws[2] = {Wg, Wu};
    float * ys[2] = {gu, gu + n_ff};
    const int64_t rows[2] = {n_ff, n_ff};
    int64_t total = 0;
    if (make_group(mg, Ws, ys, rows, 2, &total) != 0) return 1;
    mg.norm_w = norm_w;
    mg.eps = eps;
    mg.epi.sync = sync;
    mg.epi.h_signs = h_signs;
    mg.epi.hq = static_cast<uint8_t *>(hq);
    mg.epi.status = status;
    mg.epi.nblk = (int)(n_ff / HBLK);
    const bool al = group_w_aligned(mg, 2) && ((uintptr_t)x & 15u) == 0 && ((uintptr_t)x_signs & 15u) == 0 &&
                    ((uintptr_t)norm_w & 15u) == 0;
    if (al && knob(pq2host::K_GEMV_KERNEL, 0) == 0) {
        int rc = -1;
        if (norm_w != nullptr) {
#define PQ2_RMS_EPI_CASE(N)                                                                         \
    case N: rc = x_signs ? launch_nb_rot<N, 2, false, true, true>(mg, 2, x, x_signs, st)            \
                         : launch_nb_rot<N, 1, false, true, true>(mg, 2, x, x_signs, st); break;
            switch (n_embd / QK_PQ2) {
                PQ2_RMS_EPI_CASE(8) PQ2_RMS_EPI_CASE(40) PQ2_RMS_EPI_CASE(48)
                default: break;
            }
#undef PQ2_RMS_EPI_CASE
        } else {
#define PQ2_ROT_EPI_CASE(N)                                                                         \
    case N: rc = x_signs ? launch_nb_rot<N, 2, false, false, true>(mg, 2, x, x_signs, st)           \
                         : launch_nb_rot<N, 1, false, false, true>(mg, 2, x, x_signs, st); break;
            switch (n_embd / QK_PQ2) {
                PQ2_ROT_EPI_CASE(8) PQ2_ROT_EPI_CASE(40) PQ2_ROT_EPI_CASE(48) PQ2_ROT_EPI_CASE(80)
                PQ2_ROT_EPI_CASE(96) PQ2_ROT_EPI_CASE(136)
                default: break;
            }
#undef PQ2_ROT_EPI_CASE
        }
        if (rc >= 0) return rc;
    }
    // other widths or alignments: the grouped fused GEMV, then the SwiGLU
    // pre-pass (two launches, the same bytes)
    const int rc = fwht_gemv_group_dispatch(mg, 2, x, x_signs, n_embd, st);
    if (rc != 0) return rc;
    return bonsai_p40_swiglu_fwht_quant(gu, gu + n_ff, h_signs, hq, n_ff, st);
}

}  // namespace pq2

// ---------------------------------------------------------------------------
// Allocation-free form of the FFN gate/up launch: its workspace is this
// file-scope device array.  Each GPU the library runs on holds its own copy
// until the process ends.  In host code `scratch` names a host-side stand-in,
// not device memory: its device address comes from hipGetSymbolAddress, once
// per device, and only that address is passed to kernels.
namespace {

constexpr int64_t FFN_NOALLOC_MAX_NFF = BONSAI_P40_FFN_NOALLOC_MAX_NFF;
constexpr size_t FFN_SCRATCH_BYTES = (size_t)BONSAI_P40_FFN_WORKSPACE_BYTES(FFN_NOALLOC_MAX_NFF);

__device__ __attribute__((aligned(256))) uint8_t scratch[FFN_SCRATCH_BYTES];

// Repair of the static workspace after a launch whose block wait gave up
// (sync[1] set): zeroes the row words and the flag; otherwise it reads one
// word and returns.  A kernel rather than a memset, so that a captured graph
// replays it correctly.
__global__ void __launch_bounds__(256) ffn_sync_clear_kernel(uint32_t * sync, uint32_t * rows, int n_words) {
    if (__hip_atomic_load(&sync[1], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == 0u) return;
    for (int i = threadIdx.x; i < n_words; i += 256) rows[i] = 0u;
    __syncthreads();
    if (threadIdx.x == 0) sync[1] = 0u;
}

struct ScratchAddr {
    uint8_t * ptr = nullptr;
    hipError_t err = hipSuccess;
};

// device address of `scratch` on the calling thread's current device, looked
// up with that device current; only a successful lookup is kept (a failed one
// is retried on the next call)
ScratchAddr scratch_address() {
    static std::atomic<uint8_t *> addr[pq2host::MAX_DEVICES];
    static std::mutex mu[pq2host::MAX_DEVICES];
    ScratchAddr a;
    const int d = pq2host::current_device();
    if (d < 0 || d >= pq2host::MAX_DEVICES) {
        a.err = hipErrorInvalidDevice;
        return a;
    }
    a.ptr = addr[d].load(std::memory_order_acquire);
    if (a.ptr != nullptr) return a;
    std::lock_guard<std::mutex> g(mu[d]);
    a.ptr = addr[d].load(std::memory_order_relaxed);
    if (a.ptr != nullptr) return a;
    void * p = nullptr;
    a.err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (a.err != hipSuccess || p == nullptr) {
        (void)hipGetLastError();
        if (a.err == hipSuccess) a.err = hipErrorInvalidSymbol;
        return a;
    }
    a.ptr = static_cast<uint8_t *>(p);
    addr[d].store(a.ptr, std::memory_order_release);
    return a;
}

}  // namespace

extern "C" {

int bonsai_p40_gemv(const void * W, const void * xq, float * y, int64_t n_out, int64_t n_in,
                    bonsai_stream stream) {
    if (n_in <= 0 || n_in % QK_PQ2 != 0 || ((uintptr_t)xq & 3u) != 0) return 1;
    if (n_out <= 0) return 0;
    if (n_out > 0x3fffffff || n_in / QK_PQ2 > (1 << 24) || pq2host::any_null(W, xq, y)) return 1;
    return gemv_group_dispatch<false>(single_group(W, y, n_out), 1, xq, nullptr, n_in, (hipStream_t)stream);
}

int bonsai_p40_gemv_group(const void * const * W, float * const * y, const int64_t * n_out, int n_mat,
                          const void * xq, int64_t n_in, bonsai_stream stream) {
    if (n_in <= 0 || n_in % QK_PQ2 != 0 || ((uintptr_t)xq & 3u) != 0) return 1;
    if (n_in / QK_PQ2 > (1 << 24)) return 1;
    MatGroup mg{};
    int64_t rows = 0;
    if (make_group(mg, W, y, n_out, n_mat, &rows) != 0) return 1;
    if (rows == 0) return 0;
    if (xq == nullptr) return 1;
    return gemv_group_dispatch<false>(mg, n_mat, xq, nullptr, n_in, (hipStream_t)stream);
}

int bonsai_p40_fwht_gemv(const void * W, const float * x, const float * signs, float * y,
                         int64_t n_out, int64_t n_in, bonsai_stream stream) {
    if (n_in <= 0 || n_in % HBLK != 0 || x == nullptr) return 1;
    if (n_out <= 0) return 0;
    if (n_out > 0x3fffffff || n_in / QK_PQ2 > (1 << 24) || pq2host::any_null(W, y)) return 1;
    return fwht_gemv_group_dispatch(single_group(W, y, n_out), 1, x, signs, n_in, (hipStream_t)stream);
}

int bonsai_p40_quant_gemv(const void * W, const float * x, float * y, int64_t n_out, int64_t n_in,
                          bonsai_stream stream) {
    if (n_in <= 0 || n_in % HBLK != 0 || x == nullptr) return 1;
    if (n_out <= 0) return 0;
    if (n_out > 0x3fffffff || n_in / QK_PQ2 > (1 << 24) || pq2host::any_null(W, y)) return 1;
    return quant_gemv_dispatch(single_group(W, y, n_out), x, n_in, (hipStream_t)stream);
}

int bonsai_p40_fwht_gemv_group(const void * const * W, float * const * y, const int64_t * n_out, int n_mat,
                               const float * x, const float * signs, int64_t n_in, bonsai_stream stream) {
    if (n_in <= 0 || n_in % HBLK != 0 || x == nullptr) return 1;
    if (n_in / QK_PQ2 > (1 << 24)) return 1;
    MatGroup mg{};
    int64_t rows = 0;
    if (make_group(mg, W, y, n_out, n_mat, &rows) != 0) return 1;
    if (rows == 0) return 0;
    return fwht_gemv_group_dispatch(mg, n_mat, x, signs, n_in, (hipStream_t)stream);
}

int bonsai_p40_rmsnorm_fwht_gemv_group(const void * const * W, float * const * y, const int64_t * n_out,
                                       int n_mat, const float * x, const float * norm_w, const float * signs,
                                       int64_t n_in, float eps, bonsai_stream stream) {
    if (n_in <= 0 || n_in % HBLK != 0 || x == nullptr || norm_w == nullptr) return 1;
    if (n_in / QK_PQ2 > (1 << 24)) return 1;
    MatGroup mg{};
    int64_t rows = 0;
    if (make_group(mg, W, y, n_out, n_mat, &rows) != 0) return 1;
    if (rows == 0) return 0;
    mg.norm_w = norm_w;
    mg.eps = eps;
    return fwht_gemv_group_dispatch(mg, n_mat, x, signs, n_in, (hipStream_t)stream);
}

int bonsai_p40_ffn_gate_up_swiglu(const void * Wg, const void * Wu, const float * x, const float * norm_w,
                                  const float * x_signs, const float * h_signs, void * hq, int64_t n_ff,
                                  int64_t n_embd, float eps, void * workspace, uint32_t * status,
                                  bonsai_stream stream) {
    if (!pq2::ffn_args_ok(Wg, Wu, x, hq, n_ff, n_embd) || workspace == nullptr ||
        ((uintptr_t)workspace & 15u) != 0)
        return 1;
    uint8_t * ws = static_cast<uint8_t *>(workspace);
    return pq2::ffn_gate_up_swiglu(Wg, Wu, x, norm_w, x_signs, h_signs, hq, n_ff, n_embd, eps,
                                   reinterpret_cast<uint32_t *>(ws),
                                   reinterpret_cast<float *>(ws + BONSAI_P40_FFN_SYNC_BYTES), status,
                                   (hipStream_t)stream);
}

int bonsai_p40_ffn_gate_up_swiglu_noalloc(const void * Wg, const void * Wu, const float * x,
                                          const float * norm_w, const float * x_signs, const float * h_signs,
                                          void * hq, int64_t n_ff, int64_t n_embd, float eps, uint32_t * status,
                                          bonsai_stream stream) {
    if (!pq2::ffn_args_ok(Wg, Wu, x, hq, n_ff, n_embd)) return 1;
    if (n_ff > FFN_NOALLOC_MAX_NFF) return 1;          // beyond the static scratch
    const ScratchAddr a = scratch_address();
    if (a.err != hipSuccess) return (int)a.err;
    hipStream_t st = (hipStream_t)stream;
    uint32_t * sync = reinterpret_cast<uint32_t *>(a.ptr);
    hipLaunchKernelGGL(ffn_sync_clear_kernel, dim3(1), dim3(256), 0, st, sync,
                       reinterpret_cast<uint32_t *>(a.ptr + BONSAI_P40_FFN_SYNC_BYTES), (int)(2 * n_ff));
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return (int)e;
    return pq2::ffn_gate_up_swiglu(Wg, Wu, x, norm_w, x_signs, h_signs, hq, n_ff, n_embd, eps, sync,
                                   reinterpret_cast<float *>(a.ptr + BONSAI_P40_FFN_SYNC_BYTES), status, st);
}

int bonsai_p40_chunk_dots(const void * W, const void * xq, int32_t * out, int64_t n_out,
                          int64_t n_in, bonsai_stream stream) {
    if (n_in <= 0 || n_in % QK_PQ2 != 0 || ((uintptr_t)xq & 3u) != 0) return 1;
    if (n_out <= 0) return 0;
    if (n_out > 0x3fffffff || n_in / QK_PQ2 > (1 << 24) || pq2host::any_null(W, xq, out)) return 1;
    return gemv_group_dispatch<true>(single_group(W, nullptr, n_out), 1, xq, out, n_in, (hipStream_t)stream);
}

}  // extern "C"
