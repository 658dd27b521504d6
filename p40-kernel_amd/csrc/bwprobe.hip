// bwprobe.hip -- measurement probes used by bench.py to report "% of
// achievable" next to "% of peak":
//  * HBM streaming-read ceiling (the analog of the reference's tools/bwtest.cu
//    read_kernel, tools/bwtest.cu:37-47): every lane reads 16-byte vectors
//    grid-stride and folds them with XOR, one word per workgroup is written so
//    the loads cannot be elided;
//  * MFMA peak: back-to-back independent int8 (v_mfma_i32_16x16x64_i8) or f16
//    (v_mfma_f32_16x16x32_f16) matrix instructions, with each wave's shader
//    clock and real-time counters read around its loop so the host can derive
//    the clock the MFMAs ran at;
//  * VALU / MFMA overlap: the same MFMAs with and without independent fp32
//    FMAs in the same wave stream;
//  * the decode GEMV's weight stream alone (the analog of the reference's
//    GEMV-addressing read, tools/bwtest.cu:70-90): the unit LDS-DMA schedule
//    of gemv_nb_kernel (same units, grid, wave numbering, ring depth, issue
//    rounds and waits) with no activation and no arithmetic.
#include "gemv_device.h"
#include "host_state.h"
#include "../../include/bonsai_p40.h"

namespace {

typedef uint32_t v4u __attribute__((ext_vector_type(4)));

__global__ void __launch_bounds__(256)
stream_read_kernel(const v4u * __restrict__ src, size_t n16, uint32_t * __restrict__ out) {
    const size_t stride = (size_t)gridDim.x * 256;
    v4u acc = {0u, 0u, 0u, 0u};
    size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    for (; i + 3 * stride < n16; i += 4 * stride) {
        const v4u a = __builtin_nontemporal_load(src + i);
        const v4u b = __builtin_nontemporal_load(src + i + stride);
        const v4u c = __builtin_nontemporal_load(src + i + 2 * stride);
        const v4u d = __builtin_nontemporal_load(src + i + 3 * stride);
        acc ^= a ^ b ^ c ^ d;
    }
    for (; i < n16; i += stride) acc ^= __builtin_nontemporal_load(src + i);
    const uint32_t v = acc.x ^ acc.y ^ acc.z ^ acc.w;
    if (v == 0x9e3779b9u) out[blockIdx.x] = v;   // practically never true; keeps the loads live
}

typedef int v4i __attribute__((ext_vector_type(4)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int PROBE_ACC = 4;        // independent accumulators per wave (more get shuffled)

// KIND 0: int8 16x16x64 (32768 ops per instruction), KIND 1: f16 16x16x32
// (16384 ops).  Each wave issues iters * PROBE_ACC MFMAs in chains of
// PROBE_ACC independent accumulators.  Wave 0 of each workgroup records its
// shader-clock and real-time deltas in clk[2 * blockIdx.x + {0, 1}].
template <int KIND>
__global__ void __launch_bounds__(256)
mfma_probe_kernel(int iters, uint64_t * __restrict__ clk, uint32_t * __restrict__ sink) {
    const int lane = threadIdx.x & 63;
    v4i ai = {lane, lane * 3, lane ^ 5, 7};
    v4i bi = {lane + 1, lane * 5, lane ^ 9, 3};
    v8h ah, bh;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        ah[k] = (_Float16)(0.001f * (float)(lane + k));
        bh[k] = (_Float16)(0.002f * (float)(lane - k));
    }
    v4i acci[PROBE_ACC];
    v4f accf[PROBE_ACC];
    // distinct lane-dependent starting values: accumulators that start equal
    // get coalesced by the compiler into shuffled register copies in the loop
#pragma unroll
    for (int k = 0; k < PROBE_ACC; ++k) {
        acci[k] = (v4i){lane + k, lane * (k + 2), lane ^ (k + 1), 3 * k - lane};
        accf[k] = (v4f){(float)(lane + k), (float)(lane * (k + 2)), (float)(lane ^ (k + 1)),
                        (float)(3 * k - lane)};
    }
    const uint64_t c0 = __builtin_readcyclecounter();
    const uint64_t r0 = __builtin_amdgcn_s_memrealtime();
    for (int i = 0; i < iters; ++i) {
#pragma unroll
        for (int k = 0; k < PROBE_ACC; ++k) {
            if constexpr (KIND == 0)
                acci[k] = __builtin_amdgcn_mfma_i32_16x16x64_i8(ai, bi, acci[k], 0, 0, 0);
            else
                accf[k] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bh, accf[k], 0, 0, 0);
        }
    }
    // the deltas are read after the last MFMA's result is consumed
    uint32_t fold = 0;
#pragma unroll
    for (int k = 0; k < PROBE_ACC; ++k) {
        if constexpr (KIND == 0) fold ^= (uint32_t)(acci[k][0] ^ acci[k][1] ^ acci[k][2] ^ acci[k][3]);
        else fold ^= __float_as_uint(accf[k][0] + accf[k][1] + accf[k][2] + accf[k][3]);
    }
    fold = __builtin_amdgcn_readfirstlane(fold);
    const uint64_t c1 = __builtin_readcyclecounter();
    const uint64_t r1 = __builtin_amdgcn_s_memrealtime();
    if (threadIdx.x == 0) {
        clk[2 * blockIdx.x] = c1 - c0;
        clk[2 * blockIdx.x + 1] = r1 - r0;
    }
    if (fold == 0x9e3779b9u) sink[blockIdx.x] = fold;   // keeps the MFMAs live
}

// VALU / MFMA overlap probe.  Per iteration a wave issues 4 independent
// v_mfma_f32_16x16x32_f16 (MODE 0 or 2) and nf x 16 independent fp32 FMAs
// (MODE 1 or 2): with nf = 1 that is 4 FMAs per MFMA, the ratio of the
// prefill GEMM's per-chunk rescale.  Comparing the three modes' times shows
// whether the matrix core and the VALU work at the same time for one wave
// stream.  The MFMAs are inline asm so that the compiler keeps the four
// accumulators in place (it otherwise shuffles equal-looking ones).
template <int MODE>
__global__ void __launch_bounds__(256)
overlap_probe_kernel(int iters, int nf, uint32_t * __restrict__ sink) {
    const int lane = threadIdx.x & 63;
    v8h a, b;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        a[i] = (_Float16)(0.001f * (float)(lane + i));
        b[i] = (_Float16)(0.002f * (float)(lane - i));
    }
    v4f acc[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
        acc[i] = (v4f){(float)(lane + i), (float)(lane * (i + 2)), (float)(lane ^ (i + 1)), (float)(3 * i - lane)};
    float f[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) f[i] = 0.5f * (float)lane + (float)i;
    const float sc = 1.0001f + 1e-6f * (float)lane, tc = 0.999f;
    for (int it = 0; it < iters; ++it) {
        if constexpr (MODE != 1) {
#pragma unroll
            for (int i = 0; i < 4; ++i)
                asm volatile("v_mfma_f32_16x16x32_f16 %0, %1, %2, %0" : "+v"(acc[i]) : "v"(a), "v"(b));
        }
        if constexpr (MODE != 0) {
            for (int r = 0; r < nf; ++r) {
#pragma unroll
                for (int i = 0; i < 16; ++i) f[i] = fmaf(f[i], sc, tc);
            }
        }
    }
    float z = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) z += acc[i][0] + acc[i][1] + acc[i][2] + acc[i][3];
#pragma unroll
    for (int i = 0; i < 16; ++i) z += f[i];
    if (z == 1234.5f) sink[blockIdx.x] = 1u;       // practically never: keeps the work live
}

// The prefill GEMM's chunk step for one 32 x 32 wave tile, with nothing
// else: 4 v_mfma_f32_16x16x32_f16 with a zero accumulator input, then the 16
// fp32 FMAs that fold their results into the output accumulators with the
// token scale -- compiler-scheduled, as in the GEMM.  The time per
// iteration is the floor of the GEMM's per-chunk cost without operand
// staging, LDS reads or barriers.
__global__ void __launch_bounds__(256)
gemm_core_probe_kernel(int iters, uint32_t * __restrict__ sink) {
    const int lane = threadIdx.x & 63;
    // four distinct A operands (four equal MFMAs would be merged into one by
    // the compiler) and a B operand that changes every iteration (so that no
    // MFMA is loop-invariant): one f16 add per iteration beside the work
    v8h a[4], b;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
#pragma unroll
        for (int t = 0; t < 4; ++t) a[t][i] = (_Float16)(0.001f * (float)(lane + i + 7 * t));
        b[i] = (_Float16)(0.002f * (float)(lane - i));
    }
    float acc[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[i] = 0.25f * (float)lane + (float)i;
    const float da = 1.0001f + 1e-6f * (float)lane;
    // software-pipelined as in the GEMM: the FMAs of iteration it fold the
    // products of iteration it - 1, so the four products are live at once
    // and no FMA waits for the MFMA just issued
    // (two iterations per trip with the product sets alternating, so that no
    // register copies carry them across)
    v4f s0[4], s1[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) s0[t] = s1[t] = (v4f){0.0f, 0.0f, 0.0f, 0.0f};
    auto step = [&](v4f (&out)[4], const v4f (&in)[4]) __attribute__((always_inline)) {
#pragma unroll
        for (int t = 0; t < 4; ++t)
            out[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a[t], b, (v4f){0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int i = 0; i < 4; ++i) acc[4 * t + i] = fmaf(da, in[t][i], acc[4 * t + i]);
        b[0] += (_Float16)1.0f;                     // a new B operand every iteration
    };
    for (int it = 0; it + 1 < iters; it += 2) {
        step(s1, s0);
        step(s0, s1);
    }
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[4 * t + i] = fmaf(da, s0[t][i], acc[4 * t + i]);
    float z = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) z += acc[i];
    if (z == 1234.5f) sink[blockIdx.x] = 1u;       // practically never: keeps the work live
}

// The GEMV's unit DMA alone.  Units of G rows are dealt to the grid's waves
// grid-strided with the GEMV's XCD-grouped numbering; each wave keeps D units
// in flight in a ring of D + 1 LDS slots: wait for unit i, issue unit i + D,
// and do nothing with the bytes.  Issue rounds are separated by workgroup
// barriers as in the GEMV.  Wave 0 folds one word of its last unit into a
// sink word that is written only in a practically impossible case.
template <int NB, int D, int WAVES>
__global__ void __launch_bounds__(64 * WAVES)
unit_dma_probe_kernel(const uint8_t * __restrict__ W, int n_out, int units_per_wave, int xcd_log2m,
                      uint32_t * __restrict__ sink) {
    using P = pq2::NbSpec<NB>;
    constexpr int SL = D + 1;
    __shared__ __attribute__((aligned(16))) uint8_t ring_all[WAVES][SL][P::LDSB];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    uint8_t (*ring)[P::LDSB] = ring_all[wave];
    const int n_units = (n_out + P::G - 1) / P::G;
    int gw = wave * gridDim.x + blockIdx.x;
    if (xcd_log2m > 0) {
        const int K = gridDim.x >> 3;
        const int t = wave * K + (blockIdx.x >> 3);
        const int m = (1 << xcd_log2m) - 1;
        gw = (((t >> xcd_log2m) << 3) + (blockIdx.x & 7)) << xcd_log2m | (t & m);
    }
    const int NW = gridDim.x * WAVES;
    const int nu = gw < n_units ? min(units_per_wave, (n_units - 1 - gw) / NW + 1) : 0;
    const int m_bytes = n_out * pq2::PQ2_BYTES * NB;
    uint32_t poff[P::NPL];
#pragma unroll
    for (int k = 0; k < P::NPL; ++k) poff[k] = 16u * (uint32_t)min(lane + 64 * k, P::NPIECE - 1);
#pragma unroll
    for (int i = 0; i < D; ++i) {
        __builtin_amdgcn_s_barrier();
        if (nu > 0)
            pq2::unit_buffer_dma<P::NPL>(W, m_bytes, (uint32_t)(gw + min(i, nu - 1) * NW) * (uint32_t)P::UB, poff,
                                         ring[i]);
        __builtin_amdgcn_sched_barrier(0);
    }
    for (int i = 0; i < nu; ++i) {
        const int newer = min(D - 1, nu - 1 - i);
        if (newer >= 2) pq2::wait_vmcnt<2 * P::NPL>();
        else if (newer == 1) pq2::wait_vmcnt<P::NPL>();
        else pq2::wait_vmcnt<0>();
        __builtin_amdgcn_wave_barrier();
        if (i + D < nu)
            pq2::unit_buffer_dma<P::NPL>(W, m_bytes, (uint32_t)(gw + (i + D) * NW) * (uint32_t)P::UB, poff,
                                         ring[(i + D) % SL]);
    }
    pq2::wait_vmcnt<0>();
    if (nu > 0 && lane == 0 && wave == 0) {
        const uint32_t v = *reinterpret_cast<const uint32_t *>(&ring[(nu - 1) % SL][0]);
        if (v == 0x9e3779b9u && n_out < 0) sink[blockIdx.x] = v;   // never: n_out > 0
    }
}

// An empty kernel: the cost of a launch that depends on the one before it.
__global__ void __launch_bounds__(1024) empty_probe_kernel(uint32_t * __restrict__ sink) {
    if (threadIdx.x == 0x7fffffff) sink[0] = 1u;    // never
}

}  // namespace

// VALU / MFMA overlap probe: `blocks` workgroups of 4 waves, each wave
// iters x (4 MFMAs if mode != 1, nf x 16 FMAs if mode != 0); mode 3 is the
// prefill GEMM's chunk step (4 MFMAs, then 16 FMAs on their results; nf
// unused).  sink needs `blocks` words.  Errors: 1 on bad arguments.
extern "C" int bonsai_p40_overlap_probe(int mode, int nf, int blocks, int iters, uint32_t * sink,
                                        bonsai_stream stream) {
    if (blocks <= 0 || iters <= 0 || nf < 0 || nf > 16 || sink == nullptr || mode < 0 || mode > 3) return 1;
    const hipStream_t st = (hipStream_t)stream;
    if (mode == 3) hipLaunchKernelGGL(gemm_core_probe_kernel, dim3((unsigned)blocks), dim3(256), 0, st, iters, sink);
    else if (mode == 0) hipLaunchKernelGGL(overlap_probe_kernel<0>, dim3((unsigned)blocks), dim3(256), 0, st, iters, nf, sink);
    else if (mode == 1) hipLaunchKernelGGL(overlap_probe_kernel<1>, dim3((unsigned)blocks), dim3(256), 0, st, iters, nf, sink);
    else hipLaunchKernelGGL(overlap_probe_kernel<2>, dim3((unsigned)blocks), dim3(256), 0, st, iters, nf, sink);
    return (int)hipGetLastError();
}

// MFMA peak probe: `blocks` workgroups of 4 waves, each wave issuing iters *
// 4 MFMAs of the chosen kind (0: int8 16x16x64, 1: f16 16x16x32).  clk needs
// 2 * blocks words (shader-clock and real-time deltas of each workgroup's
// wave 0), sink `blocks` words (written only in a practically impossible
// case).  Errors: 1 on bad arguments.
extern "C" int bonsai_p40_mfma_probe(int kind, int blocks, int iters, uint64_t * clk, uint32_t * sink,
                                     bonsai_stream stream) {
    if (blocks <= 0 || iters <= 0 || clk == nullptr || sink == nullptr || (kind != 0 && kind != 1)) return 1;
    if (kind == 0)
        hipLaunchKernelGGL(mfma_probe_kernel<0>, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, iters,
                           clk, sink);
    else
        hipLaunchKernelGGL(mfma_probe_kernel<1>, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, iters,
                           clk, sink);
    return (int)hipGetLastError();
}

// Launch-cost probe: one empty kernel of `blocks` workgroups of `threads`
// threads (1..1024).  Replayed back to back, its time per launch is what any
// launch that depends on the one before it costs.  Errors: 1 on bad arguments.
extern "C" int bonsai_p40_launch_probe(int blocks, int threads, uint32_t * sink, bonsai_stream stream) {
    if (blocks <= 0 || threads <= 0 || threads > 1024 || sink == nullptr) return 1;
    hipLaunchKernelGGL(empty_probe_kernel, dim3((unsigned)blocks), dim3((unsigned)threads), 0, (hipStream_t)stream,
                       sink);
    return (int)hipGetLastError();
}

namespace {

// the GEMV's launch geometry for the probe's two row widths: 5120 columns (2-row
// units, one 8-wave workgroup per CU, ring depth 2) and 17408 columns (1-row
// units, one 4-wave workgroup per CU, ring depth 2); grid, units per wave and
// XCD grouping follow the GEMV's dispatcher for a single matrix
template <int NB, int D, int WAVES>
int launch_unit_dma_probe(const uint8_t * W, int n_out, uint32_t * sink, hipStream_t st) {
    using P = pq2::NbSpec<NB>;
    const int n_units = (n_out + P::G - 1) / P::G;
    int blocks = pq2host::device_info().cus;
    const int max_blocks = (n_units + WAVES - 1) / WAVES;
    if (blocks > max_blocks) blocks = max_blocks;
    const int NW = blocks * WAVES;
    int upw = (n_units + NW - 1) / NW;
    if (upw > 64 / P::G) {
        upw = 64 / P::G;
        blocks = (n_units + upw * WAVES - 1) / (upw * WAVES);
    }
    int xl = 3;
    if (blocks % 8 != 0) xl = 0;
    while (xl > 0 && ((blocks / 8) * WAVES) % (1 << xl) != 0) --xl;
    hipLaunchKernelGGL((unit_dma_probe_kernel<NB, D, WAVES>), dim3(blocks), dim3(64 * WAVES), 0, st, W, n_out, upw,
                       xl, sink);
    return (int)hipGetLastError();
}

}  // namespace

extern "C" int bonsai_p40_unit_dma_probe(const void * W, int64_t n_out, int64_t n_in, uint32_t * sink,
                                         bonsai_stream stream) {
    if (W == nullptr || sink == nullptr || n_out <= 0 || ((uintptr_t)W & 3u) != 0) return 1;
    if (n_in != 5120 && n_in != 17408) return 1;
    if (n_out * (n_in / 128) * 34 >= 0x80000000ll) return 1;
    const hipStream_t st = (hipStream_t)stream;
    const uint8_t * w = static_cast<const uint8_t *>(W);
    if (n_in == 5120) return launch_unit_dma_probe<40, 2, 8>(w, (int)n_out, sink, st);
    return launch_unit_dma_probe<136, 2, 4>(w, (int)n_out, sink, st);
}

extern "C" int bonsai_p40_stream_read(const void * buf, int64_t bytes, uint32_t * out, int blocks,
                                      bonsai_stream stream) {
    if (bytes <= 0 || bytes % 16 != 0 || ((uintptr_t)buf & 15u) != 0 || blocks <= 0) return 1;
    if (buf == nullptr || out == nullptr) return 1;
    hipLaunchKernelGGL(stream_read_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream,
                       (const v4u *)buf, (size_t)bytes / 16, out);
    return (int)hipGetLastError();
}
