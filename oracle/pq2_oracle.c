/*
 * pq2_oracle.c -- CPU restatement of the Bonsai-P40 PQ2_0 matmul path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the parity checker for the HIP
 * library in p40-kernel_amd/csrc.  Only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg may load it, and only to check or to time the
 * CPU side; no product code path calls it.
 *
 * Every function restates the semantics of one reference function (cited as
 * path:line in /root/reference).  Byte layouts are handled as raw byte arrays
 * with explicit little-endian packing, so the file is plain C99.
 *
 * Pinning (what fixes each function independently of this restatement):
 *   orc_f32_to_f16      -- compiled reference over all 2^32 float patterns
 *                          (tests/test_oracle.py, hash comparison) + F1 fixture
 *   orc_f16_to_f32      -- all 2^16 patterns vs the compiled reference
 *   orc_quantize_q8_1   -- F2 fixtures (seeded, constructed ties, zero chunks)
 *   orc_fwht_blocks     -- F3 fixtures (bit patterns) + naive Sylvester matrix
 *   orc_chunk_sumi      -- F4 fixtures + brute-force integer dot on the plain layout
 *   orc_row_dot/gemv    -- F4 fixtures (reference row dots, bit patterns)
 *   orc_repack_*        -- F5 fixtures + round trip
 *   orc_gemm            -- F6 fixtures + double-precision dequantised reference
 *   orc_swiglu          -- F7 fixtures (chain) within expf ulp tolerance
 *   orc_rmsnorm         -- F8 fixtures (bit patterns) + float64 closed form
 *   orc_quantize_pq2_0  -- F9 fixture (lroundf ties, zero, fp16-tie, subnormal
 *                          and overflowing scales) + closed form
 *   orc_dequantize_pq2_0-- F9 fixture (bit patterns, code 3) + value rule
 *   orc_pq2_0_dot_f32   -- F9 fixture (bit patterns) + float64 dot
 */
#include <math.h>
#include <stdint.h>
#include <string.h>
#include <stdlib.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define QK_PQ2 128           /* weights per block_pq2_0   (src/pq2_0.h:39-43)  */
#define QK8 32               /* elements per block_q8_1    (src/pq2_0.h:35-41)  */
#define PQ2_BYTES 34         /* fp16 d + 32 code bytes     (src/pq2_0.h:45-48)  */
#define Q81_BYTES 36         /* fp16 d + int16 s + 32 int8 (src/pq2_0.h:50-54)  */
#define HBLK 1024            /* Hadamard block             (src/fwht.h:15-16)   */

static inline uint16_t ld16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }
static inline void st16(uint8_t *p, uint16_t v) { p[0] = (uint8_t)v; p[1] = (uint8_t)(v >> 8); }

/* ---- fp16 conversions: src/p40_common.h:57-80 (decode), :82-114 (encode,
 *      magnitude rounded half away from zero) -------------------------------- */
float orc_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu, bits;
    if (e == 0) {
        if (m == 0) {
            bits = sign;
        } else {                              /* subnormal: renormalise */
            int ex = 113;                     /* 127 - 15 + 1 */
            while (!(m & 0x400u)) { m <<= 1; --ex; }
            bits = sign | ((uint32_t)ex << 23) | ((m & 0x3ffu) << 13);
        }
    } else if (e == 31) {
        bits = sign | 0x7f800000u | (m << 13);
    } else {
        bits = sign | ((e + 112u) << 23) | (m << 13);
    }
    float f; memcpy(&f, &bits, 4); return f;
}

uint16_t orc_f32_to_f16(float f) {
    uint32_t x; memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t fe = (x >> 23) & 0xffu;
    uint32_t mant = x & 0x7fffffu;
    int32_t e = (int32_t)fe - 112;            /* rebias 127 -> 15 */
    if (fe == 0xffu) return (uint16_t)(sign | 0x7c00u | (mant ? 0x200u : 0u));
    if (e >= 31) return (uint16_t)(sign | 0x7c00u);
    if (e <= 0) {                              /* f16 subnormal or zero */
        if (e < -10) return (uint16_t)sign;
        uint32_t full = mant | 0x800000u;
        uint32_t sh = (uint32_t)(14 - e);      /* 14..24 */
        uint32_t q = full >> sh;
        q += (full >> (sh - 1)) & 1u;          /* half (and above) rounds up */
        return (uint16_t)(sign | q);
    }
    uint32_t q = mant >> 13;
    if (mant & 0x1000u) {
        ++q;
        if (q == 0x400u) { q = 0; ++e; if (e >= 31) return (uint16_t)(sign | 0x7c00u); }
    }
    return (uint16_t)(sign | ((uint32_t)e << 10) | q);
}

/* FNV-1a style hash over encodes of bit patterns start, start+stride, ... */
uint64_t orc_f16_encode_hash(uint64_t start, uint64_t count, uint64_t stride) {
    uint64_t h = 1469598103934665603ull;
    for (uint64_t i = 0; i < count; ++i) {
        uint32_t bits = (uint32_t)(start + i * stride);
        float f; memcpy(&f, &bits, 4);
        h = (h ^ orc_f32_to_f16(f)) * 1099511628211ull;
    }
    return h;
}

/* round half away from zero, the lroundf of src/pq2_0.h:117 */
static inline long round_away(float v) { return lroundf(v); }

/* ---- Q8_1 activation quantiser: src/pq2_0.h:99-126 -----------------------
 * Per 32: amax, d = amax/127, id = 1/d (0 for an all-zero chunk),
 * q = lroundf(x*id) clamped to +-127, s = raw int16 sum of q.
 * permute != 0: position j holds element 16(j>>4) + 4(j&3) + ((j>>2)&3).   */
void orc_quantize_q8_1(const float *x, uint8_t *y, int64_t k, int permute) {
    for (int64_t c = 0; c < k / QK8; ++c) {
        const float *xc = x + c * QK8;
        uint8_t *yb = y + c * Q81_BYTES;
        float amax = 0.0f;
        for (int j = 0; j < QK8; ++j) amax = fmaxf(amax, fabsf(xc[j]));
        const float d = amax / 127.0f;
        const float id = d > 0.0f ? 1.0f / d : 0.0f;
        int8_t q[QK8];
        int sum = 0;
        for (int j = 0; j < QK8; ++j) {
            volatile float prod = xc[j] * id;   /* one rounded fp32 product */
            long v = round_away(prod);
            if (v < -127) v = -127;
            if (v > 127) v = 127;
            q[j] = (int8_t)v; sum += (int)v;
        }
        st16(yb, orc_f32_to_f16(d));
        st16(yb + 2, (uint16_t)(int16_t)sum);
        for (int j = 0; j < QK8; ++j) {
            const int src = permute ? (16 * (j >> 4) + 4 * (j & 3) + ((j >> 2) & 3)) : j;
            yb[4 + j] = (uint8_t)q[src];
        }
    }
}

/* Each of n_tok token rows x[t][0..k) quantised on its own (permuted) and
 * stored chunk-major: block (c, t) at index c*n_tok + t.  This is the X layout
 * of the reference GEMM (src/kernels/gemm_p40.cu:75, tests/test_p40.cpp:438-447). */
void orc_quantize_chunk_major(const float *x, uint8_t *y, int64_t k, int64_t n_tok) {
    uint8_t tmp[Q81_BYTES];
    for (int64_t t = 0; t < n_tok; ++t)
        for (int64_t c = 0; c < k / QK8; ++c) {
            orc_quantize_q8_1(x + t * k + c * QK8, tmp, QK8, 1);
            memcpy(y + (c * n_tok + t) * Q81_BYTES, tmp, Q81_BYTES);
        }
}

/* ---- FWHT-1024: src/fwht.h:20-42.  Signs (optional) are a length-n vector,
 * block b uses signs + 1024*b (the host form, src/fwht.h:40).  Stage order
 * h = 1, 2, ..., 512 is kept, so results are bit-exact with the reference.  */
void orc_fwht_1024(float *x, const float *signs) {
    if (signs) for (int i = 0; i < HBLK; ++i) x[i] *= signs[i];
    for (int h = 1; h < HBLK; h <<= 1)
        for (int i = 0; i < HBLK; i += 2 * h)
            for (int j = i; j < i + h; ++j) {
                const float a = x[j], b = x[j + h];
                x[j] = a + b;
                x[j + h] = a - b;
            }
    for (int i = 0; i < HBLK; ++i) x[i] *= (1.0f / 32.0f);
}

void orc_fwht_blocks(float *x, const float *signs, int64_t n) {
    for (int64_t b = 0; b < n; b += HBLK) orc_fwht_1024(x + b, signs ? signs + b : NULL);
}

/* ---- PQ2_0 reference quantiser / dequantiser: src/pq2_0.h:62-90 -------- */
void orc_dequantize_pq2_0(const uint8_t *w, float *y, int64_t k) {
    for (int64_t b = 0; b < k / QK_PQ2; ++b) {
        const uint8_t *blk = w + b * PQ2_BYTES;
        const float d = orc_f16_to_f32(ld16(blk));
        for (int j = 0; j < QK_PQ2; ++j) {
            const int code = (blk[2 + (j >> 2)] >> ((j & 3) * 2)) & 3;
            y[b * QK_PQ2 + j] = (float)(code - 1) * d;
        }
    }
}

void orc_quantize_pq2_0(const float *x, uint8_t *w, int64_t k) {
    for (int64_t b = 0; b < k / QK_PQ2; ++b) {
        const float *xb = x + b * QK_PQ2;
        uint8_t *blk = w + b * PQ2_BYTES;
        float amax = 0.0f;
        for (int j = 0; j < QK_PQ2; ++j) amax = fmaxf(amax, fabsf(xb[j]));
        const float id = amax > 0.0f ? 1.0f / amax : 0.0f;
        st16(blk, orc_f32_to_f16(amax));
        memset(blk + 2, 0, 32);
        for (int j = 0; j < QK_PQ2; ++j) {
            volatile float prod = xb[j] * id;
            long q = round_away(prod) + 1;
            if (q < 0) q = 0;
            if (q > 3) q = 3;
            blk[2 + (j >> 2)] |= (uint8_t)(q << ((j & 3) * 2));
        }
    }
}

/* ---- float block dot: src/pq2_0.h:134-142 -------------------------------
 * the definition every kernel reproduces: sum_j (code_j - 1) * a[j] in
 * element order (fp32, no contraction), then times the block scale.      */
float orc_pq2_0_dot_f32(const uint8_t *w, const float *a) {
    const float d = orc_f16_to_f32(ld16(w));
    float acc = 0.0f;
    for (int j = 0; j < QK_PQ2; ++j) {
        const int code = (w[2 + (j >> 2)] >> ((j & 3) * 2)) & 3;
        volatile float prod = (float)(code - 1) * a[j];
        acc += prod;
    }
    return acc * d;
}

/* ---- integer chunk dot: src/pq2_0.h:149-172 ------------------------------
 * sumi = sum_k dp4a((w >> 2k) & 0x03030303, a_k) - s over the two 16-code
 * words of chunk iqs; each dp4a is four signed byte products.             */
static inline int dp4a(uint32_t a, uint32_t b, int c) {
    for (int i = 0; i < 4; ++i) c += (int)(int8_t)(a >> (8 * i)) * (int)(int8_t)(b >> (8 * i));
    return c;
}

int32_t orc_chunk_sumi(const uint8_t *wblock, const uint8_t *ablock, int iqs) {
    const uint8_t *qs = wblock + 2 + iqs * 8;
    const uint8_t *as = ablock + 4;
    int sumi = 0;
    for (int word = 0; word < 2; ++word) {
        uint32_t wv = (uint32_t)qs[4 * word] | ((uint32_t)qs[4 * word + 1] << 8) |
                      ((uint32_t)qs[4 * word + 2] << 16) | ((uint32_t)qs[4 * word + 3] << 24);
        for (int k = 0; k < 4; ++k) {
            const uint8_t *ap = as + 16 * word + 4 * k;
            uint32_t av = (uint32_t)ap[0] | ((uint32_t)ap[1] << 8) | ((uint32_t)ap[2] << 16) |
                          ((uint32_t)ap[3] << 24);
            sumi = dp4a((wv >> (2 * k)) & 0x03030303u, av, sumi);
        }
    }
    return sumi - (int16_t)ld16(ablock + 2);
}

/* float contribution: (f16(dw) * f16(da)) * sumi, src/pq2_0.h:171-172 */
static inline float chunk_dot(const uint8_t *wblock, const uint8_t *ablock, int iqs) {
    const float d = orc_f16_to_f32(ld16(wblock)) * orc_f16_to_f32(ld16(ablock));
    return d * (float)orc_chunk_sumi(wblock, ablock, iqs);
}

/* pq2_0_row_dot_perm, src/pq2_0.h:183-191: sequential fp32 over blocks, chunks */
float orc_row_dot(const uint8_t *w, const uint8_t *a, int64_t n) {
    float acc = 0.0f;
    for (int64_t b = 0; b < n / QK_PQ2; ++b)
        for (int iqs = 0; iqs < 4; ++iqs)
            acc += chunk_dot(w + b * PQ2_BYTES, a + (b * 4 + iqs) * Q81_BYTES, iqs);
    return acc;
}

/* y[r] = row_dot(W[r], xq) for every row -- the bonsai_p40_gemv contract
 * (include/bonsai_p40.h:18-22).  nthreads > 1 splits rows with OpenMP.    */
void orc_gemv(const uint8_t *W, const uint8_t *xq, float *y, int64_t n_out, int64_t n_in,
              int nthreads) {
    const int64_t stride = n_in / QK_PQ2 * PQ2_BYTES;
#ifdef _OPENMP
#pragma omp parallel for schedule(static) num_threads(nthreads > 0 ? nthreads : 1)
#endif
    for (int64_t r = 0; r < n_out; ++r) y[r] = orc_row_dot(W + r * stride, xq, n_in);
    (void)nthreads;
}

/* int32 sumi of every (row, chunk): out[r * n_in/32 + c] */
void orc_chunk_dots(const uint8_t *W, const uint8_t *xq, int32_t *out, int64_t n_out,
                    int64_t n_in) {
    const int64_t nb = n_in / QK_PQ2, stride = nb * PQ2_BYTES;
    for (int64_t r = 0; r < n_out; ++r)
        for (int64_t c = 0; c < n_in / QK8; ++c)
            out[r * (n_in / QK8) + c] =
                orc_chunk_sumi(W + r * stride + (c / 4) * PQ2_BYTES, xq + c * Q81_BYTES, (int)(c % 4));
}

/* Chunk-major GEMM, the semantics of tests/test_p40.cpp:449-470 (and of
 * gemm_pq2_0_p40_kernel, src/kernels/gemm_p40.cu:44-139):
 *   Y[r*n_tok + t] = sum_b sum_iqs pq2_0_dot_q8_1_block(W[r,b], X[(4b+iqs)*n_tok+t], iqs) */
void orc_gemm(const uint8_t *W, const uint8_t *X, float *Y, int64_t n_out, int64_t n_in,
              int64_t n_tok, int nthreads) {
    const int64_t nb = n_in / QK_PQ2, stride = nb * PQ2_BYTES;
#ifdef _OPENMP
#pragma omp parallel for schedule(static) num_threads(nthreads > 0 ? nthreads : 1)
#endif
    for (int64_t r = 0; r < n_out; ++r)
        for (int64_t t = 0; t < n_tok; ++t) {
            float acc = 0.0f;
            for (int64_t b = 0; b < nb; ++b)
                for (int iqs = 0; iqs < 4; ++iqs)
                    acc += chunk_dot(W + r * stride + b * PQ2_BYTES,
                                     X + ((b * 4 + iqs) * n_tok + t) * Q81_BYTES, iqs);
            Y[r * n_tok + t] = acc;
        }
    (void)nthreads;
}

/* ---- repacked layout: src/pq2_0_repack.h:46-138 --------------------------
 * row = d[nb] (fp16) | codes: unit u = plane*nb + block at 2*nb + 8u.      */
int orc_repack_rows(const uint8_t *src, uint8_t *dst, int64_t n_out, int64_t n_in) {
    const int64_t nb = n_in / QK_PQ2, stride = nb * PQ2_BYTES;
    if (n_in % QK_PQ2 || nb <= 0 || nb % 8) return 1;
    for (int64_t r = 0; r < n_out; ++r) {
        const uint8_t *s = src + r * stride;
        uint8_t *d = dst + r * stride;
        for (int64_t b = 0; b < nb; ++b) {
            memcpy(d + 2 * b, s + b * PQ2_BYTES, 2);
            for (int p = 0; p < 4; ++p)
                memcpy(d + 2 * nb + (p * nb + b) * 8, s + b * PQ2_BYTES + 2 + p * 8, 8);
        }
    }
    return 0;
}

int orc_unpack_rows(const uint8_t *src, uint8_t *dst, int64_t n_out, int64_t n_in) {
    const int64_t nb = n_in / QK_PQ2, stride = nb * PQ2_BYTES;
    if (n_in % QK_PQ2 || nb <= 0 || nb % 8) return 1;
    for (int64_t r = 0; r < n_out; ++r) {
        const uint8_t *s = src + r * stride;
        uint8_t *d = dst + r * stride;
        for (int64_t b = 0; b < nb; ++b) {
            memcpy(d + b * PQ2_BYTES, s + 2 * b, 2);
            for (int p = 0; p < 4; ++p)
                memcpy(d + b * PQ2_BYTES + 2 + p * 8, s + 2 * nb + (p * nb + b) * 8, 8);
        }
    }
    return 0;
}

/* repack_row_dot, src/pq2_0_repack.h:166-182: units in order u = 0..4nb-1,
 * each (f16(dw) * f16(da)) * sumi, summed sequentially in fp32.            */
float orc_repack_row_dot(const uint8_t *row, const uint8_t *act, int64_t nb) {
    float acc = 0.0f;
    uint8_t blk[PQ2_BYTES];
    for (int64_t u = 0; u < 4 * nb; ++u) {
        const int64_t p = u / nb, b = u % nb;
        memcpy(blk, row + 2 * b, 2);
        memcpy(blk + 2 + p * 8, row + 2 * nb + u * 8, 8);
        const uint8_t *a = act + (b * 4 + p) * Q81_BYTES;
        const float dw = orc_f16_to_f32(ld16(blk)), da = orc_f16_to_f32(ld16(a));
        acc += dw * da * (float)orc_chunk_sumi(blk, a, (int)p);
    }
    return acc;
}

/* bonsai_p40_gemv_repack contract (src/kernels/gemv_repack_p40.cu:209-220):
 * x is fp32, quantised (permuted Q8_1) first, then every row through the
 * repacked layout.  The reference device kernel quantises with RNE; this
 * oracle follows the host quantiser (src/pq2_0.h:99-126).                  */
void orc_gemv_repack(const uint8_t *Wr, const float *x, float *y, int64_t n_out, int64_t n_in,
                     int nthreads) {
    const int64_t nb = n_in / QK_PQ2, stride = nb * PQ2_BYTES;
    uint8_t *act = (uint8_t *)malloc((size_t)(n_in / QK8) * Q81_BYTES);
    orc_quantize_q8_1(x, act, n_in, 1);
#ifdef _OPENMP
#pragma omp parallel for schedule(static) num_threads(nthreads > 0 ? nthreads : 1)
#endif
    for (int64_t r = 0; r < n_out; ++r) y[r] = orc_repack_row_dot(Wr + r * stride, act, nb);
    free(act);
    (void)nthreads;
}

/* ---- SwiGLU: src/ops.h:27-31 (silu(g) = g / (1 + expf(-g))) ----------- */
void orc_swiglu(const float *g, const float *u, float *y, int64_t n) {
    for (int64_t i = 0; i < n; ++i) y[i] = g[i] / (1.0f + expf(-g[i])) * u[i];
}

/* ---- RMSNorm: src/ops.h:13-22 ------------------------------------------
 * s = 1 / sqrtf(ss / n + eps) with ss the sequential fp32 sum of x[i]^2
 * (each square and each addition rounded), then y = (x * s) * w. */
void orc_rmsnorm(const float *x, const float *w, float *y, int64_t n, float eps) {
    float ss = 0.0f;
    for (int64_t i = 0; i < n; ++i) ss += x[i] * x[i];
    const float s = 1.0f / sqrtf(ss / (float)n + eps);
    for (int64_t i = 0; i < n; ++i) y[i] = x[i] * s * w[i];
}

/* ---- seeded synthetic inputs (own generator: splitmix64 + Box-Muller) --- */
static inline uint64_t splitmix64(uint64_t *s) {
    uint64_t z = (*s += 0x9e3779b97f4a7c15ull);
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}
static inline double unif01(uint64_t *s) {           /* (0, 1] */
    return ((double)(splitmix64(s) >> 11) + 1.0) * (1.0 / 9007199254740992.0);
}

void orc_gen_normal(uint64_t seed, float *x, int64_t n, float sigma) {
    uint64_t s = seed;
    for (int64_t i = 0; i < n; i += 2) {
        const double r = sqrt(-2.0 * log(unif01(&s))), th = 6.283185307179586 * unif01(&s);
        x[i] = (float)(sigma * r * cos(th));
        if (i + 1 < n) x[i + 1] = (float)(sigma * r * sin(th));
    }
}

/* PQ2_0 weights of the benchmark configs: per block d = f16(|N(0,0.02)| + 1e-4)
 * (host encode), codes i.i.d. with P(3) = p3 and P(0)=P(1)=P(2)=(1-p3)/3.    */
void orc_gen_weights(uint64_t seed, uint8_t *W, int64_t n_out, int64_t n_in, double p3) {
    uint64_t s = seed;
    const int64_t nblk = n_out * (n_in / QK_PQ2);
    for (int64_t b = 0; b < nblk; ++b) {
        uint8_t *blk = W + b * PQ2_BYTES;
        const double r = sqrt(-2.0 * log(unif01(&s))), th = 6.283185307179586 * unif01(&s);
        const float d = (float)fabs(0.02 * r * cos(th)) + 1e-4f;
        st16(blk, orc_f32_to_f16(d));
        for (int j = 0; j < 32; ++j) {
            uint8_t byte = 0;
            for (int e = 0; e < 4; ++e) {
                const double u = unif01(&s);
                int code = 3;
                if (u > p3) {
                    code = (int)((u - p3) / ((1.0 - p3) / 3.0));
                    if (code > 2) code = 2;
                }
                byte |= (uint8_t)(code << (2 * e));
            }
            blk[2 + j] = byte;
        }
    }
}
