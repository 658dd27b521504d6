// ref_shim.cpp -- a C ABI over the reference's own host headers, so tests can
// run the reference arithmetic itself (src/pq2_0.h, src/fwht.h,
// src/pq2_0_repack.h, src/ops.h under /root/reference) and compare it with the
// restatement in pq2_oracle.c.  TEST INFRASTRUCTURE ONLY: built by
// oracle/Makefile into oracle/_ref/ (git-ignored); the reference sources are
// compiled where they lie and never copied.
#include "pq2_0.h"
#include "fwht.h"
#include "pq2_0_repack.h"
#include "ops.h"

#include <cstring>

using namespace bonsai;

extern "C" {

uint16_t ref_f32_to_f16(float f) { return f32_to_f16(f); }
float ref_f16_to_f32(uint16_t h) { return f16_to_f32(h); }

uint64_t ref_f16_encode_hash(uint64_t start, uint64_t count, uint64_t stride) {
    uint64_t h = 1469598103934665603ull;
    for (uint64_t i = 0; i < count; ++i) {
        uint32_t bits = (uint32_t)(start + i * stride);
        float f; std::memcpy(&f, &bits, 4);
        h = (h ^ f32_to_f16(f)) * 1099511628211ull;
    }
    return h;
}

void ref_quantize_q8_1(const float * x, void * y, int64_t k, int permute) {
    quantize_row_q8_1(x, (block_q8_1 *)y, k, permute != 0);
}

void ref_fwht_blocks(float * x, const float * signs, int64_t n) { fwht_blocks(x, signs, (int)n); }

void ref_quantize_pq2_0(const float * x, void * w, int64_t k) { quantize_row_pq2_0(x, (block_pq2_0 *)w, k); }
void ref_dequantize_pq2_0(const void * w, float * y, int64_t k) { dequantize_row_pq2_0((const block_pq2_0 *)w, y, k); }
float ref_pq2_0_dot_f32(const void * w, const float * a) {
    block_pq2_0 b; std::memcpy(&b, w, sizeof b);
    return pq2_0_dot_f32(&b, a);
}

// int32 chunk dot through the reference's own pq2_0_dot_q8_1_block: with both
// scales forced to fp16 1.0 the returned float is exactly (float)sumi
// (|sumi| <= 16256 < 2^24).
int32_t ref_chunk_sumi(const void * wblock, const void * ablock, int iqs) {
    block_pq2_0 w; block_q8_1 a;
    std::memcpy(&w, wblock, sizeof w); std::memcpy(&a, ablock, sizeof a);
    w.d = 0x3C00; a.d = 0x3C00;
    return (int32_t)pq2_0_dot_q8_1_block(&w, &a, iqs);
}

float ref_row_dot(const void * w, const void * a, int64_t n) {
    return pq2_0_row_dot_perm((const block_pq2_0 *)w, (const block_q8_1 *)a, (int)n);
}

void ref_gemv(const void * W, const void * xq, float * y, int64_t n_out, int64_t n_in) {
    const int64_t nb = n_in / BONSAI_QK_PQ2_0;
    for (int64_t r = 0; r < n_out; ++r)
        y[r] = pq2_0_row_dot_perm((const block_pq2_0 *)W + r * nb, (const block_q8_1 *)xq, (int)n_in);
}

// The GEMM loop of tests/test_p40.cpp:449-470 over the reference's block dot.
void ref_gemm(const void * W, const void * X, float * Y, int64_t n_out, int64_t n_in, int64_t n_tok) {
    const int64_t nb = n_in / BONSAI_QK_PQ2_0;
    const block_pq2_0 * w = (const block_pq2_0 *)W;
    const block_q8_1 * x = (const block_q8_1 *)X;
    for (int64_t r = 0; r < n_out; ++r)
        for (int64_t t = 0; t < n_tok; ++t) {
            float acc = 0.0f;
            for (int64_t b = 0; b < nb; ++b)
                for (int iqs = 0; iqs < BONSAI_QI_PQ2_0; ++iqs)
                    acc += pq2_0_dot_q8_1_block(w + r * nb + b, x + (b * BONSAI_QI_PQ2_0 + iqs) * n_tok + t, iqs);
            Y[r * n_tok + t] = acc;
        }
}

int ref_repack_rows(const void * src, void * dst, int64_t n_out, int64_t n_in) {
    const int nb = (int)(n_in / 128);
    if (!repack_requires(nb)) return 1;
    for (int64_t r = 0; r < n_out; ++r)
        repack_row_pq2_0((const block_pq2_0 *)src + r * nb, nb, (uint8_t *)dst + r * repack_row_stride(nb));
    return 0;
}

int ref_unpack_rows(const void * src, void * dst, int64_t n_out, int64_t n_in) {
    const int nb = (int)(n_in / 128);
    if (!repack_requires(nb)) return 1;
    for (int64_t r = 0; r < n_out; ++r)
        unpack_row_pq2_0((const uint8_t *)src + r * repack_row_stride(nb), nb, (block_pq2_0 *)dst + r * nb);
    return 0;
}

float ref_repack_row_dot(const void * row, const void * act, int64_t nb) {
    return repack_row_dot((const uint8_t *)row, (const block_q8_1 *)act, (int)nb);
}

void ref_swiglu(const float * g, const float * u, float * y, int64_t n) { swiglu(g, u, y, (int)n); }
void ref_rmsnorm(const float * x, const float * w, float * y, int64_t n, float eps) { rmsnorm(x, w, y, (int)n, eps); }

}  // extern "C"
