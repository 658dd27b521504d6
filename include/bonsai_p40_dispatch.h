// bonsai_p40_dispatch.h -- caller-side shape contract for handing a ggml
// MUL_MAT to bonsai_p40_gemv (header-only, C and C++).
//
// Same decision as the reference predicate src/p40_dispatch_predicate.h:33-47
// (exercised by tests/test_p40.cpp:653-698): PQ2_0 weights x F32 activations
// -> F32, plain 2-D, one output column, n_in a positive multiple of 128 no
// wider than the 32768 the caller sizes its Q8_1 scratch for, and rows that
// are one contiguous run of 34-byte blocks.  On this library every such shape
// runs; shapes with n_in % 1024 == 0 and 16-byte aligned weights take the
// streaming fast path.
#pragma once

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { BONSAI_GGML_TYPE_F32 = 0, BONSAI_GGML_TYPE_PQ2_0 = 142 };
enum { BONSAI_QK_PQ2_0 = 128, BONSAI_PQ2_0_BLOCK_BYTES = 34, BONSAI_MAX_ROW = 32768 };

// The numbers the predicate needs, as a ggml hook reads them off the tensors.
typedef struct bonsai_mulmat_shape {
    int type0, type1, type2;       // src0, src1, dst ggml types
    int64_t n_in, n_out;           // src0->ne[0], src0->ne[1]
    int64_t ne20, ne30;            // src0->ne[2], src0->ne[3]
    int64_t ne11, ne12, ne13;      // src1->ne[1..3]
    int64_t dst_ne1;               // dst->ne[1]
    int64_t nb1;                   // src0->nb[1], bytes per weight row
} bonsai_mulmat_shape;

static inline int bonsai_decode_path_ok(const bonsai_mulmat_shape * s) {
    if (s->type0 != BONSAI_GGML_TYPE_PQ2_0) return 0;
    if (s->type1 != BONSAI_GGML_TYPE_F32 || s->type2 != BONSAI_GGML_TYPE_F32) return 0;
    if (s->ne20 != 1 || s->ne30 != 1) return 0;                        // 2-D weights only
    if (s->ne11 != 1 || s->ne12 != 1 || s->ne13 != 1 || s->dst_ne1 != 1) return 0;   // decode
    if (s->n_in <= 0 || s->n_out <= 0) return 0;
    if (s->n_in % BONSAI_QK_PQ2_0 != 0 || s->n_in > BONSAI_MAX_ROW) return 0;
    return s->nb1 == (s->n_in / BONSAI_QK_PQ2_0) * BONSAI_PQ2_0_BLOCK_BYTES;   // contiguous rows
}

#ifdef __cplusplus
}
#endif
