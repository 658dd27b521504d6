// bonsai_p40_ggml.h -- the llama.cpp (ggml-hip) hook of the PQ2_0 decode path:
// the gfx950 counterparts of the reference fork's bonsai_p40_should_use and
// bonsai_p40_mul_mat (integrations/prismml/bonsai-p40.diff:245-302), which
// ggml_cuda_mul_mat calls before its stock MMVQ branch (diff:1059-1062).
//
// A ggml_tensor is passed as the handful of its fields the hook reads
// (bonsai_ggml_tensor below: type, ne[4], nb[4], data, as in ggml.h), so the
// library needs no ggml headers; the fork fills the view by copying those
// fields from its ggml_tensor.  C++ header (it includes bonsai_p40.h).
#pragma once

#include "bonsai_p40.h"
#include "bonsai_p40_dispatch.h"

#ifdef __cplusplus
extern "C" {
#endif

// The fields of a ggml_tensor the hook reads.
typedef struct bonsai_ggml_tensor {
    int type;            // enum ggml_type (BONSAI_GGML_TYPE_PQ2_0 = 142, BONSAI_GGML_TYPE_F32 = 0)
    int64_t ne[4];       // elements per dimension
    size_t nb[4];        // bytes per step in each dimension
    void * data;         // device pointer
} bonsai_ggml_tensor;

// Replaces bonsai_p40_should_use (bonsai-p40.diff:245-248): 1 when the path is
// switched on (environment BONSAI_P40=1, read once per process; off by
// default, as in the reference), src0 is PQ2_0, HIP device `device` is a
// gfx950 (the reference tests compute capability 610), and the product has
// one activation column (ne11 == 1); else 0.
int bonsai_p40_ggml_should_use(int src0_type, int device, int64_t ne11);

// Replaces bonsai_p40_mul_mat (bonsai-p40.diff:250-302): dst = src0 . src1
// for a PQ2_0 weight matrix src0 [ne1 = n_out][ne0 = n_in] and an F32 column
// src1 [n_in], enqueued on `stream`; returns 1 when enqueued and 0 when the
// caller must take its stock path: a shape outside the reference's decode
// predicate (bonsai_decode_path_ok, src/p40_dispatch_predicate.h:33-47), a
// width without the one-launch kernel and no scratch, or a launch error.
// n_in % 1024 == 0 (every width of the model) runs as ONE launch with no
// scratch (bonsai_p40_quant_gemv); other widths run the reference's two
// launches (bonsai_p40_quant_activations, bonsai_p40_gemv) through
// q8_scratch, a device buffer of at least n_in / 32 * 36 bytes, 4-byte
// aligned, owned by the caller (the reference hook keeps a lazily allocated
// global, diff:275-281; the library allocates nothing).  With
// BONSAI_P40_VERBOSE set, the first call that takes an op prints one line.
int bonsai_p40_ggml_mul_mat(const bonsai_ggml_tensor * src0, const bonsai_ggml_tensor * src1,
                            const bonsai_ggml_tensor * dst, void * q8_scratch, size_t scratch_bytes,
                            bonsai_stream stream);

#ifdef __cplusplus
}
#endif
