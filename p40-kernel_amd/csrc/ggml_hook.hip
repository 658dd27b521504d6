// ggml_hook.hip -- the ggml-hip hook of the PQ2_0 decode path (host code only):
// the gfx950 counterparts of the reference fork's bonsai_p40_should_use and
// bonsai_p40_mul_mat (integrations/prismml/bonsai-p40.diff:245-302).
//
// The decision is the reference's: an opt-in switch (BONSAI_P40=1), the
// device (gfx950 here, compute capability 610 there), PQ2_0 x F32 -> F32 with
// one activation column, and the shape predicate of
// src/p40_dispatch_predicate.h:33-47 (include/bonsai_p40_dispatch.h).  The
// work differs: the model's widths (n_in % 1024 == 0) run as one launch that
// quantises the activation inside the GEMV (no Q8_1 scratch, no second
// dependent launch); other widths run the reference's two launches through
// the caller's scratch.
#include "host_state.h"
#include "../../include/bonsai_p40_ggml.h"

#include <atomic>
#include <cstdio>
#include <cstring>
#include <mutex>

namespace {

// whether HIP device `dev` is a gfx950, asked once per device
bool device_is_gfx950(int dev) {
    if (dev < 0 || dev >= pq2host::MAX_DEVICES) return false;
    static std::once_flag once[pq2host::MAX_DEVICES];
    static bool is950[pq2host::MAX_DEVICES];
    std::call_once(once[dev], [dev] {
        hipDeviceProp_t p;
        if (hipGetDeviceProperties(&p, dev) == hipSuccess) {
            is950[dev] = std::strncmp(p.gcnArchName, "gfx950", 6) == 0;
        } else {
            (void)hipGetLastError();
            is950[dev] = false;
        }
    });
    return is950[dev];
}

}  // namespace

extern "C" {

int bonsai_p40_ggml_should_use(int src0_type, int device, int64_t ne11) {
    if (pq2host::knob(pq2host::K_GGML_ENABLE, 0) != 1) return 0;
    if (src0_type != BONSAI_GGML_TYPE_PQ2_0 || ne11 != 1) return 0;
    return device_is_gfx950(device) ? 1 : 0;
}

int bonsai_p40_ggml_mul_mat(const bonsai_ggml_tensor * src0, const bonsai_ggml_tensor * src1,
                            const bonsai_ggml_tensor * dst, void * q8_scratch, size_t scratch_bytes,
                            bonsai_stream stream) {
    if (src0 == nullptr || src1 == nullptr || dst == nullptr) return 0;
    bonsai_mulmat_shape s;
    s.type0 = src0->type;
    s.type1 = src1->type;
    s.type2 = dst->type;
    s.n_in = src0->ne[0];
    s.n_out = src0->ne[1];
    s.ne20 = src0->ne[2];
    s.ne30 = src0->ne[3];
    s.ne11 = src1->ne[1];
    s.ne12 = src1->ne[2];
    s.ne13 = src1->ne[3];
    s.dst_ne1 = dst->ne[1];
    s.nb1 = (int64_t)src0->nb[1];
    if (!bonsai_decode_path_ok(&s)) return 0;
    if (src0->data == nullptr || src1->data == nullptr || dst->data == nullptr) return 0;
    const int64_t n_in = s.n_in, n_out = s.n_out;
    const float * x = static_cast<const float *>(src1->data);
    float * y = static_cast<float *>(dst->data);
    int rc;
    if (n_in % 1024 == 0) {
        rc = bonsai_p40_quant_gemv(src0->data, x, y, n_out, n_in, stream);
    } else {
        if (q8_scratch == nullptr || scratch_bytes < (size_t)(n_in / 32) * 36) return 0;
        rc = bonsai_p40_quant_activations(x, q8_scratch, n_in, stream);
        if (rc == 0) rc = bonsai_p40_gemv(src0->data, q8_scratch, y, n_out, n_in, stream);
    }
    if (rc != 0) return 0;
    if (pq2host::knob(pq2host::K_GGML_VERBOSE, 0) != 0) {
        static std::atomic<bool> reported{false};
        if (!reported.exchange(true))
            std::fprintf(stderr, "bonsai-p40: gfx950 PQ2_0 decode path active (n_in=%lld n_out=%lld)\n",
                         (long long)n_in, (long long)n_out);
    }
    return 1;
}

}  // extern "C"
