// The few lines a llama.cpp (ggml-hip) fork adds around the library's hook
// (include/bonsai_p40_ggml.h), compiled as plain C++ against a tensor struct
// with ggml.h's field names and types for what the glue reads -- the fork
// compiles the same glue against ggml.h itself.  The reference's glue is
// integrations/prismml/bonsai-p40.diff:1059-1062 (the call in
// ggml_cuda_mul_mat) with the hook at diff:245-302.
//
//   ggml_glue --args-only   decisions made before any device work
//   ggml_glue               one 17408x5120 op on the GPU through the glue,
//                           bit-identical to quant_activations + gemv
#include "../../include/bonsai_p40_ggml.h"

#include <hip/hip_runtime_api.h>

#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

// ---- the ggml side (ggml.h field names; only what the glue reads) ----------
enum ggml_type { GGML_TYPE_F32 = 0, GGML_TYPE_F16 = 1, GGML_TYPE_PQ2_0 = 142 };
struct ggml_tensor {
    enum ggml_type type;
    int64_t ne[4];
    size_t nb[4];
    void * data;
};

// ---- the glue a fork adds to ggml-cuda.cu -----------------------------------
static bonsai_ggml_tensor bonsai_view(const ggml_tensor * t) {
    bonsai_ggml_tensor v;
    v.type = (int)t->type;
    for (int i = 0; i < 4; ++i) {
        v.ne[i] = t->ne[i];
        v.nb[i] = t->nb[i];
    }
    v.data = t->data;
    return v;
}

// in ggml_cuda_mul_mat, before the stock MMVQ branch (device = ctx.device,
// stream = ctx.stream(), scratch from ctx.pool())
static bool bonsai_try_mul_mat(int device, const ggml_tensor * src0, const ggml_tensor * src1,
                               ggml_tensor * dst, void * scratch, size_t scratch_bytes, hipStream_t stream) {
    if (!bonsai_p40_ggml_should_use((int)src0->type, device, src1->ne[1])) return false;
    const bonsai_ggml_tensor a = bonsai_view(src0), b = bonsai_view(src1), d = bonsai_view(dst);
    return bonsai_p40_ggml_mul_mat(&a, &b, &d, scratch, scratch_bytes, (bonsai_stream)stream) == 1;
}

// ---- the test ---------------------------------------------------------------
namespace {

int failures = 0;
void check(bool ok, const char * what) {
    if (!ok) {
        ++failures;
        std::printf("FAIL: %s\n", what);
    }
}

ggml_tensor make(ggml_type t, int64_t ne0, int64_t ne1, size_t nb0, size_t nb1, void * data) {
    ggml_tensor x;
    x.type = t;
    x.ne[0] = ne0; x.ne[1] = ne1; x.ne[2] = 1; x.ne[3] = 1;
    x.nb[0] = nb0; x.nb[1] = nb1; x.nb[2] = nb1 * (size_t)ne1; x.nb[3] = x.nb[2];
    x.data = data;
    return x;
}

int args_only() {
    // BONSAI_P40 is not set by the test harness: the path is off
    ggml_tensor w = make(GGML_TYPE_PQ2_0, 5120, 17408, 34, 40 * 34, nullptr);
    ggml_tensor x = make(GGML_TYPE_F32, 5120, 1, 4, 5120 * 4, nullptr);
    ggml_tensor y = make(GGML_TYPE_F32, 17408, 1, 4, 17408 * 4, nullptr);
    check(!bonsai_try_mul_mat(0, &w, &x, &y, nullptr, 0, nullptr), "off unless BONSAI_P40=1");
    // the hook itself declines shapes outside the predicate before touching data
    bonsai_ggml_tensor a = bonsai_view(&w), b = bonsai_view(&x), d = bonsai_view(&y);
    b.ne[1] = 4;
    check(bonsai_p40_ggml_mul_mat(&a, &b, &d, nullptr, 0, nullptr) == 0, "declines a batch");
    b = bonsai_view(&x);
    a.type = GGML_TYPE_F16;
    check(bonsai_p40_ggml_mul_mat(&a, &b, &d, nullptr, 0, nullptr) == 0, "declines F16 weights");
    a = bonsai_view(&w);
    a.nb[1] = 4096;
    check(bonsai_p40_ggml_mul_mat(&a, &b, &d, nullptr, 0, nullptr) == 0, "declines strided rows");
    a = bonsai_view(&w);
    check(bonsai_p40_ggml_mul_mat(&a, &b, &d, nullptr, 0, nullptr) == 0, "declines null data");
    std::printf("args-only: %d failed\n", failures);
    return failures == 0 ? 0 : 1;
}

#define HIP_OK(call)                                                    \
    do {                                                                \
        if ((call) != hipSuccess) {                                     \
            std::printf("HIP error in %s\n", #call);                    \
            return 1;                                                   \
        }                                                               \
    } while (0)

int on_device() {
    const int64_t n_out = 17408, n_in = 5120;
    const size_t wb = (size_t)n_out * (n_in / 128) * 34;
    std::vector<uint8_t> hw(wb);
    std::vector<float> hx(n_in);
    uint64_t s = 0x5eed;
    auto next = [&s] {
        s ^= s << 13; s ^= s >> 7; s ^= s << 17;
        return s;
    };
    for (size_t i = 0; i < wb; i += 34) {
        const uint16_t d = 0x2000 + (uint16_t)(next() % 0x800);   // fp16 in [2^-7, 2^-6)
        std::memcpy(&hw[i], &d, 2);
        for (int k = 2; k < 34; ++k) hw[i + k] = (uint8_t)next();
    }
    for (int64_t i = 0; i < n_in; ++i) hx[i] = (float)((int64_t)(next() % 2001) - 1000) / 250.0f;
    void *W, *X, *Y1, *Y2, *XQ;
    HIP_OK(hipMalloc(&W, wb));
    HIP_OK(hipMalloc(&X, n_in * 4));
    HIP_OK(hipMalloc(&Y1, n_out * 4));
    HIP_OK(hipMalloc(&Y2, n_out * 4));
    HIP_OK(hipMalloc(&XQ, n_in / 32 * 36));
    HIP_OK(hipMemcpy(W, hw.data(), wb, hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(X, hx.data(), n_in * 4, hipMemcpyHostToDevice));
    hipStream_t st;
    HIP_OK(hipStreamCreate(&st));
    int dev = 0;
    HIP_OK(hipGetDevice(&dev));
    ggml_tensor w = make(GGML_TYPE_PQ2_0, n_in, n_out, 34, (size_t)(n_in / 128) * 34, W);
    ggml_tensor x = make(GGML_TYPE_F32, n_in, 1, 4, (size_t)n_in * 4, X);
    ggml_tensor y = make(GGML_TYPE_F32, n_out, 1, 4, (size_t)n_out * 4, Y1);
    check(bonsai_try_mul_mat(dev, &w, &x, &y, nullptr, 0, st), "takes the op on gfx950 with BONSAI_P40=1");
    check(bonsai_p40_quant_activations((const float *)X, XQ, n_in, st) == 0, "quant_activations");
    check(bonsai_p40_gemv(W, XQ, (float *)Y2, n_out, n_in, st) == 0, "gemv");
    HIP_OK(hipStreamSynchronize(st));
    std::vector<uint32_t> a(n_out), b(n_out);
    HIP_OK(hipMemcpy(a.data(), Y1, n_out * 4, hipMemcpyDeviceToHost));
    HIP_OK(hipMemcpy(b.data(), Y2, n_out * 4, hipMemcpyDeviceToHost));
    check(a == b, "one launch == quant_activations + gemv, bit for bit");
    HIP_OK(hipStreamDestroy(st));
    HIP_OK(hipFree(W)); HIP_OK(hipFree(X)); HIP_OK(hipFree(Y1)); HIP_OK(hipFree(Y2)); HIP_OK(hipFree(XQ));
    std::printf("device: %d failed\n", failures);
    return failures == 0 ? 0 : 1;
}

}  // namespace

int main(int argc, char ** argv) {
    if (argc > 1 && std::strcmp(argv[1], "--args-only") == 0) return args_only();
    return on_device();
}
