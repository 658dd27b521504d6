// C++ host using the library exactly as a reference host would: include
// include/bonsai_p40.h, link libbonsai_p40.so, pass device pointers and a
// stream.  The reference's standalone runner (docs/INTEGRATION.md:257-263)
// is the model.
//
//   example_decode --args-only   argument checks only (no device is touched)
//   example_decode               one decode layer input on the GPU: RMSNorm +
//                                FWHT + Q8_1 then a GEMV, against the same
//                                through the fused single-launch entry point
//                                (bit-identical by contract)
#include "../../include/bonsai_p40.h"

#include <hip/hip_runtime_api.h>

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <vector>

namespace {

int failures = 0;

void check(bool ok, const char * what) {
    if (!ok) {
        ++failures;
        std::printf("FAIL: %s\n", what);
    }
}

int args_only() {
    // invalid arguments return 1, empty work returns 0, nothing is launched
    check(bonsai_p40_gemv(nullptr, nullptr, nullptr, 16, 100, nullptr) == 1, "gemv n_in % 128");
    check(bonsai_p40_gemv(nullptr, nullptr, nullptr, 0, 128, nullptr) == 0, "gemv empty");
    check(bonsai_p40_gemm(nullptr, nullptr, nullptr, 16, 100, 4, nullptr) == 1, "gemm n_in % 128");
    check(bonsai_p40_fwht(nullptr, nullptr, 1000, nullptr) == 1, "fwht n % 1024");
    check(bonsai_p40_quant_activations(nullptr, nullptr, 33, nullptr) == 1, "quant n % 32");
    check(bonsai_p40_repack(nullptr, nullptr, 4, 1024 + 128, nullptr) == 1, "repack nb % 8");
    float dummy = 0.0f;
    check(bonsai_p40_rmsnorm_fwht_quant(&dummy, nullptr, nullptr, &dummy, 1024, 1, 1e-6f, nullptr) == 1,
          "rmsnorm_fwht_quant without weights");
    check(bonsai_p40_gdn_step(nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, 1, 1, 1, 1,
                              nullptr) == 2, "gdn_step out of scope");
    std::printf("args-only: %d failed\n", failures);
    return failures == 0 ? 0 : 1;
}

// splitmix64 for reproducible host data
uint64_t mix(uint64_t & s) {
    uint64_t z = (s += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

#define HIP_OK(call)                                                                  \
    do {                                                                              \
        if ((call) != hipSuccess) {                                                   \
            std::printf("HIP error in %s\n", #call);                                  \
            return 1;                                                                 \
        }                                                                             \
    } while (0)

int on_device() {
    const int64_t n_out = 4096, n_in = 5120;
    const int64_t nb = n_in / 128, w_bytes = n_out * nb * 34, q_bytes = n_in / 32 * 36;
    uint64_t seed = 2024;
    std::vector<uint8_t> W(w_bytes);
    for (int64_t b = 0; b < n_out * nb; ++b) {
        uint8_t * blk = &W[b * 34];
        const uint16_t d = (uint16_t)(0x2000 + mix(seed) % 0x0800);    // fp16 in about [0.008, 0.03)
        std::memcpy(blk, &d, 2);
        for (int k = 0; k < 32; ++k) {
            uint8_t v = 0;
            for (int j = 0; j < 4; ++j) v |= (uint8_t)((mix(seed) % 3) << (2 * j));   // ternary codes
            blk[2 + k] = v;
        }
    }
    std::vector<float> x(n_in), w(n_in);
    for (int64_t i = 0; i < n_in; ++i) {
        x[i] = (float)((int64_t)(mix(seed) % 2001) - 1000) * 0.003f;
        w[i] = 1.0f + (float)((int64_t)(mix(seed) % 201) - 100) * 0.001f;
    }

    void *dW, *dq;
    float *dx, *dw, *dy1, *dy2;
    HIP_OK(hipMalloc(&dW, w_bytes));
    HIP_OK(hipMalloc(&dq, q_bytes));
    HIP_OK(hipMalloc(&dx, n_in * 4));
    HIP_OK(hipMalloc(&dw, n_in * 4));
    HIP_OK(hipMalloc(&dy1, n_out * 4));
    HIP_OK(hipMalloc(&dy2, n_out * 4));
    HIP_OK(hipMemcpy(dW, W.data(), w_bytes, hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(dx, x.data(), n_in * 4, hipMemcpyHostToDevice));
    HIP_OK(hipMemcpy(dw, w.data(), n_in * 4, hipMemcpyHostToDevice));
    hipStream_t st;
    HIP_OK(hipStreamCreate(&st));

    // two launches: layer-input pre-pass, then the GEMV
    check(bonsai_p40_rmsnorm_fwht_quant(dx, dw, nullptr, dq, n_in, 1, 1e-6f, st) == 0, "pre-pass enqueued");
    check(bonsai_p40_gemv(dW, dq, dy1, n_out, n_in, st) == 0, "gemv enqueued");
    // one launch: the same through the grouped entry point with one matrix
    const void * Ws[1] = {dW};
    float * ys[1] = {dy2};
    const int64_t rows[1] = {n_out};
    check(bonsai_p40_rmsnorm_fwht_gemv_group(Ws, ys, rows, 1, dx, dw, nullptr, n_in, 1e-6f, st) == 0,
          "fused enqueued");
    HIP_OK(hipStreamSynchronize(st));

    std::vector<float> y1(n_out), y2(n_out);
    HIP_OK(hipMemcpy(y1.data(), dy1, n_out * 4, hipMemcpyDeviceToHost));
    HIP_OK(hipMemcpy(y2.data(), dy2, n_out * 4, hipMemcpyDeviceToHost));
    int finite = 0;
    double amax = 0.0;
    for (int64_t r = 0; r < n_out; ++r) {
        finite += std::isfinite(y1[r]) ? 1 : 0;
        amax = std::fmax(amax, std::fabs((double)y1[r]));
    }
    check(finite == n_out, "finite outputs");
    check(amax > 0.0, "non-zero outputs");
    check(std::memcmp(y1.data(), y2.data(), n_out * 4) == 0, "fused == two launches, bit for bit");

    HIP_OK(hipStreamDestroy(st));
    HIP_OK(hipFree(dW));
    HIP_OK(hipFree(dq));
    HIP_OK(hipFree(dx));
    HIP_OK(hipFree(dw));
    HIP_OK(hipFree(dy1));
    HIP_OK(hipFree(dy2));
    std::printf("device: %d failed (max |y| %.4g)\n", failures, amax);
    return failures == 0 ? 0 : 1;
}

}  // namespace

int main(int argc, char ** argv) {
    if (argc > 1 && std::strcmp(argv[1], "--args-only") == 0) return args_only();
    return on_device();
}
