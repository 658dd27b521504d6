// other.hip -- entry points of the reference header that are not on the PQ2_0
// matmul path, kept so a host written against include/bonsai_p40.h links.
//   * bonsai_p40_rmsnorm: per-row RMSNorm, y = x * (1/sqrt(mean(x^2)+eps)) * w
//     (src/ops.h:13-22; the reference device kernel is elementwise_p40.cu:48-88);
//   * bonsai_p40_gdn_step / bonsai_p40_attn: outside this library's scope,
//     they return 2 without touching memory;
// plus bonsai_p40_reload_tuning, which re-reads the library's BONSAI_* tuning
// variables (read once per process otherwise).
#include "pq2_device.h"
#include "host_state.h"
#include "../../include/bonsai_p40.h"

using namespace pq2;

namespace {

__global__ void __launch_bounds__(256)
rmsnorm_kernel(const float * __restrict__ x, const float * __restrict__ w, float * __restrict__ y,
               int n, float eps) {
    __shared__ float red[4];
    const size_t row = blockIdx.x;
    const float * xr = x + row * n;
    float ss = 0.0f;
    for (int i = threadIdx.x; i < n; i += 256) ss += xr[i] * xr[i];
    ss = wave_sum_to_lane63(ss);
    if ((threadIdx.x & 63) == 63) red[threadIdx.x >> 6] = ss;
    __syncthreads();
    const float tot = red[0] + red[1] + red[2] + red[3];
    const float s = 1.0f / sqrtf(tot / (float)n + eps);
    for (int i = threadIdx.x; i < n; i += 256) y[row * n + i] = xr[i] * s * w[i];
}

}  // namespace

extern "C" {

int bonsai_p40_rmsnorm(const float * x, const float * w, float * y, int64_t n_rows, int64_t n,
                       float eps, bonsai_stream stream) {
    if (n <= 0 || n > 0x7fffffff) return 1;
    if (n_rows <= 0) return 0;
    if (n_rows > 0x7fffffff || pq2host::any_null(x, w, y)) return 1;
    hipLaunchKernelGGL(rmsnorm_kernel, dim3((unsigned)n_rows), dim3(256), 0, (hipStream_t)stream,
                       x, w, y, (int)n, eps);
    return (int)hipGetLastError();
}

int bonsai_p40_gdn_step(float *, const float *, const float *, const float *, const float *,
                        const float *, float *, int, int, int, int, bonsai_stream) {
    return 2;
}

int bonsai_p40_attn(const float *, const float *, const float *, float *, int, int, int, int, float,
                    bonsai_stream) {
    return 2;
}

}  // extern "C"

extern "C" int bonsai_p40_reload_tuning(void) {
    pq2host::reload_knobs();
    return 0;
}
