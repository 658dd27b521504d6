// bwprobe.hip -- HBM streaming-read ceiling probe (the analog of the
// reference's tools/bwtest.cu read_kernel, tools/bwtest.cu:37-47): every
// lane reads 16-byte vectors grid-stride and folds them with XOR, one word
// per workgroup is written so the loads cannot be elided.  Used by bench.py to
// report "% of achievable" next to "% of peak".
#include "pq2_device.h"
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

}  // namespace

extern "C" int bonsai_p40_stream_read(const void * buf, int64_t bytes, uint32_t * out, int blocks,
                                      bonsai_stream stream) {
    if (bytes <= 0 || bytes % 16 != 0 || ((uintptr_t)buf & 15u) != 0 || blocks <= 0) return 1;
    hipLaunchKernelGGL(stream_read_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream,
                       (const v4u *)buf, (size_t)bytes / 16, out);
    return (int)hipGetLastError();
}
