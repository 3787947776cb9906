// Read-ceiling kernel: streams a buffer with plain 16-byte non-temporal
// loads and keeps nothing but a conditional one-word store (so the loads
// cannot be dropped).  bench.py times it over the same bytes as a decode
// step: the fastest one launch can read them on this device, which bounds
// any single-launch decode from below.
#include "ss_common.hpp"

namespace ss {

typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));

// Each thread keeps 4 loads in flight per iteration over a grid-stride
// range; every address is below n16 16-byte units.
__global__ void __launch_bounds__(256) stream_read_kernel(const u32x4_t *p, int64_t n16,
                                                          uint32_t *sink) {
    constexpr int U = 4;
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    uint32_t acc = 0;
    for (; i + (U - 1) * stride < n16; i += U * stride) {
        u32x4_t v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) v[u] = __builtin_nontemporal_load(p + i + u * stride);
#pragma unroll
        for (int u = 0; u < U; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
    for (; i < n16; i += stride) {
        const u32x4_t v = __builtin_nontemporal_load(p + i);
        acc ^= v.x ^ v.y ^ v.z ^ v.w;
    }
    // never true for the buffers bench.py streams; keeps the loads live
    if (acc == 0x9e3779b9u && sink) sink[0] = acc;
}

}  // namespace ss

using namespace ss;

extern "C" int ss_stream_read(const void *buf, int64_t bytes, int n_workgroups, uint32_t *sink,
                              void *stream) {
    SS_REQUIRE(buf && sink, "null pointer argument");
    SS_REQUIRE(bytes >= 16 && bytes % 16 == 0, "bytes must be a positive multiple of 16");
    SS_REQUIRE(((uintptr_t)buf % 16) == 0, "buffer must be 16-byte aligned");
    SS_REQUIRE(n_workgroups >= 1 && n_workgroups <= 65536, "n_workgroups out of range");
    hipLaunchKernelGGL(stream_read_kernel, dim3(n_workgroups), dim3(256), 0,
                       reinterpret_cast<hipStream_t>(stream),
                       static_cast<const u32x4_t *>(buf), bytes / 16, sink);
    SS_LAUNCH_CHECK("stream_read_kernel launch");
    return SS_OK;
}
