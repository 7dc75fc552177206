// m27q_stream.hip -- the plain streaming read the benchmark reports as the
// measured HBM read peak (libm27q_stream.so; not part of the product ABI).
//
// Each workgroup of 256 threads reads one 16 KiB chunk of the buffer: four
// independent 16-byte loads per thread, issued before any is consumed, then a
// sum that is stored only when it equals a value a zero-filled buffer cannot
// give (so the loads stay live).  Of the shapes measured on MI355X (grid-stride
// with 4 / 8 / 16 workgroups per CU and 8 loads in flight per thread,
// contiguous chunks per workgroup, one chunk per workgroup), this one was at or
// near the best at every size from 17.8 MB to 1 GB.
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace {

typedef float f4 __attribute__((ext_vector_type(4)));
constexpr int kThreads = 256, kLoads = 4;
constexpr size_t kChunk = (size_t)kThreads * kLoads * 16;  // 16 KiB

__global__ __launch_bounds__(kThreads) void k_stream_read(const f4 *__restrict__ p, size_t n4, float *sink) {
    const size_t base = (size_t)blockIdx.x * (kChunk / 16) + threadIdx.x;
    f4 v[kLoads];
#pragma unroll
    for (int u = 0; u < kLoads; ++u) {
        const size_t i = base + (size_t)u * kThreads;
        v[u] = i < n4 ? __builtin_nontemporal_load(p + i) : f4{0.f, 0.f, 0.f, 0.f};
    }
    f4 acc = v[0];
#pragma unroll
    for (int u = 1; u < kLoads; ++u) acc += v[u];
    const float s = acc.x + acc.y + acc.z + acc.w;
    if (s == 1234.5f) sink[blockIdx.x] = s;
}

}  // namespace

// Reads bytes (a multiple of 16, 16-byte aligned) of device memory; sink is a
// device float array of at least ceil(bytes / 16 KiB) entries that is never
// written for a zero-filled buffer.  Returns a hipError_t.
extern "C" __attribute__((visibility("default"))) int m27q_stream_read(const void *buf, size_t bytes, float *sink,
                                                                        hipStream_t stream) {
    if (!buf || !sink || bytes % 16 || (uintptr_t)buf % 16) return (int)hipErrorInvalidValue;
    const size_t grid = (bytes + kChunk - 1) / kChunk;
    if (grid == 0 || grid > 0x7fffffff) return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(k_stream_read, dim3((unsigned)grid), dim3(kThreads), 0, stream, (const f4 *)buf, bytes / 16, sink);
    return (int)hipGetLastError();
}
