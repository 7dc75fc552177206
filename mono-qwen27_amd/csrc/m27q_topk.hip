// m27q_topk.hip -- exact top-k (k <= 64) over a logits vector.
//
// Each candidate becomes a 64-bit key: the float mapped to an order-preserving
// unsigned (with -0.0 folded onto +0.0 and NaN below every number) in the high
// word, the bitwise-inverted index in the low word, so one descending order on
// keys is (value desc, index asc) and all keys are distinct.
//
// Pass 1: each wavefront scans its run of 64-value segments, keeping a sorted
// top-64 in registers (one key per lane).  A segment with no key above the
// current 64th is skipped after one ballot; otherwise it is bitonic-sorted
// across lanes and merged (max against the reversed segment, then a 6-stage
// bitonic merge).  Pass 2: one workgroup merges the per-wave lists the same way.
// Replaces the CPU selection of sample() (src/mono27b_chat.cpp:211-227) and
// k_argmax (exec:211-239).
#include "m27q_internal.h"
#include "m27q_device.h"

namespace m27q {

constexpr int kTopkTargetWaves = 512;

__device__ __forceinline__ uint64_t topk_key(float v, uint32_t idx) {
    uint32_t o = 0u;  // NaN
    if (v == v) {
        const uint32_t b = v == 0.0f ? 0u : __float_as_uint(v);
        o = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    }
    return ((uint64_t)o << 32) | (uint64_t)(~idx);
}

__device__ __forceinline__ uint64_t umax64(uint64_t a, uint64_t b) { return a > b ? a : b; }
__device__ __forceinline__ uint64_t umin64(uint64_t a, uint64_t b) { return a < b ? a : b; }

__device__ __forceinline__ uint64_t shfl64(uint64_t v, int src) {
    const uint32_t lo = (uint32_t)__shfl((int)(uint32_t)v, src, kWave);
    const uint32_t hi = (uint32_t)__shfl((int)(uint32_t)(v >> 32), src, kWave);
    return ((uint64_t)hi << 32) | lo;
}
__device__ __forceinline__ uint64_t shfl_xor64(uint64_t v, int mask) {
    const uint32_t lo = (uint32_t)__shfl_xor((int)(uint32_t)v, mask, kWave);
    const uint32_t hi = (uint32_t)__shfl_xor((int)(uint32_t)(v >> 32), mask, kWave);
    return ((uint64_t)hi << 32) | lo;
}

// Sort one key per lane descending across the 64 lanes.
__device__ __forceinline__ uint64_t wave_sort_desc(uint64_t k, int lane) {
#pragma unroll
    for (int size = 2; size <= kWave; size <<= 1) {
#pragma unroll
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            const uint64_t o = shfl_xor64(k, stride);
            const bool desc = (lane & size) == 0;
            const bool lower = (lane & stride) == 0;
            k = (lower == desc) ? umax64(k, o) : umin64(k, o);
        }
    }
    return k;
}

// top and seg both sorted descending; returns the sorted top-64 of their union.
__device__ __forceinline__ uint64_t wave_merge_desc(uint64_t top, uint64_t seg, int lane) {
    uint64_t c = umax64(top, shfl64(seg, kWave - 1 - lane));
#pragma unroll
    for (int stride = kWave / 2; stride > 0; stride >>= 1) {
        const uint64_t o = shfl_xor64(c, stride);
        c = ((lane & stride) == 0) ? umax64(c, o) : umin64(c, o);
    }
    return c;
}

__global__ __launch_bounds__(256) void k_topk_local(const float *__restrict__ v, int n, int segs, int nwaves,
                                                    uint64_t *__restrict__ out) {
    const int lane = threadIdx.x & 63;
    const int wave = (int)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (wave >= nwaves) return;
    uint64_t top = 0;  // below every real key
    const long long base = (long long)wave * segs * kWave;
    for (int s = 0; s < segs; ++s) {
        const long long i = base + (long long)s * kWave + lane;
        uint64_t k = i < n ? topk_key(v[i], (uint32_t)i) : 0ull;
        const uint64_t thr = shfl64(top, kWave - 1);
        if (__ballot(k > thr) == 0) continue;
        k = wave_sort_desc(k, lane);
        top = wave_merge_desc(top, k, lane);
    }
    out[(size_t)wave * kWave + lane] = top;
}

__global__ __launch_bounds__(1024) void k_topk_merge(const uint64_t *__restrict__ lists, int nlists, int k,
                                                     const float *__restrict__ v, int32_t *__restrict__ idx,
                                                     float *__restrict__ val) {
    __shared__ uint64_t part[16 * kWave];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    uint64_t top = 0;
    for (int l = wave; l < nlists; l += 16) {
        const uint64_t s = lists[(size_t)l * kWave + lane];
        const uint64_t thr = shfl64(top, kWave - 1);
        if (__ballot(s > thr) == 0) continue;
        top = wave_merge_desc(top, s, lane);
    }
    part[wave * kWave + lane] = top;
    __syncthreads();
    if (wave == 0) {
        top = part[lane];
        for (int w = 1; w < 16; ++w) top = wave_merge_desc(top, part[w * kWave + lane], lane);
        if (lane < k) {
            const uint32_t id = ~(uint32_t)top;
            idx[lane] = (int32_t)id;
            val[lane] = v[id];  // the original bits (keeps -0.0 and NaN payloads)
        }
    }
}

static void topk_plan(int n, int &segs, int &nwaves) {
    const int nseg = (n + kWave - 1) / kWave;
    segs = (nseg + kTopkTargetWaves - 1) / kTopkTargetWaves;
    if (segs < 1) segs = 1;
    nwaves = (nseg + segs - 1) / segs;
}

size_t topk_scratch_bytes(int n) {
    int segs, nwaves;
    topk_plan(n, segs, nwaves);
    return (size_t)nwaves * kWave * sizeof(uint64_t);
}

hipError_t launch_topk(const float *v, int n, int k, int32_t *idx, float *val, void *scratch, hipStream_t s) {
    int segs, nwaves;
    topk_plan(n, segs, nwaves);
    uint64_t *lists = (uint64_t *)scratch;
    hipLaunchKernelGGL(k_topk_local, dim3((nwaves + 3) / 4), dim3(256), 0, s, v, n, segs, nwaves, lists);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k_topk_merge, dim3(1), dim3(1024), 0, s, lists, nwaves, k, v, idx, val);
    return hipGetLastError();
}

}  // namespace m27q
