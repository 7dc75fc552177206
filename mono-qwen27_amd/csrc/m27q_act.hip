// m27q_act.hip -- fp32 activations -> per-32 int8 codes with fp32 scale.
//
// One lane per value, one 32-lane half-wave per group: amax by cross-lane max,
// d = amax/127 (IEEE divide), code = roundf(x * (1/d)) clamped to +-127 (the
// rule of quant32 in m27q_device.h), and the two 16-code integer sums.  Replaces k_quant_q8_1 / k_quant_q8_1_fused_gate
// (exec:84-107, :109-138), which keep an fp16 scale and the float sum of x.
#include "m27q_internal.h"
#include "m27q_device.h"

namespace m27q {

template <bool GATED>
__global__ __launch_bounds__(256) void k_quant_act(const float *__restrict__ x, const float *__restrict__ gate,
                                                   long long n, int8_t *__restrict__ q, float *__restrict__ d,
                                                   uint32_t *__restrict__ s) {
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    // n is a multiple of 32, so a 32-lane group is either wholly in range or wholly out.
    if (i - (threadIdx.x & 31) >= n) return;
    float v = x[i];
    if constexpr (GATED) v = gated(v, gate[i]);
    float dd;
    uint32_t ss;
    const int code = quant32(v, &dd, &ss);
    q[i] = (int8_t)code;
    if ((threadIdx.x & 31) == 0) {
        d[i / 32] = dd;
        s[i / 32] = ss;
    }
}

// Eight values per lane, one group per 4 consecutive lanes (quant32x8, the
// products' staging rule: the same codes as quant32): for 16-byte aligned
// inputs, a shorter dependency chain (two DPP steps instead of five
// cross-lane shuffles) and an eighth of the lanes.
template <bool GATED>
__global__ __launch_bounds__(256) void k_quant_act8(const float4 *__restrict__ x, const float4 *__restrict__ gate,
                                                    long long n8, uint2 *__restrict__ q, float *__restrict__ d,
                                                    uint32_t *__restrict__ s) {
    const long long t = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    // n8 = n / 8 is a multiple of 4, so a 4-lane group is wholly in range or out.
    if (t >= n8) return;
    float4 a = x[2 * t], b = x[2 * t + 1];
    if constexpr (GATED) {
        const float4 ga = gate[2 * t], gb = gate[2 * t + 1];
        a = make_float4(gated(a.x, ga.x), gated(a.y, ga.y), gated(a.z, ga.z), gated(a.w, ga.w));
        b = make_float4(gated(b.x, gb.x), gated(b.y, gb.y), gated(b.z, gb.z), gated(b.w, gb.w));
    }
    float dd;
    uint32_t ss;
    q[t] = quant32x8(a, b, &dd, &ss);
    if ((t & 3) == 0) {
        d[t / 4] = dd;
        s[t / 4] = ss;
    }
}

hipError_t launch_quant_act(const float *x, const float *gate, long long n, int8_t *q, float *d, uint32_t *s,
                            hipStream_t st) {
    const bool vec = ((uintptr_t)x % 16 == 0) && ((uintptr_t)gate % 16 == 0);
    if (vec) {
        const long long n8 = n / 8;
        const int grid = (int)((n8 + 255) / 256);
        if (gate)
            hipLaunchKernelGGL((k_quant_act8<true>), dim3(grid), dim3(256), 0, st, (const float4 *)x,
                               (const float4 *)gate, n8, (uint2 *)q, d, s);
        else
            hipLaunchKernelGGL((k_quant_act8<false>), dim3(grid), dim3(256), 0, st, (const float4 *)x, nullptr, n8,
                               (uint2 *)q, d, s);
        return hipGetLastError();
    }
    const int grid = (int)((n + 255) / 256);
    if (gate) hipLaunchKernelGGL((k_quant_act<true>), dim3(grid), dim3(256), 0, st, x, gate, n, q, d, s);
    else hipLaunchKernelGGL((k_quant_act<false>), dim3(grid), dim3(256), 0, st, x, gate, n, q, d, s);
    return hipGetLastError();
}

}  // namespace m27q
