// m27q_device.h -- gfx950 device helpers shared by the kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "m27q_layout.h"

namespace m27q {

constexpr int kWave = 64;  // CDNA wavefront width

__device__ __forceinline__ float f16_bits_to_f32(uint32_t bits16) {
    const uint16_t b = (uint16_t)bits16;
    _Float16 h;
    __builtin_memcpy(&h, &b, 2);
    return (float)h;  // v_cvt_f32_f16: exact for every half, subnormals included
}

// 4-way int8 dot product with int32 accumulate (v_dot4c_i32_i8 on gfx950).
__device__ __forceinline__ int dot4(int a, int b, int c) { return __builtin_amdgcn_sdot4(a, b, c, false); }

// 32-bit load from a 2-byte aligned address (GGUF Q6_K / Q8_0 blocks are 210 /
// 34 bytes long, so their fields are only halfword aligned).
__device__ __forceinline__ uint32_t ld_u32_a2(const uint8_t *p) {
    const uint16_t *h = (const uint16_t *)p;
    return (uint32_t)h[0] | ((uint32_t)h[1] << 16);
}

__device__ __forceinline__ uint4 ld_u128_a2(const uint8_t *p) {
    return make_uint4(ld_u32_a2(p), ld_u32_a2(p + 4), ld_u32_a2(p + 8), ld_u32_a2(p + 12));
}

__device__ __forceinline__ uint4 ld_u128(const uint8_t *p) { return *(const uint4 *)p; }

template <typename T>
__device__ __forceinline__ T shfl_xor(T v, int mask, int width = kWave) {
    return __shfl_xor(v, mask, width);
}

// Sum over the 8 lanes that share one row (lanes 8i .. 8i+7).
__device__ __forceinline__ float sum8(float v) {
    v += shfl_xor(v, 1);
    v += shfl_xor(v, 2);
    v += shfl_xor(v, 4);
    return v;
}

// Per-32 activation quantization of one value per lane over 32-lane groups:
// d = amax/127 (IEEE divide), q = roundf(v/d) clamped to +-127, 0 if amax == 0.
// Returns the code; *d_out gets d and *s_out the packed 16-lane sums (valid in
// every lane of the group).
__device__ __forceinline__ int quant32(float v, float *d_out, uint32_t *s_out) {
    float amax = fabsf(v);
#pragma unroll
    for (int m = 16; m > 0; m >>= 1) amax = fmaxf(amax, shfl_xor(amax, m, 32));
    const float d = amax / 127.0f;
    int q = 0;
    if (amax != 0.0f) {
        q = (int)roundf(v / d);
        q = q > 127 ? 127 : (q < -127 ? -127 : q);
    }
    int s = q;
#pragma unroll
    for (int m = 8; m > 0; m >>= 1) s += shfl_xor(s, m, 16);
    const int lane32 = (int)(threadIdx.x & 31);
    const int s_other = shfl_xor(s, 16, 32);
    const int lo = lane32 < 16 ? s : s_other, hi = lane32 < 16 ? s_other : s;
    *d_out = d;
    *s_out = (uint32_t)(uint16_t)(int16_t)lo | ((uint32_t)(uint16_t)(int16_t)hi << 16);
    return q;
}

}  // namespace m27q
