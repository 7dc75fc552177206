// m27q_device.h -- gfx950 device helpers shared by the kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "m27q_layout.h"

namespace m27q {

constexpr int kWave = 64;  // CDNA wavefront width

// e^t, with t clamped to [-87, 87], so that 2^n and the result stay normal
// floats; a NaN t gives NaN back (so gated() and silu() propagate it).  Cody-Waite range reduction (W. J. Cody and
// W. Waite, Software Manual for the Elementary Functions, 1980):
// n = rint(t log2 e), r = t - n ln2 with ln2 split into a float and the
// float of its remainder (the first FMA is exact), then the degree-7 Taylor
// polynomial of e^r on |r| <= ln2 / 2 (truncation below 1e-8 relative) by
// Horner's rule in FMAs, times 2^n built from its exponent bits.  Every step
// is an IEEE operation with one rounding (multiply, FMA, rint), nothing is
// contracted, so the host oracle's restatement of the same sequence gives the
// same bits; within 2 ulp of e^t.
__device__ __forceinline__ float exp_cw(float t) {
#pragma clang fp contract(off)
    const float t0 = t;
    t = fminf(fmaxf(t, -87.0f), 87.0f);
    const float n = __builtin_rintf(t * 0x1.715476p+0f);
    float r = __builtin_fmaf(-n, 0x1.62e430p-1f, t);
    r = __builtin_fmaf(-n, -0x1.05c610p-29f, r);
    float p = 0x1.a01a02p-13f;
    p = __builtin_fmaf(p, r, 0x1.6c16c2p-10f);
    p = __builtin_fmaf(p, r, 0x1.111112p-7f);
    p = __builtin_fmaf(p, r, 0x1.555556p-5f);
    p = __builtin_fmaf(p, r, 0x1.555556p-3f);
    p = __builtin_fmaf(p, r, 0.5f);
    p = __builtin_fmaf(p, r, 1.0f);
    p = __builtin_fmaf(p, r, 1.0f);
    const float e = p * __int_as_float(((int)n + 127) << 23);
    return __builtin_isnan(t0) ? t0 : e;
}

// x * sigmoid(g), the gated activation of k_quant_q8_1_fused_gate
// (exec:109-138, x * (1 / (1 + e^-g))); the one definition both quantizer
// kernels use.  IEEE divide and multiply, e^-g from exp_cw.
__device__ __forceinline__ float gated(float x, float g) {
#pragma clang fp contract(off)
    return x * (1.0f / (1.0f + exp_cw(-g)));
}

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

// The same 16 bytes from five dword loads: the 20 bytes from p rounded down
// to a multiple of 4, shifted into place (v_alignbit_b32).  The caller
// guarantees that those 20 bytes are readable (for GGUF Q6_K's ql and qh
// chunks they lie inside the block: the next field follows).
__device__ __forceinline__ uint4 ld_u128_a2w(const uint8_t *p) {
    typedef uint32_t u4a4 __attribute__((ext_vector_type(4), aligned(4)));
    // offset from p itself, so that the pointer keeps its global address space
    // (through an integer it would become a flat pointer, and flat loads also
    // count against the LDS wait counter)
    const uint32_t mis = (uint32_t)((uintptr_t)p & 2);
    const uint32_t *w = (const uint32_t *)(p - mis);
    const uint32_t sh = mis * 8;  // 0 or 16 bits
    const u4a4 v = *(const u4a4 *)w;
    const uint32_t e = w[4];
    return make_uint4(__builtin_amdgcn_alignbit(v.y, v.x, sh), __builtin_amdgcn_alignbit(v.z, v.y, sh),
                      __builtin_amdgcn_alignbit(v.w, v.z, sh), __builtin_amdgcn_alignbit(e, v.w, sh));
}

// 16-byte load.  NT marks it non-temporal (global_load_dwordx4 ... nt), the
// policy of the weight streams, which are read once per product: it keeps them
// from displacing the activations and outputs other workgroups and the next
// launch read from the caches.
template <bool NT = false>
__device__ __forceinline__ uint4 ld_u128(const uint8_t *p) {
    if constexpr (NT) {
        typedef unsigned int u4v __attribute__((ext_vector_type(4)));
        const u4v v = __builtin_nontemporal_load((const u4v *)p);
        return make_uint4(v.x, v.y, v.z, v.w);
    } else {
        return *(const uint4 *)p;
    }
}

// Raw buffer loads: a scalar base (the descriptor) and scalar offset, a 32-bit
// per-lane offset, no per-lane address arithmetic.  The record count is the
// buffer's size, so a read past it returns zeros and touches no memory.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void *base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)bytes, 0x00020000);
}
// AUX is the cache policy: 2 marks the load non-temporal (buffer_load ... nt).
template <int AUX = 0>
__device__ __forceinline__ uint4 bld_u128(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    typedef unsigned int u4v __attribute__((ext_vector_type(4)));
    const u4v v = __builtin_bit_cast(u4v, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, AUX));
    return make_uint4(v.x, v.y, v.z, v.w);
}
template <int AUX = 0>
__device__ __forceinline__ uint2 bld_u64(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    typedef unsigned int u2v __attribute__((ext_vector_type(2)));
    const u2v v = __builtin_bit_cast(u2v, __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, AUX));
    return make_uint2(v.x, v.y);
}
template <int AUX = 0>
__device__ __forceinline__ uint32_t bld_u32(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, AUX);
}
template <int AUX = 0>
__device__ __forceinline__ uint32_t bld_u16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    return __builtin_amdgcn_raw_buffer_load_b16(r, voff, soff, AUX);
}

template <typename T>
__device__ __forceinline__ T shfl_xor(T v, int mask, int width = kWave) {
    return __shfl_xor(v, mask, width);
}

// Cross-lane moves inside a row of 16 lanes (DPP: no LDS traffic).
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}
template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xf, 0xf, false);
}
constexpr int kDppXor1 = 0xB1;        // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;        // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141;  // lane i <-> 7 - i within each 8 lanes

// Sum over 8 consecutive lanes (8a .. 8a+7); every lane gets the sum.
__device__ __forceinline__ float sum8(float v) {
    v += dpp_f<kDppXor1>(v);
    v += dpp_f<kDppXor2>(v);
    v += dpp_f<kDppHalfMirror>(v);
    return v;
}

// ---------------------------------------------------------------------------
// Per-32 activation quantization.  The rule (fixed here and restated by the
// oracle): d = amax / 127 (IEEE divide), id = 1 / d (IEEE divide; 0 when
// that is not finite: d == 0, or a subnormal d below 2^-128), code =
// roundf(x * id) (one fp32 multiply, round half away from zero), clamped to
// +-127.  A group whose id is 0 has all codes 0 (its values are below
// 3.7e-37 in magnitude).  A NaN value stays out of amax (maxNum) and takes
// code 0 (the float-to-int conversion of NaN); a group of NaNs has d = 0.  This is the rule of ggml's reference quantizer
// quantize_row_q8_1_ref; the reference's GPU kernel (exec:84-107) writes
// roundf(x / d) under fast-math, which compiles to the same multiply by an
// approximate reciprocal.  Besides d, the two 16-value integer code sums are
// kept, packed as (int16 lo) | (int16 hi) << 16.
// 1 / d where that is finite, else 0 (d == 0 gives +inf first).
__device__ __forceinline__ float inv_scale(float d) {
    const float r = 1.0f / d;
    return r < __builtin_inff() ? r : 0.0f;
}

// roundf(x * id) clamped to +-127.  For |v| < 2^23, (int)(v + copysign(h, v))
// with h = 0.49999997f (the largest float below 0.5) equals (int)roundf(v):
// checked over every such float.  Below 0.5 the sum stays below 1; from 0.5
// on it lands in the right unit interval, ties going away from zero.  The
// product and the sum are each rounded once, as the host oracle's x * id and
// roundf are: contracting them into an FMA (the default for HIP) would skip
// the product's rounding.  id is finite (inv_scale), so |v| <= 127 (1 + 2^-21)
// even for a subnormal d, and the conversion is always defined.
__device__ __forceinline__ int quant_code(float x, float id) {
#pragma clang fp contract(off)
    const float v = x * id;
    const int t = (int)(v + __builtin_copysignf(0.49999997f, v));
    return t > 127 ? 127 : (t < -127 ? -127 : t);
}

// amax / 127, correctly rounded, in three operations: q = amax * rn(1/127),
// then one FMA correction from the exact residual amax - 127 q.  Equal to the
// IEEE division for every non-negative finite float, subnormals included
// (checked over all of them; the kernels keep fp32 denormals); +inf is
// passed through as the division would.
__device__ __forceinline__ float div127(float a) {
#pragma clang fp contract(off)
    const float c = 1.0f / 127.0f;
    const float q = a * c;
    const float d = __builtin_fmaf(__builtin_fmaf(-q, 127.0f, a), c, q);
    return a == __builtin_inff() ? a : d;
}

// Four codes in [-127, 127] as the bytes of one word (v_perm_b32 byte picks;
// selector 0x0c gives a zero byte).
__device__ __forceinline__ uint32_t pack_codes(int q0, int q1, int q2, int q3) {
    const uint32_t lo = __builtin_amdgcn_perm((uint32_t)q1, (uint32_t)q0, 0x0c0c0400u);
    const uint32_t hi = __builtin_amdgcn_perm((uint32_t)q3, (uint32_t)q2, 0x0c0c0400u);
    return lo | (hi << 16);
}

__device__ __forceinline__ uint32_t pack_sums(int lo, int hi) {
    return (uint32_t)(uint16_t)(int16_t)lo | ((uint32_t)(uint16_t)(int16_t)hi << 16);
}

// One value per lane, one 32-lane half-wave per group.  Returns the code;
// *d_out gets d and *s_out the packed sums (valid in every lane of the group).
__device__ __forceinline__ int quant32(float v, float *d_out, uint32_t *s_out) {
    float amax = fmaxf(fabsf(v), 0.0f);  // 0 for NaN
#pragma unroll
    for (int m = 16; m > 0; m >>= 1) amax = fmaxf(amax, __shfl_xor(amax, m, 32));
    const float d = div127(amax);
    const float id = inv_scale(d);
    const int q = quant_code(v, id);
    int s = q;
#pragma unroll
    for (int m = 8; m > 0; m >>= 1) s += __shfl_xor(s, m, 16);
    const int lane32 = (int)(threadIdx.x & 31);
    const int s_other = __shfl_xor(s, 16, 32);
    *d_out = d;
    *s_out = lane32 < 16 ? pack_sums(s, s_other) : pack_sums(s_other, s);
    return q;
}

// Eight consecutive values per lane, one group per 4 consecutive lanes
// (lanes 4a .. 4a+3; lane l of the group holds values 8 l .. 8 l + 7).
// Returns the 8 codes packed as bytes; *d_out as in quant32 (every lane), and
// *s_out as in quant32 in the group's first lane 4a only.  Bit-identical to
// quant32 on the same group: the max, the divides, the multiplies and the
// integer sums see the same values.  The staging of every fp32-input product
// runs this once per 8 values, so it is kept short: the code sums are two dot
// products with ones, and only the lane that stores them packs them (a
// per-lane choice of the packing order compiled to a branch).  Measured: the
// layer 0.6 us faster; dropping the clamp too (it never acts) made the
// compiler's schedule of config 1's loop 0.4 us slower.
__device__ __forceinline__ uint2 quant32x8(float4 a, float4 b, float *d_out, uint32_t *s_out) {
    float amax = fmaxf(fmaxf(fmaxf(fabsf(a.x), fabsf(a.y)), fmaxf(fabsf(a.z), fabsf(a.w))),
                       fmaxf(fmaxf(fabsf(b.x), fabsf(b.y)), fmaxf(fabsf(b.z), fmaxf(fabsf(b.w), 0.0f))));
    amax = fmaxf(amax, dpp_f<kDppXor1>(amax));
    amax = fmaxf(amax, dpp_f<kDppXor2>(amax));
    const float d = div127(amax);
    const float id = inv_scale(d);
    const uint32_t lo = pack_codes(quant_code(a.x, id), quant_code(a.y, id), quant_code(a.z, id), quant_code(a.w, id));
    const uint32_t hi = pack_codes(quant_code(b.x, id), quant_code(b.y, id), quant_code(b.z, id), quant_code(b.w, id));
    int s = dot4((int)hi, 0x01010101, dot4((int)lo, 0x01010101, 0));
    s += dpp_i<kDppXor1>(s);  // lanes 4a, 4a+1: values 0..15; lanes 4a+2, 4a+3: values 16..31
    *d_out = d;
    *s_out = pack_sums(s, dpp_i<kDppXor2>(s));
    return make_uint2(lo, hi);
}

// IQ4_NL / IQ4_XS table (exec:51-55) as bytes: entries 0..3, 4..7, 8..11, 12..15.
constexpr uint32_t kIq4T0 = 0xBFAD9881u, kIq4T1 = 0xF6EADDCFu, kIq4T2 = 0x26190D01u, kIq4T3 = 0x71594535u;

// Four 4-bit indices (one per byte, values 0..15) -> four int8 table values.
// v_perm_b32 picks bytes of {S0, S1} by selector (0..3: S1, 4..7: S0): one
// lookup in entries 0..7, one in 8..15, then a third picks per byte by bit 3.
__device__ __forceinline__ uint32_t iq4_lut(uint32_t n) {
    const uint32_t sel = n & 0x07070707u;
    const uint32_t lo = __builtin_amdgcn_perm(kIq4T1, kIq4T0, sel);
    const uint32_t hi = __builtin_amdgcn_perm(kIq4T3, kIq4T2, sel);
    return __builtin_amdgcn_perm(hi, lo, 0x03020100u | ((n & 0x08080808u) >> 1));
}

}  // namespace m27q
