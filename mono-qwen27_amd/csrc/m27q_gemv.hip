// m27q_gemv.hip -- M = 1 matrix-vector products on gfx950.
//
// Integer-dot products (int8 activation codes x GGUF weight codes):
//   A workgroup owns TPW tiles of 8 rows and KS wavefronts.  Wave w streams the
//   w-th K slice (a contiguous run of units) of every one of those tiles,
//   unit by unit: for each unit it reads the activation fragment from LDS once
//   and applies it to the unit's block in all TPW tiles.  The loads of the
//   next unit (TPW fragments per matrix) are issued before the current unit is
//   computed (double buffering); every load in the loop is unconditional, so
//   the number of loads in flight at each wait is fixed at compile time.
//   Splitting K over the waves multiplies the number of wavefronts a short
//   matrix launches (the 5120-row down projection launches 640 x KS waves
//   instead of 640).  Within a wave, lane 8 i + c works on row i of a tile and
//   on the c-th 16-byte chunk of the unit's quants; the 8 lane partials of a
//   row are combined with DPP adds, the KS wave partials in LDS, in a fixed
//   order (the result does not depend on timing).
//   The activation is staged once per workgroup in LDS: either copied from an
//   already quantized buffer, or quantized right there from fp32 values with
//   the rule of m27q_quant_act (same codes, bit for bit), which removes the
//   separate quantization launch in front of every product.  Its loads are
//   issued before the first weight loads.
//   Epilogues: + residual, SwiGLU of two matrices (silu(gate) * up), and the
//   per-32 quantization of the output rows for the next product.
//   Balanced tiling (GemvParams::bal): workgroup w of G owns tiles
//   [w T / G, (w + 1) T / G), so one workgroup per CU carries an even share
//   of a matrix whose tile count is not a multiple of the CU count.
//
// fp32-activation products (exact dequantization, fp32 accumulation) keep the
// simpler one-wave-per-tile mapping: they are the fallback, not the hot path.
//
// Replaces k_q4k_mv_q8_dp4a / k_q6k_mv_q8_dp4a / k_q80_mv_q8_dp4a
// (exec:320-364, :631-645, :535-580), k_q5k_mv_q8 (exec:497-531),
// k_iq4xs_mv_q8_dp4a (exec:674-686),
// k_q4k_q4k_swiglu_dp4a (exec:369-417),
// k_quant_q8_1 in front of them (exec:84-107, launched by l_quant_q8_n
// :2022-2030) and the fp32 fallbacks k_q4k_mv / k_q6k_mt / k_q80_mv / k_f16_mv
// / k_f32_mv / k_q5k_mv / k_iq4xs_mv (exec:920-951, :1053-1072, :1076-1096,
// :899-916, :1100-1114, :953-985, :992-1020).
#include <algorithm>

#include "m27q_gemv_cfg.h"
#include "m27q_internal.h"
#include "m27q_types.h"

namespace m27q {

// Activation staging into LDS: codes[Kp] | d[Kp/32] | aux[Kp/32 * T::kAuxWords]
// (zero padded from K to Kp).  stage_load() loads one batch into registers (the
// first before the first weight loads), stage_store() converts and stores it.
constexpr int kStageSlots = 4;  // per thread: 4 x 32 B of fp32 values, or 4 x 16 B of codes

template <bool XF32>
struct StageRegs {
    float4 v[kStageSlots][2];
};
template <>
struct StageRegs<false> {
    uint4 v[kStageSlots];
    float d[kStageSlots];
    uint32_t s[kStageSlots];
};

template <bool XF32>
__device__ __forceinline__ void stage_load(StageRegs<XF32> &r, const GemvParams &p, int j0, int nth) {
    if constexpr (XF32) {
        // slot b of thread t: values 8 j .. 8 j + 7 with j = j0 + b * nth
        const int k8 = p.K / 8;
        const float4 *x4 = (const float4 *)p.x;
#pragma unroll
        for (int b = 0; b < kStageSlots; ++b) {
            const int j = j0 + b * nth;
            const bool in = j < k8;
            r.v[b][0] = in ? x4[2 * j] : make_float4(0.f, 0.f, 0.f, 0.f);
            r.v[b][1] = in ? x4[2 * j + 1] : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    } else {
        const int k16 = p.K / 16, k32 = p.K / 32;
        const uint4 *src = (const uint4 *)p.xq;
#pragma unroll
        for (int b = 0; b < kStageSlots; ++b) {
            const int j = j0 + b * nth;
            r.v[b] = j < k16 ? src[j] : make_uint4(0, 0, 0, 0);
            r.d[b] = j < k32 ? p.xd[j] : 0.f;
            r.s[b] = j < k32 ? p.xs[j] : 0u;
        }
    }
}

template <class T, bool XF32>
__device__ __forceinline__ void stage_store(const StageRegs<XF32> &r, uint8_t *smem, int Kp, int j0, int nth) {
    int8_t *xc = (int8_t *)smem;
    float *xd = (float *)(smem + Kp);
    uint32_t *xs = (uint32_t *)(smem + Kp + Kp / 8);
    if constexpr (XF32) {
        // A 32-value group is 4 consecutive slots j (4 consecutive lanes; nth
        // and Kp / 8 are multiples of 4, so a group is wholly in or out).
#pragma unroll
        for (int b = 0; b < kStageSlots; ++b) {
            const int j = j0 + b * nth;
            if (j < Kp / 8) {
                float d;
                uint32_t s;
                ((uint2 *)xc)[j] = quant32x8(r.v[b][0], r.v[b][1], &d, &s);
                if ((j & 3) == 0) {
                    xd[j / 4] = d;
                    T::put_aux(xs, j / 4, d, s);
                }
            }
        }
    } else {
#pragma unroll
        for (int b = 0; b < kStageSlots; ++b) {
            const int j = j0 + b * nth;
            if (j < Kp / 16) ((uint4 *)xc)[j] = r.v[b];
            if (j < Kp / 32) {
                xd[j] = r.d[b];
                T::put_aux(xs, j, r.d[b], r.s[b]);
            }
        }
    }
}

template <bool XF32>
__device__ __forceinline__ int stage_span(int Kp) {
    return XF32 ? Kp / 8 : Kp / 16;  // slots needed for the whole activation
}

// silu(g) = g / (1 + e^-g), e^-g from exp_cw (the gated quantizer's exp).
__device__ __forceinline__ float silu(float g) {
#pragma clang fp contract(off)
    return g / (1.0f + exp_cw(-g));
}

template <class T, int NM, int TPW>
__device__ __forceinline__ void compute_unit(const typename T::Frag (&f)[NM][TPW], const ActLds &act, int u,
                                             const typename T::Lane &L, float (&acc)[NM][TPW]) {
    const typename T::AFrag a = T::load_act(act, u, L);
#pragma unroll
    for (int m = 0; m < NM; ++m)
#pragma unroll
        for (int t = 0; t < TPW; ++t) acc[m][t] += T::dot(f[m][t], a, L);
}

// Fused per-32 quantization of the output rows: the workgroup's NR rows are
// whole 32-row groups (rc % 32 == 0 and NR % 32 == 0 are checked on the host).
// Sharing a group between workgroups would need a device-scope fence, which
// on a multi-XCD part writes back the whole L2 of the XCD (measured: 20x
// slower), so output-quantizing products always launch 32-row workgroups.
template <int NR>
__device__ __forceinline__ void quant_output(const GemvParams &p, int row0, int rc, float v) {
    static_assert(NR % 32 == 0, "output-quantizing workgroups hold whole 32-row groups");
    const int t = (int)threadIdx.x;
    if (t < NR && row0 + (t & ~31) < rc) {
        const int row = row0 + t;
        float d;
        uint32_t s;
        const int q = quant32(v, &d, &s);
        p.oq[row] = (int8_t)q;
        if ((t & 31) == 0) {
            p.od[row / 32] = d;
            p.os[row / 32] = s;
        }
    }
}

#ifdef M27Q_WAVE_TIMELINE
// Measurement build only (libm27q_timeline.so): per wave of the last launch,
// {start, activation staged, end} from the 100 MHz real-time counter and
// {HW_ID, XCC_ID, workgroup << 8 | wave}.  Slots past the capacity are dropped.
constexpr int kTimelineCap = 1 << 16;
__device__ unsigned long long g_timeline_t[kTimelineCap][3];
__device__ unsigned int g_timeline_hw[kTimelineCap][3];

__device__ __forceinline__ void timeline_record(unsigned long long t0, unsigned long long t1, int nw, int wave) {
    const unsigned long long t2 = __builtin_amdgcn_s_memrealtime();
    const int slot = (int)blockIdx.x * nw + wave;
    if ((threadIdx.x & 63) == 0 && slot < kTimelineCap) {
        g_timeline_t[slot][0] = t0;
        g_timeline_t[slot][1] = t1;
        g_timeline_t[slot][2] = t2;
        g_timeline_hw[slot][0] = __builtin_amdgcn_s_getreg((31 << 11) | 4);   // HW_ID
        g_timeline_hw[slot][1] = __builtin_amdgcn_s_getreg((31 << 11) | 20);  // XCC_ID
        g_timeline_hw[slot][2] = (blockIdx.x << 8) | (unsigned)wave;
    }
}
#endif

template <class T, int LAYOUT, class C, bool SWIGLU, bool XF32>
__global__ __launch_bounds__(kWave *C::NW) void k_gemv_q8(GemvParams p) {
    extern __shared__ __align__(16) uint8_t smem[];
#ifdef M27Q_WAVE_TIMELINE
    const unsigned long long tl_start = __builtin_amdgcn_s_memrealtime();
#endif
    constexpr int KS = C::KS, TPW = C::TPW, WT = C::WT;
    constexpr int NM = SWIGLU ? 2 : 1;
    constexpr int NR = TPW * kTileRows;  // rows per workgroup
    using LM = LaneMap<T, LAYOUT>;
    const int lane = (int)(threadIdx.x & 63), i = LM::row(lane), c = LM::chunk(lane);
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int ks = wave % KS, tg = wave / KS;  // K slice and tile group of this wave
    const int nth = C::NW * kWave;

    // Matrix of this workgroup (up to kMaxMulti matrices share one launch).
    int m = 0;
#pragma unroll
    for (int k = 1; k < kMaxMulti; ++k)
        if (k < p.nmat && (int)blockIdx.x >= p.wg_start[k]) m = k;
    const int rc = p.rc[m];
    const int ntiles = (rc + kTileRows - 1) / kTileRows;
    // Tiles of this workgroup: TPW from tile0, or, with balanced tiling, nt
    // of them (TPW - 1 or TPW); the waves of the slots past nt stream no
    // units (their loads would go to HBM again: the weight loads are
    // non-temporal) and those rows are not written.
    const int wg = (int)blockIdx.x - p.wg_start[m];
    int tile0 = wg * TPW, nt = TPW;
    if (p.bal) {
        const int G = p.wg_start[m + 1] - p.wg_start[m];
        tile0 = (int)((long long)wg * ntiles / G);
        nt = (int)((long long)(wg + 1) * ntiles / G) - tile0;
    }

    // K slice of this wave: units [ub, ub + nu); a wave with no units reads a
    // valid unit and discards it.
    const int U = p.upr / KS, rem = p.upr % KS;
    const int ub = ks * U + min(ks, rem);
    const int nu = tg * WT >= nt ? 0 : U + (ks < rem ? 1 : 0);

    // 1. first batch of the activation, 2. the first unit of weights (their
    // latency overlaps the staging), 3. activation to LDS.
    const int Kp = p.upr * T::kUnitElems;
    StageRegs<XF32> sr;
    stage_load<XF32>(sr, p, (int)threadIdx.x, nth);

    const uint8_t *W[NM];
    W[0] = p.W[m];
    if constexpr (SWIGLU) W[NM - 1] = p.W[1];
    // buffer loads for the Q6_K stream only (see UnitStream).  GGUF-layout
    // weights keep temporal loads: a row's 144- or 210-byte blocks straddle
    // 128-byte lines, and the line two consecutive units share is then still
    // in L2 for the second (gate/up in GGUF layout: 23.4 us against 28.4
    // with non-temporal loads)
    const UnitStream<T, LAYOUT, NM, WT, C::NT && LAYOUT == M27Q_LAYOUT_TILED, T::kType == kQ6_K> ws(W, tile0 + tg * WT, min(ntiles, tile0 + nt), rc,
                                                                      p.rb, p.upr, lane);
    typename T::Frag fa[NM][WT], fb[NM][WT];
    ws.load(fa, min(ub, p.upr - 1));

    stage_store<T, XF32>(sr, smem, Kp, (int)threadIdx.x, nth);
    for (int j0 = (int)threadIdx.x + kStageSlots * nth; j0 < stage_span<XF32>(Kp); j0 += kStageSlots * nth) {
        stage_load<XF32>(sr, p, j0, nth);
        stage_store<T, XF32>(sr, smem, Kp, j0, nth);
    }
    const ActLds act{(const int8_t *)smem, (const float *)(smem + Kp), (const uint32_t *)(smem + Kp + Kp / 8)};
    float *red = (float *)(smem + Kp + Kp / 8 * (1 + T::kAuxWords));  // [NM][KS][NR]
    __syncthreads();
#ifdef M27Q_WAVE_TIMELINE
    const unsigned long long tl_staged = __builtin_amdgcn_s_memrealtime();
#endif

    float acc[NM][WT];
#pragma unroll
    for (int mm = 0; mm < NM; ++mm)
#pragma unroll
        for (int t = 0; t < WT; ++t) acc[mm][t] = 0.f;
    // Each unit's loads are issued before the previous unit is computed.  For
    // one tile per wave, scheduling barriers keep the compiler from hoisting
    // that computation (and its wait for the previous loads) above the new
    // loads, which leaves one unit in flight at every wait, and from sinking
    // it below the next loads into the same buffer, which costs a register
    // copy that waits for them (measured: gate/up 0.5 us and down 0.3 us
    // faster; the multi-tile shapes were 0.3 us slower with them).
    int k = 0;
    for (; k + 2 < nu; k += 2) {
        ws.load(fb, ub + k + 1);
        if constexpr (WT == 1) __builtin_amdgcn_sched_barrier(0);
        compute_unit<T, NM, WT>(fa, act, ub + k, ws.L, acc);
        if constexpr (WT == 1) __builtin_amdgcn_sched_barrier(0);
        ws.load(fa, ub + k + 2);
        if constexpr (WT == 1) __builtin_amdgcn_sched_barrier(0);
        compute_unit<T, NM, WT>(fb, act, ub + k + 1, ws.L, acc);
        if constexpr (WT == 1) __builtin_amdgcn_sched_barrier(0);
    }
    if (k + 1 < nu) {
        ws.load(fb, ub + k + 1);
        if constexpr (WT == 1) __builtin_amdgcn_sched_barrier(0);
        compute_unit<T, NM, WT>(fa, act, ub + k, ws.L, acc);
        compute_unit<T, NM, WT>(fb, act, ub + k + 1, ws.L, acc);
    } else if (k < nu) {
        compute_unit<T, NM, WT>(fa, act, ub + k, ws.L, acc);
    }

    // Row partials of this wave's slice -> LDS.
#pragma unroll
    for (int mm = 0; mm < NM; ++mm)
#pragma unroll
        for (int t = 0; t < WT; ++t) {
            const float r = LM::sum(acc[mm][t]);
            if (c == 0) red[(mm * KS + ks) * NR + (tg * WT + t) * kTileRows + i] = r;
        }
    __syncthreads();

    // Epilogue: one thread per row of the workgroup.
    const int t = (int)threadIdx.x;
    float v = 0.f;
    if (t < NR) {
        const int row = tile0 * kTileRows + t;
        v = red[t];
#pragma unroll
        for (int w = 1; w < KS; ++w) v += red[w * NR + t];
        const bool own = row < rc && t < nt * kTileRows;
        if constexpr (SWIGLU) {
            float vu = red[KS * NR + t];
#pragma unroll
            for (int w = 1; w < KS; ++w) vu += red[(KS + w) * NR + t];
            v = silu(v) * vu;
        } else {
            if (p.res[m] && own) v += p.res[m][row];
        }
        if (own) p.y[m][row] = v;
    }
    if constexpr (NR % 32 == 0)
        if (p.oq) quant_output<NR>(p, tile0 * kTileRows, rc, v);
#ifdef M27Q_WAVE_TIMELINE
    timeline_record(tl_start, tl_staged, C::NW, wave);
#endif
}

// ------------------------------------------------ fp32-activation products --

// Weight-tile iterator: per wave, yields fragment loads for unit u.
template <class T, int LAYOUT>
struct TileSrc {
    const uint8_t *base;
    int rb, i, c;
    typename T::Lane L;
    __device__ TileSrc(const uint8_t *W, int tile, int row, int rb_, int upr, int lane)
        : rb(rb_), i(LaneMap<T, LAYOUT>::row(lane)), c(LaneMap<T, LAYOUT>::chunk(lane)), L(LaneMap<T, LAYOUT>::chunk(lane)) {
        if (LAYOUT == M27Q_LAYOUT_TILED) base = W + (size_t)tile * upr * T::kUnitBytes;
        else base = W + (size_t)row * rb_ * T::kBlockBytes;
    }
    __device__ typename T::Frag load(int u) const {
        if (LAYOUT == M27Q_LAYOUT_TILED) return T::load_tiled(base + (size_t)u * T::kUnitBytes, i, c, L);
        return T::load_gguf(base, u, rb, c, L);
    }
};

// acc += sum over units of T::dot_f32 with a two-stage load pipeline.
template <class T, int LAYOUT, int kDepth, class A>
__device__ __forceinline__ float stream_row_f32(const TileSrc<T, LAYOUT> &src, const A &act, int upr) {
    typename T::Frag fa[kDepth], fb[kDepth];
    float acc = 0.f;
#pragma unroll
    for (int k = 0; k < kDepth; ++k)
        if (k < upr) fa[k] = src.load(k);
    for (int u0 = 0; u0 < upr; u0 += 2 * kDepth) {
#pragma unroll
        for (int k = 0; k < kDepth; ++k)
            if (u0 + kDepth + k < upr) fb[k] = src.load(u0 + kDepth + k);
#pragma unroll
        for (int k = 0; k < kDepth; ++k)
            if (u0 + k < upr) acc += T::dot_f32(fa[k], act, u0 + k, src.L);
#pragma unroll
        for (int k = 0; k < kDepth; ++k)
            if (u0 + 2 * kDepth + k < upr) fa[k] = src.load(u0 + 2 * kDepth + k);
#pragma unroll
        for (int k = 0; k < kDepth; ++k)
            if (u0 + kDepth + k < upr) acc += T::dot_f32(fb[k], act, u0 + kDepth + k, src.L);
    }
    return acc;
}

// One workgroup = 4 waves = 32 rows; x and its per-16 sums staged in LDS.
template <class T, int LAYOUT>
__global__ __launch_bounds__(256) void k_gemv_f32(GemvParams p) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int Kp = p.upr * T::kUnitElems;
    float *xf = (float *)smem;
    float *x16 = xf + Kp;
    for (int j = threadIdx.x; j < Kp / 4; j += blockDim.x)
        ((float4 *)xf)[j] = (j < p.K / 4) ? ((const float4 *)p.x)[j] : make_float4(0.f, 0.f, 0.f, 0.f);
    __syncthreads();
    for (int j = threadIdx.x; j < Kp / 16; j += blockDim.x) {
        float s = 0.f;
#pragma unroll
        for (int l = 0; l < 16; ++l) s += xf[16 * j + l];
        x16[j] = s;
    }
    __syncthreads();
    const ActLdsF32 act{xf, x16};

    using LM = LaneMap<T, LAYOUT>;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, i = LM::row(lane), c = LM::chunk(lane);
    const int rc = p.rc[0];
    const int tile = (int)blockIdx.x * kWavesPerWG + wave;
    const int ntiles = (rc + kTileRows - 1) / kTileRows;
    const int row = tile * kTileRows + i;
    const int row_ld = row < rc ? row : rc - 1;
    float acc = 0.f;
    if (tile < ntiles) {
        const TileSrc<T, LAYOUT> src(p.W[0], tile, row_ld, p.rb, p.upr, lane);
        acc = stream_row_f32<T, LAYOUT, 2>(src, act, p.upr);
    }
    acc = LM::sum(acc);
    if (c == 0 && tile < ntiles && row < rc) p.y[0][row] = acc + (p.res[0] ? p.res[0][row] : 0.f);
}

// F16 / F32 weights (GGUF rows of K elements): 8 lanes per row stride over
// 16-byte chunks of the row; x is read through L1/L2 (these matrices are small:
// the reference uses F16 for the 48 x 5120 ssm_beta / ssm_alpha, exec:2496-2497).
template <bool HALF>
__global__ __launch_bounds__(256) void k_gemv_dense(GemvParams p) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, i = lane >> 3, c = lane & 7;
    const int rc = p.rc[0];
    const int row = ((int)blockIdx.x * kWavesPerWG + wave) * kTileRows + i;
    const int K = p.K;
    constexpr int kPer = HALF ? 8 : 4;  // elements per 16-byte chunk
    float acc = 0.f;
    if (row < rc) {
        const uint8_t *rp = p.W[0] + (size_t)row * K * (HALF ? 2 : 4);
        for (int k0 = c * kPer; k0 < K; k0 += kLanesPerRow * kPer) {
            const uint4 w = ld_u128(rp + (size_t)k0 * (HALF ? 2 : 4));
            const float4 xa = *(const float4 *)(p.x + k0);
            if constexpr (HALF) {
                const float4 xb = *(const float4 *)(p.x + k0 + 4);
                acc += f16_bits_to_f32(w.x) * xa.x + f16_bits_to_f32(w.x >> 16) * xa.y +
                       f16_bits_to_f32(w.y) * xa.z + f16_bits_to_f32(w.y >> 16) * xa.w +
                       f16_bits_to_f32(w.z) * xb.x + f16_bits_to_f32(w.z >> 16) * xb.y +
                       f16_bits_to_f32(w.w) * xb.z + f16_bits_to_f32(w.w >> 16) * xb.w;
            } else {
                acc += __uint_as_float(w.x) * xa.x + __uint_as_float(w.y) * xa.y + __uint_as_float(w.z) * xa.z +
                       __uint_as_float(w.w) * xa.w;
            }
        }
    }
    acc = sum8(acc);
    if (c == 0 && row < rc) p.y[0][row] = acc + (p.res[0] ? p.res[0][row] : 0.f);
}

// ------------------------------------------------------------- launchers --

template <class T, class C, bool SWIGLU>
size_t gemv_q8_lds(int upr) {
    const size_t Kp = (size_t)upr * T::kUnitElems;
    return Kp + Kp / 8 * (1 + T::kAuxWords) + (size_t)(SWIGLU ? 2 : 1) * C::KS * C::TPW * kTileRows * sizeof(float);
}

template <class T, int LAYOUT, class C, bool SWIGLU, bool XF32>
static hipError_t launch_q8_cfg(const GemvParams &p, hipStream_t s) {
    const size_t lds = gemv_q8_lds<T, C, SWIGLU>(p.upr);
    hipLaunchKernelGGL((k_gemv_q8<T, LAYOUT, C, SWIGLU, XF32>), dim3(p.wg_start[p.nmat]), dim3(kWave * C::NW), lds, s,
                       p);
    return hipGetLastError();
}

template <class T, int LAYOUT, bool SWIGLU, bool XF32>
static hipError_t launch_q8_t(const GemvParams &p, int cfg, hipStream_t s) {
    switch (cfg) {
        case kCfgQ: return launch_q8_cfg<T, LAYOUT, CfgQ, SWIGLU, XF32>(p, s);
        case kCfg81: return launch_q8_cfg<T, LAYOUT, Cfg81, SWIGLU, XF32>(p, s);
        case kCfg42: return launch_q8_cfg<T, LAYOUT, Cfg42, SWIGLU, XF32>(p, s);
        case kCfg84:  // products without the SwiGLU epilogue only (it is never
                      // chosen with it, and several tiles per wave of two
                      // matrices spilled registers)
            if constexpr (!SWIGLU) return launch_q8_cfg<T, LAYOUT, Cfg84, SWIGLU, XF32>(p, s);
            return hipErrorInvalidValue;
        case kCfg161:  // chosen for small products without the SwiGLU epilogue only
            if constexpr (!SWIGLU) return launch_q8_cfg<T, LAYOUT, Cfg161, SWIGLU, XF32>(p, s);
            return launch_q8_cfg<T, LAYOUT, Cfg41, SWIGLU, XF32>(p, s);
        case kCfgB:  // balanced tiling, single products without the SwiGLU epilogue only
            if constexpr (!SWIGLU) return launch_q8_cfg<T, LAYOUT, CfgB, SWIGLU, XF32>(p, s);
            return hipErrorInvalidValue;
        case kCfgB9:
            if constexpr (!SWIGLU) return launch_q8_cfg<T, LAYOUT, CfgB9, SWIGLU, XF32>(p, s);
            return hipErrorInvalidValue;
        default: return launch_q8_cfg<T, LAYOUT, Cfg41, SWIGLU, XF32>(p, s);
    }
}

template <class T, bool SWIGLU, bool XF32>
static hipError_t launch_q8_l(const GemvParams &p, int layout, int cfg, hipStream_t s) {
    return layout == M27Q_LAYOUT_TILED ? launch_q8_t<T, M27Q_LAYOUT_TILED, SWIGLU, XF32>(p, cfg, s)
                                       : launch_q8_t<T, M27Q_LAYOUT_GGUF, SWIGLU, XF32>(p, cfg, s);
}

template <class T>
static hipError_t launch_q8_x(const GemvParams &p, int layout, bool swiglu, int cfg, hipStream_t s) {
    const bool xf = p.x != nullptr;
    if (swiglu) return xf ? launch_q8_l<T, true, true>(p, layout, cfg, s) : launch_q8_l<T, true, false>(p, layout, cfg, s);
    return xf ? launch_q8_l<T, false, true>(p, layout, cfg, s) : launch_q8_l<T, false, false>(p, layout, cfg, s);
}

template <class T, class C>
static size_t lds_sw(int upr, bool swiglu) {
    return swiglu ? gemv_q8_lds<T, C, true>(upr) : gemv_q8_lds<T, C, false>(upr);
}

template <class T>
static size_t lds_for(int upr, bool swiglu, int cfg) {
    switch (cfg) {
        case kCfg81: return lds_sw<T, Cfg81>(upr, swiglu);
        case kCfg42: return lds_sw<T, Cfg42>(upr, swiglu);
        case kCfg84: return lds_sw<T, Cfg84>(upr, swiglu);
        case kCfgQ: return lds_sw<T, CfgQ>(upr, swiglu);
        case kCfg161: return swiglu ? lds_sw<T, Cfg41>(upr, swiglu) : lds_sw<T, Cfg161>(upr, swiglu);
        case kCfgB: return lds_sw<T, CfgB>(upr, swiglu);
        case kCfgB9: return lds_sw<T, CfgB9>(upr, swiglu);
        default: return lds_sw<T, Cfg41>(upr, swiglu);
    }
}

size_t gemv_q8_lds_bytes(uint32_t type, int upr, bool swiglu, int cfg) {
    switch (type) {
        case kQ4_K: return lds_for<Q4K>(upr, swiglu, cfg);
        case kQ5_K: return lds_for<Q5K>(upr, swiglu, cfg);
        case kQ6_K: return lds_for<Q6K>(upr, swiglu, cfg);
        case kQ8_0: return lds_for<Q80>(upr, swiglu, cfg);
        case kIQ4_XS: return lds_for<IQ4XS>(upr, swiglu, cfg);
        default: return 0;
    }
}

int gemv_q8_tiles_per_wg(int cfg) {
    switch (cfg) {
        case kCfg81: return Cfg81::TPW;
        case kCfg42: return Cfg42::TPW;
        case kCfg84: return Cfg84::TPW;
        case kCfgQ: return CfgQ::TPW;
        case kCfg161: return Cfg161::TPW;
        case kCfgB: return CfgB::TPW;
        case kCfgB9: return CfgB9::TPW;
        default: return Cfg41::TPW;
    }
}

hipError_t launch_gemv_q8(uint32_t type, int layout, bool swiglu, int cfg, const GemvParams &p, hipStream_t s) {
    switch (type) {
        case kQ4_K: return launch_q8_x<Q4K>(p, layout, swiglu, cfg, s);
        case kQ5_K: return launch_q8_x<Q5K>(p, layout, swiglu, cfg, s);
        case kQ6_K: return launch_q8_x<Q6K>(p, layout, swiglu, cfg, s);
        case kQ8_0: return launch_q8_x<Q80>(p, layout, swiglu, cfg, s);
        case kIQ4_XS: return launch_q8_x<IQ4XS>(p, layout, swiglu, cfg, s);
        default: return hipErrorInvalidValue;
    }
}

size_t gemv_f32_lds_bytes(uint32_t type, int upr) {
    const int ue = type == kQ8_0 ? Q80::kUnitElems : 256;
    const size_t Kp = (size_t)upr * ue;
    return Kp * 4 + Kp / 4;
}

template <class T, int LAYOUT>
static hipError_t launch_f32_t(const GemvParams &p, int grid, hipStream_t s) {
    const size_t lds = gemv_f32_lds_bytes(T::kType, p.upr);
    hipLaunchKernelGGL((k_gemv_f32<T, LAYOUT>), dim3(grid), dim3(256), lds, s, p);
    return hipGetLastError();
}

template <class T>
static hipError_t launch_f32_l(const GemvParams &p, int layout, int grid, hipStream_t s) {
    return layout == M27Q_LAYOUT_TILED ? launch_f32_t<T, M27Q_LAYOUT_TILED>(p, grid, s)
                                       : launch_f32_t<T, M27Q_LAYOUT_GGUF>(p, grid, s);
}

hipError_t launch_gemv_f32(uint32_t type, int layout, const GemvParams &p, int grid, hipStream_t s) {
    switch (type) {
        case kQ4_K: return launch_f32_l<Q4K>(p, layout, grid, s);
        case kQ5_K: return launch_f32_l<Q5K>(p, layout, grid, s);
        case kQ6_K: return launch_f32_l<Q6K>(p, layout, grid, s);
        case kQ8_0: return launch_f32_l<Q80>(p, layout, grid, s);
        case kIQ4_XS: return launch_f32_l<IQ4XS>(p, layout, grid, s);
        case kF16:
            hipLaunchKernelGGL((k_gemv_dense<true>), dim3(grid), dim3(256), 0, s, p);
            return hipGetLastError();
        case kF32:
            hipLaunchKernelGGL((k_gemv_dense<false>), dim3(grid), dim3(256), 0, s, p);
            return hipGetLastError();
        default: return hipErrorInvalidValue;
    }
}

}  // namespace m27q

#ifdef M27Q_WAVE_TIMELINE
// Copies the first n records to the host (n <= 65536); clears them.
extern "C" __attribute__((visibility("default"))) int m27q_timeline_read(unsigned long long *t, unsigned int *hw, int n) {
    if (n < 0 || n > m27q::kTimelineCap) return -1;
    if (hipMemcpyFromSymbol(t, HIP_SYMBOL(m27q::g_timeline_t), (size_t)n * 24, 0, hipMemcpyDeviceToHost) != hipSuccess ||
        hipMemcpyFromSymbol(hw, HIP_SYMBOL(m27q::g_timeline_hw), (size_t)n * 12, 0, hipMemcpyDeviceToHost) != hipSuccess)
        return -2;
    return 0;
}
extern "C" __attribute__((visibility("default"))) int m27q_timeline_clear() {
    static unsigned long long zero[m27q::kTimelineCap][3];
    return hipMemcpyToSymbol(HIP_SYMBOL(m27q::g_timeline_t), zero, sizeof zero, 0, hipMemcpyHostToDevice) == hipSuccess
               ? 0
               : -1;
}
#endif
