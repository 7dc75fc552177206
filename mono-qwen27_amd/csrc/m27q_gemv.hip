// m27q_gemv.hip -- M = 1 matrix-vector products on gfx950.
//
// One workgroup = 4 wavefronts = 32 output rows; each wavefront owns a tile of
// 8 rows and streams its weight tile unit by unit (one 256-weight block
// column, or four Q8_0 block columns) with 16-byte loads per lane.  The
// activation is staged once per workgroup in LDS; every lane of a row reads
// its 32 activation codes from there (8 distinct addresses per instruction).
// Loads run two pipeline stages of kDepth units ahead of the arithmetic.
// The 8 partial sums of a row are combined with cross-lane adds at the end.
//
// Replaces k_q4k_mv_q8_dp4a / k_q6k_mv_q8_dp4a / k_q80_mv_q8_dp4a
// (exec:320-364, :631-645, :535-580), k_q4k_q4k_swiglu_dp4a (exec:369-417)
// and the fp32 fallbacks k_q4k_mv / k_q6k_mt / k_q80_mv / k_f16_mv / k_f32_mv
// (exec:920-951, :1053-1072, :1076-1096, :899-916, :1100-1114).
#include "m27q_internal.h"
#include "m27q_types.h"

namespace m27q {

template <class T>
__device__ __forceinline__ int padded_k(int upr) {
    return upr * T::kUnitElems;
}

// Weight-tile iterator: per wave, yields fragment loads for unit u.
template <class T, int LAYOUT>
struct TileSrc {
    const uint8_t *base;
    int rb, i, c;
    typename T::Lane L;
    __device__ TileSrc(const uint8_t *W, int tile, int row, int rb_, int upr, int lane)
        : rb(rb_), i(lane >> 3), c(lane & 7), L(lane & 7) {
        if (LAYOUT == M27Q_LAYOUT_TILED) base = W + (size_t)tile * upr * T::kUnitBytes;
        else base = W + (size_t)row * rb_ * T::kBlockBytes;
    }
    __device__ typename T::Frag load(int u) const {
        if (LAYOUT == M27Q_LAYOUT_TILED) return T::load_tiled(base + (size_t)u * T::kUnitBytes, i, c, L);
        return T::load_gguf(base, u, rb, c, L);
    }
};

// acc += sum over units of T::dot (or dot_f32) with a two-stage load pipeline.
template <class T, int LAYOUT, int kDepth, bool F32, class A>
__device__ __forceinline__ float stream_row(const TileSrc<T, LAYOUT> &src, const A &act, int upr) {
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
            if (u0 + k < upr) {
                if constexpr (F32) acc += T::dot_f32(fa[k], act, u0 + k, src.L);
                else acc += T::dot(fa[k], act, u0 + k, src.L);
            }
#pragma unroll
        for (int k = 0; k < kDepth; ++k)
            if (u0 + 2 * kDepth + k < upr) fa[k] = src.load(u0 + 2 * kDepth + k);
#pragma unroll
        for (int k = 0; k < kDepth; ++k)
            if (u0 + kDepth + k < upr) {
                if constexpr (F32) acc += T::dot_f32(fb[k], act, u0 + kDepth + k, src.L);
                else acc += T::dot(fb[k], act, u0 + kDepth + k, src.L);
            }
    }
    return acc;
}

// Stage the quantized activation (global -> LDS), zero-padding to Kp.
template <class T>
__device__ __forceinline__ ActLds stage_act_q8(uint8_t *smem, const GemvParams &p, int Kp) {
    int8_t *xc = (int8_t *)smem;
    float *xd = (float *)(smem + Kp);
    uint32_t *xs = (uint32_t *)(smem + Kp + Kp / 8);
    const uint4 *src = (const uint4 *)p.xq;
    for (int j = threadIdx.x; j < Kp / 16; j += blockDim.x)
        ((uint4 *)xc)[j] = (j < p.K / 16) ? src[j] : make_uint4(0, 0, 0, 0);
    for (int j = threadIdx.x; j < Kp / 32; j += blockDim.x) {
        float d = 0.f;
        uint32_t s = 0u;
        if (j < p.K / 32) {
            d = p.xd[j];
            s = p.xs[j];
        }
        xd[j] = d;
        xs[j] = T::stage_aux(d, s);
    }
    return {xc, xd, xs};
}

__device__ __forceinline__ float silu(float g) { return g / (1.0f + expf(-g)); }

// Fused epilogue: quantize the workgroup's 32 consecutive outputs (row0 .. row0+31).
__device__ __forceinline__ void quant_epilogue(float *outv, const GemvParams &p, int wave, int i, int c,
                                               float v, int row0) {
    if (c == 0) outv[wave * kTileRows + i] = v;
    __syncthreads();
    if (threadIdx.x < 32) {
        float d;
        uint32_t s;
        const int q = quant32(outv[threadIdx.x], &d, &s);
        p.oq[row0 + threadIdx.x] = (int8_t)q;
        if (threadIdx.x == 0) {
            p.od[row0 / 32] = d;
            p.os[row0 / 32] = s;
        }
    }
}

template <class T, int LAYOUT, bool SWIGLU>
__global__ __launch_bounds__(256) void k_gemv_q8(GemvParams p) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int Kp = padded_k<T>(p.upr);
    const ActLds act = stage_act_q8<T>(smem, p, Kp);
    float *outv = (float *)(smem + Kp + Kp / 4);
    __syncthreads();

    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, i = lane >> 3, c = lane & 7;
    int m = 0;
#pragma unroll
    for (int k = 1; k < kMaxMulti; ++k)
        if (k < p.nmat && (int)blockIdx.x >= p.wg_start[k]) m = k;
    const int wgl = (int)blockIdx.x - p.wg_start[m];
    const int rc = p.rc[m];
    const int tile = wgl * kWavesPerWG + wave;
    const int ntiles = (rc + kTileRows - 1) / kTileRows;
    const int row = tile * kTileRows + i;
    const int row_ld = row < rc ? row : rc - 1;  // GGUF rows past the end: reread the last row

    float acc = 0.f, acc_up = 0.f;
    if (tile < ntiles) {
        constexpr int kDepth = SWIGLU ? 2 : 4;
        const TileSrc<T, LAYOUT> src(p.W[m], tile, row_ld, p.rb, p.upr, lane);
        acc = stream_row<T, LAYOUT, kDepth, false>(src, act, p.upr);
        if constexpr (SWIGLU) {
            const TileSrc<T, LAYOUT> src_up(p.W[1], tile, row_ld, p.rb, p.upr, lane);
            acc_up = stream_row<T, LAYOUT, kDepth, false>(src_up, act, p.upr);
        }
    }
    acc = sum8(acc);
    float v;
    if constexpr (SWIGLU) {
        acc_up = sum8(acc_up);
        v = silu(acc) * acc_up;
    } else {
        v = acc;
        if (p.res[m] && tile < ntiles && row < rc) v += p.res[m][row];
    }
    if (c == 0 && tile < ntiles && row < rc) p.y[m][row] = v;
    if (p.oq) quant_epilogue(outv, p, wave, i, c, v, wgl * kRowsPerWG);
}

// fp32-activation product: stage x and its per-16 sums in LDS.
template <class T, int LAYOUT>
__global__ __launch_bounds__(256) void k_gemv_f32(GemvParams p) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int Kp = padded_k<T>(p.upr);
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

    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, i = lane >> 3, c = lane & 7;
    const int rc = p.rc[0];
    const int tile = (int)blockIdx.x * kWavesPerWG + wave;
    const int ntiles = (rc + kTileRows - 1) / kTileRows;
    const int row = tile * kTileRows + i;
    const int row_ld = row < rc ? row : rc - 1;
    float acc = 0.f;
    if (tile < ntiles) {
        const TileSrc<T, LAYOUT> src(p.W[0], tile, row_ld, p.rb, p.upr, lane);
        acc = stream_row<T, LAYOUT, 2, true>(src, act, p.upr);
    }
    acc = sum8(acc);
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

template <class T, int LAYOUT, bool SWIGLU>
static hipError_t launch_q8(const GemvParams &p, int grid, hipStream_t s) {
    const int Kp = p.upr * T::kUnitElems;
    const size_t lds = (size_t)Kp + (size_t)Kp / 4 + kRowsPerWG * sizeof(float);
    hipLaunchKernelGGL((k_gemv_q8<T, LAYOUT, SWIGLU>), dim3(grid), dim3(256), lds, s, p);
    return hipGetLastError();
}

template <class T, bool SWIGLU>
static hipError_t dispatch_layout_q8(const GemvParams &p, int layout, int grid, hipStream_t s) {
    return layout == M27Q_LAYOUT_TILED ? launch_q8<T, M27Q_LAYOUT_TILED, SWIGLU>(p, grid, s)
                                       : launch_q8<T, M27Q_LAYOUT_GGUF, SWIGLU>(p, grid, s);
}

size_t gemv_q8_lds_bytes(uint32_t type, int upr) {
    const int ue = type == kQ8_0 ? Q80::kUnitElems : 256;
    const size_t Kp = (size_t)upr * ue;
    return Kp + Kp / 4 + kRowsPerWG * sizeof(float);
}

size_t gemv_f32_lds_bytes(uint32_t type, int upr) {
    const int ue = type == kQ8_0 ? Q80::kUnitElems : 256;
    const size_t Kp = (size_t)upr * ue;
    return Kp * 4 + Kp / 4;
}

hipError_t launch_gemv_q8(uint32_t type, int layout, bool swiglu, const GemvParams &p, int grid, hipStream_t s) {
    switch (type) {
        case kQ4_K: return swiglu ? dispatch_layout_q8<Q4K, true>(p, layout, grid, s)
                                  : dispatch_layout_q8<Q4K, false>(p, layout, grid, s);
        case kQ6_K: return swiglu ? dispatch_layout_q8<Q6K, true>(p, layout, grid, s)
                                  : dispatch_layout_q8<Q6K, false>(p, layout, grid, s);
        case kQ8_0: return swiglu ? dispatch_layout_q8<Q80, true>(p, layout, grid, s)
                                  : dispatch_layout_q8<Q80, false>(p, layout, grid, s);
        default: return hipErrorInvalidValue;
    }
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
        case kQ6_K: return launch_f32_l<Q6K>(p, layout, grid, s);
        case kQ8_0: return launch_f32_l<Q80>(p, layout, grid, s);
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
