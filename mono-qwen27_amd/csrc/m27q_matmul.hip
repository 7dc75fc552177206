// m27q_matmul.hip -- small-M products Y[M][N] = X[M][K] W[N][K]^T, M <= 64.
//
// Same wavefront tiling as the M = 1 GEMV (8 rows per wave, 16-byte weight
// loads); the weights are read once per group of up to 16 activation rows and
// each lane keeps one accumulator per row.  Activations are staged in LDS per
// K-chunk of 4 units for all rows of the group, so LDS stays small at any K.
// No reference counterpart: the reference feeds prefill one token at a time
// (src/mono27b_chat.cpp:399-403).
#include "m27q_internal.h"
#include "m27q_types.h"

namespace m27q {

constexpr int kChunkUnits = 4;

template <class T, int LAYOUT, int MT>
__global__ __launch_bounds__(256) void k_matmul_q8(MatmulParams p, int m0) {
    extern __shared__ __align__(16) uint8_t smem[];
    constexpr int CK = kChunkUnits * T::kUnitElems;  // activation values per chunk
    int8_t *xc = (int8_t *)smem;                    // [MT][CK]
    float *xd = (float *)(smem + MT * CK);           // [MT][CK/32]
    uint32_t *xs = (uint32_t *)(xd + MT * CK / 32);  // [MT][CK/32 * T::kAuxWords]

    using LM = LaneMap<T, LAYOUT>;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, i = LM::row(lane), c = LM::chunk(lane);
    const int rc = p.rc;
    const int tile = (int)blockIdx.x * kWavesPerWG + wave;
    const int ntiles = (rc + kTileRows - 1) / kTileRows;
    const int row = tile * kTileRows + i;
    const int row_ld = row < rc ? row : rc - 1;
    typename T::Lane L(c);
    const uint8_t *base = LAYOUT == M27Q_LAYOUT_TILED ? p.W + (size_t)tile * p.upr * T::kUnitBytes
                                                      : p.W + (size_t)row_ld * p.rb * T::kBlockBytes;
    float acc[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m) acc[m] = 0.f;

    for (int u0 = 0; u0 < p.upr; u0 += kChunkUnits) {
        __syncthreads();  // the previous chunk has been consumed
        for (int j = threadIdx.x; j < MT * CK / 16; j += blockDim.x) {
            const int m = j / (CK / 16), q16 = j % (CK / 16);
            const long long kpos = (long long)u0 * T::kUnitElems + 16 * q16;
            uint4 v = make_uint4(0, 0, 0, 0);
            if (m0 + m < p.M && kpos < p.K) v = *(const uint4 *)(p.xq + (size_t)(m0 + m) * p.K + kpos);
            ((uint4 *)xc)[j] = v;
        }
        for (int j = threadIdx.x; j < MT * CK / 32; j += blockDim.x) {
            const int m = j / (CK / 32), g = j % (CK / 32);
            const long long gpos = (long long)u0 * T::kUnitElems / 32 + g;
            float d = 0.f;
            uint32_t s = 0u;
            if (m0 + m < p.M && gpos < p.K / 32) {
                d = p.xd[(size_t)(m0 + m) * (p.K / 32) + gpos];
                s = p.xs[(size_t)(m0 + m) * (p.K / 32) + gpos];
            }
            xd[j] = d;
            T::put_aux(xs, j, d, s);
        }
        __syncthreads();
        if (tile < ntiles) {
            typename T::Frag f[kChunkUnits];
#pragma unroll
            for (int k = 0; k < kChunkUnits; ++k)
                if (u0 + k < p.upr) {
                    if (LAYOUT == M27Q_LAYOUT_TILED) f[k] = T::load_tiled(base + (size_t)(u0 + k) * T::kUnitBytes, i, c, L);
                    else f[k] = T::load_gguf(base, u0 + k, p.rb, c, L);
                }
#pragma unroll
            for (int k = 0; k < kChunkUnits; ++k)
                if (u0 + k < p.upr) {
#pragma unroll
                    for (int m = 0; m < MT; ++m) {
                        const ActLds a{xc + m * CK, xd + m * (CK / 32), xs + m * (CK / 32) * T::kAuxWords};
                        acc[m] += T::dot(f[k], a, k, L);
                    }
                }
        }
    }
#pragma unroll
    for (int m = 0; m < MT; ++m) {
        const float v = LM::sum(acc[m]);
        if (c == 0 && tile < ntiles && row < rc && m0 + m < p.M) {
            const size_t o = (size_t)(m0 + m) * rc + row;
            p.Y[o] = v + (p.res ? p.res[o] : 0.f);
        }
    }
}

template <class T, int LAYOUT, int MT>
static hipError_t launch_mt(const MatmulParams &p, int m0, hipStream_t s) {
    constexpr int CK = kChunkUnits * T::kUnitElems;
    const size_t lds = (size_t)MT * CK + (size_t)MT * CK / 32 * 4 * (1 + T::kAuxWords);
    const int grid = (((p.rc + kTileRows - 1) / kTileRows) + kWavesPerWG - 1) / kWavesPerWG;
    hipLaunchKernelGGL((k_matmul_q8<T, LAYOUT, MT>), dim3(grid), dim3(256), lds, s, p, m0);
    return hipGetLastError();
}

template <class T, int LAYOUT>
static hipError_t launch_m(const MatmulParams &p, hipStream_t s) {
    for (int m0 = 0; m0 < p.M; m0 += 16) {
        const int left = p.M - m0;
        hipError_t e;
        if (left <= 2) e = launch_mt<T, LAYOUT, 2>(p, m0, s);
        else if (left <= 4) e = launch_mt<T, LAYOUT, 4>(p, m0, s);
        else if (left <= 8) e = launch_mt<T, LAYOUT, 8>(p, m0, s);
        else e = launch_mt<T, LAYOUT, 16>(p, m0, s);
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

template <class T>
static hipError_t launch_l(const MatmulParams &p, int layout, hipStream_t s) {
    return layout == M27Q_LAYOUT_TILED ? launch_m<T, M27Q_LAYOUT_TILED>(p, s) : launch_m<T, M27Q_LAYOUT_GGUF>(p, s);
}

hipError_t launch_matmul_q8(uint32_t type, int layout, const MatmulParams &p, hipStream_t s) {
    switch (type) {
        case kQ4_K: return launch_l<Q4K>(p, layout, s);
        case kQ5_K: return launch_l<Q5K>(p, layout, s);
        case kQ6_K: return launch_l<Q6K>(p, layout, s);
        case kQ8_0: return launch_l<Q80>(p, layout, s);
        case kIQ4_XS: return launch_l<IQ4XS>(p, layout, s);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace m27q
