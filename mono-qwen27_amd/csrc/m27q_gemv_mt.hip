// m27q_gemv_mt.hip -- small-M products Y[M][N] = X[M][K] W[N][K]^T for a few
// tokens on the M = 1 GEMV's streaming structure.
//
// The weights are streamed exactly as by the M = 1 kernel (8-row tiles, K
// split over KS waves, 16-byte loads of one unit per lane, double buffered and
// unconditional; TILED or, with temporal loads, GGUF layout), and every
// loaded fragment is applied to MT
// activation rows staged in LDS: the weight unpacking is shared by the tokens,
// each token adds its own integer dots and scale terms, and no lane works on a
// padding token unless M is not a multiple of MT.  Its cost grows with the
// per-token dots: on the Qwen-27B layer it takes 56 us at M = 2, against 63
// for the MFMA kernel, which is faster from M = 3 on; it serves M <= 2.
// No reference counterpart: the reference runs prefill and decode one token at
// a time (src/mono27b_chat.cpp:399-403).
#include <algorithm>

#include "m27q_internal.h"
#include "m27q_types.h"

namespace m27q {

template <class T, class C, int MT, int LAYOUT>
__global__ __launch_bounds__(kWave *C::NW) void k_gemv_mt(MatmulMultiParams p, int m0) {
    extern __shared__ __align__(16) uint8_t smem[];
    constexpr int KS = C::KS, TPW = C::TPW, WT = C::WT;
    constexpr int NR = TPW * kTileRows;  // rows per workgroup
    using LM = LaneMap<T, LAYOUT>;
    const int lane = (int)(threadIdx.x & 63), i = LM::row(lane), c = LM::chunk(lane);
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int ks = wave % KS, tg = wave / KS;
    const int nth = C::NW * kWave;

    int mi = 0;
#pragma unroll
    for (int k = 1; k < kMaxMulti; ++k)
        if (k < p.nmat && (int)blockIdx.x >= p.wg_start[k]) mi = k;
    const int rc = p.rc[mi];
    const int ntiles = (rc + kTileRows - 1) / kTileRows;
    // Tiles of this workgroup: TPW from tile0, or, with balanced tiling, nt
    // of them (TPW - 1 or TPW); the waves of the slots past nt stream no
    // units (their loads would go to HBM again: the weight loads are
    // non-temporal) and those rows are not written.
    const int wg = (int)blockIdx.x - p.wg_start[mi];
    int tile0 = wg * TPW, nt = TPW;
    if (p.bal_wgs > 0) {
        tile0 = (int)((long long)wg * ntiles / p.bal_wgs);
        nt = (int)((long long)(wg + 1) * ntiles / p.bal_wgs) - tile0;
    }
    const int U = p.upr / KS, rem = p.upr % KS;
    const int ub = ks * U + min(ks, rem);
    const int nu = tg * WT >= nt ? 0 : U + (ks < rem ? 1 : 0);

    // First unit of weights before the staging, so their latencies overlap.
    const uint8_t *W[1] = {p.W[mi]};
    // GGUF layout: temporal loads (a row's consecutive blocks share lines)
    const UnitStream<T, LAYOUT, 1, WT, C::NT && LAYOUT == M27Q_LAYOUT_TILED> ws(W, tile0 + tg * WT, min(ntiles, tile0 + nt),
                                                                               rc, p.rb, p.upr, lane);
    typename T::Frag fa[1][WT], fb[1][WT];
    ws.load(fa, min(ub, p.upr - 1));

    // Activations of tokens m0 .. m0 + MT: codes [MT][Kp] | d [MT][Kp/32] |
    // aux [MT][Kp/32 * T::kAuxWords], zero past K and past M.  Loads go out 4 per thread
    // before their stores.
    const int Kp = p.upr * T::kUnitElems, gp = Kp / 32, ng = p.K / 32;
    const int nq = Kp / 16;
    int8_t *xc = (int8_t *)smem;
    float *xd = (float *)(smem + (size_t)MT * Kp);
    uint32_t *xs = (uint32_t *)(xd + MT * gp);
    for (int j0 = (int)threadIdx.x; j0 < MT * nq; j0 += 4 * nth) {
        uint4 v[4];
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const int j = j0 + b * nth, tok = j / nq, q16 = j % nq;
            const bool in = j < MT * nq && m0 + tok < p.M && 16 * q16 < p.K;
            const size_t src = in ? (size_t)(m0 + tok) * p.K + 16 * q16 : 0;
            v[b] = *(const uint4 *)(p.xq + src);
            if (!in) v[b] = make_uint4(0u, 0u, 0u, 0u);
        }
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const int j = j0 + b * nth;
            if (j < MT * nq) ((uint4 *)xc)[j] = v[b];
        }
    }
    for (int j0 = (int)threadIdx.x; j0 < MT * gp; j0 += 4 * nth) {
        float d[4];
        uint32_t s[4];
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const int j = j0 + b * nth, tok = j / gp, g = j % gp;
            const bool in = j < MT * gp && m0 + tok < p.M && g < ng;
            const size_t src = in ? (size_t)(m0 + tok) * ng + g : 0;
            d[b] = p.xd[src];
            s[b] = p.xs[src];
            if (!in) {
                d[b] = 0.f;
                s[b] = 0u;
            }
        }
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const int j = j0 + b * nth;
            if (j < MT * gp) {
                xd[j] = d[b];
                T::put_aux(xs, j, d[b], s[b]);
            }
        }
    }
    float *red = (float *)(xs + MT * gp * T::kAuxWords);  // [MT][KS][NR]
    __syncthreads();

    float acc[MT][WT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int t = 0; t < WT; ++t) acc[mt][t] = 0.f;
    auto compute = [&](const typename T::Frag (&f)[1][WT], int u) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            const ActLds act{xc + (size_t)mt * Kp, xd + mt * gp, xs + mt * gp * T::kAuxWords};
            const typename T::AFrag a = T::load_act(act, u, ws.L);
#pragma unroll
            for (int t = 0; t < WT; ++t) acc[mt][t] += T::dot(f[0][t], a, ws.L);
        }
    };
    // Each unit's loads are issued before the previous unit is computed; for
    // one or two tiles per wave, scheduling barriers keep the compiler from
    // moving that computation, and its wait, above the new loads (as in the
    // M = 1 kernel).  Measured at M = 2: gate/up 23.3 us against 25.9, o and
    // down 0.3 us faster; q/k/v (four tiles per wave) 0.8 us slower with them.
    constexpr bool kSB = WT <= 2;
    int k = 0;
    for (; k + 2 < nu; k += 2) {
        ws.load(fb, ub + k + 1);
        if constexpr (kSB) __builtin_amdgcn_sched_barrier(0);
        compute(fa, ub + k);
        if constexpr (kSB) __builtin_amdgcn_sched_barrier(0);
        ws.load(fa, ub + k + 2);
        if constexpr (kSB) __builtin_amdgcn_sched_barrier(0);
        compute(fb, ub + k + 1);
        if constexpr (kSB) __builtin_amdgcn_sched_barrier(0);
    }
    if (k + 1 < nu) {
        ws.load(fb, ub + k + 1);
        if constexpr (kSB) __builtin_amdgcn_sched_barrier(0);
        compute(fa, ub + k);
        compute(fb, ub + k + 1);
    } else if (k < nu) {
        compute(fa, ub + k);
    }

    // Row partials of this wave's K slice -> LDS; then one thread per (token,
    // row) adds the KS partials in a fixed order.
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int t = 0; t < WT; ++t) {
            const float r = LM::sum(acc[mt][t]);
            if (c == 0) red[(mt * KS + ks) * NR + (tg * WT + t) * kTileRows + i] = r;
        }
    __syncthreads();
    for (int idx = (int)threadIdx.x; idx < MT * NR; idx += nth) {
        const int mt = idx / NR, rr = idx % NR, row = tile0 * kTileRows + rr, tok = m0 + mt;
        float v = red[mt * KS * NR + rr];
#pragma unroll
        for (int w = 1; w < KS; ++w) v += red[(mt * KS + w) * NR + rr];
        if (row < rc && rr < nt * kTileRows && tok < p.M) {
            const size_t o = (size_t)tok * rc + row;
            p.Y[mi][o] = v + (p.res[mi] ? p.res[mi][o] : 0.f);
        }
    }
}

template <class T, class C, int MT>
static size_t mt_lds(int upr) {
    const size_t Kp = (size_t)upr * T::kUnitElems;
    return MT * (Kp + Kp / 8 * (1 + T::kAuxWords)) + (size_t)MT * C::KS * C::TPW * kTileRows * sizeof(float);
}

template <class T, class C, int MT, int LAYOUT>
static hipError_t launch_mt_cfg(MatmulMultiParams p, hipStream_t s) {
    int total = 0;
    for (int i = 0; i < p.nmat; ++i) {
        p.wg_start[i] = total;
        total += p.bal_wgs > 0 ? p.bal_wgs : ((p.rc[i] + kTileRows - 1) / kTileRows + C::TPW - 1) / C::TPW;
    }
    p.wg_start[p.nmat] = total;
    const size_t lds = mt_lds<T, C, MT>(p.upr);
    for (int m0 = 0; m0 < p.M; m0 += MT) {
        hipLaunchKernelGGL((k_gemv_mt<T, C, MT, LAYOUT>), dim3(total), dim3(kWave * C::NW), lds, s, p, m0);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

// Launch shape, from sweeps of the Qwen-27B layer at M = 2 and 4: (8, 4, 2)
// for q/k/v (8192 rows of 20 units), (8, 1, 1) for o (24 units) and down (68
// units), (4, 2, 2) for gate/up (34816 rows).
static int pick_mt_cfg(long long rows, int upr) {
    if (upr >= 24) return kCfg81;
    return rows <= 12288 ? kCfg84 : kCfg42;
}

// One matrix of short rows (< 40 units) with between 2 and 3 tiles per CU
// spreads them over one workgroup per CU, as the M = 1 products do: o (640
// tiles of 24 units) 8.55-8.67 us against 8.95-9.2 with (8, 1, 1).  Down (68
// units) measured 1.8 us slower that way: one 12-wave workgroup per CU hides
// less latency than 2.5 of (8, 1, 1).
int matmul_mt_balance(long long tiles, int upr, int cus) {
    return upr < 40 && tiles > 2LL * cus && tiles <= (long long)CfgB::TPW * cus ? cus : 0;
}

template <class T, int MT, int LAYOUT>
static hipError_t launch_mt_t(const MatmulMultiParams &p, hipStream_t s) {
    if (p.bal_wgs > 0) return launch_mt_cfg<T, CfgB, MT, LAYOUT>(p, s);
    long long rows = 0;
    for (int i = 0; i < p.nmat; ++i) rows += p.rc[i];
    const int cfg = pick_mt_cfg(rows, p.upr);
    switch (cfg) {
        case kCfg81: return launch_mt_cfg<T, Cfg81, MT, LAYOUT>(p, s);
        case kCfg42: return launch_mt_cfg<T, Cfg42, MT, LAYOUT>(p, s);
        case kCfg84: return launch_mt_cfg<T, Cfg84, MT, LAYOUT>(p, s);
        default: return launch_mt_cfg<T, Cfg41, MT, LAYOUT>(p, s);
    }
}

template <class T, int MT>
static hipError_t launch_mt_l(const MatmulMultiParams &p, int layout, hipStream_t s) {
    return layout == M27Q_LAYOUT_TILED ? launch_mt_t<T, MT, M27Q_LAYOUT_TILED>(p, s)
                                       : launch_mt_t<T, MT, M27Q_LAYOUT_GGUF>(p, s);
}

size_t matmul_mt_lds_bytes(uint32_t type, int upr) {
    // the largest over the launch shapes the selection can return
    auto one = [&](auto tag) -> size_t {
        using T = decltype(tag);
        return std::max({mt_lds<T, Cfg41, 2>(upr), mt_lds<T, Cfg81, 2>(upr), mt_lds<T, Cfg42, 2>(upr),
                         mt_lds<T, Cfg84, 2>(upr), mt_lds<T, CfgB, 2>(upr)});
    };
    switch (type) {
        case kQ4_K: return one(Q4K{});
        case kQ5_K: return one(Q5K{});
        case kQ6_K: return one(Q6K{});
        case kQ8_0: return one(Q80{});
        case kIQ4_XS: return one(IQ4XS{});
        default: return 0;
    }
}

// Two tokens per launch.
hipError_t launch_matmul_mt(uint32_t type, int layout, const MatmulMultiParams &p, hipStream_t s) {
    switch (type) {
        case kQ4_K: return launch_mt_l<Q4K, 2>(p, layout, s);
        case kQ5_K: return launch_mt_l<Q5K, 2>(p, layout, s);
        case kQ6_K: return launch_mt_l<Q6K, 2>(p, layout, s);
        case kQ8_0: return launch_mt_l<Q80, 2>(p, layout, s);
        case kIQ4_XS: return launch_mt_l<IQ4XS, 2>(p, layout, s);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace m27q
