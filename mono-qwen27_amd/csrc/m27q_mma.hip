// m27q_mma.hip -- small-M products Y[M][N] = X[M][K] W[N][K]^T on int8 MFMA.
//
// For 2 <= M the per-lane dot4 path costs M times the M = 1 work and turns
// compute-bound at once; here every 32-weight group of 16 weight rows and up
// to 16 activation rows (tokens) is one v_mfma_i32_16x16x32_i8, which gives
// the exact integer group sums for all token x row pairs.  The scales are
// applied in fp32 afterwards: per group j, row r, token t
//   Q4_K: d_r sc_rj dx_tj S_trj - dmin_r m_rj dx_tj sum(codes_tj)
//   Q6_K: d_r dx_tj (sc_r,2j (S0 - 32 lo16_tj) + sc_r,2j+1 (S1 - 32 hi16_tj)),
//         one MFMA per 16-value sub-block (the other half of the operand zero)
//   Q8_0: d_r dx_tj S_trj
// which are the per-group terms of the M = 1 products.
//
// Lane roles (v_mfma_i32_16x16x32_i8, layout checked on the device):
//   A (activations): lane l holds token l % 16, K positions 8 q .. 8 q + 7 of
//                    the group, q = l / 16;
//   B (weights):     lane l holds row l % 16 of a 16-row tile, same positions;
//   C:               lane l holds tokens 4 q .. 4 q + 3 of row l % 16.
// Weights are read straight from the TILED layout (a 16-row tile is two 8-row
// tiles), the token codes from the quantized activation buffer (L1/L2 hits:
// every wave at the same K reads the same bytes), the activation scales from
// LDS, staged transposed ([group][16 tokens]) so a lane reads its 4 tokens at
// once.  K is split over the KS waves of a workgroup (as in the M = 1 GEMV);
// each wave covers RT 16-row tiles, and the KS partials are reduced in LDS in a
// fixed order.  Tokens beyond 16 are handled by further launches.
//
// No reference counterpart: the reference runs prefill and decode one token at
// a time (src/mono27b_chat.cpp:399-403).
#include <type_traits>

#include "m27q_internal.h"
#include "m27q_device.h"

namespace m27q {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
constexpr int kMmaTok = 16;  // tokens per MFMA (padded with zeros)

__device__ __forceinline__ long as_long(uint32_t lo, uint32_t hi) { return (long)(((uint64_t)hi << 32) | lo); }

__device__ __forceinline__ v4i mfma32(long a, long b, v4i c) {
    return __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ v4f mfma_f32(float a, float b, v4f c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// Activation scales in LDS, transposed to [group][16 tokens]: a lane reads the
// dx of its 4 tokens (4 q .. 4 q + 3) with one 16-byte read.
struct ScaleLds {
    const float *dT;     // [groups][16 tokens]
    const float *aT;     // [groups][16 tokens], the type's per-group token term (Q4_K only)
    __device__ float4 dx(int g, int q) const { return *(const float4 *)(dT + g * 16 + 4 * q); }
    __device__ float aux(int g, int tok) const { return aT[g * 16 + tok]; }
};

__device__ __forceinline__ int s_lo(uint32_t s) { return (int)(int16_t)(s & 0xffffu); }
__device__ __forceinline__ int s_hi(uint32_t s) { return (int)(int16_t)(s >> 16); }
__device__ __forceinline__ float f4(const float4 &v, int e) { return e == 0 ? v.x : e == 1 ? v.y : e == 2 ? v.z : v.w; }
__device__ __forceinline__ uint32_t u4(const uint4 &v, int e) { return e == 0 ? v.x : e == 1 ? v.y : e == 2 ? v.z : v.w; }

// ------------------------------------------------------------ Q4_K, Q5_K --
// Q5_K is Q4_K with a fifth code bit per weight: bit j of qh[l] for position l
// of group j (exec:953-969), added to the operand bytes as 16.
template <bool Q5>
struct MmaQ4KT {
    static constexpr int kGroups = 8;  // 32-weight groups per unit
    static constexpr int kUnitBytes = Q5 ? kQ5KUnit : kQ4KUnit;
    static constexpr bool kAux = true;
    // The min term's token factor: dx * (sum of the 32 codes).
    __device__ static float stage_aux(float d, uint32_t s) { return d * (float)(s_lo(s) + s_hi(s)); }
    struct Frag {
        uint2 qs[4];  // bytes 32 g + 8 q .. +8 of the row's quants, g = 0..3
        uint4 h;      // d | dmin, scales[12]
        uint2 qh;     // Q5_K: qh bytes 8 q .. +8
    };
    // unit: start of the 8-row TILED unit holding row i
    __device__ static Frag load(const uint8_t *unit, int i, int q) {
        Frag f;
        const uint8_t *qs = unit + 128 + 128 * i + 8 * q;
#pragma unroll
        for (int g = 0; g < 4; ++g) f.qs[g] = *(const uint2 *)(qs + 32 * g);
        f.h = *(const uint4 *)(unit + 16 * i);
        if constexpr (Q5) f.qh = *(const uint2 *)(unit + kQ5KTQh + 32 * i + 8 * q);
        return f;
    }
    __device__ static long operand(const Frag &f, int j) {
        const uint2 w = f.qs[j >> 1];
        const int sh = 4 * (j & 1);
        uint32_t lo = (w.x >> sh) & 0x0f0f0f0fu, hi = (w.y >> sh) & 0x0f0f0f0fu;
        if constexpr (Q5) {
            lo |= ((f.qh.x >> j) & 0x01010101u) << 4;
            hi |= ((f.qh.y >> j) & 0x01010101u) << 4;
        }
        return as_long(lo, hi);
    }
    // Main term: acc[t][e] += d sc_j * dx_j,e * S_j,e per group (VALU, the
    // group's integer sums from the MFMA).  Min term: cm[t] += sum_j aux_j,tok *
    // (dmin m_j,row), an fp32 MFMA over the unit's 8 groups (2 x K = 4).
    template <int RT>
    __device__ static void accumulate(const Frag (&f)[RT], const long (&a)[kGroups], const ScaleLds &sl, int g0,
                                      int q, int r16, float (&acc)[RT][4], v4f (&cm)[RT]) {
        uint32_t scA[RT], scB[RT];
        float d[RT];
#pragma unroll
        for (int t = 0; t < RT; ++t) {
            // get_scale_min_k4 (exec:690-693) for all 8 pairs at once, one byte each
            const uint4 h = f[t].h;
            scA[t] = h.y & 0x3f3f3f3fu;
            scB[t] = (h.w & 0x0f0f0f0fu) | ((h.y >> 2) & 0x30303030u);
            const uint32_t m03 = h.z & 0x3f3f3f3fu;
            const uint32_t m47 = ((h.w >> 4) & 0x0f0f0f0fu) | ((h.z >> 2) & 0x30303030u);
            d[t] = f16_bits_to_f32(h.x);
            const float dmin = f16_bits_to_f32(h.x >> 16);
            const float b0 = dmin * (float)((m03 >> (8 * q)) & 0xffu);
            const float b1 = dmin * (float)((m47 >> (8 * q)) & 0xffu);
            cm[t] = mfma_f32(sl.aux(g0 + q, r16), b0, cm[t]);
            cm[t] = mfma_f32(sl.aux(g0 + 4 + q, r16), b1, cm[t]);
        }
        // Software pipeline: the MFMAs of group j + 1 are issued before the
        // scale arithmetic of group j; the scheduling barrier keeps each group's
        // values local.
        // The activation scales of group j + 1 are read from LDS one group
        // ahead as well, so no group waits on its own LDS read.
        v4i c[RT];
#pragma unroll
        for (int t = 0; t < RT; ++t) c[t] = mfma32(a[0], operand(f[t], 0), v4i{0, 0, 0, 0});
        float4 dx = sl.dx(g0, q);
#pragma unroll
        for (int j = 0; j < kGroups; ++j) {
            v4i cn[RT];
#pragma unroll
            for (int t = 0; t < RT; ++t) cn[t] = j + 1 < kGroups ? mfma32(a[j + 1], operand(f[t], j + 1), v4i{0, 0, 0, 0}) : c[t];
            const float4 dxn = j + 1 < kGroups ? sl.dx(g0 + j + 1, q) : dx;
#pragma unroll
            for (int t = 0; t < RT; ++t) {
                const uint32_t scw = j < 4 ? scA[t] : scB[t];
                const float ws = d[t] * (float)((scw >> (8 * (j & 3))) & 0xffu);
#pragma unroll
                for (int e = 0; e < 4; ++e) acc[t][e] = fmaf(ws, f4(dx, e) * (float)c[t][e], acc[t][e]);
                c[t] = cn[t];
            }
            dx = dxn;
            __builtin_amdgcn_sched_barrier(0);
        }
    }
};

using MmaQ4K = MmaQ4KT<false>;
using MmaQ5K = MmaQ4KT<true>;

// ------------------------------------------------------------------ Q6_K --
struct MmaQ6K {
    static constexpr int kGroups = 8;
    static constexpr int kUnitBytes = kQ6KUnit;
    static constexpr bool kAux = false;
    __device__ static float stage_aux(float, uint32_t) { return 0.f; }
    struct Frag {
        uint2 ql[2][2];  // [half h][r & 1]: ql bytes 64 h + 32 (r & 1) + 8 q .. +8
        uint2 qh[2];     // [half h]: qh bytes 32 h + 8 q .. +8
        uint4 sc;        // 16 int8 scales
        uint32_t d;      // f16 bits
    };
    __device__ static Frag load(const uint8_t *unit, int i, int q) {
        Frag f;
        const uint8_t *ql = unit + kQ6KTQl + 128 * i + 8 * q;
        const uint8_t *qh = unit + kQ6KTQh + 64 * i + 8 * q;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            f.ql[h][0] = *(const uint2 *)(ql + 64 * h);
            f.ql[h][1] = *(const uint2 *)(ql + 64 * h + 32);
            f.qh[h] = *(const uint2 *)(qh + 32 * h);
        }
        f.sc = *(const uint4 *)(unit + kQ6KTSc + 16 * i);
        f.d = *(const uint16_t *)(unit + kQ6KTD + 2 * i);
        return f;
    }
    __device__ static int sc_byte(const uint4 &sc, int k) {
        return (int)(int8_t)(u4(sc, k >> 2) >> (8 * (k & 3)));
    }
    // Group j = 4 h + r covers K 32 j .. 32 j + 31 of the block (half h, quarter r
    // of the q6k_val index map, exec:1026-1048); sub-block 2 j (scale 8 h + 2 r)
    // is held by lane quarters 0, 1 and sub-block 2 j + 1 by quarters 2, 3.
    // The 6-bit codes b become the signed q = b - 32 per byte:
    // (b + 0x60) ^ 0x80 = b - 32 (mod 256) for 0 <= b <= 63, with no carry
    // between bytes.
    __device__ static long operand(const Frag &f, int j) {
        const int h = j >> 2, r = j & 3;
        const uint2 l = f.ql[h][r & 1], hb = f.qh[h];
        const int nsh = 4 * (r >> 1), hsh = 2 * r;
        const uint32_t b0 = ((l.x >> nsh) & 0x0f0f0f0fu) + (((hb.x >> hsh) & 0x03030303u) << 4) + 0x60606060u;
        const uint32_t b1 = ((l.y >> nsh) & 0x0f0f0f0fu) + (((hb.y >> hsh) & 0x03030303u) << 4) + 0x60606060u;
        return as_long(b0 ^ 0x80808080u, b1 ^ 0x80808080u);
    }
    // acc[t][e] += d * sum_j dx_j,e (sc_2j S0_j,e + sc_2j+1 S1_j,e); the group
    // sums are exact integers, d is applied once per unit.
    template <int RT>
    __device__ static void accumulate(const Frag (&f)[RT], const long (&a)[kGroups], const ScaleLds &sl, int g0,
                                      int q, int, float (&acc)[RT][4], v4f (&)[RT]) {
        const bool lo_quarter = q < 2;
        float u[RT][4];
#pragma unroll
        for (int t = 0; t < RT; ++t)
#pragma unroll
            for (int e = 0; e < 4; ++e) u[t][e] = 0.f;
        // Two MFMAs per group, one per 16-value sub-block (the lane quarters
        // holding the other sub-block pass zeros); pipelined as for Q4_K.
        v4i c0[RT], c1[RT];
        auto mm = [&](int j, v4i (&x0)[RT], v4i (&x1)[RT]) {
#pragma unroll
            for (int t = 0; t < RT; ++t) {
                const long b = operand(f[t], j);
                x0[t] = mfma32(a[j], lo_quarter ? b : 0l, v4i{0, 0, 0, 0});
                x1[t] = mfma32(a[j], lo_quarter ? 0l : b, v4i{0, 0, 0, 0});
            }
        };
        mm(0, c0, c1);
        float4 dx = sl.dx(g0, q);  // one group ahead, as for Q4_K
#pragma unroll
        for (int j = 0; j < kGroups; ++j) {
            v4i n0[RT], n1[RT];
            if (j + 1 < kGroups) mm(j + 1, n0, n1);
            const int h = j >> 2, r = j & 3;
            const float4 dxn = j + 1 < kGroups ? sl.dx(g0 + j + 1, q) : dx;
#pragma unroll
            for (int t = 0; t < RT; ++t) {
                const int s0 = sc_byte(f[t].sc, 8 * h + 2 * r), s1 = sc_byte(f[t].sc, 8 * h + 2 * r + 1);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int v = __mul24(s0, c0[t][e]) + __mul24(s1, c1[t][e]);
                    u[t][e] = fmaf(f4(dx, e), (float)v, u[t][e]);
                }
                if (j + 1 < kGroups) {
                    c0[t] = n0[t];
                    c1[t] = n1[t];
                }
            }
            dx = dxn;
            __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int t = 0; t < RT; ++t) {
            const float d = f16_bits_to_f32(f[t].d);
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[t][e] = fmaf(d, u[t][e], acc[t][e]);
        }
    }
};

// ------------------------------------------------------------------ Q8_0 --
struct MmaQ80 {
    static constexpr int kGroups = 4;  // blocks of 32 per TILED unit
    static constexpr int kUnitBytes = kQ80Unit;
    static constexpr bool kAux = false;
    __device__ static float stage_aux(float, uint32_t) { return 0.f; }
    struct Frag {
        uint2 qs[4];
        uint2 d;  // 4 f16 scales
    };
    __device__ static Frag load(const uint8_t *unit, int i, int q) {
        Frag f;
#pragma unroll
        for (int k = 0; k < 4; ++k) f.qs[k] = *(const uint2 *)(unit + 128 * i + 32 * k + 8 * q);
        f.d = *(const uint2 *)(unit + kQ80TD + 8 * i);
        return f;
    }
    template <int RT>
    __device__ static void accumulate(const Frag (&f)[RT], const long (&a)[kGroups], const ScaleLds &sl, int g0,
                                      int q, int, float (&acc)[RT][4], v4f (&)[RT]) {
#pragma unroll
        for (int j = 0; j < kGroups; ++j) {
            const float4 dx = sl.dx(g0 + j, q);
#pragma unroll
            for (int t = 0; t < RT; ++t) {
                const v4i c = mfma32(a[j], as_long(f[t].qs[j].x, f[t].qs[j].y), v4i{0, 0, 0, 0});
                const uint32_t dw2 = j < 2 ? f[t].d.x : f[t].d.y;
                const float dw = f16_bits_to_f32(dw2 >> (16 * (j & 1)));
#pragma unroll
                for (int e = 0; e < 4; ++e) acc[t][e] = fmaf(dw * f4(dx, e), (float)c[e], acc[t][e]);
            }
        }
    }
};

// ---------------------------------------------------------------- IQ4_XS --
// Group j of the block: lane quarter q holds positions 8 q .. 8 q + 7, the low
// nibbles of qs bytes 16 j + 8 q (q < 2) or the high nibbles of 16 j + 8 (q - 2)
// (q >= 2), through the 16-entry table; scale d (ls_j - 32) per group.
struct MmaIQ4XS {
    static constexpr int kGroups = 8;
    static constexpr int kUnitBytes = kIQ4XSUnit;
    static constexpr bool kAux = false;
    __device__ static float stage_aux(float, uint32_t) { return 0.f; }
    struct Frag {
        uint2 qs[8];  // 8 qs bytes of each group
        uint2 hd;     // d | scales_h << 16, scales_l[4]
    };
    __device__ static Frag load(const uint8_t *unit, int i, int q) {
        Frag f;
#pragma unroll
        for (int j = 0; j < 8; ++j) f.qs[j] = *(const uint2 *)(unit + 128 * i + 16 * j + 8 * (q & 1));
        f.hd = *(const uint2 *)(unit + kIQ4XSTHdr + 8 * i);
        return f;
    }
    template <int RT>
    __device__ static void accumulate(const Frag (&f)[RT], const long (&a)[kGroups], const ScaleLds &sl, int g0,
                                      int q, int, float (&acc)[RT][4], v4f (&)[RT]) {
        const int nsh = q < 2 ? 0 : 4;
#pragma unroll
        for (int j = 0; j < kGroups; ++j) {
            const float4 dx = sl.dx(g0 + j, q);
#pragma unroll
            for (int t = 0; t < RT; ++t) {
                const uint2 w = f[t].qs[j];
                const long b = as_long(iq4_lut((w.x >> nsh) & 0x0f0f0f0fu), iq4_lut((w.y >> nsh) & 0x0f0f0f0fu));
                const v4i c = mfma32(a[j], b, v4i{0, 0, 0, 0});
                const int ls = (int)(((f[t].hd.y >> (8 * (j >> 1) + 4 * (j & 1))) & 15u) |
                                     (((f[t].hd.x >> (16 + 2 * j)) & 3u) << 4)) - 32;
                const float dl = f16_bits_to_f32(f[t].hd.x) * (float)ls;
#pragma unroll
                for (int e = 0; e < 4; ++e) acc[t][e] = fmaf(dl * f4(dx, e), (float)c[e], acc[t][e]);
            }
        }
    }
};

// One unit (a K range of kGroups x 32) of activation operands.
template <class T>
struct ActUnit {
    long a[T::kGroups];
};

// KS waves split K; each wave covers RT 16-row tiles.  Up to kMaxMulti weights
// of one K share the launch (workgroups [wg_start[i], wg_start[i+1]) serve i).
template <class T, int KS, int RT>
__global__ __launch_bounds__(kWave *KS) void k_matmul_mfma(MatmulMultiParams p, int m0) {
    extern __shared__ __align__(16) uint8_t smem[];
    constexpr int G = T::kGroups;
    constexpr int TR = 16 * RT;  // weight rows per workgroup
    const int lane = (int)(threadIdx.x & 63), q = lane >> 4, r16 = lane & 15;
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    int mi = 0;
#pragma unroll
    for (int k = 1; k < kMaxMulti; ++k)
        if (k < p.nmat && (int)blockIdx.x >= p.wg_start[k]) mi = k;
    const uint8_t *Wm = p.W[mi];
    const int rc = p.rc[mi];
    const int M = min(p.M - m0, kMmaTok);
    const int ngroups = p.K / 32;
    const int gpad = p.upr * G;  // groups of whole units (Q8_0 units can pass K)
    const int ntiles8 = (rc + kTileRows - 1) / kTileRows;
    const int row0 = ((int)blockIdx.x - p.wg_start[mi]) * TR;

    // Activation scales, transposed to [group][16 tokens] (zeros past M and K),
    // and for Q4_K the min term's token factor in the same shape.
    float *dT = (float *)smem;
    float *aT = (float *)(smem + (size_t)gpad * kMmaTok * 4);
    // Loads issued kBatch at a time before any is used: a few L2 round trips
    // instead of one per entry.
    constexpr int kBatch = 8;
    for (int i0 = (int)threadIdx.x; i0 < gpad * kMmaTok; i0 += kBatch * KS * kWave) {
        float d[kBatch];
        uint32_t sw[kBatch];
#pragma unroll
        for (int b = 0; b < kBatch; ++b) {
            const int idx = i0 + b * KS * kWave;
            const int g = idx / kMmaTok, t = idx % kMmaTok;
            const bool in = idx < gpad * kMmaTok && t < M && g < ngroups;
            const size_t src = in ? (size_t)(m0 + t) * ngroups + g : 0;
            d[b] = p.xd[src];
            sw[b] = T::kAux ? p.xs[src] : 0u;
            if (!in) {
                d[b] = 0.f;
                sw[b] = 0u;
            }
        }
#pragma unroll
        for (int b = 0; b < kBatch; ++b) {
            const int idx = i0 + b * KS * kWave;
            if (idx < gpad * kMmaTok) {
                dT[idx] = d[b];
                if (T::kAux) aT[idx] = T::stage_aux(d[b], sw[b]);
            }
        }
    }
    const ScaleLds sl{dT, aT};
    float *red = (float *)(smem + (size_t)gpad * kMmaTok * (T::kAux ? 8 : 4));  // [KS][16 tokens][TR]
    __syncthreads();

    // This wave's K slice (units) and the lane's rows.
    const int U = p.upr / KS, rem = p.upr % KS;
    const int ub = wave * U + min(wave, rem);
    const int nu = U + (wave < rem ? 1 : 0);
    const uint8_t *unit0[RT];
    int irow[RT];
#pragma unroll
    for (int t = 0; t < RT; ++t) {
        const int row = row0 + 16 * t + r16;
        const int tt = min(row / kTileRows, ntiles8 - 1);  // rows past the end: reread the last tile
        unit0[t] = Wm + (size_t)tt * p.upr * T::kUnitBytes;
        irow[t] = row % kTileRows;
    }
    const bool tok_in = r16 < M;
    const int8_t *xrow = p.xq + (size_t)(m0 + (tok_in ? r16 : 0)) * p.K + 8 * q;

    // Unconditional loads and a bit mask (a select on the loaded value would be
    // turned into a branch around each load, with a wait inside it).
    const uint32_t tmask = tok_in ? 0xffffffffu : 0u;
    auto load_act = [&](ActUnit<T> &au, int u) {
#pragma unroll
        for (int j = 0; j < G; ++j) {
            const int g = u * G + j;
            const uint2 v = *(const uint2 *)(xrow + (size_t)min(g, ngroups - 1) * 32);
            const uint32_t msk = g < ngroups ? tmask : 0u;
            au.a[j] = as_long(v.x & msk, v.y & msk);
        }
    };
    auto load_w = [&](typename T::Frag (&f)[RT], int u) {
#pragma unroll
        for (int t = 0; t < RT; ++t) f[t] = T::load(unit0[t] + (size_t)u * T::kUnitBytes, irow[t], q);
    };

    float acc[RT][4];
    v4f cm[RT];  // Q4_K min term
#pragma unroll
    for (int t = 0; t < RT; ++t) {
        cm[t] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[t][e] = 0.f;
    }
    auto step = [&](const typename T::Frag (&f)[RT], const ActUnit<T> &x, int u) {
        T::template accumulate<RT>(f, x.a, sl, u * G, q, r16, acc, cm);
    };

    typename T::Frag fa[RT], fb[RT];
    ActUnit<T> xa, xb;
#ifdef M27Q_MFMA_STAGGER
    const int rot = nu > 0 ? (int)(blockIdx.x % (unsigned)nu) : 0;
#else
    const int rot = 0;
#endif
    auto uid = [&](int k) {
        const int v = k + rot;
        return ub + (v >= nu ? v - nu : v);
    };
    const int u_first = nu > 0 ? uid(0) : min(ub, p.upr - 1);
    load_w(fa, u_first);
    load_act(xa, u_first);
    int k = 0;
    for (; k + 2 < nu; k += 2) {
        load_w(fb, uid(k + 1));
        load_act(xb, uid(k + 1));
        step(fa, xa, uid(k));
        load_w(fa, uid(k + 2));
        load_act(xa, uid(k + 2));
        step(fb, xb, uid(k + 1));
    }
    if (k + 1 < nu) {
        load_w(fb, uid(k + 1));
        load_act(xb, uid(k + 1));
        step(fa, xa, uid(k));
        step(fb, xb, uid(k + 1));
    } else if (k < nu) {
        step(fa, xa, uid(k));
    }
    if (T::kAux) {
#pragma unroll
        for (int t = 0; t < RT; ++t)
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[t][e] -= cm[t][e];
    }

    // Partials of this wave's K slice -> LDS, then one thread per (token, row).
#pragma unroll
    for (int t = 0; t < RT; ++t)
#pragma unroll
        for (int e = 0; e < 4; ++e) red[((size_t)wave * kMmaTok + 4 * q + e) * TR + 16 * t + r16] = acc[t][e];
    __syncthreads();
    for (int idx = (int)threadIdx.x; idx < M * TR; idx += KS * kWave) {
        const int tok = idx / TR, rr = idx % TR, row = row0 + rr;
        float v = red[(size_t)tok * TR + rr];
#pragma unroll
        for (int w = 1; w < KS; ++w) v += red[((size_t)w * kMmaTok + tok) * TR + rr];
        if (row < rc) {
            const size_t o = (size_t)(m0 + tok) * rc + row;
            p.Y[mi][o] = v + (p.res[mi] ? p.res[mi][o] : 0.f);
        }
    }
}

template <class T, int KS, int RT>
static size_t mfma_lds(int upr) {
    return (size_t)upr * T::kGroups * kMmaTok * (T::kAux ? 8 : 4) + (size_t)KS * kMmaTok * 16 * RT * 4;
}

template <class T, int KS, int RT>
static hipError_t launch_mfma_t(MatmulMultiParams p, hipStream_t s) {
    const size_t lds = mfma_lds<T, KS, RT>(p.upr);
    int total = 0;
    for (int i = 0; i < p.nmat; ++i) {
        p.wg_start[i] = total;
        total += (p.rc[i] + 16 * RT - 1) / (16 * RT);
    }
    p.wg_start[p.nmat] = total;
    for (int m0 = 0; m0 < p.M; m0 += kMmaTok) {
        hipLaunchKernelGGL((k_matmul_mfma<T, KS, RT>), dim3(total), dim3(kWave * KS), lds, s, p, m0);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

// Launch shape: RT 16-row tiles per wave share each activation load and LDS
// scale read; K is split over KS waves so that a launch still has a few
// thousand waves.  KS * RT <= 16 keeps the LDS within the KS = 16, RT = 1 size
// the caller checks.
template <class T>
static hipError_t launch_mfma_cfg(const MatmulMultiParams &p, hipStream_t s) {
#if defined(M27Q_MFMA_KS) && defined(M27Q_MFMA_RT)
    static_assert(M27Q_MFMA_KS * M27Q_MFMA_RT <= 16, "LDS bound");
    return launch_mfma_t<T, M27Q_MFMA_KS, M27Q_MFMA_RT>(p, s);
#else
    // Measured on the Qwen-27B layer (M = 2 .. 16): (4, 2) for gate/up
    // (2176 tiles) and down (320 tiles, Q6_K), (8, 2) for q/k/v and o (512
    // and 320 tiles, Q4_K); RT = 4 runs at one wave per SIMD.
    long long tiles = 0;
    for (int i = 0; i < p.nmat; ++i) tiles += (p.rc[i] + 15) / 16;
    if (tiles >= 1024 || (std::is_same<T, MmaQ6K>::value && tiles >= 256)) return launch_mfma_t<T, 4, 2>(p, s);
    if (tiles >= 256) return launch_mfma_t<T, 8, 2>(p, s);
    return launch_mfma_t<T, 16, 1>(p, s);
#endif
}

size_t matmul_mfma_lds_bytes(uint32_t type, int upr) {
    switch (type) {
        case kQ4_K: return mfma_lds<MmaQ4K, 16, 1>(upr);
        case kQ5_K: return mfma_lds<MmaQ5K, 16, 1>(upr);
        case kQ6_K: return mfma_lds<MmaQ6K, 16, 1>(upr);
        case kQ8_0: return mfma_lds<MmaQ80, 16, 1>(upr);
        case kIQ4_XS: return mfma_lds<MmaIQ4XS, 16, 1>(upr);
        default: return 0;
    }
}

hipError_t launch_matmul_mfma(uint32_t type, const MatmulMultiParams &p, hipStream_t s) {
    switch (type) {
        case kQ4_K: return launch_mfma_cfg<MmaQ4K>(p, s);
        case kQ5_K: return launch_mfma_cfg<MmaQ5K>(p, s);
        case kQ6_K: return launch_mfma_cfg<MmaQ6K>(p, s);
        case kQ8_0: return launch_mfma_cfg<MmaQ80>(p, s);
        case kIQ4_XS: return launch_mfma_cfg<MmaIQ4XS>(p, s);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace m27q
