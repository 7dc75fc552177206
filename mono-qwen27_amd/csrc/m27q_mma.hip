// m27q_mma.hip -- small-M products Y[M][N] = X[M][K] W[N][K]^T on int8 MFMA.
//
// Every 32-weight group of a 16-row set and up to 16 tokens is one
// v_mfma_i32_16x16x32_i8, which gives the exact integer group sums for all
// token x row pairs; the scales are applied in fp32 afterwards, per group j,
// row r, token t:
//   Q4_K: d_r sc_rj dx_tj S_trj - dmin_r m_rj dx_tj sum(codes_tj)
//   Q6_K: d_r dx_tj (sc_r,2j S0_trj + sc_r,2j+1 S1_trj), the two 16-value
//         sub-blocks summed apart
//   Q8_0: d_rj dx_tj S_trj,   IQ4_XS: d_r (ls_rj - 32) dx_tj S_trj
// which are the per-group terms of the M = 1 products.
//
// Row packing.  The 16 x 16 output tile is 16 rows x 16 tokens, or, with the
// packing factor PK = 2, 32 rows x 8 tokens: the K positions of one MFMA are
// split between two row sets (lane quarters 0-1 hold rows 0-15, quarters 2-3
// rows 16-31), and the activation operand of a token column is zero in the
// quarters of the other row set.  Two MFMAs chained through the accumulator
// then cover the group for both sets.  The integer work is the same, but no
// lane spends scale arithmetic on padding tokens when M <= 8.
//
// Lane roles (v_mfma_i32_16x16x32_i8, layout checked on the device), with
// quarter q = lane / 16, column c = lane % 16, NQ = 4 / PK quarters per row
// set, set s = q / NQ, piece lane r = q % NQ:
//   B (weights):     lane holds row c + 16 s, the 8 positions 8 r + (32/PK) m
//                    of the group for MFMA m (Q4_K, Q5_K and Q8_0 at PK = 2:
//                    16 r + 8 m, see kPaired);
//   A (activations): lane holds token c % (16/PK) at the same positions, or
//                    zeros if c / (16/PK) != s;
//   C:               lane holds tokens 4 r .. 4 r + 3 of row c + 16 s.
// With PK = 2 each MFMA m covers positions 16 m .. 16 m + 15, which keeps
// the two Q6_K sub-blocks apart.
//
// Data movement.  The operand layouts above would need loads that each touch
// 16 rows (or 16 token rows K bytes apart); measured on gfx950, such loads
// stall in the L1 tag lookup and bound the kernel well below the HBM rate.
// So each wave streams its K slice one TILED unit at a time with 16-byte loads
// of contiguous bytes (the set's weight tiles, the tokens' codes and scales),
// issued while the previous unit computes, writes them to its own LDS area
// (padded row and token records, so the operand reads below are free of bank
// conflicts), and reads the MFMA operands from there.  TILED Q4_K / Q5_K
// weights skip that round trip (kDirect): their qs plane is stored chunk pair
// first, so the operand loads of 16 rows read whole 128-byte lines and go
// straight into registers.  The zero operand lanes read a zero record.  K is split over the KS waves of a
// workgroup, one row set per workgroup (two for one-set tiles, sharing the
// activation operands), and the KS partials are added in LDS in a fixed
// order.  Padding tokens (past M) read a real token's codes; their
// scales are zero and their outputs are dropped.  GGUF-layout Q4_K / Q5_K /
// Q6_K weights fill the same LDS records from each row's block of the unit
// (k_matmul_mfma's LAYOUT parameter).
//
// No reference counterpart: the reference runs prefill and decode one token at
// a time (src/mono27b_chat.cpp:399-403).
#include <algorithm>
#include <type_traits>

#include "m27q_internal.h"
#include "m27q_device.h"

namespace m27q {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef uint32_t v4u __attribute__((ext_vector_type(4)));  // staging registers (promoted; HIP's uint4 arrays are not)
typedef uint32_t v2u __attribute__((ext_vector_type(2)));

template <int PK>
struct Pack {
    static constexpr int NQ = 4 / PK;   // lane quarters per row set
    static constexpr int TK = 16 / PK;  // tokens per launch
    static constexpr int W8 = 32 / PK;  // position stride between a lane's pieces
    static_assert(PK == 1 || PK == 2, "row packing factor");
};

__device__ __forceinline__ long as_long(uint32_t lo, uint32_t hi) { return (long)(((uint64_t)hi << 32) | lo); }
__device__ __forceinline__ long as_long(uint2 v) { return as_long(v.x, v.y); }
__device__ __forceinline__ v4i mfma32(long a, long b, v4i c) {
    return __builtin_amdgcn_mfma_i32_16x16x32_i8(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ v4f mfma_f32(float a, float b, v4f c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ uint2 ld8(const void *p) { return *(const uint2 *)p; }
// Raw buffer loads (buf_rsrc, m27q_device.h).  AUX is the cache policy: 2
// marks the load non-temporal (buffer_load ... nt), the policy of the weight
// streams, which are read once per product.
template <int AUX = 0>
__device__ __forceinline__ v4u buf_ld16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    return __builtin_bit_cast(v4u, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, AUX));
}
template <int AUX = 0>
__device__ __forceinline__ v2u buf_ld8(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    return __builtin_bit_cast(v2u, __builtin_amdgcn_raw_buffer_load_b64(r, voff, soff, AUX));
}
// Measured on the layer's products at M = 4 / 8 / 16 (cold weights): 61.2 /
// 63.4 / 82.3 us per layer with non-temporal weight loads against 64.0 / 66.6
// / 83.6 without; sc0 or sc1 added nothing either way.
constexpr int kWeightAux = 2;
__device__ __forceinline__ int s_lo(uint32_t s) { return (int)(int16_t)(s & 0xffffu); }
__device__ __forceinline__ int s_hi(uint32_t s) { return (int)(int16_t)(s >> 16); }
__device__ __forceinline__ float f4(const float4 &v, int e) { return e == 0 ? v.x : e == 1 ? v.y : e == 2 ? v.z : v.w; }
// byte e (compile-time) of w as a float: v_cvt_f32_ubyte{0..3}
__device__ __forceinline__ float ubyte_f(uint32_t w, int e) { return (float)((w >> (8 * e)) & 0xffu); }

// Per-lane geometry.
template <int PK>
struct Lane {
    int q, c, s, r;
    __device__ explicit Lane(int lane) : q(lane >> 4), c(lane & 15), s(q / Pack<PK>::NQ), r(q % Pack<PK>::NQ) {}
};

// Activation scales in LDS, [group][TK tokens]; for Q4_K the min term's token
// factor in the same shape.
template <int PK>
struct ScaleLds {
    const float *dT, *aT;
    __device__ float4 dx(int g, int r) const { return *(const float4 *)(dT + g * Pack<PK>::TK + 4 * r); }
};

// Activation operands of one half unit: a[group][piece], NP pieces per group
// (the policy's kPieces: PK, or two zero-split views for Q6_K at PK = 1).
template <int NP>
struct AFrag {
    uint2 a[4][NP];
};

// Piece m of each group from base[m] (a token or zero record in LDS, the
// lane's position offset included).
template <int NP>
__device__ __forceinline__ void load_act(AFrag<NP> &f, const uint8_t *const (&base)[NP], int st) {
#pragma unroll
    for (int jg = 0; jg < 4; ++jg)
#pragma unroll
        for (int m = 0; m < NP; ++m) f.a[jg][m] = ld8(base[m] + 32 * (4 * st + jg));
}

// Paired pieces (a policy's kPaired at PK = 2): the lane's two pieces of a
// group are the adjacent positions 16 r .. 16 r + 15, read as one 16-byte LDS
// load.  Two 8-byte pieces 16 bytes apart issue as ds_read2_b64, which the
// LDS serves at half the rate of ds_read_b128 (measured on gfx950: 8 against
// 4 bank-conflict cycles per instruction for the same kilobyte).  The split
// of a group's 32 positions over lanes and MFMAs is free where one scale
// covers the group, as long as both operands follow it.
__device__ __forceinline__ void load_act_paired(AFrag<2> &f, const uint8_t *base, int st) {
#pragma unroll
    for (int jg = 0; jg < 4; ++jg) {
        const uint4 v = *(const uint4 *)(base + 32 * (4 * st + jg));
        f.a[jg][0] = make_uint2(v.x, v.y);
        f.a[jg][1] = make_uint2(v.z, v.w);
    }
}

// ------------------------------------------------------------ Q4_K, Q5_K --
// Q5_K is Q4_K with a fifth code bit per weight: bit j of qh[l] for position l
// of group j (exec:953-969), added to the operand bytes as 16.
template <bool Q5>
struct MmQ4KT {
    static constexpr int kGroups = 8, kSteps = 2;
    static constexpr int kUnitBytes = Q5 ? kQ5KUnit : kQ4KUnit;
    static constexpr bool kAux = true;
    // more live registers than 4 waves per SIMD allow at PK = 2 and in GGUF layout
    static constexpr bool kWide = Q5;
    static constexpr bool kPaired = true;
    static constexpr bool kDirect = true;  // TILED operands straight from memory
    template <int PK>
    static constexpr int kPieces = PK;
    // The min term's token factor: dx * (sum of the 32 codes).
    __device__ static float stage_aux(float d, uint32_t s) { return d * (float)(s_lo(s) + s_hi(s)); }
    template <int PK>
    struct Frag {
        uint2 qs[2][PK];  // the two 32-byte qs chunks of the half unit
        uint4 h;          // d | dmin, scales[12]
        uint2 qh[Q5 ? PK : 1];
    };
    // LDS row record: header 16 | qs 128 (| Q5_K qh 32).  Chunk c (16 bytes)
    // of the TILED unit of 8-row tile t goes to (qs chunk q = c - 8 of the
    // chunk-pair-first plane: row (q / 2) % 8, qs bytes 32 (q / 16) + 16 (q % 2)):
    static constexpr int kRowBytes = Q5 ? 176 : 144;
    __device__ static int lds_dst(int t, int c, int) {
        if (c < 8) return (8 * t + c) * kRowBytes;
        if (c < 72) {
            const int q = c - 8;
            return (8 * t + ((q >> 1) & 7)) * kRowBytes + 16 + 32 * (q >> 4) + 16 * (q & 1);
        }
        return (8 * t + ((c - 72) >> 1)) * kRowBytes + 144 + 16 * ((c - 72) & 1);  // Q5_K qh
    }
    // GGUF layout: a row's block of the unit is kGgufChunks 16-byte chunks
    // (Q4_K: header | qs, the record itself; Q5_K: header | qh | qs).
    static constexpr int kBlockBytes = Q5 ? kQ5KBytes : kQ4KBytes;
    static constexpr int kGgufChunks = kBlockBytes / 16;
    static constexpr bool kGgufA2 = false;  // blocks are 16-byte aligned
    __device__ static int gguf_dst(int j, int c) {
        if (!Q5 || c == 0) return j * kRowBytes + 16 * c;
        if (c < 3) return j * kRowBytes + 144 + 16 * (c - 1);  // qh
        return j * kRowBytes + 16 + 16 * (c - 3);                // qs
    }
    template <int PK>
    __device__ static void load(Frag<PK> &f, const uint8_t *wl, int row, int r, int st, int) {
        const uint8_t *rb = wl + row * kRowBytes;
        if constexpr (PK == 2) {  // paired pieces: bytes 16 r .. 16 r + 15
#pragma unroll
            for (int cc = 0; cc < 2; ++cc) {
                const uint4 v = *(const uint4 *)(rb + 16 + 64 * st + 32 * cc + 16 * r);
                f.qs[cc][0] = make_uint2(v.x, v.y);
                f.qs[cc][1] = make_uint2(v.z, v.w);
            }
        } else {
#pragma unroll
            for (int cc = 0; cc < 2; ++cc) f.qs[cc][0] = ld8(rb + 16 + 64 * st + 32 * cc + 8 * r);
        }
        f.h = *(const uint4 *)rb;
        if constexpr (Q5) {
            if constexpr (PK == 2) {
                const uint4 v = *(const uint4 *)(rb + 144 + 16 * r);
                f.qh[0] = make_uint2(v.x, v.y);
                f.qh[1] = make_uint2(v.z, v.w);
            } else {
                f.qh[0] = ld8(rb + 144 + 8 * r);
            }
        }
    }
    // TILED operands loaded straight into registers (kDirect): for the lane's
    // row i of its tile and piece lane r, the 8 PK qs bytes 8 PK r .. of each
    // chunk pair j (its pieces of groups 2 j and 2 j + 1), the row's header
    // and (Q5_K) qh bytes 8 PK r ..; the chunk-pair-first qs plane puts the
    // same bytes of a tile's 8 rows in one 256-byte run, so a wave's load
    // reads whole 128-byte lines.
    template <int PK>
    using DVec = typename std::conditional<PK == 2, v4u, v2u>::type;
    template <int PK>
    struct Direct {
        DVec<PK> q[4];
        v4u h;
        DVec<PK> qh[1];  // Q5_K only
    };
    template <int PK>
    __device__ static DVec<PK> dld(__amdgpu_buffer_rsrc_t rs, uint32_t voff, uint32_t soff) {
        if constexpr (PK == 2) return buf_ld16<kWeightAux>(rs, voff, soff);
        else return buf_ld8<kWeightAux>(rs, voff, soff);
    }
    template <int PK>
    __device__ static void load_direct(Direct<PK> &d, __amdgpu_buffer_rsrc_t rs, uint32_t tile_off, int i, int r,
                                       uint32_t soff) {
#pragma unroll
        for (int j = 0; j < 4; ++j) d.q[j] = dld<PK>(rs, tile_off + (uint32_t)(q4k_tqs(i, j) + 8 * PK * r), soff);
        d.h = buf_ld16<kWeightAux>(rs, tile_off + 16u * (uint32_t)i, soff);
        if constexpr (Q5) d.qh[0] = dld<PK>(rs, tile_off + (uint32_t)(kQ5KTQh + 32 * i + 8 * PK * r), soff);
    }
    // The half unit's fragment from those registers, as load() reads it from LDS.
    template <int PK>
    __device__ static void frag_direct(Frag<PK> &f, const Direct<PK> &d, int st) {
#pragma unroll
        for (int cc = 0; cc < 2; ++cc) {
            const DVec<PK> &v = d.q[2 * st + cc];
            f.qs[cc][0] = make_uint2(v[0], v[1]);
            if constexpr (PK == 2) f.qs[cc][1] = make_uint2(v[2], v[3]);
        }
        f.h = make_uint4(d.h.x, d.h.y, d.h.z, d.h.w);
        if constexpr (Q5) {
            f.qh[0] = make_uint2(d.qh[0][0], d.qh[0][1]);
            if constexpr (PK == 2) f.qh[1] = make_uint2(d.qh[0][2], d.qh[0][3]);
        }
    }
    template <int PK, int ST>
    __device__ static long operand(const Frag<PK> &f, int jg, int m) {
        const uint2 w = f.qs[jg >> 1][m];
        const int sh = 4 * (jg & 1);
        uint32_t lo = (w.x >> sh) & 0x0f0f0f0fu, hi = (w.y >> sh) & 0x0f0f0f0fu;
        if constexpr (Q5) {
            const int g = 4 * ST + jg;
            lo |= ((f.qh[m].x >> g) & 0x01010101u) << 4;
            hi |= ((f.qh[m].y >> g) & 0x01010101u) << 4;
        }
        return as_long(lo, hi);
    }
    template <int PK, int ST>
    __device__ static void mma(const Frag<PK> &f, const AFrag<PK> &a, int jg, const Lane<PK> &, v4i &S, v4i &) {
        S = mfma32(as_long(a.a[jg][0]), operand<PK, ST>(f, jg, 0), v4i{0, 0, 0, 0});
#pragma unroll
        for (int m = 1; m < PK; ++m) S = mfma32(as_long(a.a[jg][m]), operand<PK, ST>(f, jg, m), S);
    }
    // Per half unit: main-term group scales and the min term (an fp32 MFMA,
    // K = 4: NQ groups of each row set per MFMA).
    template <int PK, int ST>
    struct Half {
        float d;
        uint32_t scw;
        __device__ Half(const Frag<PK> &f, const ScaleLds<PK> &sl, int gu, const Lane<PK> &L, bool areal, int atok,
                        v4f &cm) {
            const uint4 h = f.h;
            d = f16_bits_to_f32(h.x);
            const float dmin = f16_bits_to_f32(h.x >> 16);
            // get_scale_min_k4 (exec:690-693) for the four groups of this half,
            // one byte each
            scw = ST == 0 ? (h.y & 0x3f3f3f3fu) : ((h.w & 0x0f0f0f0fu) | ((h.y >> 2) & 0x30303030u));
            const uint32_t mw = ST == 0 ? (h.z & 0x3f3f3f3fu) : (((h.w >> 4) & 0x0f0f0f0fu) | ((h.z >> 2) & 0x30303030u));
            constexpr int NQ = Pack<PK>::NQ, TK = Pack<PK>::TK;
#pragma unroll
            for (int n = 0; n < PK; ++n) {
                const int gl = NQ * n + L.r;  // group within the half, this lane's K index
                const float bm = dmin * (float)((mw >> (8 * gl)) & 0xffu);
                const float av = sl.aT[(gu + 4 * ST + gl) * TK + atok];
                cm = mfma_f32(areal ? av : 0.f, bm, cm);
            }
        }
        __device__ void scale(int jg, const float4 &dx, const v4i &S, const v4i &, float (&acc)[4], float (&)[4]) const {
            const float ws = d * ubyte_f(scw, jg);
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[e] = fmaf(ws, f4(dx, e) * (float)S[e], acc[e]);
        }
        __device__ void finish(float (&)[4], float (&)[4]) const {}
    };
};

using MmQ4K = MmQ4KT<false>;
using MmQ5K = MmQ4KT<true>;

// ------------------------------------------------------------------ Q6_K --
struct MmQ6K {
    static constexpr int kGroups = 8, kSteps = 2;
    static constexpr int kUnitBytes = kQ6KUnit;
    static constexpr bool kAux = false;
    // S0 and S1 each take the activations of one 16-value sub-block: at
    // PK = 1 two views of the group with the other half zero, at PK = 2 the
    // group's two pieces
    template <int PK>
    static constexpr int kPieces = 2;
    static constexpr bool kWide = true;
    static constexpr bool kPaired = false;  // MFMA m is sub-block m (its own scale)
    static constexpr bool kDirect = false;
    template <int PK>
    struct Direct {};
    __device__ static float stage_aux(float, uint32_t) { return 0.f; }
    template <int PK>
    struct Frag {
        uint2 ql[2][PK];  // [rr & 1][piece]: ql bytes 64 h + 32 (rr & 1) + ...
        uint2 qh[PK];     // qh bytes 32 h + ...
        uint2 sc;         // the half's 8 int8 scales
        uint32_t d;       // f16 bits
    };
    // LDS row record: ql 128 | qh 64 | scales 16 | pad 32; the eight d of a
    // tile in the side area (16 bytes per tile).
    static constexpr int kRowBytes = 240;
    __device__ static int lds_dst(int t, int c, int side) {
        if (c < 64) return (8 * t + (c >> 3)) * kRowBytes + 16 * (c & 7);
        if (c < 96) return (8 * t + ((c - 64) >> 2)) * kRowBytes + 128 + 16 * ((c - 64) & 3);
        if (c < 104) return (8 * t + (c - 96)) * kRowBytes + 192;
        return side + 16 * t;
    }
    // GGUF layout: ql | qh | scales are the block's first 13 chunks, in the
    // record's order; d (bytes 208-209) is staged apart into the side area.
    // The 210-byte blocks leave the chunks 2-byte aligned (kGgufA2).
    static constexpr int kBlockBytes = kQ6KBytes;
    static constexpr int kGgufChunks = 13;
    static constexpr bool kGgufA2 = true;
    __device__ static int gguf_dst(int j, int c) { return j * kRowBytes + 16 * c; }
    template <int PK>
    __device__ static void load(Frag<PK> &f, const uint8_t *wl, int row, int r, int st, int side) {
        constexpr int W8 = Pack<PK>::W8;
        const uint8_t *rb = wl + row * kRowBytes;
        const uint8_t *ql = rb + 64 * st + 8 * r;
        const uint8_t *qh = rb + 128 + 32 * st + 8 * r;
#pragma unroll
        for (int m = 0; m < PK; ++m) {
            f.ql[0][m] = ld8(ql + W8 * m);
            f.ql[1][m] = ld8(ql + 32 + W8 * m);
            f.qh[m] = ld8(qh + W8 * m);
        }
        f.sc = ld8(rb + 192 + 8 * st);
        f.d = *(const uint16_t *)(wl + side + 16 * (row >> 3) + 2 * (row & 7));
    }
    // Group rr of half h covers block positions 128 h + 32 rr .. + 31 (the
    // q6k_val index map, exec:1026-1048): low 4 bits from the ql bytes of
    // quarter rr & 1 (high nibbles for rr >= 2), high 2 bits at bit 2 rr of
    // the qh bytes.  The 6-bit codes b become the signed q = b - 32 per byte:
    // (b + 0x60) ^ 0x80 = b - 32 (mod 256) for 0 <= b <= 63, with no carry
    // between bytes.
    template <int PK>
    __device__ static long operand(const Frag<PK> &f, int rr, int m) {
        const uint2 l = f.ql[rr & 1][m], hb = f.qh[m];
        const int nsh = 4 * (rr >> 1), hsh = 2 * rr;
        const uint32_t b0 = ((l.x >> nsh) & 0x0f0f0f0fu) + (((hb.x >> hsh) & 0x03030303u) << 4) + 0x60606060u;
        const uint32_t b1 = ((l.y >> nsh) & 0x0f0f0f0fu) + (((hb.y >> hsh) & 0x03030303u) << 4) + 0x60606060u;
        return as_long(b0 ^ 0x80808080u, b1 ^ 0x80808080u);
    }
    // S0 / S1: the sums over the two 16-value sub-blocks.  PK = 1: quarters
    // 0-1 hold sub-block 0, so two MFMAs on the same weights, each with the
    // activation view whose other half reads the zero record; PK = 2: MFMA m
    // covers sub-block m.
    template <int PK, int ST>
    __device__ static void mma(const Frag<PK> &f, const AFrag<2> &a, int jg, const Lane<PK> &, v4i &S0, v4i &S1) {
        const long b0 = operand<PK>(f, jg, 0);
        const long b1 = PK == 1 ? b0 : operand<PK>(f, jg, PK - 1);
        S0 = mfma32(as_long(a.a[jg][0]), b0, v4i{0, 0, 0, 0});
        S1 = mfma32(as_long(a.a[jg][1]), b1, v4i{0, 0, 0, 0});
    }
    template <int PK, int ST>
    struct Half {
        uint2 sc;
        float d;
        __device__ Half(const Frag<PK> &f, const ScaleLds<PK> &, int, const Lane<PK> &, bool, int, v4f &)
            : sc(f.sc), d(f16_bits_to_f32(f.d)) {}
        // u += dx * (sc_2j S0 + sc_2j+1 S1): exact integers until the dx
        // product; d is applied once per unit.
        __device__ void scale(int rr, const float4 &dx, const v4i &S0, const v4i &S1, float (&)[4],
                              float (&u)[4]) const {
            const uint32_t w = rr < 2 ? sc.x : sc.y;
            const int s0 = (int)(int8_t)(w >> (16 * (rr & 1))), s1 = (int)(int8_t)(w >> (16 * (rr & 1) + 8));
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int v = __mul24(s0, S0[e]) + __mul24(s1, S1[e]);
                u[e] = fmaf(f4(dx, e), (float)v, u[e]);
            }
        }
        __device__ void finish(float (&acc)[4], float (&u)[4]) const {
            if constexpr (ST == 1) {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    acc[e] = fmaf(d, u[e], acc[e]);
                    u[e] = 0.f;
                }
            }
        }
    };
};

// ------------------------------------------------------------------ Q8_0 --
struct MmQ80 {
    static constexpr int kGroups = 4, kSteps = 1;  // four 32-blocks per TILED unit
    static constexpr int kUnitBytes = kQ80Unit;
    static constexpr bool kAux = false;
    static constexpr bool kWide = false;
    static constexpr bool kPaired = true;
    static constexpr bool kDirect = false;
    template <int PK>
    struct Direct {};
    // TILED only (34-byte GGUF blocks take the VALU kernel: matmul_mfma_takes)
    static constexpr int kBlockBytes = kQ80Bytes, kGgufChunks = 0;
    static constexpr bool kGgufA2 = false;
    __device__ static int gguf_dst(int, int) { return 0; }
    template <int PK>
    static constexpr int kPieces = PK;
    __device__ static float stage_aux(float, uint32_t) { return 0.f; }
    template <int PK>
    struct Frag {
        uint2 qs[4][PK];
        uint2 d;  // 4 f16 scales
    };
    // LDS row record: qs 128 | pad 16; the rows' d (8 bytes each) in the side
    // area, 64 bytes per tile.
    static constexpr int kRowBytes = 144;
    __device__ static int lds_dst(int t, int c, int side) {
        if (c < 64) return (8 * t + (c >> 3)) * kRowBytes + 16 * (c & 7);
        return side + 64 * t + 16 * (c - 64);
    }
    template <int PK>
    __device__ static void load(Frag<PK> &f, const uint8_t *wl, int row, int r, int, int side) {
        const uint8_t *rb = wl + row * kRowBytes;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            if constexpr (PK == 2) {  // paired pieces
                const uint4 v = *(const uint4 *)(rb + 32 * k + 16 * r);
                f.qs[k][0] = make_uint2(v.x, v.y);
                f.qs[k][1] = make_uint2(v.z, v.w);
            } else {
                f.qs[k][0] = ld8(rb + 32 * k + 8 * r);
            }
        }
        f.d = ld8(wl + side + 64 * (row >> 3) + 8 * (row & 7));
    }
    template <int PK, int ST>
    __device__ static void mma(const Frag<PK> &f, const AFrag<PK> &a, int jg, const Lane<PK> &, v4i &S, v4i &) {
        S = mfma32(as_long(a.a[jg][0]), as_long(f.qs[jg][0]), v4i{0, 0, 0, 0});
#pragma unroll
        for (int m = 1; m < PK; ++m) S = mfma32(as_long(a.a[jg][m]), as_long(f.qs[jg][m]), S);
    }
    template <int PK, int ST>
    struct Half {
        uint2 dw;
        __device__ Half(const Frag<PK> &f, const ScaleLds<PK> &, int, const Lane<PK> &, bool, int, v4f &) : dw(f.d) {}
        __device__ void scale(int k, const float4 &dx, const v4i &S, const v4i &, float (&acc)[4], float (&)[4]) const {
            const float d = f16_bits_to_f32((k < 2 ? dw.x : dw.y) >> (16 * (k & 1)));
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[e] = fmaf(d * f4(dx, e), (float)S[e], acc[e]);
        }
        __device__ void finish(float (&)[4], float (&)[4]) const {}
    };
};

// ---------------------------------------------------------------- IQ4_XS --
// Group j's 16 qs bytes hold positions l (low nibble) and l + 16 (high
// nibble) of byte l.  A lane's 8-position piece is the low or high nibbles of
// 8 consecutive bytes: PK = 1, quarter q: bytes 8 (q & 1), nibble q >> 1;
// PK = 2, piece m: bytes 8 r, nibble m.  Codes go through the 16-entry table;
// scale d (ls_j - 32) per group.
struct MmIQ4XS {
    static constexpr int kGroups = 8, kSteps = 2;
    static constexpr int kUnitBytes = kIQ4XSUnit;
    static constexpr bool kAux = false;
    static constexpr bool kWide = false;
    static constexpr bool kPaired = false;  // a piece is one nibble of 8 bytes
    static constexpr bool kDirect = false;
    template <int PK>
    struct Direct {};
    // TILED only (136-byte GGUF blocks take the VALU kernel: matmul_mfma_takes)
    static constexpr int kBlockBytes = kIQ4XSBytes, kGgufChunks = 0;
    static constexpr bool kGgufA2 = false;
    __device__ static int gguf_dst(int, int) { return 0; }
    template <int PK>
    static constexpr int kPieces = PK;
    __device__ static float stage_aux(float, uint32_t) { return 0.f; }
    template <int PK>
    struct Frag {
        uint2 qs[4];
        uint2 hd;  // d | scales_h << 16, scales_l[4]
        int nib;   // PK = 1: the lane's nibble
    };
    // LDS row record: qs 128 | pad 16; the rows' headers (8 bytes each) in
    // the side area, 64 bytes per tile.
    static constexpr int kRowBytes = 144;
    __device__ static int lds_dst(int t, int c, int side) {
        if (c < 64) return (8 * t + (c >> 3)) * kRowBytes + 16 * (c & 7);
        return side + 64 * t + 16 * (c - 64);
    }
    template <int PK>
    __device__ static void load(Frag<PK> &f, const uint8_t *wl, int row, int r, int st, int side) {
        // PK = 1: r = q; bytes 8 (q & 1); PK = 2: bytes 8 r
        const int boff = PK == 1 ? 8 * (r & 1) : 8 * r;
        const uint8_t *rb = wl + row * kRowBytes;
#pragma unroll
        for (int jg = 0; jg < 4; ++jg) f.qs[jg] = ld8(rb + 16 * (4 * st + jg) + boff);
        f.hd = ld8(wl + side + 64 * (row >> 3) + 8 * (row & 7));
        f.nib = PK == 1 ? 4 * (r >> 1) : 0;
    }
    template <int PK>
    __device__ static long operand(const Frag<PK> &f, int jg, int m) {
        const int sh = PK == 1 ? f.nib : 4 * m;
        const uint2 w = f.qs[jg];
        return as_long(iq4_lut((w.x >> sh) & 0x0f0f0f0fu), iq4_lut((w.y >> sh) & 0x0f0f0f0fu));
    }
    template <int PK, int ST>
    __device__ static void mma(const Frag<PK> &f, const AFrag<PK> &a, int jg, const Lane<PK> &, v4i &S, v4i &) {
        S = mfma32(as_long(a.a[jg][0]), operand<PK>(f, jg, 0), v4i{0, 0, 0, 0});
#pragma unroll
        for (int m = 1; m < PK; ++m) S = mfma32(as_long(a.a[jg][m]), operand<PK>(f, jg, m), S);
    }
    template <int PK, int ST>
    struct Half {
        uint2 hd;
        __device__ Half(const Frag<PK> &f, const ScaleLds<PK> &, int, const Lane<PK> &, bool, int, v4f &) : hd(f.hd) {}
        __device__ void scale(int jg, const float4 &dx, const v4i &S, const v4i &, float (&acc)[4], float (&)[4]) const {
            const int j = 4 * ST + jg;
            const int ls = (int)(((hd.y >> (8 * (j >> 1) + 4 * (j & 1))) & 15u) | (((hd.x >> (16 + 2 * j)) & 3u) << 4)) - 32;
            const float dl = f16_bits_to_f32(hd.x) * (float)ls;
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[e] = fmaf(dl * f4(dx, e), (float)S[e], acc[e]);
        }
        __device__ void finish(float (&)[4], float (&)[4]) const {}
    };
};

template <int V>
struct IntTag {
    static constexpr int value = V;
};

// One half unit: the four groups' MFMAs, each issued one group ahead of the
// previous group's scale arithmetic.
template <class T, int PK, int ST>
__device__ __forceinline__ void compute_half(const typename T::template Frag<PK> &f,
                                             const AFrag<T::template kPieces<PK>> &a,
                                             const ScaleLds<PK> &sl, int gu, const Lane<PK> &L, bool areal, int atok,
                                             float (&acc)[4], float (&u)[4], v4f &cm) {
    const typename T::template Half<PK, ST> hs(f, sl, gu, L, areal, atok, cm);
    v4i S0, S1;
    T::template mma<PK, ST>(f, a, 0, L, S0, S1);
    float4 dx = sl.dx(gu + 4 * ST, L.r);
#pragma unroll
    for (int jg = 0; jg < 4; ++jg) {
        v4i N0, N1;
        float4 dxn = dx;
        if (jg + 1 < 4) {
            T::template mma<PK, ST>(f, a, jg + 1, L, N0, N1);
            dxn = sl.dx(gu + 4 * ST + jg + 1, L.r);
        }
        hs.scale(jg, dx, S0, S1, acc, u);
        if (jg + 1 < 4) {
            S0 = N0;
            S1 = N1;
        }
        dx = dxn;
        __builtin_amdgcn_sched_barrier(0);
    }
    hs.finish(acc, u);
}

// Per-wave LDS staging area for one unit (bytes):
//   W: 16 PK RS row records of T::kRowBytes (RS row sets per workgroup), then
//      a side area (64 bytes per tile); none where the weight operands are
//      loaded straight into registers (DW)
//   A: TK token records of 32 G + 16 bytes (G groups of codes + pad), then,
//      for PK = 2 (and Q6_K's zero-split views), one record of zeros for the
//      operand lanes of the other set (or sub-block)
//   S: dT [G][TK] and, for Q4_K, aT [G][TK] floats
//   a 16-byte slot that absorbs the writes of lanes past the data
// The paddings keep the MFMA-layout reads free of bank conflicts: the row
// strides 144, 176, 240 and the token strides 272, 144 put the 16 rows (or
// tokens) of a half wave on distinct 4-bank groups.
template <class T, int PK, int RS = 1, bool DW = false>
struct Stage {
    static constexpr int G = T::kGroups, TK = Pack<PK>::TK, UE = 32 * G, UB = T::kUnitBytes;
    static constexpr int kSide = DW ? 0 : 16 * PK * RS * T::kRowBytes;
    static constexpr int kW = DW ? 0 : kSide + 2 * PK * RS * 64;
    static constexpr int kARow = UE + 16;
    static constexpr int oA = kW;
    static constexpr int oZero = oA + TK * kARow;
    static constexpr bool kZeroRec = PK == 2 || T::template kPieces<PK> != PK;
    static constexpr int oS = oZero + (kZeroRec ? UE : 0);
    static constexpr int oDummy = oS + G * TK * 4 * (T::kAux ? 2 : 1);
    static constexpr int kBytes = (oDummy + 16 + 15) / 16 * 16;
    static constexpr int kWChunks = DW ? 0 : 2 * PK * RS * UB / 16;  // 16-byte chunks of the sets' unit
    static constexpr int kNW = (kWChunks + kWave - 1) / kWave;
    static constexpr int kNWR = kNW > 0 ? kNW : 1;  // staging register arrays
    static constexpr int kAChunks = TK * UE / 16;
    static constexpr int kNA = (kAChunks + kWave - 1) / kWave;
    static constexpr int kSLanes = TK * G / 4;  // lanes staging 4 scales each
    static_assert(kSLanes <= kWave, "scale staging lanes");
    static_assert(kAChunks % kWave == 0, "whole activation staging rounds");
    static_assert(UB % 16 == 0 && kARow % 16 == 0 && T::kRowBytes % 16 == 0, "16-byte staging");
    static_assert(kBytes >= RS * 4 * kWave * 4, "the partial sums fit the wave areas");
};

// One workgroup: RS row sets of 16 PK rows of one matrix (RS = 2 only with
// PK = 1), K split over the KS waves.  Each wave streams its K slice one unit
// at a time: 16-byte loads of the unit's weight tiles, activation codes and
// scales into registers (issued while the previous unit computes), written to
// the wave's LDS area, read back in the MFMA operand layout.  Up to kMaxMulti
// weights of one K share the launch (workgroups [wg_start[i], wg_start[i+1])
// serve i).
// Waves per SIMD the register budget is cut for, the most that compiles
// without spills (128 VGPRs for 4): 4, but 3 for the two-set Q5_K and Q6_K
// kernels, for GGUF-layout Q5_K / Q6_K and for Q4_K / Q5_K / Q6_K with two
// row sets per workgroup, and 2 for GGUF-layout Q6_K with two row sets (185
// VGPRs with its shifted chunk loads; its 8-wave launches take 104 KB of LDS,
// so one workgroup per CU runs 2 waves per SIMD in any case).  With direct
// operands (TILED Q4_K / Q5_K: the current and the next unit's weights in
// registers) 3, and 2 for Q5_K with two row sets (187 VGPRs); at 4 the
// two-set Q4_K kernel spilled 100 bytes per lane.
template <class T, int PK, int LAYOUT, int RS>
constexpr int mm_waves_per_eu() {
    if (LAYOUT == M27Q_LAYOUT_GGUF && T::kGgufA2 && RS == 2) return 2;
    if (LAYOUT == M27Q_LAYOUT_TILED && T::kDirect) return T::kWide && RS == 2 ? 2 : 3;
    return (T::kWide || (RS == 2 && T::kAux)) && (PK == 2 || RS == 2 || LAYOUT == M27Q_LAYOUT_GGUF) ? 3 : 4;
}
// GGUF-layout weights (LAYOUT == M27Q_LAYOUT_GGUF; Q4_K, Q5_K and Q6_K): the
// same LDS records, staged from each row's block of the unit (row_blocks ==
// units per row for these types).  Rows past the matrix's end reread its last
// row.  Temporal loads: a row's consecutive blocks share 128-byte lines.
// Q6_K's 2-byte-aligned chunks are read as 20 bytes from the 4-aligned offset
// below them and shifted into place; every read is inside the buffer's range
// or, past it, a buffer load that returns zeros.
template <int AUX>
__device__ __forceinline__ uint32_t buf_ld4(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    return bld_u32<AUX>(r, voff, soff);
}
__device__ __forceinline__ v4u shift16(const v4u &v, uint32_t e, uint32_t sh) {
    return v4u{__builtin_amdgcn_alignbit(v.y, v.x, sh), __builtin_amdgcn_alignbit(v.z, v.y, sh),
               __builtin_amdgcn_alignbit(v.w, v.z, sh), __builtin_amdgcn_alignbit(e, v.w, sh)};
}

template <class T, int PK, int KS, int LAYOUT, int RS>
__global__ __launch_bounds__(kWave *KS, (mm_waves_per_eu<T, PK, LAYOUT, RS>())) void k_matmul_mfma(
    MatmulMultiParams p, int m0) {
    extern __shared__ __align__(16) uint8_t smem[];
    constexpr bool kG = LAYOUT == M27Q_LAYOUT_GGUF;
    constexpr bool kD = !kG && T::kDirect;  // TILED weight operands straight into registers
    using SG = Stage<T, PK, RS, kD>;
    constexpr int SR = 16 * PK * RS;  // rows of the workgroup
    static_assert(RS == 1 || PK == 1, "two row sets per workgroup only with one-set tiles");
    static_assert(!kG || SR * T::kGgufChunks <= SG::kNW * kWave, "GGUF chunks fit the staging registers");
    constexpr int G = T::kGroups, NS = T::kSteps, TK = Pack<PK>::TK, UE = SG::UE, UB = SG::UB;
    constexpr int CPU = UB / 16;  // chunks per tile unit
    const int lane = (int)(threadIdx.x & 63);
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const Lane<PK> L(lane);
    int mi = 0;
#pragma unroll
    for (int k = 1; k < kMaxMulti; ++k)
        if (k < p.nmat && (int)blockIdx.x >= p.wg_start[k]) mi = k;
    const uint8_t *Wm = p.W[mi];
    const int rc = p.rc[mi];
    const int Mloc = min(p.M - m0, TK);
    const int ngroups = p.K / 32;
    const int ntiles8 = (rc + kTileRows - 1) / kTileRows;
    const int row0 = ((int)blockIdx.x - p.wg_start[mi]) * SR;
    uint8_t *wl = smem + (size_t)wave * SG::kBytes;

    // This wave's K slice (units).
    const int U = p.upr / KS, rem = p.upr % KS;
    const int ub = wave * U + min(wave, rem);
    const int nu = U + (wave < rem ? 1 : 0);

    // Staging map of this lane: weight chunks (tiles past the end reread the
    // last tile), activation chunks (padding tokens read token m0), scales.
    // 32-bit lane offsets into buffer descriptors, the unit's offset in a
    // scalar register (a TILED matrix is below 4 GiB: the host checks it).
    // Reads past the activation codes (the last Q8_0 unit past K) return
    // zeros; their groups have zero scales.
    uint32_t goff[SG::kNWR];
    int wdst[SG::kNWR];
    constexpr int UBW = kG ? T::kBlockBytes : UB;  // weight bytes of one unit per tile (GGUF: per row)
    const uint32_t rowb = (uint32_t)p.upr * (uint32_t)T::kBlockBytes;  // GGUF row bytes
#pragma unroll
    for (int n = 0; n < SG::kNW; ++n) {
        const int id = n * kWave + lane;
        if constexpr (kG) {
            const bool ok = id < SR * T::kGgufChunks;
            const int j = ok ? id / T::kGgufChunks : 0, c = ok ? id % T::kGgufChunks : 0;
            goff[n] = (uint32_t)min(row0 + j, rc - 1) * rowb + 16u * c;
            wdst[n] = ok ? T::gguf_dst(j, c) : SG::oDummy;
        } else {
            const bool ok = id < SG::kWChunks;
            int t = ok ? id / CPU : 0, c = ok ? id % CPU : 0;
            if constexpr (std::is_same<T, MmQ6K>::value) {
                // Q6_K's 240-byte records: each 16-lane pass of the staging
                // writes takes rows whose records fall on distinct banks (the
                // same row of two adjacent tiles for ql, rows i, i + 4 of two
                // tiles for qh), 8 or 4 lanes still reading a row's whole
                // 128 / 64 bytes.  Down at M = 4: 20.6 us against 21.2 with
                // consecutive chunks.
                constexpr int NT = SG::kWChunks / CPU;
                if (ok && id < 64 * NT) {
                    const int pp = id >> 4, j = id & 15;
                    t = 2 * (pp >> 3) + (j >> 3);
                    c = 8 * (pp & 7) + (j & 7);
                } else if (ok && id < 96 * NT) {
                    const int q = id - 64 * NT, pp = q >> 4, j = q & 15, sub = j >> 2;
                    t = 2 * (pp >> 2) + (sub >> 1);
                    c = 64 + 4 * ((pp & 3) + 4 * (sub & 1)) + (j & 3);
                } else if (ok) {
                    const int q = id - 96 * NT;
                    t = q / 9;
                    c = 96 + q % 9;
                }
            }
            const int tile = min(row0 / kTileRows + t, ntiles8 - 1);
            goff[n] = (uint32_t)tile * (uint32_t)(p.upr * UB) + 16u * c;
            wdst[n] = ok ? T::lds_dst(t, c, SG::kSide) : SG::oDummy;
        }
    }
    // GGUF Q6_K (2-byte aligned base): the descriptor starts at the 4-aligned
    // address at or below the matrix (inside its allocation, whose start is
    // 256-byte aligned), and every offset carries the base's low bits, so
    // the dword reads and shifts follow the absolute addresses.
    const uint32_t blo = kG && T::kGgufA2 ? (uint32_t)((uintptr_t)Wm & 3u) : 0u;
    // GGUF Q6_K: lanes 0 .. SR - 1 stage the d of row `lane` of the sets
    const uint32_t doff = blo + (uint32_t)min(row0 + (lane & (SR - 1)), rc - 1) * rowb + (uint32_t)kQ6KD;
    const int ddst = lane < SR ? SG::kSide + 16 * (lane >> 3) + 2 * (lane & 7) : SG::oDummy;
    uint32_t aoff[SG::kNA];
    int adst[SG::kNA];
#pragma unroll
    for (int n = 0; n < SG::kNA; ++n) {
        const int id = n * kWave + lane;
        const int tok = id / (UE / 16), c = id % (UE / 16);
        aoff[n] = (uint32_t)(m0 + (tok < Mloc ? tok : 0)) * (uint32_t)p.K + 16u * c;
        adst[n] = SG::oA + tok * SG::kARow + 16 * c;
    }
    const int s_tok = lane / (G / 4), s_h = lane % (G / 4);
    const bool s_on = lane < SG::kSLanes;
    const bool s_tok_in = s_on && s_tok < Mloc;
    const uint32_t s_row = (uint32_t)(m0 + (s_tok_in ? s_tok : 0)) * (uint32_t)ngroups + 4u * s_h;

    const __amdgpu_buffer_rsrc_t wr = buf_rsrc(Wm - blo, kG ? blo + (uint32_t)rc * rowb
                                                             : (uint32_t)ntiles8 * (uint32_t)(p.upr * UB));
    const __amdgpu_buffer_rsrc_t xr = buf_rsrc(p.xq, (uint32_t)p.M * (uint32_t)p.K);
    const uint32_t sbytes = (uint32_t)p.M * (uint32_t)ngroups * 4u;
    const __amdgpu_buffer_rsrc_t dr = buf_rsrc(p.xd, sbytes), sr = buf_rsrc(p.xs, sbytes);
    constexpr bool kA2 = kG && T::kGgufA2;
    v4u rw[SG::kNWR], ra[SG::kNA];
    uint32_t re[kA2 ? SG::kNW : 1], rsh[kA2 ? SG::kNW : 1], rd = 0u;
    float sd[4];
    uint32_t ss[4] = {0u, 0u, 0u, 0u};
    auto issue = [&](int u) __attribute__((always_inline)) {
        if constexpr (kA2) {
#pragma unroll
            for (int n = 0; n < SG::kNW; ++n) {
                const uint32_t v = blo + goff[n] + (uint32_t)u * UBW, a = v & ~3u;
                rw[n] = buf_ld16(wr, a, 0u);
                re[n] = buf_ld4<0>(wr, a + 16u, 0u);
                rsh[n] = (v & 2u) * 8u;
            }
            rd = bld_u16(wr, doff, (uint32_t)u * UBW);
        } else {
#pragma unroll
            for (int n = 0; n < SG::kNW; ++n) rw[n] = buf_ld16<kG ? 0 : kWeightAux>(wr, goff[n], (uint32_t)u * UBW);
        }
#pragma unroll
        for (int n = 0; n < SG::kNA; ++n) ra[n] = buf_ld16(xr, aoff[n], (uint32_t)u * UE);
        if constexpr (G == 8) {  // whole units: rows of 8 k groups, 16-byte aligned
            const v4u d = buf_ld16(dr, 4u * s_row, (uint32_t)u * (4 * G));
            sd[0] = __uint_as_float(d.x);
            sd[1] = __uint_as_float(d.y);
            sd[2] = __uint_as_float(d.z);
            sd[3] = __uint_as_float(d.w);
            if constexpr (T::kAux) {
                const v4u v = buf_ld16(sr, 4u * s_row, (uint32_t)u * (4 * G));
                ss[0] = v.x;
                ss[1] = v.y;
                ss[2] = v.z;
                ss[3] = v.w;
            }
        } else {  // Q8_0: the last unit can pass K
#pragma unroll
            for (int e = 0; e < 4; ++e) sd[e] = p.xd[s_row + min(u * G + e, ngroups - 1)];  // s_h = 0
        }
    };
    auto commit = [&](int u) __attribute__((always_inline)) {
        if constexpr (kA2) {
#pragma unroll
            for (int n = 0; n < SG::kNW; ++n) *(v4u *)(wl + wdst[n]) = shift16(rw[n], re[n], rsh[n]);
            *(uint16_t *)(wl + ddst) = (uint16_t)rd;
        } else {
#pragma unroll
            for (int n = 0; n < SG::kNW; ++n) *(v4u *)(wl + wdst[n]) = rw[n];
        }
#pragma unroll
        for (int n = 0; n < SG::kNA; ++n) *(v4u *)(wl + adst[n]) = ra[n];
        float *dT = (float *)(wl + SG::oS), *aT = dT + G * TK;
        float *dummy = (float *)(wl + SG::oDummy);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int g = 4 * s_h + e;
            const bool in = s_tok_in && (G == 8 || u * G + g < ngroups);  // K-quant units are whole
            *(s_on ? dT + g * TK + s_tok : dummy) = in ? sd[e] : 0.f;
            if constexpr (T::kAux) *(s_on ? aT + g * TK + s_tok : dummy + 1) = in ? T::stage_aux(sd[e], ss[e]) : 0.f;
        }
    };

    // The lane's weight row within the set and its activation record: token
    // c % TK of row set c / TK, the zero record for the other set.
    const int wrow = L.c + 16 * L.s;
    const bool areal = L.c / TK == L.s;
    const int atok = L.c % TK;
    constexpr bool kPair = PK == 2 && T::kPaired;  // paired pieces: positions 16 r + 8 m
    const uint8_t *ar = wl + (areal ? SG::oA + atok * SG::kARow : SG::oZero) + (kPair ? 16 : 8) * L.r;
    constexpr int NP = T::template kPieces<PK>;
    const uint8_t *ab[NP];
    if constexpr (NP == PK) {
#pragma unroll
        for (int m = 0; m < NP; ++m) ab[m] = ar + Pack<PK>::W8 * m;
    } else {  // Q6_K at PK = 1: quarters 0-1 (sub-block 0) and 2-3 (sub-block 1)
        static_assert(PK == 1 && NP == 2, "zero-split activation views");
        const uint8_t *z = wl + SG::oZero + 8 * L.r;
        ab[0] = L.q < 2 ? ar : z;
        ab[1] = L.q < 2 ? z : ar;
    }
    if constexpr (SG::kZeroRec) {
        if (lane < UE / 16) *(uint4 *)(wl + SG::oZero + 16 * lane) = make_uint4(0u, 0u, 0u, 0u);
    }
    const ScaleLds<PK> sl{(const float *)(wl + SG::oS), (const float *)(wl + SG::oS) + G * TK};

    // Direct operands: row set r's row of this lane (rows past the matrix
    // reread the last tile; their outputs are dropped), as the tile's offset
    // and the row within it.
    uint32_t dtile[RS];
    int drow[RS];
#pragma unroll
    for (int r = 0; r < RS; ++r) {
        const int R = row0 + wrow + 16 * r;
        dtile[r] = (uint32_t)min(R / kTileRows, ntiles8 - 1) * (uint32_t)(p.upr * UB);
        drow[r] = R % kTileRows;
    }
    typename T::template Direct<PK> dc[RS], dn[RS];
    auto dload = [&](int u, typename T::template Direct<PK>(&d)[RS]) __attribute__((always_inline)) {
        if constexpr (kD) {
#pragma unroll
            for (int r = 0; r < RS; ++r) T::template load_direct<PK>(d[r], wr, dtile[r], drow[r], L.r, (uint32_t)u * UB);
        }
    };

    float acc[RS][4], u4[RS][4];
    v4f cm[RS];  // Q4_K min term
#pragma unroll
    for (int r = 0; r < RS; ++r) {
        cm[r] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[r][e] = u4[r][e] = 0.f;
    }
    // One half unit at a time: its operands are read from LDS just before
    // its MFMAs, so only one half's fragments are live (the two-set Q4_K
    // kernel 129 VGPRs against 155 with both halves read first).  With RS = 2
    // the half's activation operands serve both row sets.
    auto half = [&](auto st) __attribute__((always_inline)) {
        constexpr int ST = decltype(st)::value;
        AFrag<NP> x;
        if constexpr (kPair)
            load_act_paired(x, ar, ST);
        else
            load_act<NP>(x, ab, ST);
#pragma unroll
        for (int r = 0; r < RS; ++r) {
            typename T::template Frag<PK> f;
            if constexpr (kD)
                T::template frag_direct<PK>(f, dc[r], ST);
            else
                T::template load<PK>(f, wl, wrow + 16 * r, L.r, ST, SG::kSide);
            compute_half<T, PK, ST>(f, x, sl, 0, L, areal, atok, acc[r], u4[r], cm[r]);
            if (r + 1 < RS) __builtin_amdgcn_sched_barrier(0);
        }
    };
    auto compute = [&]() __attribute__((always_inline)) {
        half(IntTag<0>{});
        if constexpr (NS == 2) {
            __builtin_amdgcn_sched_barrier(0);
            half(IntTag<1>{});
        }
    };
    // Loads are unconditional inside the loop (a conditional reload makes the
    // compiler wait for every load before each use); the last unit is peeled.
    // A wave's LDS reads and writes are executed in order, so a unit's
    // staging writes follow the previous unit's operand reads.
    // Direct operands: the next unit's weights are loaded after its
    // activations, so the staging writes wait only for the activations.
    if (nu > 0) {
        issue(ub);
        dload(ub, dc);
        commit(ub);
        for (int k = 0; k + 1 < nu; ++k) {
            issue(ub + k + 1);
            dload(ub + k + 1, dn);
            compute();
            commit(ub + k + 1);
            if constexpr (kD) {
#pragma unroll
                for (int r = 0; r < RS; ++r) dc[r] = dn[r];
            }
        }
        compute();
    }
    if (T::kAux) {
#pragma unroll
        for (int r = 0; r < RS; ++r)
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[r][e] -= cm[r][e];
    }

    // Partials of this wave's K slice -> LDS (over the staging areas), then
    // one thread per (set, lane, e) adds the KS waves in a fixed order.
    __syncthreads();
    float *red = (float *)smem;  // [KS][RS][4][64]
#pragma unroll
    for (int r = 0; r < RS; ++r)
#pragma unroll
        for (int e = 0; e < 4; ++e) red[((wave * RS + r) * 4 + e) * kWave + lane] = acc[r][e];
    __syncthreads();
    for (int idx = (int)threadIdx.x; idx < RS * 4 * kWave; idx += KS * kWave) {
        const int r = idx / (4 * kWave), e = idx / kWave % 4, ln = idx % kWave;
        float v = red[idx];
#pragma unroll
        for (int w = 1; w < KS; ++w) v += red[((w * RS + r) * 4 + e) * kWave + ln];
        const Lane<PK> O(ln);
        const int row = row0 + 16 * r + O.c + 16 * O.s, tok = 4 * O.r + e;
        if (row < rc && tok < Mloc) {
            const size_t o = (size_t)(m0 + tok) * rc + row;
            p.Y[mi][o] = v + (p.res[mi] ? p.res[mi][o] : 0.f);
        }
    }
}

// ------------------------------------------- resident activation rows --
// One-set tiles (16 tokens) over many row sets.  The kernel above re-stages
// every unit's 16 activation rows in each wave (4.4 KB per unit against
// 2.3 KB of Q4_K weights for 16 rows); here each workgroup stages the M x K
// activation codes and scales into LDS once and then streams its share of the
// row sets' weights through per-wave staging areas as above (TILED Q4_K /
// Q5_K: straight into registers, as above).
//
// LDS: TK token records of Kp + 16 bytes (Kp = the units' K; the 16-byte pad
// keeps the token stride at 16 mod 128 bytes, as the per-unit records'), a
// zero record (Q6_K's zero-split views), dT [Kp/32][TK] and, for Q4_K / Q5_K,
// aT [Kp/32][TK] floats, then one area per wave (the unit's weight records and
// side area, later its two partial sums).
//
// Work: workgroup g of G takes row sets [S g / G, S (g + 1) / G) of the S sets
// of all matrices; its units (set, k unit) in order are split into NWV
// contiguous runs, one per wave.  The host keeps the sets per workgroup at
// most NWV, so a run has at most upr units and covers at most two sets: the
// wave keeps the first set's sums in registers while it accumulates the
// second.  At the end each set's sums are added over the waves that covered
// it, in wave order.
template <class T>
struct XStage {
    using SG = Stage<T, 1>;
    static constexpr int G = T::kGroups, TK = 16, UE = SG::UE, UB = SG::UB;
    static constexpr int kWaveBytes = (SG::kW + 16 + 15) / 16 * 16;  // weights, side area, dummy slot
    static constexpr int oDummy = SG::kW;
    static_assert(kWaveBytes >= 2 * 4 * kWave * 4, "two partial-sum slots per wave area");
    static constexpr int xrow(int upr) { return upr * UE + 16; }
    static constexpr int oZero(int upr) { return TK * xrow(upr); }
    static constexpr int oDT(int upr) { return oZero(upr) + UE; }
    static constexpr int oAT(int upr) { return oDT(upr) + upr * G * TK * 4; }
    static constexpr int oWaves(int upr) { return (oAT(upr) + (T::kAux ? upr * G * TK * 4 : 0) + 15) / 16 * 16; }
    static constexpr size_t bytes(int upr, int nwv) { return (size_t)oWaves(upr) + (size_t)nwv * kWaveBytes; }
};

// 16-byte activation chunks each thread has in flight while staging: 16
// tokens x 6144 codes / 1024 threads in one round.
constexpr int kXBatch = 6;
template <class T, int NWV, int LAYOUT>
__global__ __launch_bounds__(kWave *NWV, 1) void k_matmul_mfma_xres(MatmulMultiParams p, int m0) {
    extern __shared__ __align__(16) uint8_t smem[];
    using XS = XStage<T>;
    using SG = typename XS::SG;
    constexpr bool kG = LAYOUT == M27Q_LAYOUT_GGUF;  // as in k_matmul_mfma
    constexpr bool kD = !kG && T::kDirect;            // weight operands straight into registers
    static_assert(!kG || 16 * T::kGgufChunks <= SG::kNW * kWave, "GGUF chunks fit the staging registers");
    constexpr int G = T::kGroups, NS = T::kSteps, TK = 16, UE = SG::UE, UB = SG::UB;
    constexpr int CPU = UB / 16;
    constexpr int NP = T::template kPieces<1>;
    const int lane = (int)(threadIdx.x & 63);
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int nth = NWV * kWave;
    const Lane<1> L(lane);
    const int upr = p.upr, K = p.K, Kp = upr * UE, ngk = K / 32;
    const int xrow = XS::xrow(upr);
    const int Mloc = min(p.M - m0, TK);
    uint8_t *X = smem;
    float *dT = (float *)(smem + XS::oDT(upr)), *aT = (float *)(smem + XS::oAT(upr));
    uint8_t *wl = smem + XS::oWaves(upr) + wave * XS::kWaveBytes;

    // 1. The activation rows, codes and scales, into LDS.  Padding tokens
    // (past M) read token m0's codes and get zero scales; codes past K (a
    // Q8_0 unit's padding) are zero.
    const __amdgpu_buffer_rsrc_t xr = buf_rsrc(p.xq, (uint32_t)p.M * (uint32_t)K);
    {
        const int cpr = Kp / 16, nch = TK * cpr;
        for (int i0 = (int)threadIdx.x; i0 < nch; i0 += kXBatch * nth) {
            v4u v[kXBatch];
#pragma unroll
            for (int b = 0; b < kXBatch; ++b) {
                const int i = i0 + b * nth, tok = i / cpr, j = i % cpr;
                const int src = m0 + (tok < Mloc ? tok : 0);
                v[b] = (i < nch && 16 * j < K) ? buf_ld16(xr, (uint32_t)src * (uint32_t)K + 16u * (uint32_t)j, 0u)
                                               : v4u{0u, 0u, 0u, 0u};
            }
#pragma unroll
            for (int b = 0; b < kXBatch; ++b) {
                const int i = i0 + b * nth;
                if (i < nch) *(v4u *)(X + (i / cpr) * xrow + 16 * (i % cpr)) = v[b];
            }
        }
        if ((int)threadIdx.x < UE / 16) *(v4u *)(smem + XS::oZero(upr) + 16 * threadIdx.x) = v4u{0u, 0u, 0u, 0u};
        const int ns = upr * G * TK;
        for (int i = (int)threadIdx.x; i < ns; i += nth) {
            const int g = i / TK, tok = i % TK;
            const bool in = tok < Mloc && g < ngk;
            const size_t o = (size_t)(m0 + (in ? tok : 0)) * ngk + (in ? g : 0);
            const float d = in ? p.xd[o] : 0.f;
            dT[i] = d;
            if constexpr (T::kAux) aT[i] = in ? T::stage_aux(d, p.xs[o]) : 0.f;
        }
    }

    // 2. This workgroup's sets and this wave's run of units.
    const int S = p.wg_start[p.nmat];
    const int s0 = (int)((long long)S * blockIdx.x / gridDim.x);
    const int nsets = (int)((long long)S * (blockIdx.x + 1) / gridDim.x) - s0;
    const int N = nsets * upr;
    const int ua = (int)((long long)N * wave / NWV), ub = (int)((long long)N * (wave + 1) / NWV);

    // Weight staging map of this lane (the same for every set; tiles past the
    // matrix's end reread its last tile).
    // (GGUF: wt = the row within the set, wc = the chunk of its block)
    int wdst[SG::kNW], wt[SG::kNW], wc[SG::kNW];
#pragma unroll
    for (int n = 0; n < SG::kNW; ++n) {
        const int id = n * kWave + lane;
        if constexpr (kG) {
            const bool ok = id < 16 * T::kGgufChunks;
            wt[n] = ok ? id / T::kGgufChunks : 0;
            wc[n] = ok ? id % T::kGgufChunks : 0;
            wdst[n] = ok ? T::gguf_dst(wt[n], wc[n]) : XS::oDummy;
        } else {
            const bool ok = id < SG::kWChunks;
            wt[n] = ok ? id / CPU : 0;
            wc[n] = ok ? id % CPU : 0;
            wdst[n] = ok ? T::lds_dst(wt[n], wc[n], SG::kSide) : XS::oDummy;
        }
    }
    constexpr bool kA2 = kG && T::kGgufA2;
    const uint32_t rowb = (uint32_t)upr * (uint32_t)T::kBlockBytes;  // GGUF row bytes
    const int ddst = lane < 16 ? SG::kSide + 16 * (lane >> 3) + 2 * (lane & 7) : XS::oDummy;
    v4u rw[SG::kNW];
    uint32_t re[kA2 ? SG::kNW : 1], rsh[kA2 ? SG::kNW : 1], rd = 0u;
    auto issue = [&](int idx) __attribute__((always_inline)) {
        if constexpr (kD) return;
        const int gs = s0 + idx / upr, u = idx % upr;
        int mi = 0;
#pragma unroll
        for (int k = 1; k < kMaxMulti; ++k)
            if (k < p.nmat && gs >= p.wg_start[k]) mi = k;
        const int rc = p.rc[mi], ntiles8 = (rc + kTileRows - 1) / kTileRows;
        if constexpr (kG) {
            const int row0 = (gs - p.wg_start[mi]) * 16;
            const __amdgpu_buffer_rsrc_t wr = buf_rsrc(p.W[mi], (uint32_t)rc * rowb);
            const uint32_t ub = (uint32_t)u * (uint32_t)T::kBlockBytes;
#pragma unroll
            for (int n = 0; n < SG::kNW; ++n) {
                const uint32_t v = (uint32_t)min(row0 + wt[n], rc - 1) * rowb + 16u * (uint32_t)wc[n] + ub;
                if constexpr (kA2) {
                    const uint32_t a = v & ~3u;
                    rw[n] = buf_ld16(wr, a, 0u);
                    re[n] = buf_ld4<0>(wr, a + 16u, 0u);
                    rsh[n] = (v & 2u) * 8u;
                } else {
                    rw[n] = buf_ld16(wr, v, 0u);
                }
            }
            if constexpr (kA2) rd = bld_u16(wr, (uint32_t)min(row0 + (lane & 15), rc - 1) * rowb + (uint32_t)kQ6KD, ub);
        } else {
            const int tile0 = (gs - p.wg_start[mi]) * 2;
            const __amdgpu_buffer_rsrc_t wr = buf_rsrc(p.W[mi], (uint32_t)ntiles8 * (uint32_t)(upr * UB));
#pragma unroll
            for (int n = 0; n < SG::kNW; ++n) {
                const int tile = min(tile0 + wt[n], ntiles8 - 1);
                rw[n] = buf_ld16<kWeightAux>(wr, (uint32_t)tile * (uint32_t)(upr * UB) + 16u * (uint32_t)wc[n],
                                             (uint32_t)u * UB);
            }
        }
    };
    auto commit = [&]() __attribute__((always_inline)) {
        if constexpr (kD) {
        } else if constexpr (kA2) {
#pragma unroll
            for (int n = 0; n < SG::kNW; ++n) *(v4u *)(wl + wdst[n]) = shift16(rw[n], re[n], rsh[n]);
            *(uint16_t *)(wl + ddst) = (uint16_t)rd;
        } else {
#pragma unroll
            for (int n = 0; n < SG::kNW; ++n) *(v4u *)(wl + wdst[n]) = rw[n];
        }
    };

    const int wrow = L.c;  // the lane's weight row within the set
    const int atok = L.c;  // and its token
    // Direct operands of unit idx of the run: row wrow of its set.
    typename T::template Direct<1> dc, dn;
    auto dload = [&](int idx, typename T::template Direct<1> &d) __attribute__((always_inline)) {
        if constexpr (kD) {
            const int gs = s0 + idx / upr, u = idx % upr;
            int mi = 0;
#pragma unroll
            for (int k = 1; k < kMaxMulti; ++k)
                if (k < p.nmat && gs >= p.wg_start[k]) mi = k;
            const int ntiles8 = (p.rc[mi] + kTileRows - 1) / kTileRows;
            const __amdgpu_buffer_rsrc_t wr = buf_rsrc(p.W[mi], (uint32_t)ntiles8 * (uint32_t)(upr * UB));
            const int tile = min((gs - p.wg_start[mi]) * 2 + (wrow >> 3), ntiles8 - 1);
            T::template load_direct<1>(d, wr, (uint32_t)tile * (uint32_t)(upr * UB), wrow & 7, L.r, (uint32_t)u * UB);
        }
    };
    const uint8_t *xa = X + atok * xrow + 8 * L.r;
    const uint8_t *xz = smem + XS::oZero(upr) + 8 * L.r;
    const ScaleLds<1> sl{dT, aT};
    float acc[4] = {0.f, 0.f, 0.f, 0.f}, u4[4] = {0.f, 0.f, 0.f, 0.f}, first[4] = {0.f, 0.f, 0.f, 0.f};
    v4f cm = v4f{0.f, 0.f, 0.f, 0.f};  // Q4_K min term
    auto compute = [&](int idx) __attribute__((always_inline)) {
        const int u = idx % upr;
        const uint8_t *ab[NP];
        if constexpr (NP == 1) {
            ab[0] = xa + u * UE;
        } else {  // Q6_K: quarters 0-1 (sub-block 0) and 2-3 (sub-block 1)
            ab[0] = L.q < 2 ? xa + u * UE : xz;
            ab[1] = L.q < 2 ? xz : xa + u * UE;
        }
        typename T::template Frag<1> f0, f1;
        AFrag<NP> x0, x1;
        if constexpr (kD)
            T::template frag_direct<1>(f0, dc, 0);
        else
            T::template load<1>(f0, wl, wrow, L.r, 0, SG::kSide);
        load_act<NP>(x0, ab, 0);
        if constexpr (NS == 2) {
            if constexpr (kD)
                T::template frag_direct<1>(f1, dc, 1);
            else
                T::template load<1>(f1, wl, wrow, L.r, 1, SG::kSide);
            load_act<NP>(x1, ab, 1);
        }
        compute_half<T, 1, 0>(f0, x0, sl, u * G, L, true, atok, acc, u4, cm);
        if constexpr (NS == 2) compute_half<T, 1, 1>(f1, x1, sl, u * G, L, true, atok, acc, u4, cm);
    };
    // The first set's sums move to `first` when the run enters the second.
    auto close_first = [&]() __attribute__((always_inline)) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            first[e] = T::kAux ? acc[e] - cm[e] : acc[e];
            acc[e] = 0.f;
        }
        cm = v4f{0.f, 0.f, 0.f, 0.f};
    };
    // The first unit's weights load while the activation staging completes.
    if (ua < ub) {
        issue(ua);
        dload(ua, dc);
    }
    __syncthreads();

    // 3. The run, one unit ahead as in the kernel above (unconditional loads,
    // last unit peeled).  Waves with an empty run skip it.
    const int n_first = ua < ub ? min(ub, (ua / upr + 1) * upr) - ua : 0;  // units of the first set
    if (ua < ub) {
        commit();
        for (int k = 0; k + 1 < ub - ua; ++k) {
            issue(ua + k + 1);
            dload(ua + k + 1, dn);
            compute(ua + k);
            if (k + 1 == n_first) close_first();
            commit();
            if constexpr (kD) dc = dn;
        }
        compute(ub - 1);
        if (ub - ua == n_first) {
            close_first();
        } else if (T::kAux) {
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[e] -= cm[e];
        }
    }

    // 4. Partial sums -> this wave's area (slot 0: first set, slot 1: second),
    // then each output adds the waves that covered its set, in wave order.
    {
        float *P = (float *)wl;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            P[e * kWave + lane] = first[e];
            P[4 * kWave + e * kWave + lane] = acc[e];
        }
    }
    __syncthreads();
    for (int idx = (int)threadIdx.x; idx < nsets * 4 * kWave; idx += nth) {
        const int sl_ = idx / (4 * kWave), r = idx % (4 * kWave), e = r / kWave, ln = r % kWave;
        const int lo = sl_ * upr, hi = lo + upr;  // the set's units in the workgroup's order
        float v = 0.f;
        for (int w = 0; w < NWV; ++w) {
            const int a = (int)((long long)N * w / NWV), b = (int)((long long)N * (w + 1) / NWV);
            if (a < hi && b > lo) {
                const int slot = a / upr == sl_ ? 0 : 1;
                v += ((const float *)(smem + XS::oWaves(upr) + w * XS::kWaveBytes))[slot * 4 * kWave + r];
            }
        }
        const int gs = s0 + sl_;
        int mi = 0;
#pragma unroll
        for (int k = 1; k < kMaxMulti; ++k)
            if (k < p.nmat && gs >= p.wg_start[k]) mi = k;
        const Lane<1> O(ln);
        const int rc = p.rc[mi], row = (gs - p.wg_start[mi]) * 16 + O.c, tok = 4 * O.r + e;
        if (row < rc && tok < Mloc) {
            const size_t o = (size_t)(m0 + tok) * rc + row;
            p.Y[mi][o] = v + (p.res[mi] ? p.res[mi][o] : 0.f);
        }
    }
}

template <class T, int PK, int KS, int RS = 1, bool DW = false>
static size_t mfma_lds() {
    return (size_t)KS * Stage<T, PK, RS, DW>::kBytes;
}

template <class T, int PK, int KS, int LAYOUT, int RS>
static hipError_t launch_mfma_t(MatmulMultiParams p, int m0, hipStream_t s) {
    const size_t lds = mfma_lds<T, PK, KS, RS, LAYOUT == M27Q_LAYOUT_TILED && T::kDirect>();
    constexpr int SR = 16 * PK * RS;
    int total = 0;
    for (int i = 0; i < p.nmat; ++i) {
        p.wg_start[i] = total;
        total += (p.rc[i] + SR - 1) / SR;
    }
    p.wg_start[p.nmat] = total;
    hipLaunchKernelGGL((k_matmul_mfma<T, PK, KS, LAYOUT, RS>), dim3(total), dim3(kWave * KS), lds, s, p, m0);
    return hipGetLastError();
}

// The resident-activation kernel serves a launch of 16 tokens when every CU
// gets at least kXresMinSetsPerCu row sets (the activation staging is
// paid once per workgroup) and its LDS fits.  16 waves per workgroup (every
// type compiles within 128 registers, 4 waves per SIMD).  Measured on the
// layer's gate/up (2176 sets): 32 us against 36 at M = 16, 32.5 against 33.5
// at M = 12, where the layer's other launches ran about 0.3 us slower each
// after it, so only full 16-token launches take it; q/k/v (2 sets per CU)
// took 14 us against 9.5 with it.
constexpr int kXresMinSetsPerCu = 4;
template <class T>
constexpr int xres_waves() {
    return 16;
}
template <class T, int LAYOUT>
static bool launch_xres_t(MatmulMultiParams p, int m0, hipStream_t s, hipError_t *err) {
    constexpr int NWV = xres_waves<T>();
    int S = 0;
    for (int i = 0; i < p.nmat; ++i) {
        p.wg_start[i] = S;
        S += (p.rc[i] + 15) / 16;
    }
    p.wg_start[p.nmat] = S;
    const int cus = cu_count();
    if (p.M - m0 < 16 || S < kXresMinSetsPerCu * cus) return false;
    const size_t lds = XStage<T>::bytes(p.upr, NWV);
    if (lds > lds_limit()) return false;
    // at most NWV sets per workgroup, so each wave's run covers at most two
    const int G = std::min(S, std::max(cus, (S + NWV - 1) / NWV));
    hipLaunchKernelGGL((k_matmul_mfma_xres<T, NWV, LAYOUT>), dim3(G), dim3(kWave * NWV), lds, s, p, m0);
    *err = hipGetLastError();
    return true;
}
// GGUF-layout Q6_K's shifted chunk loads do not fit the resident kernel's 128
// registers without spilling: those launches take the per-unit kernel.
// TILED Q4_K / Q5_K take it with their weight operands loaded straight into
// registers (gate/up at M = 16: 29.4 us against 31.8 on the per-unit kernel
// with direct operands and 30.5 resident with staged weights, same box).
template <class T, int LAYOUT>
static bool launch_xres(const MatmulMultiParams &p, int m0, hipStream_t s, hipError_t *err) {
    if constexpr (LAYOUT == M27Q_LAYOUT_GGUF && T::kGgufA2)
        return false;
    else
        return launch_xres_t<T, LAYOUT>(p, m0, s, err);
}

// Launch shape, from sweeps of the Qwen-27B layer at M = 4, 8, 12, 16:
// two-set tiles split K over 8 waves (gate/up's 1088 workgroups at M = 4 / 8:
// 22.4 / 23.1 us against 23.3 / 23.7 with 4 waves, since the paired operand
// reads; q/k/v, o and down took 8 already); one-set tiles over 8 waves in a
// launch of fewer than 320 workgroups, else 4 (more waves per set cost more
// than they hide there).  Two row sets per tile
// whenever at most 8 tokens are left and the product has at least 128 sets
// of 32 rows (every product of the layer): down at M = 8 takes 21.7 us
// against 28.8 with one-set tiles.  One-set tiles (more than 8 tokens left)
// take two row sets per workgroup (RS = 2), each wave's activation operands
// serving both: at M = 16 q/k/v 9.6 us against 10.4, o 10.1 against 11.5,
// down 27.4 against 28.2; gate/up at M = 12 30.1 against 32.0; GGUF-layout
// down 32.6 against 35.5 at M = 16, 31.3 against 32.6 at M = 12.  One set per
// workgroup split K over 8 waves also on K <= 6144 (at M = 16 gate/up 35.6 us
// against 37.7).
constexpr int kPk2MinSets = 128;
// Q6_K launches of at most one workgroup per CU (down: 160 of 32 rows) split
// K over 12 waves: their 8-wave workgroups (85 KB of staging areas for
// two-set tiles, 105 KB for two row sets of one-set tiles) run one per CU
// anyway, and 12 (128 / 157 KB, 3 waves per SIMD) shorten each wave's unit
// chain from 8.5 to 5.7 units: down at M = 4 / 8 20.7 / 21.6 us against
// 22.5 / 23.1, at M = 12 / 16 25.5 / 26.8 against 26.9 / 28.2 (GGUF layout
// at M <= 8 unchanged, 26.9 / 27.6 against 26.8 / 27.8; its one-set kernel
// spills at 12 waves and keeps 8).  The same for Q4_K's q/k/v and o was
// slower at M <= 8 (q/k/v 7.5 against 7.2 us) and equal at M = 16 with
// staged weights; with direct operands (one workgroup per CU at 3 waves per
// SIMD) the one-set launches gain: at M = 16 q/k/v 8.6 against 9.2 us, o 9.3
// against 10.0, while two-set ones lose (q/k/v 6.9 against 6.7 at M = 4).
// Q5_K with two row sets needs 187 VGPRs and spills at 12 waves.
constexpr long long kQ6Wide12MaxWgs = 256;
// Two-set tiles with direct operands (TILED Q4_K / Q5_K, 155-168 VGPRs, 3
// waves per SIMD) in launches of 320 or more workgroups split K over 4 waves,
// so three workgroups share a CU: gate/up at M = 4 / 8 21.5 / 22.2 us against
// 25.0 / 25.9 with 8 waves (one workgroup per CU), 22.1 / 23.4 with 2; q/k/v
// and o (256 and 160 workgroups) keep 8: 6.6 / 6.8 us against 7.4 / 7.7 with 4.
constexpr long long kDirectKs4MinWgs = 320;
template <class T, int PK, int LAYOUT>
static hipError_t launch_mfma_pk(const MatmulMultiParams &p, int m0, hipStream_t s) {
    constexpr int RS = PK == 1 ? 2 : 1;
    constexpr int SR = 16 * PK * RS;
    long long wgs = 0;
    for (int i = 0; i < p.nmat; ++i) wgs += (p.rc[i] + SR - 1) / SR;
    if constexpr (PK == 2) {
        if constexpr (std::is_same<T, MmQ6K>::value)
            if (wgs <= kQ6Wide12MaxWgs) return launch_mfma_t<T, 2, 12, LAYOUT, RS>(p, m0, s);
        if constexpr (LAYOUT == M27Q_LAYOUT_TILED && T::kDirect)
            if (wgs >= kDirectKs4MinWgs) return launch_mfma_t<T, 2, 4, LAYOUT, RS>(p, m0, s);
        return launch_mfma_t<T, 2, 8, LAYOUT, RS>(p, m0, s);
    } else {
        if constexpr ((std::is_same<T, MmQ6K>::value || (T::kDirect && !T::kWide)) && LAYOUT == M27Q_LAYOUT_TILED)
            if (wgs <= kQ6Wide12MaxWgs) return launch_mfma_t<T, 1, 12, LAYOUT, RS>(p, m0, s);
        const int ks = wgs < 320 ? 8 : 4;
        return ks == 8 ? launch_mfma_t<T, 1, 8, LAYOUT, RS>(p, m0, s) : launch_mfma_t<T, 1, 4, LAYOUT, RS>(p, m0, s);
    }
}

template <class T, int LAYOUT>
static hipError_t launch_mfma_cfg(const MatmulMultiParams &p, hipStream_t s) {
    long long sets32 = 0;
    for (int i = 0; i < p.nmat; ++i) sets32 += (p.rc[i] + 31) / 32;
    for (int m0 = 0; m0 < p.M;) {
        const int left = p.M - m0;
        const bool pk2 = left <= 8 && sets32 >= kPk2MinSets;
        hipError_t e = hipSuccess;
        if (pk2)
            e = launch_mfma_pk<T, 2, LAYOUT>(p, m0, s);
        else if (!launch_xres<T, LAYOUT>(p, m0, s, &e))
            e = launch_mfma_pk<T, 1, LAYOUT>(p, m0, s);
        if (e != hipSuccess) return e;
        m0 += pk2 ? Pack<2>::TK : Pack<1>::TK;
    }
    return hipSuccess;
}

template <class T>
static size_t mfma_lds_max() {
    return std::max({mfma_lds<T, 1, 8>(), mfma_lds<T, 2, 8>(), mfma_lds<T, 1, 8, 2>(),
                     std::is_same<T, MmQ6K>::value ? mfma_lds<T, 2, 12>() : (size_t)0,
                     std::is_same<T, MmQ6K>::value ? mfma_lds<T, 1, 12, 2>() : (size_t)0});
}

size_t matmul_mfma_lds_bytes(uint32_t type) {
    // the largest over the shapes the selection can return (KS = 8); the
    // staging is per unit, so it does not depend on K
    switch (type) {
        case kQ4_K: return mfma_lds_max<MmQ4K>();
        case kQ5_K: return mfma_lds_max<MmQ5K>();
        case kQ6_K: return mfma_lds_max<MmQ6K>();
        case kQ8_0: return mfma_lds_max<MmQ80>();
        case kIQ4_XS: return mfma_lds_max<MmIQ4XS>();
        default: return 0;
    }
}

bool matmul_mfma_takes(uint32_t type, int layout) {
    return layout == M27Q_LAYOUT_TILED || type == kQ4_K || type == kQ5_K || type == kQ6_K;
}

bool matmul_mfma_direct(uint32_t type, int layout) {
    return layout == M27Q_LAYOUT_TILED && (type == kQ4_K || type == kQ5_K);
}

hipError_t launch_matmul_mfma(uint32_t type, int layout, const MatmulMultiParams &p, hipStream_t s) {
    if (layout == M27Q_LAYOUT_GGUF) {
        switch (type) {
            case kQ4_K: return launch_mfma_cfg<MmQ4K, M27Q_LAYOUT_GGUF>(p, s);
            case kQ5_K: return launch_mfma_cfg<MmQ5K, M27Q_LAYOUT_GGUF>(p, s);
            case kQ6_K: return launch_mfma_cfg<MmQ6K, M27Q_LAYOUT_GGUF>(p, s);
            default: return hipErrorInvalidValue;
        }
    }
    switch (type) {
        case kQ4_K: return launch_mfma_cfg<MmQ4K, M27Q_LAYOUT_TILED>(p, s);
        case kQ5_K: return launch_mfma_cfg<MmQ5K, M27Q_LAYOUT_TILED>(p, s);
        case kQ6_K: return launch_mfma_cfg<MmQ6K, M27Q_LAYOUT_TILED>(p, s);
        case kQ8_0: return launch_mfma_cfg<MmQ80, M27Q_LAYOUT_TILED>(p, s);
        case kIQ4_XS: return launch_mfma_cfg<MmIQ4XS, M27Q_LAYOUT_TILED>(p, s);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace m27q
