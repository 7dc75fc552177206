// m27q_types.h -- per-type lane fragments for the gfx950 GEMV kernels.
//
// Work mapping shared by every GEMV kernel: a wavefront owns a tile of 8 rows;
// each lane works on one row i and on the c-th 16-byte chunk of that row's
// quants in the current unit (one 256-weight block for Q4_K / Q6_K, four
// 32-weight blocks for Q8_0): lane = 8 i + c, or, for the chunk-pair-first
// Q4_K / Q5_K qs plane of the TILED layout, lane = 16 (c / 2) + 2 i + c % 2
// (LaneMap).  One unit of 8 rows is therefore read by one 16-byte-per-lane
// load per plane: 1 KiB of contiguous bytes per instruction in the TILED
// layout.
//
// Activations are staged in LDS by the calling kernel:
//   int8  xc[Kp]       codes (Kp = K padded to whole units, pad = 0)
//   float xd[Kp/32]    per-32 scale
//   u32   xs[Kp/32 * T::kAuxWords]  per-type auxiliary words (T::put_aux)
// and, for the fp32-activation kernels:
//   float xf[Kp]       values
//   float x16[Kp/16]   per-16 sums of the values
#pragma once

#include "m27q_device.h"

namespace m27q {

constexpr uint32_t kM4 = 0x0f0f0f0fu;

struct ActLds {
    const int8_t *xc;
    const float *xd;
    const uint32_t *xs;
};

struct ActLdsF32 {
    const float *xf;
    const float *x16;
};

__device__ __forceinline__ float ubyte_f(uint32_t w, int k) { return (float)((w >> (8 * k)) & 0xffu); }

// ------------------------------------------------------------------ Q4_K --
// Chunk c of a block's 128 qs bytes holds qs[16c, 16c+16): with g = c/2 and
// h = c%2, the low nibbles are weights 64g + 16h + [0,16) (scale pair 2g), the
// high nibbles weights 64g + 32 + 16h + [0,16) (pair 2g+1)
// (debug/official_dequant.c:56-62 for the index map).  Lane c also carries
// the min term of pair j = c for the whole block.
struct Q4K {
    static constexpr uint32_t kType = kQ4_K;
    static constexpr bool kChunkMajor = true;  // TILED qs plane chunk pair first
    static constexpr int kUnitElems = 256;
    static constexpr int kUnitBytes = kQ4KUnit;
    static constexpr int kBlockBytes = kQ4KBytes;

    struct Frag {
        uint4 q;  // 16 qs bytes
        uint4 h;  // d | dmin << 16, scales[0..4), scales[4..8), scales[8..12)
    };

    struct Lane {
        int c, g, off, shA, shm;
        bool gl, cl;
        // Branch-free decode of the 6-bit scales (get_scale_min_k4, exec:690-693):
        // sc pair = ((X >> sx) & sm) | ((h.y >> sy) & sh) with X = h.y (g < 2) or h.w,
        // min     = ((Y >> mx) & mm) | ((h.z >> my) & mh) with Y = h.z (c < 4) or h.w.
        uint32_t sx, sm, sy, shm6, mx, mm, my, mh;
        __device__ explicit Lane(int c_) : c(c_) {
            g = c >> 1;
            off = 64 * g + 16 * (c & 1);
            shA = 16 * (g & 1);
            shm = 8 * (c & 3);
            gl = g < 2;
            cl = c < 4;
            sx = shA;
            sm = gl ? 0x3f3fu : 0x0f0fu;
            sy = shA + 2;
            shm6 = gl ? 0u : 0x3030u;
            mx = cl ? shm : shm + 4;
            mm = cl ? 63u : 15u;
            my = shm + 2;
            mh = cl ? 0u : 0x30u;
        }
    };

    // Activation fragment of one unit for lane c: its 2 x 16 codes, the scales
    // of its two 32-groups, and d * (code sum) of group c for the min term.
    struct AFrag {
        int4 lo, hi;
        float2 dx;
        float dsum;
    };

    __device__ static int qs_chunk(int i, int c) { return q4k_tqs(i, c >> 1) + 16 * (c & 1); }
    template <bool NT = false>
    __device__ static Frag load_tiled(const uint8_t *unit, int i, int c, const Lane &) {
        return {ld_u128<NT>(unit + qs_chunk(i, c)), ld_u128<NT>(unit + 16 * i)};
    }
    // The same for the GEMV's lane order over the plane (LaneMap): lane l
    // reads qs plane bytes 16 l, its row i's header.
    template <bool NT = false>
    __device__ static Frag load_tiled_lane(const uint8_t *unit, int lane, int i) {
        return {ld_u128<NT>(unit + kQ4KTQs + 16 * lane), ld_u128<NT>(unit + 16 * i)};
    }
    template <bool NT = false>
    __device__ static Frag load_gguf(const uint8_t *row, int u, int /*rb*/, int c, const Lane &) {
        const uint8_t *blk = row + (size_t)u * kQ4KBytes;
        return {ld_u128<NT>(blk + kQ4KHdr + 16 * c), ld_u128<NT>(blk)};
    }
    // The same planes through a buffer descriptor of the tile; soff = the unit's offset.
    template <int AUX>
    __device__ static Frag load_tiled_buf(__amdgpu_buffer_rsrc_t r, uint32_t soff, int i, int c, const Lane &) {
        return {bld_u128<AUX>(r, qs_chunk(i, c), soff), bld_u128<AUX>(r, 16 * i, soff)};
    }

    // 6-bit scales of pairs 2g, 2g+1 (bits 0-5 and 8-13) and the min of pair c.
    __device__ static uint32_t scale_pair(const uint4 &h, const Lane &L) {
        const uint32_t X = L.gl ? h.y : h.w;
        return ((X >> L.sx) & L.sm) | ((h.y >> L.sy) & L.shm6);
    }
    __device__ static int min_c(const uint4 &h, const Lane &L) {
        const uint32_t Y = L.cl ? h.z : h.w;
        return (int)(((Y >> L.mx) & L.mm) | ((h.z >> L.my) & L.mh));
    }

    // LDS aux word of group g: d * (sum of the 32 codes), the scale of the
    // block-min term.
    static constexpr int kAuxWords = 1;
    __device__ static void put_aux(uint32_t *xs, int g, float d, uint32_t s) {
        const int S = (int)(int16_t)(s & 0xffffu) + (int)(int16_t)(s >> 16);
        xs[g] = __float_as_uint(d * (float)S);
    }

    __device__ static AFrag load_act(const ActLds &a, int u, const Lane &L) {
        AFrag r;
        r.lo = *(const int4 *)(a.xc + 256 * u + L.off);
        r.hi = *(const int4 *)(a.xc + 256 * u + L.off + 32);
        r.dx = *(const float2 *)(a.xd + 8 * u + 2 * L.g);
        r.dsum = __uint_as_float(a.xs[8 * u + L.c]);
        return r;
    }

    // Per 32-group j of the block: d sc_j dx_j sum(q4 q8) - dmin m_j dx_j sum(q8)
    // (the vec_dot_q4_K_q8_1 terms, exec:250-310), for this lane's share.
    __device__ static float dot(const Frag &f, const AFrag &a, const Lane &L) {
        int slo = dot4((int)(f.q.x & kM4), a.lo.x, 0);
        slo = dot4((int)(f.q.y & kM4), a.lo.y, slo);
        slo = dot4((int)(f.q.z & kM4), a.lo.z, slo);
        slo = dot4((int)(f.q.w & kM4), a.lo.w, slo);
        int shi = dot4((int)((f.q.x >> 4) & kM4), a.hi.x, 0);
        shi = dot4((int)((f.q.y >> 4) & kM4), a.hi.y, shi);
        shi = dot4((int)((f.q.z >> 4) & kM4), a.hi.z, shi);
        shi = dot4((int)((f.q.w >> 4) & kM4), a.hi.w, shi);
        return combine(f.h, a, L, slo, shi);
    }
    // The scale terms of the lane's two 16-value halves from their integer sums
    // (each 32-group is split over lanes c = 2g, 2g + 1, so its two halves are
    // scaled apart and added in fp32; completing the group's integer sum first,
    // with one DPP swap per pair, made config 1 0.5 us slower).
    __device__ static float combine(const uint4 &h, const AFrag &a, const Lane &L, int slo, int shi) {
        const uint32_t pair = scale_pair(h, L);
        const int m = min_c(h, L);
        // |code sums| < 2^16 and scales < 2^6: the 24-bit products are exact.
        const float t = fmaf(a.dx.y, (float)__mul24((int)(pair >> 8), shi), a.dx.x * (float)__mul24((int)(pair & 0xffu), slo));
        const float dw = f16_bits_to_f32(h.x), dm = f16_bits_to_f32(h.x >> 16);
        return fmaf(dw, t, -dm * ((float)m * a.dsum));
    }
    __device__ static float dot(const Frag &f, const ActLds &a, int u, const Lane &L) {
        return dot(f, load_act(a, u, L), L);
    }

    __device__ static float dot_f32(const Frag &f, const ActLdsF32 &a, int u, const Lane &L) {
        const float4 *xl = (const float4 *)(a.xf + 256 * u + L.off);
        const float4 *xh = (const float4 *)(a.xf + 256 * u + L.off + 32);
        const uint32_t qw[4] = {f.q.x, f.q.y, f.q.z, f.q.w};
        float flo = 0.f, fhi = 0.f;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint32_t lo = qw[k] & kM4, hi = (qw[k] >> 4) & kM4;
            const float4 vl = xl[k], vh = xh[k];
            flo += ubyte_f(lo, 0) * vl.x + ubyte_f(lo, 1) * vl.y + ubyte_f(lo, 2) * vl.z + ubyte_f(lo, 3) * vl.w;
            fhi += ubyte_f(hi, 0) * vh.x + ubyte_f(hi, 1) * vh.y + ubyte_f(hi, 2) * vh.z + ubyte_f(hi, 3) * vh.w;
        }
        return combine_f32(f.h, a, u, L, flo, fhi);
    }
    __device__ static float combine_f32(const uint4 &h, const ActLdsF32 &a, int u, const Lane &L, float flo,
                                        float fhi) {
        const uint32_t pair = scale_pair(h, L);
        const int m = min_c(h, L);
        const float xsum = a.x16[16 * u + 2 * L.c] + a.x16[16 * u + 2 * L.c + 1];
        const float dw = f16_bits_to_f32(h.x), dm = f16_bits_to_f32(h.x >> 16);
        return dw * ((float)(pair & 0xffu) * flo + (float)(pair >> 8) * fhi) - dm * ((float)m * xsum);
    }
};

// ------------------------------------------------------------------ Q5_K --
// Q4_K plus a fifth bit per weight (exec:953-969): position l of 32-group j
// adds 16 * bit j of qh[l].  Lane c reads the same 16 qs bytes as for Q4_K
// and the 16 qh bytes of its half (qh[16 (c % 2) .. + 16)), whose bits 2g and
// 2g + 1 (g = c / 2) belong to its low and high nibbles.  Everything else --
// the activation fragment, the scales, the min term -- is Q4_K's.
struct Q5K : Q4K {
    static constexpr uint32_t kType = kQ5_K;
    static constexpr int kUnitBytes = kQ5KUnit;
    static constexpr int kBlockBytes = kQ5KBytes;

    struct Frag {
        uint4 q;   // 16 qs bytes
        uint4 hb;  // 16 qh bytes
        uint4 h;   // d | dmin << 16, scales[12]
    };

    template <bool NT = false>
    __device__ static Frag load_tiled(const uint8_t *unit, int i, int c, const Lane &) {
        return {ld_u128<NT>(unit + qs_chunk(i, c)), ld_u128<NT>(unit + kQ5KTQh + 32 * i + 16 * (c & 1)),
                ld_u128<NT>(unit + 16 * i)};
    }
    // GEMV lane order (LaneMap): qs plane bytes 16 l; qh bytes 16 (l % 2) of row i = (l / 2) % 8.
    template <bool NT = false>
    __device__ static Frag load_tiled_lane(const uint8_t *unit, int lane, int i) {
        return {ld_u128<NT>(unit + kQ4KTQs + 16 * lane), ld_u128<NT>(unit + kQ5KTQh + 16 * (lane & 15)),
                ld_u128<NT>(unit + 16 * i)};
    }
    template <bool NT = false>
    __device__ static Frag load_gguf(const uint8_t *row, int u, int /*rb*/, int c, const Lane &) {
        const uint8_t *blk = row + (size_t)u * kQ5KBytes;
        return {ld_u128<NT>(blk + kQ5KQs + 16 * c), ld_u128<NT>(blk + kQ5KQh + 16 * (c & 1)), ld_u128<NT>(blk)};
    }
    template <int AUX>
    __device__ static Frag load_tiled_buf(__amdgpu_buffer_rsrc_t r, uint32_t soff, int i, int c, const Lane &) {
        return {bld_u128<AUX>(r, qs_chunk(i, c), soff), bld_u128<AUX>(r, kQ5KTQh + 32 * i + 16 * (c & 1), soff),
                bld_u128<AUX>(r, 16 * i, soff)};
    }

    // 5-bit codes of one dword: the nibbles plus bit 2g (low) / 2g + 1 (high)
    // of each qh byte, moved to bit 4.  Shifted right first: a left shift of the
    // whole word would drop the top byte's bits 4..7 (groups 4..7).
    __device__ static void codes(uint32_t q, uint32_t hb, const Lane &L, uint32_t &lo, uint32_t &hi) {
        lo = (q & kM4) | (((hb >> (2 * L.g)) & 0x01010101u) << 4);
        hi = ((q >> 4) & kM4) | (((hb >> (2 * L.g + 1)) & 0x01010101u) << 4);
    }

    __device__ static float dot(const Frag &f, const AFrag &a, const Lane &L) {
        const uint32_t qw[4] = {f.q.x, f.q.y, f.q.z, f.q.w};
        const uint32_t hw[4] = {f.hb.x, f.hb.y, f.hb.z, f.hb.w};
        const int alo[4] = {a.lo.x, a.lo.y, a.lo.z, a.lo.w};
        const int ahi[4] = {a.hi.x, a.hi.y, a.hi.z, a.hi.w};
        int slo = 0, shi = 0;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            uint32_t lo, hi;
            codes(qw[k], hw[k], L, lo, hi);
            slo = dot4((int)lo, alo[k], slo);
            shi = dot4((int)hi, ahi[k], shi);
        }
        // |code sums| <= 16 * 31 * 127 < 2^16: the 24-bit scale products stay exact
        return combine(f.h, a, L, slo, shi);
    }
    __device__ static float dot(const Frag &f, const ActLds &a, int u, const Lane &L) {
        return dot(f, load_act(a, u, L), L);
    }

    __device__ static float dot_f32(const Frag &f, const ActLdsF32 &a, int u, const Lane &L) {
        const float4 *xl = (const float4 *)(a.xf + 256 * u + L.off);
        const float4 *xh = (const float4 *)(a.xf + 256 * u + L.off + 32);
        const uint32_t qw[4] = {f.q.x, f.q.y, f.q.z, f.q.w};
        const uint32_t hw[4] = {f.hb.x, f.hb.y, f.hb.z, f.hb.w};
        float flo = 0.f, fhi = 0.f;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            uint32_t lo, hi;
            codes(qw[k], hw[k], L, lo, hi);
            const float4 vl = xl[k], vh = xh[k];
            flo += ubyte_f(lo, 0) * vl.x + ubyte_f(lo, 1) * vl.y + ubyte_f(lo, 2) * vl.z + ubyte_f(lo, 3) * vl.w;
            fhi += ubyte_f(hi, 0) * vh.x + ubyte_f(hi, 1) * vh.y + ubyte_f(hi, 2) * vh.z + ubyte_f(hi, 3) * vh.w;
        }
        return combine_f32(f.h, a, u, L, flo, fhi);
    }
};

// ------------------------------------------------------------------ Q6_K --
// Chunk c of ql: half hh = c/4, cc = c%4, l0 = 16 (cc%2), r = cc/2.  Low
// nibbles are q_r at positions 128hh + 32r + l0 + [0,16), high nibbles q_{r+2}
// at +64; their top two bits are bits 2r / 2r+4 of qh[32hh + l0 + [0,16)], and
// their scales are scales[8hh + cc] / scales[8hh + 4 + cc]
// (exec:1026-1048 for the index map).
struct Q6K {
    static constexpr uint32_t kType = kQ6_K;
    static constexpr bool kChunkMajor = false;
    static constexpr int kUnitElems = 256;
    static constexpr int kUnitBytes = kQ6KUnit;
    static constexpr int kBlockBytes = kQ6KBytes;

    struct Frag {
        uint4 ql, qh;
        uint2 sc;      // scales[8hh .. 8hh+8)
        uint32_t d;    // f16 bits of d at bit dsh
        uint32_t dsh;  // 0 or 16
    };

    struct Lane {
        int hh, cc, qh_off, aoff, jlo, shl_lo, shr_hi, hsel;
        uint32_t scsel;  // v_perm_b32: byte cc of sc.x, byte cc of sc.y
        __device__ explicit Lane(int c) {
            hh = c >> 2;
            cc = c & 3;
            const int r = cc >> 1, l0 = 16 * (cc & 1);
            qh_off = 32 * hh + l0;
            aoff = 128 * hh + 32 * r + l0;
            jlo = 4 * hh + r;
            shl_lo = 4 - 2 * r;
            shr_hi = 2 * (r + 2) - 4;
            hsel = cc & 1;
            scsel = 0x0c0c0000u | ((uint32_t)(cc + 4) << 8) | (uint32_t)cc;
        }
    };

    template <bool NT = false>
    __device__ static Frag load_tiled(const uint8_t *unit, int i, int c, const Lane &L) {
        Frag f;
        f.ql = ld_u128<NT>(unit + kQ6KTQl + 128 * i + 16 * c);
        f.qh = ld_u128<NT>(unit + kQ6KTQh + 64 * i + L.qh_off);
        f.sc = *(const uint2 *)(unit + kQ6KTSc + 16 * i + 8 * L.hh);
        f.d = *(const uint32_t *)(unit + kQ6KTD + 4 * (i >> 1));  // the d pair of rows i & ~1, i | 1
        f.dsh = 16 * (i & 1);
        return f;
    }
    template <int AUX>
    __device__ static Frag load_tiled_buf(__amdgpu_buffer_rsrc_t r, uint32_t soff, int i, int c, const Lane &L) {
        Frag f;
        f.ql = bld_u128<AUX>(r, kQ6KTQl + 128 * i + 16 * c, soff);
        f.qh = bld_u128<AUX>(r, kQ6KTQh + 64 * i + L.qh_off, soff);
        f.sc = bld_u64(r, kQ6KTSc + 16 * i + 8 * L.hh, soff);
        f.d = bld_u32(r, kQ6KTD + 4 * (i >> 1), soff);  // the d pair of rows i & ~1, i | 1
        f.dsh = 16 * (i & 1);
        return f;
    }
    // WIDE: ql and qh as five dword loads each (20 bytes from each 4-aligned
    // start: ql's last chunk runs into qh, qh's last into the scales, so every
    // read stays in the block) instead of eight halfword loads.  Measured on
    // GGUF-layout weights: down (one tile per wave) 20.9 us against 22.6; the
    // LM head (two tiles per wave) 238 against 232, so it keeps the halfwords.
    template <bool NT = false, bool WIDE = false>
    __device__ static Frag load_gguf(const uint8_t *row, int u, int /*rb*/, int c, const Lane &L) {
        const uint8_t *blk = row + (size_t)u * kQ6KBytes;
        Frag f;
        f.ql = WIDE ? ld_u128_a2w(blk + kQ6KQl + 16 * c) : ld_u128_a2(blk + kQ6KQl + 16 * c);
        f.qh = WIDE ? ld_u128_a2w(blk + kQ6KQh + L.qh_off) : ld_u128_a2(blk + kQ6KQh + L.qh_off);
        f.sc = make_uint2(ld_u32_a2(blk + kQ6KSc + 8 * L.hh), ld_u32_a2(blk + kQ6KSc + 8 * L.hh + 4));
        f.d = *(const uint16_t *)(blk + kQ6KD);
        f.dsh = 0;
        return f;
    }

    // LDS aux words of group g: -32 x the code sums of its two 16-value
    // halves.  The weight codes are q + 32, so the dot sums start from these
    // and the offset is removed exactly.
    static constexpr int kAuxWords = 2;
    __device__ static void put_aux(uint32_t *xs, int g, float, uint32_t s) {
        xs[2 * g] = (uint32_t)(-32 * (int)(int16_t)(s & 0xffffu));
        xs[2 * g + 1] = (uint32_t)(-32 * (int)(int16_t)(s >> 16));
    }

    __device__ static void codes(const Frag &f, const Lane &L, uint32_t lo6[4], uint32_t hi6[4]) {
        const uint32_t qlw[4] = {f.ql.x, f.ql.y, f.ql.z, f.ql.w};
        const uint32_t qhw[4] = {f.qh.x, f.qh.y, f.qh.z, f.qh.w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            lo6[k] = (qlw[k] & kM4) | ((qhw[k] << L.shl_lo) & 0x30303030u);
            hi6[k] = ((qlw[k] >> 4) & kM4) | ((qhw[k] >> L.shr_hi) & 0x30303030u);
        }
    }

    // Activation fragment of one unit for lane c: 2 x 16 codes, their scales,
    // and -32 x (code sums) of the two 16-value halves.
    struct AFrag {
        int4 lo, hi;
        float dlo, dhi;
        int olo, ohi;
    };

    __device__ static AFrag load_act(const ActLds &a, int u, const Lane &L) {
        AFrag r;
        r.lo = *(const int4 *)(a.xc + 256 * u + L.aoff);
        r.hi = *(const int4 *)(a.xc + 256 * u + L.aoff + 64);
        const int jl = 8 * u + L.jlo;
        r.dlo = a.xd[jl];
        r.dhi = a.xd[jl + 2];
        r.olo = (int)a.xs[2 * jl + L.hsel];
        r.ohi = (int)a.xs[2 * jl + 4 + L.hsel];
        return r;
    }

    // Per 16-group j: d sc_j dx_(j/2) sum((q6 - 32) q8) (vec_dot_q6_K_q8_1, exec:586-628).
    __device__ static float dot(const Frag &f, const AFrag &a, const Lane &L) {
        uint32_t lo6[4], hi6[4];
        codes(f, L, lo6, hi6);
        int slo = dot4((int)lo6[0], a.lo.x, a.olo);
        slo = dot4((int)lo6[1], a.lo.y, slo);
        slo = dot4((int)lo6[2], a.lo.z, slo);
        slo = dot4((int)lo6[3], a.lo.w, slo);
        int shi = dot4((int)hi6[0], a.hi.x, a.ohi);
        shi = dot4((int)hi6[1], a.hi.y, shi);
        shi = dot4((int)hi6[2], a.hi.z, shi);
        shi = dot4((int)hi6[3], a.hi.w, shi);
        const uint32_t sp = __builtin_amdgcn_perm(f.sc.y, f.sc.x, L.scsel);
        const int sclo = (int)(int8_t)sp;
        const int schi = (int)(int8_t)(sp >> 8);
        // |sums| <= 32 * 127 * 16 < 2^23 and |scales| <= 128: exact 24-bit products.
        const float t = fmaf(a.dhi, (float)__mul24(shi, schi), a.dlo * (float)__mul24(slo, sclo));
        return f16_bits_to_f32(f.d >> f.dsh) * t;
    }
    __device__ static float dot(const Frag &f, const ActLds &a, int u, const Lane &L) {
        return dot(f, load_act(a, u, L), L);
    }

    __device__ static float dot_f32(const Frag &f, const ActLdsF32 &a, int u, const Lane &L) {
        uint32_t lo6[4], hi6[4];
        codes(f, L, lo6, hi6);
        const float4 *xl = (const float4 *)(a.xf + 256 * u + L.aoff);
        const float4 *xh = (const float4 *)(a.xf + 256 * u + L.aoff + 64);
        float flo = 0.f, fhi = 0.f;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const float4 vl = xl[k], vh = xh[k];
            flo += ubyte_f(lo6[k], 0) * vl.x + ubyte_f(lo6[k], 1) * vl.y + ubyte_f(lo6[k], 2) * vl.z +
                   ubyte_f(lo6[k], 3) * vl.w;
            fhi += ubyte_f(hi6[k], 0) * vh.x + ubyte_f(hi6[k], 1) * vh.y + ubyte_f(hi6[k], 2) * vh.z +
                   ubyte_f(hi6[k], 3) * vh.w;
        }
        const int g16 = 16 * u + L.aoff / 16;
        flo -= 32.f * a.x16[g16];
        fhi -= 32.f * a.x16[g16 + 4];
        const float sclo = (float)(int8_t)(f.sc.x >> (8 * L.cc));
        const float schi = (float)(int8_t)(f.sc.y >> (8 * L.cc));
        return f16_bits_to_f32(f.d >> f.dsh) * (sclo * flo + schi * fhi);
    }
};

// ---------------------------------------------------------------- IQ4_XS --
// Lane c holds the 16 qs bytes of 32-group c: low nibbles are its positions
// 0..15, high nibbles 16..31 (exec:992-1011).  Codes go through the 16-entry
// table to int8 and into dot4; per group d (ls_c - 32) dx_c sum(kv[q] q8)
// (vec_dot_iq4_xs_q8_1, exec:647-671).  GGUF blocks are 136 B: 8-byte loads.
struct IQ4XS {
    static constexpr uint32_t kType = kIQ4_XS;
    static constexpr bool kChunkMajor = false;
    static constexpr int kUnitElems = 256;
    static constexpr int kUnitBytes = kIQ4XSUnit;
    static constexpr int kBlockBytes = kIQ4XSBytes;

    struct Frag {
        uint4 q;   // 16 qs bytes of group c
        uint2 hd;  // d | scales_h << 16, scales_l[4]
    };
    struct Lane {
        int c, lsh, hsh;
        __device__ explicit Lane(int c_) : c(c_), lsh(8 * (c_ >> 1) + 4 * (c_ & 1)), hsh(16 + 2 * c_) {}
    };
    struct AFrag {
        int4 lo, hi;
        float dx;
    };

    template <bool NT = false>
    __device__ static Frag load_tiled(const uint8_t *unit, int i, int c, const Lane &) {
        return {ld_u128<NT>(unit + 128 * i + 16 * c), *(const uint2 *)(unit + kIQ4XSTHdr + 8 * i)};
    }
    template <int AUX>
    __device__ static Frag load_tiled_buf(__amdgpu_buffer_rsrc_t r, uint32_t soff, int i, int c, const Lane &) {
        return {bld_u128<AUX>(r, 128 * i + 16 * c, soff), bld_u64(r, kIQ4XSTHdr + 8 * i, soff)};
    }
    template <bool NT = false>
    __device__ static Frag load_gguf(const uint8_t *row, int u, int /*rb*/, int c, const Lane &) {
        const uint8_t *blk = row + (size_t)u * kIQ4XSBytes;
        const uint2 a = *(const uint2 *)(blk + kIQ4XSQs + 16 * c), b = *(const uint2 *)(blk + kIQ4XSQs + 16 * c + 8);
        return {make_uint4(a.x, a.y, b.x, b.y), *(const uint2 *)blk};
    }
    static constexpr int kAuxWords = 0;  // codes and scales only
    __device__ static void put_aux(uint32_t *, int, float, uint32_t) {}

    __device__ static AFrag load_act(const ActLds &a, int u, const Lane &L) {
        AFrag r;
        r.lo = *(const int4 *)(a.xc + 256 * u + 32 * L.c);
        r.hi = *(const int4 *)(a.xc + 256 * u + 32 * L.c + 16);
        r.dx = a.xd[8 * u + L.c];
        return r;
    }
    __device__ static int ls_minus_32(const uint2 &hd, const Lane &L) {
        return (int)(((hd.y >> L.lsh) & 15u) | (((hd.x >> L.hsh) & 3u) << 4)) - 32;
    }
    __device__ static float dot(const Frag &f, const AFrag &a, const Lane &L) {
        const uint32_t qw[4] = {f.q.x, f.q.y, f.q.z, f.q.w};
        const int alo[4] = {a.lo.x, a.lo.y, a.lo.z, a.lo.w};
        const int ahi[4] = {a.hi.x, a.hi.y, a.hi.z, a.hi.w};
        int s = 0;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            s = dot4((int)iq4_lut(qw[k] & kM4), alo[k], s);
            s = dot4((int)iq4_lut((qw[k] >> 4) & kM4), ahi[k], s);
        }
        // |s| <= 32 * 127 * 127 and |ls - 32| <= 32: the product is exact in 24 bits
        return f16_bits_to_f32(f.hd.x) * a.dx * (float)__mul24(s, ls_minus_32(f.hd, L));
    }
    __device__ static float dot(const Frag &f, const ActLds &a, int u, const Lane &L) {
        return dot(f, load_act(a, u, L), L);
    }

    __device__ static float dot_f32(const Frag &f, const ActLdsF32 &a, int u, const Lane &L) {
        const float4 *xl = (const float4 *)(a.xf + 256 * u + 32 * L.c);
        const float4 *xh = (const float4 *)(a.xf + 256 * u + 32 * L.c + 16);
        const uint32_t qw[4] = {f.q.x, f.q.y, f.q.z, f.q.w};
        float acc = 0.f;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint32_t vl = iq4_lut(qw[k] & kM4), vh = iq4_lut((qw[k] >> 4) & kM4);
            const float4 x0 = xl[k], x1 = xh[k];
            acc += (float)(int8_t)vl * x0.x + (float)(int8_t)(vl >> 8) * x0.y + (float)(int8_t)(vl >> 16) * x0.z +
                   (float)(int8_t)(vl >> 24) * x0.w;
            acc += (float)(int8_t)vh * x1.x + (float)(int8_t)(vh >> 8) * x1.y + (float)(int8_t)(vh >> 16) * x1.z +
                   (float)(int8_t)(vh >> 24) * x1.w;
        }
        return f16_bits_to_f32(f.hd.x) * (float)ls_minus_32(f.hd, L) * acc;
    }
};

// ------------------------------------------------------------------ Q8_0 --
// Unit = 4 blocks of 32.  Lane c: block k = c/2 of the unit, half c%2.
struct Q80 {
    static constexpr uint32_t kType = kQ8_0;
    static constexpr bool kChunkMajor = false;
    static constexpr int kUnitElems = 128;
    static constexpr int kUnitBytes = kQ80Unit;
    static constexpr int kBlockBytes = kQ80Bytes;

    struct Frag {
        uint4 q;
        uint32_t d;
    };

    struct Lane {
        int k, hf;
        __device__ explicit Lane(int c) : k(c >> 1), hf(c & 1) {}
    };

    template <bool NT = false>
    __device__ static Frag load_tiled(const uint8_t *unit, int i, int /*c*/, const Lane &L) {
        return {ld_u128<NT>(unit + 128 * i + 32 * L.k + 16 * L.hf), *(const uint16_t *)(unit + kQ80TD + 8 * i + 2 * L.k)};
    }
    template <int AUX>
    __device__ static Frag load_tiled_buf(__amdgpu_buffer_rsrc_t r, uint32_t soff, int i, int /*c*/, const Lane &L) {
        return {bld_u128<AUX>(r, 128 * i + 32 * L.k + 16 * L.hf, soff), bld_u16(r, kQ80TD + 8 * i + 2 * L.k, soff)};
    }
    template <bool NT = false>
    __device__ static Frag load_gguf(const uint8_t *row, int u, int rb, int /*c*/, const Lane &L) {
        const int bi = 4 * u + L.k;
        if (bi >= rb) return {make_uint4(0, 0, 0, 0), 0u};
        const uint8_t *blk = row + (size_t)bi * kQ80Bytes;
        return {ld_u128_a2(blk + 2 + 16 * L.hf), *(const uint16_t *)blk};
    }

    static constexpr int kAuxWords = 0;  // codes and scales only
    __device__ static void put_aux(uint32_t *, int, float, uint32_t) {}

    struct AFrag {
        int4 x;
        float d;
    };

    __device__ static AFrag load_act(const ActLds &a, int u, const Lane &L) {
        return {*(const int4 *)(a.xc + 128 * u + 32 * L.k + 16 * L.hf), a.xd[4 * u + L.k]};
    }

    // d_w dx sum(q q8) per block (vec_dot_q8_0_q8_1, exec:535-580).  The two
    // lanes of a block add their half sums (DPP) and the first scales the
    // whole block, so each block's integer sum is complete before its scales.
    __device__ static float dot(const Frag &f, const AFrag &a, const Lane &L) {
        int s = dot4((int)f.q.x, a.x.x, 0);
        s = dot4((int)f.q.y, a.x.y, s);
        s = dot4((int)f.q.z, a.x.z, s);
        s = dot4((int)f.q.w, a.x.w, s);
        s += dpp_i<kDppXor1>(s);
        return L.hf ? 0.f : f16_bits_to_f32(f.d) * (a.d * (float)s);
    }
    __device__ static float dot(const Frag &f, const ActLds &a, int u, const Lane &L) {
        return dot(f, load_act(a, u, L), L);
    }

    __device__ static float dot_f32(const Frag &f, const ActLdsF32 &a, int u, const Lane &L) {
        const float4 *x = (const float4 *)(a.xf + 128 * u + 32 * L.k + 16 * L.hf);
        const uint32_t qw[4] = {f.q.x, f.q.y, f.q.z, f.q.w};
        float acc = 0.f;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const float4 v = x[k];
            acc += (float)(int8_t)(qw[k]) * v.x + (float)(int8_t)(qw[k] >> 8) * v.y +
                   (float)(int8_t)(qw[k] >> 16) * v.z + (float)(int8_t)(qw[k] >> 24) * v.w;
        }
        return f16_bits_to_f32(f.d) * acc;
    }
};

// Lane roles of the GEMV kernels (row i of the wave's 8-row tile, 16-byte
// chunk c of the row's unit) and the sum over the 8 lanes of a row.  With the
// chunk-pair-first qs plane of TILED Q4_K / Q5_K, lane l reads plane bytes
// 16 l as row (l / 2) % 8, chunk 2 (l / 16) + l % 2, so a row's lanes are
// l = 2 i + {0, 1} + {0, 16, 32, 48}.
template <class T, int LAYOUT>
struct LaneMap {
    static constexpr bool kCM = LAYOUT == M27Q_LAYOUT_TILED && T::kChunkMajor;
    __device__ static int row(int lane) { return kCM ? (lane >> 1) & 7 : lane >> 3; }
    __device__ static int chunk(int lane) { return kCM ? ((lane >> 4) << 1) | (lane & 1) : lane & 7; }
    // Every lane of the row gets the sum.
    __device__ static float sum(float v) {
        if constexpr (kCM) {
            v += dpp_f<kDppXor1>(v);
            // gfx950's row swaps: each sum pairs lane l with l ^ 16, then with l ^ 32
            const auto h = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
            v = __uint_as_float(h[0]) + __uint_as_float(h[1]);
            const auto w = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
            return __uint_as_float(w[0]) + __uint_as_float(w[1]);
        } else {
            return sum8(v);
        }
    }
};

// ------------------------------------------------------- weight stream --
// Weight fragments of one unit for the TPW tiles of every matrix (the caller
// includes m27q.h for the layout tags).  NT selects non-temporal 16-byte loads
// (ld_u128<true>); the GGUF blocks that are only 2- or 8-byte aligned (Q6_K,
// Q8_0, IQ4_XS) are read in smaller pieces and keep the default policy.
// With BUF, TILED weights are read through one buffer descriptor per tile
// (its base and byte count in scalar registers): the plane offsets of the
// lane are one loop-invariant register and the unit's offset a scalar, so a
// load costs no vector address arithmetic (with 64-bit per-lane addresses it
// cost 3-7 vector instructions per unit).  Measured per kernel (its callers
// choose): down 0.2 us and the few-token layer 1 us faster with them, the
// multi-tile Q4_K shapes (config 1, o) 0.2-0.5 us slower.
template <class T, int LAYOUT, int NM, int TPW, bool NT = false, bool BUF = true>
struct UnitStream {
    static constexpr bool kTiled = LAYOUT == M27Q_LAYOUT_TILED, kBuf = kTiled && BUF;
    __amdgpu_buffer_rsrc_t rs[kBuf ? NM : 1][kBuf ? TPW : 1];  // TILED with BUF: one tile each
    const uint8_t *base[NM][TPW];  // TILED: first unit of the tile; GGUF: this lane's row
    int i, c, rb, ln;
    typename T::Lane L;

    __device__ UnitStream(const uint8_t *const *W, int tile0, int ntiles, int rc, int rb_, int upr, int lane)
        : i(LaneMap<T, LAYOUT>::row(lane)), c(LaneMap<T, LAYOUT>::chunk(lane)), rb(rb_), ln(lane),
          L(LaneMap<T, LAYOUT>::chunk(lane)) {
#pragma unroll
        for (int m = 0; m < NM; ++m)
#pragma unroll
            for (int t = 0; t < TPW; ++t) {
                const int tile = min(tile0 + t, ntiles - 1);  // past the end: reread the last tile
                if constexpr (kTiled) {
                    const uint32_t tb = (uint32_t)upr * (uint32_t)T::kUnitBytes;
                    base[m][t] = W[m] + (size_t)tile * tb;
                    if constexpr (kBuf) rs[m][t] = buf_rsrc(base[m][t], tb);
                } else {
                    const int row = min(tile * kTileRows + i, rc - 1);
                    base[m][t] = W[m] + (size_t)row * rb_ * T::kBlockBytes;
                }
            }
    }

    __device__ void load(typename T::Frag (&f)[NM][TPW], int u) const {
#pragma unroll
        for (int m = 0; m < NM; ++m)
#pragma unroll
            for (int t = 0; t < TPW; ++t) {
                if constexpr (kBuf)
                    f[m][t] = T::template load_tiled_buf<NT ? 2 : 0>(rs[m][t], (uint32_t)u * (uint32_t)T::kUnitBytes,
                                                                     i, c, L);
                else if constexpr (LaneMap<T, LAYOUT>::kCM)
                    f[m][t] = T::template load_tiled_lane<NT>(base[m][t] + (uint32_t)u * (uint32_t)T::kUnitBytes, ln, i);
                else if constexpr (kTiled)
                    f[m][t] = T::template load_tiled<NT>(base[m][t] + (uint32_t)u * (uint32_t)T::kUnitBytes, i, c, L);
                else if constexpr (T::kType == kQ6_K)
                    f[m][t] = T::template load_gguf<NT, TPW == 1>(base[m][t], u, rb, c, L);
                else
                    f[m][t] = T::template load_gguf<NT>(base[m][t], u, rb, c, L);
            }
    }
};

}  // namespace m27q
