// m27q_gather.hip -- row gather + dequantization to fp32 (bit-exact).
//
// One wavefront dequantizes 256-value chunks of one row (one Q4_K/Q6_K block,
// eight Q8_0 blocks, or 256 F16/F32 elements): lane l produces values
// 4l .. 4l+3 of a chunk and stores them as one float4, so a wave writes 1 KiB
// contiguous per chunk.  A wave takes up to 8 chunks of the row and issues all
// their loads before converting any (5 chunks per wave for a 5120-wide row).
// Generalizes k_q4k_embed (exec:1233-1254: one Q4_K row, one workgroup) to any
// supported type/layout and to a device array of row ids.
#include "m27q_internal.h"
#include "m27q_device.h"

namespace m27q {

// get_scale_min_k4 (exec:690-693) on the 12 scale bytes held as words
// y = q[0..4), z = q[4..8), w = q[8..12), with shifts instead of byte indexing.
__device__ __forceinline__ void scale_min_k4(int j, uint32_t y, uint32_t z, uint32_t w, int &sc, int &m) {
    const int sh = 8 * (j & 3);
    const uint32_t by = y >> sh, bz = z >> sh, bw = w >> sh;
    if (j < 4) {
        sc = (int)(by & 63u);
        m = (int)(bz & 63u);
    } else {
        sc = (int)((bw & 15u) | (((by >> 6) & 3u) << 4));
        m = (int)(((bw >> 4) & 15u) | (((bz >> 6) & 3u) << 4));
    }
}

// Raw words of one lane's 4 values of a 256-value chunk, loaded for all the
// chunks of a wave before any of them is converted (one round trip per wave
// instead of one per chunk).
struct Raw {
    uint4 a;
    uint32_t b, c, d;
};

__device__ __forceinline__ Raw load_q4k(const GatherParams &p, int r, int b, int l) {
    const int g = l >> 4, t = 4 * (l & 15), lq = t & 31;
    Raw w;
    const uint8_t *hdr, *qs;
    if (p.layout == M27Q_LAYOUT_TILED) {
        const uint8_t *unit = p.W + ((size_t)(r / kTileRows) * p.upr + b) * kQ4KUnit;
        const int i = r % kTileRows;
        hdr = unit + 16 * i;
        qs = unit + q4k_tqs(i, g);  // qs bytes [32 g, 32 g + 32)
    } else {
        hdr = p.W + ((size_t)r * p.rb + b) * kQ4KBytes;
        qs = hdr + kQ4KHdr + 32 * g;
    }
    w.a = *(const uint4 *)hdr;
    w.b = *(const uint32_t *)(qs + lq);
    return w;
}
__device__ __forceinline__ float4 cvt_q4k(const Raw &w, int l) {
    const int g = l >> 4, t = 4 * (l & 15), hi = t >> 5, j = 2 * g + hi;
    int sc, m;
    scale_min_k4(j, w.a.y, w.a.z, w.a.w, sc, m);
    const float d1 = f16_bits_to_f32(w.a.x) * (float)sc;
    const float m1 = f16_bits_to_f32(w.a.x >> 16) * (float)m;
    const int sh = 4 * hi;
    const uint32_t q = w.b;
    return make_float4(d1 * (float)((q >> sh) & 15u) - m1, d1 * (float)((q >> (8 + sh)) & 15u) - m1,
                       d1 * (float)((q >> (16 + sh)) & 15u) - m1, d1 * (float)((q >> (24 + sh)) & 15u) - m1);
}

// Q5_K: the Q4_K words plus the 4 qh bytes of the lane's positions.
__device__ __forceinline__ Raw load_q5k(const GatherParams &p, int r, int b, int l) {
    const int g = l >> 4, t = 4 * (l & 15), lq = t & 31;
    Raw w;
    const uint8_t *hdr, *qs, *qh;
    if (p.layout == M27Q_LAYOUT_TILED) {
        const uint8_t *unit = p.W + ((size_t)(r / kTileRows) * p.upr + b) * kQ5KUnit;
        const int i = r % kTileRows;
        hdr = unit + 16 * i;
        qs = unit + q4k_tqs(i, g);  // qs bytes [32 g, 32 g + 32)
        qh = unit + kQ5KTQh + 32 * i;
    } else {
        hdr = p.W + ((size_t)r * p.rb + b) * kQ5KBytes;
        qs = hdr + kQ5KQs + 32 * g;
        qh = hdr + kQ5KQh;
    }
    w.a = *(const uint4 *)hdr;
    w.b = *(const uint32_t *)(qs + lq);
    w.c = *(const uint32_t *)(qh + lq);
    return w;
}
__device__ __forceinline__ float4 cvt_q5k(const Raw &w, int l) {
    const int g = l >> 4, t = 4 * (l & 15), hi = t >> 5, j = 2 * g + hi;
    int sc, m;
    scale_min_k4(j, w.a.y, w.a.z, w.a.w, sc, m);
    const float d1 = f16_bits_to_f32(w.a.x) * (float)sc;
    const float m1 = f16_bits_to_f32(w.a.x >> 16) * (float)m;
    const int sh = 4 * hi;
    float o[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const uint32_t q = ((w.b >> (8 * k + sh)) & 15u) | (((w.c >> (8 * k + j)) & 1u) << 4);
        o[k] = d1 * (float)q - m1;
    }
    return make_float4(o[0], o[1], o[2], o[3]);
}

__device__ __forceinline__ Raw load_q6k(const GatherParams &p, int r, int b, int l) {
    const int h = l >> 5, r4 = (l & 31) >> 3, lq = 4 * (l & 7);
    const int qlo = 64 * h + 32 * (r4 & 1) + lq, qho = 32 * h + lq, sci = 8 * h + lq / 16 + 2 * r4;
    Raw w;
    if (p.layout == M27Q_LAYOUT_TILED) {
        const uint8_t *unit = p.W + ((size_t)(r / kTileRows) * p.upr + b) * kQ6KUnit;
        const int i = r % kTileRows;
        w.b = *(const uint32_t *)(unit + kQ6KTQl + 128 * i + qlo);
        w.c = *(const uint32_t *)(unit + kQ6KTQh + 64 * i + qho);
        w.d = (uint32_t)(uint8_t)unit[kQ6KTSc + 16 * i + sci];
        w.a.x = *(const uint16_t *)(unit + kQ6KTD + 2 * i);
    } else {
        const uint8_t *blk = p.W + ((size_t)r * p.rb + b) * kQ6KBytes;
        w.b = ld_u32_a2(blk + kQ6KQl + qlo);
        w.c = ld_u32_a2(blk + kQ6KQh + qho);
        w.d = (uint32_t)(uint8_t)blk[kQ6KSc + sci];
        w.a.x = *(const uint16_t *)(blk + kQ6KD);
    }
    return w;
}
__device__ __forceinline__ float4 cvt_q6k(const Raw &w, int l) {
    const int r4 = (l & 31) >> 3;
    const int nib = 4 * (r4 >> 1), hs = 2 * r4;
    const float ds = f16_bits_to_f32(w.a.x) * (float)(int8_t)w.d;  // (d*sc)*q: the product order of exec:1046
    float o[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int q = (int)(((w.b >> (8 * k + nib)) & 15u) | (((w.c >> (8 * k + hs)) & 3u) << 4)) - 32;
        o[k] = ds * (float)q;
    }
    return make_float4(o[0], o[1], o[2], o[3]);
}

// IQ4_XS: lane l covers positions t .. t + 3 (t = 4 (l % 8)) of 32-group l / 8:
// the low (t < 16) or high nibbles of qs bytes 16 g + t % 16 .. + 4.
__device__ __forceinline__ Raw load_iq4xs(const GatherParams &p, int r, int b, int l) {
    const int g = l >> 3, t = 4 * (l & 7);
    Raw w;
    const uint8_t *hdr, *qs;
    if (p.layout == M27Q_LAYOUT_TILED) {
        const uint8_t *unit = p.W + ((size_t)(r / kTileRows) * p.upr + b) * kIQ4XSUnit;
        const int i = r % kTileRows;
        qs = unit + 128 * i;
        hdr = unit + kIQ4XSTHdr + 8 * i;
    } else {
        hdr = p.W + ((size_t)r * p.rb + b) * kIQ4XSBytes;
        qs = hdr + kIQ4XSQs;
    }
    const uint2 hd = *(const uint2 *)hdr;
    w.a.x = hd.x;
    w.a.y = hd.y;
    w.b = *(const uint32_t *)(qs + 16 * g + (t & 15));
    return w;
}
__device__ __forceinline__ float4 cvt_iq4xs(const Raw &w, int l) {
    const int g = l >> 3, t = 4 * (l & 7);
    const int ls = (int)(((w.a.y >> (8 * (g >> 1) + 4 * (g & 1))) & 15u) | (((w.a.x >> (16 + 2 * g)) & 3u) << 4));
    const float dl = f16_bits_to_f32(w.a.x) * (float)(ls - 32);
    const uint32_t v = iq4_lut((w.b >> (t < 16 ? 0 : 4)) & 0x0f0f0f0fu);
    return make_float4(dl * (float)(int8_t)v, dl * (float)(int8_t)(v >> 8), dl * (float)(int8_t)(v >> 16),
                       dl * (float)(int8_t)(v >> 24));
}

// Q8_0: the lane's 4 values start at position k4 of block b.
__device__ __forceinline__ Raw load_q80(const GatherParams &p, int r, int b, int k4) {
    Raw w;
    if (p.layout == M27Q_LAYOUT_TILED) {
        const uint8_t *unit = p.W + ((size_t)(r / kTileRows) * p.upr + b / kQ80UnitBlocks) * kQ80Unit;
        const int i = r % kTileRows, kk = b % kQ80UnitBlocks;
        w.b = *(const uint32_t *)(unit + 128 * i + 32 * kk + k4);
        w.a.x = *(const uint16_t *)(unit + kQ80TD + 8 * i + 2 * kk);
    } else {
        const uint8_t *blk = p.W + ((size_t)r * p.rb + b) * kQ80Bytes;
        w.b = ld_u32_a2(blk + 2 + k4);
        w.a.x = *(const uint16_t *)blk;
    }
    return w;
}
__device__ __forceinline__ float4 cvt_q80(const Raw &w) {
    const float d = f16_bits_to_f32(w.a.x);
    return make_float4(d * (float)(int8_t)w.b, d * (float)(int8_t)(w.b >> 8), d * (float)(int8_t)(w.b >> 16),
                       d * (float)(int8_t)(w.b >> 24));
}

constexpr int kGatherCpw = 8;  // chunks per wave in one workgroup column

__device__ __forceinline__ int gather_k(const GatherParams &p) {
    return p.type == kQ8_0 ? p.rb * 32 : (p.type == kF16 || p.type == kF32 ? p.rb : p.rb * 256);
}

// grid.x = output row; workgroup column blockIdx.y covers chunks
// [32 y, 32 y + 32): wave w takes chunks 32 y + 4 j + w, j < kGatherCpw.
template <uint32_t TYPE>
__global__ __launch_bounds__(256) void k_gather(GatherParams p) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int orow = (int)blockIdx.x;
    const int K = gather_k(p);
    const int nchunk = (K + 255) / 256;
    const int c0 = (int)blockIdx.y * 4 * kGatherCpw + wave;
    const int r = p.ids ? p.ids[orow] : p.row0 + orow;
    float *out = p.out + (size_t)orow * K;
    if (r < 0 || r >= p.rc) {
        for (int j = 0; j < kGatherCpw; ++j) {
            const int ch = c0 + 4 * j, pos = ch * 256 + 4 * lane;
            if (ch < nchunk && pos < K) *(float4 *)(out + pos) = make_float4(0.f, 0.f, 0.f, 0.f);
        }
        if (p.bad && blockIdx.y == 0 && threadIdx.x == 0) atomicAdd(p.bad, 1);
        return;
    }
    Raw w[kGatherCpw];
#pragma unroll
    for (int j = 0; j < kGatherCpw; ++j) {
        const int ch = min(c0 + 4 * j, nchunk - 1);  // past the end: reload the last chunk, store nothing
        const int pos = min(ch * 256 + 4 * lane, K - 4);
        if constexpr (TYPE == kQ4_K) w[j] = load_q4k(p, r, ch, lane);
        else if constexpr (TYPE == kQ5_K) w[j] = load_q5k(p, r, ch, lane);
        else if constexpr (TYPE == kIQ4_XS) w[j] = load_iq4xs(p, r, ch, lane);
        else if constexpr (TYPE == kQ6_K) w[j] = load_q6k(p, r, ch, lane);
        else if constexpr (TYPE == kQ8_0) w[j] = load_q80(p, r, pos / 32, pos % 32);  // K % 32 == 0
        else if constexpr (TYPE == kF16) {
            const uint2 h = *(const uint2 *)(p.W + ((size_t)r * K + pos) * 2);
            w[j].b = h.x;
            w[j].c = h.y;
        } else {
            w[j].a = *(const uint4 *)(p.W + ((size_t)r * K + pos) * 4);
        }
    }
#pragma unroll
    for (int j = 0; j < kGatherCpw; ++j) {
        const int ch = c0 + 4 * j, pos = ch * 256 + 4 * lane;
        if (ch >= nchunk || pos >= K) continue;
        float4 v;
        if constexpr (TYPE == kQ4_K) v = cvt_q4k(w[j], lane);
        else if constexpr (TYPE == kQ5_K) v = cvt_q5k(w[j], lane);
        else if constexpr (TYPE == kIQ4_XS) v = cvt_iq4xs(w[j], lane);
        else if constexpr (TYPE == kQ6_K) v = cvt_q6k(w[j], lane);
        else if constexpr (TYPE == kQ8_0) v = cvt_q80(w[j]);
        else if constexpr (TYPE == kF16)
            v = make_float4(f16_bits_to_f32(w[j].b), f16_bits_to_f32(w[j].b >> 16), f16_bits_to_f32(w[j].c),
                            f16_bits_to_f32(w[j].c >> 16));
        else v = make_float4(__uint_as_float(w[j].a.x), __uint_as_float(w[j].a.y), __uint_as_float(w[j].a.z),
                             __uint_as_float(w[j].a.w));
        *(float4 *)(out + pos) = v;
    }
}

hipError_t launch_gather(const GatherParams &p, hipStream_t s) {
    const int K = p.type == kQ8_0 ? p.rb * 32 : (is_quant(p.type) ? p.rb * 256 : p.rb);
    const int chunks = (K + 255) / 256;
    const dim3 grid(p.n, (chunks + 4 * kGatherCpw - 1) / (4 * kGatherCpw)), block(256);
    switch (p.type) {
        case kQ4_K: hipLaunchKernelGGL(k_gather<kQ4_K>, grid, block, 0, s, p); break;
        case kQ5_K: hipLaunchKernelGGL(k_gather<kQ5_K>, grid, block, 0, s, p); break;
        case kIQ4_XS: hipLaunchKernelGGL(k_gather<kIQ4_XS>, grid, block, 0, s, p); break;
        case kQ6_K: hipLaunchKernelGGL(k_gather<kQ6_K>, grid, block, 0, s, p); break;
        case kQ8_0: hipLaunchKernelGGL(k_gather<kQ8_0>, grid, block, 0, s, p); break;
        case kF16: hipLaunchKernelGGL(k_gather<kF16>, grid, block, 0, s, p); break;
        default: hipLaunchKernelGGL(k_gather<kF32>, grid, block, 0, s, p); break;
    }
    return hipGetLastError();
}

}  // namespace m27q
