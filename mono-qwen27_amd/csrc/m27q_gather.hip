// m27q_gather.hip -- row gather + dequantization to fp32 (bit-exact).
//
// One wavefront dequantizes 256 consecutive values of one row (one Q4_K/Q6_K
// block, eight Q8_0 blocks, or 256 F16/F32 elements): lane l produces values
// 4l .. 4l+3 and stores them as one float4, so a wave writes 1 KiB contiguous.
// Generalizes k_q4k_embed (exec:1233-1254: one Q4_K row, one workgroup) to any
// supported type/layout and to a device array of row ids.
#include "m27q_internal.h"
#include "m27q_device.h"

namespace m27q {

__device__ __forceinline__ void scale_min_k4(int j, const uint8_t *q, int &sc, int &m) {
    // get_scale_min_k4, exec:690-693
    if (j < 4) {
        sc = q[j] & 63;
        m = q[j + 4] & 63;
    } else {
        sc = (q[j + 4] & 0x0f) | ((q[j - 4] >> 6) << 4);
        m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
    }
}

// Byte address of block b of row r in either layout (K-quants).
template <int BB, int UNIT>
__device__ __forceinline__ const uint8_t *unit_of(const GatherParams &p, int r, int b) {
    return p.W + ((size_t)(r / kTileRows) * p.upr + b) * UNIT;
}

__device__ float4 deq_q4k(const GatherParams &p, int r, int b, int l) {
    const int g = l >> 4, t = 4 * (l & 15), hi = t >> 5, lq = t & 31, j = 2 * g + hi;
    const uint8_t *hdr, *qs;
    if (p.layout == M27Q_LAYOUT_TILED) {
        const uint8_t *unit = unit_of<kQ4KBytes, kQ4KUnit>(p, r, b);
        const int i = r % kTileRows;
        hdr = unit + 16 * i;
        qs = unit + 128 + 128 * i;
    } else {
        hdr = p.W + ((size_t)r * p.rb + b) * kQ4KBytes;
        qs = hdr + kQ4KHdr;
    }
    const uint4 h = *(const uint4 *)hdr;
    const uint32_t sc12[3] = {h.y, h.z, h.w};
    int sc, m;
    scale_min_k4(j, (const uint8_t *)sc12, sc, m);
    const uint32_t w = *(const uint32_t *)(qs + 32 * g + lq);
    const float d1 = f16_bits_to_f32(h.x) * (float)sc;
    const float m1 = f16_bits_to_f32(h.x >> 16) * (float)m;
    const int sh = 4 * hi;
    return make_float4(d1 * (float)((w >> sh) & 15u) - m1, d1 * (float)((w >> (8 + sh)) & 15u) - m1,
                       d1 * (float)((w >> (16 + sh)) & 15u) - m1, d1 * (float)((w >> (24 + sh)) & 15u) - m1);
}

__device__ float4 deq_q6k(const GatherParams &p, int r, int b, int l) {
    const int h = l >> 5, r4 = (l & 31) >> 3, lq = 4 * (l & 7);
    const int qlo = 64 * h + 32 * (r4 & 1) + lq, qho = 32 * h + lq, sci = 8 * h + lq / 16 + 2 * r4;
    uint32_t ql, qh;
    int sc;
    float d;
    if (p.layout == M27Q_LAYOUT_TILED) {
        const uint8_t *unit = unit_of<kQ6KBytes, kQ6KUnit>(p, r, b);
        const int i = r % kTileRows;
        ql = *(const uint32_t *)(unit + kQ6KTQl + 128 * i + qlo);
        qh = *(const uint32_t *)(unit + kQ6KTQh + 64 * i + qho);
        sc = (int)((const int8_t *)(unit + kQ6KTSc + 16 * i))[sci];
        d = f16_bits_to_f32(*(const uint16_t *)(unit + kQ6KTD + 2 * i));
    } else {
        const uint8_t *blk = p.W + ((size_t)r * p.rb + b) * kQ6KBytes;
        ql = ld_u32_a2(blk + kQ6KQl + qlo);
        qh = ld_u32_a2(blk + kQ6KQh + qho);
        sc = (int)((const int8_t *)(blk + kQ6KSc))[sci];
        d = f16_bits_to_f32(*(const uint16_t *)(blk + kQ6KD));
    }
    const int nib = 4 * (r4 >> 1), hs = 2 * r4;
    const float ds = d * (float)sc;  // (d*sc)*q: the product order of exec:1046 (signed zeros)
    float o[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int q = (int)(((ql >> (8 * k + nib)) & 15u) | (((qh >> (8 * k + hs)) & 3u) << 4)) - 32;
        o[k] = ds * (float)q;
    }
    return make_float4(o[0], o[1], o[2], o[3]);
}

__device__ float4 deq_q80(const GatherParams &p, int r, int b, int k4) {
    float d;
    uint32_t w;
    if (p.layout == M27Q_LAYOUT_TILED) {
        const uint8_t *unit = p.W + ((size_t)(r / kTileRows) * p.upr + b / kQ80UnitBlocks) * kQ80Unit;
        const int i = r % kTileRows, kk = b % kQ80UnitBlocks;
        w = *(const uint32_t *)(unit + 128 * i + 32 * kk + k4);
        d = f16_bits_to_f32(*(const uint16_t *)(unit + kQ80TD + 8 * i + 2 * kk));
    } else {
        const uint8_t *blk = p.W + ((size_t)r * p.rb + b) * kQ80Bytes;
        w = ld_u32_a2(blk + 2 + k4);
        d = f16_bits_to_f32(*(const uint16_t *)blk);
    }
    return make_float4(d * (float)(int8_t)w, d * (float)(int8_t)(w >> 8), d * (float)(int8_t)(w >> 16),
                       d * (float)(int8_t)(w >> 24));
}

// grid.x = output row, grid.y * 4 + wave = 256-value chunk of the row.
__global__ __launch_bounds__(256) void k_gather(GatherParams p) {
    const int lane = threadIdx.x & 63, chunk = (int)blockIdx.y * 4 + (threadIdx.x >> 6);
    const int orow = (int)blockIdx.x;
    const int K = p.type == kQ8_0 ? p.rb * 32 : (p.type == kQ4_K || p.type == kQ6_K ? p.rb * 256 : p.rb);
    const int pos = chunk * 256 + 4 * lane;
    if (pos >= K) return;
    const int r = p.ids ? p.ids[orow] : p.row0 + orow;
    float4 *dst = (float4 *)(p.out + (size_t)orow * K + pos);
    if (r < 0 || r >= p.rc) {
        *dst = make_float4(0.f, 0.f, 0.f, 0.f);
        if (p.bad && pos == 0) atomicAdd(p.bad, 1);
        return;
    }
    float4 v;
    switch (p.type) {
        case kQ4_K: v = deq_q4k(p, r, chunk, lane); break;
        case kQ6_K: v = deq_q6k(p, r, chunk, lane); break;
        case kQ8_0: v = deq_q80(p, r, chunk * 8 + (lane >> 3), 4 * (lane & 7)); break;
        case kF16: {
            const uint2 h = *(const uint2 *)(p.W + ((size_t)r * K + pos) * 2);
            v = make_float4(f16_bits_to_f32(h.x), f16_bits_to_f32(h.x >> 16), f16_bits_to_f32(h.y),
                            f16_bits_to_f32(h.y >> 16));
            break;
        }
        default: v = *(const float4 *)(p.W + ((size_t)r * K + pos) * 4); break;
    }
    *dst = v;
}

hipError_t launch_gather(const GatherParams &p, hipStream_t s) {
    const int K = p.type == kQ8_0 ? p.rb * 32 : (p.type == kQ4_K || p.type == kQ6_K ? p.rb * 256 : p.rb);
    const int chunks = (K + 255) / 256;
    hipLaunchKernelGGL(k_gather, dim3(p.n, (chunks + 3) / 4), dim3(256), 0, s, p);
    return hipGetLastError();
}

}  // namespace m27q
