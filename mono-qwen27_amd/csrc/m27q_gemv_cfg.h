// m27q_gemv_cfg.h -- launch configurations of the integer-dot GEMV.
//
//  KS  : K slices per tile; wave (ks, g) streams slice ks of its tile group g
//  TPW : 8-row tiles per workgroup
//  WT  : tiles per wave (TPW / WT tile groups), so a workgroup has
//        NW = KS * TPW / WT wavefronts
//  NT  : 1 = non-temporal weight loads (global_load_dwordx4 ... nt)
//
// Non-temporal weight loads were measured per shape, every product on cold
// weights: gate/up 18.6-19.0 us against 20.2, down 16.5-16.8 against 17.9,
// config 1 11.1 against 12.0, the LM head 152 against 164; q/k/v and o were
// 0.3-0.6 us faster alone with them, but the decode layer (q/k/v, o, gate/up,
// down in one graph) was 0.4-0.6 us slower with them on q/k/v and 0.3-0.7 us
// slower with them on o, in two sessions, so those two shapes keep temporal
// loads.  With the choices below the layer took 46.3-46.6 us against 50.2-50.4
// with temporal loads everywhere.
//
// More, shorter wavefronts stream HBM better, but every workgroup stages (and,
// for fp32 input, quantizes) the whole activation, so the best shape depends
// on the input form, the row count and K.  Measured on MI355X with cold
// weights (rotated copies >= 2 x the 256 MB Infinity Cache), average per
// graph-replayed launch including the dispatch gap:
//
//   product (TILED)                          fp32 x in           quantized x in
//   q/k/v 6144+1024+1024 x 5120 Q4_K         (8,4)  7.00 us      (4,1) 6.69 us
//     (later, in graphs of 32 launches: (8,4,2) 5.95, (8,2,2) 5.96,
//     (8,4,4) 6.00, (16,4,4) 6.39, (4,4,2) 6.54, (4,4,4) 7.20, (8,2,1) 7.37;
//     the layer 0.45 us faster with (8,4,2) in two sessions; at M = 2 q/k/v
//     7.8 against 8.4)
//   o 5120 x 6144 Q4_K                       (8,2,2) 7.51 us     (8,1) 6.01 us
//                                            (8,1) 7.88, (6,2,1) 7.98, (4,2,2) 8.24
//     (with the chunk-pair-first qs plane, in graphs of 32 launches:
//     (8,4,2) 6.23, (8,1,1) 6.28, (8,2,2) 6.59, (16,1,1) 7.42, (4,2,2) 7.63;
//     the layer 46.09 against 46.28 us with (8,4,2), median of six rounds)
//   gate/up SwiGLU 2 x 17408 x 5120 Q4_K     (4,1) 20.91 us      (8,1) 20.19 us
//   down 5120 x 17408 Q6_K                   (4,1) 21.30 us      (4,1) 17.09 us
//   gate/up + fused output quantization      (2,4,2) 24.2 us (2,4,1) 24.85, (4,4,4) 24.4,
//                                            (1,4,1) 24.65, (4,4,1) 26.3, (2,4,4) 26.9
//   Q4_K 17408 x 5120 alone                  (4,2) 11.92 us
//   LM head Q6_K 248320 x 5120               (4,2) 164.1 us (6.36 TB/s)
//   Q8_0 2048 x 2048 (draft)                 (16,1) 3.43 us, (8,1) 3.70, (8,4) 4.32
//   Q8_0 6144 x 2048 (draft)                 (8,1)  4.83 us, (8,4) 5.12, (16,1) 6.78
//   Q8_0 2048 x 6144 (draft)                 (16,1) 5.26 us, (8,1) 5.78, (4,1) 6.80
// (shapes written (KS, TPW) have WT = TPW; figures from when they were
// chosen, before the cheaper activation quantizer).  Small products need more
// waves per row than their row count provides: 2048 rows are 256 tiles, one
// per CU.
//
// A launch ends with its most loaded CUs (the memory system shares bandwidth
// roughly per CU), so how evenly the workgroups spread over the 256 CUs
// matters as much as their shape:
//   - products that quantize their output (yq) in the kernel need whole 32-row
//     groups per workgroup (TPW >= 4) and use CfgQ; SwiGLU products instead
//     take their own shape and leave the quantization to a second launch (544
//     32-row workgroups put 3 on 32 CUs: (4,1) + the quantizer 23.05 us
//     against 23.93 in one launch);
//   - a single product with 2 to 3 tiles per CU (down, 640 tiles) takes CfgB
//     with balanced tiling, one workgroup per CU (on a quantized x 15.8 us
//     against 16.45 with one tile per workgroup; on an fp32 x, quantized by
//     every workgroup, 17.3 us against 19.7, but only on rows of 10240
//     columns or more: o's 6144 measured slower).
// GGUF-layout weights (the compatibility
// path) follow the same rules: q/k/v 7.97 us and o 7.83 with them against 8.66
// and 8.20 on (4,1) alone; gate/up and down pay for the row-major blocks
// (30.6 and 21.6 us against 24.2 and 16.4 TILED).
#pragma once

#include <cstdint>

#include "m27q_layout.h"

namespace m27q {

template <int KS_, int TPW_, int WT_, int NT_ = 1>
struct GemvCfg {
    static constexpr int KS = KS_, TPW = TPW_, WT = WT_, NW = KS_ * TPW_ / WT_;
    static constexpr bool NT = NT_ != 0;  // non-temporal weight loads
    static_assert(KS >= 1 && TPW >= 1 && WT >= 1 && TPW % WT == 0, "bad GEMV configuration");
    static_assert(NW >= 1 && NW <= 16, "a workgroup holds at most 16 wavefronts");
};

using Cfg41 = GemvCfg<4, 1, 1, 1>;
using Cfg81 = GemvCfg<8, 1, 1, 1>;
using Cfg42 = GemvCfg<4, 2, 2, 1>;
using Cfg84 = GemvCfg<8, 4, 2, 0>;
using CfgQ = GemvCfg<2, 4, 2, 1>;
using Cfg161 = GemvCfg<16, 1, 1, 1>;
using CfgB = GemvCfg<4, 3, 1, 1>;  // balanced tiling (GemvParams::bal), up to TPW tiles per workgroup
using CfgB9 = GemvCfg<5, 9, 3, 1>;  // balanced tiling for 8-9 tiles per CU (config 1); swept against
                                     // (4, 9, 3) +0.3, (3, 9, 3) +0.5, (8, 9, 9) +0.4, (4, 9, 9) +1.8,
                                     // (2, 9, 3) +1.5 us
static_assert(CfgQ::TPW * 8 % 32 == 0, "output-quantizing workgroups hold whole 32-row groups");
static_assert(Cfg161::TPW == Cfg41::TPW, "a fallback instantiation keeps the grid's tiles per workgroup");

enum { kCfg41 = 0, kCfg81 = 1, kCfg42 = 2, kCfg84 = 3, kCfgQ = 4, kCfg161 = 5, kCfgB = 7, kCfgB9 = 8 };

// Host-side choice for a product of rows_total output rows (all matrices of a
// multi-matrix launch) of one weight type and layout over upr units per row.
// Q6_K on an fp32 x at 6144-12288 rows takes (4, 1, 1) where Q4_K takes
// (8, 4, 2): the SSM layer's wqkv (Q6_K 10240 x 5120) measured 9.8 us against
// 12.9 (cold copies, events); the other shapes measured within 0.3 us of each
// other or slower for Q6_K, Q5_K 6144 x 5120 and IQ4_XS 17408 x 5120.  On
// GGUF-layout weights o's shape (24-39 units, fp32 x) takes (4, 1, 1) too:
// 7.0 us against 8.1 with (8, 2, 2); q/k/v, gate/up, down and the LM head
// measured best with the TILED choices.
inline int pick_gemv_cfg(uint32_t type, bool tiled, bool xf32, bool swiglu, bool out_quant, long long rows_total,
                         int upr) {
    if (out_quant) return kCfgQ;
    if (swiglu) return upr >= 40 || xf32 ? kCfg41 : kCfg81;
    if (upr >= 40) return rows_total <= 4096 ? kCfg161 : kCfg41;
    if (rows_total <= 12288) {
        if (upr >= 24) return xf32 ? (tiled ? kCfg84 : kCfg41) : kCfg81;
        if (!xf32) return kCfg41;
        if (rows_total <= 2048) return kCfg161;
        if (rows_total <= 6144) return kCfg81;
        return type == kQ6_K ? kCfg41 : kCfg84;
    }
    return kCfg42;
}

}  // namespace m27q
