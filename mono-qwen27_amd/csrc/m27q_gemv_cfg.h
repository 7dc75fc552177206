// m27q_gemv_cfg.h -- launch configurations of the integer-dot GEMV.
//
//  KS  : K slices per tile; wave (ks, g) streams slice ks of its tile group g
//  TPW : 8-row tiles per workgroup
//  WT  : tiles per wave (TPW / WT tile groups), so a workgroup has
//        NW = KS * TPW / WT wavefronts
//
// More, shorter wavefronts stream HBM better, but every workgroup stages (and,
// for fp32 input, quantizes) the whole activation, so the best shape depends
// on the input form, the row count and K.  Measured on MI355X with cold
// weights (rotated copies >= 2 x the 256 MB Infinity Cache), average per
// graph-replayed launch including the dispatch gap:
//
//   product (TILED)                          fp32 x in           quantized x in
//   q/k/v 6144+1024+1024 x 5120 Q4_K         (8,4)  7.00 us      (4,1) 6.69 us
//   o 5120 x 6144 Q4_K                       (8,1)  6.77 us      (8,1) 6.01 us
//   gate/up SwiGLU 2 x 17408 x 5120 Q4_K     (4,1) 20.91 us      (8,1) 20.19 us
//   down 5120 x 17408 Q6_K                   (4,1) 21.30 us      (4,1) 17.09 us
//   gate/up + fused output quantization      (2,4,1) 24.55 us    (2,4,1) 23.38 us
//   Q4_K 17408 x 5120 alone                  (4,2) 11.92 us
//   LM head Q6_K 248320 x 5120               (4,2) 165.2 us (6.31 TB/s)
// (shapes written (KS, TPW) have WT = TPW).
//
// Products that quantize their output (yq) need whole 32-row groups per
// workgroup (TPW >= 4) and use CfgQ.  GGUF-layout weights (the compatibility
// path) use one shape.  Each can be overridden at build time
// (-DM27Q_CFG_41=KS,TPW,WT ...) to sweep.
#pragma once

namespace m27q {

template <int KS_, int TPW_, int WT_>
struct GemvCfg {
    static constexpr int KS = KS_, TPW = TPW_, WT = WT_, NW = KS_ * TPW_ / WT_;
    static_assert(KS >= 1 && TPW >= 1 && WT >= 1 && TPW % WT == 0, "bad GEMV configuration");
    static_assert(NW >= 1 && NW <= 16, "a workgroup holds at most 16 wavefronts");
};

#ifndef M27Q_CFG_41
#define M27Q_CFG_41 4, 1, 1
#endif
#ifndef M27Q_CFG_81
#define M27Q_CFG_81 8, 1, 1
#endif
#ifndef M27Q_CFG_42
#define M27Q_CFG_42 4, 2, 2
#endif
#ifndef M27Q_CFG_84
#define M27Q_CFG_84 8, 4, 4
#endif
#ifndef M27Q_CFG_Q
#define M27Q_CFG_Q 2, 4, 1
#endif

using Cfg41 = GemvCfg<M27Q_CFG_41>;
using Cfg81 = GemvCfg<M27Q_CFG_81>;
using Cfg42 = GemvCfg<M27Q_CFG_42>;
using Cfg84 = GemvCfg<M27Q_CFG_84>;
using CfgQ = GemvCfg<M27Q_CFG_Q>;
static_assert(CfgQ::TPW * 8 % 32 == 0, "output-quantizing workgroups hold whole 32-row groups");

enum { kCfg41 = 0, kCfg81 = 1, kCfg42 = 2, kCfg84 = 3, kCfgQ = 4 };

// Host-side choice for a product of rows_total output rows (all matrices of a
// multi-matrix launch) over upr units per row.
inline int pick_gemv_cfg(bool tiled, bool xf32, bool swiglu, bool out_quant, long long rows_total, int upr) {
    if (out_quant) return kCfgQ;
    if (!tiled) return kCfg41;
    if (upr >= 40) return kCfg41;
    if (swiglu) return xf32 ? kCfg41 : kCfg81;
    if (rows_total <= 12288) {
        if (upr >= 24) return kCfg81;
        return xf32 ? kCfg84 : kCfg41;
    }
    return kCfg42;
}

}  // namespace m27q
