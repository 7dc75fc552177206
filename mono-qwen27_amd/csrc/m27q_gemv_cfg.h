// m27q_gemv_cfg.h -- launch configurations of the integer-dot GEMV.
//
//  KS  : wavefronts per workgroup; each streams one K slice of every tile
//  TPW : 8-row tiles per workgroup (every wave covers all of them)
//
// Measured on MI355X with cold weights (rotated copies >= 2 x the 256 MB
// Infinity Cache), fp32 input, average over graph-replayed launches:
//  OutQ  4,4 : fused gate/up 2 x 17408 x 5120 Q4_K + output quantization
//  ShortK 8,4: q/k/v 8192 x 5120 and o 5120 x 6144 Q4_K
//  LongK 4,1 : down 5120 x 17408 Q6_K (quantized input)
//
// Chosen per call from the shape (m27q_api.hip, pick_gemv_cfg):
//  OutQ   : every product that quantizes its output (32-row workgroups)
//  ShortK : K of up to 24 units (5120 / 6144 inputs)
//  MidK   : 25 .. 39 units
//  LongK  : 40 units and more (the 17408-input down projection: 68 units)
// Each can be overridden at build time (-DM27Q_CFG_SHORT=KS,TPW) to sweep.
#pragma once

namespace m27q {

template <int KS_, int TPW_>
struct GemvCfg {
    static constexpr int KS = KS_, TPW = TPW_;
    static_assert(KS >= 1 && KS <= 16 && TPW >= 1 && TPW <= 8, "bad GEMV configuration");
};

#ifndef M27Q_CFG_OUTQ
#define M27Q_CFG_OUTQ 4, 4
#endif
#ifndef M27Q_CFG_SHORT
#define M27Q_CFG_SHORT 8, 4
#endif
#ifndef M27Q_CFG_MID
#define M27Q_CFG_MID 4, 2
#endif
#ifndef M27Q_CFG_LONG
#define M27Q_CFG_LONG 4, 1
#endif

using CfgOutQ = GemvCfg<M27Q_CFG_OUTQ>;
using CfgShortK = GemvCfg<M27Q_CFG_SHORT>;
using CfgMidK = GemvCfg<M27Q_CFG_MID>;
using CfgLongK = GemvCfg<M27Q_CFG_LONG>;

enum { kCfgShortK = 0, kCfgMidK = 1, kCfgLongK = 2, kCfgOutQ = 3 };

static_assert(CfgOutQ::TPW * 8 % 32 == 0, "the output-quantizing products need 32-row workgroups");

}  // namespace m27q
