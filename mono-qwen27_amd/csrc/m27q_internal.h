// m27q_internal.h -- kernel launch interface between the C ABI and the kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "../../include/m27q.h"
#include "m27q_gemv_cfg.h"
#include "m27q_layout.h"

namespace m27q {

constexpr int kMaxMulti = 4;  // weights sharing one activation in one launch

struct GemvParams {
    const uint8_t *W[kMaxMulti];
    float *y[kMaxMulti];
    const float *res[kMaxMulti];
    int rc[kMaxMulti];
    int wg_start[kMaxMulti + 1];  // first workgroup of each weight
    int nmat;
    int rb;   // GGUF blocks per row (K elements for F16 / F32)
    int upr;  // layout units per row
    int K;    // activation length
    // int8 activation (m27q_quant_act format) ...
    const int8_t *xq;
    const float *xd;
    const uint32_t *xs;
    // ... or fp32 activation
    const float *x;
    // balanced tiling: workgroup w of matrix m (G workgroups, T tiles) owns
    // tiles [w T / G, (w + 1) T / G), at most C::TPW of them
    int bal;
    // optional fused quantization of the output vector
    int8_t *oq;
    float *od;
    uint32_t *os;
};

// Integer-dot GEMV (m27q_gemv.hip).  cfg: a launch shape of m27q_gemv_cfg.h
// (pick_gemv_cfg).  The grid is p.wg_start[p.nmat] workgroups.  The
// activation is p.x (fp32, quantized in the kernel) when not NULL, else p.xq.
size_t gemv_q8_lds_bytes(uint32_t type, int upr, bool swiglu, int cfg);
int gemv_q8_tiles_per_wg(int cfg);
hipError_t launch_gemv_q8(uint32_t type, int layout, bool swiglu, int cfg, const GemvParams &p, hipStream_t s);
size_t gemv_f32_lds_bytes(uint32_t type, int upr);
hipError_t launch_gemv_f32(uint32_t type, int layout, const GemvParams &p, int grid, hipStream_t s);

hipError_t launch_quant_act(const float *x, const float *gate, long long n, int8_t *q, float *d, uint32_t *s,
                            hipStream_t st);

struct GatherParams {
    const uint8_t *W;
    uint32_t type;
    int layout;
    int rb, rc, upr;
    const int32_t *ids;  // device ids, or NULL: rows row0 + i
    int row0;
    int n;
    float *out;
    int32_t *bad;
};
hipError_t launch_gather(const GatherParams &p, hipStream_t s);

size_t topk_scratch_bytes(int n);
// The top-k scratch array of m27q_topk.hip (static, per device): its size, and
// its device address on the current device (resolved on the first call there).
size_t topk_static_scratch_bytes();
hipError_t topk_static_scratch(void **ptr);
hipError_t launch_topk(const float *v, int n, int k, int32_t *idx, float *val, void *scratch, hipStream_t s);
hipError_t launch_sample(const int32_t *idx, const float *val, int k, float temperature, float min_p, float top_p,
                         const float *u, int32_t *token, hipStream_t s);

struct MatmulParams {
    const uint8_t *W;
    int rb, rc, upr, K, M;
    const int8_t *xq;
    const float *xd;
    const uint32_t *xs;
    float *Y;
    const float *res;
};

// Small-M products over up to kMaxMulti weights that share the activation (same
// type, layout and K), in one launch.
struct MatmulMultiParams {
    const uint8_t *W[kMaxMulti];
    float *Y[kMaxMulti];
    const float *res[kMaxMulti];
    int rc[kMaxMulti];
    int wg_start[kMaxMulti + 1];
    int nmat;
    int upr, K, M;
    int rb;  // GGUF blocks per row (the few-token kernel's GGUF rows)
    const int8_t *xq;
    const float *xd;
    const uint32_t *xs;
    // few-token kernel only: when > 0, balanced tiling over this many
    // workgroups for the one matrix (as GemvParams::bal)
    int bal_wgs;
};
hipError_t launch_matmul_q8(uint32_t type, int layout, const MatmulParams &p, hipStream_t s);
// Few-token products on the GEMV streaming structure (m27q_gemv_mt.hip): two
// activation rows, either layout.  matmul_mt_balance(): the balanced
// workgroup count for one matrix of `tiles` tiles of `upr` units on `cus`
// CUs, or 0.
size_t matmul_mt_lds_bytes(uint32_t type, int upr);
int matmul_mt_balance(long long tiles, int upr, int cus);
hipError_t launch_matmul_mt(uint32_t type, int layout, const MatmulMultiParams &p, hipStream_t s);
// int8-MFMA small-M products (m27q_mma.hip): TILED weights of every type and
// GGUF-layout Q4_K / Q5_K / Q6_K (matmul_mfma_takes), any M (16 tokens per
// launch).
size_t matmul_mfma_lds_bytes(uint32_t type);
bool matmul_mfma_takes(uint32_t type, int layout);
// Whether its weight operands go straight into registers (TILED Q4_K / Q5_K).
bool matmul_mfma_direct(uint32_t type, int layout);
// The current device's CU count and LDS bytes per workgroup (cached per device).
int cu_count();
size_t lds_limit();
hipError_t launch_matmul_mfma(uint32_t type, int layout, const MatmulMultiParams &p, hipStream_t s);

}  // namespace m27q
