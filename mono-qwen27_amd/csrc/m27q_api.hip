// m27q_api.hip -- extern "C" entry points: argument validation, then launches.
//
// Every check runs on the host before the first HIP call, so a bad argument
// returns a status without touching the device (the reference's launchers
// return silently instead, exec:2034, :2056-2059).
#include <atomic>
#include <cmath>

#include "m27q_internal.h"

using namespace m27q;

namespace {

constexpr size_t kActAlign = 256;
constexpr int kMaxK = 1 << 20;
// Rows per weight: one-tile workgroups of up to 1024 threads keep every grid
// below 2^32 work-items (the dispatch packet's limit).
constexpr uint32_t kMaxRows = 1u << 24;
constexpr int kMaxM = 64;
constexpr int kMaxTopK = 64;

size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

bool aligned(const void *p, size_t a) { return ((uintptr_t)p % a) == 0; }

// An attribute of the current device, cached per device (a partitioned
// MI355X shows fewer CUs per device, and a process may drive several).
// Concurrent first calls may both query; they store the same value.
constexpr int kMaxDevices = 64;
int device_attr(hipDeviceAttribute_t a, std::atomic<int> (&cache)[kMaxDevices], int fallback) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0) return fallback;
    if (dev < kMaxDevices) {
        const int c = cache[dev].load(std::memory_order_relaxed);
        if (c > 0) return c;
    }
    int v = 0;
    if (hipDeviceGetAttribute(&v, a, dev) != hipSuccess || v <= 0) return fallback;
    if (dev < kMaxDevices) cache[dev].store(v, std::memory_order_relaxed);
    return v;
}

}  // namespace

// Compute units of the current device (256 on MI355X), for balanced tiling.
int m27q::cu_count() {
    static std::atomic<int> cache[kMaxDevices];
    return device_attr(hipDeviceAttributeMultiprocessorCount, cache, 256);
}

// LDS limit of one workgroup on the current device (160 KiB on gfx950).
size_t m27q::lds_limit() {
    static std::atomic<int> cache[kMaxDevices];
    return (size_t)device_attr(hipDeviceAttributeMaxSharedMemoryPerBlock, cache, 64 * 1024);
}

namespace {

int k_of(const m27q_weight *w) { return (int)w->row_blocks * block_elems(w->ggml_type); }

// Shared weight checks.  quant_only: the integer-dot types (Q4_K, Q5_K,
// Q6_K, Q8_0, IQ4_XS), not F16 / F32.
m27q_status check_weight(const m27q_weight *w, bool quant_only) {
    if (!w || !w->ptr) return M27Q_ERR_NULL;
    const uint32_t t = w->ggml_type;
    if (!block_elems(t)) return M27Q_ERR_TYPE;
    if (quant_only && !is_quant(t)) return M27Q_ERR_TYPE;
    if (w->row_blocks == 0 || w->row_count == 0 || w->row_count > kMaxRows) return M27Q_ERR_SHAPE;
    if ((long long)w->row_blocks * block_elems(t) > kMaxK) return M27Q_ERR_SHAPE;
    if (w->layout == M27Q_LAYOUT_TILED) {
        if (!is_quant(t)) return M27Q_ERR_LAYOUT;
        if (!aligned(w->ptr, 16)) return M27Q_ERR_LAYOUT;
    } else if (w->layout == M27Q_LAYOUT_GGUF) {
        const size_t need = (t == kQ6_K || t == kQ8_0) ? 2 : (t == kIQ4_XS ? 8 : 16);
        if (!aligned(w->ptr, need)) return M27Q_ERR_LAYOUT;
        if (t == kF16 && (w->row_blocks % 8)) return M27Q_ERR_SHAPE;
        if (t == kF32 && (w->row_blocks % 4)) return M27Q_ERR_SHAPE;
    } else {
        return M27Q_ERR_LAYOUT;
    }
    return M27Q_OK;
}

struct ActView {
    const int8_t *q;
    const float *d;
    const uint32_t *s;
};

ActView act_view(const void *xq, int M, int K) {
    const uint8_t *b = (const uint8_t *)xq;
    return {(const int8_t *)b, (const float *)(b + m27q_act_d_offset(M, K)),
            (const uint32_t *)(b + m27q_act_s_offset(M, K))};
}

int wg_count(int rows) { return ((rows + kTileRows - 1) / kTileRows + kWavesPerWG - 1) / kWavesPerWG; }

m27q_status hip_status(hipError_t e) { return e == hipSuccess ? M27Q_OK : M27Q_ERR_HIP; }

m27q_status check_out_quant(const m27q_weight *w, const void *yq) {
    if (!yq) return M27Q_OK;
    if (!aligned(yq, 16)) return M27Q_ERR_LAYOUT;
    if (w->row_count % 32) return M27Q_ERR_SHAPE;
    return M27Q_OK;
}

// Shared body of every integer-dot M = 1 product.  n weights of one type,
// layout and K share the activation (fp32 x, or the quantized xq); with
// swiglu, ws = {gate, up} and ys[0] receives silu(gate x) * (up x).  With
// dry, every check runs and nothing is launched.
m27q_status gemv_impl(int n, const m27q_weight *ws, const void *xq, const float *x, float *const *ys,
                      const float *residual, bool swiglu, void *yq, hipStream_t stream, bool dry = false) {
    if (!ws || !ys) return M27Q_ERR_NULL;
    if (n < 1 || n > kMaxMulti || (swiglu && n != 2)) return M27Q_ERR_SHAPE;
    for (int i = 0; i < n; ++i) {
        const m27q_status st = check_weight(&ws[i], true);
        if (st != M27Q_OK) return st;
        if (ws[i].ggml_type != ws[0].ggml_type) return M27Q_ERR_TYPE;
        if (ws[i].layout != ws[0].layout) return M27Q_ERR_LAYOUT;
        if (ws[i].row_blocks != ws[0].row_blocks) return M27Q_ERR_SHAPE;
        if (swiglu && ws[i].row_count != ws[0].row_count) return M27Q_ERR_SHAPE;
    }
    const int nout = swiglu ? 1 : n;
    for (int i = 0; i < nout; ++i)
        if (!ys[i]) return M27Q_ERR_NULL;
    if (!xq && !x) return M27Q_ERR_NULL;
    if (xq && !aligned(xq, 16)) return M27Q_ERR_LAYOUT;
    if (x && !aligned(x, 16)) return M27Q_ERR_LAYOUT;
    if (yq && nout != 1) return M27Q_ERR_SHAPE;
    m27q_status st = check_out_quant(&ws[0], yq);
    if (st != M27Q_OK) return st;

    GemvParams p{};
    p.rb = (int)ws[0].row_blocks;
    p.upr = units_per_row(ws[0].ggml_type, ws[0].row_blocks);
    p.K = k_of(&ws[0]);
    long long rows_total = 0;
    for (int i = 0; i < n; ++i) rows_total += ws[i].row_count;
    if (swiglu) rows_total = ws[0].row_count;
    // A SwiGLU product quantizes its output in a second launch (the quantizer
    // of m27q_quant_act, same codes): its 8-row workgroups spread evenly over
    // the CUs (2176 for gate/up, 8.5 per CU), where quantizing in the product
    // needs whole 32-row groups per workgroup (544, 2 or 3 per CU, and a launch
    // ends with its most loaded CUs).  Measured 0.9 us faster per layer.
    const bool quant_after = yq && swiglu;
    // A single product with between 2 and TPW tiles per CU (down: 640 tiles
    // on 256 CUs) spreads its tiles evenly over one workgroup per CU: one tile
    // per workgroup puts 3 on half the CUs and 2 on the rest, and a launch ends
    // with its most loaded CUs (down on int8 codes 15.9 us against 16.45, on
    // fp32 x 17.3 us against 19.7).  On an fp32 activation each workgroup also
    // quantizes x, which on short rows costs more than the balance gains (o,
    // 6144 columns: 0.2 us slower), so fp32 input balances from 10240 columns.
    const long long tiles0 = tiles_of(ws[0].row_count);
    const int cus = cu_count();
    const bool bal = n == 1 && !swiglu && !yq && (!x || p.K >= 10240) && tiles0 > 2LL * cus &&
                     tiles0 <= (long long)gemv_q8_tiles_per_wg(kCfgB) * cus;
    // The same with 8 to 9 tiles per CU (config 1's Q4_K 17408 x 5120: 8.5),
    // where the other shapes leave a fifth two-tile workgroup on a quarter of
    // the CUs: 10.5 us against 11.1 on an fp32 x (cold copies, events), and
    // x is staged 256 times instead of 1088.
    const bool bal9 = n == 1 && !swiglu && !yq && tiles0 > 8LL * cus &&
                      tiles0 <= (long long)gemv_q8_tiles_per_wg(kCfgB9) * cus;
    const int cfg = bal9 ? kCfgB9
                  : bal ? kCfgB
                        : pick_gemv_cfg(ws[0].ggml_type, ws[0].layout == M27Q_LAYOUT_TILED, x != nullptr, swiglu,
                                        yq && !quant_after, rows_total, p.upr);
    if (gemv_q8_lds_bytes(ws[0].ggml_type, p.upr, swiglu, cfg) > lds_limit()) return M27Q_ERR_SHAPE;
    if (dry) return M27Q_OK;
    if (x) {
        p.x = x;
    } else {
        const ActView a = act_view(xq, 1, p.K);
        p.xq = a.q;
        p.xd = a.d;
        p.xs = a.s;
    }
    const int tpw = gemv_q8_tiles_per_wg(cfg);
    int total = 0;
    for (int i = 0; i < nout; ++i) {
        p.W[i] = (const uint8_t *)ws[i].ptr;
        p.y[i] = ys[i];
        p.rc[i] = (int)ws[i].row_count;
        p.wg_start[i] = total;
        total += bal || bal9 ? cus : (tiles_of(ws[i].row_count) + tpw - 1) / tpw;
    }
    p.bal = bal || bal9 ? 1 : 0;
    if (swiglu) p.W[1] = (const uint8_t *)ws[1].ptr;
    else p.res[0] = residual;
    p.wg_start[nout] = total;
    p.nmat = nout;
    const ActView ya = yq ? act_view(yq, 1, (int)ws[0].row_count) : ActView{};
    if (yq && !quant_after) {
        p.oq = (int8_t *)ya.q;
        p.od = (float *)ya.d;
        p.os = (uint32_t *)ya.s;
    }
    hipError_t e = launch_gemv_q8(ws[0].ggml_type, (int)ws[0].layout, swiglu, cfg, p, stream);
    if (e == hipSuccess && quant_after)
        e = launch_quant_act(ys[0], nullptr, ws[0].row_count, (int8_t *)ya.q, (float *)ya.d, (uint32_t *)ya.s, stream);
    return hip_status(e);
}

// Small-M products: for TILED weights, up to kMtMaxM tokens on the GEMV
// streaming structure when their activations fit the LDS budget
// (m27q_gemv_mt.hip), otherwise on int8 MFMA (m27q_mma.hip).  Measured on the
// Qwen-27B layer: 56 us against 63 at M = 2; from M = 3 on the MFMA kernel
// with two row sets per tile is faster (63 against 75 us at M = 4).  TILED
// Q4_K / Q5_K, whose MFMA kernel loads the weight operands straight into
// registers, take it from M = 2: q/k/v 6.5 against 9.1 us, o 6.5 against
// 7.8, gate/up 20.5 against 21.6 (Q6_K down keeps the GEMV structure: 17.7
// against 20.1 on MFMA).
// GGUF-layout weights take the same few-token kernel (with temporal loads);
// from M = 3, GGUF-layout Q4_K / Q5_K / Q6_K take the MFMA kernel (staged from
// the row blocks), GGUF-layout Q8_0 and IQ4_XS one launch per matrix of the
// VALU kernel (m27q_matmul.hip).
constexpr int kMtMaxM = 2;
constexpr size_t kMtLdsBudget = 80 * 1024;  // two workgroups per CU

m27q_status matmul_multi_impl(int n, const m27q_weight *ws, int M, const void *xq, float *const *Ys,
                              const float *const *res, hipStream_t stream, bool dry = false) {
    for (int i = 0; i < n; ++i) {
        const m27q_status st = check_weight(&ws[i], true);
        if (st != M27Q_OK) return st;
        if (!Ys[i]) return M27Q_ERR_NULL;
        if (ws[i].ggml_type != ws[0].ggml_type) return M27Q_ERR_TYPE;
        if (ws[i].layout != ws[0].layout) return M27Q_ERR_LAYOUT;
        if (ws[i].row_blocks != ws[0].row_blocks) return M27Q_ERR_SHAPE;
    }
    if (!aligned(xq, 16)) return M27Q_ERR_LAYOUT;
    const uint32_t type = ws[0].ggml_type;
    const int layout = (int)ws[0].layout;
    const bool tiled = layout == M27Q_LAYOUT_TILED;
    MatmulMultiParams p{};
    p.upr = units_per_row(type, ws[0].row_blocks);
    p.rb = (int)ws[0].row_blocks;
    p.K = k_of(&ws[0]);
    p.M = M;
    const ActView a = act_view(xq, M, p.K);
    const bool few = M <= kMtMaxM && (M == 1 || !matmul_mfma_direct(type, layout)) &&
                     matmul_mt_lds_bytes(type, p.upr) <= kMtLdsBudget;
    if (!few && !matmul_mfma_takes(type, layout)) {  // GGUF Q8_0 / IQ4_XS from M = 3
        if (dry) return M27Q_OK;
        for (int i = 0; i < n; ++i) {
            MatmulParams q{};
            q.W = (const uint8_t *)ws[i].ptr;
            q.rb = (int)ws[i].row_blocks;
            q.rc = (int)ws[i].row_count;
            q.upr = p.upr;
            q.K = p.K;
            q.M = M;
            q.xq = a.q;
            q.xd = a.d;
            q.xs = a.s;
            q.Y = Ys[i];
            q.res = res[i];
            const hipError_t e = launch_matmul_q8(type, layout, q, stream);
            if (e != hipSuccess) return hip_status(e);
        }
        return M27Q_OK;
    }
    if (!few && matmul_mfma_lds_bytes(type) > lds_limit()) return M27Q_ERR_SHAPE;
    // The MFMA kernel reads each matrix through a buffer descriptor with a
    // 32-bit size; the activations (M <= kMaxM rows of K <= kMaxK) stay far
    // below it.
    for (int i = 0; i < n && !few; ++i) {
        const size_t wb = tiled ? tiled_bytes(type, ws[i].row_blocks, ws[i].row_count)
                                : (size_t)ws[i].row_blocks * ws[i].row_count * (size_t)block_bytes(type);
        if (wb >= (1ull << 32)) return M27Q_ERR_SHAPE;
    }
    if (dry) return M27Q_OK;
    p.xq = a.q;
    p.xd = a.d;
    p.xs = a.s;
    p.nmat = n;
    if (few && n == 1) p.bal_wgs = matmul_mt_balance(tiles_of(ws[0].row_count), p.upr, cu_count());
    for (int i = 0; i < n; ++i) {
        p.W[i] = (const uint8_t *)ws[i].ptr;
        p.Y[i] = Ys[i];
        p.res[i] = res[i];
        p.rc[i] = (int)ws[i].row_count;
    }
    return hip_status(few ? launch_matmul_mt(type, layout, p, stream) : launch_matmul_mfma(type, layout, p, stream));
}

// Up to kMaxMulti weights of one K sharing one activation, of any mix of
// types and layouts (l_mv_pair runs wqkv and wqkv_gate of different types on
// one quantized x, exec:2106-2125, :2492): each (type, layout) group is one
// launch, in order of first appearance, on the same stream.  Every group is
// checked before the first launch.  M == 0 selects the M = 1 products.
m27q_status grouped_multi(int n, const m27q_weight *ws, int M, const void *xq, const float *x, float *const *ys,
                          hipStream_t stream) {
    if (!ws || !ys) return M27Q_ERR_NULL;
    if (n < 1 || n > kMaxMulti) return M27Q_ERR_SHAPE;
    for (int i = 0; i < n; ++i) {
        const m27q_status st = check_weight(&ws[i], true);
        if (st != M27Q_OK) return st;
        if (k_of(&ws[i]) != k_of(&ws[0])) return M27Q_ERR_SHAPE;
    }
    int group[kMaxMulti], ng = 0;
    for (int i = 0; i < n; ++i) {
        group[i] = -1;
        for (int j = 0; j < i && group[i] < 0; ++j)
            if (ws[j].ggml_type == ws[i].ggml_type && ws[j].layout == ws[i].layout) group[i] = group[j];
        if (group[i] < 0) group[i] = ng++;
    }
    for (int pass = 0; pass < 2; ++pass) {
        for (int g = 0; g < ng; ++g) {
            m27q_weight gw[kMaxMulti];
            float *gy[kMaxMulti];
            const float *gr[kMaxMulti] = {nullptr, nullptr, nullptr, nullptr};
            int m = 0;
            for (int i = 0; i < n; ++i)
                if (group[i] == g) {
                    gw[m] = ws[i];
                    gy[m++] = ys[i];
                }
            const bool dry = pass == 0;
            const m27q_status st = M == 0 ? gemv_impl(m, gw, xq, x, gy, nullptr, false, nullptr, stream, dry)
                                          : matmul_multi_impl(m, gw, M, xq, gy, gr, stream, dry);
            if (st != M27Q_OK) return st;
        }
    }
    return M27Q_OK;
}

}  // namespace

extern "C" {

M27Q_API size_t m27q_act_d_offset(int M, int K) {
    return align_up((size_t)M * K, kActAlign);
}
M27Q_API size_t m27q_act_s_offset(int M, int K) {
    return m27q_act_d_offset(M, K) + align_up((size_t)M * (K / 32) * 4, kActAlign);
}
M27Q_API size_t m27q_act_bytes(int M, int K) {
    if (M <= 0 || K <= 0 || K % 32) return 0;
    return m27q_act_s_offset(M, K) + align_up((size_t)M * (K / 32) * 4, kActAlign);
}

static m27q_status quant_act_impl(const float *x, const float *gate, int M, int K, void *xq, hipStream_t s) {
    if (!x || !xq) return M27Q_ERR_NULL;
    if (M <= 0 || M > 1 << 16 || K < 32 || K % 32 || K > kMaxK) return M27Q_ERR_SHAPE;
    if (!aligned(xq, 16) || !aligned(x, 4) || (gate && !aligned(gate, 4))) return M27Q_ERR_LAYOUT;
    const ActView a = act_view(xq, M, K);
    return hip_status(launch_quant_act(x, gate, (long long)M * K, (int8_t *)a.q, (float *)a.d, (uint32_t *)a.s, s));
}

M27Q_API m27q_status m27q_quant_act(const float *x, int M, int K, void *xq, hipStream_t stream) {
    return quant_act_impl(x, nullptr, M, K, xq, stream);
}

M27Q_API m27q_status m27q_quant_act_gated(const float *x, const float *gate, int M, int K, void *xq,
                                          hipStream_t stream) {
    if (!gate) return M27Q_ERR_NULL;
    return quant_act_impl(x, gate, M, K, xq, stream);
}

M27Q_API m27q_status m27q_matvec_q8(const m27q_weight *w, const void *xq, float *y, const float *residual,
                                    void *yq, hipStream_t stream) {
    if (!xq) return M27Q_ERR_NULL;
    return gemv_impl(1, w, xq, nullptr, &y, residual, false, yq, stream);
}

M27Q_API m27q_status m27q_matvec_q8_multi(int n, const m27q_weight *ws, const void *xq, float *const *ys,
                                          hipStream_t stream) {
    if (!xq) return M27Q_ERR_NULL;
    return grouped_multi(n, ws, 0, xq, nullptr, ys, stream);
}

M27Q_API m27q_status m27q_ffn_swiglu_q8(const m27q_weight *gate, const m27q_weight *up, const void *xq, float *y,
                                        void *yq, hipStream_t stream) {
    if (!gate || !up || !xq) return M27Q_ERR_NULL;
    const m27q_weight ws[2] = {*gate, *up};
    return gemv_impl(2, ws, xq, nullptr, &y, nullptr, true, yq, stream);
}

M27Q_API m27q_status m27q_matvec_f32(const m27q_weight *w, const float *x, float *y, const float *residual,
                                     hipStream_t stream) {
    const m27q_status st = check_weight(w, false);
    if (st != M27Q_OK) return st;
    if (!x || !y) return M27Q_ERR_NULL;
    if (!aligned(x, 16)) return M27Q_ERR_LAYOUT;
    GemvParams p{};
    p.rb = (int)w->row_blocks;
    p.K = k_of(w);
    p.upr = is_quant(w->ggml_type) ? units_per_row(w->ggml_type, w->row_blocks) : 0;
    if (is_quant(w->ggml_type) && gemv_f32_lds_bytes(w->ggml_type, p.upr) > lds_limit()) return M27Q_ERR_SHAPE;
    p.x = x;
    p.W[0] = (const uint8_t *)w->ptr;
    p.y[0] = y;
    p.res[0] = residual;
    p.rc[0] = (int)w->row_count;
    p.nmat = 1;
    const int grid = wg_count((int)w->row_count);
    p.wg_start[1] = grid;
    return hip_status(launch_gemv_f32(w->ggml_type, (int)w->layout, p, grid, stream));
}

M27Q_API m27q_status m27q_matvec(const m27q_weight *w, const float *x, float *y, const float *residual, void *yq,
                                 hipStream_t stream) {
    const m27q_status st = check_weight(w, false);
    if (st != M27Q_OK) return st;
    if (!is_quant(w->ggml_type)) {
        if (yq) return M27Q_ERR_TYPE;
        return m27q_matvec_f32(w, x, y, residual, stream);
    }
    if (!x) return M27Q_ERR_NULL;
    return gemv_impl(1, w, nullptr, x, &y, residual, false, yq, stream);
}

M27Q_API m27q_status m27q_matvec_multi(int n, const m27q_weight *ws, const float *x, float *const *ys,
                                       hipStream_t stream) {
    if (!x) return M27Q_ERR_NULL;
    return grouped_multi(n, ws, 0, nullptr, x, ys, stream);
}

M27Q_API m27q_status m27q_ffn_swiglu(const m27q_weight *gate, const m27q_weight *up, const float *x, float *y,
                                     void *yq, hipStream_t stream) {
    if (!gate || !up || !x) return M27Q_ERR_NULL;
    const m27q_weight ws[2] = {*gate, *up};
    return gemv_impl(2, ws, nullptr, x, &y, nullptr, true, yq, stream);
}

M27Q_API m27q_status m27q_matmul_q8(const m27q_weight *w, int M, const void *xq, float *Y, const float *residual,
                                    hipStream_t stream) {
    const m27q_status st = check_weight(w, true);
    if (st != M27Q_OK) return st;
    if (!xq || !Y) return M27Q_ERR_NULL;
    if (M < 1 || M > kMaxM) return M27Q_ERR_SHAPE;
    if (!aligned(xq, 16)) return M27Q_ERR_LAYOUT;
    if (M == 1) return m27q_matvec_q8(w, xq, Y, residual, nullptr, stream);
    float *Ys[1] = {Y};
    const float *rs[1] = {residual};
    return matmul_multi_impl(1, w, M, xq, Ys, rs, stream);
}

M27Q_API m27q_status m27q_matmul_q8_multi(int n, const m27q_weight *ws, int M, const void *xq, float *const *Ys,
                                          hipStream_t stream) {
    if (!ws || !Ys || !xq) return M27Q_ERR_NULL;
    if (n < 1 || n > kMaxMulti || M < 1 || M > kMaxM) return M27Q_ERR_SHAPE;
    if (M == 1) return m27q_matvec_q8_multi(n, ws, xq, Ys, stream);
    return grouped_multi(n, ws, M, xq, nullptr, Ys, stream);
}

static m27q_status gather_impl(const m27q_weight *w, const int32_t *ids, int row0, int n, float *out,
                               int32_t *bad, hipStream_t stream) {
    const m27q_status st = check_weight(w, false);
    if (st != M27Q_OK) return st;
    if (!out) return M27Q_ERR_NULL;
    if (!aligned(out, 16)) return M27Q_ERR_LAYOUT;
    if (n < 1 || n > 65535) return M27Q_ERR_SHAPE;
    GatherParams p{};
    p.W = (const uint8_t *)w->ptr;
    p.type = w->ggml_type;
    p.layout = (int)w->layout;
    p.rb = (int)w->row_blocks;
    p.rc = (int)w->row_count;
    p.upr = is_quant(w->ggml_type) ? units_per_row(w->ggml_type, w->row_blocks) : 0;
    p.ids = ids;
    p.row0 = row0;
    p.n = n;
    p.out = out;
    p.bad = bad;
    return hip_status(launch_gather(p, stream));
}

M27Q_API m27q_status m27q_dequant_rows(const m27q_weight *w, int row0, int nrows, float *out, hipStream_t stream) {
    const m27q_status st = check_weight(w, false);
    if (st != M27Q_OK) return st;
    if (row0 < 0 || nrows < 1 || (long long)row0 + nrows > (long long)w->row_count) return M27Q_ERR_RANGE;
    return gather_impl(w, nullptr, row0, nrows, out, nullptr, stream);
}

M27Q_API m27q_status m27q_embed_rows(const m27q_weight *w, const int32_t *ids, int n, float *out, int32_t *bad_count,
                                     hipStream_t stream) {
    if (!ids) return M27Q_ERR_NULL;
    if (bad_count && !aligned(bad_count, 4)) return M27Q_ERR_LAYOUT;
    return gather_impl(w, ids, 0, n, out, bad_count, stream);
}

M27Q_API m27q_status m27q_embed_token(const m27q_weight *w, int32_t token_id, float *out, hipStream_t stream) {
    const m27q_status st = check_weight(w, false);
    if (st != M27Q_OK) return st;
    if (token_id < 0 || (uint32_t)token_id >= w->row_count) return M27Q_ERR_RANGE;
    return gather_impl(w, nullptr, token_id, 1, out, nullptr, stream);
}

M27Q_API size_t m27q_topk_scratch_bytes(int n, int k) {
    if (n <= 0 || k < 1 || k > kMaxTopK || k > n) return 0;
    return topk_scratch_bytes(n);
}

M27Q_API m27q_status m27q_topk(const float *logits, int n, int k, int32_t *idx, float *val, void *scratch,
                               size_t scratch_bytes, hipStream_t stream) {
    if (!logits || !idx || !val || !scratch) return M27Q_ERR_NULL;
    if (n <= 0) return M27Q_ERR_SHAPE;
    if (k < 1 || k > kMaxTopK || k > n) return M27Q_ERR_RANGE;
    if (scratch_bytes < topk_scratch_bytes(n)) return M27Q_ERR_SCRATCH;
    if (!aligned(scratch, 8)) return M27Q_ERR_LAYOUT;
    return hip_status(launch_topk(logits, n, k, idx, val, scratch, stream));
}

M27Q_API m27q_status m27q_topk_noalloc(const float *logits, int n, int k, int32_t *idx, float *val,
                                       hipStream_t stream) {
    if (!logits || !idx || !val) return M27Q_ERR_NULL;
    if (n <= 0) return M27Q_ERR_SHAPE;
    if (k < 1 || k > kMaxTopK || k > n) return M27Q_ERR_RANGE;
    const size_t need = topk_scratch_bytes(n);
    if (need == 0 || need > topk_static_scratch_bytes()) return M27Q_ERR_SCRATCH;
    void *scratch = nullptr;
    if (topk_static_scratch(&scratch) != hipSuccess) return M27Q_ERR_HIP;
    return hip_status(launch_topk(logits, n, k, idx, val, scratch, stream));
}

M27Q_API m27q_status m27q_sample(const int32_t *idx, const float *val, int k, float temperature, float min_p,
                                 float top_p, const float *u, int32_t *token, hipStream_t stream) {
    if (!idx || !val || !u || !token) return M27Q_ERR_NULL;
    if (k < 1 || k > kMaxTopK) return M27Q_ERR_RANGE;
    if (!(min_p >= 0.f) || !(top_p > 0.f) || std::isnan(temperature)) return M27Q_ERR_RANGE;
    if (!aligned(idx, 4) || !aligned(val, 4) || !aligned(u, 4) || !aligned(token, 4)) return M27Q_ERR_LAYOUT;
    return hip_status(launch_sample(idx, val, k, temperature, min_p, top_p, u, token, stream));
}

}  // extern "C"
