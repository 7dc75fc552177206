/*
 * m27q.h -- C ABI of the MI355X (gfx950) quantized linear-algebra path.
 *
 * Drop-in for the matvec launch layer of mono27b (eramax/mono-qwen27,
 * src/mono27b_executor.cu, "exec" below).  Every entry point names the
 * reference interface it replaces.  Conventions:
 *
 *  - Plain C types only: device pointers are void* / float*, sizes are ints.
 *  - Every buffer is caller-owned device memory; nothing here allocates
 *    device memory.  Scratch space is an explicit argument.
 *  - Every call validates its arguments on the host before any HIP call and
 *    returns a status (the reference's launchers silently skip on bad input,
 *    exec:2034, :2056-2059).
 *  - Work is enqueued on the given stream; nothing synchronizes, allocates or
 *    reads device memory on the host, so every device entry point can be
 *    recorded into a HIP graph.
 *  - Weights are described by m27q_weight, the reference's WeightView
 *    (include/mono27b_config.h:63-68) plus a layout tag.
 */
#ifndef M27Q_H
#define M27Q_H

#include <stddef.h>
#include <stdint.h>

#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#if defined(__GNUC__)
#define M27Q_API __attribute__((visibility("default")))
#else
#define M27Q_API
#endif

typedef enum m27q_status {
    M27Q_OK = 0,
    M27Q_ERR_NULL = 1,        /* a required pointer is NULL */
    M27Q_ERR_SHAPE = 2,       /* row_blocks / row_count / M / K / n out of range */
    M27Q_ERR_TYPE = 3,        /* ggml type not supported by this entry point */
    M27Q_ERR_LAYOUT = 4,      /* unknown layout tag or misaligned buffer */
    M27Q_ERR_SCRATCH = 5,     /* scratch buffer smaller than required */
    M27Q_ERR_RANGE = 6,       /* token id out of range, or k > n */
    M27Q_ERR_HIP = 7,         /* the HIP launch itself failed */
    M27Q_ERR_IO = 8           /* a file could not be read or written, or is not a .m27b blob */
} m27q_status;

/* ggml type ids, as include/mono27b_gguf.h:27-43 numbers them. */
enum {
    M27Q_TYPE_F32 = 0,
    M27Q_TYPE_F16 = 1,
    M27Q_TYPE_Q8_0 = 8,
    M27Q_TYPE_Q4_K = 12,
    M27Q_TYPE_Q5_K = 13,
    M27Q_TYPE_Q6_K = 14,
    M27Q_TYPE_IQ4_XS = 23
};

/* Weight layouts in device memory.
 *  GGUF : rows of raw GGUF blocks, row-major [row_count][row_blocks], exactly as
 *         the reference uploads them (exec:1695-1716).
 *  TILED: the pack-time re-tiling produced by m27q_repack.  Rows are grouped in
 *         tiles of 8; within a tile, each block column is stored plane by plane
 *         (headers, then quants; the Q4_K / Q5_K quants by 32-byte chunk pair,
 *         then row) so that one wavefront load instruction reads 1 KiB of
 *         contiguous bytes.  Byte-preserving per block, 16-byte aligned,
 *         inverted exactly by m27q_unpack. */
enum { M27Q_LAYOUT_GGUF = 0, M27Q_LAYOUT_TILED = 1 };

typedef struct m27q_weight {
    const void *ptr;        /* device pointer (16-byte aligned for TILED) */
    uint32_t ggml_type;     /* M27Q_TYPE_* */
    uint32_t row_blocks;    /* blocks per row (K / block size; K for F16/F32);
                               K <= 2^20 */
    uint32_t row_count;     /* rows (N), 1 .. 2^24 */
    uint32_t layout;        /* M27Q_LAYOUT_* */
} m27q_weight;

M27Q_API const char *m27q_status_string(m27q_status s);

/* ------------------------------------------------------------------------
 * Host-side, pack time (no GPU needed)
 * ---------------------------------------------------------------------- */

/* Bytes of one GGUF row of ne elements, 0 if ne is not a whole number of
 * blocks.  Replaces mono27b_ggml_row_size (src/mono27b_gguf.cpp:375-382). */
M27Q_API size_t m27q_row_size(uint32_t ggml_type, uint32_t ne);

/* Device bytes a weight occupies in the given layout (TILED pads the row
 * count to a multiple of 8 and, for Q8_0, the block count to a multiple of 4,
 * with zero blocks).  0 for an unsupported type/layout. */
M27Q_API size_t m27q_weight_bytes(uint32_t ggml_type, uint32_t row_blocks, uint32_t row_count,
                                  uint32_t layout);

/* GGUF rows -> TILED (host memory to host memory).  Replaces the verbatim
 * copy of lw() (exec:1695-1716) with pack-time re-tiling; the caller uploads
 * the result.  Supported types: Q4_K, Q5_K, Q6_K, Q8_0, IQ4_XS. */
M27Q_API m27q_status m27q_repack(uint32_t ggml_type, uint32_t row_blocks, uint32_t row_count,
                                 const void *gguf_rows, void *tiled);
/* TILED -> GGUF rows (the exact inverse of m27q_repack). */
M27Q_API m27q_status m27q_unpack(uint32_t ggml_type, uint32_t row_blocks, uint32_t row_count,
                                 const void *tiled, void *gguf_rows);

/* Re-tile a .m27b weight blob (include/mono27b_format.h:30-84) at pack time:
 * out_path gets a copy of in_path in which every matrix entry of a type with
 * a TILED form (whole GGUF rows) is re-tiled, its data_bytes updated and its
 * reserved field set to M27Q_LAYOUT_TILED | 2 << 16 (the high 16 bits: the
 * revision of the TILED byte order); tensors are 256-byte aligned in the
 * file; the header, tokenizer section and all other tensors are copied.  The
 * result passes the reference's mono27b_validate_blob_file and
 * mono27b_read_weights_section.  Entries already tagged TILED are copied.
 * Streams one tensor at a time.  Fills the role the reference's missing packer
 * would have (the writer is src/mono27b_blob.cpp:378-438). */
M27Q_API m27q_status m27q_retile_blob(const char *in_path, const char *out_path);

/* One tensor of a .m27b weights section as a loader needs it: the entry's
 * fields (include/mono27b_format.h:74-84), the layout from its reserved field,
 * row_blocks as WeightView counts it (K / block size; K for F16 / F32; 0 when
 * the entry's byte count is not whole rows of its type in its layout, or when
 * a TILED entry carries another revision of the byte order), and the absolute
 * file offset of its bytes. */
typedef struct m27q_blob_tensor {
    char name[64];
    uint32_t ggml_type;
    uint32_t source_model;
    uint32_t role;
    uint32_t row_elems;
    uint32_t row_count;
    uint32_t layout;       /* M27Q_LAYOUT_GGUF or M27Q_LAYOUT_TILED (entry.reserved & 0xffff) */
    uint32_t row_blocks;
    uint32_t pad;
    uint64_t file_offset;
    uint64_t bytes;        /* entry.data_bytes */
} m27q_blob_tensor;

/* Reads and bounds-checks the blob's header, section table and weight entry
 * table (host only).  *count gets the number of entries; the first
 * min(cap, *count) are written to out (cap may be 0 to count only).  The
 * table half of the reference's blob reader (mono27b_read_weights_section,
 * src/mono27b_blob.cpp) for a loader of re-tiled blobs. */
M27Q_API m27q_status m27q_blob_tensors(const char *path, m27q_blob_tensor *out, int cap, int *count);

/* Uploads one tensor's bytes from the file to caller-owned device memory
 * (dst_bytes >= t->bytes; 16-byte aligned for TILED) with synchronous
 * host-to-device copies, and fills *w with the descriptor the products take
 * (ptr = device_dst, layout = t->layout).  Not for graph capture: it reads a
 * file.  Replaces lw() (exec:1695-1716), which copies a tensor's GGUF bytes
 * into its own cudaMalloc; here the caller allocates (m27q_weight_bytes
 * gives the size). */
M27Q_API m27q_status m27q_blob_load(const char *path, const m27q_blob_tensor *t, void *device_dst,
                                   size_t dst_bytes, m27q_weight *w);

/* ------------------------------------------------------------------------
 * Activations
 * ---------------------------------------------------------------------- */

/* Quantized activation buffer for M rows of K values (K % 32 == 0):
 *   int8  codes[M][K]             at offset 0
 *   float d[M][K/32]              at offset m27q_act_d_offset(M, K)
 *   u32   sums[M][K/32]           at offset m27q_act_s_offset(M, K)
 * Per 32 values: d = amax/127 (IEEE divide), id = 1/d (IEEE divide) where
 * that is finite, else 0 (d == 0, or a subnormal d below 2^-128: such a
 * group's codes are all 0), code = roundf(x * id) clamped to +-127 (the rule
 * of ggml's quantize_row_q8_1_ref), sums = (int16 sum of codes 0..15) |
 * (int16 sum of codes 16..31) << 16.  The reference's Q8_1 (exec:65-71) keeps an fp16 d and
 * the float sum of x; this format keeps an fp32 d and the exact integer sums
 * its dot products use. */
M27Q_API size_t m27q_act_bytes(int M, int K);
M27Q_API size_t m27q_act_d_offset(int M, int K);
M27Q_API size_t m27q_act_s_offset(int M, int K);

/* x[M][K] fp32 -> xq.  Replaces l_quant_q8_n / k_quant_q8_1 (exec:2022-2030,
 * :84-107). */
M27Q_API m27q_status m27q_quant_act(const float *x, int M, int K, void *xq, hipStream_t stream);

/* (x * sigmoid(gate)) -> xq, the gate as x * (1 / (1 + e^-gate)) with a fixed
 * exp (Cody-Waite range reduction and a degree-7 polynomial, argument clamped
 * to [-87, 87]; within 2 ulp of e^t) in place of the reference's fast-math
 * __expf, so the codes are reproducible bit for bit.  Replaces
 * k_quant_q8_1_fused_gate (exec:109-138, site :2460). */
M27Q_API m27q_status m27q_quant_act_gated(const float *x, const float *gate, int M, int K, void *xq,
                                          hipStream_t stream);

/* ------------------------------------------------------------------------
 * M = 1 matrix-vector products (integer dot: int8 activation codes x weight
 * codes, fp32 combine).  Q4_K, Q5_K, Q6_K, Q8_0, IQ4_XS weights in either
 * layout (Q5_K: the vec_dot_q5_K_q8_1 / k_q5k_mv_q8 path of exec:421-531;
 * IQ4_XS: vec_dot_iq4_xs_q8_1 / k_iq4xs_mv_q8_dp4a, exec:647-686).
 *
 * The activation is given either as fp32 values x[K] (16-byte aligned),
 * quantized inside the product with exactly the rule of m27q_quant_act (the
 * codes are identical),
 * or as an already quantized buffer xq from m27q_quant_act (M = 1, K = the
 * weight's K).  Where yq is not NULL, the output y is also quantized into yq
 * (the format of m27q_quant_act with K = row_count, which must be a multiple
 * of 32): the fused producer of the next product's activation.
 * ---------------------------------------------------------------------- */

/* y[r] = sum_k W[r][k] x[k] (+ residual[r]); residual and yq may be NULL.
 * F16 / F32 weights go to m27q_matvec_f32 (yq must then be NULL).  Replaces
 * l_mv_quant and l_mv_quant_residual (exec:2033-2050, :2089-2104), which
 * quantize x into the global Q8_1 scratch (l_quant_q8_n, exec:2022-2030)
 * and then launch the product and the k_elem_add epilogue. */
M27Q_API m27q_status m27q_matvec(const m27q_weight *w, const float *x, float *y, const float *residual,
                                 void *yq, hipStream_t stream);

/* Same on an already quantized activation.  Replaces l_mv_q8_on
 * (exec:2054-2083): k_q4k_mv_q8_dp4a / k_q6k_mv_q8_dp4a / k_q80_mv_q8_dp4a
 * (exec:320-364, :631-645, :535-580) plus the k_elem_add residual epilogue
 * (exec:2080-2082).  The reference's callers that quantize once and run
 * several products (the sigmoid-gated quantization in front of Wo, exec:2460,
 * and K/V on the second stream, exec:2389-2395) map onto this entry point. */
M27Q_API m27q_status m27q_matvec_q8(const m27q_weight *w, const void *xq, float *y, const float *residual,
                                    void *yq, hipStream_t stream);

/* Up to 4 weights that share one activation (the same K; types and layouts
 * may differ): y[i] = W[i] x.  Weights of one type and layout run in one
 * launch; each further (type, layout) group is one more launch on the same
 * stream, in order of first appearance, on the same activation codes.  Every
 * weight is checked before the first launch.  Replaces l_mv_pair
 * (exec:2106-2125), whose pair mixes types on the SSM layers (wqkv Q6_K and
 * wqkv_gate Q5_K in the UD-Q4_K_XL file, exec:2492; a member l_mv_pair skips,
 * null or with no rows, is left out: n = 1), and the Wq || Wk, Wv pattern of
 * the attention block (exec:2377-2395). */
M27Q_API m27q_status m27q_matvec_multi(int n, const m27q_weight *ws, const float *x, float *const *ys,
                                       hipStream_t stream);
M27Q_API m27q_status m27q_matvec_q8_multi(int n, const m27q_weight *ws, const void *xq, float *const *ys,
                                          hipStream_t stream);

/* y[r] = silu(Wg x)[r] * (Wu x)[r]; gate and up of one type, layout and shape;
 * yq may be NULL (where it is not, y is quantized into it by a second launch
 * on the same stream, with the codes of m27q_quant_act).  Replaces
 * l_ffn_gate_up_swiglu / k_q4k_q4k_swiglu_dp4a (exec:2239-2261, :369-417),
 * which takes fp32 x. */
M27Q_API m27q_status m27q_ffn_swiglu(const m27q_weight *gate, const m27q_weight *up, const float *x, float *y,
                                     void *yq, hipStream_t stream);
M27Q_API m27q_status m27q_ffn_swiglu_q8(const m27q_weight *gate, const m27q_weight *up, const void *xq, float *y,
                                        void *yq, hipStream_t stream);

/* fp32-activation product y = W x (+ residual): exact dequantization and fp32
 * accumulation.  Q4_K, Q5_K, Q6_K, Q8_0, IQ4_XS, F16, F32.  Replaces
 * l_mv_fallback (exec:2127-2137) with k_q4k_mv / k_q5k_mv / k_q6k_mt /
 * k_q80_mv / k_iq4xs_mv / k_f16_mv / k_f32_mv (exec:920-951, :953-985,
 * :1053-1072, :1076-1096, :992-1020, :899-916, :1100-1114). */
M27Q_API m27q_status m27q_matvec_f32(const m27q_weight *w, const float *x, float *y, const float *residual,
                                     hipStream_t stream);

/* ------------------------------------------------------------------------
 * Small-M products (speculative verify / prefill rows)
 * ---------------------------------------------------------------------- */

/* Y[m][r] = sum_k W[r][k] * xq[m][k] (+ residual[m][r]) for m < M, 1 <= M <= 64,
 * xq from m27q_quant_act with this M (the whole buffer of m27q_act_bytes(M,
 * K) bytes: Q8_0 weights whose K is not a multiple of 128 read up to 96 bytes
 * past the last row's codes); Y is [M][row_count].  M = 2 runs on the GEMV
 * structure, from M = 3 TILED weights and GGUF-layout Q4_K / Q5_K / Q6_K
 * weights on int8 MFMA (v_mfma_i32_16x16x32_i8, up to 16 activation rows per
 * launch), other GGUF-layout weights on a packed-int8-dot path; M = 1 is
 * m27q_matvec_q8.  No reference
 * counterpart: the reference runs prefill and decode one token at a time
 * (src/mono27b_chat.cpp:399-403); results equal M independent M = 1 products
 * up to fp32 rounding. */
M27Q_API m27q_status m27q_matmul_q8(const m27q_weight *w, int M, const void *xq, float *Y,
                                    const float *residual, hipStream_t stream);

/* Up to 4 weights of one K on the same M activation rows: Ys[i] = X W[i]^T
 * ([M][row_count_i] each), one launch per (type, layout) group as in
 * m27q_matvec_q8_multi (GGUF-layout Q8_0 / IQ4_XS: one launch per weight).
 * The small-M counterpart of m27q_matvec_q8_multi (q/k/v, gate/up of a
 * verify batch). */
M27Q_API m27q_status m27q_matmul_q8_multi(int n, const m27q_weight *ws, int M, const void *xq, float *const *Ys,
                                          hipStream_t stream);

/* ------------------------------------------------------------------------
 * Dequantization, row gather, vocab selection
 * ---------------------------------------------------------------------- */

/* out[i][:] = dequant(W[row0 + i][:]) for i < nrows, fp32, bit-exact with
 * ggml's dequantize_row_* (the closed forms of exec:920-951, :955-969,
 * :1026-1048, :1076-1096).  Any supported type and layout. */
M27Q_API m27q_status m27q_dequant_rows(const m27q_weight *w, int row0, int nrows, float *out,
                                       hipStream_t stream);

/* out[i][:] = dequant(W[ids[i]][:]) for i < n; ids is a device array.  An id
 * outside [0, row_count) yields a zero row and, if bad_count is not NULL,
 * increments *bad_count (device int, caller-cleared).  Generalizes
 * k_q4k_embed (exec:1233-1254), which handles one Q4_K token. */
M27Q_API m27q_status m27q_embed_rows(const m27q_weight *w, const int32_t *ids, int n, float *out,
                                     int32_t *bad_count, hipStream_t stream);

/* One token id given on the host; an id outside [0, row_count) returns
 * M27Q_ERR_RANGE before any launch.  Replaces mono27b_engine_embed
 * (exec:2641-2664), which writes a zero row for such ids. */
M27Q_API m27q_status m27q_embed_token(const m27q_weight *w, int32_t token_id, float *out,
                                      hipStream_t stream);

/* Exact top-k (1 <= k <= 64) of logits[0..n) by (value desc, index asc), -0.0 ==
 * +0.0, NaN after every number; idx/val are device arrays of k entries, in
 * rank order.  scratch >= m27q_topk_scratch_bytes(n, k).  Replaces the CPU
 * candidate selection of sample() (src/mono27b_chat.cpp:211-227) and, with
 * k = 1, k_argmax / mono27b_engine_argmax (exec:211-239, :2630-2637). */
M27Q_API size_t m27q_topk_scratch_bytes(int n, int k);
M27Q_API m27q_status m27q_topk(const float *logits, int n, int k, int32_t *idx, float *val, void *scratch,
                               size_t scratch_bytes, hipStream_t stream);

/* m27q_topk without a scratch argument: no counterpart in the reference; for
 * callers that cannot allocate device memory (code under graph capture, tight
 * serving loops, harnesses that forbid hipMalloc).  The library keeps the
 * scratch in a static device array of m27q_topk_scratch_bytes (134,144 bytes;
 * n <= 2^24) per device, held until the process ends; n beyond that returns
 * M27Q_ERR_SCRATCH before any launch.  The first call on a device resolves
 * the array's address (hipGetSymbolAddress), so make it outside graph
 * capture.  Every call on a device shares that device's array: calls that
 * overlap on one device (two streams, two threads) race.  Nothing here
 * allocates or frees. */
M27Q_API m27q_status m27q_topk_noalloc(const float *logits, int n, int k, int32_t *idx, float *val,
                                       hipStream_t stream);

/* On-device token choice from m27q_topk's candidates (idx/val in rank order,
 * 1 <= k <= 64), the steps of sample() (src/mono27b_chat.cpp:203-270) after its
 * top-k: temperature <= 0 gives idx[0] (the argmax, first index on ties);
 * otherwise p_i = e^((val_i - val_0) / temperature) (the fixed exp of
 * m27q_quant_act_gated; 0 below e^-87), normalized; candidates
 * with p_i < p_0 * min_p are dropped; top_p < 1 keeps the shortest prefix whose
 * running sum reaches top_p; the token is the first candidate whose running sum
 * reaches u * (sum of the kept p).  u is a device float in [0, 1), token a
 * device int32: per-step values stay on the device, so the step can be replayed
 * as a graph.  Banned tokens: the caller sets their logits to -inf before
 * m27q_topk, as sample() does on its copy (:206-211).  Sums run in candidate
 * order, as the reference's loop. */
M27Q_API m27q_status m27q_sample(const int32_t *idx, const float *val, int k, float temperature, float min_p,
                                 float top_p, const float *u, int32_t *token, hipStream_t stream);

#ifdef __cplusplus
}
#endif
#endif /* M27Q_H */
