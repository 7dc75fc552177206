/*
 * m27q_oracle.h -- CPU oracle for the quantized linear-algebra path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker: only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it.  The
 * product path (libm27q.so) never links, loads or calls anything here.
 *
 * It restates, in plain C99, the arithmetic of the reference's quant path
 * (eramax/mono-qwen27 @ src/mono27b_executor.cu, "exec" below) and of the
 * ggml CPU routines that path mirrors.  Every routine cites the reference
 * file:line it follows.  The GGUF block byte layouts are fixed by the file
 * format and are therefore identical to the reference's structs.
 *
 * Parity pins (what checks each function independently of its own formula):
 *   ora_fp16_to_fp32      all 65536 inputs vs numpy float16->float32, and vs the
 *                         conversion inside debug/official_dequant.c built from
 *                         the reference's source (oracle/_ref).
 *   ora_fp32_to_fp16      vs numpy float32->float16 (round-to-nearest-even).
 *   ora_dequant_row_q4_K  reference known-answer bytes (debug/official_dequant.c:71-74
 *                         -> debug/mono_give_current.debug.tsv:2), random blocks vs
 *                         dequantize_row_q4_K compiled from debug/official_dequant.c,
 *                         and the reference's second formulation (the dp4a vec-dot,
 *                         ora_ref_vec_dot_q4_K_q8_1) with one-hot activations.
 *   ora_dequant_row_q5_K  the reference's dp4a vec-dot formulation
 *                         (ora_ref_vec_dot_q5_K_q8_1, exec:421-495) with one-hot
 *                         activations; with qh = 0 it equals ora_dequant_row_q4_K
 *                         on the same d / dmin / scales / qs (pinned above), and
 *                         setting qh bit j adds exactly 16 d sc_j to sub-block j.
 *   ora_dequant_row_q6_K  the reference's dp4a vec-dot formulation
 *                         (ora_ref_vec_dot_q6_K_q8_1, exec:586-628) with one-hot
 *                         activations, plus single-bit known answers.
 *   ora_dequant_row_q8_0  the reference's dp4a formulation (exec:535-580).
 *   ora_dequant_row_iq4_xs the reference's dp4a formulation (exec:647-671) with
 *                         one-hot activations, and hand-set single blocks whose
 *                         values are the table entries times d (ls - 32).
 *   ora_quant_act         an independent numpy restatement of the rule (float32
 *                         divide / reciprocal / multiply, round half away in float64),
 *                         and closed-form properties (|q|<=127, the max maps to +-127,
 *                         |x - d q| <= d/2 (1 + 2^-22), round-half-away on ties).
 *   ora_dot_act           brute force (dequantized weights x dequantized activation
 *                         in fp64) on small shapes, and one-hot / zero inputs.
 *   ora_topk              numpy lexsort on the same values.
 *   ora_sample            closed-form properties: temperature <= 0 and u = 0 give
 *                         the first candidate, top_p -> 0 and min_p = 1 keep only
 *                         it, and over a fine grid of u the share of each token
 *                         equals its kept probability.
 *   ggml q8_K routines    PARITY UNPINNED: ggml itself (ref/llama.cpp) is absent from
 *                         the reference checkout and no version is pinned.  They are a
 *                         restatement of ggml's published generic C path, used only as
 *                         the CPU baseline and as the "no worse than q8_K" yardstick.
 *   quantizers            not parity functions: they only generate valid blocks.
 */
#ifndef M27Q_ORACLE_H
#define M27Q_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml type ids (include/mono27b_gguf.h:27-43 in the reference). */
enum { ORA_F32 = 0, ORA_F16 = 1, ORA_Q8_0 = 8, ORA_Q4_K = 12, ORA_Q5_K = 13, ORA_Q6_K = 14, ORA_Q8_K = 15,
       ORA_IQ4_XS = 23 };

/* GGUF block layouts (exec:18-23, :25-28, :38-42, :57-62). */
typedef struct { uint16_t d, dmin; uint8_t scales[12]; uint8_t qs[128]; } ora_block_q4_K;
typedef struct { uint16_t d, dmin; uint8_t scales[12]; uint8_t qh[32]; uint8_t qs[128]; } ora_block_q5_K; /* exec:30-36 */
typedef struct { uint8_t ql[128]; uint8_t qh[64]; int8_t scales[16]; uint16_t d; } ora_block_q6_K;
/* exec:44-49: f16 d, u16 scales_h, u8 scales_l[4], u8 qs[128] (136 B, 8-byte aligned in a row) */
typedef struct { uint16_t d, scales_h; uint8_t scales_l[4]; uint8_t qs[128]; } ora_block_iq4_xs;
/* The IQ4_NL / IQ4_XS value table (exec:51-55). */
extern const int8_t ora_kvalues_iq4nl[16];
typedef struct { uint16_t d; int8_t qs[32]; } ora_block_q8_0;
typedef struct { float d; int8_t qs[256]; int16_t bsums[16]; } ora_block_q8_K;
/* The reference's activation block (exec:65-71): half2 {d, sum(x)} + 32 codes. */
typedef struct { uint16_t d, s; int8_t qs[32]; } ora_block_q8_1;

size_t ora_type_size(int type);   /* bytes per block (src/mono27b_gguf.cpp:167-180) */
int    ora_block_elems(int type); /* weights per block (src/mono27b_gguf.cpp:182-195) */

float    ora_fp16_to_fp32(uint16_t h);
uint16_t ora_fp32_to_fp16(float f);
void     ora_fp16_to_fp32_n(const uint16_t *h, float *f, size_t n);
void     ora_fp32_to_fp16_n(const float *f, uint16_t *h, size_t n);

void ora_get_scale_min_k4(int j, const uint8_t *q, uint8_t *sc, uint8_t *m);

/* Dequantization of k = n_blocks * block_elems weights. */
void ora_dequant_row_q4_K(const void *blocks, float *y, int64_t k);
void ora_dequant_row_q5_K(const void *blocks, float *y, int64_t k);
void ora_dequant_row_q6_K(const void *blocks, float *y, int64_t k);
void ora_dequant_row_q8_0(const void *blocks, float *y, int64_t k);
void ora_dequant_row_iq4_xs(const void *blocks, float *y, int64_t k);
/* rc rows of rb blocks each, GGUF row-major; F16/F32 rows of rb elements. */
int  ora_dequant_rows(int type, const void *w, int rb, int rc, float *y);

/* Seeded block generators (own simple min/max quantizers). */
void ora_quantize_row_q4_K(const float *x, void *blocks, int64_t k);
void ora_quantize_row_q5_K(const float *x, void *blocks, int64_t k);
void ora_quantize_row_q6_K(const float *x, void *blocks, int64_t k);
void ora_quantize_row_q8_0(const float *x, void *blocks, int64_t k);
void ora_quantize_row_iq4_xs(const float *x, void *blocks, int64_t k);

/* Activation format of the MI355X path: per 32 values, int8 codes, an fp32
 * scale d = amax/127 (IEEE divide), id = 1/d (IEEE divide) where that is
 * finite and 0 otherwise (d == 0, or d subnormal below 2^-128), q = roundf(x *
 * id) clamped to +-127 (ggml's quantize_row_q8_1_ref rule), and the two
 * 16-value integer code sums packed as (int16 lo) | (int16 hi) << 16. */
void ora_quant_act(const float *x, int64_t k, int8_t *q, float *d, uint32_t *s);
/* The build's fixed exp (Cody-Waite reduction + degree-7 Taylor polynomial,
 * argument clamped to [-87, 87]) and the gate x * (1 / (1 + e^-g)). */
float ora_exp_cw(float t);
float ora_gated(float x, float g);
void ora_exp_cw_n(const float *t, float *out, size_t n);
void ora_gated_n(const float *x, const float *g, float *out, size_t n);
/* Same on ora_gated(x, g) (exec:109-138). */
void ora_quant_act_gated(const float *x, const float *g, int64_t k, int8_t *q, float *d, uint32_t *s);

/* Integer-dot of one weight row against the activation format, evaluated in
 * fp64 from the exact integer partial sums.  *norm (may be NULL) receives
 * sum |term| over the per-group terms: the scale of fp32 reassociation error. */
double ora_dot_act(int type, const void *wrow, int rb, const int8_t *q, const float *d,
                   const uint32_t *s, double *norm);
int    ora_gemv_act(int type, const void *w, int rb, int rc, const int8_t *q, const float *d,
                    const uint32_t *s, double *y, double *norm);

/* fp64 dequant-then-dot: y[r] = sum_k W[r][k] x[k]. */
int ora_gemv_f64(int type, const void *w, int rb, int rc, const float *x, double *y);

/* Restatements of the reference's own dp4a vec-dot formulations, used to
 * cross-check the dequant restatements (two independent codings of one format). */
void  ora_quant_q8_1(const float *x, int64_t k, ora_block_q8_1 *y);
float ora_ref_vec_dot_q4_K_q8_1(const void *wrow, const ora_block_q8_1 *xq, int rb);
float ora_ref_vec_dot_q5_K_q8_1(const void *wrow, const ora_block_q8_1 *xq, int rb);
float ora_ref_vec_dot_q6_K_q8_1(const void *wrow, const ora_block_q8_1 *xq, int rb);
float ora_ref_vec_dot_q8_0_q8_1(const void *wrow, const ora_block_q8_1 *xq, int rb);
float ora_ref_vec_dot_iq4_xs_q8_1(const void *wrow, const ora_block_q8_1 *xq, int rb);

/* ggml CPU path restatement (parity unpinned; CPU baseline). */
void  ora_quantize_row_q8_K(const float *x, void *y, int64_t k);
float ora_vec_dot_q4_K_q8_K(int n, const void *vx, const void *vy);
float ora_vec_dot_q6_K_q8_K(int n, const void *vx, const void *vy);
void  ora_quantize_row_q8_0_act(const float *x, void *y, int64_t k);
float ora_vec_dot_q8_0_q8_0(int n, const void *vx, const void *vy);
/* y[r] for r in [0, rc), rows split over nthreads pthreads.  xq is the
 * activation quantized to q8_K (K-quants) or q8_0 (Q8_0). */
int ora_gemv_cpu(int type, const void *w, int rb, int rc, const void *xq, float *y, int nthreads);
/* The same dots and row split in AVX2 (m27q_cpu_simd.c): the CPU baseline's
 * SIMD build. */
float ora_simd_vec_dot_q4_K_q8_K(int n, const void *vx, const void *vy);
float ora_simd_vec_dot_q6_K_q8_K(int n, const void *vx, const void *vy);
float ora_simd_vec_dot_q8_0_q8_0(int n, const void *vx, const void *vy);
int ora_gemv_cpu_simd(int type, const void *w, int rb, int rc, const void *xq, float *y, int nthreads);

/* sample() (src/mono27b_chat.cpp:203-270) after its top-k, on candidates
 * idx/val in rank order: temperature <= 0 -> idx[0]; softmax at the
 * temperature (ora_exp_cw, 0 below e^-87; float32, sums in candidate order), min_p and top_p cuts,
 * pick = u * total, the first candidate whose running sum reaches it. */
int ora_sample(const int32_t *idx, const float *val, int k, float temperature, float min_p, float top_p, float u);

/* Exact top-k by (value desc, index asc); NaN ranks after every number. */
int ora_topk(const float *v, int n, int k, int32_t *idx, float *val);

#ifdef __cplusplus
}
#endif
#endif
