/*
 * abi_caller.c -- a C99 caller of include/m27q.h, built with gcc against
 * libm27q.so the way the reference's host code would link it.
 *
 *   abi_caller --cpu   host-side entry points and the host validation of the
 *                      device entry points (no GPU needed)
 *   abi_caller --gpu   products on MI355X through the C ABI, each checked
 *                      against the library's own bit-exact dequantization
 *                      (m27q_dequant_rows) dotted in double with the
 *                      dequantized activation codes of m27q_quant_act
 *
 * Prints "abi_caller: ok" and exits 0 when every check passes; otherwise
 * prints the first failure and exits 1.
 */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "m27q.h"

static int fails = 0;

#define CHECK(cond, ...)                                   \
    do {                                                   \
        if (!(cond)) {                                     \
            fprintf(stderr, "abi_caller: FAIL %s:%d: ", __FILE__, __LINE__); \
            fprintf(stderr, __VA_ARGS__);                  \
            fprintf(stderr, "\n");                         \
            fails++;                                       \
            return 1;                                      \
        }                                                  \
    } while (0)

#define HIPCHECK(call) CHECK((call) == hipSuccess, "%s failed", #call)

static uint64_t rng_state = 0x9e3779b97f4a7c15ull;
static uint32_t rnd32(void) {
    rng_state = rng_state * 6364136223846793005ull + 1442695040888963407ull;
    return (uint32_t)(rng_state >> 32);
}
static float rnd_unit(void) { return (float)((rnd32() >> 8) * (1.0 / 16777216.0)) * 2.0f - 1.0f; }

/* Random blocks of a type with finite fp16 scales: every byte random, then
 * the fp16 scale fields set to small normal values. */
static void fill_blocks(uint32_t type, uint8_t *b, size_t nblocks) {
    const size_t bb = m27q_row_size(type, type == M27Q_TYPE_Q8_0 ? 32u : 256u);
    for (size_t i = 0; i < nblocks * bb; ++i) b[i] = (uint8_t)rnd32();
    for (size_t i = 0; i < nblocks; ++i) {
        uint8_t *blk = b + i * bb;
        const uint16_t d = (uint16_t)(0x1c00u + (rnd32() & 0x3ffu)); /* 2^-8 .. 2^-7 */
        if (type == M27Q_TYPE_Q6_K) {
            memcpy(blk + 208, &d, 2);
        } else if (type == M27Q_TYPE_Q8_0) {
            memcpy(blk, &d, 2);
        } else { /* Q4_K: d, dmin */
            const uint16_t dm = (uint16_t)(0x1800u + (rnd32() & 0x3ffu));
            memcpy(blk, &d, 2);
            memcpy(blk + 2, &dm, 2);
        }
    }
}

static int cpu_checks(void) {
    /* status strings and GGUF row sizes (src/mono27b_gguf.cpp:375-382) */
    for (int s = 0; s <= 8; ++s) CHECK(m27q_status_string((m27q_status)s) != NULL, "status string %d", s);
    CHECK(m27q_row_size(M27Q_TYPE_Q4_K, 5120) == 20 * 144, "Q4_K row size");
    CHECK(m27q_row_size(M27Q_TYPE_Q6_K, 17408) == 68 * 210, "Q6_K row size");
    CHECK(m27q_row_size(M27Q_TYPE_Q8_0, 2048) == 64 * 34, "Q8_0 row size");
    CHECK(m27q_row_size(M27Q_TYPE_Q4_K, 100) == 0, "partial block row size");
    /* TILED pads rows to 8 */
    CHECK(m27q_weight_bytes(M27Q_TYPE_Q4_K, 4, 61, M27Q_LAYOUT_TILED) == (size_t)8 * 4 * 1152,
          "TILED bytes of 61 rows");
    CHECK(m27q_weight_bytes(M27Q_TYPE_Q4_K, 4, 61, M27Q_LAYOUT_GGUF) == (size_t)61 * 4 * 144, "GGUF bytes");

    /* repack / unpack round trip, bit for bit */
    const uint32_t types[3] = {M27Q_TYPE_Q4_K, M27Q_TYPE_Q6_K, M27Q_TYPE_Q8_0};
    for (int ti = 0; ti < 3; ++ti) {
        const uint32_t t = types[ti], rc = 21, rb = t == M27Q_TYPE_Q8_0 ? 13 : 3;
        const size_t gb = m27q_weight_bytes(t, rb, rc, M27Q_LAYOUT_GGUF);
        const size_t tb = m27q_weight_bytes(t, rb, rc, M27Q_LAYOUT_TILED);
        uint8_t *g = malloc(gb), *tl = malloc(tb), *back = malloc(gb);
        CHECK(g && tl && back, "host allocation");
        fill_blocks(t, g, (size_t)rb * rc);
        CHECK(m27q_repack(t, rb, rc, g, tl) == M27Q_OK, "repack type %u", t);
        CHECK(m27q_unpack(t, rb, rc, tl, back) == M27Q_OK, "unpack type %u", t);
        CHECK(memcmp(g, back, gb) == 0, "repack/unpack round trip type %u", t);
        CHECK(m27q_repack(t, rb, rc, NULL, tl) == M27Q_ERR_NULL, "repack NULL input");
        free(g);
        free(tl);
        free(back);
    }

    /* host validation of device entry points: errors before any HIP call */
    m27q_weight w = {(const void *)0x1000, M27Q_TYPE_Q4_K, 4, 64, M27Q_LAYOUT_TILED};
    float *fake = (float *)0x2000;
    CHECK(m27q_matvec(NULL, fake, fake, NULL, NULL, 0) == M27Q_ERR_NULL, "matvec NULL weight");
    CHECK(m27q_matvec(&w, NULL, fake, NULL, NULL, 0) == M27Q_ERR_NULL, "matvec NULL x");
    m27q_weight bad = w;
    bad.ggml_type = 99;
    CHECK(m27q_matvec(&bad, fake, fake, NULL, NULL, 0) == M27Q_ERR_TYPE, "matvec unknown type");
    bad = w;
    bad.layout = 7;
    CHECK(m27q_matvec(&bad, fake, fake, NULL, NULL, 0) == M27Q_ERR_LAYOUT, "matvec unknown layout");
    bad = w;
    bad.row_count = 0;
    CHECK(m27q_matvec(&bad, fake, fake, NULL, NULL, 0) == M27Q_ERR_SHAPE, "matvec zero rows");
    CHECK(m27q_quant_act(fake, 0, 256, fake, 0) == M27Q_ERR_SHAPE, "quant_act M = 0");
    CHECK(m27q_embed_token(&w, 64, fake, 0) == M27Q_ERR_RANGE, "embed_token id out of range");
    CHECK(m27q_topk_scratch_bytes(248320, 64) > 0, "top-k scratch size");
    return 0;
}

/* One product on the GPU: W (rc x K, type t) in both layouts, x random. */
static int gpu_product(uint32_t t, uint32_t rc, uint32_t K) {
    const uint32_t rb = K / (t == M27Q_TYPE_Q8_0 ? 32u : 256u);
    const size_t gb = m27q_weight_bytes(t, rb, rc, M27Q_LAYOUT_GGUF);
    const size_t tb = m27q_weight_bytes(t, rb, rc, M27Q_LAYOUT_TILED);
    const size_t ab = m27q_act_bytes(1, (int)K);
    uint8_t *g = malloc(gb), *tl = malloc(tb), *xq = malloc(ab);
    float *x = malloc(K * sizeof(float)), *wd = malloc((size_t)rc * K * sizeof(float));
    float *y[3], *res = malloc(rc * sizeof(float)), *row = malloc(K * sizeof(float));
    for (int i = 0; i < 3; ++i) y[i] = malloc(rc * sizeof(float));
    CHECK(g && tl && xq && x && wd && res && row && y[0] && y[1] && y[2], "host allocation");
    fill_blocks(t, g, (size_t)rb * rc);
    CHECK(m27q_repack(t, rb, rc, g, tl) == M27Q_OK, "repack");
    for (uint32_t k = 0; k < K; ++k) x[k] = 2.0f * rnd_unit();
    for (uint32_t r = 0; r < rc; ++r) res[r] = rnd_unit();

    void *dg, *dt, *dxq;
    float *dx, *dy, *dres, *dwd, *drow;
    HIPCHECK(hipMalloc(&dg, gb));
    HIPCHECK(hipMalloc(&dt, tb));
    HIPCHECK(hipMalloc(&dxq, ab));
    HIPCHECK(hipMalloc((void **)&dx, K * sizeof(float)));
    HIPCHECK(hipMalloc((void **)&dy, 3 * rc * sizeof(float)));
    HIPCHECK(hipMalloc((void **)&dres, rc * sizeof(float)));
    HIPCHECK(hipMalloc((void **)&dwd, (size_t)rc * K * sizeof(float)));
    HIPCHECK(hipMalloc((void **)&drow, K * sizeof(float)));
    HIPCHECK(hipMemcpy(dg, g, gb, hipMemcpyHostToDevice));
    HIPCHECK(hipMemcpy(dt, tl, tb, hipMemcpyHostToDevice));
    HIPCHECK(hipMemcpy(dx, x, K * sizeof(float), hipMemcpyHostToDevice));
    HIPCHECK(hipMemcpy(dres, res, rc * sizeof(float), hipMemcpyHostToDevice));

    const m27q_weight wt = {dt, t, rb, rc, M27Q_LAYOUT_TILED};
    const m27q_weight wg = {dg, t, rb, rc, M27Q_LAYOUT_GGUF};
    CHECK(m27q_quant_act(dx, 1, (int)K, dxq, 0) == M27Q_OK, "quant_act");
    CHECK(m27q_matvec(&wt, dx, dy, dres, NULL, 0) == M27Q_OK, "matvec (fp32 x, TILED)");
    CHECK(m27q_matvec_q8(&wt, dxq, dy + rc, dres, NULL, 0) == M27Q_OK, "matvec_q8 (TILED)");
    CHECK(m27q_matvec_q8(&wg, dxq, dy + 2 * rc, dres, NULL, 0) == M27Q_OK, "matvec_q8 (GGUF)");
    CHECK(m27q_dequant_rows(&wt, 0, (int)rc, dwd, 0) == M27Q_OK, "dequant_rows");
    CHECK(m27q_embed_token(&wg, (int32_t)(rc - 1), drow, 0) == M27Q_OK, "embed_token");
    HIPCHECK(hipDeviceSynchronize());
    for (int i = 0; i < 3; ++i) HIPCHECK(hipMemcpy(y[i], dy + (size_t)i * rc, rc * sizeof(float), hipMemcpyDeviceToHost));
    HIPCHECK(hipMemcpy(xq, dxq, ab, hipMemcpyDeviceToHost));
    HIPCHECK(hipMemcpy(wd, dwd, (size_t)rc * K * sizeof(float), hipMemcpyDeviceToHost));
    HIPCHECK(hipMemcpy(row, drow, K * sizeof(float), hipMemcpyDeviceToHost));

    /* the embedded row equals the dequantized row, bit for bit, across layouts */
    CHECK(memcmp(row, wd + (size_t)(rc - 1) * K, K * sizeof(float)) == 0, "embed_token row != dequant_rows row");

    /* reference: sum_k dequant(W)[r][k] * d[k / 32] * code[k] + residual, in
     * double; the integer dot equals it up to fp32 reassociation */
    const int8_t *codes = (const int8_t *)xq;
    const float *d = (const float *)(xq + m27q_act_d_offset(1, (int)K));
    double worst = 0.0;
    for (uint32_t r = 0; r < rc; ++r) {
        double ref = res[r], nrm = fabs((double)res[r]);
        for (uint32_t k = 0; k < K; ++k) {
            const double term = (double)wd[(size_t)r * K + k] * ((double)d[k / 32] * (double)codes[k]);
            ref += term;
            nrm += fabs(term);
        }
        for (int i = 0; i < 3; ++i) {
            const double e = fabs((double)y[i][r] - ref) / (nrm + 1e-30);
            if (e > worst) worst = e;
            CHECK(e <= 1e-5, "type %u %ux%u form %d row %u: %.9g against %.9g (scaled error %.3g)", t, rc, K, i, r,
                  (double)y[i][r], ref, e);
        }
    }
    printf("abi_caller: type %u %ux%u: fp32-x TILED, q8 TILED, q8 GGUF within %.2e of the dequant-dot\n", t, rc, K,
           worst);
    HIPCHECK(hipFree(dg));
    HIPCHECK(hipFree(dt));
    HIPCHECK(hipFree(dxq));
    HIPCHECK(hipFree(dx));
    HIPCHECK(hipFree(dy));
    HIPCHECK(hipFree(dres));
    HIPCHECK(hipFree(dwd));
    HIPCHECK(hipFree(drow));
    free(g);
    free(tl);
    free(xq);
    free(x);
    free(wd);
    free(res);
    free(row);
    for (int i = 0; i < 3; ++i) free(y[i]);
    return 0;
}

int main(int argc, char **argv) {
    const int gpu = argc > 1 && strcmp(argv[1], "--gpu") == 0;
    if (cpu_checks()) return 1;
    if (gpu) {
        int n = 0;
        if (hipGetDeviceCount(&n) != hipSuccess || n < 1) {
            fprintf(stderr, "abi_caller: FAIL: --gpu given but no HIP device\n");
            return 1;
        }
        if (gpu_product(M27Q_TYPE_Q4_K, 64, 1024)) return 1;
        if (gpu_product(M27Q_TYPE_Q6_K, 45, 512)) return 1;
        if (gpu_product(M27Q_TYPE_Q8_0, 37, 160)) return 1;
    }
    printf("abi_caller: ok%s\n", gpu ? " (cpu and gpu checks)" : " (cpu checks)");
    return fails ? 1 : 0;
}
