/* Two shortcuts of the device quantizer (m27q_device.h) against the rules
 * they replace, over every input they can see:
 *   quant_code: (int)(v + copysignf(h, v)), h the largest float below 0.5,
 *               against (int)roundf(v), for every float with |v| < 2^23;
 *   div127:     fma(fma(-q, 127, a), c, q) with q = a * c, c = rn(1/127),
 *               against a / 127.0f, for every non-negative finite float.
 * Exit status 0 when both agree everywhere.  Plain IEEE float arithmetic (no
 * -ffast-math, no contraction: the single operations are what the device
 * code is compiled to). */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

static float f_of(uint32_t u) {
    float v;
    memcpy(&v, &u, 4);
    return v;
}

int main(void) {
    const float h = 0.49999997f, c = 1.0f / 127.0f;
    uint32_t hb;
    memcpy(&hb, &h, 4);
    if (hb != 0x3effffffu) return 2;
    long long n_round = 0, bad_round = 0, n_div = 0, bad_div = 0;
#pragma omp parallel for reduction(+ : n_round, bad_round, n_div, bad_div) schedule(static)
    for (long long b = 0; b < 0x100000000ll; ++b) {
        const uint32_t u = (uint32_t)b;
        const float v = f_of(u);
        if (fabsf(v) < 8388608.0f) {
            ++n_round;
            bad_round += (int)roundf(v) != (int)(v + copysignf(h, v));
        }
        if (u < 0x7f800000u) {  /* finite, sign bit clear */
            ++n_div;
            const float q = v * c;
            const float d = fmaf(fmaf(-q, 127.0f, v), c, q);
            const float ref = v / 127.0f;
            bad_div += memcmp(&d, &ref, 4) != 0;
        }
    }
    printf("round: %lld values, %lld mismatches\n", n_round, bad_round);
    printf("div127: %lld values, %lld mismatches\n", n_div, bad_div);
    return bad_round != 0 || bad_div != 0;
}
