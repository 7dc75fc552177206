/* The device quantizer's rounding rule, (int)(v + copysignf(h, v)) with h the
 * largest float below 0.5, against (int)roundf(v) (the oracle's rule) for
 * every float with |v| < 2^23, the range the rule is used on.  Exit status 0
 * when they agree everywhere.  Built with plain IEEE float arithmetic (no
 * -ffast-math, no FMA contraction of the single add). */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

int main(void) {
    const float h = 0.49999997f;
    uint32_t hb;
    memcpy(&hb, &h, 4);
    if (hb != 0x3effffffu) return 2;
    uint64_t n = 0, bad = 0;
    for (uint64_t b = 0; b < 0x100000000ull; ++b) {
        const uint32_t u = (uint32_t)b;
        float v;
        memcpy(&v, &u, 4);
        if (!(fabsf(v) < 8388608.0f)) continue;
        ++n;
        if ((int)roundf(v) != (int)(v + copysignf(h, v))) {
            if (bad < 4) printf("mismatch at %08x\n", u);
            ++bad;
        }
    }
    printf("%llu values, %llu mismatches\n", (unsigned long long)n, (unsigned long long)bad);
    return bad != 0;
}
