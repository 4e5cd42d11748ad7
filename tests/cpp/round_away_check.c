/* The device kernels' round-half-away-from-zero (qmm.hip qmm_quant):
 * trunc(t + copysign(0x1.fffffep-2, t)) against roundf, bit for bit, over
 * every finite f32.  Exit status 0 when all agree. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

int main(void) {
    const float c = 0x1.fffffep-2f; /* 0.5 - 2^-25 */
    unsigned long long n = 0, bad = 0;
    for (uint64_t u = 0; u < (1ull << 32); u++) {
        const uint32_t b = (uint32_t)u;
        float t;
        memcpy(&t, &b, 4);
        if (!isfinite(t)) continue;
        const float want = roundf(t);
        volatile float s = t + copysignf(c, t); /* one rounded f32 add */
        const float got = truncf(s);
        n++;
        if (memcmp(&want, &got, 4) != 0) {
            if (bad < 5) printf("t=%a: roundf %a, trunc form %a\n", t, want, got);
            bad++;
        }
    }
    printf("%llu finite floats, %llu differ\n", n, bad);
    return bad != 0;
}
