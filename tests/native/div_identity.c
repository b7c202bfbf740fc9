/* Exhaustive check of the append kernel's division identity (CPU).
 *
 * The FP8 append kernel computes x / s as q0 = x*r, rem = fma(-q0, s, x),
 * q = fma(rem, r, q0) with r = 1/s correctly rounded, when s >= 2^-100 and
 * |x| >= 2^-100, and a true division otherwise. For every finite bf16 amax > 0
 * (s = amax/448) and every bf16 x with |x| <= amax, this program checks that
 * the E4M3 code of that q equals the E4M3 code of the IEEE quotient x / s.
 * Prints "pairs P code_mismatches M"; exit status 0 iff M == 0.
 * Built and run by tests/test_div_identity.py (links oracle/ps_oracle.c). */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

uint8_t or_e4m3_encode(float x);

static float bf(uint32_t h) {
    uint32_t u = h << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

int main(void) {
    long long pairs = 0, bad = 0;
#pragma omp parallel for reduction(+ : pairs, bad) schedule(dynamic, 64)
    for (uint32_t ha = 1; ha < 0x7F80u; ++ha) {
        const float amax = bf(ha);
        const float s = amax / 448.0f;
        const float r = 1.0f / s;
        const int fast_scale = s >= 0x1p-100f;
        for (uint32_t hx = 0; hx <= ha; ++hx) {
            for (int sign = 0; sign < 2; ++sign) {
                const float x = sign ? -bf(hx) : bf(hx);
                float q;
                if (fast_scale && fabsf(x) >= 0x1p-100f) {
                    const float q0 = x * r;
                    const float rem = fmaf(-q0, s, x);
                    q = fmaf(rem, r, q0);
                } else {
                    q = x / s;
                }
                pairs++;
                if (or_e4m3_encode(q) != or_e4m3_encode(x / s)) bad++;
            }
        }
    }
    printf("pairs %lld code_mismatches %lld\n", pairs, bad);
    return bad == 0 ? 0 : 1;
}
