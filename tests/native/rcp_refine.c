/* Check: for every bf16 scale s in [2^-126, 2^126] and every float r within
 * one ulp of the correctly rounded 1/s (the hardware reciprocal's accuracy),
 * e = fma(-s, r, 1), q = fma(e, r, r) is the correctly rounded 1/s (the PSQ
 * append kernel's bf16_scale_reciprocal, phaseshift_amd/csrc/kv_append.hip). */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

static float from_bits(uint32_t u) {
    float x;
    memcpy(&x, &u, 4);
    return x;
}
static uint32_t to_bits(float x) {
    uint32_t u;
    memcpy(&u, &x, 4);
    return u;
}

int main(void) {
    long bad = 0, cases = 0;
    for (uint32_t h = 0x0001u; h < 0x7F80u; ++h) {
        const float s = from_bits(h << 16);
        if (!(s >= 0x1p-126f && s <= 0x1p126f)) continue;
        const float want = 1.0f / s;
        for (int d = -1; d <= 1; ++d) {
            const float r = from_bits(to_bits(want) + (uint32_t)d);
            const float q = fmaf(fmaf(-s, r, 1.0f), r, r);
            ++cases;
            if (to_bits(q) != to_bits(want)) {
                if (bad < 8) printf("mismatch s=%a r=%a: %a vs %a\n", s, r, q, want);
                ++bad;
            }
        }
    }
    printf("cases %ld mismatches %ld\n", cases, bad);
    return bad != 0 || cases < 90000;
}
