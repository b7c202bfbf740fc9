/* Exhaustive check: the branch-free cb10 magnitude index of the PSQ4 append
 * kernel (phaseshift_amd/csrc/kv_append.hip, cb10_code) equals the
 * reference's comparison chain (psq_device.h:22-31, restated as
 * or_cb10_encode in oracle/ps_oracle.c) for every float bit pattern a >= 0
 * (including +inf and every NaN), i.e. for every |x| * inv. Uses the same
 * IEEE operations as the device code: fminf / fmaxf (NaN -> other operand),
 * ceilf, fmaf (one rounding). */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

uint8_t or_cb10_encode(float x, float inv_scale);

static uint32_t branchless(float a) {
    const float t1 = fminf(ceilf(a - 0.5f), 4.0f);
    const float t2 = 3.0f - fminf(fmaxf(3.0f - ceilf(fmaf(a, 0.5f, -2.5f)), 0.0f), 3.0f);
    return (uint32_t)(t1 + t2);
}

int main(void) {
    uint64_t bad = 0;
#pragma omp parallel for reduction(+ : bad) schedule(static, 1 << 16)
    for (int64_t b = 0; b <= 0x7FFFFFFFll; ++b) {
        const uint32_t u = (uint32_t)b;
        float a;
        memcpy(&a, &u, 4);
        const uint32_t want = or_cb10_encode(a, 1.0f) & 7u;
        if (branchless(a) != want) {
            if (bad < 8) printf("mismatch a=%a (0x%08x): %u vs %u\n", a, u, branchless(a), want);
            ++bad;
        }
    }
    printf("mismatches %llu\n", (unsigned long long)bad);
    return bad != 0;
}
