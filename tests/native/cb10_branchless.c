/* Check: the branch-free cb10 code of the PSQ4 append kernel
 * (phaseshift_amd/csrc/kv_append.hip, cb10_code: k = min(ceil(|x| * 2inv), 19)
 * and a 3-bit lookup of k) equals the reference's comparison chain
 * (psq_device.h:22-31, restated as or_cb10_encode in oracle/ps_oracle.c):
 *   1. exhaustively for every float bit pattern x >= 0 at inv = 1 (including
 *      +inf and every NaN), i.e. for every |x| * inv;
 *   2. for 2^26 random (x, bf16 scale) pairs over 2^-80 .. 2^20 magnitudes,
 *      with inv = 1 / s as the kernel computes it, signs included.
 * Uses the same IEEE operations as the device code: fminf (NaN -> other
 * operand), ceilf, one rounding per multiply. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

uint8_t or_cb10_encode(float x, float inv_scale);

static uint32_t lut_code(float x, float inv) {
    const float inv2 = 2.0f * inv;
    const uint64_t lut = 0x0fb6d6db246d2240ull;   /* code(k), k = 0..19, 3 bits each */
    const float k = fminf(ceilf(fabsf(x) * inv2), 19.0f);
    const uint32_t m = (uint32_t)(lut >> (3u * (uint32_t)k)) & 7u;
    return m | (x < 0.0f ? 8u : 0u);
}

static uint64_t rng_state = 0x9E3779B97F4A7C15ull;
static uint64_t next_u64(void) {
    rng_state ^= rng_state << 13;
    rng_state ^= rng_state >> 7;
    rng_state ^= rng_state << 17;
    return rng_state;
}

int main(void) {
    uint64_t bad = 0;
#pragma omp parallel for reduction(+ : bad) schedule(static, 1 << 16)
    for (int64_t b = 0; b <= 0x7FFFFFFFll; ++b) {
        const uint32_t u = (uint32_t)b;
        float a;
        memcpy(&a, &u, 4);
        const uint32_t want = or_cb10_encode(a, 1.0f);
        if (lut_code(a, 1.0f) != want) {
            if (bad < 8) printf("mismatch a=%a (0x%08x): %u vs %u\n", a, u, lut_code(a, 1.0f), want);
            ++bad;
        }
    }
    for (int64_t i = 0; i < (1ll << 26); ++i) {
        const uint64_t r = next_u64();
        /* x: random sign, exponent 2^-80 .. 2^20, random mantissa */
        const uint32_t xb = (uint32_t)((r >> 63) << 31) | (uint32_t)((47 + (r >> 40) % 100) << 23) |
                            (uint32_t)(r & 0x7FFFFFu);
        /* s: a positive normal bf16 */
        const uint32_t sb = (uint32_t)(0x0080u + (next_u64() % (0x7F80u - 0x0080u))) << 16;
        float x, s;
        memcpy(&x, &xb, 4);
        memcpy(&s, &sb, 4);
        const float inv = 1.0f / s;
        const uint32_t want = or_cb10_encode(x, inv);
        if (lut_code(x, inv) != want) {
            if (bad < 16) printf("mismatch x=%a s=%a: %u vs %u\n", x, s, lut_code(x, inv), want);
            ++bad;
        }
    }
    printf("mismatches %llu\n", (unsigned long long)bad);
    return bad != 0;
}
