/* Check: the branch-free cb10 code of the PSQ4 append kernel
 * (phaseshift_amd/csrc/kv_append.hip, cb10_code: k = min(ceil((|x| * inv) * 2), 19)
 * and a 3-bit lookup of k) equals the reference's comparison chain
 * (psq_device.h:22-31, restated as or_cb10_encode in oracle/ps_oracle.c):
 *   1. exhaustively for every float bit pattern x >= 0 at inv = 1 (including
 *      +inf and every NaN), i.e. for every |x| * inv;
 *   2. for 2^26 random (x, bf16 scale) pairs over 2^-80 .. 2^20 magnitudes,
 *      with inv = 1 / s as the kernel computes it, signs included;
 *   3. for every positive bf16 scale 0x0001..0x7F7F, subnormals included
 *      (where 2 / s overflows while 1 / s is finite), against 2048 x values
 *      each: 0, the code boundaries times s and their float neighbours, and
 *      random x of magnitude 2^-39 .. 2^13 times s.
 * Both the lookup form and the kernel's popcount form (below) are checked.
 * Uses the same IEEE operations as the device code: fminf (NaN -> other
 * operand), ceilf, one rounding per multiply. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>

uint8_t or_cb10_encode(float x, float inv_scale);

static uint32_t lut_code(float x, float inv) {
    const uint64_t lut = 0x0fb6d6db246d2240ull;   /* code(k), k = 0..19, 3 bits each */
    const float k = fminf(ceilf((fabsf(x) * inv) * 2.0f), 19.0f);
    const uint32_t m = (uint32_t)(lut >> (3u * (uint32_t)k)) & 7u;
    return m | (x < 0.0f ? 8u : 0u);
}

/* The kernel's form: n = floor(max(-2a, -19)) = -min(k, 19), the 64-bit
 * shift of {lo = 0, hi = H} by n mod 64, the popcount of the low dword; H has
 * the bits 32 - T for the thresholds T = 2 4 6 8 11 15 19 of k. Where 2 * inv
 * is finite the kernel may also use |x| * (-2 * inv) (pre2 = 1). */
static uint32_t pop_code(float x, float inv, int pre2) {
    const uint32_t h = (1u << 30) | (1u << 28) | (1u << 26) | (1u << 24) | (1u << 21) | (1u << 17) |
                       (1u << 13);
    const float y = fmaxf(pre2 ? fabsf(x) * (inv * -2.0f) : (fabsf(x) * inv) * -2.0f, -19.0f);
    const int n = (int)floorf(y);
    const uint64_t t = ((uint64_t)h << 32) >> ((uint32_t)n & 63u);
    return (uint32_t)__builtin_popcount((uint32_t)t) + (x < 0.0f ? 8u : 0u);
}

/* Without the clamp (the kernel's LSQ1 passes, used when -2a >= -32 for the
 * block's largest |x| and so for every x of the block). */
static uint32_t pop_code_unclamped(float x, float inv) {
    const uint32_t h = (1u << 30) | (1u << 28) | (1u << 26) | (1u << 24) | (1u << 21) | (1u << 17) |
                       (1u << 13);
    const int n = (int)floorf(fabsf(x) * (inv * -2.0f));
    const uint64_t t = ((uint64_t)h << 32) >> ((uint32_t)n & 63u);
    return (uint32_t)__builtin_popcount((uint32_t)t) + (x < 0.0f ? 8u : 0u);
}

static uint32_t check(float x, float inv, uint32_t want) {
    uint32_t bad = lut_code(x, inv) != want;
    bad |= (pop_code(x, inv, 0) != want) << 1;
    if (isfinite(inv * 2.0f)) bad |= (pop_code(x, inv, 1) != want) << 2;
    if (fabsf(x) * (inv * -2.0f) >= -32.0f) bad |= (pop_code_unclamped(x, inv) != want) << 3;
    return bad;
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
        const uint32_t m = check(a, 1.0f, want);
        if (m) {
            if (bad < 8) printf("mismatch a=%a (0x%08x): form mask %u, want %u\n", a, u, m, want);
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
        const uint32_t m = check(x, inv, want);
        if (m) {
            if (bad < 16) printf("mismatch x=%a s=%a: form mask %u, want %u\n", x, s, m, want);
            ++bad;
        }
    }
    static const float kBounds[7] = {0.5f, 1.5f, 2.5f, 3.5f, 5.0f, 7.0f, 9.0f};
#pragma omp parallel for reduction(+ : bad) schedule(dynamic, 64)
    for (int32_t sbits = 1; sbits <= 0x7F7F; ++sbits) {
        const uint32_t sb = (uint32_t)sbits << 16;
        float s;
        memcpy(&s, &sb, 4);
        const float inv = 1.0f / s;
        uint64_t st = 0x243F6A8885A308D3ull ^ ((uint64_t)sbits * 0x9E3779B97F4A7C15ull);
        for (int j = 0; j < 2048; ++j) {
            float x;
            if (j == 0) {
                x = 0.0f;
            } else if (j <= 42) {
                const float b = kBounds[(j - 1) % 7] * s;     /* boundary times s */
                const int nb = (j - 1) / 7;                    /* 0..5: neighbours */
                x = nb == 0 ? b : nb == 1 ? nextafterf(b, 0.0f) : nb == 2 ? nextafterf(b, INFINITY)
                  : nb == 3 ? -b : nb == 4 ? nextafterf(nextafterf(b, 0.0f), 0.0f)
                  : nextafterf(nextafterf(b, INFINITY), INFINITY);
            } else {
                st ^= st << 13;
                st ^= st >> 7;
                st ^= st << 17;
                const int e = (int)(st >> 58) - 12;             /* -12 .. 51 */
                const float m = 1.0f + (float)((st >> 20) & 0xFFFFF) / 1048576.0f;
                x = ldexpf(m, e > 12 ? e - 52 : e) * s;   /* 2^-39 .. 2^13 */
                if (st & 1u) x = -x;
            }
            const uint32_t want = or_cb10_encode(x, inv);
            const uint32_t m = check(x, inv, want);
            if (m) {
                if (bad < 24) printf("mismatch x=%a s=%a: form mask %u, want %u\n", x, s, m, want);
                ++bad;
            }
        }
    }
    printf("mismatches %llu\n", (unsigned long long)bad);
    return bad != 0;
}
