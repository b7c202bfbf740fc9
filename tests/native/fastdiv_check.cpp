// Check: psk::make_fastdiv / fastdiv_host (phaseshift_amd/csrc/fastdiv.h)
// equal n / d for every divisor 1..4096 and 2^k +- 1, against the 32-bit
// numerators 0..65535, 2^32 - 1 - (0..65535), every multiple of d near those,
// and 2^20 pseudo-random n each.
#include <cstdio>
#include <vector>
#include "fastdiv.h"

int main() {
    std::vector<uint32_t> ds;
    for (uint32_t d = 1; d <= 4096; ++d) ds.push_back(d);
    for (int k = 12; k < 32; ++k) {
        ds.push_back((1u << k) - 1u);
        ds.push_back(1u << k);
        ds.push_back((1u << k) + 1u);
    }
    ds.push_back(0xFFFFFFFFu);
    uint64_t bad = 0, st = 0x9E3779B97F4A7C15ull;
    for (uint32_t d : ds) {
        const psk::FastDiv f = psk::make_fastdiv(d);
        auto chk = [&](uint32_t n) {
            if (psk::fastdiv_host(n, f) != n / d) {
                if (bad < 10) std::printf("mismatch n=%u d=%u: %u vs %u\n", n, d, psk::fastdiv_host(n, f), n / d);
                ++bad;
            }
        };
        for (uint32_t n = 0; n < 65536u; ++n) {
            chk(n);
            chk(0xFFFFFFFFu - n);
        }
        for (uint64_t q = 0xFFFFFFFFull / d, j = 0; j < 64 && q >= j; ++j) {
            const uint64_t n = (q - j) * d;
            chk((uint32_t)n);
            if (n) chk((uint32_t)(n - 1));
        }
        const int reps = d <= 4096 ? (1 << 12) : (1 << 20);
        for (int i = 0; i < reps; ++i) {
            st ^= st << 13;
            st ^= st >> 7;
            st ^= st << 17;
            chk((uint32_t)st);
        }
    }
    std::printf("mismatches %llu\n", (unsigned long long)bad);
    return bad != 0;
}
