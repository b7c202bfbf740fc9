// Division of a 32-bit unsigned n by a divisor d >= 1 fixed at launch:
// q = (t + ((n - t) >> s1)) >> s2 with t = mulhi(n, m), exact for every n in
// [0, 2^32) (Granlund and Montgomery, "Division by invariant integers using
// multiplication", PLDI 1994, figure 4.1: l = ceil(log2 d),
// m = floor(2^32 (2^l - d) / d) + 1, s1 = min(l, 1), s2 = max(l - 1, 0)).
// Five integer operations on the device instead of the generic division's
// twenty. Plain C++: the host side builds the constants, and the CPU tests
// check the evaluation below against n / d.
#pragma once
#include <cstdint>

namespace psk {

struct FastDiv {
    uint32_t m;
    uint32_t s1;
    uint32_t s2;
};

inline FastDiv make_fastdiv(uint32_t d) {
    uint32_t l = 0;
    while (l < 32u && (uint64_t{1} << l) < d) ++l;
    const uint64_t m = ((uint64_t{1} << 32) * ((uint64_t{1} << l) - d)) / d + 1u;
    return FastDiv{(uint32_t)m, l < 1u ? l : 1u, l > 1u ? l - 1u : 0u};
}

// The evaluation on the host (the device form uses __umulhi for t).
inline uint32_t fastdiv_host(uint32_t n, const FastDiv& f) {
    const uint32_t t = (uint32_t)(((uint64_t)n * f.m) >> 32);
    return (t + ((n - t) >> f.s1)) >> f.s2;
}

}  // namespace psk
