// Writes the FP8 golden fixtures of tests/golden from ROCm's own converter,
// __hip_cvt_float_to_fp8(x, __HIP_SATFINITE, __HIP_E4M3) of hip/hip_fp8.h —
// the function the reference calls on the device (reference
// include/phaseshift/quantization/fpx/e4m3_detail.h:13-15, kv_append.hip:144-146).
// Host build (software path of the same header):
//   hipcc -O2 -std=c++17 tests/golden/gen_fp8_golden.cpp -o /tmp/gen && /tmp/gen tests/golden
// Outputs (little-endian raw arrays):
//   e4m3_rocm_inputs.f32 / e4m3_rocm_codes.u8   float inputs and their codes
//   fp8_append_{k,v}_in.bf16   [128][4*256] bf16 K/V rows (N(0,1), 1% x20 outliers)
//   fp8_append_{k,v}_codes.u8  [128][4][256] codes of x/scale
//   fp8_append_{k,v}_scale.f32 [128][4] scales amax/448 (1 when amax == 0)
#include <hip/hip_fp8.h>

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

static uint64_t g_state = 0x9E3779B97F4A7C15ull;
static uint64_t next_u64() {  // splitmix64
    uint64_t z = (g_state += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
static double next_unit() { return (next_u64() >> 11) * (1.0 / 9007199254740992.0); }
static float next_normal() {
    const double u1 = next_unit() + 1e-300, u2 = next_unit();
    return (float)(std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2));
}
static uint16_t bf16_rne(float f) {
    uint32_t u;
    std::memcpy(&u, &f, 4);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}
static float bf16_f(uint16_t h) {
    uint32_t u = (uint32_t)h << 16;
    float f;
    std::memcpy(&f, &u, 4);
    return f;
}
static uint8_t rocm_e4m3(float x) {
    return (uint8_t)__hip_cvt_float_to_fp8(x, __HIP_SATFINITE, __HIP_E4M3);
}
template <class T>
static void dump(const std::string& path, const std::vector<T>& v) {
    FILE* f = std::fopen(path.c_str(), "wb");
    if (!f) { std::perror(path.c_str()); std::exit(1); }
    std::fwrite(v.data(), sizeof(T), v.size(), f);
    std::fclose(f);
}

int main(int argc, char** argv) {
    const std::string dir = argc > 1 ? argv[1] : ".";
    // 1) codec vectors: every finite bf16 value, the e4m3 rounding midpoints and
    //    their fp32 neighbours, and seeded random fp32 bit patterns.
    std::vector<float> xs;
    for (uint32_t h = 0; h < 65536u; ++h) {
        const float f = bf16_f((uint16_t)h);
        if (std::isfinite(f)) xs.push_back(f);
    }
    std::vector<float> grid;
    for (uint32_t c = 0; c < 0x7Fu; ++c) {
        const uint32_t e = (c >> 3) & 15u, m = c & 7u;
        grid.push_back(e == 0 ? std::ldexp((float)m, -9) : std::ldexp((float)(8 + m), (int)e - 10));
    }
    for (size_t i = 0; i + 1 < grid.size(); ++i) {
        const float mid = 0.5f * (grid[i] + grid[i + 1]);
        for (float s : {1.0f, -1.0f}) {
            xs.push_back(s * mid);
            xs.push_back(s * std::nextafter(mid, 0.0f));
            xs.push_back(s * std::nextafter(mid, 1e9f));
        }
    }
    for (float s : {1.0f, -1.0f})
        for (float v : {448.0f, 464.0f, 480.0f, 1e6f, 1e-30f, 0.0f})
            xs.push_back(s * v);
    for (int i = 0; i < 60000; ++i) {
        uint32_t b = (uint32_t)next_u64();
        float f;
        std::memcpy(&f, &b, 4);
        if (std::isfinite(f)) xs.push_back(f);
    }
    std::vector<uint8_t> codes(xs.size());
    for (size_t i = 0; i < xs.size(); ++i) codes[i] = rocm_e4m3(xs[i]);
    dump(dir + "/e4m3_rocm_inputs.f32", xs);
    dump(dir + "/e4m3_rocm_codes.u8", codes);

    // 2) FP8 append of 128 rows x 4 KV heads x 256 dims (BASELINE config 2 shape).
    const int R = 128, H = 4, D = 256;
    for (const char* name : {"k", "v"}) {
        std::vector<uint16_t> in((size_t)R * H * D);
        for (auto& x : in) {
            float f = next_normal();
            if (next_unit() < 0.01) f *= 20.0f;
            x = bf16_rne(f);
        }
        // one all-zero head (scale 1.0 special case) per tensor
        for (int d = 0; d < D; ++d) in[(size_t)(5 * H + 2) * D + d] = 0;
        std::vector<uint8_t> out((size_t)R * H * D);
        std::vector<float> sc((size_t)R * H);
        for (int r = 0; r < R; ++r)
            for (int h = 0; h < H; ++h) {
                const uint16_t* x = &in[((size_t)r * H + h) * D];
                float amax = 0.0f;
                for (int d = 0; d < D; ++d) amax = std::fmax(amax, std::fabs(bf16_f(x[d])));
                const float s = amax == 0.0f ? 1.0f : amax / 448.0f;
                sc[(size_t)r * H + h] = s;
                for (int d = 0; d < D; ++d)
                    out[((size_t)r * H + h) * D + d] = rocm_e4m3(bf16_f(x[d]) / s);
            }
        dump(dir + "/fp8_append_" + name + "_in.bf16", in);
        dump(dir + "/fp8_append_" + name + "_codes.u8", out);
        dump(dir + "/fp8_append_" + name + "_scale.f32", sc);
    }
    std::printf("wrote %zu codec vectors and the fp8 append fixture to %s\n", xs.size(), dir.c_str());
    return 0;
}
