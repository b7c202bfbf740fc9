// C entry points over the reference's own host codecs, compiled from the
// reference sources in place (see oracle/Makefile) into oracle/_ref/.
// TEST INFRASTRUCTURE ONLY: used by tests/ to pin the oracle's codecs.
//   ps::quantization::fpx::e4m3_encode_u8 / e4m3_decode_f32
//       reference src/phaseshift/quantization/fpx/e4m3.cpp:45-99
//   ps::f32_to_bf16_rne   reference include/phaseshift/core/memory/types.h:11-21
#include <phaseshift/core/memory/types.h>
#include <phaseshift/quantization/fpx/e4m3.h>

#include <cstdint>
#include <cstring>

extern "C" {

void ref_e4m3_encode_range(uint32_t start_bits, uint32_t count, uint8_t* out) {
    for (uint32_t i = 0; i < count; ++i) {
        const uint32_t b = start_bits + i;
        float f;
        std::memcpy(&f, &b, 4);
        out[i] = ps::quantization::fpx::e4m3_encode_u8(f);
    }
}

void ref_e4m3_decode_all(float* out256) {
    for (uint32_t x = 0; x < 256; ++x)
        out256[x] = ps::quantization::fpx::e4m3_decode_f32(static_cast<uint8_t>(x));
}

void ref_f32_to_bf16_range(uint32_t start_bits, uint32_t count, uint16_t* out) {
    for (uint32_t i = 0; i < count; ++i) {
        const uint32_t b = start_bits + i;
        float f;
        std::memcpy(&f, &b, 4);
        out[i] = ps::f32_to_bf16_rne(f);
    }
}

}  // extern "C"
