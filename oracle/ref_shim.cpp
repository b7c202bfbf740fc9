// C entry points over the reference's own host codecs, compiled from the
// reference sources in place (see oracle/Makefile) into oracle/_ref/.
// TEST INFRASTRUCTURE ONLY: used by tests/ to pin the oracle's codecs.
//   ps::quantization::fpx::e4m3_encode_u8 / e4m3_decode_f32
//       reference src/phaseshift/quantization/fpx/e4m3.cpp:45-99
//   ps::f32_to_bf16_rne   reference include/phaseshift/core/memory/types.h:11-21
//   ps::quantization::psq::psq4_{maxabs,lsq1}_encode_block, psq4_pack_codes,
//   psq_bf16_round, cb10_encode / cb10_code_to_f32
//       reference include/phaseshift/quantization/psq/psq4_kv.h:9-79,
//       psq_device.h:13-35 (header-only host code)
//   ps::quantization::psq::psq8_{maxabs,lsq1}_encode_block
//       reference include/phaseshift/quantization/psq/psq8_kv.h:30-90 (host
//       branch: the reference's own e4m3 codec). psq8_kv.h includes
//       hip/hip_fp8.h, so this file is compiled by hipcc's host pass only.
#include <phaseshift/core/memory/types.h>
#include <phaseshift/quantization/fpx/e4m3.h>
#include <phaseshift/quantization/psq/psq4_kv.h>
#include <phaseshift/quantization/psq/psq8_kv.h>

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

void ref_psq4_encode_block(const float* x, uint32_t lsq1, float* scale, uint8_t* codes) {
    if (lsq1)
        ps::quantization::psq::psq4_lsq1_encode_block(x, 32u, *scale, codes);
    else
        ps::quantization::psq::psq4_maxabs_encode_block(x, 32u, *scale, codes);
}

void ref_psq4_pack_codes(const uint8_t* codes32, uint8_t* bytes16) {
    ps::quantization::psq::psq4_pack_codes(codes32, bytes16);
}

void ref_psq_bf16_round_array(const float* in, float* out, uint64_t n) {
    for (uint64_t i = 0; i < n; ++i) out[i] = ps::quantization::psq::psq_bf16_round(in[i]);
}

void ref_cb10_encode_array(const float* x, const float* inv, uint8_t* out, uint64_t n) {
    for (uint64_t i = 0; i < n; ++i) out[i] = ps::quantization::psq::cb10_encode(x[i], inv[i]);
}

void ref_psq8_encode_block(const float* x, uint32_t lsq1, float* scale, uint8_t* codes) {
    if (lsq1)
        ps::quantization::psq::psq8_lsq1_encode_block(x, 32u, *scale, codes);
    else
        ps::quantization::psq::psq8_maxabs_encode_block(x, 32u, *scale, codes);
}

float ref_cb10_code_to_f32(uint8_t c) { return ps::quantization::psq::cb10_code_to_f32(c); }

}  // extern "C"
