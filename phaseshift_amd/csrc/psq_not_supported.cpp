// The PSQ4_W32 / PSQ8_W32 part of the reference launcher surface, so this
// library links in place of the reference's kv_append.hip, paged_decode.hip
// and paged_prefill.hip. PSQ KV is not built here yet: every launcher returns
// hipErrorNotSupported, which the reference dispatcher maps to NotApplicable
// and its correctness-kernel fallback (runtime/paged_attention_dispatch.hip:917-926).
#include <phaseshift_kv/kv_append.h>
#include <phaseshift_kv/paged_attention.h>

namespace ps::kernel {

hipError_t launch_kv_append_psq4(const KvAppendCommonArgs&, uint8_t*, uint8_t*, bf16_t*, bf16_t*,
                                 uint32_t, ::ps::qwen35::Psq4ScaleEstimator, hipStream_t) {
    return hipErrorNotSupported;
}
hipError_t launch_kv_append_psq8(const KvAppendCommonArgs&, uint8_t*, uint8_t*, bf16_t*, bf16_t*,
                                 uint32_t, ::ps::qwen35::Psq8ScaleEstimator, hipStream_t) {
    return hipErrorNotSupported;
}
uint32_t paged_attention_split_reduce_qh_per_wg() { return 1u; }
hipError_t launch_attention_paged_psq4(const PagedAttentionCommonArgs&, const uint8_t*,
                                       const uint8_t*, const bf16_t*, const bf16_t*, uint32_t,
                                       hipStream_t) {
    return hipErrorNotSupported;
}
hipError_t launch_attention_paged_psq8(const PagedAttentionCommonArgs&, const uint8_t*,
                                       const uint8_t*, const bf16_t*, const bf16_t*, uint32_t,
                                       hipStream_t) {
    return hipErrorNotSupported;
}
hipError_t launch_attention_paged_prefill_psq4(const PagedAttentionCommonArgs&, const uint8_t*,
                                               const uint8_t*, const bf16_t*, const bf16_t*,
                                               uint32_t, hipStream_t) {
    return hipErrorNotSupported;
}
hipError_t launch_attention_paged_prefill_psq8(const PagedAttentionCommonArgs&, const uint8_t*,
                                               const uint8_t*, const bf16_t*, const bf16_t*,
                                               uint32_t, hipStream_t) {
    return hipErrorNotSupported;
}
hipError_t launch_attention_paged_psq8_split(const PagedAttentionCommonArgs&, const uint8_t*,
                                             const uint8_t*, const bf16_t*, const bf16_t*, uint32_t,
                                             float*, uint32_t, hipStream_t) {
    return hipErrorNotSupported;
}
hipError_t launch_attention_paged_psq4_split(const PagedAttentionCommonArgs&, const uint8_t*,
                                             const uint8_t*, const bf16_t*, const bf16_t*, uint32_t,
                                             float*, uint32_t, hipStream_t) {
    return hipErrorNotSupported;
}

}  // namespace ps::kernel
