// Library-level C-ABI entry points and the multi-row tile launchers.
#include <phaseshift_kv/paged_attention.h>
#include <phaseshift_kv_c.h>
#include <hip/hip_runtime.h>

extern "C" const char* psk_version(void) { return "phaseshift-kv-mi355x 0.1.0"; }

extern "C" const char* psk_build_arch(void) { return "gfx950"; }

extern "C" const char* psk_error_string(int err) {
    return hipGetErrorName(static_cast<hipError_t>(err));
}

namespace ps::kernel {

hipError_t launch_attention_paged_prefill_bf16(const PagedAttentionCommonArgs& common,
                                               const bf16_t* k_pool, const bf16_t* v_pool,
                                               hipStream_t stream) {
    return static_cast<hipError_t>(psk_attention_paged_prefill_bf16(
        reinterpret_cast<const psk_paged_attention_args*>(&common), k_pool, v_pool, stream));
}

hipError_t launch_attention_paged_prefill_fp8_e4m3(
    const PagedAttentionCommonArgs& common, const ::ps::qwen35::fp8e4m3_storage_t* k_pool,
    const ::ps::qwen35::fp8e4m3_storage_t* v_pool, const float* k_scale_pool,
    const float* v_scale_pool, hipStream_t stream) {
    return static_cast<hipError_t>(psk_attention_paged_prefill_fp8_e4m3(
        reinterpret_cast<const psk_paged_attention_args*>(&common), k_pool, v_pool, k_scale_pool,
        v_scale_pool, stream));
}

}  // namespace ps::kernel
