// Paged-attention launchers with the reference's C++ signatures.
// Structs and signatures: reference
// include/phaseshift/models/qwen35/kernels/optimized/attention/paged_attention.h:12-201.
#pragma once
#include <phaseshift_kv/types.h>
#include <phaseshift_kv_c.h>
#include <hip/hip_runtime.h>
#include <cstddef>
#include <cstdint>

namespace ps::kernel {

constexpr uint32_t kPagedAttentionHeadLimit = 256u;
inline constexpr uint32_t kPagedAttentionPrefillTileRows = 32u;

enum class PagedAttentionOutputDType : uint8_t {
    BF16,
    F32,
};

struct PagedAttentionCommonArgs {
    const bf16_t* q = nullptr;
    void* output = nullptr;
    PagedAttentionOutputDType output_dtype = PagedAttentionOutputDType::BF16;
    uint32_t q_row_stride = 0;
    uint32_t output_row_stride = 0;
    const uint32_t* row_sequence_slots = nullptr;
    const uint32_t* row_positions = nullptr;
    const uint32_t* block_tables = nullptr;
    uint32_t block_table_stride = 0;
    uint32_t max_sequences = 0;
    uint32_t rows = 0;
    uint32_t layer = 0;
    uint32_t page_tokens = 0;
    uint32_t num_pages = 0;
    uint32_t num_attention_layers = 0;
    uint32_t q_heads = 0;
    uint32_t kv_heads = 0;
    uint32_t head_dim = 0;
    uint32_t elems_per_token = 0;
    uint32_t elems_per_page = 0;
    uint32_t elems_per_layer = 0;
    float scale = 0.0f;
};

// The ABI of the reference (paged_attention.h:86-109) and of the C struct.
static_assert(sizeof(PagedAttentionCommonArgs) == 112);
static_assert(alignof(PagedAttentionCommonArgs) == 8);
static_assert(offsetof(PagedAttentionCommonArgs, output_dtype) == 16);
static_assert(offsetof(PagedAttentionCommonArgs, q_row_stride) == 20);
static_assert(offsetof(PagedAttentionCommonArgs, row_sequence_slots) == 32);
static_assert(offsetof(PagedAttentionCommonArgs, block_table_stride) == 56);
static_assert(offsetof(PagedAttentionCommonArgs, rows) == 64);
static_assert(offsetof(PagedAttentionCommonArgs, q_heads) == 84);
static_assert(offsetof(PagedAttentionCommonArgs, elems_per_layer) == 104);
static_assert(offsetof(PagedAttentionCommonArgs, scale) == 108);
static_assert(sizeof(psk_paged_attention_args) == sizeof(PagedAttentionCommonArgs));
static_assert(offsetof(psk_paged_attention_args, output_dtype) ==
              offsetof(PagedAttentionCommonArgs, output_dtype));
static_assert(offsetof(psk_paged_attention_args, scale) ==
              offsetof(PagedAttentionCommonArgs, scale));

hipError_t launch_attention_paged_bf16(const PagedAttentionCommonArgs& common,
                                       const bf16_t* k_pool, const bf16_t* v_pool,
                                       hipStream_t stream);

hipError_t launch_attention_paged_prefill_bf16(const PagedAttentionCommonArgs& common,
                                               const bf16_t* k_pool, const bf16_t* v_pool,
                                               hipStream_t stream);

hipError_t launch_attention_paged_prefill_fp8_e4m3(
    const PagedAttentionCommonArgs& common, const ::ps::qwen35::fp8e4m3_storage_t* k_pool,
    const ::ps::qwen35::fp8e4m3_storage_t* v_pool, const float* k_scale_pool,
    const float* v_scale_pool, hipStream_t stream);

hipError_t launch_attention_paged_fp8_e4m3(
    const PagedAttentionCommonArgs& common, const ::ps::qwen35::fp8e4m3_storage_t* k_pool,
    const ::ps::qwen35::fp8e4m3_storage_t* v_pool, const float* k_scale_pool,
    const float* v_scale_pool, hipStream_t stream);

hipError_t launch_attention_paged_bf16_split(const PagedAttentionCommonArgs& common,
                                             const bf16_t* k_pool, const bf16_t* v_pool,
                                             float* partials, uint32_t splits,
                                             hipStream_t stream);

hipError_t launch_attention_paged_bf16_split_reduce(const PagedAttentionCommonArgs& common,
                                                    const float* partials, uint32_t splits,
                                                    hipStream_t stream);

// Additive FP8 split-K pair (no reference counterpart; the reference FP8 path
// has no split, paged_decode.hip:941-1177).
hipError_t launch_attention_paged_fp8_e4m3_split(
    const PagedAttentionCommonArgs& common, const ::ps::qwen35::fp8e4m3_storage_t* k_pool,
    const ::ps::qwen35::fp8e4m3_storage_t* v_pool, const float* k_scale_pool,
    const float* v_scale_pool, float* partials, uint32_t splits, uint32_t pages_per_split,
    hipStream_t stream);

hipError_t launch_attention_paged_split_reduce_ex(const PagedAttentionCommonArgs& common,
                                                  const float* partials, uint32_t splits,
                                                  uint32_t pages_per_split,
                                                  hipStream_t stream);

}  // namespace ps::kernel

namespace ps::kernel {
// PSQ attention launchers (paged_attention.h:203-283 of the reference) and the
// split-reduce variant knob (:35): not provided by this build (PSQ KV is a
// later row); the launchers return hipErrorNotSupported, which the reference
// dispatcher turns into its correctness-kernel fallback.
uint32_t paged_attention_split_reduce_qh_per_wg();
hipError_t launch_attention_paged_psq4(const PagedAttentionCommonArgs& common,
                                       const uint8_t* k_code_pool, const uint8_t* v_code_pool,
                                       const bf16_t* k_scale_pool, const bf16_t* v_scale_pool,
                                       uint32_t blocks_per_head, hipStream_t stream);
hipError_t launch_attention_paged_psq8(const PagedAttentionCommonArgs& common,
                                       const uint8_t* k_code_pool, const uint8_t* v_code_pool,
                                       const bf16_t* k_scale_pool, const bf16_t* v_scale_pool,
                                       uint32_t blocks_per_head, hipStream_t stream);
hipError_t launch_attention_paged_prefill_psq4(const PagedAttentionCommonArgs& common,
                                               const uint8_t* k_code_pool,
                                               const uint8_t* v_code_pool,
                                               const bf16_t* k_scale_pool,
                                               const bf16_t* v_scale_pool,
                                               uint32_t blocks_per_head, hipStream_t stream);
hipError_t launch_attention_paged_prefill_psq8(const PagedAttentionCommonArgs& common,
                                               const uint8_t* k_code_pool,
                                               const uint8_t* v_code_pool,
                                               const bf16_t* k_scale_pool,
                                               const bf16_t* v_scale_pool,
                                               uint32_t blocks_per_head, hipStream_t stream);
hipError_t launch_attention_paged_psq8_split(const PagedAttentionCommonArgs& common,
                                             const uint8_t* k_code_pool, const uint8_t* v_code_pool,
                                             const bf16_t* k_scale_pool, const bf16_t* v_scale_pool,
                                             uint32_t blocks_per_head, float* partials,
                                             uint32_t splits, hipStream_t stream);
hipError_t launch_attention_paged_psq4_split(const PagedAttentionCommonArgs& common,
                                             const uint8_t* k_code_pool, const uint8_t* v_code_pool,
                                             const bf16_t* k_scale_pool, const bf16_t* v_scale_pool,
                                             uint32_t blocks_per_head, float* partials,
                                             uint32_t splits, hipStream_t stream);
}  // namespace ps::kernel
