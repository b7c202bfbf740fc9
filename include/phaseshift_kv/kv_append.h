// KV append launchers with the reference's C++ signatures, so the reference's
// dispatcher (runtime/kv_append_dispatch.hip) links against them unchanged.
// Struct and signatures: reference
// include/phaseshift/models/qwen35/kernels/optimized/kv_append.h:12-97.
#pragma once
#include <phaseshift_kv/types.h>
#include <phaseshift_kv_c.h>
#include <hip/hip_runtime.h>
#include <cstddef>
#include <cstdint>

namespace ps::kernel {

struct KvAppendCommonArgs {
    const bf16_t* k_input = nullptr;
    const bf16_t* v_input = nullptr;
    uint32_t k_row_stride = 0;
    uint32_t v_row_stride = 0;
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
    uint32_t kv_heads = 0;
    uint32_t head_dim = 0;
    uint32_t elems_per_token = 0;
    uint32_t elems_per_page = 0;
    uint32_t elems_per_layer = 0;
};

// The ABI of the reference (kv_append.h:52-72) and of the C struct.
static_assert(sizeof(KvAppendCommonArgs) == 96);
static_assert(alignof(KvAppendCommonArgs) == 8);
static_assert(offsetof(KvAppendCommonArgs, k_row_stride) == 16);
static_assert(offsetof(KvAppendCommonArgs, row_sequence_slots) == 24);
static_assert(offsetof(KvAppendCommonArgs, block_tables) == 40);
static_assert(offsetof(KvAppendCommonArgs, block_table_stride) == 48);
static_assert(offsetof(KvAppendCommonArgs, rows) == 56);
static_assert(offsetof(KvAppendCommonArgs, page_tokens) == 64);
static_assert(offsetof(KvAppendCommonArgs, kv_heads) == 76);
static_assert(offsetof(KvAppendCommonArgs, elems_per_layer) == 92);
static_assert(sizeof(psk_kv_append_args) == sizeof(KvAppendCommonArgs));
static_assert(offsetof(psk_kv_append_args, rows) == offsetof(KvAppendCommonArgs, rows));
static_assert(offsetof(psk_kv_append_args, elems_per_layer) ==
              offsetof(KvAppendCommonArgs, elems_per_layer));

hipError_t launch_kv_append_bf16(const KvAppendCommonArgs& common, bf16_t* k_pool,
                                 bf16_t* v_pool, hipStream_t stream);

hipError_t launch_kv_append_fp8_e4m3(const KvAppendCommonArgs& common,
                                     ::ps::qwen35::fp8e4m3_storage_t* k_pool,
                                     ::ps::qwen35::fp8e4m3_storage_t* v_pool,
                                     float* k_scale_pool, float* v_scale_pool,
                                     hipStream_t stream);

}  // namespace ps::kernel

namespace ps::kernel {
// PSQ4_W32 / PSQ8_W32 appends (kv_append.h:99-125 of the reference): not
// provided by this build; they return hipErrorNotSupported, which the
// reference dispatcher turns into its correctness-kernel fallback.
hipError_t launch_kv_append_psq4(const KvAppendCommonArgs& common, uint8_t* k_code_pool,
                                 uint8_t* v_code_pool, bf16_t* k_scale_pool, bf16_t* v_scale_pool,
                                 uint32_t blocks_per_head,
                                 ::ps::qwen35::Psq4ScaleEstimator estimator, hipStream_t stream);
hipError_t launch_kv_append_psq8(const KvAppendCommonArgs& common, uint8_t* k_code_pool,
                                 uint8_t* v_code_pool, bf16_t* k_scale_pool, bf16_t* v_scale_pool,
                                 uint32_t blocks_per_head,
                                 ::ps::qwen35::Psq8ScaleEstimator estimator, hipStream_t stream);
}  // namespace ps::kernel
