// Planner of the PAGED_ATTENTION binding for one continuous-batching step.
// Mirrors the reference's resolve -> plan -> physical launch
// (src/phaseshift/models/qwen35/runtime/paged_attention_dispatch.hip:437-477,
// 705-894); see dispatch.cpp for the rules.
#pragma once
#include <phaseshift_kv/kv_state.h>
#include <phaseshift_kv/paged_attention.h>

#include <cstdint>
#include <vector>

namespace ps::qwen35::runtime {

// ExecutionClass values (include/phaseshift/runtime/execution/execution_types.h:11-16).
inline constexpr uint8_t kExecDecode = 0, kExecSpecVerify = 1, kExecPrefill = 2, kExecSpecDraft = 3;
// Reference constants: prefill kernel from 128 rows (paged_attention_dispatch.h:49),
// split-K from 2048 visible tokens (paged_attention_dispatch.hip:437).
inline constexpr uint32_t kPrefillMinRows = 128u;
inline constexpr uint32_t kSplitMinVisible = 2048u;
// Split sizing on MI355X: tile launches aim at ~8 workgroups per CU over 256
// CUs; every split holds at least 16 pages (256 tokens at page 16).
inline constexpr uint64_t kTargetWorkgroups = 2048u;
inline constexpr uint64_t kMinPagesPerSplit = 16u;
inline constexpr uint64_t kMaxSplits = 1024u;
inline constexpr uint32_t kMaxPlannedKernels = 16u;
// Requests routed to the multi-row tile kernel: PREFILL chunks of >= 128 rows
// (the reference's rule) and, new here, SPEC_VERIFY blocks of >= 8 rows, whose
// K/V is then read once per block instead of once per draft row.
inline constexpr uint32_t kVerifyTileMinRows = 8u;
inline constexpr uint32_t kTileRowsPerTile = 16u;
// A step's other launches run beside a tile launch of at least this many rows.
inline constexpr uint64_t kForkMinTileRows = 1024u;

struct StepRequest {
    uint32_t row_begin = 0;
    uint32_t row_count = 0;
    uint8_t execution_class = kExecDecode;
    uint32_t max_visible = 0;   // largest visible length of its rows; 0: unknown
};

struct PagedAttentionStep {
    ::ps::kernel::PagedAttentionCommonArgs common{};   // all rows of the step
    KVCacheDType kv_dtype = KVCacheDType::BF16;
    const void* k_pool = nullptr;
    const void* v_pool = nullptr;
    const void* k_scale_pool = nullptr;                 // FP8: f32; PSQ: bf16 block scales
    const void* v_scale_pool = nullptr;
    const StepRequest* requests = nullptr;              // host array
    uint32_t num_requests = 0;
    uint32_t max_visible_tokens = 0;
    float* partials = nullptr;                          // split-K workspace (device)
    uint64_t partial_bytes = 0;
    bool concurrent_decode = true;                      // other launches beside the largest tile launch
};

struct DecodeSplit {
    uint32_t splits = 1;
    uint32_t pages_per_split = 0;
};

struct PlannedKernel {
    enum class Kind : uint8_t { Decode, Tile } kind = Kind::Decode;
    uint32_t row_begin = 0;       // region of the launch (absolute step rows)
    uint32_t rows = 0;
    uint32_t splits = 1;
    uint32_t pages_per_split = 0;
    uint32_t tile_first = 0;      // Tile: range in PagedAttentionPlan::tiles
    uint32_t tile_count = 0;
    uint32_t tiles_per_group = 1; // Tile: consecutive tiles per workgroup (rows == 0 pads)
    uint32_t req_first = 0;       // Tile with splits > 1: combine ranges
    uint32_t req_count = 0;
    uint32_t side = 0;            // 1 / 2: runs on side lane 1 (decode) / 2 (other tile launches), beside the step's largest tile launch
    uint64_t partial_offset = 0;  // floats into the split-K workspace this launch uses
};

struct PlannedTile {
    uint32_t row_begin;   // absolute step row
    uint32_t rows;        // 1..16, one sequence; 0: padding of a tile group
};

struct PagedAttentionPlan {
    PlannedKernel kernels[kMaxPlannedKernels];
    uint32_t count = 0;
    std::vector<PlannedTile> tiles;
    std::vector<StepRequest> combine;   // row ranges combined after a split tile launch
};

// Split-K sizing of a decode launch: the split count (and pages per split)
// whose units finish first under the decode kernel's XCD-aware dispatch, given
// the rows' visible lengths (row_visible, host array; nullptr: every row at
// max_visible_tokens) and the partials workspace. splits == 1: do not split.
// kv_dtype: PSK_KV_* (KVCacheDType value).
DecodeSplit choose_decode_split(uint32_t rows, uint32_t kv_heads, uint32_t q_heads,
                                uint32_t head_dim, uint32_t kv_dtype, uint32_t page_tokens,
                                uint32_t max_visible_tokens, const uint32_t* row_visible,
                                uint64_t partial_bytes);
Status plan_paged_attention_step(const PagedAttentionStep& step, PagedAttentionPlan& plan);
hipError_t launch_paged_attention_plan(const PagedAttentionStep& step,
                                       const PagedAttentionPlan& plan, hipStream_t stream);

}  // namespace ps::qwen35::runtime
