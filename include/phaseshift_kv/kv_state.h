// Host-side KV state of the paged path: pool, sequence slots / block tables,
// per-sequence paging, prefix-cache page copy.
//
// Names, fields and error behaviour follow the reference so its runtime can
// keep its call sites:
//   PagedKVPool            include/phaseshift/models/qwen35/state/paged_kv_pool.h,
//                          src/phaseshift/models/qwen35/state/paged_kv_pool.cpp:27-244,338-542
//   SequenceSlotPool       state/sequence_slot_pool.h:14-45, .cpp:192-238
//   PagedSequenceState,
//   reserve/rollback/commit state/paged_sequence_state.h, .cpp:111-271
// Differences by design: device memory comes from hipMalloc (256 B aligned)
// instead of the reference's GpuArena; block-table truncation uses a fill
// kernel instead of hipMemsetAsync (stays correct under HIP-graph capture);
// page copies of any number of pages and layers run as one kernel launch.
#pragma once
#include <phaseshift_kv/types.h>
#include <phaseshift_kv_c.h>
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <string>
#include <vector>

namespace ps {

// Minimal Status with the reference's categories (core/status.h).
struct Status {
    enum class Code : uint8_t {
        Ok = 0,
        InvalidArgument,
        OutOfRange,
        InvalidState,
        InsufficientMemory,
        HipError,
    };
    Code code = Code::Ok;
    std::string message;

    bool ok() const noexcept { return code == Code::Ok; }
    static Status make_ok() { return {}; }
    static Status invalid_argument(std::string m) { return {Code::InvalidArgument, std::move(m)}; }
    static Status out_of_range(std::string m) { return {Code::OutOfRange, std::move(m)}; }
    static Status invalid_state(std::string m) { return {Code::InvalidState, std::move(m)}; }
    static Status insufficient_memory(std::string m) {
        return {Code::InsufficientMemory, std::move(m)};
    }
    static Status hip_error(std::string where, hipError_t e) {
        return {Code::HipError, where + ": " + hipGetErrorString(e)};
    }
};

namespace qwen35 {

class PagedKVPool {
public:
    PagedKVPool() = default;
    ~PagedKVPool();
    PagedKVPool(const PagedKVPool&) = delete;
    PagedKVPool& operator=(const PagedKVPool&) = delete;
    PagedKVPool(PagedKVPool&& o) noexcept;
    PagedKVPool& operator=(PagedKVPool&& o) noexcept;

    // K/V pools [layers][num_pages][page_tokens][kv_heads][head_dim] (bf16 or
    // e4m3 bytes) and, for FP8, f32 scale pools [layers][num_pages][page_tokens][kv_heads].
    // PSQ4_W32 / PSQ8_W32: code pools of 16 / 32 bytes per 32-value block and
    // bf16 scale pools, one per block, block index
    // ((((layer*num_pages + page)*page_tokens + off)*kv_heads + head)*head_dim/32 + d/32)
    // (kv_cache_types.h:16-46; psq4 reserves 1152 B per token at 4 x 256).
    static Status create(PagedKVPool& out, uint32_t num_pages, uint32_t page_tokens,
                         uint32_t num_attention_layers, uint32_t kv_heads, uint32_t head_dim,
                         KVCacheDType dtype);

    // Free list: LIFO, pages handed out from the back (paged_kv_pool.cpp:196-205).
    Status allocate(PageId& page);
    Status release(PageId page);
    Status release_many(const std::vector<PageId>& pages);
    uint32_t num_free_pages() const noexcept { return static_cast<uint32_t>(free_list_.size()); }
    uint32_t used_count() const noexcept { return used_count_; }
    bool in_use(PageId page) const noexcept { return page < num_pages_ && in_use_[page]; }

    // Copies page src_page of `src` into dst_page of this pool, every layer,
    // K and V bodies plus the FP8 scale rows (paged_kv_pool.cpp:338-542).
    Status copy_page_from(PageId dst_page, const PagedKVPool& src, PageId src_page,
                          hipStream_t stream);
    // Any number of (dst, src) page pairs in one launch per 256 pairs.
    Status copy_pages_from(const std::vector<PageId>& dst_pages, const PagedKVPool& src,
                           const std::vector<PageId>& src_pages, hipStream_t stream);
    // The checked copy arguments and pairs of such a copy, for callers that
    // batch it with other copies into one launch.
    Status copy_pairs_from(const std::vector<PageId>& dst_pages, const PagedKVPool& src,
                           const std::vector<PageId>& src_pages, psk_page_copy_args& args,
                           std::vector<psk_page_copy_pair>& pairs) const;
    // Bytes of one page of one layer: K (or V) body and scale rows.
    uint64_t page_body_bytes() const noexcept;
    uint64_t page_scale_bytes() const noexcept;

    uint32_t num_pages() const noexcept { return num_pages_; }
    uint32_t page_tokens() const noexcept { return page_tokens_; }
    uint32_t num_attention_layers() const noexcept { return num_attention_layers_; }
    uint32_t kv_heads() const noexcept { return kv_heads_; }
    uint32_t head_dim() const noexcept { return head_dim_; }
    KVCacheDType dtype() const noexcept { return dtype_; }
    uint32_t elems_per_token() const noexcept { return kv_heads_ * head_dim_; }
    uint32_t elems_per_page() const noexcept { return page_tokens_ * elems_per_token(); }
    uint64_t elems_per_layer() const noexcept { return (uint64_t)num_pages_ * elems_per_page(); }
    uint64_t reserved_bytes() const noexcept { return reserved_bytes_; }

    void* k_pool() const noexcept { return k_; }
    void* v_pool() const noexcept { return v_; }
    // FP8: f32 scales; PSQ: the bf16 block scales (bit patterns) at this address
    float* k_scale_pool() const noexcept { return k_scale_; }
    float* v_scale_pool() const noexcept { return v_scale_; }

private:
    void destroy() noexcept;
    uint32_t num_pages_ = 0, page_tokens_ = 0, num_attention_layers_ = 0, kv_heads_ = 0,
             head_dim_ = 0;
    KVCacheDType dtype_ = KVCacheDType::BF16;
    void* k_ = nullptr;
    void* v_ = nullptr;
    float* k_scale_ = nullptr;
    float* v_scale_ = nullptr;
    uint64_t reserved_bytes_ = 0;
    std::vector<PageId> free_list_;
    std::vector<bool> in_use_;
    uint32_t used_count_ = 0;
};

// Device block tables uint32 [max_sequences][max_blocks], empty = kInvalidPageId.
class SequenceSlotPool {
public:
    SequenceSlotPool() = default;
    ~SequenceSlotPool();
    SequenceSlotPool(const SequenceSlotPool&) = delete;
    SequenceSlotPool& operator=(const SequenceSlotPool&) = delete;

    static Status create(SequenceSlotPool& out, uint32_t max_sequences, uint32_t max_blocks,
                         hipStream_t stream);
    Status allocate(SequenceSlotId& slot);
    Status release(SequenceSlotId slot, hipStream_t stream);
    Status set_blocks(SequenceSlotId slot, uint32_t first_block, const PageId* pages,
                      uint32_t count, hipStream_t stream);
    // Entries [first_block, first_block + block_count) of the slot <- kInvalidPageId.
    Status clear_blocks(SequenceSlotId slot, uint32_t first_block, uint32_t block_count,
                        hipStream_t stream);
    Status clear_slot(SequenceSlotId slot, hipStream_t stream);

    uint32_t max_sequences() const noexcept { return max_sequences_; }
    uint32_t max_blocks() const noexcept { return max_blocks_; }
    uint32_t* device_block_tables() const noexcept { return tables_; }
    bool in_use(SequenceSlotId s) const noexcept { return s < max_sequences_ && in_use_[s]; }

private:
    uint32_t max_sequences_ = 0, max_blocks_ = 0;
    uint32_t* tables_ = nullptr;
    std::vector<bool> in_use_;
    std::vector<SequenceSlotId> free_slots_;
};

struct PagedSequenceState {
    SequenceSlotId slot = kInvalidSlot;
    uint32_t generation = 0;
    uint32_t position = 0;          // committed tokens
    uint32_t max_seq_len = 0;
    std::vector<PageId> block_table;

    bool is_allocated() const noexcept { return slot != kInvalidSlot; }
    bool is_usable() const noexcept { return is_allocated() && generation != 0u && !poisoned; }
    bool is_poisoned() const noexcept { return poisoned; }
    void mark_poisoned() noexcept { poisoned = true; }

    PagedKVPool* kv_pool = nullptr;
    SequenceSlotPool* seq_pool = nullptr;
    uint32_t max_blocks = 0;
    bool poisoned = false;
};

Status create_paged_sequence_state(PagedSequenceState& out, SequenceSlotPool& seq_pool,
                                   PagedKVPool& kv_pool, uint32_t max_seq_len,
                                   hipStream_t stream);
Status release_paged_sequence_state(PagedSequenceState& seq, hipStream_t stream);
// Pages for `token_count` more tokens past `position`; new block-table entries
// are written to the device table (paged_sequence_state.cpp:111-187).
Status reserve_sequence_append(PagedSequenceState& seq, uint32_t token_count, hipStream_t stream);
// Truncation back to old_block_count pages: device entries cleared, pages
// freed; any failure poisons the sequence (paged_sequence_state.cpp:189-229).
Status rollback_sequence_append(PagedSequenceState& seq, uint32_t old_block_count,
                                hipStream_t stream);
Status commit_sequence_append(PagedSequenceState& seq, uint32_t committed_tokens);

}  // namespace qwen35
}  // namespace ps
