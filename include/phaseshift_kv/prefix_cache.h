// Prefix cache of the paged KV path: checkpoints of a sequence's KV pages,
// its GDN recurrent-state slot and (optionally) its DFlash context ring, kept
// in cache-owned pools with LRU eviction, restored into a fresh sequence.
//
// Names, fields and behaviour follow the reference so its runtime keeps its
// call sites:
//   PrefixCache, PrefixCheckpoint, PrefixCacheStats
//       include/phaseshift/models/qwen35/runtime/prefix_cache.h,
//       src/phaseshift/models/qwen35/runtime/prefix_cache.cpp:84-486
//   GdnStatePool, GdnStatePoolLayout
//       include/phaseshift/models/qwen35/state/gdn_state_pool.h:41-120,
//       src/phaseshift/models/qwen35/state/gdn_state_pool.cpp:10-355
// Differences by design: a save or a restore moves all of its bytes (every
// page of every layer, K/V bodies and scale rows, both GDN state tensors of
// the slot, both ring tensors) with one batched copy launch instead of 4 x L
// copies per page plus four more; slot zeroing uses a fill kernel (no
// hipMemsetAsync), and a cache slot is not zeroed before the copy that
// overwrites all of it.
#pragma once
#include <phaseshift_kv/kv_state.h>

#include <cstdint>
#include <optional>
#include <vector>

namespace ps::qwen35 {

struct GdnStatePoolLayout {
    uint32_t num_gdn_states = 0;
    uint32_t conv_dim = 0;
    uint32_t conv_dim_padded = 0;
    uint32_t conv_history = 0;
    uint32_t conv_history_stride = 0;
    uint32_t num_v_heads = 0;
    uint32_t head_k = 0;
    uint32_t head_v = 0;

    // gdn_state_pool.h:52-66: conv_dim padded to a multiple of 8, which is
    // also the history row stride.
    static GdnStatePoolLayout make(uint32_t gdn_layers, uint32_t conv_dim, uint32_t conv_history,
                                   uint32_t num_v_heads, uint32_t head_k, uint32_t head_v) {
        const uint32_t padded = (conv_dim + 7u) & ~7u;
        return {gdn_layers, conv_dim, padded, conv_history, padded, num_v_heads, head_k, head_v};
    }
    bool operator==(const GdnStatePoolLayout& o) const noexcept {
        return num_gdn_states == o.num_gdn_states && conv_dim == o.conv_dim &&
               conv_dim_padded == o.conv_dim_padded && conv_history == o.conv_history &&
               conv_history_stride == o.conv_history_stride && num_v_heads == o.num_v_heads &&
               head_k == o.head_k && head_v == o.head_v;
    }
    // Per slot: bf16 conv history [states][conv_history][stride] and f32
    // recurrent state [states][v_heads][head_k][head_v].
    uint64_t conv_slot_bytes() const noexcept {
        return (uint64_t)num_gdn_states * conv_history * conv_history_stride * 2;
    }
    uint64_t recurrent_slot_bytes() const noexcept {
        return (uint64_t)num_gdn_states * num_v_heads * head_k * head_v * 4;
    }
};

class GdnStatePool {
public:
    GdnStatePool() = default;
    ~GdnStatePool();
    GdnStatePool(const GdnStatePool&) = delete;
    GdnStatePool& operator=(const GdnStatePool&) = delete;
    GdnStatePool(GdnStatePool&& o) noexcept;
    GdnStatePool& operator=(GdnStatePool&& o) noexcept;

    static Status create(GdnStatePool& out, uint32_t max_sequences, const GdnStatePoolLayout& layout);
    // Marks the slot in use and zeroes its state (gdn_state_pool.cpp:139-183).
    Status initialize(SequenceSlotId slot, hipStream_t stream);
    Status reset(SequenceSlotId slot, hipStream_t stream);
    Status release(SequenceSlotId slot);
    // Marks the slot in use without zeroing (the caller overwrites all of it).
    Status acquire(SequenceSlotId slot);
    Status copy_slot_from(SequenceSlotId dst_slot, const GdnStatePool& src, SequenceSlotId src_slot,
                          hipStream_t stream);

    uint32_t max_sequences() const noexcept { return max_slots_; }
    const GdnStatePoolLayout& layout() const noexcept { return layout_; }
    uint64_t reserved_bytes() const noexcept {
        return (uint64_t)max_slots_ * (layout_.conv_slot_bytes() + layout_.recurrent_slot_bytes());
    }
    uint64_t bytes_per_slot() const noexcept {
        return layout_.conv_slot_bytes() + layout_.recurrent_slot_bytes();
    }
    uint32_t num_used_slots() const noexcept { return used_count_; }
    bool in_use(SequenceSlotId s) const noexcept { return s < max_slots_ && initialized_[s]; }
    void* conv_slot(SequenceSlotId s) const noexcept {
        return static_cast<uint8_t*>(conv_) + (uint64_t)s * layout_.conv_slot_bytes();
    }
    void* recurrent_slot(SequenceSlotId s) const noexcept {
        return static_cast<uint8_t*>(recurrent_) + (uint64_t)s * layout_.recurrent_slot_bytes();
    }
    void* conv_base() const noexcept { return conv_; }
    void* recurrent_base() const noexcept { return recurrent_; }

private:
    void destroy() noexcept;
    uint32_t max_slots_ = 0;
    GdnStatePoolLayout layout_{};
    void* conv_ = nullptr;
    void* recurrent_ = nullptr;
    std::vector<bool> initialized_;
    uint32_t used_count_ = 0;
};

// The drafter's DFlash2 context ring as the prefix cache sees it
// (dflash2/context_state.h:15-27): two ring tensors of ring_bytes each plus
// the ring's fill length and next position.
struct DFlashContextView {
    void* k_ring = nullptr;
    void* v_ring = nullptr;
    uint64_t ring_bytes = 0;
    uint32_t length = 0;
    uint32_t next_position = 0;
};

struct PrefixCheckpoint {
    uint64_t id = 0;   // stable handle (the entry vector is reordered on eviction)
    std::vector<int32_t> tokens;
    uint32_t position = 0;
    std::vector<PageId> cache_pages;
    SequenceSlotId cache_state_slot = kInvalidSlot;
    uint64_t last_used = 0;

    bool dflash = false;
    uint32_t dflash_slot = 0u;
    uint32_t dflash_length = 0u;
    uint32_t dflash_next_position = 0u;
};

struct PrefixCacheStats {
    uint64_t lookups = 0;
    uint64_t hits = 0;
    uint64_t misses = 0;
    uint64_t inserts = 0;
    uint64_t duplicate_hits = 0;
    uint64_t evictions = 0;
    uint64_t skipped_too_large = 0;
    uint64_t restored_tokens = 0;
    uint64_t saved_tokens = 0;
    uint64_t save_d2d_bytes = 0;
    uint64_t restore_d2d_bytes = 0;
    uint64_t copy_launches = 0;   // batched copy launches issued by save / restore
};

class PrefixCache {
public:
    PrefixCache() = default;
    ~PrefixCache();
    PrefixCache(const PrefixCache&) = delete;
    PrefixCache& operator=(const PrefixCache&) = delete;

    // Cache pools shaped like the active ones: ceil(capacity_tokens / P) KV
    // pages, max_entries GDN slots (prefix_cache.cpp:84-127).
    static Status create(PrefixCache& out, const PagedKVPool& active_kv,
                         const GdnStatePool& active_gdn, uint32_t capacity_tokens,
                         uint32_t max_entries, uint32_t min_prefix_tokens = 64);
    // One DFlash ring pair of ring_bytes each per entry (prefix_cache.cpp:175-197).
    Status enable_dflash_ring(uint64_t ring_bytes);

    bool enabled() const noexcept { return capacity_tokens_ != 0 && max_entries_ != 0; }
    bool dflash_ring_enabled() const noexcept { return !k_rings_.empty(); }
    uint32_t capacity_tokens() const noexcept { return capacity_tokens_; }
    uint32_t max_entries() const noexcept { return max_entries_; }
    uint32_t cache_pages() const noexcept { return cache_kv_ ? cache_kv_->num_pages() : 0; }
    uint32_t cache_free_pages() const noexcept { return cache_kv_ ? cache_kv_->num_free_pages() : 0; }
    uint32_t cache_free_slots() const noexcept { return (uint32_t)free_state_slots_.size(); }
    uint64_t cache_kv_bytes() const noexcept { return cache_kv_ ? cache_kv_->reserved_bytes() : 0; }
    uint64_t cache_gdn_bytes() const noexcept { return cache_gdn_ ? cache_gdn_->reserved_bytes() : 0; }
    uint64_t dflash_ring_bytes() const noexcept { return ring_bytes_ * 2u; }

    // The longest cached prefix of `tokens` (strictly shorter if asked);
    // refreshes its LRU stamp (prefix_cache.cpp:138-173).
    const PrefixCheckpoint* find_longest(const std::vector<int32_t>& tokens,
                                         bool strictly_shorter = false);
    const PrefixCheckpoint* find_id(uint64_t id) const;

    // Checkpoint of `sequence` (tokens.size() == position) unless shorter than
    // min_prefix_tokens, already cached, or larger than the cache; evicts LRU
    // entries to make room (prefix_cache.cpp:213-360).
    Status save(const PagedSequenceState& sequence, const GdnStatePool& gdn_pool,
                const PagedKVPool& kv_pool, std::vector<int32_t> tokens, hipStream_t stream,
                bool prompt_boundary = false, const DFlashContextView* dflash_context = nullptr);
    // Into an empty sequence: reserve, copy pages, GDN slot and ring, commit
    // (prefix_cache.cpp:362-460).
    Status restore(PagedSequenceState& sequence, GdnStatePool& gdn_pool, PagedKVPool& kv_pool,
                   const PrefixCheckpoint& checkpoint, hipStream_t stream,
                   DFlashContextView* dflash_context = nullptr);
    void clear() noexcept;

    size_t size() const noexcept { return entries_.size(); }
    const PrefixCacheStats& stats() const noexcept { return stats_; }

private:
    void evict_lru();
    void release_checkpoint(PrefixCheckpoint& entry) noexcept;
    void destroy_rings() noexcept;
    void destroy_staging() noexcept;
    // The page pairs of one save / restore, copied to the device so that the
    // whole copy is one launch: a pinned host staging buffer (reused once the
    // previous upload from it has completed) and a device buffer (reused in
    // stream order; one stream per cache).
    Status launch_copy(const psk_page_copy_args& kv, const std::vector<psk_page_copy_pair>& pairs,
                       const void* segs, uint32_t nseg, hipStream_t stream);

    std::optional<PagedKVPool> cache_kv_;
    std::optional<GdnStatePool> cache_gdn_;
    std::vector<void*> k_rings_, v_rings_;
    std::vector<uint32_t> free_ring_slots_;
    uint64_t ring_bytes_ = 0;
    psk_page_copy_pair* pairs_host_ = nullptr;   // pinned
    psk_page_copy_pair* pairs_dev_ = nullptr;
    uint32_t pairs_cap_ = 0;
    hipEvent_t pairs_ev_ = nullptr;
    bool pairs_ev_pending_ = false;
    uint32_t capacity_tokens_ = 0;
    uint32_t max_entries_ = 0;
    uint32_t min_prefix_tokens_ = 64;
    std::vector<PrefixCheckpoint> entries_;
    std::vector<uint32_t> free_state_slots_;
    uint64_t clock_ = 0;
    uint64_t next_id_ = 1;
    PrefixCacheStats stats_{};
};

}  // namespace ps::qwen35
