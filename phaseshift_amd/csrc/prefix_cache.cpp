// Prefix cache and GDN state pool (host side). Behaviour restated from the
// reference (file:line in the reference repository):
//   GdnStatePool::create / initialize / reset / release / copy_slot_from
//       src/phaseshift/models/qwen35/state/gdn_state_pool.cpp:10-355
//   PrefixCache::create                 runtime/prefix_cache.cpp:84-127
//   find_exact / find_longest           runtime/prefix_cache.cpp:129-173
//   release_checkpoint / evict_lru      runtime/prefix_cache.cpp:175-211
//   save                                runtime/prefix_cache.cpp:213-360
//   restore                             runtime/prefix_cache.cpp:362-460
//   clear                               runtime/prefix_cache.cpp:462-480
// A save or restore issues its copies as one batched launch (page_ops.hip
// copy plan): the checkpoint's pages x layers x {K, V, K scales, V scales},
// the GDN slot's conv history and recurrent state, and the two DFlash rings.
#include <phaseshift_kv/prefix_cache.h>

#include "page_ops.h"

#include <algorithm>
#include <utility>

namespace ps::qwen35 {

namespace {
uint32_t pages_for(uint32_t position, uint32_t page_tokens) {
    return page_tokens == 0 ? 0 : (position + page_tokens - 1u) / page_tokens;
}
}  // namespace

// ------------------------------------------------------------ GdnStatePool
GdnStatePool::~GdnStatePool() { destroy(); }

void GdnStatePool::destroy() noexcept {
    if (conv_) (void)hipFree(conv_);
    if (recurrent_) (void)hipFree(recurrent_);
    conv_ = recurrent_ = nullptr;
}

GdnStatePool::GdnStatePool(GdnStatePool&& o) noexcept { *this = std::move(o); }

GdnStatePool& GdnStatePool::operator=(GdnStatePool&& o) noexcept {
    if (this != &o) {
        destroy();
        max_slots_ = o.max_slots_;
        layout_ = o.layout_;
        conv_ = o.conv_;
        recurrent_ = o.recurrent_;
        initialized_ = std::move(o.initialized_);
        used_count_ = o.used_count_;
        o.conv_ = o.recurrent_ = nullptr;
        o.max_slots_ = o.used_count_ = 0;
    }
    return *this;
}

Status GdnStatePool::create(GdnStatePool& out, uint32_t max_sequences,
                            const GdnStatePoolLayout& layout) {
    if (max_sequences == 0) return Status::invalid_argument("max_sequences must be > 0");
    if (layout.num_gdn_states == 0 || layout.conv_dim == 0 || layout.conv_dim_padded == 0 ||
        layout.conv_history == 0 || layout.conv_history_stride == 0 || layout.num_v_heads == 0 ||
        layout.head_k == 0 || layout.head_v == 0)
        return Status::invalid_argument("GdnStatePoolLayout must be fully specified");
    if (layout.conv_history_stride % 2 != 0)
        return Status::invalid_argument("GDN conv history stride must be even");
    GdnStatePool pool;
    pool.max_slots_ = max_sequences;
    pool.layout_ = layout;
    hipError_t e = hipMalloc(&pool.conv_, (size_t)max_sequences * layout.conv_slot_bytes());
    if (e != hipSuccess) return Status::hip_error("hipMalloc GDN conv state", e);
    e = hipMalloc(&pool.recurrent_, (size_t)max_sequences * layout.recurrent_slot_bytes());
    if (e != hipSuccess) return Status::hip_error("hipMalloc GDN recurrent state", e);
    pool.initialized_.assign(max_sequences, false);
    out = std::move(pool);
    return Status::make_ok();
}

Status GdnStatePool::acquire(SequenceSlotId slot) {
    if (slot >= max_slots_) return Status::out_of_range("slot out of range");
    if (initialized_[slot]) return Status::invalid_state("slot already initialized");
    initialized_[slot] = true;
    ++used_count_;
    return Status::make_ok();
}

Status GdnStatePool::initialize(SequenceSlotId slot, hipStream_t stream) {
    Status st = acquire(slot);
    if (!st.ok()) return st;
    st = reset(slot, stream);
    if (!st.ok()) {
        initialized_[slot] = false;
        --used_count_;
    }
    return st;
}

Status GdnStatePool::reset(SequenceSlotId slot, hipStream_t stream) {
    if (slot >= max_slots_) return Status::out_of_range("slot out of range");
    if (!initialized_[slot]) return Status::invalid_state("slot not initialized");
    hipError_t e = psk::zero_fill(conv_slot(slot), layout_.conv_slot_bytes(), stream);
    if (e == hipSuccess) e = psk::zero_fill(recurrent_slot(slot), layout_.recurrent_slot_bytes(), stream);
    if (e != hipSuccess) return Status::hip_error("GDN slot zero", e);
    return Status::make_ok();
}

Status GdnStatePool::release(SequenceSlotId slot) {
    if (slot >= max_slots_) return Status::out_of_range("slot out of range");
    if (!initialized_[slot]) return Status::invalid_state("slot not initialized");
    initialized_[slot] = false;
    --used_count_;
    return Status::make_ok();
}

Status GdnStatePool::copy_slot_from(SequenceSlotId dst_slot, const GdnStatePool& src,
                                    SequenceSlotId src_slot, hipStream_t stream) {
    if (dst_slot >= max_slots_) return Status::out_of_range("copy_slot_from destination out of range");
    if (src_slot >= src.max_slots_) return Status::out_of_range("copy_slot_from source out of range");
    if (!(layout_ == src.layout_)) return Status::invalid_argument("GDN slot copy layout mismatch");
    const psk::CopySegment segs[2] = {
        {conv_slot(dst_slot), src.conv_slot(src_slot), layout_.conv_slot_bytes()},
        {recurrent_slot(dst_slot), src.recurrent_slot(src_slot), layout_.recurrent_slot_bytes()},
    };
    const hipError_t e = psk::copy_plan_host(nullptr, nullptr, 0, segs, 2, stream);
    if (e != hipSuccess) return Status::hip_error("copy_slot_from", e);
    return Status::make_ok();
}

// ------------------------------------------------------------- PrefixCache
PrefixCache::~PrefixCache() {
    destroy_rings();
    destroy_staging();
}

void PrefixCache::destroy_staging() noexcept {
    if (pairs_ev_) {
        (void)hipEventSynchronize(pairs_ev_);
        (void)hipEventDestroy(pairs_ev_);
    }
    if (pairs_host_) (void)hipHostFree(pairs_host_);
    if (pairs_dev_) (void)hipFree(pairs_dev_);
    pairs_ev_ = nullptr;
    pairs_host_ = nullptr;
    pairs_dev_ = nullptr;
    pairs_cap_ = 0;
    pairs_ev_pending_ = false;
}

Status PrefixCache::launch_copy(const psk_page_copy_args& kv,
                                const std::vector<psk_page_copy_pair>& pairs, const void* segs,
                                uint32_t nseg, hipStream_t stream) {
    const auto* sg = static_cast<const psk::CopySegment*>(segs);
    const uint32_t n = static_cast<uint32_t>(pairs.size());
    psk::CopySegment none{};
    if (n <= psk::kInlinePairs || pairs_cap_ < n) {
        const hipError_t e = psk::copy_plan_host(&kv, pairs.data(), n, nseg ? sg : &none, nseg, stream);
        if (e != hipSuccess) return Status::hip_error("prefix cache copy", e);
        stats_.copy_launches += std::max<uint64_t>(1, (n + psk::kInlinePairs - 1) / psk::kInlinePairs);
        return Status::make_ok();
    }
    if (pairs_ev_pending_) {
        const hipError_t w = hipEventSynchronize(pairs_ev_);
        if (w != hipSuccess) return Status::hip_error("prefix cache staging wait", w);
    }
    std::copy(pairs.begin(), pairs.end(), pairs_host_);
    hipError_t e = psk::copy_plan_host(&kv, pairs_host_, n, sg, nseg, stream, pairs_dev_);
    if (e == hipSuccess) e = hipEventRecord(pairs_ev_, stream);
    if (e != hipSuccess) return Status::hip_error("prefix cache copy", e);
    pairs_ev_pending_ = true;
    ++stats_.copy_launches;
    return Status::make_ok();
}

void PrefixCache::destroy_rings() noexcept {
    for (void* p : k_rings_) (void)hipFree(p);
    for (void* p : v_rings_) (void)hipFree(p);
    k_rings_.clear();
    v_rings_.clear();
    free_ring_slots_.clear();
    ring_bytes_ = 0;
}

Status PrefixCache::create(PrefixCache& out, const PagedKVPool& active_kv,
                           const GdnStatePool& active_gdn, uint32_t capacity_tokens,
                           uint32_t max_entries, uint32_t min_prefix_tokens) {
    if (capacity_tokens == 0) return Status::invalid_argument("prefix cache capacity must be > 0");
    if (max_entries == 0) return Status::invalid_argument("prefix cache max_entries must be > 0");
    if (active_kv.page_tokens() == 0)
        return Status::invalid_argument("prefix cache requires page_tokens > 0");
    const uint32_t cache_pages = pages_for(capacity_tokens, active_kv.page_tokens());
    PagedKVPool kv;
    Status st = PagedKVPool::create(kv, cache_pages, active_kv.page_tokens(),
                                    active_kv.num_attention_layers(), active_kv.kv_heads(),
                                    active_kv.head_dim(), active_kv.dtype());
    if (!st.ok()) return st;
    GdnStatePool gdn;
    st = GdnStatePool::create(gdn, max_entries, active_gdn.layout());
    if (!st.ok()) return st;
    out.clear();
    out.destroy_rings();
    out.destroy_staging();
    // staging for one launch per save / restore (up to every cache page)
    hipError_t e = hipHostMalloc(reinterpret_cast<void**>(&out.pairs_host_),
                                 (size_t)cache_pages * sizeof(psk_page_copy_pair), 0);
    if (e == hipSuccess)
        e = hipMalloc(reinterpret_cast<void**>(&out.pairs_dev_),
                      (size_t)cache_pages * sizeof(psk_page_copy_pair));
    if (e == hipSuccess) e = hipEventCreateWithFlags(&out.pairs_ev_, hipEventDisableTiming);
    if (e != hipSuccess) {
        out.destroy_staging();
        return Status::hip_error("prefix cache staging", e);
    }
    out.pairs_cap_ = cache_pages;
    out.cache_kv_.emplace(std::move(kv));
    out.cache_gdn_.emplace(std::move(gdn));
    out.capacity_tokens_ = capacity_tokens;
    out.max_entries_ = max_entries;
    out.min_prefix_tokens_ = min_prefix_tokens;
    out.entries_.clear();
    out.free_state_slots_.clear();
    for (uint32_t i = 0; i < max_entries; ++i) out.free_state_slots_.push_back(i);
    out.clock_ = 0;
    out.stats_ = PrefixCacheStats{};
    return Status::make_ok();
}

Status PrefixCache::enable_dflash_ring(uint64_t ring_bytes) {
    if (dflash_ring_enabled()) return Status::make_ok();
    if (max_entries_ == 0) return Status::invalid_state("prefix cache has no entries");
    if (ring_bytes == 0) return Status::invalid_argument("dflash ring bytes must be > 0");
    for (uint32_t i = 0; i < max_entries_; ++i) {
        void* k = nullptr;
        void* v = nullptr;
        hipError_t e = hipMalloc(&k, ring_bytes);
        if (e == hipSuccess) {
            e = hipMalloc(&v, ring_bytes);
            if (e != hipSuccess) (void)hipFree(k);
        }
        if (e != hipSuccess) {
            destroy_rings();
            return Status::hip_error("hipMalloc dflash ring", e);
        }
        k_rings_.push_back(k);
        v_rings_.push_back(v);
        free_ring_slots_.push_back(i);
    }
    ring_bytes_ = ring_bytes;
    return Status::make_ok();
}

const PrefixCheckpoint* PrefixCache::find_longest(const std::vector<int32_t>& tokens,
                                                  bool strictly_shorter) {
    if (!enabled()) return nullptr;
    ++stats_.lookups;
    PrefixCheckpoint* best = nullptr;
    size_t best_len = 0;
    for (PrefixCheckpoint& e : entries_) {
        const size_t n = e.tokens.size();
        if (n == 0 || n > tokens.size() || n <= best_len) continue;
        if (strictly_shorter && n >= tokens.size()) continue;
        if (!std::equal(e.tokens.begin(), e.tokens.end(), tokens.begin())) continue;
        best = &e;
        best_len = n;
    }
    if (best == nullptr) {
        ++stats_.misses;
        return nullptr;
    }
    best->last_used = ++clock_;
    ++stats_.hits;
    return best;
}

const PrefixCheckpoint* PrefixCache::find_id(uint64_t id) const {
    for (const PrefixCheckpoint& e : entries_)
        if (e.id == id) return &e;
    return nullptr;
}

void PrefixCache::release_checkpoint(PrefixCheckpoint& entry) noexcept {
    if (cache_kv_ && !entry.cache_pages.empty()) {
        (void)cache_kv_->release_many(entry.cache_pages);
        entry.cache_pages.clear();
    }
    if (cache_gdn_ && entry.cache_state_slot != kInvalidSlot) {
        (void)cache_gdn_->release(entry.cache_state_slot);
        free_state_slots_.push_back(entry.cache_state_slot);
        entry.cache_state_slot = kInvalidSlot;
    }
    if (entry.dflash) {
        free_ring_slots_.push_back(entry.dflash_slot);
        entry.dflash = false;
    }
}

void PrefixCache::evict_lru() {
    if (entries_.empty()) return;
    size_t victim = 0;
    for (size_t i = 1; i < entries_.size(); ++i)
        if (entries_[i].last_used < entries_[victim].last_used) victim = i;
    ++stats_.evictions;
    release_checkpoint(entries_[victim]);
    entries_.erase(entries_.begin() + (std::ptrdiff_t)victim);
}

Status PrefixCache::save(const PagedSequenceState& sequence, const GdnStatePool& gdn_pool,
                         const PagedKVPool& kv_pool, std::vector<int32_t> tokens,
                         hipStream_t stream, bool prompt_boundary,
                         const DFlashContextView* dflash_context) {
    (void)prompt_boundary;   // the reference only traces it
    if (!enabled()) return Status::make_ok();
    if (!sequence.is_usable()) return Status::invalid_state("prefix save: sequence not usable");
    if (sequence.position == 0) return Status::invalid_argument("prefix save: empty sequence");
    if (tokens.size() != sequence.position)
        return Status::invalid_argument("prefix save: token count != sequence position");
    if (tokens.size() < min_prefix_tokens_) return Status::make_ok();
    if (cache_kv_->dtype() != kv_pool.dtype())
        return Status::invalid_state("prefix save: KV dtype mismatch");
    const uint32_t pages = pages_for(sequence.position, cache_kv_->page_tokens());
    if (pages == 0 || pages > sequence.block_table.size())
        return Status::invalid_state("prefix save: block table shorter than position");
    if (pages > cache_kv_->num_pages()) {
        ++stats_.skipped_too_large;
        return Status::make_ok();
    }
    for (PrefixCheckpoint& e : entries_) {
        if (e.tokens == tokens) {
            e.last_used = ++clock_;
            ++stats_.duplicate_hits;
            return Status::make_ok();
        }
    }
    const bool dflash_needed = dflash_context != nullptr && dflash_ring_enabled();
    if (dflash_needed && dflash_context->ring_bytes != ring_bytes_)
        return Status::invalid_argument("prefix save: dflash ring size mismatch");
    auto no_room = [&]() {
        return cache_kv_->num_free_pages() < pages || free_state_slots_.empty() ||
               (dflash_needed && free_ring_slots_.empty());
    };
    while (no_room() && !entries_.empty()) evict_lru();
    if (no_room()) {
        ++stats_.skipped_too_large;
        return Status::make_ok();
    }

    PrefixCheckpoint cp;
    cp.id = next_id_++;
    cp.tokens = std::move(tokens);
    cp.position = sequence.position;
    cp.cache_pages.reserve(pages);
    for (uint32_t p = 0; p < pages; ++p) {
        PageId page;
        const Status st = cache_kv_->allocate(page);
        if (!st.ok()) {
            release_checkpoint(cp);
            return st;
        }
        cp.cache_pages.push_back(page);
    }
    const uint32_t slot = free_state_slots_.back();
    free_state_slots_.pop_back();
    cp.cache_state_slot = slot;
    Status st = cache_gdn_->acquire(slot);
    if (!st.ok()) {
        free_state_slots_.push_back(slot);
        cp.cache_state_slot = kInvalidSlot;
        release_checkpoint(cp);
        return st;
    }
    if (!(cache_gdn_->layout() == gdn_pool.layout()) || sequence.slot >= gdn_pool.max_sequences()) {
        release_checkpoint(cp);
        return Status::invalid_argument("prefix save: GDN pool layout or slot mismatch");
    }

    // one launch: pages, GDN slot, rings
    psk_page_copy_args kv{};
    std::vector<psk_page_copy_pair> pairs;
    st = cache_kv_->copy_pairs_from(cp.cache_pages,
                                    kv_pool,
                                    std::vector<PageId>(sequence.block_table.begin(),
                                                        sequence.block_table.begin() + pages),
                                    kv, pairs);
    if (!st.ok()) {
        release_checkpoint(cp);
        return st;
    }
    psk::CopySegment segs[4];
    uint32_t nseg = 0;
    segs[nseg++] = {cache_gdn_->conv_slot(slot), gdn_pool.conv_slot(sequence.slot),
                    gdn_pool.layout().conv_slot_bytes()};
    segs[nseg++] = {cache_gdn_->recurrent_slot(slot), gdn_pool.recurrent_slot(sequence.slot),
                    gdn_pool.layout().recurrent_slot_bytes()};
    if (dflash_needed) {
        const uint32_t ring = free_ring_slots_.back();
        free_ring_slots_.pop_back();
        cp.dflash = true;
        cp.dflash_slot = ring;
        cp.dflash_length = dflash_context->length;
        cp.dflash_next_position = dflash_context->next_position;
        segs[nseg++] = {k_rings_[ring], dflash_context->k_ring, ring_bytes_};
        segs[nseg++] = {v_rings_[ring], dflash_context->v_ring, ring_bytes_};
    }
    st = launch_copy(kv, pairs, segs, nseg, stream);
    if (!st.ok()) {
        release_checkpoint(cp);
        return st;
    }
    // the reference's accounting (prefix_cache.cpp:340-344): K+V pages of every
    // layer with their scale rows, plus twice the GDN slot
    const uint64_t per_page = (kv_pool.page_body_bytes() + kv_pool.page_scale_bytes()) * 2u *
                              kv_pool.num_attention_layers();
    stats_.save_d2d_bytes += per_page * pages + 2u * gdn_pool.bytes_per_slot();
    stats_.saved_tokens += cp.position;
    ++stats_.inserts;
    cp.last_used = ++clock_;
    entries_.push_back(std::move(cp));
    return Status::make_ok();
}

Status PrefixCache::restore(PagedSequenceState& sequence, GdnStatePool& gdn_pool,
                            PagedKVPool& kv_pool, const PrefixCheckpoint& checkpoint,
                            hipStream_t stream, DFlashContextView* dflash_context) {
    if (!enabled()) return Status::invalid_state("prefix restore: cache disabled");
    if (!sequence.is_usable()) return Status::invalid_state("prefix restore: sequence not usable");
    if (sequence.position != 0 || !sequence.block_table.empty())
        return Status::invalid_state("prefix restore: sequence not empty");
    if (checkpoint.position == 0) return Status::invalid_argument("prefix restore: empty checkpoint");
    if (checkpoint.tokens.size() != checkpoint.position)
        return Status::invalid_argument("prefix restore: checkpoint token count mismatch");
    if (cache_kv_->dtype() != kv_pool.dtype())
        return Status::invalid_state("prefix restore: KV dtype mismatch");
    const uint32_t pages = pages_for(checkpoint.position, cache_kv_->page_tokens());
    if (checkpoint.cache_pages.size() != pages)
        return Status::invalid_argument("prefix restore: checkpoint page count mismatch");
    if (dflash_context != nullptr) {
        if (!checkpoint.dflash)
            return Status::invalid_state("prefix restore: checkpoint has no dflash ring");
        if (checkpoint.dflash_slot >= k_rings_.size())
            return Status::invalid_state("prefix restore: dflash ring slot out of range");
        if (dflash_context->ring_bytes != ring_bytes_)
            return Status::invalid_argument("prefix restore: dflash ring size mismatch");
    }
    if (!(cache_gdn_->layout() == gdn_pool.layout()) || sequence.slot >= gdn_pool.max_sequences())
        return Status::invalid_argument("prefix restore: GDN pool layout or slot mismatch");

    Status st = reserve_sequence_append(sequence, checkpoint.position, stream);
    if (!st.ok()) return st;
    if (sequence.block_table.size() != pages)
        return Status::invalid_state("prefix restore: allocated page count mismatch");

    psk_page_copy_args kv{};
    std::vector<psk_page_copy_pair> pairs;
    st = kv_pool.copy_pairs_from(sequence.block_table, *cache_kv_, checkpoint.cache_pages, kv, pairs);
    if (!st.ok()) return st;
    psk::CopySegment segs[4];
    uint32_t nseg = 0;
    segs[nseg++] = {gdn_pool.conv_slot(sequence.slot),
                    cache_gdn_->conv_slot(checkpoint.cache_state_slot),
                    gdn_pool.layout().conv_slot_bytes()};
    segs[nseg++] = {gdn_pool.recurrent_slot(sequence.slot),
                    cache_gdn_->recurrent_slot(checkpoint.cache_state_slot),
                    gdn_pool.layout().recurrent_slot_bytes()};
    if (dflash_context != nullptr) {
        segs[nseg++] = {dflash_context->k_ring, k_rings_[checkpoint.dflash_slot], ring_bytes_};
        segs[nseg++] = {dflash_context->v_ring, v_rings_[checkpoint.dflash_slot], ring_bytes_};
    }
    st = launch_copy(kv, pairs, segs, nseg, stream);
    if (!st.ok()) return st;
    if (dflash_context != nullptr) {
        dflash_context->length = checkpoint.dflash_length;
        dflash_context->next_position = checkpoint.dflash_next_position;
    }
    st = commit_sequence_append(sequence, checkpoint.position);
    if (!st.ok()) return st;
    const uint64_t per_page = (kv_pool.page_body_bytes() + kv_pool.page_scale_bytes()) * 2u *
                              kv_pool.num_attention_layers();
    stats_.restore_d2d_bytes += per_page * pages + 2u * gdn_pool.bytes_per_slot();
    stats_.restored_tokens += checkpoint.position;
    return Status::make_ok();
}

void PrefixCache::clear() noexcept {
    for (PrefixCheckpoint& e : entries_) release_checkpoint(e);
    entries_.clear();
    free_state_slots_.clear();
    if (cache_gdn_)
        for (uint32_t i = 0; i < cache_gdn_->max_sequences(); ++i) free_state_slots_.push_back(i);
    free_ring_slots_.clear();
    for (uint32_t i = 0; i < k_rings_.size(); ++i) free_ring_slots_.push_back(i);
}

}  // namespace ps::qwen35
