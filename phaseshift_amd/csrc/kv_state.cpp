// Host-side KV state: pool + free list, device block tables, per-sequence
// paging (reserve / rollback / commit) and page copy. Behaviour restated from
// the reference (file:line in the reference repository):
//   PagedKVPool::create / allocate / release / release_many   state/paged_kv_pool.cpp:27-244
//   PagedKVPool::copy_page_from                               state/paged_kv_pool.cpp:338-542
//   SequenceSlotPool::clear_blocks / clear_slot               state/sequence_slot_pool.cpp:192-238
//   reserve / rollback / commit_sequence_append               state/paged_sequence_state.cpp:111-271
#include <phaseshift_kv/kv_state.h>
#include <phaseshift_kv_c.h>

#include "page_ops.h"

#include <algorithm>
#include <utility>

namespace ps::qwen35 {

namespace {
Status alloc256(void** p, size_t bytes, const char* what) {
    // hipMalloc returns allocations aligned to at least 256 B.
    const hipError_t e = hipMalloc(p, bytes == 0 ? 256 : bytes);
    if (e != hipSuccess) return Status::hip_error(what, e);
    return Status::make_ok();
}
}  // namespace

PagedKVPool::~PagedKVPool() { destroy(); }

void PagedKVPool::destroy() noexcept {
    for (void* p : {k_, v_, static_cast<void*>(k_scale_), static_cast<void*>(v_scale_)})
        if (p) (void)hipFree(p);
    k_ = v_ = nullptr;
    k_scale_ = v_scale_ = nullptr;
}

PagedKVPool::PagedKVPool(PagedKVPool&& o) noexcept { *this = std::move(o); }

PagedKVPool& PagedKVPool::operator=(PagedKVPool&& o) noexcept {
    if (this != &o) {
        destroy();
        num_pages_ = o.num_pages_;
        page_tokens_ = o.page_tokens_;
        num_attention_layers_ = o.num_attention_layers_;
        kv_heads_ = o.kv_heads_;
        head_dim_ = o.head_dim_;
        dtype_ = o.dtype_;
        k_ = std::exchange(o.k_, nullptr);
        v_ = std::exchange(o.v_, nullptr);
        k_scale_ = std::exchange(o.k_scale_, nullptr);
        v_scale_ = std::exchange(o.v_scale_, nullptr);
        reserved_bytes_ = o.reserved_bytes_;
        free_list_ = std::move(o.free_list_);
        in_use_ = std::move(o.in_use_);
        used_count_ = o.used_count_;
    }
    return *this;
}

Status PagedKVPool::create(PagedKVPool& out, uint32_t num_pages, uint32_t page_tokens,
                           uint32_t num_attention_layers, uint32_t kv_heads, uint32_t head_dim,
                           KVCacheDType dtype) {
    if (num_pages == 0) return Status::invalid_argument("num_pages must be > 0");
    if (page_tokens == 0) return Status::invalid_argument("page_tokens must be > 0");
    if (num_attention_layers == 0) return Status::invalid_argument("num_attention_layers must be > 0");
    if (kv_heads == 0) return Status::invalid_argument("kv_heads must be > 0");
    if (head_dim == 0) return Status::invalid_argument("head_dim must be > 0");
    const bool psq = dtype == KVCacheDType::PSQ4_W32 || dtype == KVCacheDType::PSQ8_W32;
    if (dtype != KVCacheDType::BF16 && dtype != KVCacheDType::FP8_E4M3 && !psq)
        return Status::invalid_argument("unknown KV cache dtype");
    // PSQ: blocks of 32 values (kv_cache_types.h:16-46)
    if (psq && head_dim % 32u != 0u)
        return Status::invalid_argument("PSQ KV needs head_dim divisible by 32");
    PagedKVPool pool;
    pool.num_pages_ = num_pages;
    pool.page_tokens_ = page_tokens;
    pool.num_attention_layers_ = num_attention_layers;
    pool.kv_heads_ = kv_heads;
    pool.head_dim_ = head_dim;
    pool.dtype_ = dtype;
    const uint64_t elems = (uint64_t)num_attention_layers * num_pages * page_tokens * kv_heads * head_dim;
    // The launcher structs carry elems_per_layer as uint32 (kv_append.h:40).
    if ((uint64_t)num_pages * page_tokens * kv_heads * head_dim > 0xFFFFFFFFull)
        return Status::invalid_argument("pool layer exceeds 2^32 elements");
    const uint64_t slices = (uint64_t)num_attention_layers * num_pages * page_tokens * kv_heads;
    // body bytes (bf16 values, E4M3 codes, PSQ4 nibbles) and scale bytes
    // (FP8: f32 per slice; PSQ: bf16 per 32-value block)
    const uint64_t body = dtype == KVCacheDType::BF16             ? elems * 2
                          : dtype == KVCacheDType::PSQ4_W32       ? elems / 2
                                                                  : elems;
    const uint64_t scale_bytes = dtype == KVCacheDType::FP8_E4M3 ? slices * 4
                                 : psq                           ? elems / 32 * 2
                                                                 : 0;
    Status st = alloc256(&pool.k_, body, "hipMalloc K pool");
    if (!st.ok()) return st;
    st = alloc256(&pool.v_, body, "hipMalloc V pool");
    if (!st.ok()) return st;
    pool.reserved_bytes_ = 2 * body;
    if (scale_bytes != 0) {
        st = alloc256(reinterpret_cast<void**>(&pool.k_scale_), scale_bytes, "hipMalloc K scales");
        if (!st.ok()) return st;
        st = alloc256(reinterpret_cast<void**>(&pool.v_scale_), scale_bytes, "hipMalloc V scales");
        if (!st.ok()) return st;
        pool.reserved_bytes_ += 2 * scale_bytes;
    }
    pool.in_use_.assign(num_pages, false);
    pool.free_list_.reserve(num_pages);
    for (uint32_t i = 0; i < num_pages; ++i) pool.free_list_.push_back(i);
    out = std::move(pool);
    return Status::make_ok();
}

uint64_t PagedKVPool::page_body_bytes() const noexcept {
    const uint64_t e = (uint64_t)page_tokens_ * kv_heads_ * head_dim_;
    switch (dtype_) {
        case KVCacheDType::BF16: return e * 2;
        case KVCacheDType::PSQ4_W32: return e / 2;
        default: return e;
    }
}

uint64_t PagedKVPool::page_scale_bytes() const noexcept {
    const uint64_t th = (uint64_t)page_tokens_ * kv_heads_;
    switch (dtype_) {
        case KVCacheDType::FP8_E4M3: return th * 4;
        case KVCacheDType::PSQ4_W32:
        case KVCacheDType::PSQ8_W32: return th * (head_dim_ / 32) * 2;
        default: return 0;
    }
}

Status PagedKVPool::allocate(PageId& page) {
    if (free_list_.empty()) return Status::insufficient_memory("KV page pool exhausted");
    page = free_list_.back();
    free_list_.pop_back();
    in_use_[page] = true;
    ++used_count_;
    return Status::make_ok();
}

Status PagedKVPool::release(PageId page) {
    if (page >= num_pages_) return Status::invalid_argument("page id out of range");
    if (!in_use_[page]) return Status::invalid_argument("page not in use");
    in_use_[page] = false;
    free_list_.push_back(page);
    --used_count_;
    return Status::make_ok();
}

Status PagedKVPool::release_many(const std::vector<PageId>& pages) {
    // validate everything first (paged_kv_pool.cpp:218-244): nothing is freed
    // unless every id is valid, in use and distinct
    std::vector<PageId> sorted(pages);
    std::sort(sorted.begin(), sorted.end());
    for (size_t i = 0; i < sorted.size(); ++i) {
        const PageId p = sorted[i];
        if (p == kInvalidPageId) return Status::invalid_argument("invalid page id");
        if (p >= num_pages_) return Status::invalid_argument("page id out of range");
        if (!in_use_[p]) return Status::invalid_argument("page not in use");
        if (i > 0 && sorted[i - 1] == p) return Status::invalid_argument("duplicate page id");
    }
    for (PageId p : pages) {
        in_use_[p] = false;
        free_list_.push_back(p);
        --used_count_;
    }
    return Status::make_ok();
}

Status PagedKVPool::copy_page_from(PageId dst_page, const PagedKVPool& src, PageId src_page,
                                   hipStream_t stream) {
    return copy_pages_from({dst_page}, src, {src_page}, stream);
}

Status PagedKVPool::copy_pairs_from(const std::vector<PageId>& dst_pages, const PagedKVPool& src,
                                    const std::vector<PageId>& src_pages, psk_page_copy_args& a,
                                    std::vector<psk_page_copy_pair>& pairs) const {
    if (dtype_ != src.dtype_) return Status::invalid_argument("KV page copy dtype mismatch");
    if (page_tokens_ != src.page_tokens_ || num_attention_layers_ != src.num_attention_layers_ ||
        kv_heads_ != src.kv_heads_ || head_dim_ != src.head_dim_)
        return Status::invalid_argument("KV page copy layout mismatch");
    if (dst_pages.size() != src_pages.size())
        return Status::invalid_argument("KV page copy list sizes differ");
    pairs.resize(dst_pages.size());
    for (size_t i = 0; i < dst_pages.size(); ++i) {
        if (dst_pages[i] >= num_pages_)
            return Status::invalid_argument("KV page copy destination out of range");
        if (src_pages[i] >= src.num_pages_)
            return Status::invalid_argument("KV page copy source out of range");
        pairs[i] = {dst_pages[i], src_pages[i]};
    }
    a = psk_page_copy_args{};
    a.dst_k = k_;
    a.dst_v = v_;
    a.dst_k_scale = k_scale_;
    a.dst_v_scale = v_scale_;
    a.src_k = src.k_;
    a.src_v = src.v_;
    a.src_k_scale = src.k_scale_;
    a.src_v_scale = src.v_scale_;
    a.num_layers = num_attention_layers_;
    a.dst_num_pages = num_pages_;
    a.src_num_pages = src.num_pages_;
    a.page_tokens = page_tokens_;
    a.kv_heads = kv_heads_;
    a.head_dim = head_dim_;
    a.kv_dtype = static_cast<uint32_t>(dtype_);
    return Status::make_ok();
}

Status PagedKVPool::copy_pages_from(const std::vector<PageId>& dst_pages, const PagedKVPool& src,
                                    const std::vector<PageId>& src_pages, hipStream_t stream) {
    psk_page_copy_args a{};
    std::vector<psk_page_copy_pair> pairs;
    Status st = copy_pairs_from(dst_pages, src, src_pages, a, pairs);
    if (!st.ok() || pairs.empty()) return st;
    const hipError_t e =
        psk::copy_pages_host_pairs(a, pairs.data(), static_cast<uint32_t>(pairs.size()), stream);
    if (e != hipSuccess) return Status::hip_error("copy_page_from", e);
    return Status::make_ok();
}

// ------------------------------------------------------------ slot pool
SequenceSlotPool::~SequenceSlotPool() {
    if (tables_) (void)hipFree(tables_);
}

Status SequenceSlotPool::create(SequenceSlotPool& out, uint32_t max_sequences, uint32_t max_blocks,
                                hipStream_t stream) {
    if (max_sequences == 0 || max_blocks == 0)
        return Status::invalid_argument("max_sequences and max_blocks must be > 0");
    if (out.tables_) {
        (void)hipFree(out.tables_);
        out.tables_ = nullptr;
    }
    void* p = nullptr;
    Status st = alloc256(&p, (size_t)max_sequences * max_blocks * 4, "hipMalloc block tables");
    if (!st.ok()) return st;
    out.tables_ = static_cast<uint32_t*>(p);
    out.max_sequences_ = max_sequences;
    out.max_blocks_ = max_blocks;
    out.in_use_.assign(max_sequences, false);
    out.free_slots_.clear();
    for (uint32_t s = max_sequences; s-- > 0;) out.free_slots_.push_back(s);
    const int e = psk_fill_u32(out.tables_, kInvalidPageId, (uint64_t)max_sequences * max_blocks, stream);
    if (e != hipSuccess) return Status::hip_error("clear block tables", static_cast<hipError_t>(e));
    return Status::make_ok();
}

Status SequenceSlotPool::allocate(SequenceSlotId& slot) {
    if (free_slots_.empty()) return Status::insufficient_memory("no free sequence slot");
    slot = free_slots_.back();
    free_slots_.pop_back();
    in_use_[slot] = true;
    return Status::make_ok();
}

Status SequenceSlotPool::release(SequenceSlotId slot, hipStream_t stream) {
    if (slot >= max_sequences_) return Status::out_of_range("slot out of range");
    if (!in_use_[slot]) return Status::invalid_state("slot not allocated");
    Status st = clear_slot(slot, stream);
    in_use_[slot] = false;
    free_slots_.push_back(slot);
    return st;
}

Status SequenceSlotPool::set_blocks(SequenceSlotId slot, uint32_t first_block, const PageId* pages,
                                    uint32_t count, hipStream_t stream) {
    if (slot >= max_sequences_) return Status::out_of_range("slot out of range");
    if (!in_use_[slot]) return Status::invalid_state("slot not allocated");
    if (first_block >= max_blocks_ || count > max_blocks_ - first_block)
        return Status::out_of_range("block range out of range");
    if (count == 0) return Status::make_ok();
    const hipError_t e =
        hipMemcpyAsync(tables_ + (size_t)slot * max_blocks_ + first_block, pages,
                       (size_t)count * sizeof(PageId), hipMemcpyHostToDevice, stream);
    if (e != hipSuccess) return Status::hip_error("hipMemcpyAsync set_blocks", e);
    return Status::make_ok();
}

Status SequenceSlotPool::clear_blocks(SequenceSlotId slot, uint32_t first_block, uint32_t block_count,
                                      hipStream_t stream) {
    if (slot >= max_sequences_) return Status::out_of_range("slot out of range");
    if (!in_use_[slot]) return Status::invalid_state("slot not allocated");
    if (first_block >= max_blocks_) return Status::out_of_range("first_block out of range");
    if (block_count > max_blocks_ - first_block) return Status::out_of_range("block_count out of range");
    if (block_count == 0) return Status::make_ok();
    const int e = psk_fill_u32(tables_ + (size_t)slot * max_blocks_ + first_block, kInvalidPageId,
                               block_count, stream);
    if (e != hipSuccess) return Status::hip_error("clear_blocks", static_cast<hipError_t>(e));
    return Status::make_ok();
}

Status SequenceSlotPool::clear_slot(SequenceSlotId slot, hipStream_t stream) {
    return clear_blocks(slot, 0, max_blocks_, stream);
}

// ------------------------------------------------------ sequence state
Status create_paged_sequence_state(PagedSequenceState& out, SequenceSlotPool& seq_pool,
                                   PagedKVPool& kv_pool, uint32_t max_seq_len, hipStream_t stream) {
    if (max_seq_len == 0) return Status::invalid_argument("max_seq_len must be > 0");
    const uint32_t blocks = (max_seq_len + kv_pool.page_tokens() - 1) / kv_pool.page_tokens();
    if (blocks > seq_pool.max_blocks())
        return Status::out_of_range("max_seq_len exceeds the block-table stride");
    SequenceSlotId slot = kInvalidSlot;
    Status st = seq_pool.allocate(slot);
    if (!st.ok()) return st;
    st = seq_pool.clear_slot(slot, stream);
    if (!st.ok()) return st;
    static uint32_t generation_counter = 0;
    out = PagedSequenceState{};
    out.slot = slot;
    out.generation = ++generation_counter == 0 ? ++generation_counter : generation_counter;
    out.max_seq_len = max_seq_len;
    out.kv_pool = &kv_pool;
    out.seq_pool = &seq_pool;
    out.max_blocks = blocks;
    return Status::make_ok();
}

Status release_paged_sequence_state(PagedSequenceState& seq, hipStream_t stream) {
    if (!seq.is_allocated()) return Status::invalid_argument("sequence state is not allocated");
    Status first = Status::make_ok();
    if (!seq.block_table.empty()) first = seq.kv_pool->release_many(seq.block_table);
    Status st = seq.seq_pool->release(seq.slot, stream);
    if (first.ok() && !st.ok()) first = st;
    seq = PagedSequenceState{};
    return first;
}

Status reserve_sequence_append(PagedSequenceState& seq, uint32_t token_count, hipStream_t stream) {
    if (!seq.is_usable()) return Status::invalid_argument("sequence state is not usable");
    if (token_count == 0) return Status::make_ok();
    if (token_count > seq.max_seq_len - seq.position)
        return Status::out_of_range("token_count exceeds max_seq_len");
    const uint32_t P = seq.kv_pool->page_tokens();
    const uint32_t end_position = seq.position + token_count;
    const uint32_t required = (end_position + P - 1) / P;
    const size_t current = seq.block_table.size();
    if (required <= current) return Status::make_ok();
    const uint32_t new_blocks = required - static_cast<uint32_t>(current);
    if (required > seq.max_blocks) return Status::out_of_range("required_blocks exceeds max_blocks_per_sequence");
    if (new_blocks > seq.kv_pool->num_free_pages())
        return Status::insufficient_memory("not enough free pages for chunk");
    for (uint32_t i = 0; i < new_blocks; ++i) {
        PageId page = kInvalidPageId;
        Status st = seq.kv_pool->allocate(page);
        if (!st.ok()) {
            for (size_t j = current; j < seq.block_table.size(); ++j) (void)seq.kv_pool->release(seq.block_table[j]);
            seq.block_table.resize(current);
            return st;
        }
        seq.block_table.push_back(page);
    }
    Status st = seq.seq_pool->set_blocks(seq.slot, static_cast<uint32_t>(current),
                                         seq.block_table.data() + current, new_blocks, stream);
    if (!st.ok()) {
        for (size_t j = current; j < seq.block_table.size(); ++j) (void)seq.kv_pool->release(seq.block_table[j]);
        seq.block_table.resize(current);
        return st;
    }
    return Status::make_ok();
}

Status rollback_sequence_append(PagedSequenceState& seq, uint32_t old_block_count, hipStream_t stream) {
    if (!seq.is_allocated()) return Status::invalid_argument("sequence state is not allocated");
    if (seq.seq_pool == nullptr || seq.kv_pool == nullptr)
        return Status::invalid_state("sequence pool ownership is invalid");
    if (old_block_count > seq.block_table.size())
        return Status::out_of_range("old_block_count exceeds block_table");
    if (old_block_count == seq.block_table.size()) return Status::make_ok();
    const uint32_t n = static_cast<uint32_t>(seq.block_table.size());
    Status first = seq.seq_pool->clear_blocks(seq.slot, old_block_count, n - old_block_count, stream);
    for (size_t i = old_block_count; i < seq.block_table.size(); ++i) {
        Status st = seq.kv_pool->release(seq.block_table[i]);
        if (!st.ok() && first.ok()) first = st;
    }
    seq.block_table.resize(old_block_count);
    if (!first.ok()) {
        seq.mark_poisoned();
        return first;
    }
    return Status::make_ok();
}

Status commit_sequence_append(PagedSequenceState& seq, uint32_t committed_tokens) {
    if (!seq.is_usable()) return Status::invalid_state("sequence state is not usable");
    if (committed_tokens == 0u) return Status::invalid_argument("committed_tokens must be > 0");
    if (committed_tokens > seq.max_seq_len - seq.position)
        return Status::out_of_range("sequence commit exceeds max_seq_len");
    seq.position += committed_tokens;
    return Status::make_ok();
}

}  // namespace ps::qwen35
