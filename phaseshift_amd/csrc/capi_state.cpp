// C-ABI over the host KV state and the step planner (opaque handles).
#include <phaseshift_kv/dispatch.h>
#include <phaseshift_kv/kv_state.h>
#include <phaseshift_kv/prefix_cache.h>
#include <phaseshift_kv_c.h>

#include <cstring>
#include <new>
#include <string>

using namespace ps;
using namespace ps::qwen35;

struct psk_kv_pool {
    PagedKVPool pool;
};
struct psk_slot_pool {
    SequenceSlotPool slots;
};
struct psk_sequence {
    PagedSequenceState seq;
};
struct psk_gdn_pool {
    GdnStatePool pool;
};
struct psk_prefix_cache {
    PrefixCache cache;
};

namespace {
thread_local std::string g_last_error;

int to_code(const Status& st) {
    if (st.ok()) return 0;
    g_last_error = st.message;
    switch (st.code) {
        case Status::Code::InvalidArgument: return PSK_ERR_INVALID_ARGUMENT;
        case Status::Code::OutOfRange: return PSK_ERR_OUT_OF_RANGE;
        case Status::Code::InvalidState: return PSK_ERR_INVALID_STATE;
        case Status::Code::InsufficientMemory: return PSK_ERR_INSUFFICIENT_MEMORY;
        default: return PSK_ERR_HIP;
    }
}
hipStream_t S(void* s) { return static_cast<hipStream_t>(s); }
}  // namespace

extern "C" const char* psk_last_error_message(void) { return g_last_error.c_str(); }

extern "C" int psk_pool_create(psk_kv_pool** out, uint32_t num_pages, uint32_t page_tokens,
                               uint32_t num_layers, uint32_t kv_heads, uint32_t head_dim,
                               uint32_t kv_dtype) {
    if (out == nullptr) return PSK_ERR_INVALID_ARGUMENT;
    if (kv_dtype != PSK_KV_BF16 && kv_dtype != PSK_KV_FP8_E4M3 && kv_dtype != PSK_KV_PSQ4_W32 &&
        kv_dtype != PSK_KV_PSQ8_W32) {
        g_last_error = "unknown KV cache dtype";
        return PSK_ERR_INVALID_ARGUMENT;
    }
    auto* h = new (std::nothrow) psk_kv_pool();
    if (h == nullptr) return PSK_ERR_INSUFFICIENT_MEMORY;
    const Status st = PagedKVPool::create(h->pool, num_pages, page_tokens, num_layers, kv_heads,
                                          head_dim, static_cast<KVCacheDType>(kv_dtype));
    if (!st.ok()) {
        delete h;
        return to_code(st);
    }
    *out = h;
    return 0;
}

extern "C" void psk_pool_destroy(psk_kv_pool* p) { delete p; }

extern "C" int psk_pool_info(const psk_kv_pool* p, psk_pool_info_t* out) {
    if (p == nullptr || out == nullptr) return PSK_ERR_INVALID_ARGUMENT;
    const auto& q = p->pool;
    out->k_pool = q.k_pool();
    out->v_pool = q.v_pool();
    out->k_scale_pool = q.k_scale_pool();
    out->v_scale_pool = q.v_scale_pool();
    out->num_pages = q.num_pages();
    out->page_tokens = q.page_tokens();
    out->num_layers = q.num_attention_layers();
    out->kv_heads = q.kv_heads();
    out->head_dim = q.head_dim();
    out->kv_dtype = static_cast<uint32_t>(q.dtype());
    out->free_pages = q.num_free_pages();
    out->used_pages = q.used_count();
    out->reserved_bytes = q.reserved_bytes();
    return 0;
}

extern "C" int psk_pool_allocate(psk_kv_pool* p, uint32_t* page) {
    if (p == nullptr || page == nullptr) return PSK_ERR_INVALID_ARGUMENT;
    return to_code(p->pool.allocate(*page));
}

extern "C" int psk_pool_release(psk_kv_pool* p, uint32_t page) {
    if (p == nullptr) return PSK_ERR_INVALID_ARGUMENT;
    return to_code(p->pool.release(page));
}

extern "C" int psk_pool_copy_pages(psk_kv_pool* dst, const psk_kv_pool* src, const uint32_t* dst_pages,
                                   const uint32_t* src_pages, uint32_t n, void* stream) {
    if (dst == nullptr || src == nullptr || (n > 0 && (dst_pages == nullptr || src_pages == nullptr)))
        return PSK_ERR_INVALID_ARGUMENT;
    return to_code(dst->pool.copy_pages_from(std::vector<PageId>(dst_pages, dst_pages + n), src->pool,
                                             std::vector<PageId>(src_pages, src_pages + n), S(stream)));
}

extern "C" int psk_slot_pool_create(psk_slot_pool** out, uint32_t max_sequences, uint32_t max_blocks,
                                    void* stream) {
    if (out == nullptr) return PSK_ERR_INVALID_ARGUMENT;
    auto* h = new (std::nothrow) psk_slot_pool();
    if (h == nullptr) return PSK_ERR_INSUFFICIENT_MEMORY;
    const Status st = SequenceSlotPool::create(h->slots, max_sequences, max_blocks, S(stream));
    if (!st.ok()) {
        delete h;
        return to_code(st);
    }
    *out = h;
    return 0;
}

extern "C" void psk_slot_pool_destroy(psk_slot_pool* p) { delete p; }

extern "C" uint32_t* psk_slot_pool_block_tables(const psk_slot_pool* p) {
    return p ? p->slots.device_block_tables() : nullptr;
}

extern "C" int psk_sequence_create(psk_sequence** out, psk_slot_pool* slots, psk_kv_pool* pool,
                                   uint32_t max_seq_len, void* stream) {
    if (out == nullptr || slots == nullptr || pool == nullptr) return PSK_ERR_INVALID_ARGUMENT;
    auto* h = new (std::nothrow) psk_sequence();
    if (h == nullptr) return PSK_ERR_INSUFFICIENT_MEMORY;
    const Status st = create_paged_sequence_state(h->seq, slots->slots, pool->pool, max_seq_len, S(stream));
    if (!st.ok()) {
        delete h;
        return to_code(st);
    }
    *out = h;
    return 0;
}

extern "C" int psk_sequence_release(psk_sequence* s, void* stream) {
    if (s == nullptr) return PSK_ERR_INVALID_ARGUMENT;
    const int rc = to_code(release_paged_sequence_state(s->seq, S(stream)));
    delete s;
    return rc;
}

extern "C" int psk_sequence_reserve(psk_sequence* s, uint32_t token_count, void* stream) {
    if (s == nullptr) return PSK_ERR_INVALID_ARGUMENT;
    return to_code(reserve_sequence_append(s->seq, token_count, S(stream)));
}

extern "C" int psk_sequence_rollback(psk_sequence* s, uint32_t old_block_count, void* stream) {
    if (s == nullptr) return PSK_ERR_INVALID_ARGUMENT;
    return to_code(rollback_sequence_append(s->seq, old_block_count, S(stream)));
}

extern "C" int psk_sequence_commit(psk_sequence* s, uint32_t tokens) {
    if (s == nullptr) return PSK_ERR_INVALID_ARGUMENT;
    return to_code(commit_sequence_append(s->seq, tokens));
}

extern "C" int psk_sequence_info(const psk_sequence* s, psk_sequence_info_t* out) {
    if (s == nullptr || out == nullptr) return PSK_ERR_INVALID_ARGUMENT;
    out->slot = s->seq.slot;
    out->generation = s->seq.generation;
    out->position = s->seq.position;
    out->max_seq_len = s->seq.max_seq_len;
    out->num_blocks = static_cast<uint32_t>(s->seq.block_table.size());
    out->poisoned = s->seq.is_poisoned() ? 1u : 0u;
    return 0;
}

extern "C" uint32_t psk_sequence_block_table(const psk_sequence* s, uint32_t* out, uint32_t cap) {
    if (s == nullptr) return 0;
    const uint32_t n = static_cast<uint32_t>(s->seq.block_table.size());
    for (uint32_t i = 0; i < n && i < cap && out; ++i) out[i] = s->seq.block_table[i];
    return n;
}

// The step and its plan from the C arguments (shared with the graphed step,
// step_graph.cpp).
int psk_build_step(const psk_paged_attention_args* common, uint32_t kv_dtype, const void* k_pool,
                   const void* v_pool, const void* k_scale_pool, const void* v_scale_pool,
                   const psk_step_request* requests, uint32_t num_requests,
                   uint32_t max_visible_tokens, float* partials, uint64_t partial_bytes,
                   ps::qwen35::runtime::PagedAttentionStep& step,
                   std::vector<ps::qwen35::runtime::StepRequest>& reqs,
                   ps::qwen35::runtime::PagedAttentionPlan& plan, psk_step_plan_t* plan_out) {
    using namespace ps::qwen35::runtime;
    if (common == nullptr || (num_requests > 0 && requests == nullptr)) return hipErrorInvalidValue;
    std::memcpy(&step.common, common, sizeof(step.common));
    if (kv_dtype != PSK_KV_FP8_E4M3 && kv_dtype != PSK_KV_BF16 && kv_dtype != PSK_KV_PSQ4_W32 &&
        kv_dtype != PSK_KV_PSQ8_W32)
        return hipErrorInvalidValue;
    step.kv_dtype = static_cast<KVCacheDType>(kv_dtype);
    step.k_pool = k_pool;
    step.v_pool = v_pool;
    step.k_scale_pool = k_scale_pool;
    step.v_scale_pool = v_scale_pool;
    reqs.assign(num_requests, StepRequest{});
    for (uint32_t i = 0; i < num_requests; ++i)
        reqs[i] = {requests[i].row_begin, requests[i].row_count, requests[i].execution_class,
                   requests[i].max_visible};
    step.requests = reqs.data();
    step.num_requests = num_requests;
    step.max_visible_tokens = max_visible_tokens;
    step.partials = partials;
    step.partial_bytes = partial_bytes;
    const Status st = plan_paged_attention_step(step, plan);
    if (!st.ok()) {
        g_last_error = st.message;
        return hipErrorInvalidValue;
    }
    if (plan_out) {
        plan_out->count = plan.count;
        for (uint32_t i = 0; i < plan.count && i < PSK_MAX_PLANNED; ++i) {
            plan_out->kernels[i].kind = plan.kernels[i].kind == PlannedKernel::Kind::Tile ? 1u : 0u;
            plan_out->kernels[i].row_begin = plan.kernels[i].row_begin;
            plan_out->kernels[i].rows = plan.kernels[i].rows;
            plan_out->kernels[i].splits = plan.kernels[i].splits;
            plan_out->kernels[i].pages_per_split = plan.kernels[i].pages_per_split;
            plan_out->kernels[i].side = plan.kernels[i].side;
        }
    }
    return hipSuccess;
}

extern "C" int psk_paged_attention_step(const psk_paged_attention_args* common, uint32_t kv_dtype,
                                        const void* k_pool, const void* v_pool,
                                        const void* k_scale_pool, const void* v_scale_pool,
                                        const psk_step_request* requests, uint32_t num_requests,
                                        uint32_t max_visible_tokens, float* partials,
                                        uint64_t partial_bytes, psk_step_plan_t* plan_out,
                                        void* stream) {
    using namespace ps::qwen35::runtime;
    PagedAttentionStep step;
    std::vector<StepRequest> reqs;
    PagedAttentionPlan plan;
    const int rc = psk_build_step(common, kv_dtype, k_pool, v_pool, k_scale_pool, v_scale_pool,
                                  requests, num_requests, max_visible_tokens, partials,
                                  partial_bytes, step, reqs, plan, plan_out);
    if (rc != hipSuccess) return rc;
    if (stream == reinterpret_cast<void*>(~uintptr_t(0))) return hipSuccess;   // plan only
    return launch_paged_attention_plan(step, plan, S(stream));
}

extern "C" int psk_choose_decode_split(const psk_paged_attention_args* a, uint32_t kv_dtype,
                                       const uint32_t* row_visible, uint32_t max_visible_tokens,
                                       uint64_t partial_bytes, uint32_t* splits,
                                       uint32_t* pages_per_split) {
    using namespace ps::qwen35::runtime;
    if (a == nullptr || splits == nullptr || pages_per_split == nullptr || a->kv_heads == 0u ||
        a->q_heads % a->kv_heads != 0u || a->page_tokens == 0u)
        return hipErrorInvalidValue;
    if (kv_dtype != PSK_KV_FP8_E4M3 && kv_dtype != PSK_KV_BF16 && kv_dtype != PSK_KV_PSQ4_W32 &&
        kv_dtype != PSK_KV_PSQ8_W32)
        return hipErrorInvalidValue;
    const DecodeSplit s = choose_decode_split(a->rows, a->kv_heads, a->q_heads, a->head_dim,
                                              kv_dtype, a->page_tokens,
                                              max_visible_tokens, row_visible, partial_bytes);
    *splits = s.splits;
    *pages_per_split = s.pages_per_split;
    return hipSuccess;
}

// ------------------------------------------------------------ GDN pool
static GdnStatePoolLayout from_c(const psk_gdn_layout& l) {
    GdnStatePoolLayout o;
    o.num_gdn_states = l.num_gdn_states;
    o.conv_dim = l.conv_dim;
    o.conv_dim_padded = l.conv_dim_padded;
    o.conv_history = l.conv_history;
    o.conv_history_stride = l.conv_history_stride;
    o.num_v_heads = l.num_v_heads;
    o.head_k = l.head_k;
    o.head_v = l.head_v;
    return o;
}

extern "C" int psk_gdn_layout_make(uint32_t gdn_layers, uint32_t conv_dim, uint32_t conv_history,
                                   uint32_t num_v_heads, uint32_t head_k, uint32_t head_v,
                                   psk_gdn_layout* out) {
    if (out == nullptr) return PSK_ERR_INVALID_ARGUMENT;
    const GdnStatePoolLayout l =
        GdnStatePoolLayout::make(gdn_layers, conv_dim, conv_history, num_v_heads, head_k, head_v);
    *out = {l.num_gdn_states, l.conv_dim,    l.conv_dim_padded, l.conv_history,
            l.conv_history_stride, l.num_v_heads, l.head_k, l.head_v};
    return 0;
}

extern "C" int psk_gdn_pool_create(psk_gdn_pool** out, uint32_t max_sequences,
                                   const psk_gdn_layout* layout) {
    if (out == nullptr || layout == nullptr) return PSK_ERR_INVALID_ARGUMENT;
    auto* h = new (std::nothrow) psk_gdn_pool();
    if (h == nullptr) return PSK_ERR_INSUFFICIENT_MEMORY;
    const Status st = GdnStatePool::create(h->pool, max_sequences, from_c(*layout));
    if (!st.ok()) {
        delete h;
        return to_code(st);
    }
    *out = h;
    return 0;
}

extern "C" void psk_gdn_pool_destroy(psk_gdn_pool* p) { delete p; }

extern "C" int psk_gdn_pool_info(const psk_gdn_pool* p, psk_gdn_pool_info_t* out) {
    if (p == nullptr || out == nullptr) return PSK_ERR_INVALID_ARGUMENT;
    out->conv_base = p->pool.conv_base();
    out->recurrent_base = p->pool.recurrent_base();
    out->conv_slot_bytes = p->pool.layout().conv_slot_bytes();
    out->recurrent_slot_bytes = p->pool.layout().recurrent_slot_bytes();
    out->reserved_bytes = p->pool.reserved_bytes();
    out->max_sequences = p->pool.max_sequences();
    out->used_slots = p->pool.num_used_slots();
    return 0;
}

extern "C" int psk_gdn_pool_initialize(psk_gdn_pool* p, uint32_t slot, void* stream) {
    if (p == nullptr) return PSK_ERR_INVALID_ARGUMENT;
    return to_code(p->pool.initialize(slot, S(stream)));
}

extern "C" int psk_gdn_pool_reset(psk_gdn_pool* p, uint32_t slot, void* stream) {
    if (p == nullptr) return PSK_ERR_INVALID_ARGUMENT;
    return to_code(p->pool.reset(slot, S(stream)));
}

extern "C" int psk_gdn_pool_release(psk_gdn_pool* p, uint32_t slot) {
    if (p == nullptr) return PSK_ERR_INVALID_ARGUMENT;
    return to_code(p->pool.release(slot));
}

extern "C" int psk_gdn_pool_copy_slot(psk_gdn_pool* dst, uint32_t dst_slot, const psk_gdn_pool* src,
                                      uint32_t src_slot, void* stream) {
    if (dst == nullptr || src == nullptr) return PSK_ERR_INVALID_ARGUMENT;
    return to_code(dst->pool.copy_slot_from(dst_slot, src->pool, src_slot, S(stream)));
}

// --------------------------------------------------------- prefix cache
extern "C" int psk_prefix_cache_create(psk_prefix_cache** out, const psk_kv_pool* active_kv,
                                       const psk_gdn_pool* active_gdn, uint32_t capacity_tokens,
                                       uint32_t max_entries, uint32_t min_prefix_tokens) {
    if (out == nullptr || active_kv == nullptr || active_gdn == nullptr)
        return PSK_ERR_INVALID_ARGUMENT;
    auto* h = new (std::nothrow) psk_prefix_cache();
    if (h == nullptr) return PSK_ERR_INSUFFICIENT_MEMORY;
    const Status st = PrefixCache::create(h->cache, active_kv->pool, active_gdn->pool,
                                          capacity_tokens, max_entries, min_prefix_tokens);
    if (!st.ok()) {
        delete h;
        return to_code(st);
    }
    *out = h;
    return 0;
}

extern "C" void psk_prefix_cache_destroy(psk_prefix_cache* c) { delete c; }

extern "C" int psk_prefix_cache_enable_dflash_ring(psk_prefix_cache* c, uint64_t ring_bytes) {
    if (c == nullptr) return PSK_ERR_INVALID_ARGUMENT;
    return to_code(c->cache.enable_dflash_ring(ring_bytes));
}

static void info_of(const PrefixCheckpoint* cp, psk_prefix_checkpoint_info* out) {
    *out = psk_prefix_checkpoint_info{};
    if (cp == nullptr) return;
    out->id = cp->id;
    out->last_used = cp->last_used;
    out->position = cp->position;
    out->num_pages = static_cast<uint32_t>(cp->cache_pages.size());
    out->cache_state_slot = cp->cache_state_slot;
    out->dflash = cp->dflash ? 1u : 0u;
}

extern "C" int psk_prefix_cache_find_longest(psk_prefix_cache* c, const int32_t* tokens, uint32_t n,
                                             uint32_t strictly_shorter,
                                             psk_prefix_checkpoint_info* out) {
    if (c == nullptr || out == nullptr || (n > 0 && tokens == nullptr)) return PSK_ERR_INVALID_ARGUMENT;
    info_of(c->cache.find_longest(std::vector<int32_t>(tokens, tokens + n), strictly_shorter != 0u),
            out);
    return 0;
}

static DFlashContextView view_of(const psk_dflash_context& d) {
    DFlashContextView v;
    v.k_ring = d.k_ring;
    v.v_ring = d.v_ring;
    v.ring_bytes = d.ring_bytes;
    v.length = d.length;
    v.next_position = d.next_position;
    return v;
}

extern "C" int psk_prefix_cache_save(psk_prefix_cache* c, const psk_sequence* seq,
                                     const psk_gdn_pool* gdn, const psk_kv_pool* kv,
                                     const int32_t* tokens, uint32_t n, uint32_t prompt_boundary,
                                     const psk_dflash_context* dflash, void* stream) {
    if (c == nullptr || seq == nullptr || gdn == nullptr || kv == nullptr ||
        (n > 0 && tokens == nullptr))
        return PSK_ERR_INVALID_ARGUMENT;
    DFlashContextView v;
    if (dflash != nullptr) v = view_of(*dflash);
    return to_code(c->cache.save(seq->seq, gdn->pool, kv->pool, std::vector<int32_t>(tokens, tokens + n),
                                 S(stream), prompt_boundary != 0u, dflash ? &v : nullptr));
}

extern "C" int psk_prefix_cache_restore(psk_prefix_cache* c, psk_sequence* seq, psk_gdn_pool* gdn,
                                        psk_kv_pool* kv, uint64_t checkpoint_id,
                                        psk_dflash_context* dflash, void* stream) {
    if (c == nullptr || seq == nullptr || gdn == nullptr || kv == nullptr)
        return PSK_ERR_INVALID_ARGUMENT;
    const PrefixCheckpoint* cp = c->cache.find_id(checkpoint_id);
    if (cp == nullptr) {
        g_last_error = "prefix restore: no checkpoint with this id";
        return PSK_ERR_INVALID_ARGUMENT;
    }
    DFlashContextView v;
    if (dflash != nullptr) v = view_of(*dflash);
    const int rc = to_code(c->cache.restore(seq->seq, gdn->pool, kv->pool, *cp, S(stream),
                                            dflash ? &v : nullptr));
    if (rc == 0 && dflash != nullptr) {
        dflash->length = v.length;
        dflash->next_position = v.next_position;
    }
    return rc;
}

extern "C" int psk_prefix_cache_clear(psk_prefix_cache* c) {
    if (c == nullptr) return PSK_ERR_INVALID_ARGUMENT;
    c->cache.clear();
    return 0;
}

extern "C" int psk_prefix_cache_stats(const psk_prefix_cache* c, psk_prefix_cache_stats_t* out) {
    if (c == nullptr || out == nullptr) return PSK_ERR_INVALID_ARGUMENT;
    const PrefixCacheStats& s = c->cache.stats();
    *out = psk_prefix_cache_stats_t{};
    out->lookups = s.lookups;
    out->hits = s.hits;
    out->misses = s.misses;
    out->inserts = s.inserts;
    out->duplicate_hits = s.duplicate_hits;
    out->evictions = s.evictions;
    out->skipped_too_large = s.skipped_too_large;
    out->restored_tokens = s.restored_tokens;
    out->saved_tokens = s.saved_tokens;
    out->save_d2d_bytes = s.save_d2d_bytes;
    out->restore_d2d_bytes = s.restore_d2d_bytes;
    out->copy_launches = s.copy_launches;
    out->cache_kv_bytes = c->cache.cache_kv_bytes();
    out->cache_gdn_bytes = c->cache.cache_gdn_bytes();
    out->dflash_ring_bytes = c->cache.dflash_ring_bytes();
    out->size = static_cast<uint32_t>(c->cache.size());
    out->cache_pages = c->cache.cache_pages();
    out->cache_free_pages = c->cache.cache_free_pages();
    out->cache_free_slots = c->cache.cache_free_slots();
    out->max_entries = c->cache.max_entries();
    out->capacity_tokens = c->cache.capacity_tokens();
    return 0;
}
