// HIP-graph capture of planned PAGED_ATTENTION steps, keyed by a plan
// signature (reference: paged_attention_dispatch.hip:896-908 computes a plan
// key; executor.hip:990-1075 captures a batch into a graph per row bucket,
// replays it while the key and the batch shape match, and captures only once
// the bucket is warm).
//
// Here the key is the whole launch sequence of the plan: every planned kernel
// (kind, region, splits, pages per split), the tile and combine tables, the
// KV dtype, the 112 argument bytes and the pool, scale and workspace
// pointers. Everything the kernels read at run time (row slots, positions,
// block tables, Q, pools) stays in the same device buffers, so a replay reads
// the step's current contents: the decode kernels derive their work mapping
// from the row positions on the device. The first sighting of a key launches
// eagerly, the second captures (thread-local capture mode) and launches the
// graph, later ones replay. No kernel of the path records a memset node.
#include <phaseshift_kv/dispatch.h>
#include <phaseshift_kv_c.h>

#include <cstring>
#include <list>
#include <new>
#include <vector>

namespace ps::qwen35::runtime {
namespace {

void put(std::vector<uint8_t>& k, const void* p, size_t n) {
    const uint8_t* b = static_cast<const uint8_t*>(p);
    k.insert(k.end(), b, b + n);
}
template <typename T>
void put(std::vector<uint8_t>& k, const T& v) {
    put(k, &v, sizeof(T));
}

}  // namespace

std::vector<uint8_t> plan_signature_bytes(const PagedAttentionStep& step, const PagedAttentionPlan& plan) {
    std::vector<uint8_t> k;
    k.reserve(256 + plan.count * 40 + plan.tiles.size() * 8 + plan.combine.size() * 16);
    put(k, static_cast<uint32_t>(step.kv_dtype));
    put(k, &step.common, sizeof(step.common));
    put(k, step.k_pool);
    put(k, step.v_pool);
    put(k, step.k_scale_pool);
    put(k, step.v_scale_pool);
    put(k, step.partials);
    put(k, plan.count);
    for (uint32_t i = 0; i < plan.count; ++i) {
        const PlannedKernel& p = plan.kernels[i];
        put(k, static_cast<uint32_t>(p.kind));
        put(k, p.row_begin);
        put(k, p.rows);
        put(k, p.splits);
        put(k, p.pages_per_split);
        put(k, p.tile_first);
        put(k, p.tile_count);
        put(k, p.tiles_per_group);
        put(k, p.side);
        put(k, static_cast<uint32_t>(p.partial_offset));
        put(k, static_cast<uint32_t>(p.partial_offset >> 32));
        put(k, p.req_first);
        put(k, p.req_count);
    }
    for (const PlannedTile& t : plan.tiles) {
        put(k, t.row_begin);
        put(k, t.rows);
    }
    for (const StepRequest& r : plan.combine) {
        put(k, r.row_begin);
        put(k, r.row_count);
    }
    return k;
}

uint64_t fnv1a64(const std::vector<uint8_t>& b) {
    uint64_t h = 1469598103934665603ull;
    for (uint8_t c : b) {
        h ^= c;
        h *= 1099511628211ull;
    }
    return h;
}

}  // namespace ps::qwen35::runtime

using namespace ps::qwen35::runtime;

struct psk_step_graph_cache {
    struct Entry {
        std::vector<uint8_t> key;
        hipGraphExec_t exec = nullptr;   // nullptr: seen once, not captured yet
    };
    uint32_t capacity = 8;
    std::list<Entry> lru;                // most recent first
    psk_step_graph_stats_t stats{};
    // Capture records launches without running them, so it happens on a
    // stream of the cache's own (the caller's may be the null stream, which
    // cannot be captured); the graph is then launched on the caller's stream.
    hipStream_t capture_stream = nullptr;

    ~psk_step_graph_cache() {
        for (Entry& e : lru)
            if (e.exec) (void)hipGraphExecDestroy(e.exec);
        if (capture_stream) (void)hipStreamDestroy(capture_stream);
    }
};

namespace {

hipError_t run_graphed(psk_step_graph_cache* c, const PagedAttentionStep& step,
                       const PagedAttentionPlan& plan, hipStream_t stream, uint32_t* how) {
    std::vector<uint8_t> key = plan_signature_bytes(step, plan);
    auto it = c->lru.begin();
    for (; it != c->lru.end(); ++it)
        if (it->key == key) break;
    if (it != c->lru.end() && it->exec != nullptr) {
        c->lru.splice(c->lru.begin(), c->lru, it);
        ++c->stats.replays;
        if (how) *how = 2u;
        return hipGraphLaunch(it->exec, stream);
    }
    if (it == c->lru.end()) {
        // first sighting: eager launch, remember the key
        c->lru.push_front({std::move(key), nullptr});
        while (c->lru.size() > c->capacity) {
            if (c->lru.back().exec) (void)hipGraphExecDestroy(c->lru.back().exec);
            c->lru.pop_back();
            ++c->stats.evictions;
        }
        ++c->stats.eager;
        if (how) *how = 0u;
        return launch_paged_attention_plan(step, plan, stream);
    }
    // second sighting: capture, instantiate, launch
    c->lru.splice(c->lru.begin(), c->lru, it);
    hipError_t e = hipSuccess;
    if (c->capture_stream == nullptr) {
        e = hipStreamCreateWithFlags(&c->capture_stream, hipStreamNonBlocking);
        if (e != hipSuccess) return e;
    }
    e = hipStreamBeginCapture(c->capture_stream, hipStreamCaptureModeThreadLocal);
    if (e != hipSuccess) return e;
    const hipError_t le = launch_paged_attention_plan(step, plan, c->capture_stream);
    hipGraph_t graph = nullptr;
    e = hipStreamEndCapture(c->capture_stream, &graph);
    if (le != hipSuccess || e != hipSuccess || graph == nullptr) {
        if (graph) (void)hipGraphDestroy(graph);
        return le != hipSuccess ? le : (e != hipSuccess ? e : hipErrorUnknown);
    }
    hipGraphExec_t exec = nullptr;
    e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
    (void)hipGraphDestroy(graph);
    if (e != hipSuccess) return e;
    it = c->lru.begin();
    it->exec = exec;
    ++c->stats.captures;
    if (how) *how = 1u;
    return hipGraphLaunch(exec, stream);
}

}  // namespace

extern "C" int psk_step_graph_cache_create(psk_step_graph_cache** out, uint32_t capacity) {
    if (out == nullptr || capacity == 0u) return hipErrorInvalidValue;
    auto* c = new (std::nothrow) psk_step_graph_cache();
    if (c == nullptr) return hipErrorOutOfMemory;
    c->capacity = capacity;
    *out = c;
    return hipSuccess;
}

extern "C" void psk_step_graph_cache_destroy(psk_step_graph_cache* c) { delete c; }

extern "C" int psk_step_graph_cache_stats(const psk_step_graph_cache* c, psk_step_graph_stats_t* out) {
    if (c == nullptr || out == nullptr) return hipErrorInvalidValue;
    *out = c->stats;
    out->entries = static_cast<uint32_t>(c->lru.size());
    uint32_t g = 0;
    for (const auto& e : c->lru) g += e.exec != nullptr;
    out->graphs = g;
    return hipSuccess;
}

// Defined with psk_paged_attention_step (capi_state.cpp): builds the step and
// its plan from the C arguments.
int psk_build_step(const psk_paged_attention_args* common, uint32_t kv_dtype, const void* k_pool,
                   const void* v_pool, const void* k_scale_pool, const void* v_scale_pool,
                   const psk_step_request* requests, uint32_t num_requests,
                   uint32_t max_visible_tokens, float* partials, uint64_t partial_bytes,
                   PagedAttentionStep& step, std::vector<StepRequest>& reqs,
                   PagedAttentionPlan& plan, psk_step_plan_t* plan_out);

extern "C" int psk_paged_attention_step_graphed(
    psk_step_graph_cache* cache, const psk_paged_attention_args* common, uint32_t kv_dtype,
    const void* k_pool, const void* v_pool, const void* k_scale_pool, const void* v_scale_pool,
    const psk_step_request* requests, uint32_t num_requests, uint32_t max_visible_tokens,
    float* partials, uint64_t partial_bytes, psk_step_plan_t* plan_out, void* stream,
    uint32_t* how) {
    if (cache == nullptr) return hipErrorInvalidValue;
    PagedAttentionStep step;
    std::vector<StepRequest> reqs;
    PagedAttentionPlan plan;
    const int rc = psk_build_step(common, kv_dtype, k_pool, v_pool, k_scale_pool, v_scale_pool,
                                  requests, num_requests, max_visible_tokens, partials,
                                  partial_bytes, step, reqs, plan, plan_out);
    if (rc != hipSuccess) return rc;
    return run_graphed(cache, step, plan, static_cast<hipStream_t>(stream), how);
}

extern "C" uint64_t psk_paged_attention_plan_signature(
    const psk_paged_attention_args* common, uint32_t kv_dtype, const void* k_pool,
    const void* v_pool, const void* k_scale_pool, const void* v_scale_pool,
    const psk_step_request* requests, uint32_t num_requests, uint32_t max_visible_tokens,
    float* partials, uint64_t partial_bytes) {
    PagedAttentionStep step;
    std::vector<StepRequest> reqs;
    PagedAttentionPlan plan;
    if (psk_build_step(common, kv_dtype, k_pool, v_pool, k_scale_pool, v_scale_pool, requests,
                       num_requests, max_visible_tokens, partials, partial_bytes, step, reqs, plan,
                       nullptr) != hipSuccess)
        return 0u;
    return fnv1a64(plan_signature_bytes(step, plan));
}
