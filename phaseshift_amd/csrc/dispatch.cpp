// resolve -> plan -> launch for one PAGED_ATTENTION binding of a step.
//
// Reference planner: runtime/paged_attention_dispatch.hip:437-477 (split rule),
// :705-788 (regions), :790-894 (physical launch). Regions follow the
// reference: the decode region is every row before the first PREFILL request
// (decode and SPEC_VERIFY rows alike); each PREFILL request is its own region,
// run by the multi-row tile launcher when it has >= 128 rows
// (paged_attention_dispatch.h:49). New here: FP8 KV also gets split-K, and the
// split size is chosen from the step's work instead of a fixed 16.
#include <phaseshift_kv/dispatch.h>

#include <algorithm>
#include <map>
#include <mutex>
#include <queue>
#include <functional>
#include <vector>

namespace psk {
size_t decode_workgroup_lds_bytes(uint32_t kv_dtype, uint32_t head_dim);
uint32_t tile_workgroups_per_cu(uint32_t kv_dtype, uint32_t head_dim, uint32_t q_per_kv, bool grouped);
hipError_t launch_paged_tiles(const psk_paged_attention_args& a, uint32_t kv_dtype, const void* k,
                              const void* v, const void* ks, const void* vs,
                              const uint32_t* tile_begin, const uint32_t* tile_rows,
                              uint32_t n_tiles, uint32_t tiles_per_group, float* partials,
                              uint32_t splits, uint32_t pages_per_split, hipStream_t stream);
uint32_t tile_group_size(uint32_t q_per_kv, uint32_t kv_dtype);
uint32_t tile_dense_units_limit();
uint64_t tile_launch_workgroups(uint64_t n_tiles, uint32_t tiles_per_group, uint32_t q_per_kv,
                                uint32_t kv_heads);
bool paged_tiles_supported(const psk_paged_attention_args& a, uint32_t kv_dtype, const void* k,
                           const void* v, const void* ks, const void* vs);
}  // namespace psk

namespace ps::qwen35::runtime {

using ::ps::kernel::PagedAttentionCommonArgs;
using ::ps::kernel::PagedAttentionOutputDType;

namespace {

PagedAttentionCommonArgs region_args(const PagedAttentionCommonArgs& c, uint32_t row_begin,
                                     uint32_t rows) {
    PagedAttentionCommonArgs r = c;
    const size_t out_elem = c.output_dtype == PagedAttentionOutputDType::F32 ? 4 : 2;
    r.q = c.q + (size_t)row_begin * c.q_row_stride;
    r.output = static_cast<uint8_t*>(c.output) + (size_t)row_begin * c.output_row_stride * out_elem;
    r.row_sequence_slots = c.row_sequence_slots + row_begin;
    r.row_positions = c.row_positions + row_begin;
    r.rows = rows;
    return r;
}

}  // namespace

namespace {

// MI355X geometry the chooser models: workgroups are dealt round-robin to 8
// XCDs (block b runs on XCD b mod 8), each with multiProcessorCount/8 CUs.
constexpr uint32_t kXcds = 8;

uint32_t device_cus() {
    static const uint32_t cus = [] {
        int dev = 0;
        hipDeviceProp_t prop{};
        if (hipGetDevice(&dev) != hipSuccess || hipGetDeviceProperties(&prop, dev) != hipSuccess ||
            prop.multiProcessorCount <= 0) {
            (void)hipGetLastError();
            return 256u;   // MI355X
        }
        return static_cast<uint32_t>(prop.multiProcessorCount);
    }();
    return cus;
}

// Makespan (seconds) of the decode kernel's units (dense, longest first, unit
// u on XCD u mod 8, given in bytes) under greedy dispatch onto `slots`
// workgroup slots per XCD. Fluid model fitted on MI355X (FP8 hd256, 18 split
// sizes of two workloads, 2.5% rms): each XCD streams at most `xcd_bw` B/s,
// shared evenly by its streaming workgroups; one workgroup streams at most
// `wg_bw` (1.5x its fair share, so a tail runs faster than the bulk); every
// unit first spends `c0` seconds of start-up (unit scan, block-table window,
// first-chunk latency, epilogue) without streaming. The XCDs are independent.
double split_makespan(const std::vector<double>& units, uint32_t slots, double xcd_bw,
                      double wg_bw, double c0) {
    double worst = 0.0;
    using Q = std::priority_queue<std::pair<double, double>, std::vector<std::pair<double, double>>,
                                  std::greater<std::pair<double, double>>>;
    for (uint32_t x = 0; x < kXcds; ++x) {
        // start-ups: (end time, bytes); streams: virtual progress at which
        // they end (every streaming unit receives the same rate)
        Q delays;
        std::priority_queue<double, std::vector<double>, std::greater<double>> streams;
        double t = 0.0, vp = 0.0;
        size_t next = x;
        auto fill = [&] {
            while (delays.size() + streams.size() < slots && next < units.size()) {
                delays.push({t + c0, units[next]});
                next += kXcds;
            }
        };
        fill();
        while (!delays.empty() || !streams.empty()) {
            const double rate =
                streams.empty() ? 0.0 : std::min(wg_bw, xcd_bw / (double)streams.size());
            const double ts = streams.empty() ? 1e30 : t + (streams.top() - vp) / rate;
            const double td = delays.empty() ? 1e30 : delays.top().first;
            if (td <= ts) {
                vp += (td - t) * rate;
                t = td;
                streams.push(vp + delays.top().second);
                delays.pop();
            } else {
                vp = streams.top();
                t = ts;
                streams.pop();
                fill();
            }
        }
        worst = std::max(worst, t);
    }
    return worst;
}

}  // namespace

DecodeSplit choose_decode_split(uint32_t rows, uint32_t kv_heads, uint32_t q_heads,
                                uint32_t head_dim, uint32_t kv_dtype, uint32_t page_tokens,
                                uint32_t max_visible_tokens, const uint32_t* row_visible,
                                uint64_t partial_bytes) {
    DecodeSplit best;
    if (max_visible_tokens < kSplitMinVisible || rows == 0 || kv_heads == 0 || page_tokens == 0)
        return best;
    const uint32_t max_pages = (max_visible_tokens + page_tokens - 1) / page_tokens;
    std::vector<uint32_t> pages(rows, max_pages);
    if (row_visible != nullptr)
        for (uint32_t r = 0; r < rows; ++r)
            pages[r] = std::min(max_pages, (row_visible[r] + page_tokens - 1) / page_tokens);
    const uint32_t q_per_kv = q_heads / kv_heads;
    // Plan reuse across decode steps. Consecutive steps of one batch differ by
    // one token per row, so a row's page count moves by one page every
    // page_tokens steps and the simulation below (about 1 ms for 64 long
    // rows) would run on most steps. The last few choices of this thread are
    // kept with the page counts they were computed for, and one is reused
    // while (1) every input but the page counts is the same, (2) the plan
    // stays valid: no row needs more than its split count, (3) the number of
    // units (row splits) is unchanged, so no start-up or round is added, and
    // (4) the page counts moved by at most 1/64 of the work in total (at
    // most 1.6% of the modelled bytes, inside the model's own error).
    struct Memo {
        uint64_t shape[8] = {};
        std::vector<uint32_t> pages;
        uint64_t total = 0;
        uint64_t n_units = 0;
        DecodeSplit val;
        bool used = false;
    };
    thread_local Memo memo[4];
    thread_local uint32_t memo_next = 0;
    const uint64_t shape[8] = {rows, kv_heads, q_heads, head_dim, kv_dtype, page_tokens,
                               partial_bytes, device_cus()};
    uint64_t total = 0;
    for (uint32_t r = 0; r < rows; ++r) total += pages[r];
    auto units_of = [&](const DecodeSplit& v) {
        if (v.splits <= 1u || v.pages_per_split == 0u) return (uint64_t)rows;
        uint64_t n = 0;
        for (uint32_t r = 0; r < rows; ++r) n += (pages[r] + v.pages_per_split - 1u) / v.pages_per_split;
        return n;
    };
    for (Memo& m : memo) {
        if (!m.used || !std::equal(shape, shape + 8, m.shape)) continue;
        const DecodeSplit& v = m.val;
        if (v.splits > 1u && (max_pages + v.pages_per_split - 1u) / v.pages_per_split > v.splits)
            continue;
        if (units_of(v) != m.n_units) continue;
        uint64_t moved = 0;
        for (uint32_t r = 0; r < rows; ++r)
            moved += pages[r] > m.pages[r] ? pages[r] - m.pages[r] : m.pages[r] - pages[r];
        if (moved * 64u > m.total) continue;
        return v;
    }
    auto remember = [&](const DecodeSplit& v) {
        Memo& m = memo[memo_next];
        std::copy(shape, shape + 8, m.shape);
        m.pages = pages;
        m.total = total;
        m.n_units = units_of(v);
        m.val = v;
        m.used = true;
        memo_next = (memo_next + 1u) % 4u;
        return v;
    };
    const uint32_t groups = (kv_heads + 3u) / 4u;   // independent-wave workgroups per unit
    const size_t lds = psk::decode_workgroup_lds_bytes(kv_dtype, head_dim);
    const uint32_t per_cu = std::max<uint32_t>(1u, (uint32_t)((160u * 1024u) / lds));
    const uint32_t slots = std::max<uint32_t>(1u, device_cus() / kXcds) * per_cu;
    const uint64_t total_slots = (uint64_t)slots * kXcds;
    // K and V bytes of one (token, head) with their scales, per page of the
    // 4 kv heads one workgroup streams; the fitted fluid model
    // (split_makespan) runs in bytes
    const double slice = kv_dtype == PSK_KV_BF16        ? 4.0 * head_dim
                         : kv_dtype == PSK_KV_FP8_E4M3  ? 2.0 * head_dim + 8.0
                         : kv_dtype == PSK_KV_PSQ4_W32  ? head_dim + head_dim / 8.0
                                                        : 2.0 * head_dim + head_dim / 8.0;
    const double page_bytes = 4.0 * page_tokens * slice;
    const double xcd_bw = 6.7e12 / kXcds;
    // a workgroup alone on its CU streams up to 1.5x its fair share; where two
    // share a CU (PSQ4, VALU-bound) the tail gains nothing (measured: 7 splits
    // of 293 pages ran 4% slower than 8 of 256 at b64 x 32k)
    const double wg_bw = (per_cu > 1 ? 1.0 : 1.5) * xcd_bw / (double)slots;
    const double c0 = 10e-6;
    // Candidates (predicted makespan, splits, pages per split); splits == 1
    // competes when the rows alone fill every slot (it saves the combine pass,
    // ~2%).
    struct Cand { double t; uint32_t splits, per; };
    std::vector<Cand> cands;
    std::vector<double> units;
    // Units of one launch in dispatch order: every row's splits but the last,
    // then every row's last split. At >= 128 workgroups each (row, split) is
    // `groups` independent-wave workgroups; below that the decode launcher
    // runs one 4-wave workgroup per (row, split, kv head), a quarter of the
    // work each (in pages of 4 kv heads).
    auto build = [&](uint32_t per, uint64_t n_units) {
        units.clear();
        const bool indep = n_units * groups >= 128;
        const uint32_t copies = indep ? groups : kv_heads;
        const double share = indep ? 1.0 : 0.25;
        for (uint32_t r = 0; r < rows; ++r)
            for (uint32_t s = 0; s + 1 < (pages[r] + per - 1) / per; ++s)
                for (uint32_t k = 0; k < copies; ++k) units.push_back(per * share * page_bytes);
        for (uint32_t r = 0; r < rows; ++r) {
            const uint32_t n = (pages[r] + per - 1) / per;
            if (n == 0) continue;
            for (uint32_t k = 0; k < copies; ++k) units.push_back((pages[r] - (n - 1) * per) * share * page_bytes);
        }
    };
    if ((uint64_t)rows * groups >= total_slots) {
        // Enough rows to fill every slot unsplit: splitting must then win by
        // more than the combine pass costs (~2%).
        build(max_pages, rows);
        std::sort(units.begin(), units.end(), std::greater<double>());
        cands.push_back({split_makespan(units, slots, xcd_bw, wg_bw, c0) / 1.02, 1u, 0u});
    }
    for (uint32_t splits = 2; splits <= std::min<uint32_t>(kMaxSplits, max_pages); ++splits) {
        const uint32_t per = (max_pages + splits - 1) / splits;
        if (per < kMinPagesPerSplit) break;
        if ((max_pages + per - 1) / per != splits) continue;   // same as a smaller count
        const uint64_t need = (uint64_t)rows * kv_heads * splits * q_per_kv *
                              (2u + ::ps::kernel::kPagedAttentionHeadLimit) * sizeof(float);
        if (need > partial_bytes) break;
        uint64_t n_units = 0;
        for (uint32_t r = 0; r < rows; ++r) n_units += (pages[r] + per - 1) / per;
        if (n_units * groups > 4 * total_slots) break;   // finer splits only add start-ups
        build(per, n_units);
        // the shared-item mode (below 128 workgroups) merges its 4 waves
        // through LDS and measured up to 18% slower than the model
        const double shared = n_units * groups >= 128 ? 1.0 : 1.1;
        cands.push_back({split_makespan(units, slots, xcd_bw, wg_bw, c0) * shared, splits, per});
    }
    if (cands.empty()) return remember(best);
    const Cand* pick = &cands[0];
    for (const Cand& c : cands)
        if (c.t < pick->t) pick = &c;
    best.splits = pick->splits;
    best.pages_per_split = pick->per;
    return remember(best);
}

namespace {

// Tile launches: split only until the grid fills the GPU's tile workgroup
// slots (prefill chunks of 512 rows usually fill them unsplit; a few verify
// blocks over long contexts need splits to occupy the CUs).
DecodeSplit choose_tile_split(uint32_t n_tiles, uint32_t tiles_per_group, uint32_t region_rows,
                              uint32_t kv_heads, uint32_t q_heads, uint32_t head_dim,
                              uint32_t kv_dtype, uint32_t page_tokens,
                              uint32_t max_visible_tokens, uint64_t partial_bytes,
                              const std::vector<uint32_t>& tile_visible) {
    DecodeSplit s;
    if (max_visible_tokens < kSplitMinVisible || n_tiles == 0 || kv_heads == 0) return s;
    const uint32_t q_per_kv = q_heads / kv_heads;
    auto fits = [&](uint64_t splits) {
        return (uint64_t)region_rows * kv_heads * splits * q_per_kv *
                   (2u + ::ps::kernel::kPagedAttentionHeadLimit) * sizeof(float) <=
               partial_bytes;
    };
    if (tiles_per_group == 1u && tile_visible.size() == n_tiles) {
        // Ungrouped tiles split into dense (tile, split) units, dealt
        // longest first over the XCDs. Cost model, in pages: rounds of units
        // over the CUs x (pages per split + kTileSplitFixedPages of start-up:
        // Q split, block-table window, partial write). One workgroup per CU:
        // a 6-wave workgroup (5-6 heads) puts two waves on SIMDs 0 and 1, and
        // a second one doubles those (measured on 8 verify blocks of config
        // 5: 236 units of 80 pages 66 us, 280 units of 66 pages 102 us).
        constexpr uint64_t kTileSplitFixedPages = 16;
        // 5-6 heads: the 6-wave kernel (PSQ: 8 waves, 2 per SIMD, which fill the
        // registers of a CU's SIMDs at 168 each)
        const bool nw6 = q_per_kv > 4u && q_per_kv <= 6u;
        const uint64_t slots =
            (uint64_t)device_cus() * (nw6 ? 1u : psk::tile_workgroups_per_cu(kv_dtype, head_dim, q_per_kv, false));
        const uint64_t max_pages = (max_visible_tokens + page_tokens - 1) / page_tokens;
        std::vector<uint64_t> pages(n_tiles);
        uint64_t longest = 0;
        for (uint32_t t = 0; t < n_tiles; ++t) {
            pages[t] = std::min<uint64_t>(max_pages, (tile_visible[t] + page_tokens - 1) / page_tokens);
            longest = std::max(longest, pages[t]);
        }
        auto cost = [&](uint64_t per) {
            uint64_t units = 0;
            for (uint64_t pg : pages) units += (pg + per - 1) / per;
            units *= kv_heads;
            return ((units + slots - 1) / slots) * (std::min(per, longest) + kTileSplitFixedPages);
        };
        uint64_t best_cost = cost(max_pages), best_splits = 1, best_per = 0;
        const uint64_t top = std::min<uint64_t>(kMaxSplits, std::min<uint64_t>(64, max_pages / kMinPagesPerSplit));
        for (uint64_t splits = 2; splits <= top; ++splits) {
            const uint64_t per = (max_pages + splits - 1) / splits;
            if ((max_pages + per - 1) / per != splits) continue;   // same as a smaller count
            if (!fits(splits)) break;
            // the model holds for launches that run as dense units
            if ((uint64_t)n_tiles * splits > psk::tile_dense_units_limit()) break;
            const uint64_t cst = cost(per);
            if (cst < best_cost) {
                best_cost = cst;
                best_splits = splits;
                best_per = per;
            }
        }
        if (best_splits > 1) {
            s.splits = static_cast<uint32_t>(best_splits);
            s.pages_per_split = static_cast<uint32_t>(best_per);
        }
        return s;
    }
    const uint64_t slots = (uint64_t)device_cus() *
                           psk::tile_workgroups_per_cu(kv_dtype, head_dim, q_per_kv, tiles_per_group > 1u);
    const uint64_t wgs = psk::tile_launch_workgroups(n_tiles, tiles_per_group, q_per_kv, kv_heads);
    if (wgs >= slots) return s;
    const uint64_t max_pages = (max_visible_tokens + page_tokens - 1) / page_tokens;
    uint64_t splits = std::min<uint64_t>((slots + wgs - 1) / wgs, max_pages / kMinPagesPerSplit);
    splits = std::min<uint64_t>(splits, kMaxSplits);
    while (splits > 1) {
        const uint64_t need = (uint64_t)region_rows * kv_heads * splits * q_per_kv *
                              (2u + ::ps::kernel::kPagedAttentionHeadLimit) * sizeof(float);
        if (need <= partial_bytes) break;
        splits /= 2;
    }
    if (splits <= 1) return s;
    const uint64_t per = (max_pages + splits - 1) / splits;
    s.splits = static_cast<uint32_t>((max_pages + per - 1) / per);
    s.pages_per_split = static_cast<uint32_t>(per);
    return s;
}

bool is_tile_request(const StepRequest& r) {
    return (r.execution_class == kExecPrefill && r.row_count >= kPrefillMinRows) ||
           (r.execution_class == kExecSpecVerify && r.row_count >= kVerifyTileMinRows);
}

}  // namespace

Status plan_paged_attention_step(const PagedAttentionStep& step, PagedAttentionPlan& plan) {
    plan = PagedAttentionPlan{};
    const auto& c = step.common;
    if (c.rows == 0) return Status::make_ok();
    const bool psq = step.kv_dtype == KVCacheDType::PSQ4_W32 || step.kv_dtype == KVCacheDType::PSQ8_W32;
    if (step.kv_dtype != KVCacheDType::BF16 && step.kv_dtype != KVCacheDType::FP8_E4M3 && !psq)
        return Status::invalid_argument("unknown KV cache dtype");
    const uint64_t pbytes = step.partials ? step.partial_bytes : 0;
    auto push = [&](const PlannedKernel& k) -> Status {
        if (plan.count >= kMaxPlannedKernels) return Status::out_of_range("too many launches in a step");
        plan.kernels[plan.count++] = k;
        return Status::make_ok();
    };
    // Upper bounds of the rows' visible lengths where the requests carry them
    // (StepRequest::max_visible), else the step's max_visible_tokens.
    std::vector<uint32_t> row_vis;
    auto add_decode = [&](uint32_t row_begin, uint32_t rows) -> Status {
        PlannedKernel k;
        k.kind = PlannedKernel::Kind::Decode;
        k.row_begin = row_begin;
        k.rows = rows;
        row_vis.assign(rows, step.max_visible_tokens);
        for (uint32_t i = 0; i < step.num_requests; ++i) {
            const StepRequest& r = step.requests[i];
            if (r.max_visible == 0 || r.row_begin >= row_begin + rows ||
                r.row_begin + r.row_count <= row_begin)
                continue;
            const uint32_t lo = std::max(r.row_begin, row_begin);
            const uint32_t hi = std::min(r.row_begin + r.row_count, row_begin + rows);
            for (uint32_t j = lo; j < hi; ++j)
                row_vis[j - row_begin] = std::min(r.max_visible, step.max_visible_tokens);
        }
        const DecodeSplit s = choose_decode_split(
            rows, c.kv_heads, c.q_heads, c.head_dim, static_cast<uint32_t>(step.kv_dtype),
            c.page_tokens, step.max_visible_tokens, row_vis.data(), pbytes);
        k.splits = s.splits;
        k.pages_per_split = s.pages_per_split;
        return push(k);
    };

    // Requests must partition [0, rows); otherwise every row runs on the
    // decode kernel (always correct: each row attends to its own prefix).
    std::vector<StepRequest> reqs(step.requests, step.requests + step.num_requests);
    std::sort(reqs.begin(), reqs.end(),
              [](const StepRequest& x, const StepRequest& y) { return x.row_begin < y.row_begin; });
    bool partition = !reqs.empty();
    uint32_t next = 0;
    for (const auto& r : reqs) {
        if (r.row_begin != next || r.row_count == 0) partition = false;
        next = r.row_begin + r.row_count;
    }
    if (next != c.rows) partition = false;
    // PSQ tiles cover head_dim 128 and 256 (q_per_kv <= 8 as every tile);
    // other PSQ shapes run every row of the step as a decode row (each
    // attends to its own prefix, the reference's causal rule).
    const bool psq_tiles = (c.head_dim == 128 || c.head_dim == 256) && c.kv_heads != 0 &&
                           c.q_heads / c.kv_heads <= 8u;
    if (!partition || (psq && !psq_tiles)) return add_decode(0, c.rows);

    // decode launches: maximal runs of consecutive non-tile requests
    for (size_t i = 0; i < reqs.size();) {
        if (is_tile_request(reqs[i])) {
            ++i;
            continue;
        }
        const uint32_t b = reqs[i].row_begin;
        uint32_t e = b;
        while (i < reqs.size() && !is_tile_request(reqs[i])) e = reqs[i].row_begin + reqs[i++].row_count;
        Status st = add_decode(b, e - b);
        if (!st.ok()) return st;
    }
    // one tile launch per class (verify blocks typically split, prefill not)
    for (const uint8_t cls : {kExecSpecVerify, kExecPrefill}) {
        PlannedKernel k;
        k.kind = PlannedKernel::Kind::Tile;
        k.tile_first = static_cast<uint32_t>(plan.tiles.size());
        k.req_first = static_cast<uint32_t>(plan.combine.size());
        uint32_t lo = UINT32_MAX, hi = 0;
        // prefill tiles go in groups of consecutive tiles of one request (the
        // kernel stages each K/V chunk once for the group); rows == 0 pads
        const uint32_t group =
            cls == kExecPrefill ? psk::tile_group_size(c.kv_heads ? c.q_heads / c.kv_heads : 0u,
                                                       static_cast<uint32_t>(step.kv_dtype))
                                : 1u;
        // (visible bound, first tile of the group in `flat`)
        std::vector<std::pair<uint32_t, size_t>> groups;
        std::vector<PlannedTile> flat;
        for (const auto& r : reqs) {
            if (r.execution_class != cls || !is_tile_request(r)) continue;
            for (uint32_t t = 0; t < r.row_count; t += kTileRowsPerTile * group) {
                const size_t first = flat.size();
                uint32_t vis = 0;
                for (uint32_t j = 0; j < group; ++j) {
                    const uint32_t tt = t + j * kTileRowsPerTile;
                    if (tt >= r.row_count) {
                        flat.push_back({r.row_begin + t, 0u});
                        continue;
                    }
                    const uint32_t n = std::min(kTileRowsPerTile, r.row_count - tt);
                    // rows of a request see prefix + index + 1 tokens
                    vis = r.max_visible != 0 ? r.max_visible - (r.row_count - tt - n)
                                             : step.max_visible_tokens;
                    flat.push_back({r.row_begin + tt, n});
                }
                groups.push_back({vis, first});
            }
            plan.combine.push_back(r);
            lo = std::min(lo, r.row_begin);
            hi = std::max(hi, r.row_begin + r.row_count);
        }
        // longest groups first: workgroups are dispatched in tile order
        std::stable_sort(groups.begin(), groups.end(),
                         [](const auto& x, const auto& y) { return x.first > y.first; });
        for (const auto& gr : groups)
            for (uint32_t j = 0; j < group; ++j) plan.tiles.push_back(flat[gr.second + j]);
        k.tiles_per_group = group;
        k.tile_count = static_cast<uint32_t>(plan.tiles.size()) - k.tile_first;
        k.req_count = static_cast<uint32_t>(plan.combine.size()) - k.req_first;
        if (k.tile_count == 0) continue;
        k.row_begin = lo;
        k.rows = hi - lo;
        std::vector<uint32_t> tile_vis;
        if (group == 1u)
            for (const auto& gr : groups) tile_vis.push_back(gr.first);
        const DecodeSplit s = choose_tile_split(
            k.tile_count, k.tiles_per_group, k.rows, c.kv_heads, c.q_heads, c.head_dim,
            static_cast<uint32_t>(step.kv_dtype), c.page_tokens,
            step.max_visible_tokens, pbytes, tile_vis);
        k.splits = s.splits;
        k.pages_per_split = s.pages_per_split;
        Status st = push(k);
        if (!st.ok()) return st;
    }
    // In a step with a large tile launch (>= kForkMinTileRows rows), every
    // other launch runs beside it on a side lane: the decode launches on lane
    // 1, the other tile launches (verify blocks) on lane 2, in order within a
    // lane. Their workgroups take the CUs the compute-bound tile launch leaves
    // idle (its second round of workgroups, its tail), and the two lanes run
    // concurrently with each other too. The large launch keeps the start of
    // the split-K workspace; lane 1 uses the region after it and lane 2 the
    // region after lane 1's. When those do not fit, every side launch goes to
    // lane 1 and shares its region (one after another); when even that does
    // not fit, the step stays in order on one stream.
    const uint32_t qpk = c.kv_heads ? c.q_heads / c.kv_heads : 0u;
    auto need_of = [&](const PlannedKernel& k) -> uint64_t {
        return k.splits > 1 ? (uint64_t)k.rows * c.kv_heads * k.splits * qpk *
                                  (2u + ::ps::kernel::kPagedAttentionHeadLimit) * 4u
                            : 0u;
    };
    int main_k = -1;
    for (uint32_t i = 0; i < plan.count; ++i)
        if (plan.kernels[i].kind == PlannedKernel::Kind::Tile &&
            (main_k < 0 || plan.kernels[i].rows > plan.kernels[main_k].rows))
            main_k = (int)i;
    if (step.concurrent_decode && main_k >= 0 && plan.count > 1 &&
        plan.kernels[main_k].rows >= kForkMinTileRows) {
        uint64_t need_side = 0, need1 = 0, need2 = 0;
        bool any1 = false, any2 = false;
        for (uint32_t i = 0; i < plan.count; ++i) {
            if ((int)i == main_k) continue;
            const uint64_t n = need_of(plan.kernels[i]);
            need_side = std::max(need_side, n);
            if (plan.kernels[i].kind == PlannedKernel::Kind::Decode) {
                need1 = std::max(need1, n);
                any1 = true;
            } else {
                need2 = std::max(need2, n);
                any2 = true;
            }
        }
        const uint64_t side_at = (need_of(plan.kernels[main_k]) + 255u) & ~uint64_t{255};
        const uint64_t lane2_at = side_at + ((need1 + 255u) & ~uint64_t{255});
        const bool two_lanes = any1 && any2 && (need2 == 0 || lane2_at + need2 <= pbytes) &&
                               (need1 == 0 || side_at + need1 <= pbytes);
        if (two_lanes || need_side == 0 || side_at + need_side <= pbytes) {
            for (uint32_t i = 0; i < plan.count; ++i) {
                if ((int)i == main_k) continue;
                const bool lane2 = two_lanes && plan.kernels[i].kind != PlannedKernel::Kind::Decode;
                plan.kernels[i].side = lane2 ? 2u : 1u;
                plan.kernels[i].partial_offset = (lane2 ? lane2_at : side_at) / 4u;
            }
        }
    }
    return Status::make_ok();
}

namespace {

// Side lanes (two streams) and fork/join events per (device, caller
// stream), created on first use and kept for the life of the process.
// Default priority, no blocking with the null stream.
struct SideStream {
    hipStream_t stream = nullptr;    // lane 1
    hipStream_t stream2 = nullptr;   // lane 2
    hipEvent_t fork = nullptr;
    hipEvent_t join = nullptr;
    hipEvent_t join2 = nullptr;
};

SideStream* side_stream_for(hipStream_t main) {
    static std::mutex mu;
    static std::map<std::pair<int, hipStream_t>, SideStream> table;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) {
        (void)hipGetLastError();
        return nullptr;
    }
    std::lock_guard<std::mutex> lock(mu);
    auto it = table.find({dev, main});
    if (it != table.end()) return &it->second;
    SideStream s;
    if (hipStreamCreateWithFlags(&s.stream, hipStreamNonBlocking) != hipSuccess ||
        hipStreamCreateWithFlags(&s.stream2, hipStreamNonBlocking) != hipSuccess ||
        hipEventCreateWithFlags(&s.fork, hipEventDisableTiming) != hipSuccess ||
        hipEventCreateWithFlags(&s.join, hipEventDisableTiming) != hipSuccess ||
        hipEventCreateWithFlags(&s.join2, hipEventDisableTiming) != hipSuccess) {
        (void)hipGetLastError();
        if (s.join2) (void)hipEventDestroy(s.join2);
        if (s.join) (void)hipEventDestroy(s.join);
        if (s.fork) (void)hipEventDestroy(s.fork);
        if (s.stream2) (void)hipStreamDestroy(s.stream2);
        if (s.stream) (void)hipStreamDestroy(s.stream);
        return nullptr;   // the step then runs in order on `main`
    }
    return &table.emplace(std::make_pair(dev, main), s).first->second;
}

}  // namespace

hipError_t launch_paged_attention_plan(const PagedAttentionStep& step, const PagedAttentionPlan& plan,
                                       hipStream_t stream) {
    using namespace ::ps::kernel;
    const bool fp8 = step.kv_dtype == KVCacheDType::FP8_E4M3;
    const bool psq = step.kv_dtype == KVCacheDType::PSQ4_W32 || step.kv_dtype == KVCacheDType::PSQ8_W32;
    const auto* ksf = static_cast<const float*>(step.k_scale_pool);
    const auto* vsf = static_cast<const float*>(step.v_scale_pool);
    const auto* k8 = static_cast<const ::ps::qwen35::fp8e4m3_storage_t*>(step.k_pool);
    const auto* v8 = static_cast<const ::ps::qwen35::fp8e4m3_storage_t*>(step.v_pool);
    const auto* k16 = static_cast<const bf16_t*>(step.k_pool);
    const auto* v16 = static_cast<const bf16_t*>(step.v_pool);
    auto run = [&](const PlannedKernel& k, hipStream_t stream) -> hipError_t {
        float* const parts = step.partials ? step.partials + k.partial_offset : nullptr;
        const PagedAttentionCommonArgs a = region_args(step.common, k.row_begin, k.rows);
        hipError_t e = hipSuccess;
        if (k.kind == PlannedKernel::Kind::Tile) {
            // tile rows are relative to the launch region
            std::vector<uint32_t> tb(k.tile_count), tr(k.tile_count);
            for (uint32_t t = 0; t < k.tile_count; ++t) {
                tb[t] = plan.tiles[k.tile_first + t].row_begin - k.row_begin;
                tr[t] = plan.tiles[k.tile_first + t].rows;
            }
            const psk_paged_attention_args* ca = reinterpret_cast<const psk_paged_attention_args*>(&a);
            const uint32_t kvd = static_cast<uint32_t>(step.kv_dtype);
            if (psk::paged_tiles_supported(*ca, kvd, step.k_pool, step.v_pool, step.k_scale_pool,
                                           step.v_scale_pool)) {
                e = psk::launch_paged_tiles(*ca, kvd, step.k_pool, step.v_pool, step.k_scale_pool,
                                            step.v_scale_pool, tb.data(), tr.data(), k.tile_count,
                                            k.tiles_per_group, parts, k.splits,
                                            k.pages_per_split, stream);
                // one combine per run of adjacent requests of the launch (rows of
                // other requests inside the launch's region hold no partials)
                for (uint32_t q = 0; e == hipSuccess && k.splits > 1 && q < k.req_count;) {
                    const uint32_t begin = plan.combine[k.req_first + q].row_begin;
                    uint32_t end = begin + plan.combine[k.req_first + q].row_count;
                    for (++q; q < k.req_count && plan.combine[k.req_first + q].row_begin == end; ++q)
                        end += plan.combine[k.req_first + q].row_count;
                    const PagedAttentionCommonArgs ra = region_args(a, begin - k.row_begin, end - begin);
                    // the combine reads partials of the region's rows; shift them with it
                    const uint64_t row_floats = (uint64_t)a.kv_heads * k.splits *
                                                (a.q_heads / a.kv_heads) * (2u + kPagedAttentionHeadLimit);
                    e = launch_attention_paged_split_reduce_ex(
                        ra, parts + (uint64_t)(begin - k.row_begin) * row_floats,
                        k.splits, k.pages_per_split, stream);
                }
            } else {
                // shapes outside the tile kernel: every row of each tile on the decode kernel
                for (uint32_t t = 0; e == hipSuccess && t < k.tile_count; ++t) {
                    if (tr[t] == 0u) continue;   // group padding
                    const PagedAttentionCommonArgs ta = region_args(a, tb[t], tr[t]);
                    if (psq)
                        e = static_cast<hipError_t>(psk_attention_paged_psq(
                            reinterpret_cast<const psk_paged_attention_args*>(&ta), kvd,
                            static_cast<const uint8_t*>(step.k_pool), static_cast<const uint8_t*>(step.v_pool),
                            static_cast<const uint16_t*>(step.k_scale_pool),
                            static_cast<const uint16_t*>(step.v_scale_pool), a.head_dim / 32u, stream));
                    else
                        e = fp8 ? launch_attention_paged_fp8_e4m3(ta, k8, v8, ksf, vsf, stream)
                                : launch_attention_paged_bf16(ta, k16, v16, stream);
                }
            }
        } else if (psq) {
            const auto* ca = reinterpret_cast<const psk_paged_attention_args*>(&a);
            const auto* kc = static_cast<const uint8_t*>(step.k_pool);
            const auto* vc = static_cast<const uint8_t*>(step.v_pool);
            const auto* ks = static_cast<const uint16_t*>(step.k_scale_pool);
            const auto* vs = static_cast<const uint16_t*>(step.v_scale_pool);
            const uint32_t kvd = static_cast<uint32_t>(step.kv_dtype);
            const uint32_t bph = a.head_dim / 32u;
            if (k.splits > 1) {
                e = static_cast<hipError_t>(psk_attention_paged_psq_split_ex(
                    ca, kvd, kc, vc, ks, vs, bph, parts, k.splits, k.pages_per_split, stream));
                if (e == hipSuccess)
                    e = launch_attention_paged_split_reduce_ex(a, parts, k.splits,
                                                               k.pages_per_split, stream);
            } else {
                e = static_cast<hipError_t>(psk_attention_paged_psq(ca, kvd, kc, vc, ks, vs, bph, stream));
            }
        } else if (k.splits > 1) {
            e = fp8 ? launch_attention_paged_fp8_e4m3_split(a, k8, v8, ksf, vsf, parts,
                                                            k.splits, k.pages_per_split, stream)
                    : static_cast<hipError_t>(psk_attention_paged_bf16_split_ex(
                          reinterpret_cast<const psk_paged_attention_args*>(&a), k16, v16,
                          parts, k.splits, k.pages_per_split, stream));
            if (e == hipSuccess)
                e = launch_attention_paged_split_reduce_ex(a, parts, k.splits,
                                                           k.pages_per_split, stream);
        } else {
            e = fp8 ? launch_attention_paged_fp8_e4m3(a, k8, v8, ksf, vsf, stream)
                    : launch_attention_paged_bf16(a, k16, v16, stream);
        }
        return e;
    };
    bool fork = false;
    for (uint32_t i = 0; i < plan.count; ++i) fork = fork || plan.kernels[i].side != 0;
    SideStream* side = fork ? side_stream_for(stream) : nullptr;
    if (side == nullptr) {
        for (uint32_t i = 0; i < plan.count; ++i) {
            const hipError_t e = run(plan.kernels[i], stream);
            if (e != hipSuccess) return e;
        }
        return hipSuccess;
    }
    bool lane2 = false;
    for (uint32_t i = 0; i < plan.count; ++i) lane2 = lane2 || plan.kernels[i].side == 2u;
    // fork: the side lanes start after the work before this step on
    // `stream`; `stream` continues only after the side launches (join)
    hipError_t e = hipEventRecord(side->fork, stream);
    if (e != hipSuccess) return e;
    e = hipStreamWaitEvent(side->stream, side->fork, 0);
    if (e == hipSuccess && lane2) e = hipStreamWaitEvent(side->stream2, side->fork, 0);
    if (e != hipSuccess) return e;
    // the large launch is enqueued first, so its workgroups take the CUs
    // first and the side launches fill what it leaves
    for (uint32_t i = 0; e == hipSuccess && i < plan.count; ++i)
        if (!plan.kernels[i].side) e = run(plan.kernels[i], stream);
    for (uint32_t i = 0; e == hipSuccess && i < plan.count; ++i)
        if (plan.kernels[i].side == 1u) e = run(plan.kernels[i], side->stream);
    for (uint32_t i = 0; e == hipSuccess && i < plan.count; ++i)
        if (plan.kernels[i].side == 2u) e = run(plan.kernels[i], side->stream2);
    // join even after an error, so a capture never ends with a side lane forked
    hipError_t j = hipEventRecord(side->join, side->stream);
    if (j == hipSuccess) j = hipStreamWaitEvent(stream, side->join, 0);
    if (lane2) {
        hipError_t j2 = hipEventRecord(side->join2, side->stream2);
        if (j2 == hipSuccess) j2 = hipStreamWaitEvent(stream, side->join2, 0);
        if (j == hipSuccess) j = j2;
    }
    return e != hipSuccess ? e : j;
}

}  // namespace ps::qwen35::runtime
