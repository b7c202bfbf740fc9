// KV append into the paged pool: BF16 copy and BF16 -> FP8 E4M3 with fused
// per-(token, head) absmax quantization. gfx950, wave64.
//
// Reference behaviour restated (file:line in the reference repository):
//   row -> (page, slot) resolution and skip rules   kv_append.hip:31-55
//   BF16 body                                       kv_append.hip:21-103
//   FP8 body: amax, scale = amax==0 ? 1 : amax/448,
//   code = e4m3_satfinite(x / scale), scale store   kv_append.hip:148-272
//   launcher validation                             kv_append.hip:105-115,546-558
//
//   PSQ4_W32 / PSQ8_W32 body: per 32-value block
//   amax, s = bf16(amax*0.1 | amax/448), codes of x/s,
//   LSQ1 refit s1 = bf16(sum xq / sum qq)            kv_append.hip:276-643
//   block index, nibble packing, bf16 scale store   kv_append.hip:368-399
//
// Layout of the work: one "head task" = (row, kv_head). A task is handled by
// L = lanes_per_head lanes (a power of two <= 64), each lane owning chunks of
// 8 consecutive elements (16 B of bf16 input); a wave runs 64/L tasks. For
// head_dim 256 that is 32 lanes x 16 B per K and V, i.e. fully coalesced
// 512 B reads and 256 B (FP8) or 512 B (BF16) writes per tensor per task.
#include "device_common.h"
#include "fastdiv.h"

#include <phaseshift_kv/kv_append.h>
#include <phaseshift_kv_c.h>

namespace psk {
namespace {

struct AppendParams {
    psk_kv_append_args a;
    void* k_pool;
    void* v_pool;
    float* k_scale;
    float* v_scale;
    uint32_t lanes_per_head;   // L
    uint32_t log2_lanes;
    uint32_t chunks;           // ceil(head_dim / 8)
    uint32_t vec_ok;           // 16 B loads / vector stores legal
    // kReq launches: rows take (slot, position) from these request
    // descriptors and the kernel writes them to a.row_sequence_slots /
    // a.row_positions for the later launches of the step
    const psk_request_descriptor* req;
    uint32_t num_req;
};

// Loads chunk `c` (elements 8c..8c+7) of a head slice as 8 floats; elements
// past head_dim read as 0.
__device__ __forceinline__ void load_chunk(const uint16_t* src, uint32_t c, uint32_t D, bool vec,
                                           float (&x)[8]) {
    const uint32_t e0 = c * 8u;
    if (vec) {
        const u32x4 w = *reinterpret_cast<const u32x4*>(src + e0);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            x[2 * i] = __uint_as_float(w[i] << 16);
            x[2 * i + 1] = __uint_as_float(w[i] & 0xFFFF0000u);
        }
    } else {
#pragma unroll
        for (int i = 0; i < 8; ++i)
            x[i] = (e0 + i < D) ? bf16_bits_to_f32(src[e0 + i]) : 0.0f;
    }
}

// Quantizes 8 values of one head slice and packs the E4M3 codes (byte i =
// element i): x / scale as the reference computes it (IEEE quotient, then the
// SATFINITE RNE conversion).
__device__ __forceinline__ u32x2 encode8(const float (&x)[8], float scale, float rcp, bool fast) {
    float q[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) q[i] = div_by_scale(x[i], scale, rcp, fast);
    u32x2 c;
    c[0] = e4m3_encode_pair(q[2], q[3], e4m3_encode_pair(q[0], q[1], 0u, false), true);
    c[1] = e4m3_encode_pair(q[6], q[7], e4m3_encode_pair(q[4], q[5], 0u, false), true);
    return c;
}

__device__ __forceinline__ float head_scale(float amax) {
    return amax == 0.0f ? 1.0f : amax / kFp8Max;
}

__device__ __forceinline__ bool fast_div_ok(float scale) {
    return scale >= 0x1p-100f && scale <= 0x1.fffffep+127f;
}

// Fast path: head_dim % 8 == 0, head_dim <= 8 * L, every access aligned. A
// wave runs U groups of 64/L tasks. The slot/position loads go out first,
// then the input loads, then the block-table loads (which wait only for
// slot/position), so the HBM reads overlap the lookup chain (reference skip
// rules: kv_append.hip:31-55). GPU time per launch (replayed graph for the
// small sizes): one group per wave is fastest up to 2^15 rows (128 rows
// 3.06 us against 4.41 with two groups and 7.38 with four), two groups from
// 2^16 rows (2^16 rows 75.5-76.4 us against 78.6-79.3 with one; 2^17 rows
// 149.8-150.5 against 155.7-156.4); kTwoGroupTasks picks.
constexpr uint64_t kTwoGroupTasks = 1u << 18;

// kReq: the row metadata of a planned step is formed here instead of by a
// launch of its own (device_batch_context.hip:69-90): the wave loads 64
// request descriptors at a time, one per lane, and each distinct row of its
// tasks finds the request whose [row_begin, row_begin + row_count) holds it
// by a ballot (requests do not overlap); lane 0 of the row's first head
// writes the row's slot and position. A row outside every request keeps its
// metadata and is not appended.
template <bool kFp8, bool kReq, int kUnroll>
__global__ __launch_bounds__(256) void kv_append_fast_kernel(const AppendParams p) {
    const psk_kv_append_args& a = p.a;
    const uint32_t L = p.lanes_per_head;
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave_global = (blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    const uint32_t tasks_per_wave = 64u >> p.log2_lanes;
    const uint32_t sub = lane & (L - 1u);
    const uint32_t total = a.rows * a.kv_heads;   // launcher checks < 2^32
    const uint32_t D = a.head_dim;
    const bool has_chunk = sub < p.chunks;
    const uint32_t e0 = sub * 8u;

    uint32_t row[kUnroll], head[kUnroll];
    bool live[kUnroll];
    u32x4 kw[kUnroll], vw[kUnroll];
    uint32_t slot[kUnroll], pos[kUnroll];
    // slot/position loads first: the block-table loads below need only them
    // (vmcnt retires in order), so their round trip overlaps the K/V reads
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
        const uint32_t task = (wave_global * kUnroll + u) * tasks_per_wave + (lane >> p.log2_lanes);
        live[u] = task < total;
        const uint32_t t = live[u] ? task : 0u;
        row[u] = t / a.kv_heads;
        head[u] = t - row[u] * a.kv_heads;
        if constexpr (!kReq) {
            slot[u] = a.row_sequence_slots[row[u]];
            pos[u] = a.row_positions[row[u]];
        }
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
        // lanes without a chunk read the slice start (always in bounds) and
        // drop the value, so the loads need no branch
        const uint32_t e = has_chunk ? e0 : 0u;
        const uint16_t* ks = static_cast<const uint16_t*>(a.k_input) +
                             (uint64_t)row[u] * a.k_row_stride + head[u] * D + e;
        const uint16_t* vs = static_cast<const uint16_t*>(a.v_input) +
                             (uint64_t)row[u] * a.v_row_stride + head[u] * D + e;
        // input rows are read once: non-temporal loads (and stores of the
        // codes below) measured ~3.5% faster at 2^16 rows than the default
        // policy (the PSQ kernel's 64 B-per-lane blocks measured slower with it)
        kw[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(ks));
        vw[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(vs));
    }
    // (request rows: the descriptor scan runs while the K/V loads are in flight)
    if constexpr (kReq) {
        static_assert(kUnroll == 1, "request rows: one task group per wave");
        // the wave's rows are consecutive: [row_lo, row_hi] of its live tasks
        // (wave-uniform; a wave without live tasks scans nothing)
        const uint32_t first_task = wave_global * tasks_per_wave;
        const uint32_t row_lo = first_task / a.kv_heads;
        const uint32_t row_hi = first_task < total ? (min(first_task + tasks_per_wave, total) - 1u) / a.kv_heads
                                                   : row_lo - 1u;
        slot[0] = 0xFFFFFFFFu;
        pos[0] = 0u;
        bool found = false;
        // first the 64 descriptors ending at index row_lo (the request of
        // row R has index <= R when requests come in row order, one row or
        // more each), then every 64-descriptor window in turn
        const uint32_t b0 = row_lo >= 63u ? row_lo - 63u : 0u;
        const uint32_t first = p.num_req > 64u ? min(b0, p.num_req - 64u) : 0u;
        const uint32_t nwin = (p.num_req + 63u) / 64u;
        for (uint32_t k = 0; k <= nwin; ++k) {
            const uint32_t base = k == 0u ? first : (k - 1u) * 64u;
            if (k != 0u && base == first) continue;   // scanned in the first pass
            const uint32_t r = base + lane;
            uint32_t rb = 0u, rc = 0u, rs = 0u, rp = 0u;
            if (r < p.num_req) {
                const psk_request_descriptor* d = p.req + r;
                rb = d->row_begin;
                rc = d->row_count;
                rs = d->slot;
                rp = d->prefix_length;
            }
            for (uint32_t R = row_lo; R <= row_hi && first_task < total; ++R) {
                const uint64_t m = __ballot(r < p.num_req && R >= rb && R - rb < rc);
                if (m == 0u) continue;
                const int idx = __builtin_ctzll(m);
                const uint32_t s_ = __builtin_amdgcn_readlane(rs, idx);
                const uint32_t p_ = __builtin_amdgcn_readlane(rp, idx) + (R - __builtin_amdgcn_readlane(rb, idx));
                if (row[0] == R && !found) {
                    slot[0] = s_;
                    pos[0] = p_;
                    found = true;
                }
            }
            if (__all(found || !live[0])) break;
        }
        live[0] = live[0] && found;
        if (live[0] && head[0] == 0u && sub == 0u) {
            const_cast<uint32_t*>(a.row_sequence_slots)[row[0]] = slot[0];
            const_cast<uint32_t*>(a.row_positions)[row[0]] = pos[0];
        }
    }
    uint32_t page[kUnroll], off[kUnroll];
    bool valid[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
        const uint32_t lb = pos[u] / a.page_tokens;
        off[u] = pos[u] - lb * a.page_tokens;
        const bool ok = live[u] && slot[u] < a.max_sequences && lb < a.block_table_stride;
        page[u] = a.block_tables[ok ? (uint64_t)slot[u] * a.block_table_stride + lb : 0u];
        valid[u] = ok;
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
        if (!has_chunk) kw[u] = vw[u] = (u32x4){0u, 0u, 0u, 0u};
        valid[u] = valid[u] && page[u] < a.num_pages;
        const uint64_t dst = (uint64_t)a.layer * a.elems_per_layer +
                             (uint64_t)page[u] * a.elems_per_page +
                             (uint64_t)off[u] * a.elems_per_token + head[u] * D + e0;
        if constexpr (!kFp8) {
            if (valid[u] && has_chunk) {
                *reinterpret_cast<u32x4*>(static_cast<uint16_t*>(p.k_pool) + dst) = kw[u];
                *reinterpret_cast<u32x4*>(static_cast<uint16_t*>(p.v_pool) + dst) = vw[u];
            }
        } else {
            float kx[8], vx[8];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                kx[2 * i] = __uint_as_float(kw[u][i] << 16);
                kx[2 * i + 1] = __uint_as_float(kw[u][i] & 0xFFFF0000u);
                vx[2 * i] = __uint_as_float(vw[u][i] << 16);
                vx[2 * i + 1] = __uint_as_float(vw[u][i] & 0xFFFF0000u);
            }
            // per-head absmax over the L lanes; fmaxf ignores NaN as the
            // reference's fmaxf(k_max, fabsf(kf)) does
            float km = 0.0f, vm = 0.0f;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                km = __builtin_fmaxf(km, __builtin_fabsf(kx[i]));
                vm = __builtin_fmaxf(vm, __builtin_fabsf(vx[i]));
            }
            for (uint32_t o = L >> 1; o >= 1u; o >>= 1) {
                km = __builtin_fmaxf(km, __shfl_xor(km, (int)o, 64));
                vm = __builtin_fmaxf(vm, __shfl_xor(vm, (int)o, 64));
            }
            if (!valid[u]) continue;
            const float k_scale = head_scale(km), v_scale = head_scale(vm);
            if (sub == 0u) {
                const uint64_t si =
                    (((uint64_t)a.layer * a.num_pages + page[u]) * a.page_tokens + off[u]) *
                        a.kv_heads + head[u];
                p.k_scale[si] = k_scale;
                p.v_scale[si] = v_scale;
            }
            if (has_chunk) {
                const u32x2 kc = encode8(kx, k_scale, 1.0f / k_scale, fast_div_ok(k_scale));
                const u32x2 vc = encode8(vx, v_scale, 1.0f / v_scale, fast_div_ok(v_scale));
                __builtin_nontemporal_store(kc, reinterpret_cast<u32x2*>(static_cast<uint8_t*>(p.k_pool) + dst));
                __builtin_nontemporal_store(vc, reinterpret_cast<u32x2*>(static_cast<uint8_t*>(p.v_pool) + dst));
            }
        }
    }
}

// General shapes (any head_dim, unaligned slices): one task group per wave,
// lanes loop over 8-element chunks, element-wise accesses at the edges.
template <bool kFp8>
__global__ __launch_bounds__(256) void kv_append_generic_kernel(const AppendParams p) {
    const psk_kv_append_args& a = p.a;
    const uint32_t L = p.lanes_per_head;
    const uint32_t lane = threadIdx.x & 63u;
    const uint64_t wave_global = ((uint64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    const uint64_t task = wave_global * (64u >> p.log2_lanes) + (lane >> p.log2_lanes);
    const uint32_t sub = lane & (L - 1u);
    const bool live = task < (uint64_t)a.rows * a.kv_heads;
    const uint32_t row = live ? (uint32_t)(task / a.kv_heads) : 0u;
    const uint32_t head = live ? (uint32_t)(task % a.kv_heads) : 0u;
    const uint32_t D = a.head_dim;
    const bool vec = p.vec_ok != 0u;
    bool valid = false;
    uint32_t page = 0, off = 0;
    if (live) {
        const uint32_t slot = a.row_sequence_slots[row];
        const uint32_t pos = a.row_positions[row];
        const uint32_t lb = pos / a.page_tokens;
        off = pos % a.page_tokens;
        if (slot < a.max_sequences && lb < a.block_table_stride) {
            page = a.block_tables[(uint64_t)slot * a.block_table_stride + lb];
            valid = page < a.num_pages;
        }
    }
    const uint16_t* ks = static_cast<const uint16_t*>(a.k_input) + (uint64_t)row * a.k_row_stride +
                         (uint64_t)head * D;
    const uint16_t* vs = static_cast<const uint16_t*>(a.v_input) + (uint64_t)row * a.v_row_stride +
                         (uint64_t)head * D;
    const uint64_t dst = (uint64_t)a.layer * a.elems_per_layer + (uint64_t)page * a.elems_per_page +
                         (uint64_t)off * a.elems_per_token + (uint64_t)head * D;
    if constexpr (!kFp8) {
        if (!valid) return;
        uint16_t* kd = static_cast<uint16_t*>(p.k_pool) + dst;
        uint16_t* vd = static_cast<uint16_t*>(p.v_pool) + dst;
        for (uint32_t c = sub; c < p.chunks; c += L)
            for (uint32_t i = c * 8u; i < c * 8u + 8u && i < D; ++i) {
                kd[i] = ks[i];
                vd[i] = vs[i];
            }
    } else {
        float km = 0.0f, vm = 0.0f;
        float kx[8], vx[8];
        if (valid) {
            for (uint32_t c = sub; c < p.chunks; c += L) {
                load_chunk(ks, c, D, vec, kx);
                load_chunk(vs, c, D, vec, vx);
                for (int i = 0; i < 8; ++i) {
                    km = __builtin_fmaxf(km, __builtin_fabsf(kx[i]));
                    vm = __builtin_fmaxf(vm, __builtin_fabsf(vx[i]));
                }
            }
        }
        for (uint32_t o = L >> 1; o >= 1u; o >>= 1) {
            km = __builtin_fmaxf(km, __shfl_xor(km, (int)o, 64));
            vm = __builtin_fmaxf(vm, __shfl_xor(vm, (int)o, 64));
        }
        if (!valid) return;
        const float k_scale = head_scale(km), v_scale = head_scale(vm);
        if (sub == 0u) {
            const uint64_t si =
                (((uint64_t)a.layer * a.num_pages + page) * a.page_tokens + off) * a.kv_heads + head;
            p.k_scale[si] = k_scale;
            p.v_scale[si] = v_scale;
        }
        uint8_t* kd = static_cast<uint8_t*>(p.k_pool) + dst;
        uint8_t* vd = static_cast<uint8_t*>(p.v_pool) + dst;
        for (uint32_t c = sub; c < p.chunks; c += L) {
            load_chunk(ks, c, D, vec, kx);
            load_chunk(vs, c, D, vec, vx);
            const u32x2 kc = encode8(kx, k_scale, 1.0f / k_scale, fast_div_ok(k_scale));
            const u32x2 vc = encode8(vx, v_scale, 1.0f / v_scale, fast_div_ok(v_scale));
            for (uint32_t i = 0; i < 8u && c * 8u + i < D; ++i) {
                kd[c * 8u + i] = (uint8_t)(kc[i >> 2] >> (8u * (i & 3u)));
                vd[c * 8u + i] = (uint8_t)(vc[i >> 2] >> (8u * (i & 3u)));
            }
        }
    }
}

// ---------------------------------------------------------------- PSQ
// One lane = one task = one 32-value block of one (row, K|V, kv head): the
// block's 64 input bytes reach that lane (four 16 B loads, or the wave's 4 KB
// staged in LDS by whole-line DMAs, see the kernel), and every reduction of
// the block (amax, the LSQ1 sums) stays inside the lane. Tasks are ordered
// (row, K|V, head, block): consecutive lanes read consecutive blocks and
// write consecutive code blocks.
struct PsqAppendParams {
    psk_kv_append_args a;
    uint8_t* k_code;
    uint8_t* v_code;
    uint16_t* k_scale;
    uint16_t* v_scale;
    uint32_t bph;           // blocks per head
    uint32_t head_blocks;   // kv_heads * bph
    uint32_t tasks;         // rows * 2 * head_blocks (< 2^31, checked by the launcher)
    uint32_t vec_in;        // 16 B input loads legal
    uint32_t dma_in;        // vec_in and 64 % head_blocks == 0: whole-line input DMAs legal
    uint32_t vec_out;       // 16 B code stores legal
    FastDiv div_head_blocks;
    FastDiv div_page_tokens;
};

__device__ __forceinline__ uint32_t fastdiv(uint32_t n, const FastDiv& f) {
    const uint32_t t = __umulhi(n, f.m);
    return (t + ((n - t) >> f.s1)) >> f.s2;
}

// psq_bf16_round (psq4_kv.h:9-18): round to bf16 by adding 0x7FFF plus the
// kept LSB, then truncating.
__device__ __forceinline__ float psq_bf16_round(float v) {
    uint32_t u = __float_as_uint(v);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return __uint_as_float(u & 0xFFFF0000u);
}

// cb10_encode (psq_device.h:22-35): magnitude index of a = |x| * inv against
// the midpoints 0.5 1.5 2.5 3.5 5 7 9 (7 above 9 and for NaN), sign in bit 3.
// Computed without comparisons from k = ceil(2a), see below. Equal to the
// reference's chain for every float a >= 0, for every positive bf16 scale
// (subnormals included) over a spread of x, and for 2^26 random (x, bf16
// scale) pairs, checked on the CPU (tests/native/cb10_branchless.c).
//
// The code boundaries a > 0.5, 1.5, 2.5, 3.5, 5, 7, 9 are thresholds on
// k = ceil(2a): the code is the number of T in {2, 4, 6, 8, 11, 15, 19} with
// k >= T. With n = floor(max(-2a, -19)) = -min(k, 19) (NaN and Inf give -19,
// a max operand that is NaN yields the other), the 64-bit shift of the pair
// {lo = 0, hi = H} by n mod 64 = 64 - k (0 for k = 0) keeps in its low dword
// exactly the bits 32 - T of H with k >= T, and the code is their popcount:
// multiply, max, floor-convert, shift, bit count (the count's accumulator
// adds the sign). -2a is |x| * (-2 * inv) where -2 * inv is finite, which
// equals (|x| * inv) * -2 up to a subnormal a (code 0 either way); bf16
// subnormal scales s <= 2^-127 have a finite 1/s but an infinite 2/s, and a
// wave with such a block doubles after the product instead (exact whenever a
// is finite, overflowing only where a > 9 already gives 7).
constexpr uint32_t kCb10H = (1u << 30) | (1u << 28) | (1u << 26) | (1u << 24) | (1u << 21) |
                           (1u << 17) | (1u << 13);

__device__ __forceinline__ uint32_t cb10_bits(float y) {
    // floor and convert in one instruction (the compiler emits two for
    // (int)floorf); y is in [-19, 0], where a flushed denormal input gives
    // n = 0 instead of -1, both code 0
    int n;
    asm("v_cvt_flr_i32_f32 %0, %1" : "=v"(n) : "v"(y));
    return (uint32_t)(((uint64_t)kCb10H << 32) >> ((uint32_t)n & 63u));
}

// Codes of the 32 values for scale s (all 0 unless s > 0): PSQ4 cb10 codes of
// x * (1/s), PSQ8 SATFINITE E4M3 codes of x * (1/s) packed 4 per dword.
//
// kNoNaN (PSQ4, the LSQ1 refit): s > 0 implies the block has no NaN (a NaN
// made the fitted scale 0). Then a wave whose blocks all have s == 0 or
// -2 amax / s >= -32 drops the clamp: every n = floor(-2a) is then in [-32, 0]
// (a shift of 64 - k >= 32 keeps the low dword right up to k = 32); with
// s == 0, -2a is -inf or NaN, whose conversion (INT_MIN or 0) shifts by 0 and
// gives code 0.
//
// 1/s: for a bf16 s in [2^-126, 2^126] (every lane of the wave), the hardware
// reciprocal r (within one ulp of 1/s) refined by e = fma(-s, r, 1),
// fma(e, r, r) is the correctly rounded 1/s, checked on the CPU for every such
// bf16 s and each of the three floats within one ulp of 1/s
// (tests/native/rcp_refine.c); other scales divide.
__device__ __forceinline__ float bf16_scale_reciprocal(float s) {
    if (__all(s >= 0x1p-126f && s <= 0x1p126f)) {
        const float r = __builtin_amdgcn_rcpf(s);
        return __builtin_fmaf(__builtin_fmaf(-s, r, 1.0f), r, r);
    }
    return 1.0f / s;
}

// PSQ4 LSQ1 fit, first pass: the decoded magnitude q (fp32) of each value's
// cb10 code at scale s, looked up by n = floor(-2a) in a 33-entry LDS table
// (q_lut[32 + n] = the cb10 value of code(k = -n)). Only |x| q and q q use
// them: x q with the signed q equals |x| |q| bit for bit (a product's zero
// sign aside, which cannot change a sum with a nonzero term, nor the scale 0
// of one without), so no signs and no zeroing for s == 0 (the fit then ends
// at scale 0 either way: every x is zero or NaN), and a NaN value's q does
// not matter (its |x| q is NaN whatever q is, and so is the fitted scale,
// which becomes 0). n stays in [-32, 0] on every path: without the clamp
// where the wave's blocks all have -2 amax / s >= -32 (or s == 0, taken as
// -2/s = 0, n = 0), else clamped at -19.
__device__ __forceinline__ void psq4_first_pass_q(const float (&x)[32], float s, float amax,
                                                  const float* q_lut, float (&q)[32]) {
#pragma clang fp contract(off)
    const float inv = bf16_scale_reciprocal(s);
    const bool sp = s > 0.0f;
    const float m2 = inv * -2.0f;
    const float inv2 = sp ? m2 : 0.0f;
    auto look = [&](float y) __attribute__((always_inline)) {
        int n;
        asm("v_cvt_flr_i32_f32 %0, %1" : "=v"(n) : "v"(y));
        return q_lut[32 + n];
    };
    if (__all(!sp || amax * inv2 >= -32.0f)) {
#pragma unroll
        for (int i = 0; i < 32; ++i) q[i] = look(__builtin_fabsf(x[i]) * inv2);
    } else if (__all(!sp || __builtin_isfinite(m2))) {
#pragma unroll
        for (int i = 0; i < 32; ++i) q[i] = look(__builtin_fmaxf(__builtin_fabsf(x[i]) * inv2, -19.0f));
    } else {
#pragma unroll
        for (int i = 0; i < 32; ++i) q[i] = look(__builtin_fmaxf((__builtin_fabsf(x[i]) * inv) * -2.0f, -19.0f));
    }
}

template <bool kPsq4, bool kNoNaN = false>
__device__ __forceinline__ void psq_codes(const float (&x)[32], float s, float amax, uint32_t (&c)[32]) {
#pragma clang fp contract(off)
    const float inv = bf16_scale_reciprocal(s);
    if constexpr (kPsq4) {
        const float inv2 = inv * -2.0f;   // -inf for s == 0
        if constexpr (kNoNaN) {
            const bool sp = s > 0.0f;
            const uint32_t sg = sp ? 8u : 0u;   // the sign code bit, if any
            if (__all(!sp || amax * inv2 >= -32.0f)) {
#pragma unroll
                for (int i = 0; i < 32; ++i) {
                    int n;
                    asm("v_cvt_flr_i32_f32 %0, %1" : "=v"(n) : "v"(__builtin_fabsf(x[i]) * inv2));
                    c[i] = (uint32_t)__builtin_popcount(
                               (uint32_t)((uint64_t{kCb10H} << 32) >> ((uint32_t)n & 63u))) +
                           (x[i] < 0.0f ? sg : 0u);
                }
                return;
            }
        }
        // s == 0: every magnitude 0 through the clamp (lo = +0) and no signs
        const bool kp = s > 0.0f;
        const float lo = kp ? -19.0f : 0.0f;
        const bool pre = !kp || __builtin_isfinite(inv2);   // -inf harmless under lo = +0
        const uint32_t sg = kp ? 8u : 0u;
        if (__all(pre)) {
#pragma unroll
            for (int i = 0; i < 32; ++i)
                c[i] = (uint32_t)__builtin_popcount(
                           cb10_bits(__builtin_fmaxf(__builtin_fabsf(x[i]) * inv2, lo))) +
                       (x[i] < 0.0f ? sg : 0u);
        } else {
#pragma unroll
            for (int i = 0; i < 32; ++i)
                c[i] = (uint32_t)__builtin_popcount(
                           cb10_bits(__builtin_fmaxf((__builtin_fabsf(x[i]) * inv) * -2.0f, lo))) +
                       (x[i] < 0.0f ? sg : 0u);
        }
    } else {
        const uint32_t keep = s > 0.0f ? 0xFFFFFFFFu : 0u;   // all codes 0 unless s > 0
#pragma unroll
        for (int i = 0; i < 32; i += 4) {
            const uint32_t w = e4m3_encode_pair(x[i + 2] * inv, x[i + 3] * inv,
                                                e4m3_encode_pair(x[i] * inv, x[i + 1] * inv, 0u, false),
                                                true);
            c[i >> 2] = w & keep;   // c[0..7]: packed dwords
        }
    }
}

// Sum of the products a[j] * b[j], j = 0..31, in the order of the reference's
// 32-lane xor butterfly (x += shfl_xor(x, o) for o = 16, 8, 4, 2, 1;
// kv_append.hip:293-299): the tree (p[j] + p[j^16]), then ^8, ^4, ^2, ^1 on
// the partial sums. kFma: every product is exact in fp32 and none is negative,
// so the first level p[j] + p[j + 16] is one FMA onto the second product (the
// exact sum rounded once equals the add of the two rounded products, and an
// overflowing product gives inf both ways; with mixed signs an overflow could
// give inf where the adds give NaN).
template <bool kFma>
__device__ __forceinline__ float butterfly_dot32(const float (&a)[32], const float (&b)[32]) {
#pragma clang fp contract(off)
    float v[16];
#pragma unroll
    for (int j = 0; j < 16; ++j)
        v[j] = kFma ? __builtin_fmaf(a[j], b[j], a[j + 16] * b[j + 16]) : a[j] * b[j] + a[j + 16] * b[j + 16];
#pragma unroll
    for (int o = 8; o >= 1; o >>= 1)
#pragma unroll
        for (int j = 0; j < o; ++j) v[j] = v[j] + v[j + o];
    return v[0];
}

template <bool kPsq4, bool kLsq1>
__global__ __launch_bounds__(256) void kv_append_psq_kernel(const PsqAppendParams p) {
#pragma clang fp contract(off)
    const psk_kv_append_args& a = p.a;
    // PSQ4 LSQ1: q_lut[j] = the cb10 value of k = 32 - j (k = ceil(2a))
    __shared__ float q_lut[kPsq4 && kLsq1 ? 33 : 1];
    if constexpr (kPsq4 && kLsq1) {
        if (threadIdx.x < 33u) {
            const uint32_t k = 32u - threadIdx.x;
            const uint32_t code = k == 0u ? 0u : (uint32_t)__builtin_popcount(kCb10H >> (32u - k));
            q_lut[threadIdx.x] = (float)(code < 5u ? code : 2u * code - 4u);
        }
        __syncthreads();
    }
    // MaxAbs with dma_in: the wave's 64 blocks (whole (row, K|V) input
    // segments of head_blocks x 64 B) reach LDS by four 16 B-per-lane DMAs,
    // instruction i lane l = chunk m = 64i + l of the wave's 4 KB (block m/4,
    // quarter m%4), so every instruction reads whole 128 B lines; lane l then
    // reads its block at +64l. The chunk's address is its block's input
    // address, taken from the lane that owns the block. Lanes past the last
    // task issue nothing. (Measured at 2^16 rows: PSQ8 MaxAbs 82.5 -> 70.5 us,
    // PSQ4 MaxAbs 68.2 -> 67.5 us; both LSQ1 encoders lose 1-5 us that way: the
    // wait for the whole 4 KB exposes the latency their longer arithmetic hid
    // behind the per-lane 64 B loads.)
    constexpr bool kDmaIn = !kLsq1;
    __shared__ __align__(16) uint8_t in_lds[kDmaIn ? 4 * 4096 : 16];
    const uint32_t lane = threadIdx.x & 63u;
    uint8_t* const wst = in_lds + (kDmaIn ? (threadIdx.x >> 6) * 4096u : 0u);
    const uint32_t task = blockIdx.x * 256u + threadIdx.x;
    const bool live = task < p.tasks;
    const uint32_t rest = fastdiv(live ? task : 0u, p.div_head_blocks);
    const uint32_t hb = (live ? task : 0u) - rest * p.head_blocks;
    const bool is_v = (rest & 1u) != 0u;
    const uint32_t row = rest >> 1;
    const uint16_t* src = static_cast<const uint16_t*>(is_v ? a.v_input : a.k_input) +
                          (uint64_t)row * (is_v ? a.v_row_stride : a.k_row_stride) +
                          (uint64_t)hb * 32u;
    if (kDmaIn && p.dma_in) {
        // tasks left from the wave's first (0 for a wave wholly past the end:
        // it issues nothing, so no DMA outlives an exited wave)
        const uint32_t wfirst = blockIdx.x * 256u + (threadIdx.x & ~63u);
        const uint32_t wlast = wfirst < p.tasks ? p.tasks - wfirst : 0u;
        const uint64_t sp = reinterpret_cast<uint64_t>(src);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t b = 16u * (uint32_t)i + (lane >> 2);
            const uint32_t lo = (uint32_t)__shfl((int)(uint32_t)sp, (int)b, 64);
            const uint32_t hi = (uint32_t)__shfl((int)(uint32_t)(sp >> 32), (int)b, 64);
            if (b < wlast)
                load_lds<16, kCpolStream>(reinterpret_cast<const uint8_t*>(((uint64_t)hi << 32) | lo) + 16u * (lane & 3u),
                                          wst + 1024 * i);
        }
    }
    if (!live) return;

    // row -> (page, offset), the reference skip rules (kv_append.hip:335-360)
    const uint32_t slot = a.row_sequence_slots[row];
    const uint32_t pos = a.row_positions[row];
    // input loads go out before the block-table load, which waits on slot
    float x[32];
    if (p.vec_in) {
        u32x4 w[4];
        if (kDmaIn && p.dma_in) {
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#pragma unroll
            for (int i = 0; i < 4; ++i) w[i] = *reinterpret_cast<const u32x4*>(wst + 64u * lane + 16 * i);
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) w[i] = reinterpret_cast<const u32x4*>(src)[i];
        }
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            x[2 * i] = __uint_as_float(w[i >> 2][i & 3] << 16);
            x[2 * i + 1] = __uint_as_float(w[i >> 2][i & 3] & 0xFFFF0000u);
        }
    } else {
#pragma unroll
        for (int i = 0; i < 32; ++i) x[i] = bf16_bits_to_f32(src[i]);
    }
    if (slot >= a.max_sequences) return;
    const uint32_t lb = fastdiv(pos, p.div_page_tokens);
    if (lb >= a.block_table_stride) return;
    const uint32_t page = a.block_tables[(uint64_t)slot * a.block_table_stride + lb];
    if (page >= a.num_pages) return;
    const uint32_t off = pos - lb * a.page_tokens;

    // block amax (order-free; fmaxf drops NaN as the reference's does)
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 32; ++i) amax = __builtin_fmaxf(amax, __builtin_fabsf(x[i]));
    float s = amax > 0.0f ? psq_bf16_round(amax * (kPsq4 ? 0.1f : (1.0f / 448.0f))) : 0.0f;
    uint32_t c[32];
    [[maybe_unused]] float qf[32];   // PSQ4 LSQ1: the first pass's decoded magnitudes
    if constexpr (kPsq4 && kLsq1)
        psq4_first_pass_q(x, s, amax, q_lut, qf);
    else
        psq_codes<kPsq4>(x, s, amax, c);

    if constexpr (kLsq1) {
        // num = sum x q, den = sum q q over the decoded codes, in the
        // reference's butterfly order; s1 = bf16(num / den), then re-encode
        // The products x q and q q are exact in fp32: x is bf16 (8 significant
        // bits, granularity 2^-133), q an E4M3 value (4 bits, granularity
        // 2^-9), so a product has at most 12 significant bits on a grid of
        // 2^-142, above fp32's 2^-149 (overflow gives inf either way).
        float xa[32];
        if constexpr (!kPsq4) {
#pragma unroll
            for (int i = 0; i < 32; i += 4) {
                // PSQ8: 4 E4M3 codes -> f32 by the hardware conversion
                const f32x2 q01 = __builtin_amdgcn_cvt_pk_f32_fp8(c[i >> 2], false);
                const f32x2 q23 = __builtin_amdgcn_cvt_pk_f32_fp8(c[i >> 2], true);
                qf[i] = q01[0];
                qf[i + 1] = q01[1];
                qf[i + 2] = q23[0];
                qf[i + 3] = q23[1];
            }
        }
#pragma unroll
        for (int i = 0; i < 32; ++i) xa[i] = kPsq4 ? __builtin_fabsf(x[i]) : x[i];
        const float num = butterfly_dot32<kPsq4>(xa, qf);   // PSQ8: x q has signs
        // PSQ4: every q q and partial sum is an integer below 2^24, so the
        // butterfly's float sum is the exact sum in any order
        float den;
        if constexpr (kPsq4) {
            den = 0.0f;
#pragma unroll
            for (int i = 0; i < 32; ++i) den = __builtin_fmaf(qf[i], qf[i], den);
        } else {
            den = butterfly_dot32<true>(qf, qf);
        }
        const float sl = den > 0.0f ? num / den : 0.0f;
        float s1 = psq_bf16_round(sl);
        if (!(s1 > 0.0f)) s1 = 0.0f;
        psq_codes<kPsq4, true>(x, s1, amax, c);
        s = s1;
    }

    const uint64_t bi = ((((uint64_t)a.layer * a.num_pages + page) * a.page_tokens + off) *
                         a.kv_heads) * p.bph + hb;
    uint8_t* code = is_v ? p.v_code : p.k_code;
    if constexpr (kPsq4) {
        // byte j = code j | code j+16 << 4 (psq4_pack_codes, psq4_kv.h:73-77);
        // every code is below 16 (a count of 7 bits plus the sign 8)
        u32x4 w;
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            uint32_t v = c[4 * d] | (c[4 * d + 16] << 4);
#pragma unroll
            for (int b = 1; b < 4; ++b) {
                const int j = 4 * d + b;
                v |= (c[j] | (c[j + 16] << 4)) << (8 * b);
            }
            w[d] = v;
        }
        uint8_t* dst = code + bi * 16u;
        if (p.vec_out) {
            *reinterpret_cast<u32x4*>(dst) = w;
        } else {
#pragma unroll
            for (int i = 0; i < 16; ++i) dst[i] = (uint8_t)(w[i >> 2] >> (8 * (i & 3)));
        }
    } else {
        uint8_t* dst = code + bi * 32u;
        if (p.vec_out) {
            reinterpret_cast<u32x4*>(dst)[0] = (u32x4){c[0], c[1], c[2], c[3]};
            reinterpret_cast<u32x4*>(dst)[1] = (u32x4){c[4], c[5], c[6], c[7]};
        } else {
#pragma unroll
            for (int i = 0; i < 32; ++i) dst[i] = (uint8_t)(c[i >> 2] >> (8 * (i & 3)));
        }
    }
    (is_v ? p.v_scale : p.k_scale)[bi] = (uint16_t)(__float_as_uint(s) >> 16);
}

hipError_t validate(const psk_kv_append_args& c, const void* k_pool, const void* v_pool) {
    if (c.rows == 0u || c.head_dim == 0u || c.kv_heads == 0u) return hipErrorInvalidValue;
    if (c.page_tokens == 0u || c.block_table_stride == 0u || c.num_pages == 0u)
        return hipErrorInvalidValue;
    if (c.k_input == nullptr || c.v_input == nullptr || c.row_sequence_slots == nullptr ||
        c.row_positions == nullptr || c.block_tables == nullptr || k_pool == nullptr ||
        v_pool == nullptr)
        return hipErrorInvalidValue;
    return hipSuccess;
}

AppendParams make_params(const psk_kv_append_args& c, void* k_pool, void* v_pool, float* ks,
                         float* vs, uint32_t pool_elem_bytes) {
    AppendParams p{};
    p.a = c;
    p.k_pool = k_pool;
    p.v_pool = v_pool;
    p.k_scale = ks;
    p.v_scale = vs;
    p.chunks = (c.head_dim + 7u) / 8u;
    uint32_t L = 1, lg = 0;
    while (L < p.chunks && L < 64u) {
        L <<= 1;
        ++lg;
    }
    p.lanes_per_head = L;
    p.log2_lanes = lg;
    // 16 B input loads and 16 B (bf16) / 8 B (fp8) pool stores need every
    // head slice start aligned: element offsets multiple of 8, base pointers
    // aligned to the access size.
    const uintptr_t ka = reinterpret_cast<uintptr_t>(c.k_input);
    const uintptr_t va = reinterpret_cast<uintptr_t>(c.v_input);
    const uintptr_t kp = reinterpret_cast<uintptr_t>(k_pool);
    const uintptr_t vp = reinterpret_cast<uintptr_t>(v_pool);
    const uintptr_t store_align = pool_elem_bytes == 2u ? 16u : 8u;
    const bool ok = (c.head_dim % 8u == 0u) && (c.k_row_stride % 8u == 0u) &&
                    (c.v_row_stride % 8u == 0u) && (c.elems_per_token % 8u == 0u) &&
                    (c.elems_per_page % 8u == 0u) && (c.elems_per_layer % 8u == 0u) &&
                    (ka % 16u == 0u) && (va % 16u == 0u) && (kp % store_align == 0u) &&
                    (vp % store_align == 0u);
    p.vec_ok = ok ? 1u : 0u;
    return p;
}

template <bool kFp8>
hipError_t launch(const AppendParams& p, hipStream_t stream) {
    const uint64_t tasks = (uint64_t)p.a.rows * p.a.kv_heads;
    const uint64_t tasks_per_wave = 64u >> p.log2_lanes;
    const uint64_t groups = (tasks + tasks_per_wave - 1) / tasks_per_wave;
    const bool fast = p.vec_ok != 0u && p.chunks <= p.lanes_per_head && tasks < 0xFFFFFFFFull;
    const int U = fast && tasks >= kTwoGroupTasks ? 2 : 1;
    const uint64_t waves = (groups + U - 1) / U;
    const uint64_t blocks = (waves + 3) / 4;
    if (blocks > 0x7FFFFFFFull) return hipErrorInvalidValue;
    if (fast && U == 2)
        hipLaunchKernelGGL((kv_append_fast_kernel<kFp8, false, 2>), dim3((uint32_t)blocks), dim3(256), 0, stream, p);
    else if (fast)
        hipLaunchKernelGGL((kv_append_fast_kernel<kFp8, false, 1>), dim3((uint32_t)blocks), dim3(256), 0, stream, p);
    else
        hipLaunchKernelGGL(kv_append_generic_kernel<kFp8>, dim3((uint32_t)blocks), dim3(256), 0, stream,
                           p);
    return hipGetLastError();
}

// Row metadata from request descriptors fused into the append (fast path);
// other shapes run the row-metadata launch and then the plain append.
template <bool kFp8>
hipError_t launch_req(AppendParams p, const psk_request_descriptor* req, uint32_t num_req,
                      hipStream_t stream) {
    const uint64_t tasks = (uint64_t)p.a.rows * p.a.kv_heads;
    const uint64_t tasks_per_wave = 64u >> p.log2_lanes;
    const bool fast = p.vec_ok != 0u && p.chunks <= p.lanes_per_head && tasks < 0xFFFFFFFFull;
    if (!fast) {
        const int e = psk_prepare_row_metadata(req, num_req, p.a.rows, const_cast<uint32_t*>(p.a.row_sequence_slots),
                                               const_cast<uint32_t*>(p.a.row_positions), stream);
        if (e != hipSuccess) return static_cast<hipError_t>(e);
        return launch<kFp8>(p, stream);
    }
    p.req = req;
    p.num_req = num_req;
    const uint64_t waves = (tasks + tasks_per_wave - 1) / tasks_per_wave;
    const uint64_t blocks = (waves + 3) / 4;
    if (blocks > 0x7FFFFFFFull) return hipErrorInvalidValue;
    hipLaunchKernelGGL((kv_append_fast_kernel<kFp8, true, 1>), dim3((uint32_t)blocks), dim3(256), 0, stream, p);
    return hipGetLastError();
}

hipError_t launch_psq(const psk_kv_append_args& c, bool psq4, uint8_t* kc, uint8_t* vc,
                      uint16_t* ks, uint16_t* vs, uint32_t bph, uint32_t estimator,
                      hipStream_t stream) {
    // the reference's checks (kv_append.hip:578-590); any blocks_per_head
    // >= 1 runs here (the reference's kernel needs exactly 8)
    if (c.rows == 0u || c.head_dim == 0u || c.kv_heads == 0u) return hipErrorInvalidValue;
    if (c.page_tokens == 0u || c.block_table_stride == 0u || c.num_pages == 0u)
        return hipErrorInvalidValue;
    if (c.k_input == nullptr || c.v_input == nullptr || c.row_sequence_slots == nullptr ||
        c.row_positions == nullptr || c.block_tables == nullptr || kc == nullptr || vc == nullptr ||
        ks == nullptr || vs == nullptr)
        return hipErrorInvalidValue;
    if (bph == 0u || c.head_dim != 32u * bph) return hipErrorNotSupported;
    if (estimator > 1u) return hipErrorInvalidValue;
    PsqAppendParams p{};
    p.a = c;
    p.k_code = kc;
    p.v_code = vc;
    p.k_scale = ks;
    p.v_scale = vs;
    p.bph = bph;
    p.head_blocks = c.kv_heads * bph;
    p.div_head_blocks = make_fastdiv(p.head_blocks);
    p.div_page_tokens = make_fastdiv(c.page_tokens);
    const uint64_t tasks = (uint64_t)c.rows * 2u * p.head_blocks;
    if (tasks >= (1ull << 31)) return hipErrorInvalidValue;
    p.tasks = (uint32_t)tasks;
    auto al = [](const void* ptr, uintptr_t n) { return reinterpret_cast<uintptr_t>(ptr) % n == 0u; };
    p.vec_in = (c.k_row_stride % 8u == 0u && c.v_row_stride % 8u == 0u && al(c.k_input, 16) &&
                al(c.v_input, 16)) ? 1u : 0u;
    p.vec_out = (al(kc, 16) && al(vc, 16)) ? 1u : 0u;
    p.dma_in = (p.vec_in && p.head_blocks >= 2u && 64u % p.head_blocks == 0u) ? 1u : 0u;
    const uint64_t blocks = (tasks + 255u) / 256u;
    if (blocks == 0u || blocks > 0x7FFFFFFFull) return hipErrorInvalidValue;
    const dim3 grid((uint32_t)blocks);
    if (psq4) {
        if (estimator == 1u)
            hipLaunchKernelGGL((kv_append_psq_kernel<true, true>), grid, dim3(256), 0, stream, p);
        else
            hipLaunchKernelGGL((kv_append_psq_kernel<true, false>), grid, dim3(256), 0, stream, p);
    } else {
        if (estimator == 1u)
            hipLaunchKernelGGL((kv_append_psq_kernel<false, true>), grid, dim3(256), 0, stream, p);
        else
            hipLaunchKernelGGL((kv_append_psq_kernel<false, false>), grid, dim3(256), 0, stream, p);
    }
    return hipGetLastError();
}

}  // namespace
}  // namespace psk

// ---------------------------------------------------------------- C-ABI
extern "C" int psk_kv_append_bf16(const psk_kv_append_args* a, void* k_pool, void* v_pool,
                                  void* stream) {
    if (a == nullptr) return hipErrorInvalidValue;
    const hipError_t e = psk::validate(*a, k_pool, v_pool);
    if (e != hipSuccess) return e;
    return psk::launch<false>(psk::make_params(*a, k_pool, v_pool, nullptr, nullptr, 2u),
                              static_cast<hipStream_t>(stream));
}

extern "C" int psk_kv_append_fp8_e4m3(const psk_kv_append_args* a, void* k_pool, void* v_pool,
                                      float* k_scale_pool, float* v_scale_pool, void* stream) {
    if (a == nullptr) return hipErrorInvalidValue;
    hipError_t e = psk::validate(*a, k_pool, v_pool);
    if (e != hipSuccess) return e;
    if (k_scale_pool == nullptr || v_scale_pool == nullptr) return hipErrorInvalidValue;
    return psk::launch<true>(
        psk::make_params(*a, k_pool, v_pool, k_scale_pool, v_scale_pool, 1u),
        static_cast<hipStream_t>(stream));
}

extern "C" int psk_kv_append_bf16_from_requests(const psk_kv_append_args* a,
                                                const psk_request_descriptor* requests,
                                                uint32_t num_requests, void* k_pool, void* v_pool,
                                                void* stream) {
    if (a == nullptr || requests == nullptr || num_requests == 0u) return hipErrorInvalidValue;
    const hipError_t e = psk::validate(*a, k_pool, v_pool);
    if (e != hipSuccess) return e;
    return psk::launch_req<false>(psk::make_params(*a, k_pool, v_pool, nullptr, nullptr, 2u), requests,
                                  num_requests, static_cast<hipStream_t>(stream));
}

extern "C" int psk_kv_append_fp8_e4m3_from_requests(const psk_kv_append_args* a,
                                                    const psk_request_descriptor* requests,
                                                    uint32_t num_requests, void* k_pool, void* v_pool,
                                                    float* k_scale_pool, float* v_scale_pool,
                                                    void* stream) {
    if (a == nullptr || requests == nullptr || num_requests == 0u) return hipErrorInvalidValue;
    hipError_t e = psk::validate(*a, k_pool, v_pool);
    if (e != hipSuccess) return e;
    if (k_scale_pool == nullptr || v_scale_pool == nullptr) return hipErrorInvalidValue;
    return psk::launch_req<true>(psk::make_params(*a, k_pool, v_pool, k_scale_pool, v_scale_pool, 1u),
                                 requests, num_requests, static_cast<hipStream_t>(stream));
}

extern "C" int psk_kv_append_psq4(const psk_kv_append_args* a, uint8_t* k_code_pool,
                                  uint8_t* v_code_pool, uint16_t* k_scale_pool,
                                  uint16_t* v_scale_pool, uint32_t blocks_per_head,
                                  uint32_t estimator, void* stream) {
    if (a == nullptr) return hipErrorInvalidValue;
    return psk::launch_psq(*a, true, k_code_pool, v_code_pool, k_scale_pool, v_scale_pool,
                           blocks_per_head, estimator, static_cast<hipStream_t>(stream));
}

extern "C" int psk_kv_append_psq8(const psk_kv_append_args* a, uint8_t* k_code_pool,
                                  uint8_t* v_code_pool, uint16_t* k_scale_pool,
                                  uint16_t* v_scale_pool, uint32_t blocks_per_head,
                                  uint32_t estimator, void* stream) {
    if (a == nullptr) return hipErrorInvalidValue;
    return psk::launch_psq(*a, false, k_code_pool, v_code_pool, k_scale_pool, v_scale_pool,
                           blocks_per_head, estimator, static_cast<hipStream_t>(stream));
}

// ------------------------------------------------- reference C++ signatures
namespace ps::kernel {

hipError_t launch_kv_append_bf16(const KvAppendCommonArgs& common, bf16_t* k_pool,
                                 bf16_t* v_pool, hipStream_t stream) {
    return static_cast<hipError_t>(psk_kv_append_bf16(
        reinterpret_cast<const psk_kv_append_args*>(&common), k_pool, v_pool, stream));
}

hipError_t launch_kv_append_fp8_e4m3(const KvAppendCommonArgs& common,
                                     ::ps::qwen35::fp8e4m3_storage_t* k_pool,
                                     ::ps::qwen35::fp8e4m3_storage_t* v_pool,
                                     float* k_scale_pool, float* v_scale_pool,
                                     hipStream_t stream) {
    return static_cast<hipError_t>(
        psk_kv_append_fp8_e4m3(reinterpret_cast<const psk_kv_append_args*>(&common), k_pool,
                               v_pool, k_scale_pool, v_scale_pool, stream));
}

hipError_t launch_kv_append_psq4(const KvAppendCommonArgs& common, uint8_t* k_code_pool,
                                 uint8_t* v_code_pool, bf16_t* k_scale_pool, bf16_t* v_scale_pool,
                                 uint32_t blocks_per_head,
                                 ::ps::qwen35::Psq4ScaleEstimator estimator, hipStream_t stream) {
    return static_cast<hipError_t>(psk_kv_append_psq4(
        reinterpret_cast<const psk_kv_append_args*>(&common), k_code_pool, v_code_pool,
        reinterpret_cast<uint16_t*>(k_scale_pool), reinterpret_cast<uint16_t*>(v_scale_pool),
        blocks_per_head, static_cast<uint32_t>(estimator), stream));
}

hipError_t launch_kv_append_psq8(const KvAppendCommonArgs& common, uint8_t* k_code_pool,
                                 uint8_t* v_code_pool, bf16_t* k_scale_pool, bf16_t* v_scale_pool,
                                 uint32_t blocks_per_head,
                                 ::ps::qwen35::Psq8ScaleEstimator estimator, hipStream_t stream) {
    return static_cast<hipError_t>(psk_kv_append_psq8(
        reinterpret_cast<const psk_kv_append_args*>(&common), k_code_pool, v_code_pool,
        reinterpret_cast<uint16_t*>(k_scale_pool), reinterpret_cast<uint16_t*>(v_scale_pool),
        blocks_per_head, static_cast<uint32_t>(estimator), stream));
}

}  // namespace ps::kernel
