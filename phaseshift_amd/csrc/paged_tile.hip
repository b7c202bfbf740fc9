// Multi-row paged attention tiles (speculative-verify blocks, chunked prefill)
// over BF16 or FP8 E4M3 KV pages, gfx950.
//
// Reference behaviour restated (file:line in the reference repository):
//   tile = rows of one sequence (slot of the tile's first row), causal rule
//   page_start + t < pos_r + 1 per row                  paged_prefill.hip:152-164,342-352
//   FP8: s = (q.dec(k))*k_scale*scale, acc += (p*v_scale)*dec(v)
//                                                        paged_prefill.hip:586-825
//   launcher validation                                  paged_prefill.hip:437-459
//
// MI355X design. Workgroup = (16-row tile, kv_head, split); one wave per query
// head of the GQA group. The 16 rows of the tile are the N=16 side of
// v_mfma_f32_16x16x32_bf16, so each lane owns one row's causal limit and
// softmax state; K/V chunks (32 tokens) are staged once in LDS and read by all
// q_per_kv waves. Waves own disjoint (row, head) outputs, so there is no
// cross-wave merge; split-K writes the decode kernel's partial layout and the
// same combine kernel finishes it.
#include "device_common.h"

#include <phaseshift_kv/paged_attention.h>

namespace psk {
namespace {

using ps::kernel::kPagedAttentionHeadLimit;

constexpr int kTileRows = 16;
constexpr int kMaxTileWaves = 8;   // q_per_kv <= 8 (one head per wave)
constexpr uint32_t kMaxTileSplits = 1024;

// Explicit tiles (row start, row count <= 16) passed by value in the kernel
// arguments; n_tiles == 0 means the implicit windows [16t, 16t+16).
constexpr uint32_t kInlineTiles = 256;

struct TileParams {
    psk_paged_attention_args a;
    uint32_t n_tiles;
    uint32_t tile_begin[kInlineTiles];
    uint8_t tile_rows[kInlineTiles];
    const uint8_t* k_pool;
    const uint8_t* v_pool;
    const float* k_scale;
    const float* v_scale;
    float* partials;          // nullptr: write the output directly
    uint32_t splits;
    uint32_t pages_per_split; // > 0 whenever splits > 1
    float scale_log2;
};

typedef __attribute__((ext_vector_type(2))) int i32x2;
typedef __attribute__((ext_vector_type(4))) short i16x4;
typedef __attribute__((address_space(3))) i32x2 lds_i32x2;
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;

__device__ __forceinline__ i32x2 tr8(const uint8_t* p) {
    return __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_i32x2*)(p));
}
__device__ __forceinline__ i16x4 tr16(const uint8_t* p) {
    return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(p));
}

__device__ __forceinline__ bf16x8 q8(const uint16_t* q, bool ok) {
    u32x4 r = {0u, 0u, 0u, 0u};
    if (ok) {
#pragma unroll
        for (int i = 0; i < 4; ++i) r[i] = (uint32_t)q[2 * i] | ((uint32_t)q[2 * i + 1] << 16);
    }
    return __builtin_bit_cast(bf16x8, r);
}

template <int KVB, int D>
__global__ __launch_bounds__(kMaxTileWaves * 64) void paged_tile_kernel(const TileParams p) {
    constexpr int CT = 32;               // tokens per chunk (two 16-token halves)
    constexpr int TB = D * KVB;          // bytes of one token's head slice
    constexpr int ROW = TB + 16;         // padded LDS row
    constexpr int NL = TB / 64;          // 16 B pieces per lane per half
    constexpr int NS = D / 32;           // K-steps of QK^T
    constexpr int NDB = D / 16;          // 16-dim output blocks
    constexpr int PIECES = CT * TB / 16; // 16 B pieces of one K (or V) chunk

    __shared__ __align__(16) uint8_t k_lds[CT * ROW];
    __shared__ __align__(16) uint8_t v_lds[CT * ROW];
    __shared__ float ks_lds[CT], vs_lds[CT];
    __shared__ uint32_t bad_lds;

    const psk_paged_attention_args& a = p.a;
    const uint32_t tid = threadIdx.x, nthreads = blockDim.x;
    const uint32_t lane = tid & 63u, w = tid >> 6;
    const uint32_t n = lane & 15u, g = lane >> 4;
    const uint32_t qpk = a.q_heads / a.kv_heads;

    const uint32_t split = blockIdx.x % p.splits;
    const uint32_t rest = blockIdx.x / p.splits;
    const uint32_t kv_head = rest % a.kv_heads;
    const uint32_t tile = rest / a.kv_heads;
    uint32_t r0, nrows;
    if (p.n_tiles != 0u) {
        if (tile >= p.n_tiles) return;
        r0 = p.tile_begin[tile];
        nrows = p.tile_rows[tile];
    } else {
        r0 = tile * kTileRows;
        nrows = r0 < a.rows ? min((uint32_t)kTileRows, a.rows - r0) : 0u;
    }
    if (nrows == 0u || r0 >= a.rows) return;
    nrows = min(nrows, a.rows - r0);

    const uint32_t slot = a.row_sequence_slots[r0];
    if (slot >= a.max_sequences) return;
    const uint64_t cap = (uint64_t)a.block_table_stride * a.page_tokens;
    // row n of the tile (column n of every MFMA): its own visibility
    const uint32_t row = r0 + n;
    bool row_ok = n < nrows && a.row_sequence_slots[min(row, a.rows - 1u)] == slot;
    uint32_t vis = 0;
    if (row_ok) {
        const uint64_t v64 = (uint64_t)a.row_positions[row] + 1u;
        row_ok = v64 <= cap;
        vis = row_ok ? (uint32_t)v64 : 0u;
    }
    uint32_t vis_max = vis;
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) vis_max = max(vis_max, (uint32_t)__shfl_xor((int)vis_max, o, 64));
    if (vis_max == 0u) return;   // uniform: every lane saw the same 16 rows
    const uint32_t P = a.page_tokens;
    const uint32_t pc = (vis_max + P - 1u) / P;
    const uint32_t per = p.pages_per_split != 0u ? p.pages_per_split : (pc + p.splits - 1u) / p.splits;
    const uint32_t pb = split * per;
    if (pb >= pc) return;
    const uint32_t pe = (split == p.splits - 1u) ? pc : min(pc, pb + per);
    const uint32_t t_begin = pb * P, t_end = min(pe * P, vis_max);
    const uint32_t* bt = a.block_tables + (uint64_t)slot * a.block_table_stride;
    const uint64_t layer_base = (uint64_t)a.layer * a.elems_per_layer;
    const uint64_t scale_layer = (uint64_t)a.layer * a.num_pages;

    if (tid == 0) bad_lds = 0u;

    // this wave's query head; Q fragments of the 16 rows (column n = row n)
    const uint32_t head = kv_head * qpk + w;
    bf16x8 qf[NS];
    {
        const uint16_t* qrow = static_cast<const uint16_t*>(a.q) +
                               (uint64_t)(row_ok ? row : r0) * a.q_row_stride + (uint64_t)head * D;
#pragma unroll
        for (int s = 0; s < NS; ++s) {
            const int d0 = KVB == 2 ? s * 32 + (int)g * 8 : (s >> 1) * 64 + (int)g * 16 + (s & 1) * 8;
            qf[s] = q8(qrow + d0, row_ok);
        }
    }

    float m_run = -INFINITY, l_run = 0.0f;
    f32x4 o[NDB];
#pragma unroll
    for (int db = 0; db < NDB; ++db) o[db] = (f32x4){0.f, 0.f, 0.f, 0.f};

    // tr-read offsets of this lane inside a V tile (token slots as in the decode kernel)
    uint32_t tr_off0, tr_off1 = 0;
    if constexpr (KVB == 1) {
        const uint32_t j = n >> 1;
        const uint32_t tok = j < 4u ? 4u * g + j : 16u + 4u * g + (j - 4u);
        tr_off0 = tok * ROW + 8u * (n & 1u);
    } else {
        tr_off0 = (4u * g + (n >> 2)) * ROW + 8u * (n & 3u);
        tr_off1 = (16u + 4u * g + (n >> 2)) * ROW + 8u * (n & 3u);
    }

    for (uint32_t cb = t_begin; cb < t_end; cb += CT) {
        __syncthreads();   // previous chunk fully consumed
        // ---- stage K/V (and FP8 scales) of tokens cb .. cb+31 in LDS
        for (uint32_t idx = tid; idx < (uint32_t)PIECES; idx += nthreads) {
            const uint32_t t = idx / (TB / 16), part = idx % (TB / 16);
            const uint32_t tau = cb + t;
            u32x4 kv = {0u, 0u, 0u, 0u}, vv = {0u, 0u, 0u, 0u};
            if (tau < t_end) {
                const uint32_t page = bt[tau / P];
                if (page < a.num_pages) {
                    const uint64_t e = layer_base + (uint64_t)page * a.elems_per_page +
                                       (uint64_t)(tau % P) * a.elems_per_token + (uint64_t)kv_head * D;
                    kv = *reinterpret_cast<const u32x4*>(p.k_pool + e * KVB + part * 16);
                    vv = *reinterpret_cast<const u32x4*>(p.v_pool + e * KVB + part * 16);
                } else {
                    bad_lds = 1u;
                }
            }
            *reinterpret_cast<u32x4*>(k_lds + t * ROW + part * 16) = kv;
            *reinterpret_cast<u32x4*>(v_lds + t * ROW + part * 16) = vv;
        }
        if constexpr (KVB == 1) {
            if (tid < (uint32_t)CT) {
                const uint32_t tau = cb + tid;
                float ksv = 0.0f, vsv = 0.0f;
                if (tau < t_end) {
                    const uint32_t page = bt[tau / P];
                    if (page < a.num_pages) {
                        const uint64_t si = ((scale_layer + page) * P + tau % P) * a.kv_heads + kv_head;
                        ksv = p.k_scale[si];
                        vsv = p.v_scale[si];
                    }
                }
                ks_lds[tid] = ksv;
                vs_lds[tid] = vsv;
            }
        }
        __syncthreads();
        if (w >= qpk) continue;   // spare waves only help staging

        // ---- S^T for both halves: K fragment of token hf*16+n from LDS
        f32x4 sc[2];
#pragma unroll
        for (int hf = 0; hf < 2; ++hf) {
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
            const uint8_t* kr = k_lds + (hf * 16 + n) * ROW + g * 16;
#pragma unroll
            for (int i = 0; i < NL; ++i) {
                const u32x4 wv = *reinterpret_cast<const u32x4*>(kr + i * 64);
                if constexpr (KVB == 2) {
                    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, wv), qf[i],
                                                                  acc, 0, 0, 0);
                } else {
                    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fp8x8_to_bf16x8(wv[0], wv[1]),
                                                                  qf[2 * i], acc, 0, 0, 0);
                    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fp8x8_to_bf16x8(wv[2], wv[3]),
                                                                  qf[2 * i + 1], acc, 0, 0, 0);
                }
            }
            sc[hf] = acc;
        }
        // ---- lane (n, g): row n, tokens cb + 16*hf + 4*g + r; causal per row
        float s2[2][4], vsc[2][4];
        float mx = -INFINITY;
#pragma unroll
        for (int hf = 0; hf < 2; ++hf)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const uint32_t tl = hf * 16 + 4 * g + r;
                const uint32_t tau = cb + tl;
                float f = p.scale_log2, vs = 1.0f;
                if constexpr (KVB == 1) {
                    f *= ks_lds[tl];
                    vs = vs_lds[tl];
                }
                s2[hf][r] = (tau < vis && tau < t_end) ? sc[hf][r] * f : -INFINITY;
                vsc[hf][r] = vs;
                mx = __builtin_fmaxf(mx, s2[hf][r]);
            }
        mx = __builtin_fmaxf(mx, __shfl_xor(mx, 16, 64));
        mx = __builtin_fmaxf(mx, __shfl_xor(mx, 32, 64));
        const float m_new = __builtin_fmaxf(m_run, mx);
        const float m_use = m_new == -INFINITY ? 0.0f : m_new;
        const float alpha = __builtin_amdgcn_exp2f(m_run - m_use);
        float pv[2][4], psum = 0.0f;
#pragma unroll
        for (int hf = 0; hf < 2; ++hf)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float e = __builtin_amdgcn_exp2f(s2[hf][r] - m_use);
                psum += e;
                pv[hf][r] = e * vsc[hf][r];
            }
        l_run = l_run * alpha + psum;
        m_run = m_new;
        if (__any(alpha != 1.0f)) {
#pragma unroll
            for (int db = 0; db < NDB; ++db) o[db] *= alpha;
        }
        // P as hi + lo bf16 pairs (two MFMAs, ~16 mantissa bits per weight)
        u32x4 ph, pl;
        { const u32x2 t_ = split_bf16x2(pv[0][0], pv[0][1]); ph[0] = t_[0]; pl[0] = t_[1]; }
        { const u32x2 t_ = split_bf16x2(pv[0][2], pv[0][3]); ph[1] = t_[0]; pl[1] = t_[1]; }
        { const u32x2 t_ = split_bf16x2(pv[1][0], pv[1][1]); ph[2] = t_[0]; pl[2] = t_[1]; }
        { const u32x2 t_ = split_bf16x2(pv[1][2], pv[1][3]); ph[3] = t_[0]; pl[3] = t_[1]; }
        const bf16x8 pfh = __builtin_bit_cast(bf16x8, ph);
        const bf16x8 pfl = __builtin_bit_cast(bf16x8, pl);
        // ---- O^T += V^T P^T
#pragma unroll
        for (int db = 0; db < NDB; ++db) {
            bf16x8 vf;
            if constexpr (KVB == 1) {
                const i32x2 x = tr8(v_lds + tr_off0 + 16 * db);
                vf = fp8x8_to_bf16x8((uint32_t)x[0], (uint32_t)x[1]);
            } else {
                const i16x4 x0 = tr16(v_lds + tr_off0 + 32 * db);
                const i16x4 x1 = tr16(v_lds + tr_off1 + 32 * db);
                u32x4 u;
                u[0] = __builtin_bit_cast(u32x2, x0)[0];
                u[1] = __builtin_bit_cast(u32x2, x0)[1];
                u[2] = __builtin_bit_cast(u32x2, x1)[0];
                u[3] = __builtin_bit_cast(u32x2, x1)[1];
                vf = __builtin_bit_cast(bf16x8, u);
            }
            o[db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf, pfh, o[db], 0, 0, 0);
            o[db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf, pfl, o[db], 0, 0, 0);
        }
    }
    __syncthreads();
    if (w >= qpk) return;
    const float l_tot = l_run + __shfl_xor(l_run, 16, 64);
    const float l_all = l_tot + __shfl_xor(l_tot, 32, 64);
    float* part = nullptr;
    if (p.partials != nullptr)
        part = p.partials + ((uint64_t)(row * a.kv_heads + kv_head) * p.splits + split) *
                                (uint64_t)(qpk * (2u + kPagedAttentionHeadLimit));
    if (bad_lds != 0u) {
        // an invalid page on the way leaves the tile's outputs unwritten
        if (part != nullptr && row_ok && g == 0) part[w] = __builtin_nanf("");
        return;
    }
    // rows without tokens in this split (tau >= vis for all of them) are not
    // read by the combine (it uses ceil(pages(row) / per) splits)
    if (!row_ok || t_begin >= vis) return;
    if (part == nullptr) {
#pragma unroll
        for (int db = 0; db < NDB; ++db) {
            const uint64_t oi = (uint64_t)row * a.output_row_stride + (uint64_t)head * D + db * 16 + 4 * g;
            if (a.output_dtype == PSK_OUT_F32) {
                f32x4 v = o[db] / l_all;
                *reinterpret_cast<f32x4*>(static_cast<float*>(a.output) + oi) = v;
            } else {
                uint16_t* dst = static_cast<uint16_t*>(a.output) + oi;
                u32x2 pk;
                pk[0] = pack_bf16x2(o[db][0] / l_all, o[db][1] / l_all);
                pk[1] = pack_bf16x2(o[db][2] / l_all, o[db][3] / l_all);
                *reinterpret_cast<u32x2*>(dst) = pk;
            }
        }
    } else {
        if (g == 0) {
            part[w] = m_run * 0.69314718055994531f;
            part[qpk + w] = l_all;
        }
#pragma unroll
        for (int db = 0; db < NDB; ++db)
            *reinterpret_cast<f32x4*>(part + 2u * qpk + w * kPagedAttentionHeadLimit + db * 16 + 4 * g) = o[db];
    }
}

bool tile_shape_ok(const psk_paged_attention_args& c, int kvb, const void* kp, const void* vp) {
    const uint32_t qpk = c.q_heads / c.kv_heads;
    if (qpk == 0u || qpk > (uint32_t)kMaxTileWaves) return false;
    const uint32_t D = c.head_dim;
    if (!(D == 64 || D == 128 || D == 256 || (D == 32 && kvb == 2))) return false;
    const uint32_t al = 16u / (uint32_t)kvb;
    if (c.elems_per_token % al || c.elems_per_page % al || c.elems_per_layer % al) return false;
    if (reinterpret_cast<uintptr_t>(kp) % 16u || reinterpret_cast<uintptr_t>(vp) % 16u) return false;
    // vector output stores: 16 B (f32) / 8 B (bf16) at head*D + 4*k
    const uint32_t oal = c.output_dtype == PSK_OUT_F32 ? 4u : 4u;
    if (c.output_row_stride % oal || reinterpret_cast<uintptr_t>(c.output) % 16u) return false;
    return true;
}

template <int KVB, int D>
hipError_t launch_tile_t(const TileParams& p, hipStream_t stream) {
    const uint32_t qpk = p.a.q_heads / p.a.kv_heads;
    const uint64_t tiles = p.n_tiles != 0u ? p.n_tiles : (p.a.rows + kTileRows - 1) / kTileRows;
    const uint64_t grid = tiles * p.a.kv_heads * p.splits;
    if (grid == 0u || grid > 0x7FFFFFFFull) return hipErrorInvalidValue;
    // at least 4 waves so every SIMD helps stage K/V
    const uint32_t waves = qpk < 4u ? 4u : qpk;
    hipLaunchKernelGGL((paged_tile_kernel<KVB, D>), dim3((uint32_t)grid), dim3(waves * 64), 0, stream, p);
    return hipGetLastError();
}

template <int KVB>
hipError_t launch_tile(const TileParams& p, hipStream_t stream) {
    switch (p.a.head_dim) {
        case 256: return launch_tile_t<KVB, 256>(p, stream);
        case 128: return launch_tile_t<KVB, 128>(p, stream);
        case 64: return launch_tile_t<KVB, 64>(p, stream);
        case 32:
            if constexpr (KVB == 2) return launch_tile_t<2, 32>(p, stream);
            return hipErrorNotSupported;
        default: return hipErrorNotSupported;
    }
}

hipError_t tile_validate(const psk_paged_attention_args* a, const void* k, const void* v) {
    if (a == nullptr || k == nullptr || v == nullptr) return hipErrorInvalidValue;
    if (a->rows == 0u || a->head_dim == 0u || a->head_dim > kPagedAttentionHeadLimit)
        return hipErrorInvalidValue;
    if (a->q_heads == 0u || a->kv_heads == 0u || a->q_heads % a->kv_heads != 0u)
        return hipErrorInvalidValue;
    if (a->page_tokens == 0u || a->block_table_stride == 0u || a->num_pages == 0u)
        return hipErrorInvalidValue;
    if (a->q == nullptr || a->output == nullptr || a->row_sequence_slots == nullptr ||
        a->row_positions == nullptr || a->block_tables == nullptr)
        return hipErrorInvalidValue;
    if (a->output_dtype != PSK_OUT_BF16 && a->output_dtype != PSK_OUT_F32) return hipErrorInvalidValue;
    return hipSuccess;
}

TileParams make_tile(const psk_paged_attention_args& c, const void* k, const void* v, const float* ks,
                     const float* vs, float* partials, uint32_t splits, uint32_t pps) {
    TileParams p{};
    p.a = c;
    p.k_pool = static_cast<const uint8_t*>(k);
    p.v_pool = static_cast<const uint8_t*>(v);
    p.k_scale = ks;
    p.v_scale = vs;
    p.partials = partials;
    p.splits = splits;
    p.pages_per_split = pps;
    p.scale_log2 = c.scale * kLog2e;
    return p;
}

}  // namespace

// Tile launch over explicit tiles (row_begin, rows) of one launch, any
// number of them (chunks of kInlineTiles per launch). Used by the step
// planner; every tile's rows must belong to one sequence.
hipError_t launch_paged_tiles(const psk_paged_attention_args& a, uint32_t kv_dtype, const void* k,
                              const void* v, const float* ks, const float* vs,
                              const uint32_t* tile_begin, const uint32_t* tile_rows,
                              uint32_t n_tiles, float* partials, uint32_t splits,
                              uint32_t pages_per_split, hipStream_t stream) {
    const hipError_t e = tile_validate(&a, k, v);
    if (e != hipSuccess) return e;
    const int kvb = kv_dtype == PSK_KV_FP8_E4M3 ? 1 : 2;
    if (!tile_shape_ok(a, kvb, k, v)) return hipErrorNotSupported;
    if (splits > 1u && (partials == nullptr || pages_per_split == 0u)) return hipErrorInvalidValue;
    for (uint32_t b = 0; b < n_tiles; b += kInlineTiles) {
        TileParams p = make_tile(a, k, v, ks, vs, splits > 1u ? partials : nullptr, splits,
                                 pages_per_split);
        p.n_tiles = n_tiles - b < kInlineTiles ? n_tiles - b : kInlineTiles;
        for (uint32_t i = 0; i < p.n_tiles; ++i) {
            if (tile_rows[b + i] == 0u || tile_rows[b + i] > (uint32_t)kTileRows)
                return hipErrorInvalidValue;
            p.tile_begin[i] = tile_begin[b + i];
            p.tile_rows[i] = static_cast<uint8_t>(tile_rows[b + i]);
        }
        const hipError_t le = kvb == 1 ? launch_tile<1>(p, stream) : launch_tile<2>(p, stream);
        if (le != hipSuccess) return le;
    }
    return hipSuccess;
}

bool paged_tiles_supported(const psk_paged_attention_args& a, uint32_t kv_dtype, const void* k,
                           const void* v) {
    return tile_shape_ok(a, kv_dtype == PSK_KV_FP8_E4M3 ? 1 : 2, k, v);
}

}  // namespace psk

// Tile launchers: rows [16t, 16t+16) of a launch form one tile and belong to
// the sequence of the tile's first row (the reference's tile contract,
// paged_prefill.hip:152-164; rows of another slot are left unwritten). Shapes
// outside the tile kernel run row by row on the decode launcher.
extern "C" int psk_attention_paged_prefill_bf16(const psk_paged_attention_args* a, const void* k_pool,
                                                const void* v_pool, void* stream) {
    const hipError_t e = psk::tile_validate(a, k_pool, v_pool);
    if (e != hipSuccess) return e;
    if (!psk::tile_shape_ok(*a, 2, k_pool, v_pool))
        return psk_attention_paged_bf16(a, k_pool, v_pool, stream);
    return psk::launch_tile<2>(psk::make_tile(*a, k_pool, v_pool, nullptr, nullptr, nullptr, 1u, 0u),
                               static_cast<hipStream_t>(stream));
}

extern "C" int psk_attention_paged_prefill_fp8_e4m3(const psk_paged_attention_args* a,
                                                    const void* k_pool, const void* v_pool,
                                                    const float* k_scale_pool,
                                                    const float* v_scale_pool, void* stream) {
    const hipError_t e = psk::tile_validate(a, k_pool, v_pool);
    if (e != hipSuccess) return e;
    if (k_scale_pool == nullptr || v_scale_pool == nullptr) return hipErrorInvalidValue;
    if (!psk::tile_shape_ok(*a, 1, k_pool, v_pool))
        return psk_attention_paged_fp8_e4m3(a, k_pool, v_pool, k_scale_pool, v_scale_pool, stream);
    return psk::launch_tile<1>(
        psk::make_tile(*a, k_pool, v_pool, k_scale_pool, v_scale_pool, nullptr, 1u, 0u),
        static_cast<hipStream_t>(stream));
}

extern "C" int psk_attention_paged_tile_split(const psk_paged_attention_args* a, uint32_t kv_dtype,
                                              const void* k_pool, const void* v_pool,
                                              const float* k_scale_pool, const float* v_scale_pool,
                                              float* partials, uint32_t splits,
                                              uint32_t pages_per_split, void* stream) {
    const hipError_t e = psk::tile_validate(a, k_pool, v_pool);
    if (e != hipSuccess) return e;
    if (partials == nullptr || splits == 0u || splits > psk::kMaxTileSplits || pages_per_split == 0u)
        return hipErrorInvalidValue;
    const int kvb = kv_dtype == PSK_KV_FP8_E4M3 ? 1 : 2;
    if (kv_dtype != PSK_KV_FP8_E4M3 && kv_dtype != PSK_KV_BF16) return hipErrorInvalidValue;
    if (kvb == 1 && (k_scale_pool == nullptr || v_scale_pool == nullptr)) return hipErrorInvalidValue;
    if (!psk::tile_shape_ok(*a, kvb, k_pool, v_pool)) return hipErrorNotSupported;
    const psk::TileParams p = psk::make_tile(*a, k_pool, v_pool, k_scale_pool, v_scale_pool, partials,
                                             splits, pages_per_split);
    return kvb == 1 ? psk::launch_tile<1>(p, static_cast<hipStream_t>(stream))
                    : psk::launch_tile<2>(p, static_cast<hipStream_t>(stream));
}
