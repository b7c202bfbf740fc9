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
// MI355X design. Workgroup = (16-row tile, kv_head, split); each wave owns HPW
// query heads of the GQA group. The 16 rows of the tile are the N=16 side of
// v_mfma_f32_16x16x32, so each lane owns one row's causal limit and softmax
// state; K/V chunks (32 tokens) are staged once in LDS and read by all waves,
// and every K (V) fragment a wave converts feeds the MFMAs of all its heads.
// Waves own disjoint (row, head) outputs, so there is no cross-wave merge;
// split-K writes the decode kernel's partial layout and the same combine
// kernel finishes it.
#include "device_common.h"

#include <type_traits>

#include <phaseshift_kv/paged_attention.h>

namespace psk {
namespace {

using ps::kernel::kPagedAttentionHeadLimit;

constexpr int kTileRows = 16;
constexpr int kMaxTileHeads = 8;   // q_per_kv <= 8
constexpr uint32_t kMaxTileSplits = 1024;

// Explicit tiles (row start, row count <= 16) passed by value in the kernel
// arguments; n_tiles == 0 means the implicit windows [16t, 16t+16).
constexpr uint32_t kInlineTiles = 256;

// Tiles per workgroup of a grouped launch (consecutive list entries of one
// sequence; rows == 0 pads a group): 8 waves, one per tile, two per SIMD, so
// one workgroup fills a CU. Against 4 tiles (two workgroups per CU) each
// staged K/V chunk serves twice the rows: config 5's step 1.140 -> 1.08-1.09
// ms, its prefill chunks alone 902-923 -> 884 us (alternated builds, one box).
constexpr int kTileGroup = 8;

struct TileParams {
    psk_paged_attention_args a;
    uint32_t n_tiles;
    uint32_t tiles_per_group;   // 1, or kTileGroup: explicit tiles grouped
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

typedef __attribute__((ext_vector_type(8))) int i32x8;


// FP8 QK^T on v_mfma_f32_16x16x128_f8f6f4: Q of one (row, head) as E4M3
// hi + lo parts of q * 2^sh, sh = 8 - E with max|q| = m * 2^E (m in
// [0.5, 1)), so max|q * 2^sh| is in [128, 256). hi = RNE(q * 2^sh) and lo =
// RNE(q * 2^sh - hi) keep q to 2^-8 relative (the residual is exact in
// fp32); scores are the MFMA sums times 2^-sh. Lane (n, g) holds dims
// [64i + 16g, +16) of every 64-dim block i: bytes 0-15 of operand j are
// block 2j, bytes 16-31 block 2j + 1, the K fragment's layout (the MFMA
// pairs equal (lane group, byte) positions of its two operands).
template <int D>
__device__ __forceinline__ float q_split_e4m3(const uint16_t* qrow, bool ok, uint32_t g,
                                              i32x8 (&hi)[D / 128], i32x8 (&lo)[D / 128]) {
    constexpr int NB = D / 64;
    float x[NB][16];
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < NB; ++i) {
        u32x4 w0 = {0u, 0u, 0u, 0u}, w1 = {0u, 0u, 0u, 0u};
        if (ok) {
            const u32x4* src = reinterpret_cast<const u32x4*>(qrow + 64 * i + 16 * g);
            w0 = src[0];
            w1 = src[1];
        }
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const uint32_t wd = k < 4 ? w0[k] : w1[k - 4];
            x[i][2 * k] = __builtin_bit_cast(float, wd << 16);
            x[i][2 * k + 1] = __builtin_bit_cast(float, wd & 0xFFFF0000u);
        }
#pragma unroll
        for (int k = 0; k < 16; ++k) amax = __builtin_fmaxf(amax, __builtin_fabsf(x[i][k]));
    }
    amax = __builtin_fmaxf(amax, __shfl_xor(amax, 16, 64));
    amax = __builtin_fmaxf(amax, __shfl_xor(amax, 32, 64));
    const int sh = (amax > 0.0f && amax <= 3.0e38f) ? 8 - __builtin_amdgcn_frexp_expf(amax) : 0;
#pragma unroll
    for (int i = 0; i < NB; ++i) {
        uint32_t h[4], l[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            float y[4], r[4];
#pragma unroll
            for (int t = 0; t < 4; ++t) y[t] = __builtin_ldexpf(x[i][4 * k + t], sh);
            h[k] = e4m3x4_rne(y[0], y[1], y[2], y[3]);
            r[0] = y[0] - __builtin_amdgcn_cvt_f32_fp8((int)h[k], 0);
            r[1] = y[1] - __builtin_amdgcn_cvt_f32_fp8((int)h[k], 1);
            r[2] = y[2] - __builtin_amdgcn_cvt_f32_fp8((int)h[k], 2);
            r[3] = y[3] - __builtin_amdgcn_cvt_f32_fp8((int)h[k], 3);
            l[k] = e4m3x4_rne(r[0], r[1], r[2], r[3]);
        }
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            hi[i / 2][4 * (i & 1) + k] = (int)h[k];
            lo[i / 2][4 * (i & 1) + k] = (int)l[k];
        }
    }
    return __builtin_ldexpf(1.0f, -sh);
}

constexpr uint32_t kTilePageWindow = 1024;   // block-table entries staged in LDS per pass

// LDS bytes of one pipeline stage: K and V of a 32-token chunk (lane-major DMA
// layout) and, FP8 and PSQ, the k/v scales of its tokens (256 B per 16-token
// half: FP8 one f32 per token, PSQ dword w of token t at 64w + 4t).
template <int FMT, int D>
constexpr int tile_stage_bytes() {
    return 2 * 2 * (16 * code_bytes<FMT, D>() + 128) + (FMT != kFmtBf16 ? 2 * 2 * 256 : 0);
}
constexpr int kTileStages = 4;   // two pairs of chunks (see the main loop)

// kAl16: page_tokens % 16 == 0, so every page-aligned 16-token half lies in one
// page and its page id, base address and in-page offset are wave-uniform.
// Waves per SIMD the register budget targets: 3 with one head per wave, 2
// with two (the accumulators of 2 heads take 128 registers at D=256).
constexpr int tile_waves_per_simd(int hpw) { return hpw == 1 ? 3 : 2; }

// GQA groups that grouped launches take: 1-8 heads per kv head, as head
// pairs (a 1-head group or the last pair of an odd group computes one head
// of the pair on zero Q). Measured on 8 prefill chunks of 512 rows (FP8,
// 4 kv heads, hd 256, contexts 5.3k-14.3k) against one tile per workgroup:
// 1 head per group 826 -> 484 us, 2 heads 862 -> 511, 4 heads 956 -> 705,
// 8 heads 1294 -> 1100.
constexpr bool grouped_heads(uint32_t q_per_kv) { return q_per_kv >= 1u && q_per_kv <= 8u; }

// RT: row tiles per workgroup. RT == 1: the NW waves split the GQA group's
// heads (HPW each) of one tile. RT > 1 (NW == RT): wave w owns tile w of a
// group of RT consecutive tiles of one sequence and HPW heads of the group's
// head part (blockIdx); the tiles share every staged K/V chunk.
// Split units of ungrouped tile t: the splits of its visible range that hold
// pages (0 for a tile the kernels skip). Follows the kernels' own rules: the
// tile's first row names the sequence, rows of another sequence or past the
// block table see nothing, and the tile streams the largest visible range of
// its rows.
__device__ uint32_t tile_units(const TileParams& p, uint32_t t) {
    const psk_paged_attention_args& a = p.a;
    uint32_t r0, nrows;
    if (p.n_tiles != 0u) {
        if (t >= p.n_tiles) return 0u;
        r0 = p.tile_begin[t];
        nrows = p.tile_rows[t];
    } else {
        r0 = t * kTileRows;
        nrows = kTileRows;
    }
    if (r0 >= a.rows) return 0u;
    nrows = min(nrows, a.rows - r0);
    if (nrows == 0u) return 0u;
    const uint32_t slot = a.row_sequence_slots[r0];
    if (slot >= a.max_sequences) return 0u;
    const uint64_t cap = (uint64_t)a.block_table_stride * a.page_tokens;
    // all rows' loads first (rows past the tile repeat its last row)
    uint32_t sl[kTileRows], ps[kTileRows];
#pragma unroll
    for (int j = 0; j < kTileRows; ++j) {
        const uint32_t r = r0 + min((uint32_t)j, nrows - 1u);
        sl[j] = a.row_sequence_slots[r];
        ps[j] = a.row_positions[r];
    }
    uint32_t vis_max = 0u;
#pragma unroll
    for (int j = 0; j < kTileRows; ++j) {
        const uint64_t v64 = (uint64_t)ps[j] + 1u;
        if (sl[j] == slot && v64 <= cap) vis_max = max(vis_max, (uint32_t)v64);
    }
    if (vis_max == 0u) return 0u;
    const uint32_t pc = (vis_max + a.page_tokens - 1u) / a.page_tokens;
    const uint32_t per = p.pages_per_split != 0u ? p.pages_per_split : (pc + p.splits - 1u) / p.splits;
    return min(p.splits, (pc + per - 1u) / per);
}

// Largest tiles x splits of a launch whose workgroups take dense units: each
// workgroup scans every tile's rows to find its unit, which stays cheap (one
// tile per thread, at most a few thousand workgroups) up to this size; larger
// launches have enough workgroups to balance without it.
constexpr uint32_t kDenseTileUnits = 1024;

// Workgroup -> (split, head part, kv head, tile group). Split ungrouped
// launches (RT == 1, splits > 1, tiles x splits <= kDenseTileUnits) number
// only the (tile, split) units that hold pages, densely and longest first
// (find_dense_unit), as blockIdx = unit * kv_heads + kv_head: a verify launch
// over blocks of different context lengths otherwise leaves most of its grid
// empty and the active workgroups unevenly spread over the XCDs. Returns
// false for a workgroup without work.
template <int NW, int HPW, int RT>
__device__ __forceinline__ bool tile_workgroup(const TileParams& p, uint32_t qpk, uint32_t& split,
                                               uint32_t& hpart, uint32_t& kv_head, uint32_t& group) {
    hpart = 0u;
    if constexpr (RT == 1) {
        const uint32_t count = p.n_tiles != 0u ? p.n_tiles : (p.a.rows + kTileRows - 1u) / kTileRows;
        if (p.splits > 1u && (uint64_t)count * p.splits <= kDenseTileUnits) {
            kv_head = blockIdx.x % p.a.kv_heads;
            return find_dense_unit<NW>(
                count, [&](uint32_t t) { return tile_units(p, t); }, blockIdx.x / p.a.kv_heads, group, split);
        }
    }
    split = blockIdx.x % p.splits;
    uint32_t rest = blockIdx.x / p.splits;
    if constexpr (RT > 1) {
        const uint32_t hparts = (qpk + HPW - 1u) / HPW;
        hpart = rest % hparts;
        rest /= hparts;
    }
    kv_head = rest % p.a.kv_heads;
    group = rest / p.a.kv_heads;
    return true;
}

template <int FMT, int D, int NW, int HPW, int RT, bool kAl16>
__global__ __launch_bounds__(NW * 64, tile_waves_per_simd(HPW)) void paged_tile_kernel(const TileParams p) {
    static_assert(RT == 1 || RT == NW, "grouped tiles: one wave per tile");
    static_assert(FMT == kFmtBf16 || FMT == kFmtFp8, "PSQ tiles: paged_tile_psq_group_kernel");
    constexpr int KVB = FMT == kFmtBf16 ? 2 : 1;   // bytes per value
    constexpr int CB = code_bytes<FMT, D>();       // K (V) bytes of one token's head slice
    constexpr int WH = NW / RT;          // waves along the heads of one tile
    constexpr int H = 2;                 // 16-token halves per chunk
    constexpr int CT = 16 * H;           // tokens per chunk
    constexpr int NL = CB / 64;          // 16 B DMA pieces per lane per half
    constexpr int NS = D / 32;           // K-steps of QK^T
    constexpr int NDB = D / 16;          // 16-dim output blocks
    constexpr bool kF8Mfma = FMT == kFmtFp8 && D % 128 == 0;
    // a 16-token half of K (V) in LDS, padded by 128 B so that the two halves
    // of a chunk fall on opposite halves of the 64 LDS banks (the transposing
    // V reads of one instruction touch both)
    constexpr int HALF_STRIDE = 16 * CB + 128;
    constexpr int KV_BYTES = H * HALF_STRIDE;
    constexpr int SC_BYTES = KVB == 1 ? H * 256 : 0;
    constexpr int STAGE = tile_stage_bytes<FMT, D>();
    // DMA instructions of one chunk (K, V, then FP8 k/v scales), dealt
    // round-robin over the NW waves; every wave issues DPW of them (the
    // remainder repeats earlier ones, which rewrite identical bytes), so the
    // vmcnt bookkeeping is one compile-time count per wave.
    constexpr int NI = 2 * H * NL + (KVB == 1 ? 2 * H : 0);
    // NW >= 2H: wave w < 2H owns one stream, K (w < H) or V, half w % H: its
    // NL body pieces and (FP8) that half's scales, so the dealing is fixed per
    // wave; waves past 2H issue none (their vmcnt waits pass at once)
    constexpr bool kOwnStream = NW >= 2 * H;
    constexpr int DPW = kOwnStream ? NL + (KVB == 1 ? 1 : 0) : (NI + NW - 1) / NW;
    constexpr int kWinBytes = (int)kTilePageWindow * 4;
    static_assert(NL >= 1 && NS >= 1 && 2 * DPW < 64, "tile geometry");

    extern __shared__ __align__(16) uint8_t lds[];
    __shared__ uint32_t bad_lds;

    const psk_paged_attention_args& a = p.a;
    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid & 63u, w = tid >> 6;
    const uint32_t n = lane & 15u, g = lane >> 4;
    const uint32_t qpk = a.q_heads / a.kv_heads;

    uint32_t split, hpart, kv_head, group;
    if (!tile_workgroup<NW, HPW, RT>(p, qpk, split, hpart, kv_head, group)) return;
    const uint32_t rt = RT > 1 ? w : 0u;
    const uint32_t tile = group * RT + rt;
    // the group's first tile names the sequence (workgroup-uniform)
    uint32_t g0;
    if (p.n_tiles != 0u) {
        if (group * RT >= p.n_tiles) return;
        g0 = p.tile_begin[group * RT];
    } else {
        g0 = group * RT * kTileRows;
    }
    if (g0 >= a.rows) return;
    const uint32_t slot = a.row_sequence_slots[g0];
    if (slot >= a.max_sequences) return;
    // this wave's tile; a grouped tile past the list or of no rows computes nothing
    uint32_t r0, nrows;
    if (p.n_tiles != 0u) {
        const bool have = tile < p.n_tiles;
        r0 = have ? p.tile_begin[tile] : g0;
        nrows = have ? p.tile_rows[tile] : 0u;
    } else {
        r0 = tile * kTileRows;
        nrows = r0 < a.rows ? min((uint32_t)kTileRows, a.rows - r0) : 0u;
    }
    if (r0 >= a.rows) nrows = 0u;
    nrows = min(nrows, a.rows - min(r0, a.rows));

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
    const uint32_t wave_vis = vis_max;   // this wave's rows see tokens [0, wave_vis)
    // tokens [0, wave_vis_min) are visible to every row of the wave that is written
    uint32_t wave_vis_min = row_ok ? vis : 0xFFFFFFFFu;
#pragma unroll
    for (int o = 1; o < 16; o <<= 1)
        wave_vis_min = min(wave_vis_min, (uint32_t)__shfl_xor((int)wave_vis_min, o, 64));
    if constexpr (RT > 1) {
        // the workgroup streams the longest visible range of its tiles
        __shared__ uint32_t group_vis;
        if (tid == 0) group_vis = 0u;
        __syncthreads();
        if (lane == 0) atomicMax(&group_vis, wave_vis);
        __syncthreads();
        vis_max = group_vis;
    }
    if (vis_max == 0u) return;   // uniform over the workgroup
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
    // Everything above is uniform over the workgroup, so all waves reach the
    // barriers below; a wave past the last query head of the group only
    // issues its share of the DMAs.
    const uint32_t hbase = RT > 1 ? hpart * HPW : w * HPW;   // first head (group index)
    const bool computes = hbase < qpk && wave_vis > 0u;

    if (tid == 0) bad_lds = 0u;

    // this wave's query head; Q fragments of the 16 rows (column n = row n)
    // this wave's query heads (group index w*HPW + i); heads past the group
    // compute on zero Q and are never written
    bool hv[HPW];
    bf16x8 qf[HPW][NS];
    // FP8 KV at D % 128 == 0: K codes go to the MFMA unconverted (Q as E4M3
    // hi + lo, see q_split_e4m3); qinv = 2^-sh of each head's row
    i32x8 qh[HPW][kF8Mfma ? D / 128 : 1], ql[HPW][kF8Mfma ? D / 128 : 1];
    float qinv[HPW];
#pragma unroll
    for (int i = 0; i < HPW; ++i) {
        const uint32_t gh = hbase + (uint32_t)i;
        hv[i] = gh < qpk;
        const uint32_t head = kv_head * qpk + (hv[i] ? gh : 0u);
        const uint16_t* qrow = static_cast<const uint16_t*>(a.q) +
                               (uint64_t)(row_ok ? row : r0) * a.q_row_stride + (uint64_t)head * D;
        qinv[i] = 1.0f;
        if constexpr (kF8Mfma) {
            qinv[i] = q_split_e4m3<D>(qrow, row_ok && hv[i], g, qh[i], ql[i]);
        } else {
#pragma unroll
            for (int s = 0; s < NS; ++s) {
                // BF16: dims 32s + 8g..; FP8: the 16 B of 64-dim block s/2
                // split in two K-steps
                const int d0 = FMT == kFmtBf16 ? s * 32 + (int)g * 8 : (s >> 1) * 64 + (int)g * 16 + (s & 1) * 8;
                qf[i][s] = q8(qrow + d0, row_ok && hv[i]);
            }
        }
    }

    float m_run[HPW], l_run[HPW];
    f32x4 o[HPW][NDB];
#pragma unroll
    for (int i = 0; i < HPW; ++i) {
        m_run[i] = -INFINITY;
        l_run[i] = 0.0f;
#pragma unroll
        for (int db = 0; db < NDB; ++db) o[i][db] = (f32x4){0.f, 0.f, 0.f, 0.f};
    }

    // tr-read offsets of this lane inside the V part of a stage. Lane r of a
    // 16-lane block names row r of the transpose; in the DMA layout byte b of
    // token t sits at (t/16)*HALF_STRIDE + 1024*(b/64) + 16*(16*((b%64)/16) + t%16) + b%16.
    //   FP8:  token (r>>1 < 4 ? 4g + (r>>1) : 16 + 4g + (r>>1) - 4), dims +8*(r&1); block db +256*db
    //   BF16: token 4g + (r>>2) of each half, dims +4*(r&3); block db +512*db
    uint32_t tr_off;
    if constexpr (KVB == 1) {
        const uint32_t j = n >> 1;
        tr_off = (j < 4u ? 0u : (uint32_t)HALF_STRIDE) + 16u * (4u * g + (j & 3u)) + 8u * (n & 1u);
    } else {
        tr_off = 16u * (4u * g + (n >> 2)) + 256u * ((n >> 1) & 1u) + 8u * (n & 1u);
    }

    uint32_t* const win = reinterpret_cast<uint32_t*>(lds);
    uint8_t* const stages = lds + kWinBytes;
    // pool pointers and the wave index in scalar registers: the DMA dealing
    // below selects among them per wave without memory accesses
    const uint8_t* const k_pool = p.k_pool;
    const uint8_t* const v_pool = p.v_pool;
    const float* const k_scale = p.k_scale;
    const float* const v_scale = p.v_scale;
    const uint32_t wu = __builtin_amdgcn_readfirstlane(w);

    for (uint32_t wp = pb; wp < pe; wp += kTilePageWindow) {
        const uint32_t wp_end = min(pe, wp + kTilePageWindow);
        __syncthreads();
        for (uint32_t i = tid; i < wp_end - wp; i += NW * 64u) win[i] = bt[wp + i];
        __syncthreads();
        const uint32_t ts = max(wp * P, t_begin);
        const uint32_t te = min(wp_end * P, t_end);
        if (ts >= te) continue;
        const uint32_t t_last = te - 1u;

        // Byte offset of the (page pg, token 0, kv_head) slice in a pool, and
        // the bytes between consecutive tokens' slices
        auto slice_base = [&](uint32_t pg) __attribute__((always_inline)) -> uint64_t {
            return (layer_base + (uint64_t)pg * a.elems_per_page + (uint64_t)kv_head * D) * KVB;
        };
        const uint32_t tok_bytes = a.elems_per_token * (uint32_t)KVB;
        // Source of this lane's FP8 scale DMA for the token at (pg, off)
        auto scale_src = [&](uint32_t kind, uint32_t pg, uint32_t off) __attribute__((always_inline)) {
            const uint64_t si = ((scale_layer + pg) * P + off) * a.kv_heads + kv_head;
            const float* base = kind == 0u ? k_scale : v_scale;
            return static_cast<const void*>(base + si);
        };

        // This wave's DMAs of the chunk at c into stage st (branch-free;
        // tokens past the range read the last token and are masked later).
        auto issue_own = [&](uint32_t c, uint8_t* st) __attribute__((always_inline)) {
            if (NW > 2 * H && wu >= 2u * H) return;
            const uint32_t hf = wu % (uint32_t)H;   // scalar
            const uint32_t kind = wu / (uint32_t)H;
            const uint32_t tau = min(c + hf * 16u + n, t_last);
            uint32_t page, off;
            if constexpr (kAl16) {
                const uint32_t hb = min(c + hf * 16u, t_last);
                const uint32_t pi = hb / P;
                page = __builtin_amdgcn_readfirstlane(win[pi - wp]);
                off = tau - pi * P;
            } else {
                page = win[tau / P - wp];
                off = tau % P;
            }
            const bool inv = page >= a.num_pages;
            if (inv) bad_lds = 1u;
            const uint32_t pg = inv ? 0u : page;
            const uint8_t* pool = kind == 0u ? k_pool : v_pool;
            uint8_t* dst = st + kind * KV_BYTES + hf * HALF_STRIDE;
            if constexpr (kAl16) {
                const uint8_t* src = pool + slice_base(pg);
                const uint32_t lo = off * tok_bytes + g * 16u;
#pragma unroll
                for (int i = 0; i < NL; ++i) load_lds<16>(src + (lo + i * 64u), dst + i * 1024);
            } else {
                const uint8_t* src = pool + slice_base(pg) + (uint64_t)off * tok_bytes + g * 16u;
#pragma unroll
                for (int i = 0; i < NL; ++i) load_lds<16>(src + i * 64, dst + i * 1024);
            }
            if constexpr (KVB == 1) load_lds<4>(scale_src(kind, pg, off), st + 2 * KV_BYTES + kind * SC_BYTES + hf * 256);
        };
        auto issue = [&](uint32_t c, uint8_t* st) __attribute__((always_inline)) {
            if constexpr (kOwnStream) {
                issue_own(c, st);
                return;
            }
            // page ids of this lane's token in both halves first: no LDS read
            // follows a DMA of this step
            uint32_t pg[H], off[H];
#pragma unroll
            for (int hf = 0; hf < H; ++hf) {
                const uint32_t tau = min(c + (uint32_t)hf * 16u + n, t_last);
                uint32_t page;
                if constexpr (kAl16) {
                    // the half's page (chunks start page-aligned), read once
                    const uint32_t hb = min(c + (uint32_t)hf * 16u, t_last);
                    const uint32_t pi = hb / P;
                    page = __builtin_amdgcn_readfirstlane(win[pi - wp]);
                    off[hf] = tau - pi * P;
                } else {
                    page = win[tau / P - wp];
                    off[hf] = tau % P;
                }
                const bool inv = page >= a.num_pages;
                if (inv) bad_lds = 1u;
                pg[hf] = inv ? 0u : page;
            }
#pragma unroll
            for (int t = 0; t < DPW; ++t) {
                const uint32_t j = (wu + (uint32_t)NW * t) % (uint32_t)NI;   // scalar
                if (j < 2u * H * NL) {
                    const uint32_t kind = j / (H * NL), hf = (j % (H * NL)) / NL, i = j % NL;
                    const uint8_t* src;
                    if constexpr (kAl16) {
                        // uniform page base + 32-bit lane offset
                        src = (kind == 0u ? k_pool : v_pool) + slice_base(pg[hf]) +
                              (off[hf] * tok_bytes + g * 16u + i * 64u);
                    } else {
                        src = (kind == 0u ? k_pool : v_pool) + slice_base(pg[hf]) +
                              (uint64_t)off[hf] * tok_bytes + g * 16 + i * 64;
                    }
                    load_lds<16>(src, st + kind * KV_BYTES + hf * HALF_STRIDE + i * 1024);
                } else {
                    const uint32_t kind = (j - 2u * H * NL) & 1u, hf = (j - 2u * H * NL) >> 1;
                    load_lds<4>(scale_src(kind, pg[hf], off[hf]), st + 2 * KV_BYTES + kind * SC_BYTES + hf * 256);
                }
            }
        };

        // Scores, causal online softmax and PV of the chunk at c in stage st.
        // kFull: every token of the chunk is visible to every written row and
        // inside the split, so no causal mask is formed
        auto consume = [&](uint32_t c, const uint8_t* st, auto full_tag) __attribute__((always_inline)) {
            constexpr bool kFull = decltype(full_tag)::value;
            f32x4 sc[HPW][H];
            if constexpr (kF8Mfma) {
                // 128 dims per MFMA: the lane's 16 B of blocks 2j and 2j + 1
                // (one half), read one step ahead of the MFMAs they feed
                constexpr int NJ = D / 128;
                auto kread = [&](int u) __attribute__((always_inline)) {
                    const uint8_t* kb = st + (u / NJ) * HALF_STRIDE + 16 * lane + 2048 * (u % NJ);
                    const u32x4 x0 = *reinterpret_cast<const u32x4*>(kb);
                    const u32x4 x1 = *reinterpret_cast<const u32x4*>(kb + 1024);
                    return (i32x8){(int)x0[0], (int)x0[1], (int)x0[2], (int)x0[3],
                                   (int)x1[0], (int)x1[1], (int)x1[2], (int)x1[3]};
                };
                f32x4 acc[HPW];
                i32x8 cur = kread(0);
                // Raised wave priority over each MFMA cluster: the SIMD's other
                // wave then fills the VALU while this one streams its MFMAs
                // (measured: prefill launch of config 5 1035 -> 998 us).
                __builtin_amdgcn_s_setprio(1);
#pragma unroll
                for (int u = 0; u < H * NJ; ++u) {
                    i32x8 nxt = cur;
                    if (u + 1 < H * NJ) nxt = kread(u + 1);
                    __builtin_amdgcn_sched_barrier(0);
                    const int j = u % NJ;
                    if (j == 0) {
#pragma unroll
                        for (int i = 0; i < HPW; ++i) acc[i] = (f32x4){0.f, 0.f, 0.f, 0.f};
                    }
#pragma unroll
                    for (int i = 0; i < HPW; ++i)
                        acc[i] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(cur, qh[i][j], acc[i], 0, 0, 0, 0,
                                                                                  0, 0);
#pragma unroll
                    for (int i = 0; i < HPW; ++i)
                        acc[i] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(cur, ql[i][j], acc[i], 0, 0, 0, 0,
                                                                                  0, 0);
                    if (j == NJ - 1) {
#pragma unroll
                        for (int i = 0; i < HPW; ++i) sc[i][u / NJ] = acc[i];
                    }
                    cur = nxt;
                }
                __builtin_amdgcn_s_setprio(0);
            } else if constexpr (NS % 2 == 0) {
                // K in pairs of K-steps (16 B of FP8 or 2 x 16 B of BF16 per
                // lane), each pair's LDS read issued one pair ahead so that its
                // latency hides behind the previous pair's MFMAs
                constexpr int NP = NS / 2;
                struct KRaw {
                    u32x4 a, b;
                };
                auto kread = [&](int u) __attribute__((always_inline)) {
                    const uint8_t* kb = st + (u / NP) * HALF_STRIDE + 16 * lane;
                    KRaw r;
                    if constexpr (KVB == 1) {
                        r.a = *reinterpret_cast<const u32x4*>(kb + 1024 * (u % NP));
                        r.b = r.a;
                    } else {
                        r.a = *reinterpret_cast<const u32x4*>(kb + 1024 * (2 * (u % NP)));
                        r.b = *reinterpret_cast<const u32x4*>(kb + 1024 * (2 * (u % NP) + 1));
                    }
                    return r;
                };
                f32x4 acc[HPW];
                KRaw cur = kread(0);
#pragma unroll
                for (int u = 0; u < H * NP; ++u) {
                    KRaw nxt = cur;
                    if (u + 1 < H * NP) nxt = kread(u + 1);
                    __builtin_amdgcn_sched_barrier(0);
                    const int sp = u % NP;
                    if (sp == 0) {
#pragma unroll
                        for (int i = 0; i < HPW; ++i) acc[i] = (f32x4){0.f, 0.f, 0.f, 0.f};
                    }
                    bf16x8 k0, k1;
                    if constexpr (KVB == 1) {
                        k0 = fp8x8_to_bf16x8(cur.a[0], cur.a[1]);
                        k1 = fp8x8_to_bf16x8(cur.a[2], cur.a[3]);
                    } else {
                        k0 = __builtin_bit_cast(bf16x8, cur.a);
                        k1 = __builtin_bit_cast(bf16x8, cur.b);
                    }
#pragma unroll
                    for (int i = 0; i < HPW; ++i)
                        acc[i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(k0, qf[i][2 * sp], acc[i], 0, 0, 0);
#pragma unroll
                    for (int i = 0; i < HPW; ++i)
                        acc[i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(k1, qf[i][2 * sp + 1], acc[i], 0, 0, 0);
                    if (sp == NP - 1) {
#pragma unroll
                        for (int i = 0; i < HPW; ++i) sc[i][u / NP] = acc[i];
                    }
                    cur = nxt;
                }
            } else {
#pragma unroll
                for (int hf = 0; hf < H; ++hf) {
                    f32x4 acc[HPW];
#pragma unroll
                    for (int i = 0; i < HPW; ++i) acc[i] = (f32x4){0.f, 0.f, 0.f, 0.f};
                    const uint8_t* kb = st + hf * HALF_STRIDE + 16 * lane;
#pragma unroll
                    for (int s = 0; s < NS; ++s) {
                        const bf16x8 kf = *reinterpret_cast<const bf16x8*>(kb + 1024 * s);
#pragma unroll
                        for (int i = 0; i < HPW; ++i)
                            acc[i] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf, qf[i][s], acc[i], 0, 0, 0);
                    }
#pragma unroll
                    for (int i = 0; i < HPW; ++i) sc[i][hf] = acc[i];
                }
            }
            __builtin_amdgcn_sched_barrier(0);
            // lane (n, g): row n, tokens c + 16*hf + 4*g + r; causal per row
            f32x4 kscale[H], vscale[H];
            bool tok_ok[H][4];
#pragma unroll
            for (int hf = 0; hf < H; ++hf) {
                kscale[hf] = (f32x4){1.f, 1.f, 1.f, 1.f};
                vscale[hf] = (f32x4){1.f, 1.f, 1.f, 1.f};
                if constexpr (FMT == kFmtFp8) {
                    kscale[hf] = *reinterpret_cast<const f32x4*>(st + 2 * KV_BYTES + hf * 256 + 16 * g);
                    vscale[hf] = *reinterpret_cast<const f32x4*>(st + 2 * KV_BYTES + SC_BYTES +
                                                                 hf * 256 + 16 * g);
                }
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const uint32_t tau = c + hf * 16 + 4 * g + r;
                    tok_ok[hf][r] = kFull || (tau < vis && tau < te);
                }
            }
            u32x4 pf[HPW], pl[HPW];
#pragma unroll
            for (int i = 0; i < HPW; ++i) {
                // scores in log2 units are s2 * qinv[i]: qinv > 0 scales the
                // row maximum once and enters exp2 through one FMA per score
                float s2[H][4];
                float mx = -INFINITY;
#pragma unroll
                for (int hf = 0; hf < H; ++hf)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        s2[hf][r] = tok_ok[hf][r] ? sc[i][hf][r] * (p.scale_log2 * kscale[hf][r]) : -INFINITY;
                        mx = __builtin_fmaxf(mx, s2[hf][r]);
                    }
                mx = max_xor32(max_xor16(mx));   // lane permutes, no LDS round trip
                mx *= qinv[i];
                // m_run is the row's softmax reference: it moves only when a
                // score exceeds it by more than kLazyMaxSlack (then P <= 2^slack)
                const bool moved = mx > m_run[i] + kLazyMaxSlack;
                const float m_new = moved ? mx : m_run[i];
                const float m_use = m_new == -INFINITY ? 0.0f : m_new;
                const float alpha = moved ? __builtin_amdgcn_exp2f(m_run[i] - m_use) : 1.0f;
                float pv[H][4], psum = 0.0f;
#pragma unroll
                for (int hf = 0; hf < H; ++hf)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const float e = __builtin_amdgcn_exp2f(__builtin_fmaf(s2[hf][r], qinv[i], -m_use));
                        psum += e;
                        pv[hf][r] = e * vscale[hf][r];
                    }
                l_run[i] = l_run[i] * alpha + psum;
                m_run[i] = m_new;
                if (__any(moved)) {
#pragma unroll
                    for (int db = 0; db < NDB; ++db) o[i][db] *= alpha;
                }
                if constexpr (KVB == 1) {
                    // FP8: P (v_scale folded in) as one f16 operand (11 mantissa
                    // bits); V as f16 (E4M3 values are exact in f16)
                    pf[i][0] = pack_f16x2(pv[0][0], pv[0][1]);
                    pf[i][1] = pack_f16x2(pv[0][2], pv[0][3]);
                    pf[i][2] = pack_f16x2(pv[1][0], pv[1][1]);
                    pf[i][3] = pack_f16x2(pv[1][2], pv[1][3]);
                } else {
                    // BF16: P as hi + lo bf16 pairs (two MFMAs, ~16 mantissa bits)
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const u32x2 t_ = split_bf16x2(pv[j >> 1][2 * (j & 1)], pv[j >> 1][2 * (j & 1) + 1]);
                        pf[i][j] = t_[0];
                        pl[i][j] = t_[1];
                    }
                }
            }
            // O^T += V^T P^T, one V fragment per output block for all heads.
            // V is read in pairs of output blocks, each pair's transposing LDS
            // reads issued one pair ahead of the previous pair's MFMAs.
            const uint8_t* vb = st + KV_BYTES + tr_off;
            static_assert(NDB % 2 == 0, "output blocks in pairs");
            struct VRaw {
                u32x4 x[2];
            };
            auto vread = [&](int pr) __attribute__((always_inline)) {
                VRaw r;
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const int db = 2 * pr + j;
                    if constexpr (KVB == 1) {
                        const i32x2 t = tr8(vb + 256 * db);
                        r.x[j] = (u32x4){(uint32_t)t[0], (uint32_t)t[1], 0u, 0u};
                    } else {
                        const i16x4 x0 = tr16(vb + 512 * db);
                        const i16x4 x1 = tr16(vb + HALF_STRIDE + 512 * db);
                        r.x[j] = (u32x4){__builtin_bit_cast(u32x2, x0)[0], __builtin_bit_cast(u32x2, x0)[1],
                                         __builtin_bit_cast(u32x2, x1)[0], __builtin_bit_cast(u32x2, x1)[1]};
                    }
                }
                return r;
            };
            VRaw vcur = vread(0);
            __builtin_amdgcn_s_setprio(1);
#pragma unroll
            for (int pr = 0; pr < NDB / 2; ++pr) {
                VRaw vnxt = vcur;
                if (pr + 1 < NDB / 2) vnxt = vread(pr + 1);
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const int db = 2 * pr + j;
                    if constexpr (KVB == 1) {
                        const f16x8 vf = fp8x8_to_f16x8(vcur.x[j][0], vcur.x[j][1]);
#pragma unroll
                        for (int i = 0; i < HPW; ++i)
                            o[i][db] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                                vf, __builtin_bit_cast(f16x8, pf[i]), o[i][db], 0, 0, 0);
                    } else {
                        const bf16x8 vf = __builtin_bit_cast(bf16x8, vcur.x[j]);
#pragma unroll
                        for (int i = 0; i < HPW; ++i) {
                            o[i][db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                                vf, __builtin_bit_cast(bf16x8, pf[i]), o[i][db], 0, 0, 0);
                            o[i][db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                                vf, __builtin_bit_cast(bf16x8, pl[i]), o[i][db], 0, 0, 0);
                        }
                    }
                }
                vcur = vnxt;
            }
            __builtin_amdgcn_s_setprio(0);
        };

        // Two chunks per barrier (measured: config 5's prefill launch 999 ->
        // 973 us against one chunk per barrier with three in flight): pair p
        // sits in stages 2(p&1), +1; after the wait + barrier the pair has
        // landed and every wave is done with pair p - 1, whose stages take
        // pair p + 1, in flight while pair p is computed. __restrict__ tells
        // the compiler that the DMAs into `next` and the reads of `cur` touch
        // different LDS; their real ordering is the wait + barrier.
        static_assert(kTileStages == 4, "two pairs of chunk stages");
        issue(ts, stages);
        issue(ts + CT, stages + STAGE);
        auto step2 = [&](uint32_t c, uint8_t* __restrict__ next, const uint8_t* __restrict__ cur)
                         __attribute__((always_inline)) {
            issue(c + 2 * CT, next);
            issue(c + 3 * CT, next + STAGE);
            if (computes && c < wave_vis) {
                if (c + CT <= wave_vis_min && c + CT <= te)
                    consume(c, cur, std::true_type{});
                else
                    consume(c, cur, std::false_type{});
            }
            const uint32_t c1 = c + CT;
            if (computes && c1 < te && c1 < wave_vis) {
                if (c1 + CT <= wave_vis_min && c1 + CT <= te)
                    consume(c1, cur + STAGE, std::true_type{});
                else
                    consume(c1, cur + STAGE, std::false_type{});
            }
        };
        uint32_t sp = 0;
        for (uint32_t c = ts; c < te; c += 2 * CT) {
            wait_vmcnt_barrier<0>();
            step2(c, stages + (sp ^ 1u) * 2 * STAGE, stages + sp * 2 * STAGE);
            sp ^= 1u;
        }
        // The last steps issued chunks nobody reads: their DMAs must land
        // before the LDS is reused.
        wait_vmcnt<0>();
    }
    __syncthreads();
    if (!computes) return;
    float* part_row = nullptr;
    if (p.partials != nullptr)
        part_row = p.partials + ((uint64_t)(row * a.kv_heads + kv_head) * p.splits + split) *
                                    (uint64_t)(qpk * (2u + kPagedAttentionHeadLimit));
    if (bad_lds != 0u) {
        // an invalid page on the way leaves the tile's outputs unwritten
        if (part_row != nullptr && row_ok && g == 0) {
#pragma unroll
            for (int i = 0; i < HPW; ++i)
                if (hv[i]) part_row[hbase + i] = __builtin_nanf("");
        }
        return;
    }
    // rows without tokens in this split (tau >= vis for all of them) are not
    // read by the combine (it uses ceil(pages(row) / per) splits)
    if (!row_ok || t_begin >= vis) return;
#pragma unroll
    for (int i = 0; i < HPW; ++i) {
        if (!hv[i]) continue;
        const uint32_t gh = hbase + (uint32_t)i;
        const uint32_t head = kv_head * qpk + gh;
        const float l_all = sum_xor32(sum_xor16(l_run[i]));
        if (part_row == nullptr) {
            // one division per (row, head), then a multiply per value
            const float inv_l = 1.0f / l_all;
#pragma unroll
            for (int db = 0; db < NDB; ++db) {
                const uint64_t oi =
                    (uint64_t)row * a.output_row_stride + (uint64_t)head * D + db * 16 + 4 * g;
                if (a.output_dtype == PSK_OUT_F32) {
                    f32x4 v = o[i][db] * inv_l;
                    *reinterpret_cast<f32x4*>(static_cast<float*>(a.output) + oi) = v;
                } else {
                    uint16_t* dst = static_cast<uint16_t*>(a.output) + oi;
                    u32x2 pk;
                    pk[0] = pack_bf16x2(o[i][db][0] * inv_l, o[i][db][1] * inv_l);
                    pk[1] = pack_bf16x2(o[i][db][2] * inv_l, o[i][db][3] * inv_l);
                    *reinterpret_cast<u32x2*>(dst) = pk;
                }
            }
        } else {
            if (g == 0) {
                part_row[gh] = m_run[i] * 0.69314718055994531f;
                part_row[qpk + gh] = l_all;
            }
#pragma unroll
            for (int db = 0; db < NDB; ++db)
                *reinterpret_cast<f32x4*>(part_row + 2u * qpk + gh * kPagedAttentionHeadLimit +
                                          db * 16 + 4 * g) = o[i][db];
        }
    }
}

// Grouped PSQ prefill tiles. Workgroup = (kTileGroup consecutive tiles of
// one sequence, head pair, kv_head, split), one wave per tile, wave w on tile w and both
// heads of the pair (as the FP8 grouped tiles). Each 32-token chunk's PSQ
// codes and block scales reach LDS by DMA; the workgroup then dequantizes
// the chunk once, every K and V value to f16(code value x block scale), into
// an f16 chunk in the BF16 tile layout (16-bit values), and the waves run the
// f16 MFMA score and PV products on it (Q and P as f16). The dequantization
// is shared by the 2 x kTileGroup (tile, head) products of the workgroup instead of being
// repeated per head, and no per-block scaling of scores or P remains.
// The scale's power of two rides on the E4M3 -> f16 conversion and its
// mantissa (exact in f16) multiplies the f16 pairs, so each value is
// rounded once, to f16 (11 bits; values below f16's normal range, 2^-14,
// keep fewer bits).
//
// Chunk k: wait + barrier A (its codes landed; every wave is done with the
// f16 chunk k - 1), DMAs of chunk k + CS - 1 into code stage (k - 1) % CS,
// dequantization of chunk k, barrier B, scores + softmax + PV of chunk k.
template <int FMT>
constexpr int pg_code_stages() { return FMT == kFmtPsq4 ? 3 : 2; }

template <int FMT, int D>
constexpr size_t tile_pg_lds_bytes() {
    return (size_t)kTilePageWindow * 4 + (size_t)pg_code_stages<FMT>() * tile_stage_bytes<FMT, D>() +
           (size_t)tile_stage_bytes<kFmtBf16, D>();
}

// RT == kTileGroup (grouped prefill): wave w owns tile w of the group and
// the HPW = 2 heads of the workgroup's head pair. RT == 1 (verify blocks,
// implicit tiles, other group sizes): the NW waves own HPW = 1 head each of
// one tile. The first 4 waves issue the DMAs; the first 4 (8 at head_dim
// 256 with 8 waves) dequantize.
template <int FMT, int D, int NW, int HPW, int RT, bool kAl16>
__global__ __launch_bounds__(NW * 64, tile_waves_per_simd(HPW)) void paged_tile_psq_group_kernel(const TileParams p) {
    constexpr int H = 2;
    constexpr int CT = 32;
    constexpr int CB = code_bytes<FMT, D>();          // code bytes of one token's head slice
    constexpr int NL = CB / 64;                       // 16 B DMA pieces per lane per half
    constexpr int NS = D / 32;                        // K-steps (= 32-value blocks)
    constexpr int NDB = D / 16;
    constexpr int SW = D / 64;                        // scale dwords per token
    constexpr int HSC = 16 * CB + 128;                // code half stride
    constexpr int KVC = H * HSC;
    constexpr int SC_BYTES = H * 256;
    constexpr int CSTAGE = tile_stage_bytes<FMT, D>();
    constexpr int CS = pg_code_stages<FMT>();
    constexpr int HSB = 16 * 2 * D + 128;             // f16 half stride
    constexpr int KVB_BYTES = H * HSB;
    constexpr int DPW = NL + 1;
    constexpr int kWinBytes = (int)kTilePageWindow * 4;
    // waves that dequantize each chunk: 8 at head_dim 256 with 8 or more
    // waves (one 32-value block per lane), else 4 (D / 128 blocks per lane)
    constexpr int NDQ = NW >= 8 && D == 256 ? 8 : 4;
    constexpr int QD = D / NDQ;                       // dims one lane dequantizes per token row
    // exponent headroom of the dequantized chunk: largest code x 2 x 2^kB
    // (PSQ4 10 x 2 x 2^11 = 40960, PSQ8 448 x 2 x 2^6 = 57344) stays below 65504
    constexpr int kB = FMT == kFmtPsq4 ? 11 : 6;
    static_assert((RT == NW && HPW == 2) || (RT == 1 && HPW == 1), "tile geometry");
    static_assert(NW >= 4 && NS % 2 == 0 && D % 128 == 0, "geometry");

    extern __shared__ __align__(16) uint8_t lds[];
    __shared__ uint32_t bad_lds;
    __shared__ uint32_t group_vis;

    const psk_paged_attention_args& a = p.a;
    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid & 63u, w = tid >> 6;
    const uint32_t n = lane & 15u, g = lane >> 4;
    const uint32_t qpk = a.q_heads / a.kv_heads;

    uint32_t split, hpart, kv_head, group;
    if (!tile_workgroup<NW, HPW, RT>(p, qpk, split, hpart, kv_head, group)) return;
    // the group's first tile names the sequence (workgroup-uniform)
    uint32_t g0;
    if (p.n_tiles != 0u) {
        if (group * RT >= p.n_tiles) return;
        g0 = p.tile_begin[group * RT];
    } else {
        g0 = group * RT * kTileRows;
    }
    if (g0 >= a.rows) return;
    const uint32_t slot = a.row_sequence_slots[g0];
    if (slot >= a.max_sequences) return;
    const uint32_t tile = group * RT + (RT > 1 ? w : 0u);
    uint32_t r0, nrows;
    if (p.n_tiles != 0u) {
        const bool have = tile < p.n_tiles;
        r0 = have ? p.tile_begin[tile] : g0;
        nrows = have ? p.tile_rows[tile] : 0u;
    } else {
        r0 = tile * kTileRows;
        nrows = r0 < a.rows ? min((uint32_t)kTileRows, a.rows - r0) : 0u;
    }
    if (r0 >= a.rows) nrows = 0u;
    nrows = min(nrows, a.rows - min(r0, a.rows));

    const uint64_t cap = (uint64_t)a.block_table_stride * a.page_tokens;
    const uint32_t row = r0 + n;
    bool row_ok = n < nrows && a.row_sequence_slots[min(row, a.rows - 1u)] == slot;
    uint32_t vis = 0;
    if (row_ok) {
        const uint64_t v64 = (uint64_t)a.row_positions[row] + 1u;
        row_ok = v64 <= cap;
        vis = row_ok ? (uint32_t)v64 : 0u;
    }
    uint32_t wave_vis = vis;
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) wave_vis = max(wave_vis, (uint32_t)__shfl_xor((int)wave_vis, o, 64));
    uint32_t wave_vis_min = row_ok ? vis : 0xFFFFFFFFu;
#pragma unroll
    for (int o = 1; o < 16; o <<= 1)
        wave_vis_min = min(wave_vis_min, (uint32_t)__shfl_xor((int)wave_vis_min, o, 64));
    uint32_t vis_max = wave_vis;   // RT == 1: every wave holds the tile's rows
    if constexpr (RT > 1) {
        // the workgroup streams the longest visible range of its tiles
        if (tid == 0) group_vis = 0u;
        __syncthreads();
        if (lane == 0) atomicMax(&group_vis, wave_vis);
        __syncthreads();
        vis_max = group_vis;
    }
    if (vis_max == 0u) return;   // uniform over the workgroup
    const uint32_t P = a.page_tokens;
    const uint32_t pc = (vis_max + P - 1u) / P;
    const uint32_t per = p.pages_per_split != 0u ? p.pages_per_split : (pc + p.splits - 1u) / p.splits;
    const uint32_t pb = split * per;
    if (pb >= pc) return;
    const uint32_t pe = (split == p.splits - 1u) ? pc : min(pc, pb + per);
    const uint32_t t_begin = pb * P, t_end = min(pe * P, vis_max);
    const uint32_t* bt = a.block_tables + (uint64_t)slot * a.block_table_stride;
    const uint64_t scale_layer = (uint64_t)a.layer * a.num_pages;
    // everything above is uniform over the workgroup: all waves reach the
    // barriers below
    const uint32_t hbase = RT > 1 ? hpart * HPW : w * HPW;   // first head (group index)
    const bool computes = hbase < qpk && wave_vis > 0u;
    bool hv[HPW];
#pragma unroll
    for (int i = 0; i < HPW; ++i) hv[i] = hbase + (uint32_t)i < qpk;
    if (tid == 0) bad_lds = 0u;

    // Q fragments as f16, in the BF16 tiles' order: K-step s, dims 32s + 8g ..
    // +8, of q * 2^sq with sq = 14 - E for the workgroup's max|q| = m * 2^E (m
    // in [0.5, 1)): the largest |value| lies in [2^13, 2^14), inside f16's
    // range whatever the magnitude of q, and values down to 2^-27 of it stay
    // in f16's normal range. The scores take qinv = 2^-sq (workgroup-uniform).
    //
    // K and V values likewise: with Ek (Ev) the largest biased exponent of the
    // block scales of the workgroup's K (V) tokens [t_begin, t_end), every
    // value is dequantized as f16(code x scale x 2^(kB + 127 - Ek)), so the
    // largest stays below 2^(kB + 1) x the largest code, inside f16's range for
    // any block scale. The scores take 2^(Ek - kB - 127) with the softmax
    // scale, and O is accumulated in units of 2^(Ev - kB - 127).
    __shared__ uint32_t wg_max_w[3][NW];
    f16x8 qf[HPW][NS];
    float qinv;
    int ek, ev;
    {
        u32x4 w_[HPW][NS];
        float amax = 0.0f;
#pragma unroll
        for (int i = 0; i < HPW; ++i) {
            const uint32_t head = kv_head * qpk + (hv[i] ? hbase + (uint32_t)i : 0u);
            const uint16_t* qrow = static_cast<const uint16_t*>(a.q) +
                                   (uint64_t)(row_ok ? row : r0) * a.q_row_stride + (uint64_t)head * D;
#pragma unroll
            for (int s = 0; s < NS; ++s) {
                w_[i][s] = __builtin_bit_cast(u32x4, q8(qrow + s * 32 + (int)g * 8, row_ok && hv[i]));
#pragma unroll
                for (int k = 0; k < 4; ++k)
                    amax = __builtin_fmaxf(amax,
                                           __builtin_fmaxf(__builtin_fabsf(__uint_as_float(w_[i][s][k] << 16)),
                                                           __builtin_fabsf(__uint_as_float(w_[i][s][k] & 0xFFFF0000u))));
            }
        }
        // block-scale exponents of the tokens [t_begin, t_end): 8 tokens per
        // thread per pass, their page ids first, then their SW scale dwords of
        // K and V (bf16 pairs; masks keep the exponent fields, compared as
        // integers)
        uint32_t kmax = 0u, vmax = 0u;
        const uint32_t* ksp = reinterpret_cast<const uint32_t*>(p.k_scale);
        const uint32_t* vsp = reinterpret_cast<const uint32_t*>(p.v_scale);
        for (uint32_t t0 = t_begin + tid; t0 < t_end; t0 += 8u * NW * 64u) {
            uint32_t pg[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const uint32_t t = t0 + (uint32_t)u * NW * 64u;
                pg[u] = t < t_end ? bt[t / P] : 0xFFFFFFFFu;
            }
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const uint32_t t = t0 + (uint32_t)u * NW * 64u;
                if (pg[u] >= a.num_pages) continue;
                const uint64_t si = (((scale_layer + pg[u]) * P + t % P) * a.kv_heads + kv_head) * (uint64_t)SW;
#pragma unroll
                for (int k = 0; k < SW; ++k) {
                    const uint32_t x = ksp[si + k], y = vsp[si + k];
                    kmax = max(kmax, max(x & 0x7F800000u, (x & 0x7F80u) << 16));
                    vmax = max(vmax, max(y & 0x7F800000u, (y & 0x7F80u) << 16));
                }
            }
        }
        amax = wave_max(amax);
        kmax = wave_max_u32(kmax);
        vmax = wave_max_u32(vmax);
        if (lane == 0u) {
            wg_max_w[0][w] = __float_as_uint(amax);
            wg_max_w[1][w] = kmax;
            wg_max_w[2][w] = vmax;
        }
        __syncthreads();
        uint32_t am = 0u;
        kmax = 0u;
        vmax = 0u;
#pragma unroll
        for (int j = 0; j < NW; ++j) {
            am = max(am, wg_max_w[0][j]);   // non-negative floats order as integers
            kmax = max(kmax, wg_max_w[1][j]);
            vmax = max(vmax, wg_max_w[2][j]);
        }
        amax = __uint_as_float(am);
        ek = (int)__builtin_amdgcn_readfirstlane(kmax >> 23);
        ev = (int)__builtin_amdgcn_readfirstlane(vmax >> 23);
        const int sq = __builtin_amdgcn_readfirstlane(
            (amax > 0.0f && amax <= 3.0e38f) ? 14 - __builtin_amdgcn_frexp_expf(amax) : 0);
        qinv = uniform_f32(__builtin_ldexpf(1.0f, -sq));
#pragma unroll
        for (int i = 0; i < HPW; ++i)
#pragma unroll
            for (int s = 0; s < NS; ++s) {
                u32x4 h;
#pragma unroll
                for (int k = 0; k < 4; ++k)
                    h[k] = pack_f16x2(__builtin_ldexpf(__uint_as_float(w_[i][s][k] << 16), sq),
                                      __builtin_ldexpf(__uint_as_float(w_[i][s][k] & 0xFFFF0000u), sq));
                qf[i][s] = __builtin_bit_cast(f16x8, h);
            }
    }
    // softmax scale x qinv x 2^(Ek - kB - 127); the dequantization's exponent
    // offsets (value bits - eshift) of K and V
    const float sl = uniform_f32(p.scale_log2 * qinv * __builtin_ldexpf(1.0f, ek - kB - 127));
    const int eshift_k = (ek - kB - 127) * (1 << 23);
    const int eshift_v = (ev - kB - 127) * (1 << 23);
    float m_run[HPW], l_run[HPW];
    f32x4 o[HPW][NDB];
#pragma unroll
    for (int i = 0; i < HPW; ++i) {
        m_run[i] = -INFINITY;
        l_run[i] = 0.0f;
#pragma unroll
        for (int db = 0; db < NDB; ++db) o[i][db] = (f32x4){0.f, 0.f, 0.f, 0.f};
    }
    // BF16 transposing V reads: token 4g + (n>>2) of each half, dims +4(n&3)
    const uint32_t tr_off = 16u * (4u * g + (n >> 2)) + 256u * ((n >> 1) & 1u) + 8u * (n & 1u);

    uint32_t* const win = reinterpret_cast<uint32_t*>(lds);
    uint8_t* const cstages = lds + kWinBytes;
    uint8_t* const bst = cstages + CS * CSTAGE;       // the f16 chunk
    const uint32_t wu = __builtin_amdgcn_readfirstlane(w);
    // dequantization: wave w < NDQ takes (kind, half, dim part) = ((w / 2) % 2,
    // w % 2, w / 4), lane (t, q) token t, dims [QD j, QD (j + 1)) with j =
    // (NDQ / 4) q + w / 4. The LDS serves 8 lanes of a 16 B access per clock;
    // they are 8 tokens of one 16 B column, whose rows sit 16 B apart, so the
    // 8 accesses hit distinct banks.
    const uint32_t dq = (uint32_t)(NDQ / 4) * g + (w >> 2);
    const uint32_t d_kind = (w >> 1) & 1u, d_half = w & 1u, d_tok = n;

    for (uint32_t wp = pb; wp < pe; wp += kTilePageWindow) {
        const uint32_t wp_end = min(pe, wp + kTilePageWindow);
        __syncthreads();
        for (uint32_t i = tid; i < wp_end - wp; i += NW * 64u) win[i] = bt[wp + i];
        __syncthreads();
        const uint32_t ts = max(wp * P, t_begin);
        const uint32_t te = min(wp_end * P, t_end);
        if (ts >= te) continue;
        const uint32_t t_last = te - 1u;
        const uint32_t K = (te - ts + CT - 1u) / CT;
        const uint32_t tok_bytes = a.kv_heads * (uint32_t)CB;
        // wave wu: stream (K | V, half wu % 2) of chunk ci: NL code pieces and
        // dword g of each token's block scales (lane groups past SW repeat one)
        auto issue = [&](uint32_t ci, uint8_t* st) __attribute__((always_inline)) {
            if (NW > 4 && wu >= 4u) return;
            const uint32_t c = ts + ci * CT;
            const uint32_t hf = wu % (uint32_t)H;
            const uint32_t kind = wu / (uint32_t)H;
            const uint32_t tau = min(c + hf * 16u + n, t_last);
            uint32_t page, off;
            if constexpr (kAl16) {
                const uint32_t hb = min(c + hf * 16u, t_last);
                const uint32_t pi = hb / P;
                page = __builtin_amdgcn_readfirstlane(win[pi - wp]);
                off = tau - pi * P;
            } else {
                page = win[tau / P - wp];
                off = tau % P;
            }
            const bool inv = page >= a.num_pages;
            if (inv) bad_lds = 1u;
            const uint32_t pg = inv ? 0u : page;
            const uint64_t slice0 = ((scale_layer + pg) * P * a.kv_heads + kv_head) * (uint64_t)CB;
            const uint8_t* src = (kind == 0u ? p.k_pool : p.v_pool) + slice0;
            uint8_t* dst = st + kind * KVC + hf * HSC;
            const uint32_t lo = off * tok_bytes + g * 16u;
#pragma unroll
            for (int i = 0; i < NL; ++i) load_lds<16>(src + (lo + i * 64u), dst + i * 1024);
            const uint64_t si = ((scale_layer + pg) * P + off) * a.kv_heads + kv_head;
            const uint8_t* sbase = reinterpret_cast<const uint8_t*>(kind == 0u ? p.k_scale : p.v_scale);
            load_lds<4>(sbase + si * (2u * D / 32u) + 4u * min(g, (uint32_t)SW - 1u),
                        st + 2 * KVC + kind * SC_BYTES + hf * 256);
        };
        // code stage st -> f16 chunk: this lane's token row, QD dims, each
        // value scaled by 2^(kB + 127 - Ek) (K) or 2^(kB + 127 - Ev) (V)
        auto dequant = [&](const uint8_t* st, uint8_t* bo) __attribute__((always_inline)) {
            if (NW > NDQ && wu >= (uint32_t)NDQ) return;
            const int eshift = d_kind == 0u ? eshift_k : eshift_v;   // wave-uniform
            const uint8_t* cb = st + d_kind * KVC + d_half * HSC + 16u * d_tok;
            const uint8_t* sc = st + 2 * KVC + d_kind * SC_BYTES + d_half * 256 + 4u * d_tok;
            uint8_t* ob = bo + d_kind * KVB_BYTES + d_half * HSB + 16u * d_tok;
#pragma unroll
            for (int bl = 0; bl < QD / 32; ++bl) {
                const uint32_t s = dq * (QD / 32) + bl;   // block
                const uint32_t sw = *reinterpret_cast<const uint32_t*>(sc + 64u * (s >> 1));
                const uint32_t sb = (s & 1u) ? (sw & 0xFFFF0000u) : (sw << 16);   // the scale, f32 bits
                // scale = 2^e x m: 2^e rides on the conversion, m in [1, 2)
                // (exact in f16) multiplies the f16 pairs
                const float s_pow2 = __uint_as_float((uint32_t)max((int)(sb & 0x7F800000u) - eshift, 0));
                const uint32_t m2 = pack_f16x2(__uint_as_float((sb & 0x807FFFFFu) | 0x3F800000u),
                                               __uint_as_float((sb & 0x807FFFFFu) | 0x3F800000u));
                // the block's 32 values as E4M3 bytes, dims 32s + 0 .. 31
                uint32_t e[8];
                if constexpr (FMT == kFmtPsq8) {
                    // bytes 32s .. +32 of the token: pieces (32s + 16j) / 16
#pragma unroll
                    for (int j = 0; j < 2; ++j) {
                        const uint32_t b = 32u * s + 16u * (uint32_t)j;
                        const u32x4 x = *reinterpret_cast<const u32x4*>(cb + 1024u * (b >> 6) +
                                                                        256u * ((b & 63u) >> 4));
#pragma unroll
                        for (int k = 0; k < 4; ++k) e[4 * j + k] = x[k];
                    }
                } else {
                    // bytes 16s .. +16: byte i low nibble = dim 32s + i, high = 32s + 16 + i
                    const uint32_t b = 16u * s;
                    const u32x4 x = *reinterpret_cast<const u32x4*>(cb + 1024u * (b >> 6) + 256u * ((b & 63u) >> 4));
#pragma unroll
                    for (int k = 0; k < 4; ++k) {
                        e[k] = psq4_e4m3x4(x[k], false);
                        e[4 + k] = psq4_e4m3x4(x[k], true);
                    }
                }
                // f16(value x scale): 32 values = 4 16 B pieces of the f16 row
#pragma unroll
                for (int pc2 = 0; pc2 < 4; ++pc2) {
                    u32x4 r;
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        const uint32_t x = e[2 * pc2 + h];
                        const f16x2 lo2 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(x, s_pow2, false);
                        const f16x2 hi2 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(x, s_pow2, true);
                        r[2 * h] = __builtin_bit_cast(uint32_t, lo2 * __builtin_bit_cast(f16x2, m2));
                        r[2 * h + 1] = __builtin_bit_cast(uint32_t, hi2 * __builtin_bit_cast(f16x2, m2));
                    }
                    const uint32_t b = 64u * s + 16u * (uint32_t)pc2;   // f16 row byte
                    *reinterpret_cast<u32x4*>(ob + 1024u * (b >> 6) + 256u * ((b & 63u) >> 4)) = r;
                }
            }
        };
        // scores, causal online softmax and PV of the f16 chunk at c
        auto consume = [&](uint32_t c, const uint8_t* bi, auto full_tag) __attribute__((always_inline)) {
            constexpr bool kFull = decltype(full_tag)::value;
            constexpr int NP = NS / 2;
            f32x4 sc[HPW][H];
            struct KRaw {
                u32x4 a, b;
            };
            auto kread = [&](int u) __attribute__((always_inline)) {
                const uint8_t* kb = bi + (u / NP) * HSB + 16 * lane;
                KRaw r;
                r.a = *reinterpret_cast<const u32x4*>(kb + 1024 * (2 * (u % NP)));
                r.b = *reinterpret_cast<const u32x4*>(kb + 1024 * (2 * (u % NP) + 1));
                return r;
            };
            f32x4 acc[HPW];
            KRaw cur = kread(0);
            __builtin_amdgcn_s_setprio(1);
#pragma unroll
            for (int u = 0; u < H * NP; ++u) {
                KRaw nxt = cur;
                if (u + 1 < H * NP) nxt = kread(u + 1);
                __builtin_amdgcn_sched_barrier(0);
                const int sp = u % NP;
                if (sp == 0) {
#pragma unroll
                    for (int i = 0; i < HPW; ++i) acc[i] = (f32x4){0.f, 0.f, 0.f, 0.f};
                }
                const f16x8 k0 = __builtin_bit_cast(f16x8, cur.a);
                const f16x8 k1 = __builtin_bit_cast(f16x8, cur.b);
#pragma unroll
                for (int i = 0; i < HPW; ++i)
                    acc[i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(k0, qf[i][2 * sp], acc[i], 0, 0, 0);
#pragma unroll
                for (int i = 0; i < HPW; ++i)
                    acc[i] = __builtin_amdgcn_mfma_f32_16x16x32_f16(k1, qf[i][2 * sp + 1], acc[i], 0, 0, 0);
                if (sp == NP - 1) {
#pragma unroll
                    for (int i = 0; i < HPW; ++i) sc[i][u / NP] = acc[i];
                }
                cur = nxt;
            }
            __builtin_amdgcn_s_setprio(0);
            bool tok_ok[H][4];
#pragma unroll
            for (int hf = 0; hf < H; ++hf)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const uint32_t tau = c + hf * 16 + 4 * g + r;
                    tok_ok[hf][r] = kFull || (tau < vis && tau < te);
                }
            u32x4 pf[HPW];
#pragma unroll
            for (int i = 0; i < HPW; ++i) {
                float s2[H][4];
                float mx = -INFINITY;
#pragma unroll
                for (int hf = 0; hf < H; ++hf)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        s2[hf][r] = tok_ok[hf][r] ? sc[i][hf][r] * sl : -INFINITY;
                        mx = __builtin_fmaxf(mx, s2[hf][r]);
                    }
                mx = max_xor32(max_xor16(mx));
                const bool moved = mx > m_run[i] + kLazyMaxSlack;
                const float m_new = moved ? mx : m_run[i];
                const float m_use = m_new == -INFINITY ? 0.0f : m_new;
                const float alpha = moved ? __builtin_amdgcn_exp2f(m_run[i] - m_use) : 1.0f;
                float pv[H][4], psum = 0.0f;
#pragma unroll
                for (int hf = 0; hf < H; ++hf)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const float e = __builtin_amdgcn_exp2f(s2[hf][r] - m_use);
                        psum += e;
                        pv[hf][r] = e;
                    }
                l_run[i] = l_run[i] * alpha + psum;
                m_run[i] = m_new;
                if (__any(moved)) {
#pragma unroll
                    for (int db = 0; db < NDB; ++db) o[i][db] *= alpha;
                }
                // P as one f16 operand
                pf[i][0] = pack_f16x2(pv[0][0], pv[0][1]);
                pf[i][1] = pack_f16x2(pv[0][2], pv[0][3]);
                pf[i][2] = pack_f16x2(pv[1][0], pv[1][1]);
                pf[i][3] = pack_f16x2(pv[1][2], pv[1][3]);
            }
            // O^T += V^T P^T, V^T fragments by transposing reads, in pairs of
            // output blocks read one pair ahead
            const uint8_t* vb = bi + KVB_BYTES + tr_off;
            auto vread = [&](int db) __attribute__((always_inline)) {
                const i16x4 x0 = tr16(vb + 512 * db);
                const i16x4 x1 = tr16(vb + HSB + 512 * db);
                return (u32x4){__builtin_bit_cast(u32x2, x0)[0], __builtin_bit_cast(u32x2, x0)[1],
                               __builtin_bit_cast(u32x2, x1)[0], __builtin_bit_cast(u32x2, x1)[1]};
            };
            u32x4 vc[2] = {vread(0), vread(1)};
            __builtin_amdgcn_s_setprio(1);
#pragma unroll
            for (int pr = 0; pr < NDB / 2; ++pr) {
                u32x4 vn[2] = {vc[0], vc[1]};
                if (pr + 1 < NDB / 2) {
                    vn[0] = vread(2 * pr + 2);
                    vn[1] = vread(2 * pr + 3);
                }
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const f16x8 vf = __builtin_bit_cast(f16x8, vc[j]);
#pragma unroll
                    for (int i = 0; i < HPW; ++i)
                        o[i][2 * pr + j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
                            vf, __builtin_bit_cast(f16x8, pf[i]), o[i][2 * pr + j], 0, 0, 0);
                }
                vc[0] = vn[0];
                vc[1] = vn[1];
            }
            __builtin_amdgcn_s_setprio(0);
        };

        // chunk k: barrier A, DMAs of chunk k + CS - 1, dequantization,
        // barrier B, compute. __restrict__ tells the compiler that the DMAs
        // into `next` and the reads of `cur` touch different LDS; their real
        // ordering is the wait + barrier.
        auto step = [&](uint32_t k, uint8_t* __restrict__ next, const uint8_t* __restrict__ cur,
                        uint8_t* __restrict__ bchunk) __attribute__((always_inline)) {
            issue(k + (uint32_t)CS - 1u, next);
            dequant(cur, bchunk);
            asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
            const uint32_t c = ts + k * CT;
            if (computes && c < wave_vis) {
                if (c + CT <= wave_vis_min && c + CT <= te)
                    consume(c, bchunk, std::true_type{});
                else
                    consume(c, bchunk, std::false_type{});
            }
        };
#pragma unroll
        for (int l = 0; l < CS - 1; ++l) issue((uint32_t)l, cstages + l * CSTAGE);
        for (uint32_t k = 0; k < K; ++k) {
            // chunk k landed (CS - 2 later chunks outstanding); every wave is
            // done with the f16 chunk and with code stage (k - 1) % CS
            asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"((CS - 2) * DPW) : "memory");
            step(k, cstages + ((k + (uint32_t)CS - 1u) % (uint32_t)CS) * CSTAGE, cstages + (k % (uint32_t)CS) * CSTAGE,
                 bst);
        }
        wait_vmcnt<0>();   // the DMAs of chunks nobody reads
    }
    __syncthreads();
    if (!computes) return;
    float* part_row = nullptr;
    if (p.partials != nullptr)
        part_row = p.partials + ((uint64_t)(row * a.kv_heads + kv_head) * p.splits + split) *
                                    (uint64_t)(qpk * (2u + kPagedAttentionHeadLimit));
    if (bad_lds != 0u) {
        if (part_row != nullptr && row_ok && g == 0) {
#pragma unroll
            for (int i = 0; i < HPW; ++i)
                if (hv[i]) part_row[hbase + i] = __builtin_nanf("");
        }
        return;
    }
    if (!row_ok || t_begin >= vis) return;
    // O in true units: x 2^gu, gu = Ev - kB - 127, as two factors 2^(gu / 2)
    // and 2^(gu - gu / 2), each inside fp32's range
    const int gu = ev - kB - 127;
    const float f_lo = __builtin_ldexpf(1.0f, gu >> 1);
    const float f_hi = __builtin_ldexpf(1.0f, gu - (gu >> 1));
#pragma unroll
    for (int i = 0; i < HPW; ++i) {
        if (!hv[i]) continue;
        const uint32_t gh = hbase + (uint32_t)i;
        const uint32_t head = kv_head * qpk + gh;
        const float l_all = sum_xor32(sum_xor16(l_run[i]));
        const float f_out = f_hi / l_all;
        if (part_row == nullptr) {
#pragma unroll
            for (int db = 0; db < NDB; ++db) {
                const uint64_t oi = (uint64_t)row * a.output_row_stride + (uint64_t)head * D + db * 16 + 4 * g;
                if (a.output_dtype == PSK_OUT_F32) {
                    f32x4 v;
#pragma unroll
                    for (int r = 0; r < 4; ++r) v[r] = (o[i][db][r] * f_lo) * f_out;
                    *reinterpret_cast<f32x4*>(static_cast<float*>(a.output) + oi) = v;
                } else {
                    uint16_t* dst = static_cast<uint16_t*>(a.output) + oi;
                    u32x2 pk;
                    pk[0] = pack_bf16x2((o[i][db][0] * f_lo) * f_out, (o[i][db][1] * f_lo) * f_out);
                    pk[1] = pack_bf16x2((o[i][db][2] * f_lo) * f_out, (o[i][db][3] * f_lo) * f_out);
                    *reinterpret_cast<u32x2*>(dst) = pk;
                }
            }
        } else {
            if (g == 0) {
                part_row[gh] = m_run[i] * 0.69314718055994531f;
                part_row[qpk + gh] = l_all;
            }
#pragma unroll
            for (int db = 0; db < NDB; ++db)
            {
                f32x4 v;
#pragma unroll
                for (int r = 0; r < 4; ++r) v[r] = (o[i][db][r] * f_lo) * f_hi;
                *reinterpret_cast<f32x4*>(part_row + 2u * qpk + gh * kPagedAttentionHeadLimit + db * 16 + 4 * g) = v;
            }
        }
    }
}

template <int FMT, int D, int NW, int HPW, int RT, bool kAl16>
hipError_t launch_tile_pg_t(const TileParams& p, uint64_t grid, hipStream_t stream) {
    constexpr size_t lds_bytes = tile_pg_lds_bytes<FMT, D>();
    static std::atomic<uint64_t> lds_ready{0};
    const hipError_t attr = allow_full_lds(
        reinterpret_cast<const void*>(&paged_tile_psq_group_kernel<FMT, D, NW, HPW, RT, kAl16>), lds_ready);
    if (attr != hipSuccess) return attr;
    hipLaunchKernelGGL((paged_tile_psq_group_kernel<FMT, D, NW, HPW, RT, kAl16>), dim3((uint32_t)grid),
                       dim3(NW * 64), lds_bytes, stream, p);
    return hipGetLastError();
}

template <int FMT, int D, int NW, int HPW, int RT>
hipError_t launch_tile_pg(const TileParams& p, uint64_t grid, hipStream_t stream) {
    return (p.a.page_tokens & 15u) == 0u ? launch_tile_pg_t<FMT, D, NW, HPW, RT, true>(p, grid, stream)
                                         : launch_tile_pg_t<FMT, D, NW, HPW, RT, false>(p, grid, stream);
}

// kv_dtype: PSK_KV_*. PSQ: head_dim 128 or 256 (every (token, head) code
// slice then starts on 16 B), scale pools 4 B aligned (checked by the
// launchers that take them).
bool tile_shape_ok(const psk_paged_attention_args& c, uint32_t kv_dtype, const void* kp, const void* vp) {
    const uint32_t qpk = c.q_heads / c.kv_heads;
    if (qpk == 0u || qpk > (uint32_t)kMaxTileHeads) return false;
    const uint32_t D = c.head_dim;
    const bool psq = kv_dtype == PSK_KV_PSQ4_W32 || kv_dtype == PSK_KV_PSQ8_W32;
    if (psq) {
        if (!(D == 128 || D == 256)) return false;
    } else {
        const uint32_t kvb = kv_dtype == PSK_KV_FP8_E4M3 ? 1u : 2u;
        if (!(D == 64 || D == 128 || D == 256 || (D == 32 && kvb == 2))) return false;
        const uint32_t al = 16u / kvb;
        if (c.elems_per_token % al || c.elems_per_page % al || c.elems_per_layer % al) return false;
    }
    if (reinterpret_cast<uintptr_t>(kp) % 16u || reinterpret_cast<uintptr_t>(vp) % 16u) return false;
    // vector output stores: 16 B (f32) / 8 B (bf16) at head*D + 4*k
    const uint32_t oal = c.output_dtype == PSK_OUT_F32 ? 4u : 4u;
    if (c.output_row_stride % oal || reinterpret_cast<uintptr_t>(c.output) % 16u) return false;
    return true;
}

template <int FMT, int D, int NW, int HPW, int RT, bool kAl16>
hipError_t launch_tile_t3(const TileParams& p, uint64_t grid, hipStream_t stream) {
    const size_t lds_bytes = (size_t)kTilePageWindow * 4 + (size_t)kTileStages * tile_stage_bytes<FMT, D>();
    if (lds_bytes > 64u * 1024u) {
        // gfx950 has 160 KB of LDS per CU; raise the per-kernel dynamic limit.
        static std::atomic<uint64_t> lds_ready{0};
        const hipError_t attr =
            allow_full_lds(reinterpret_cast<const void*>(&paged_tile_kernel<FMT, D, NW, HPW, RT, kAl16>), lds_ready);
        if (attr != hipSuccess) return attr;
    }
    hipLaunchKernelGGL((paged_tile_kernel<FMT, D, NW, HPW, RT, kAl16>), dim3((uint32_t)grid),
                       dim3(NW * 64), lds_bytes, stream, p);
    return hipGetLastError();
}

template <int FMT, int D, int NW, int HPW, int RT = 1>
hipError_t launch_tile_t2(const TileParams& p, uint64_t grid, hipStream_t stream) {
    return (p.a.page_tokens & 15u) == 0u ? launch_tile_t3<FMT, D, NW, HPW, RT, true>(p, grid, stream)
                                         : launch_tile_t3<FMT, D, NW, HPW, RT, false>(p, grid, stream);
}

// Waves and heads per wave by group size: up to 4 heads one per wave (4
// waves, so every SIMD issues part of the DMAs); 5-6 heads one per wave (6
// waves: two workgroups put 3 waves on every SIMD); 7-8 heads one per wave
// (8 waves, two on every SIMD). Two heads per wave on 4 waves, the earlier
// layout for 7-8 heads, spilled over 100 registers at head_dim 256 and ran
// 2.3-2.7x slower (32/4 heads: 8 verify blocks 156 -> 67 us, a 512-row
// prefill chunk 839 -> 314 us).
// Grouped launches (tiles_per_group == kTileGroup, 1-8 heads): kTileGroup
// waves, one per tile, each on two heads of the group's head part, so each
// converted K/V fragment feeds two MFMAs; 2 waves on every SIMD.
// Wave counts that load the SIMDs unevenly (3 waves per workgroup) lose: the
// chunk barrier waits on the doubly loaded SIMDs. PSQ grouped launches go to
// paged_tile_psq_group_kernel (the same workgroup shape on a shared f16
// dequantization of each chunk).
template <int FMT, int D>
hipError_t launch_tile_t(const TileParams& p, hipStream_t stream) {
    const uint32_t qpk = p.a.q_heads / p.a.kv_heads;
    const uint64_t tiles = p.n_tiles != 0u ? p.n_tiles : (p.a.rows + kTileRows - 1) / kTileRows;
    const bool grouped = p.tiles_per_group == (uint32_t)kTileGroup && grouped_heads(qpk);
    const uint64_t grid = grouped ? (tiles + kTileGroup - 1) / kTileGroup * ((qpk + 1u) / 2u) * p.a.kv_heads * p.splits
                                  : tiles * p.a.kv_heads * p.splits;
    if (grid == 0u || grid > 0x7FFFFFFFull) return hipErrorInvalidValue;
    if constexpr (fmt_psq<FMT>()) {
        // PSQ: one shared f16 dequantization per chunk, then f16 MFMAs
        // (paged_tile_psq_group_kernel); ungrouped one head per wave
        if (grouped) return launch_tile_pg<FMT, D, kTileGroup, 2, kTileGroup>(p, grid, stream);
        // 5-8 heads on 8 waves: at head_dim 256 all 8 share the chunk's
        // dequantization (5-6 heads: the reference's prefill launcher over
        // config 5's chunks 2.13 -> 1.87 ms PSQ4, 2.17 -> 1.95 ms PSQ8
        // against 6 waves with 4 dequantizing)
        if (qpk <= 4u) return launch_tile_pg<FMT, D, 4, 1, 1>(p, grid, stream);
        return launch_tile_pg<FMT, D, 8, 1, 1>(p, grid, stream);
    } else {
        if (grouped) return launch_tile_t2<FMT, D, kTileGroup, 2, kTileGroup>(p, grid, stream);
        if (qpk <= 4u) return launch_tile_t2<FMT, D, 4, 1>(p, grid, stream);
        if (qpk <= 6u) return launch_tile_t2<FMT, D, 6, 1>(p, grid, stream);
        return launch_tile_t2<FMT, D, 8, 1>(p, grid, stream);
    }
}

template <int FMT>
hipError_t launch_tile(const TileParams& p, hipStream_t stream) {
    switch (p.a.head_dim) {
        case 256: return launch_tile_t<FMT, 256>(p, stream);
        case 128: return launch_tile_t<FMT, 128>(p, stream);
        case 64:
            if constexpr (!fmt_psq<FMT>()) return launch_tile_t<FMT, 64>(p, stream);
            return hipErrorNotSupported;
        case 32:
            if constexpr (FMT == kFmtBf16) return launch_tile_t<kFmtBf16, 32>(p, stream);
            return hipErrorNotSupported;
        default: return hipErrorNotSupported;
    }
}

// kv_dtype: PSK_KV_*; checked by the callers
hipError_t launch_tile_fmt(const TileParams& p, uint32_t kv_dtype, hipStream_t stream) {
    switch (kv_dtype) {
        case PSK_KV_BF16: return launch_tile<kFmtBf16>(p, stream);
        case PSK_KV_FP8_E4M3: return launch_tile<kFmtFp8>(p, stream);
        case PSK_KV_PSQ8_W32: return launch_tile<kFmtPsq8>(p, stream);
        case PSK_KV_PSQ4_W32: return launch_tile<kFmtPsq4>(p, stream);
        default: return hipErrorInvalidValue;
    }
}

bool known_kv(uint32_t kv_dtype) {
    return kv_dtype == PSK_KV_BF16 || kv_dtype == PSK_KV_FP8_E4M3 || kv_dtype == PSK_KV_PSQ4_W32 ||
           kv_dtype == PSK_KV_PSQ8_W32;
}

// PSQ scale pools: bf16 block scales, read by 4 B DMAs
bool psq_scales_ok(uint32_t kv_dtype, const void* ks, const void* vs) {
    if (kv_dtype != PSK_KV_PSQ4_W32 && kv_dtype != PSK_KV_PSQ8_W32) return true;
    return ks != nullptr && vs != nullptr && reinterpret_cast<uintptr_t>(ks) % 4u == 0u &&
           reinterpret_cast<uintptr_t>(vs) % 4u == 0u;
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
    p.tiles_per_group = 1u;
    return p;
}

}  // namespace

// Tile launch over explicit tiles (row_begin, rows) of one launch, any
// number of them (chunks of kInlineTiles per launch). Used by the step
// planner; every tile's rows must belong to one sequence.
// ks / vs: FP8 f32 scale pools, PSQ bf16 block-scale pools, BF16 unused.
hipError_t launch_paged_tiles(const psk_paged_attention_args& a, uint32_t kv_dtype, const void* k,
                              const void* v, const void* ks, const void* vs,
                              const uint32_t* tile_begin, const uint32_t* tile_rows,
                              uint32_t n_tiles, uint32_t tiles_per_group, float* partials,
                              uint32_t splits, uint32_t pages_per_split, hipStream_t stream) {
    const hipError_t e = tile_validate(&a, k, v);
    if (e != hipSuccess) return e;
    if (!known_kv(kv_dtype)) return hipErrorInvalidValue;
    if (!tile_shape_ok(a, kv_dtype, k, v) || !psq_scales_ok(kv_dtype, ks, vs)) return hipErrorNotSupported;
    if (splits > 1u && (partials == nullptr || pages_per_split == 0u)) return hipErrorInvalidValue;
    if (tiles_per_group != 1u &&
        (tiles_per_group != (uint32_t)kTileGroup || n_tiles % (uint32_t)kTileGroup != 0u))
        return hipErrorInvalidValue;
    for (uint32_t b = 0; b < n_tiles; b += kInlineTiles) {
        TileParams p = make_tile(a, k, v, static_cast<const float*>(ks), static_cast<const float*>(vs),
                                 splits > 1u ? partials : nullptr, splits, pages_per_split);
        p.tiles_per_group = tiles_per_group;
        p.n_tiles = n_tiles - b < kInlineTiles ? n_tiles - b : kInlineTiles;
        for (uint32_t i = 0; i < p.n_tiles; ++i) {
            // rows == 0 only pads a group after its first tile
            const bool pad_ok = tiles_per_group > 1u && i % tiles_per_group != 0u;
            if ((tile_rows[b + i] == 0u && !pad_ok) || tile_rows[b + i] > (uint32_t)kTileRows)
                return hipErrorInvalidValue;
            p.tile_begin[i] = tile_begin[b + i];
            p.tile_rows[i] = static_cast<uint8_t>(tile_rows[b + i]);
        }
        const hipError_t le = launch_tile_fmt(p, kv_dtype, stream);
        if (le != hipSuccess) return le;
    }
    return hipSuccess;
}

// Tile workgroups that fit one CU: LDS (block-table window + pipeline
// stages) and waves (3 per SIMD with one head per wave, 2 with two).
// kv_dtype: PSK_KV_*; grouped: a grouped launch (tiles_per_group ==
// kTileGroup) rather than one tile per workgroup.
uint32_t tile_workgroups_per_cu(uint32_t kv_dtype, uint32_t head_dim, uint32_t q_per_kv, bool grouped) {
    const size_t D = head_dim <= 64 ? 64 : head_dim <= 128 ? 128 : 256;
    const bool psq = kv_dtype == PSK_KV_PSQ4_W32 || kv_dtype == PSK_KV_PSQ8_W32;
    size_t lds;
    if (psq) {
        // code stages + one f16 chunk
        lds = kv_dtype == PSK_KV_PSQ4_W32
                  ? (D == 256 ? tile_pg_lds_bytes<kFmtPsq4, 256>() : tile_pg_lds_bytes<kFmtPsq4, 128>())
                  : (D == 256 ? tile_pg_lds_bytes<kFmtPsq8, 256>() : tile_pg_lds_bytes<kFmtPsq8, 128>());
    } else {
        const size_t cb = kv_dtype == PSK_KV_BF16 ? 2 * D : D;
        const size_t stage = 2 * 2 * (16 * cb + 128) + (kv_dtype != PSK_KV_BF16 ? 2 * 2 * 256 : 0);
        lds = (size_t)kTilePageWindow * 4 + (size_t)kTileStages * stage;
    }
    const uint32_t by_lds = (uint32_t)((160u * 1024u) / (lds + 64u));
    // waves: grouped launches kTileGroup two-head waves; otherwise up to 4
    // heads one per wave (4 waves), 5-6 one per wave (6; PSQ 8), 7-8 one per
    // wave (8)
    grouped = grouped && grouped_heads(q_per_kv);
    const uint32_t hpw = grouped ? 2u : 1u;
    const uint32_t nw = grouped ? (uint32_t)kTileGroup : q_per_kv <= 4u ? 4u : q_per_kv <= 6u && !psq ? 6u : 8u;
    const uint32_t by_waves = 4u * (uint32_t)tile_waves_per_simd((int)hpw) / nw;
    const uint32_t n = by_lds < by_waves ? by_lds : by_waves;
    return n == 0u ? 1u : n;
}

// Tiles per workgroup the step planner should group a prefill launch into:
// kTileGroup for every GQA group the tile kernels take (1-8 heads), every KV
// format.
// Largest tiles x splits whose split launch runs as dense units (the planner
// models those launches).
uint32_t tile_dense_units_limit() { return kDenseTileUnits; }

uint32_t tile_group_size(uint32_t q_per_kv, uint32_t /*kv_dtype*/) {
    return grouped_heads(q_per_kv) ? (uint32_t)kTileGroup : 1u;
}

// Workgroups of a tile launch of n_tiles (a multiple of tiles_per_group when grouped).
uint64_t tile_launch_workgroups(uint64_t n_tiles, uint32_t tiles_per_group, uint32_t q_per_kv,
                                uint32_t kv_heads) {
    if (tiles_per_group > 1u)
        return (n_tiles + tiles_per_group - 1u) / tiles_per_group * ((q_per_kv + 1u) / 2u) * kv_heads;
    return n_tiles * kv_heads;
}

bool paged_tiles_supported(const psk_paged_attention_args& a, uint32_t kv_dtype, const void* k,
                           const void* v, const void* ks, const void* vs) {
    return known_kv(kv_dtype) && tile_shape_ok(a, kv_dtype, k, v) && psq_scales_ok(kv_dtype, ks, vs);
}

// PSQ prefill tiles (the reference's launch_attention_paged_prefill_psq{4,8}):
// implicit tiles of 16 rows; false when the shape is outside the tile kernel
// (the caller then runs the rows on the decode kernel).
bool launch_prefill_psq_tiles(const psk_paged_attention_args& a, uint32_t kv_dtype, const void* kc,
                              const void* vc, const void* ks, const void* vs, hipStream_t stream,
                              hipError_t& err) {
    if (!paged_tiles_supported(a, kv_dtype, kc, vc, ks, vs)) return false;
    err = launch_tile_fmt(make_tile(a, kc, vc, static_cast<const float*>(ks), static_cast<const float*>(vs),
                                    nullptr, 1u, 0u),
                          kv_dtype, stream);
    return true;
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
    if (!psk::tile_shape_ok(*a, PSK_KV_BF16, k_pool, v_pool))
        return psk_attention_paged_bf16(a, k_pool, v_pool, stream);
    return psk::launch_tile<psk::kFmtBf16>(
        psk::make_tile(*a, k_pool, v_pool, nullptr, nullptr, nullptr, 1u, 0u), static_cast<hipStream_t>(stream));
}

extern "C" int psk_attention_paged_prefill_fp8_e4m3(const psk_paged_attention_args* a,
                                                    const void* k_pool, const void* v_pool,
                                                    const float* k_scale_pool,
                                                    const float* v_scale_pool, void* stream) {
    const hipError_t e = psk::tile_validate(a, k_pool, v_pool);
    if (e != hipSuccess) return e;
    if (k_scale_pool == nullptr || v_scale_pool == nullptr) return hipErrorInvalidValue;
    if (!psk::tile_shape_ok(*a, PSK_KV_FP8_E4M3, k_pool, v_pool))
        return psk_attention_paged_fp8_e4m3(a, k_pool, v_pool, k_scale_pool, v_scale_pool, stream);
    return psk::launch_tile<psk::kFmtFp8>(
        psk::make_tile(*a, k_pool, v_pool, k_scale_pool, v_scale_pool, nullptr, 1u, 0u),
        static_cast<hipStream_t>(stream));
}

extern "C" int psk_attention_paged_tile_split(const psk_paged_attention_args* a, uint32_t kv_dtype,
                                              const void* k_pool, const void* v_pool,
                                              const void* k_scale_pool, const void* v_scale_pool,
                                              float* partials, uint32_t splits,
                                              uint32_t pages_per_split, void* stream) {
    const hipError_t e = psk::tile_validate(a, k_pool, v_pool);
    if (e != hipSuccess) return e;
    if (partials == nullptr || splits == 0u || splits > psk::kMaxTileSplits || pages_per_split == 0u)
        return hipErrorInvalidValue;
    if (!psk::known_kv(kv_dtype)) return hipErrorInvalidValue;
    if (kv_dtype != PSK_KV_BF16 && (k_scale_pool == nullptr || v_scale_pool == nullptr))
        return hipErrorInvalidValue;
    if (!psk::tile_shape_ok(*a, kv_dtype, k_pool, v_pool) || !psk::psq_scales_ok(kv_dtype, k_scale_pool, v_scale_pool))
        return hipErrorNotSupported;
    const psk::TileParams p =
        psk::make_tile(*a, k_pool, v_pool, static_cast<const float*>(k_scale_pool),
                       static_cast<const float*>(v_scale_pool), partials, splits, pages_per_split);
    return psk::launch_tile_fmt(p, kv_dtype, static_cast<hipStream_t>(stream));
}
