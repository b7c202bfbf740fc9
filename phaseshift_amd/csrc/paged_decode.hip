// Paged-attention decode over GQA KV pages, BF16 or FP8 E4M3 KV, gfx950.
//
// Reference behaviour restated (file:line in the reference repository):
//   visibility (pos + 1), row skip rules, invalid page  paged_decode.hip:79-97,123-128
//   BF16 math  s = scale*q.k, online softmax, out = acc/sum   paged_decode.hip:135-205
//   FP8 math   s = (q.dec(k))*k_scale*scale,
//              acc += (p*v_scale)*dec(v)                     paged_decode.hip:1064-1090
//   split rule per = ceil(pages/splits), partial (m, P, A)   paged_decode.hip:315-320,413-471
//   combine g = max m_s, W_s = e^(m_s-g),
//           out = sum W_s A_s / sum W_s P_s                  paged_decode.hip:474-555
//   launcher validation                                      paged_decode.hip:228-259,787-817
//
// MI355X design. One workgroup = (row, kv_head, split), 4 waves. The whole GQA
// group (q_per_kv <= 16 query heads) is the N=16 side of
// v_mfma_f32_16x16x32_bf16, so each K/V byte is read from HBM once per
// (row, kv_head) instead of once per query head:
//   S^T[16 tokens x 16 heads] = K[16 x D] * Q^T[D x 16]   (D/32 MFMAs)
//   O^T[16 dims x 16 heads]  += V^T[16 x 32 tokens] * P^T[32 tokens x 16 heads]
// Each wave owns 32-token chunks (round robin), keeps its own online-softmax
// state in log2 units, and the 4 waves merge through LDS at the end. K is read
// straight into MFMA A-operand registers (lane = token, 16 B per load, every
// 64 B token segment read whole by 4 lanes); V is transposed through a
// per-wave LDS tile so that a lane holds 8 tokens of one dim. FP8 codes become
// bf16 exactly (v_cvt_scalef32_pk_bf16_fp8); k_scale multiplies the score and
// v_scale is folded into P before PV.
#include "device_common.h"

#include <phaseshift_kv/paged_attention.h>

#include <cfloat>

namespace psk {
namespace {

struct DecodeParams {
    psk_paged_attention_args a;
    const uint8_t* k_pool;
    const uint8_t* v_pool;
    const float* k_scale;
    const float* v_scale;
    float* partials;          // nullptr: write the output directly
    uint32_t splits;
    uint32_t pages_per_split; // 0: ceil(pages / splits) per row
    float scale_log2;         // scale * log2(e)
};

constexpr int kThreads = 256;
constexpr int kWaves = 4;
constexpr int kMaxQPerKV = 16;
constexpr uint32_t kMaxSplits = 1024;
using ps::kernel::kPagedAttentionHeadLimit;

__device__ __forceinline__ uint32_t split_pages(uint32_t pc, uint32_t splits, uint32_t pps) {
    return pps != 0u ? pps : (pc + splits - 1u) / splits;
}

// Loads 8 bf16 of a query head as an MFMA operand (zeros past the group).
__device__ __forceinline__ bf16x8 load_q8(const uint16_t* q, bool ok) {
    u32x4 r = {0u, 0u, 0u, 0u};
    if (ok) {
#pragma unroll
        for (int i = 0; i < 4; ++i) r[i] = (uint32_t)q[2 * i] | ((uint32_t)q[2 * i + 1] << 16);
    }
    return __builtin_bit_cast(bf16x8, r);
}

template <int KVB>
constexpr int chunk_halves() { return KVB == 1 ? 2 : 1; }   // 16-token halves per chunk

typedef __attribute__((ext_vector_type(2))) int i32x2;
typedef __attribute__((ext_vector_type(4))) short i16x4;
typedef __attribute__((address_space(3))) i32x2 lds_i32x2;
typedef __attribute__((address_space(3))) i16x4 lds_i16x4;

// gfx950 transposing LDS reads. Within each 16-lane block, the 16 lanes name
// 16 rows of 8 bytes: ds_read_b64_tr_b8 gives lane i byte i%8 of rows
// 2j + i/8 (j = 0..7); ds_read_b64_tr_b16 gives lane i element i%4 of rows
// 4j + i/4 (j = 0..3).
__device__ __forceinline__ i32x2 lds_read_tr8(const uint8_t* p) {
    return __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_i32x2*)(p));
}
__device__ __forceinline__ i16x4 lds_read_tr16(const uint8_t* p) {
    return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(p));
}

// Units of work of one row: splits that hold pages, 0 for a row the kernel
// skips (invalid slot, position past the block table).
__device__ __forceinline__ uint32_t row_units(const psk_paged_attention_args& a, uint32_t splits,
                                              uint32_t pps, uint32_t r) {
    if (a.row_sequence_slots[r] >= a.max_sequences) return 0u;
    const uint64_t vis = (uint64_t)a.row_positions[r] + 1u;
    if (vis > (uint64_t)a.block_table_stride * a.page_tokens || vis > 0xFFFFFFFFull) return 0u;
    const uint32_t pc = ((uint32_t)vis + a.page_tokens - 1u) / a.page_tokens;
    const uint32_t per = split_pages(pc, splits, pps);
    return min(splits, (pc + per - 1u) / per);
}

// Exclusive scan of two counters over the NW waves of the workgroup.
template <int NW>
__device__ __forceinline__ void block_scan2(uint32_t& x, uint32_t& y, uint32_t& tx, uint32_t& ty,
                                            uint32_t* tmp /* 2*NW */) {
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
    uint32_t ix = x, iy = y;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const uint32_t ux = __shfl_up(ix, o, 64), uy = __shfl_up(iy, o, 64);
        if (lane >= (uint32_t)o) { ix += ux; iy += uy; }
    }
    if (lane == 63u) { tmp[wave] = ix; tmp[NW + wave] = iy; }
    __syncthreads();
    uint32_t bx = 0, by = 0;
    tx = 0; ty = 0;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
        if ((uint32_t)w < wave) { bx += tmp[w]; by += tmp[NW + w]; }
        tx += tmp[w];
        ty += tmp[NW + w];
    }
    x = bx + ix - x;
    y = by + iy - y;
}

// Maps a dense unit index to (row, split). Units are ordered so that the
// workgroups of one launch spread evenly over the XCDs (block b runs on XCD
// b mod 8) and the longest go first: every row's splits but the last
// (row-major), then the last split of every row. Returns false past the last
// unit. All NW*64 threads of the workgroup must call it.
template <int NW>
__device__ bool find_unit(const psk_paged_attention_args& a, uint32_t splits, uint32_t pps,
                          uint32_t unit, uint32_t& row, uint32_t& split) {
    __shared__ uint32_t tmp[2 * NW];
    __shared__ uint32_t found[2];
    const uint32_t tid = threadIdx.x;
    const uint32_t R = a.rows;
    const uint32_t each = (R + NW * 64u - 1u) / (NW * 64u);
    const uint32_t r0 = min(R, tid * each), r1 = min(R, r0 + each);
    uint32_t nf = 0, nl = 0;   // this thread's non-last and last units
    for (uint32_t r = r0; r < r1; ++r) {
        const uint32_t u = row_units(a, splits, pps, r);
        if (u != 0u) { nf += u - 1u; nl += 1u; }
    }
    if (tid == 0) found[0] = 0xFFFFFFFFu;
    uint32_t pf = nf, pl = nl, F, L;
    block_scan2<NW>(pf, pl, F, L, tmp);
    if (unit < F) {
        if (unit >= pf && unit < pf + nf) {
            uint32_t k = unit - pf;
            for (uint32_t r = r0; r < r1; ++r) {
                const uint32_t u = row_units(a, splits, pps, r);
                if (u > 1u) {
                    if (k < u - 1u) { found[0] = r; found[1] = k; break; }
                    k -= u - 1u;
                }
            }
        }
    } else if (unit - F < L) {
        const uint32_t k0 = unit - F;
        if (k0 >= pl && k0 < pl + nl) {
            uint32_t k = k0 - pl;
            for (uint32_t r = r0; r < r1; ++r) {
                const uint32_t u = row_units(a, splits, pps, r);
                if (u != 0u) {
                    if (k == 0u) { found[0] = r; found[1] = u - 1u; break; }
                    --k;
                }
            }
        }
    }
    __syncthreads();
    row = found[0];
    split = found[1];
    return row != 0xFFFFFFFFu;
}

constexpr uint32_t kPageWindow = 1024;   // block-table entries staged in LDS per pass

// LDS bytes of one pipeline stage of one wave: K and V of a chunk (lane-major
// DMA layout) and, FP8, the k/v scales of its tokens.
template <int KVB, int D>
constexpr int stage_bytes() {
    return 2 * chunk_halves<KVB>() * (16 * D * KVB + 128) + (KVB == 1 ? 2 * chunk_halves<KVB>() * 256 : 0);
}

// kIndep: the 4 waves of a workgroup are 4 independent items, the kv heads
// 4*kv_group + w of one (row, split); they stream the same tokens (adjacent
// head slices of each token row) and need no merge. Otherwise the 4 waves
// share one (row, kv_head, split) item, take its chunks round robin and merge
// through LDS at the end (used when the independent grid cannot fill the GPU).
template <int KVB, int D, bool kIndep, int NW>
__global__ __launch_bounds__(NW * 64) void paged_decode_kernel(const DecodeParams p) {
    constexpr uint32_t NT = NW * 64;   // threads of the workgroup
    static_assert(kIndep || NW == kWaves, "the shared-item merge uses 4 waves");
    constexpr int H = chunk_halves<KVB>();
    constexpr int CT = 16 * H;         // tokens per chunk
    constexpr int NL = D * KVB / 64;   // 16 B loads per lane per 16-token half
    constexpr int NS = D / 32;         // MFMA K-steps of the score product
    constexpr int NDB = D / 16;        // 16-dim blocks of the output
    // a 16-token half of K (V) in LDS, padded by 128 B so that the two halves
    // of a chunk fall on opposite halves of the 64 LDS banks (the transposing
    // V reads of one instruction touch both)
    constexpr int HALF_STRIDE = 16 * D * KVB + 128;
    constexpr int KV_BYTES = H * HALF_STRIDE;               // K (or V) of one chunk
    constexpr int SC_BYTES = KVB == 1 ? H * 256 : 0;       // k (or v) scales of one chunk
    constexpr int STAGE = stage_bytes<KVB, D>();
    constexpr int kWinBytes = (int)kPageWindow * 4;
    // vector-memory operations of one issue(): K and V DMAs and the scale DMAs
    constexpr int kStepOps = H * (2 * NL + (KVB == 1 ? 2 : 0));
    constexpr uint32_t kStride = kIndep ? CT : NW * CT;   // a wave's chunk stride
    static_assert(NL >= 1 && NS >= 1, "head_dim too small for this kernel");

    extern __shared__ __align__(16) uint8_t lds[];
    __shared__ uint32_t bad_shared;

    const psk_paged_attention_args& a = p.a;
    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid & 63u;
    const uint32_t wave = tid >> 6;
    const uint32_t n = lane & 15u;   // token (loads, S rows) or head (S cols, P, O)
    const uint32_t g = lane >> 4;    // lane group

    const uint32_t splits = p.splits;
    // blockIdx = unit * G + sub: G independent kv-head groups or G kv heads
    const uint32_t G = kIndep ? (a.kv_heads + NW - 1u) / NW : a.kv_heads;
    const uint32_t sub = blockIdx.x % G;
    uint32_t row, split;
    if (!find_unit<NW>(a, splits, p.pages_per_split, blockIdx.x / G, row, split)) return;
    const uint32_t kv_head = kIndep ? sub * NW + wave : sub;
    const uint32_t slot = a.row_sequence_slots[row];
    const uint32_t visible = a.row_positions[row] + 1u;
    const uint32_t P = a.page_tokens;
    const uint32_t pc = (visible + P - 1u) / P;
    const uint32_t per = split_pages(pc, splits, p.pages_per_split);
    const uint32_t pb = split * per;
    const uint32_t pe = (split == splits - 1u) ? pc : min(pc, pb + per);
    const uint32_t t_end = min(pe * P, visible);
    const uint32_t* bt = a.block_tables + (uint64_t)slot * a.block_table_stride;
    // Everything above is uniform over the workgroup (row, split), so every
    // wave reaches the barriers below; an independent wave past the last kv
    // head only helps stage the block table.
    const bool active = kv_head < a.kv_heads;
    const uint32_t kvh = active ? kv_head : 0u;

    const uint32_t qpk = a.q_heads / a.kv_heads;
    if (!kIndep && tid == 0) bad_shared = 0u;

    // Q fragments: lane (n, g) holds head n, the dims that lane group g covers
    // in each K-step (the dims the K DMA below puts in that lane's 16 bytes).
    bf16x8 qf[NS];
    {
        const bool hv = n < qpk;
        const uint16_t* qrow = static_cast<const uint16_t*>(a.q) + (uint64_t)row * a.q_row_stride +
                               (uint64_t)(kvh * qpk + (hv ? n : 0u)) * D;
#pragma unroll
        for (int s = 0; s < NS; ++s) {
            const int d0 = KVB == 2 ? s * 32 + (int)g * 8 : (s >> 1) * 64 + (int)g * 16 + (s & 1) * 8;
            qf[s] = load_q8(qrow + d0, hv);
        }
    }

    const uint64_t layer_base = (uint64_t)a.layer * a.elems_per_layer;
    const uint64_t scale_layer = (uint64_t)a.layer * a.num_pages;
    uint32_t* const win = reinterpret_cast<uint32_t*>(lds);
    uint8_t* const stage0 = lds + kWinBytes + (size_t)wave * 2 * STAGE;
    uint8_t* const stage1 = stage0 + STAGE;
    bool bad = false;

    // tr-read address of this lane inside the V part of a stage; output block
    // db adds 256*KVB*db. Lane r of a 16-lane block names row r of the
    // transpose:
    //   FP8:  token (r>>1 < 4 ? 4g + (r>>1) : 16 + 4g + (r>>1) - 4), dims +8*(r&1)
    //   BF16: token 4g + (r>>2), dims +4*(r&3)
    // In the DMA layout byte b of token t (half t/16) sits at
    // (t/16)*HALF_STRIDE + 1024*(b/64) + 16*(16*((b%64)/16) + t%16) + b%16.
    uint32_t tr_off;
    if constexpr (KVB == 1) {
        const uint32_t j = n >> 1;
        tr_off = (j < 4u ? 0u : (uint32_t)HALF_STRIDE) + 16u * (4u * g + (j & 3u)) + 8u * (n & 1u);
    } else {
        tr_off = 16u * (4u * g + (n >> 2)) + 256u * ((n >> 1) & 1u) + 8u * (n & 1u);
    }

    float m_run = -INFINITY;   // running max (log2 units), head n
    float l_run = 0.0f;        // partial softmax sum of this lane's tokens
    f32x4 o[NDB];
#pragma unroll
    for (int db = 0; db < NDB; ++db) o[db] = (f32x4){0.f, 0.f, 0.f, 0.f};

    // One pass per window of kPageWindow pages (a single pass unless the
    // split holds more pages than that).
    for (uint32_t wp = pb; wp < pe; wp += kPageWindow) {
        const uint32_t wp_end = min(pe, wp + kPageWindow);
        __syncthreads();
        for (uint32_t i = tid; i < wp_end - wp; i += NT) win[i] = bt[wp + i];
        __syncthreads();
        const uint32_t ts = wp * P;
        const uint32_t te = min(wp_end * P, t_end);
        const uint32_t t_last = te - 1u;
        uint32_t cb = ts + (kIndep ? 0u : wave * CT);
        if (!active || cb >= te) continue;

        // Issues the DMAs of the chunk at c into stage `st`: load i of half
        // hf of K (V) at +hf*HALF_STRIDE + 1024*i, lane (n, g) at +16*(16g + n)
        // holding bytes [64i + 16g, +16) of token n; the scales of token n at
        // +4*(16g + n) of each 256 B scale block. Loads are branch-free:
        // tokens past the range read the last token (their scores are
        // masked), so every issue() has exactly kStepOps operations.
        auto issue = [&](uint32_t c, uint8_t* st) __attribute__((always_inline)) {
#pragma unroll
            for (int hf = 0; hf < H; ++hf) {
                const uint32_t tau = min(c + (uint32_t)hf * 16u + n, t_last);
                uint32_t page = win[tau / P - wp];
                const bool inv = page >= a.num_pages;
                bad |= inv;
                page = inv ? 0u : page;
                const uint32_t off = tau % P;
                const uint64_t elem = layer_base + (uint64_t)page * a.elems_per_page +
                                      (uint64_t)off * a.elems_per_token + (uint64_t)kvh * D;
                const uint8_t* ks = p.k_pool + elem * KVB + g * 16;
                const uint8_t* vs = p.v_pool + elem * KVB + g * 16;
#pragma unroll
                for (int i = 0; i < NL; ++i) load_lds<16>(ks + i * 64, st + hf * HALF_STRIDE + i * 1024);
#pragma unroll
                for (int i = 0; i < NL; ++i)
                    load_lds<16>(vs + i * 64, st + KV_BYTES + hf * HALF_STRIDE + i * 1024);
                if constexpr (KVB == 1) {
                    const uint64_t si = ((scale_layer + page) * P + off) * a.kv_heads + kvh;
                    load_lds<4>(p.k_scale + si, st + 2 * KV_BYTES + hf * 256);
                    load_lds<4>(p.v_scale + si, st + 2 * KV_BYTES + SC_BYTES + hf * 256);
                }
            }
        };

        // Scores, online softmax and PV of the chunk at c held in stage st.
        auto consume = [&](uint32_t c, const uint8_t* st) __attribute__((always_inline)) {
            f32x4 sc[H];
#pragma unroll
            for (int hf = 0; hf < H; ++hf) {
                f32x4 acc = {0.f, 0.f, 0.f, 0.f};
                const uint8_t* kb = st + hf * HALF_STRIDE + 16 * lane;
#pragma unroll
                for (int s = 0; s < NS; ++s) {
                    bf16x8 kf;
                    if constexpr (KVB == 2) {
                        kf = *reinterpret_cast<const bf16x8*>(kb + 1024 * s);
                    } else {
                        const u32x4 w = *reinterpret_cast<const u32x4*>(kb + 1024 * (s >> 1));
                        kf = (s & 1) ? fp8x8_to_bf16x8(w[2], w[3]) : fp8x8_to_bf16x8(w[0], w[1]);
                    }
                    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf, qf[s], acc, 0, 0, 0);
                }
                sc[hf] = acc;
            }

            // online softmax (log2 units) for head n over tokens 4g + r
            float s2[H][4], vsc[H][4];
            float mx = -INFINITY;
#pragma unroll
            for (int hf = 0; hf < H; ++hf) {
                f32x4 kscale = {1.f, 1.f, 1.f, 1.f}, vscale = {1.f, 1.f, 1.f, 1.f};
                if constexpr (KVB == 1) {
                    kscale = *reinterpret_cast<const f32x4*>(st + 2 * KV_BYTES + hf * 256 + 16 * g);
                    vscale = *reinterpret_cast<const f32x4*>(st + 2 * KV_BYTES + SC_BYTES + hf * 256 +
                                                             16 * g);
                }
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const bool ok = c + hf * 16 + 4u * g + (uint32_t)r < te;
                    s2[hf][r] = ok ? sc[hf][r] * (p.scale_log2 * kscale[r]) : -INFINITY;
                    vsc[hf][r] = vscale[r];
                    mx = __builtin_fmaxf(mx, s2[hf][r]);
                }
            }
            mx = __builtin_fmaxf(mx, __shfl_xor(mx, 16, 64));
            mx = __builtin_fmaxf(mx, __shfl_xor(mx, 32, 64));
            const float m_new = __builtin_fmaxf(m_run, mx);
            const float m_use = m_new == -INFINITY ? 0.0f : m_new;
            const float alpha = __builtin_amdgcn_exp2f(m_run - m_use);
            float pv[H][4];
            float psum = 0.0f;
#pragma unroll
            for (int hf = 0; hf < H; ++hf)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float e = __builtin_amdgcn_exp2f(s2[hf][r] - m_use);
                    psum += e;
                    pv[hf][r] = e * vsc[hf][r];
                }
            l_run = l_run * alpha + psum;
            m_run = m_new;
            // O is rescaled only when some head's running max moved.
            if (__any(alpha != 1.0f)) {
#pragma unroll
                for (int db = 0; db < NDB; ++db) o[db] *= alpha;
            }

            // O^T += V^T * P^T. P (v_scale folded in) as hi + lo bf16 pairs:
            // two MFMAs keep ~16 mantissa bits of every weight (V and K are
            // exact in bf16).
            const uint8_t* vb = st + KV_BYTES + tr_off;
            if constexpr (KVB == 1) {
                u32x4 ph, pl;
                { const u32x2 t_ = split_bf16x2(pv[0][0], pv[0][1]); ph[0] = t_[0]; pl[0] = t_[1]; }
                { const u32x2 t_ = split_bf16x2(pv[0][2], pv[0][3]); ph[1] = t_[0]; pl[1] = t_[1]; }
                { const u32x2 t_ = split_bf16x2(pv[1][0], pv[1][1]); ph[2] = t_[0]; pl[2] = t_[1]; }
                { const u32x2 t_ = split_bf16x2(pv[1][2], pv[1][3]); ph[3] = t_[0]; pl[3] = t_[1]; }
                const bf16x8 pfh = __builtin_bit_cast(bf16x8, ph);
                const bf16x8 pfl = __builtin_bit_cast(bf16x8, pl);
#pragma unroll
                for (int db = 0; db < NDB; ++db) {
                    const i32x2 w = lds_read_tr8(vb + 256 * db);
                    const bf16x8 vf = fp8x8_to_bf16x8((uint32_t)w[0], (uint32_t)w[1]);
                    o[db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf, pfh, o[db], 0, 0, 0);
                    o[db] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf, pfl, o[db], 0, 0, 0);
                }
            } else {
                u32x2 ph, pl;
                { const u32x2 t_ = split_bf16x2(pv[0][0], pv[0][1]); ph[0] = t_[0]; pl[0] = t_[1]; }
                { const u32x2 t_ = split_bf16x2(pv[0][2], pv[0][3]); ph[1] = t_[0]; pl[1] = t_[1]; }
                const i16x4 pfh = __builtin_bit_cast(i16x4, ph);
                const i16x4 pfl = __builtin_bit_cast(i16x4, pl);
#pragma unroll
                for (int db = 0; db < NDB; ++db) {
                    const i16x4 vf = lds_read_tr16(vb + 512 * db);
                    o[db] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(vf, pfh, o[db], 0, 0, 0);
                    o[db] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(vf, pfl, o[db], 0, 0, 0);
                }
            }
        };

        // One pipeline step: the DMAs of the next chunk go out before the
        // wait for chunk c, so the wave keeps two chunks in flight while it
        // computes. The __restrict__ parameters tell the compiler that the
        // DMA into `next` and the reads of `cur` touch different LDS; the
        // ordering between a DMA and the later reads of its stage is the
        // explicit wait_vmcnt, which leaves exactly the kStepOps operations
        // of this step's issue() outstanding.
        auto step = [&](uint32_t c, uint8_t* __restrict__ next,
                        const uint8_t* __restrict__ cur) __attribute__((always_inline)) {
            issue(c + kStride, next);
            wait_vmcnt<kStepOps>();
            consume(c, cur);
        };

        issue(cb, stage0);
        for (;;) {
            step(cb, stage1, stage0);
            cb += kStride;
            if (cb >= te) break;
            step(cb, stage0, stage1);
            cb += kStride;
            if (cb >= te) break;
        }
        // The last step issued a chunk nobody reads: its DMAs must land
        // before the stages are reused.
        wait_vmcnt<0>();
    }

    const uint32_t q0 = kvh * qpk;
    if constexpr (kIndep) {
        if (!active) return;
        const float l_tot = l_run + __shfl_xor(l_run, 16, 64);
        const float l_all = l_tot + __shfl_xor(l_tot, 32, 64);
        if (n >= qpk) return;
        if (p.partials == nullptr) {
            // An invalid page leaves this row's output unwritten.
            if (bad) return;
            const float inv_l = 1.0f / l_all;
            const uint64_t ob = (uint64_t)row * a.output_row_stride + (uint64_t)(q0 + n) * D + 4u * g;
#pragma unroll
            for (int db = 0; db < NDB; ++db)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float res = o[db][r] * inv_l;
                    if (a.output_dtype == PSK_OUT_F32)
                        static_cast<float*>(a.output)[ob + 16 * db + r] = res;
                    else
                        static_cast<uint16_t*>(a.output)[ob + 16 * db + r] = f32_to_bf16_bits(res);
                }
        } else {
            float* part = p.partials + ((uint64_t)(row * a.kv_heads + kvh) * splits + split) *
                                           (uint64_t)(qpk * (2u + kPagedAttentionHeadLimit));
            if (g == 0) {
                // NaN marks a split that met an invalid page; the reduce then
                // leaves the row unwritten.
                part[n] = bad ? __builtin_nanf("") : m_run * 0.69314718055994531f;
                part[qpk + n] = l_all;
            }
            float* A = part + 2u * qpk + n * kPagedAttentionHeadLimit + 4u * g;
#pragma unroll
            for (int db = 0; db < NDB; ++db)
#pragma unroll
                for (int r = 0; r < 4; ++r) A[16 * db + r] = o[db][r];
        }
        return;
    } else {
        // ---- merge the 4 waves: per wave m[16], l[16], O[qpk][D] in LDS
        if (bad) bad_shared = 1u;
        const float l_tot = l_run + __shfl_xor(l_run, 16, 64);
        const float l_all = l_tot + __shfl_xor(l_tot, 32, 64);
        __syncthreads();
        float* fm = reinterpret_cast<float*>(lds);
        float* fl = fm + kWaves * 16;
        float* fo = fl + kWaves * 16;   // [wave][qpk][D]
        if (g == 0) {
            fm[wave * 16 + n] = m_run;
            fl[wave * 16 + n] = l_all;
        }
        if (n < qpk) {
#pragma unroll
            for (int db = 0; db < NDB; ++db)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    fo[((size_t)wave * qpk + n) * D + db * 16 + 4 * g + r] = o[db][r];
        }
        __syncthreads();

        float* part = nullptr;
        if (p.partials != nullptr)
            part = p.partials + ((uint64_t)(row * a.kv_heads + kvh) * splits + split) *
                                    (uint64_t)(qpk * (2u + kPagedAttentionHeadLimit));
        if (bad_shared != 0u) {
            // An invalid page leaves this row's output unwritten; the NaN marks
            // the split for the reduce, which then writes nothing either.
            if (part != nullptr && tid < qpk) part[tid] = __builtin_nanf("");
            return;
        }
        for (uint32_t idx = tid; idx < qpk * D; idx += kThreads) {
            const uint32_t h = idx / D, d = idx % D;
            float gm = -INFINITY;
#pragma unroll
            for (int w = 0; w < kWaves; ++w) gm = __builtin_fmaxf(gm, fm[w * 16 + h]);
            float L = 0.0f, O = 0.0f;
#pragma unroll
            for (int w = 0; w < kWaves; ++w) {
                const float wt = __builtin_amdgcn_exp2f(fm[w * 16 + h] - gm);
                L += wt * fl[w * 16 + h];
                O += wt * fo[((size_t)w * qpk + h) * D + d];
            }
            if (part == nullptr) {
                const uint64_t oi = (uint64_t)row * a.output_row_stride + (uint64_t)(q0 + h) * D + d;
                const float res = O / L;
                if (a.output_dtype == PSK_OUT_F32)
                    static_cast<float*>(a.output)[oi] = res;
                else
                    static_cast<uint16_t*>(a.output)[oi] = f32_to_bf16_bits(res);
            } else {
                if (d == 0) {
                    part[h] = gm * 0.69314718055994531f;   // back to natural-log units
                    part[qpk + h] = L;
                }
                part[2u * qpk + h * kPagedAttentionHeadLimit + d] = O;
            }
        }
    }
}

// Combine of the split partials: WG = (row, kv_head, query head of the
// group), thread = dim. Split weights W_s = e^(m_s - g) are computed once into
// LDS; every thread then sums W_s * A_s[d] with loads coalesced over d.
__global__ __launch_bounds__(kThreads) void split_reduce_kernel(const DecodeParams p) {
    __shared__ float w_lds[kMaxSplits];
    __shared__ float red[2 * kWaves];
    const psk_paged_attention_args& a = p.a;
    const uint32_t qpk = a.q_heads / a.kv_heads;
    const uint32_t h = blockIdx.x % qpk;
    const uint32_t kv_head = (blockIdx.x / qpk) % a.kv_heads;
    const uint32_t row = blockIdx.x / (qpk * a.kv_heads);
    if (row >= a.rows) return;
    const uint32_t slot = a.row_sequence_slots[row];
    if (slot >= a.max_sequences) return;
    const uint64_t vis64 = (uint64_t)a.row_positions[row] + 1u;
    if (vis64 > (uint64_t)a.block_table_stride * a.page_tokens) return;
    const uint32_t pc = ((uint32_t)vis64 + a.page_tokens - 1u) / a.page_tokens;
    const uint32_t per = split_pages(pc, p.splits, p.pages_per_split);
    const uint32_t n_used = min(p.splits, (pc + per - 1u) / per);
    const uint64_t stride = (uint64_t)qpk * (2u + kPagedAttentionHeadLimit);
    const float* base = p.partials + (uint64_t)(row * a.kv_heads + kv_head) * p.splits * stride;
    const uint32_t tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;

    // g = max m_s (NaN marks a split that met an invalid page)
    float gm = -INFINITY;
    bool bad = false;
    for (uint32_t s = tid; s < n_used; s += kThreads) {
        const float m = base[s * stride + h];
        bad |= __builtin_isnan(m);
        gm = __builtin_fmaxf(gm, m);
    }
    gm = wave_max(gm);
    const bool bad_w = __any(bad);
    if (lane == 0) {
        red[wave] = gm;
        red[kWaves + wave] = bad_w ? 1.0f : 0.0f;
    }
    __syncthreads();
    gm = __builtin_fmaxf(__builtin_fmaxf(red[0], red[1]), __builtin_fmaxf(red[2], red[3]));
    if (red[kWaves] + red[kWaves + 1] + red[kWaves + 2] + red[kWaves + 3] != 0.0f) return;
    __syncthreads();
    float lsum = 0.0f;
    for (uint32_t s = tid; s < n_used; s += kThreads) {
        const float w = __expf(base[s * stride + h] - gm);
        w_lds[s] = w;
        lsum += w * base[s * stride + qpk + h];
    }
    lsum = wave_sum(lsum);
    if (lane == 0) red[wave] = lsum;
    __syncthreads();
    const float L = red[0] + red[1] + red[2] + red[3];
    const uint32_t D = a.head_dim;
    const float* A = base + 2u * qpk + h * kPagedAttentionHeadLimit;
    for (uint32_t d = tid; d < D; d += kThreads) {
        float O = 0.0f;
        for (uint32_t s = 0; s < n_used; ++s) O += w_lds[s] * A[s * stride + d];
        const uint64_t oi =
            (uint64_t)row * a.output_row_stride + (uint64_t)(kv_head * qpk + h) * D + d;
        const float res = O / L;
        if (a.output_dtype == PSK_OUT_F32)
            static_cast<float*>(a.output)[oi] = res;
        else
            static_cast<uint16_t*>(a.output)[oi] = f32_to_bf16_bits(res);
    }
}

// ---------------------------------------------------------------- host side
hipError_t validate_common(const psk_paged_attention_args& c) {
    if (c.rows == 0u || c.head_dim == 0u || c.head_dim > kPagedAttentionHeadLimit)
        return hipErrorInvalidValue;
    if (c.q_heads == 0u || c.kv_heads == 0u || c.q_heads % c.kv_heads != 0u)
        return hipErrorInvalidValue;
    if (c.page_tokens == 0u || c.block_table_stride == 0u || c.num_pages == 0u)
        return hipErrorInvalidValue;
    if (c.q == nullptr || c.output == nullptr || c.row_sequence_slots == nullptr ||
        c.row_positions == nullptr || c.block_tables == nullptr)
        return hipErrorInvalidValue;
    if (c.output_dtype != PSK_OUT_BF16 && c.output_dtype != PSK_OUT_F32)
        return hipErrorInvalidValue;
    return hipSuccess;
}

// Shapes the MFMA kernel covers: q_per_kv <= 16, head_dim in {32 (bf16 only),
// 64, 128, 256}, every head slice 16 B aligned.
bool mfma_shape_ok(const psk_paged_attention_args& c, int kvb, const void* kp, const void* vp) {
    const uint32_t qpk = c.q_heads / c.kv_heads;
    if (qpk > (uint32_t)kMaxQPerKV) return false;
    const uint32_t D = c.head_dim;
    if (!(D == 64 || D == 128 || D == 256 || (D == 32 && kvb == 2))) return false;
    const uint32_t align_elems = 16u / (uint32_t)kvb;
    if (c.elems_per_token % align_elems || c.elems_per_page % align_elems ||
        c.elems_per_layer % align_elems)
        return false;
    if (reinterpret_cast<uintptr_t>(kp) % 16u || reinterpret_cast<uintptr_t>(vp) % 16u)
        return false;
    return true;
}

}  // namespace

// LDS bytes of one independent-wave decode workgroup (the split chooser
// derives workgroups per CU from it).
size_t decode_workgroup_lds_bytes(int kvb, uint32_t head_dim) {
    const size_t D = head_dim <= 64 ? 64 : head_dim <= 128 ? 128 : 256;
    const size_t H = kvb == 1 ? 2 : 1;
    const size_t stage = 2 * H * (16 * D * kvb + 128) + (kvb == 1 ? 2 * H * 256 : 0);
    return (size_t)kPageWindow * 4 + (size_t)kWaves * 2 * stage;
}

namespace {

template <int KVB, int D, bool kIndep, int NW>
hipError_t launch_decode_t2(const DecodeParams& p, uint64_t grid, hipStream_t stream) {
    const uint32_t qpk = p.a.q_heads / p.a.kv_heads;
    // block-table window + two pipeline stages per wave; the shared-item merge
    // later reuses the same LDS
    const size_t v_bytes = (size_t)kPageWindow * 4 + (size_t)NW * 2 * stage_bytes<KVB, D>();
    const size_t m_bytes = kIndep ? 0 : (size_t)NW * 32 * sizeof(float) +
                                            (size_t)NW * qpk * D * sizeof(float);
    const size_t lds_bytes = v_bytes > m_bytes ? v_bytes : m_bytes;
    if (grid == 0u || grid > 0x7FFFFFFFull) return hipErrorInvalidValue;
    if (lds_bytes > 64u * 1024u) {
        // gfx950 has 160 KB of LDS per CU; raise the per-kernel dynamic limit.
        static const hipError_t attr = hipFuncSetAttribute(
            reinterpret_cast<const void*>(&paged_decode_kernel<KVB, D, kIndep, NW>),
            hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024 - 1024);
        if (attr != hipSuccess) return attr;
    }
    hipLaunchKernelGGL((paged_decode_kernel<KVB, D, kIndep, NW>), dim3((uint32_t)grid),
                       dim3(NW * 64), lds_bytes, stream, p);
    return hipGetLastError();
}

// Independent waves (one kv head each) when that grid fills at least half of
// the GPU's 256 CUs; otherwise the 4 waves share each (row, kv_head, split)
// item. The split chooser assumes the same rule.
template <int KVB, int D>
hipError_t launch_decode_t(const DecodeParams& p, hipStream_t stream) {
    const uint64_t units = (uint64_t)p.a.rows * p.splits;
    const uint64_t groups = (p.a.kv_heads + kWaves - 1u) / kWaves;
    if (units * groups >= 128u) return launch_decode_t2<KVB, D, true, kWaves>(p, units * groups, stream);
    return launch_decode_t2<KVB, D, false, kWaves>(p, units * p.a.kv_heads, stream);
}

template <int KVB>
hipError_t launch_decode(const DecodeParams& p, hipStream_t stream) {
    switch (p.a.head_dim) {
        case 256: return launch_decode_t<KVB, 256>(p, stream);
        case 128: return launch_decode_t<KVB, 128>(p, stream);
        case 64: return launch_decode_t<KVB, 64>(p, stream);
        case 32:
            if constexpr (KVB == 2) return launch_decode_t<2, 32>(p, stream);
            return hipErrorNotSupported;
        default: return hipErrorNotSupported;
    }
}

hipError_t launch_reduce(const DecodeParams& p, hipStream_t stream) {
    const uint64_t grid = (uint64_t)p.a.rows * p.a.q_heads;
    if (grid == 0u || grid > 0x7FFFFFFFull) return hipErrorInvalidValue;
    hipLaunchKernelGGL(split_reduce_kernel, dim3((uint32_t)grid), dim3(kThreads), 0, stream, p);
    return hipGetLastError();
}

DecodeParams make(const psk_paged_attention_args& c, const void* k, const void* v, const float* ks,
                  const float* vs, float* partials, uint32_t splits, uint32_t pps) {
    DecodeParams p{};
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

// Generic fallback for shapes outside mfma_shape_ok (defined in page_ops.hip).
hipError_t launch_attention_generic(const psk_paged_attention_args& c, int kvb, const void* k,
                                    const void* v, const float* ks, const float* vs,
                                    hipStream_t stream);

}  // namespace psk

using psk::DecodeParams;

extern "C" uint64_t psk_attention_split_partials_bytes(uint32_t rows, uint32_t q_heads,
                                                       uint32_t kv_heads, uint32_t splits) {
    if (kv_heads == 0u) return 0u;
    return (uint64_t)rows * kv_heads * splits * (q_heads / kv_heads) *
           (2u + ps::kernel::kPagedAttentionHeadLimit) * sizeof(float);
}

extern "C" int psk_attention_paged_bf16(const psk_paged_attention_args* a, const void* k_pool,
                                        const void* v_pool, void* stream) {
    if (a == nullptr || k_pool == nullptr || v_pool == nullptr) return hipErrorInvalidValue;
    hipError_t e = psk::validate_common(*a);
    if (e != hipSuccess) return e;
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (!psk::mfma_shape_ok(*a, 2, k_pool, v_pool))
        return psk::launch_attention_generic(*a, 2, k_pool, v_pool, nullptr, nullptr, st);
    return psk::launch_decode<2>(psk::make(*a, k_pool, v_pool, nullptr, nullptr, nullptr, 1u, 0u), st);
}

extern "C" int psk_attention_paged_fp8_e4m3(const psk_paged_attention_args* a, const void* k_pool,
                                            const void* v_pool, const float* k_scale_pool,
                                            const float* v_scale_pool, void* stream) {
    if (a == nullptr || k_pool == nullptr || v_pool == nullptr || k_scale_pool == nullptr ||
        v_scale_pool == nullptr)
        return hipErrorInvalidValue;
    hipError_t e = psk::validate_common(*a);
    if (e != hipSuccess) return e;
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (!psk::mfma_shape_ok(*a, 1, k_pool, v_pool))
        return psk::launch_attention_generic(*a, 1, k_pool, v_pool, k_scale_pool, v_scale_pool, st);
    return psk::launch_decode<1>(
        psk::make(*a, k_pool, v_pool, k_scale_pool, v_scale_pool, nullptr, 1u, 0u), st);
}

static int split_common(const psk_paged_attention_args* a, const void* k_pool, const void* v_pool,
                        float* partials, uint32_t splits) {
    if (a == nullptr || k_pool == nullptr || v_pool == nullptr || partials == nullptr)
        return hipErrorInvalidValue;
    hipError_t e = psk::validate_common(*a);
    if (e != hipSuccess) return e;
    if (splits == 0u || splits > psk::kMaxSplits) return hipErrorInvalidValue;
    return hipSuccess;
}

extern "C" int psk_attention_paged_bf16_split_ex(const psk_paged_attention_args* a,
                                                 const void* k_pool, const void* v_pool,
                                                 float* partials, uint32_t splits,
                                                 uint32_t pages_per_split, void* stream) {
    int e = split_common(a, k_pool, v_pool, partials, splits);
    if (e != hipSuccess) return e;
    if (!psk::mfma_shape_ok(*a, 2, k_pool, v_pool)) return hipErrorNotSupported;
    return psk::launch_decode<2>(
        psk::make(*a, k_pool, v_pool, nullptr, nullptr, partials, splits, pages_per_split),
        static_cast<hipStream_t>(stream));
}

extern "C" int psk_attention_paged_bf16_split(const psk_paged_attention_args* a, const void* k_pool,
                                              const void* v_pool, float* partials, uint32_t splits,
                                              void* stream) {
    // The reference accepts 2, 4, 8 or 16 splits (paged_decode.hip:805-806).
    if (splits != 2u && splits != 4u && splits != 8u && splits != 16u) return hipErrorInvalidValue;
    return psk_attention_paged_bf16_split_ex(a, k_pool, v_pool, partials, splits, 0u, stream);
}

extern "C" int psk_attention_paged_fp8_e4m3_split(const psk_paged_attention_args* a,
                                                  const void* k_pool, const void* v_pool,
                                                  const float* k_scale_pool,
                                                  const float* v_scale_pool, float* partials,
                                                  uint32_t splits, uint32_t pages_per_split,
                                                  void* stream) {
    int e = split_common(a, k_pool, v_pool, partials, splits);
    if (e != hipSuccess) return e;
    if (k_scale_pool == nullptr || v_scale_pool == nullptr) return hipErrorInvalidValue;
    if (!psk::mfma_shape_ok(*a, 1, k_pool, v_pool)) return hipErrorNotSupported;
    return psk::launch_decode<1>(psk::make(*a, k_pool, v_pool, k_scale_pool, v_scale_pool, partials,
                                           splits, pages_per_split),
                                 static_cast<hipStream_t>(stream));
}

extern "C" int psk_attention_paged_split_reduce_ex(const psk_paged_attention_args* a,
                                                   const float* partials, uint32_t splits,
                                                   uint32_t pages_per_split, void* stream) {
    if (a == nullptr || partials == nullptr) return hipErrorInvalidValue;
    if (a->rows == 0u || a->head_dim == 0u || a->head_dim > ps::kernel::kPagedAttentionHeadLimit)
        return hipErrorInvalidValue;
    if (a->q_heads == 0u || a->kv_heads == 0u || a->q_heads % a->kv_heads != 0u)
        return hipErrorInvalidValue;
    if (a->output == nullptr || a->row_sequence_slots == nullptr || a->row_positions == nullptr)
        return hipErrorInvalidValue;
    if (a->page_tokens == 0u || splits == 0u || splits > psk::kMaxSplits) return hipErrorInvalidValue;
    return psk::launch_reduce(
        psk::make(*a, nullptr, nullptr, nullptr, nullptr, const_cast<float*>(partials), splits,
                  pages_per_split),
        static_cast<hipStream_t>(stream));
}

extern "C" int psk_attention_paged_bf16_split_reduce(const psk_paged_attention_args* a,
                                                     const float* partials, uint32_t splits,
                                                     void* stream) {
    if (splits != 2u && splits != 4u && splits != 8u && splits != 16u) return hipErrorInvalidValue;
    return psk_attention_paged_split_reduce_ex(a, partials, splits, 0u, stream);
}

// ------------------------------------------------- reference C++ signatures
namespace ps::kernel {

static const psk_paged_attention_args* C(const PagedAttentionCommonArgs& c) {
    return reinterpret_cast<const psk_paged_attention_args*>(&c);
}

hipError_t launch_attention_paged_bf16(const PagedAttentionCommonArgs& common, const bf16_t* k_pool,
                                       const bf16_t* v_pool, hipStream_t stream) {
    return static_cast<hipError_t>(psk_attention_paged_bf16(C(common), k_pool, v_pool, stream));
}

hipError_t launch_attention_paged_fp8_e4m3(const PagedAttentionCommonArgs& common,
                                           const ::ps::qwen35::fp8e4m3_storage_t* k_pool,
                                           const ::ps::qwen35::fp8e4m3_storage_t* v_pool,
                                           const float* k_scale_pool, const float* v_scale_pool,
                                           hipStream_t stream) {
    return static_cast<hipError_t>(psk_attention_paged_fp8_e4m3(C(common), k_pool, v_pool,
                                                                k_scale_pool, v_scale_pool, stream));
}

hipError_t launch_attention_paged_bf16_split(const PagedAttentionCommonArgs& common,
                                             const bf16_t* k_pool, const bf16_t* v_pool,
                                             float* partials, uint32_t splits, hipStream_t stream) {
    return static_cast<hipError_t>(
        psk_attention_paged_bf16_split(C(common), k_pool, v_pool, partials, splits, stream));
}

hipError_t launch_attention_paged_bf16_split_reduce(const PagedAttentionCommonArgs& common,
                                                    const float* partials, uint32_t splits,
                                                    hipStream_t stream) {
    return static_cast<hipError_t>(
        psk_attention_paged_bf16_split_reduce(C(common), partials, splits, stream));
}

hipError_t launch_attention_paged_fp8_e4m3_split(
    const PagedAttentionCommonArgs& common, const ::ps::qwen35::fp8e4m3_storage_t* k_pool,
    const ::ps::qwen35::fp8e4m3_storage_t* v_pool, const float* k_scale_pool,
    const float* v_scale_pool, float* partials, uint32_t splits, uint32_t pages_per_split,
    hipStream_t stream) {
    return static_cast<hipError_t>(psk_attention_paged_fp8_e4m3_split(
        C(common), k_pool, v_pool, k_scale_pool, v_scale_pool, partials, splits, pages_per_split,
        stream));
}

hipError_t launch_attention_paged_split_reduce_ex(const PagedAttentionCommonArgs& common,
                                                  const float* partials, uint32_t splits,
                                                  uint32_t pages_per_split, hipStream_t stream) {
    return static_cast<hipError_t>(
        psk_attention_paged_split_reduce_ex(C(common), partials, splits, pages_per_split, stream));
}

}  // namespace ps::kernel
