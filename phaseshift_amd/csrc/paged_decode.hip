// Paged-attention decode over GQA KV pages, gfx950: BF16, FP8 E4M3, PSQ8_W32
// or PSQ4_W32 KV.
//
// Reference behaviour restated (file:line in the reference repository):
//   visibility (pos + 1), row skip rules, invalid page  paged_decode.hip:79-97,123-128
//   BF16 math  s = scale*q.k, online softmax, out = acc/sum   paged_decode.hip:135-205
//   FP8 math   s = (q.dec(k))*k_scale*scale,
//              acc += (p*v_scale)*dec(v)                     paged_decode.hip:1064-1090
//   PSQ math   k, v = bf16 scale of the 32-value block x codebook value,
//              fp32 attention over the dequantised values   paged_decode.hip:1206-1383,1667-1847
//   split rule per = ceil(pages/splits), partial (m, P, A)   paged_decode.hip:315-320,413-471
//   combine g = max m_s, W_s = e^(m_s-g),
//           out = sum W_s A_s / sum W_s P_s                  paged_decode.hip:474-555
//   launcher validation                                      paged_decode.hip:228-259,787-817,
//                                                            1588-1610,2098-2127
//
// MI355X design. The whole GQA group (q_per_kv <= 16 query heads) is the N=16
// side of v_mfma_f32_16x16x32_bf16, so each K/V byte is read from HBM once per
// (row, kv_head) instead of once per query head:
//   S^T[16 tokens x 16 heads] = K[16 x D] * Q^T[D x 16]   (D/32 MFMAs)
//   O^T[16 dims x 16 heads]  += V^T[16 x 32 tokens] * P^T[32 tokens x 16 heads]
// A wave owns one kv head of a (row, split) and streams 32-token chunks of K,
// V and scales into LDS with LDS DMA, two chunks in flight; the K operand is
// read from LDS row-wise, the V operand with the transposing LDS reads.
// FP8 codes become bf16 exactly (v_cvt_scalef32_pk_bf16_fp8); k_scale
// multiplies the score and v_scale is folded into P before PV.
// PSQ: each K-step of the score product is exactly one 32-value block, so its
// partial score is multiplied by that block's K scale in fp32; P is multiplied
// by the V scale of each block before the PV MFMAs of the block's 32 dims.
// PSQ4 nibbles become E4M3 codes of the same value (v_perm table), exact;
// the K codes go to the fp8 MFMA as they are, against Q as E4M3 hi + lo parts
// (about 2^-8 relative per element, one power of two per 32-dim block), and
// the V codes become bf16 exactly. Two operands are rounded before the fp32
// accumulation on the PSQ paths: that Q split (PSQ4) and P x V scale, a
// single bf16 operand (8 significant bits) in the PV product; BF16 and FP8
// carry P as a bf16 hi + lo pair instead.
#include "device_common.h"

#include <phaseshift_kv/paged_attention.h>

#include <cfloat>
#include <mutex>

namespace psk {
namespace {

struct DecodeParams {
    psk_paged_attention_args a;
    const uint8_t* k_pool;
    const uint8_t* v_pool;
    const void* k_scale;      // FP8: f32 per (token, head); PSQ: bf16 per block
    const void* v_scale;
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

template <int FMT>
constexpr int chunk_halves() { return FMT == kFmtBf16 ? 1 : 2; }   // 16-token halves per chunk

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

// Largest rows x splits of a split launch whose workgroups take dense units:
// each workgroup scans every row to find its unit, which stays cheap up to
// this size; larger launches have enough workgroups to balance without it.
constexpr uint64_t kDenseDecodeUnits = 4096;

// Maps a unit index to (row, split). Split launches up to kDenseDecodeUnits:
// dense units (find_dense_unit over the rows: every row's splits but the
// last, row-major, then the last split of every row). Unsplit launches: unit
// u is row u. Larger split launches: unit u is (u / splits, u % splits).
// Returns false for a unit without work. All NW*64 threads of the workgroup
// must call it (the branch taken is uniform).
template <int NW>
__device__ bool find_unit(const psk_paged_attention_args& a, uint32_t splits, uint32_t pps,
                          uint32_t unit, uint32_t& row, uint32_t& split) {
    if (splits == 1u) {
        row = unit;
        split = 0u;
        return unit < a.rows && row_units(a, 1u, pps, unit) != 0u;
    }
    if ((uint64_t)a.rows * splits > kDenseDecodeUnits) {
        row = unit / splits;
        split = unit % splits;
        return row < a.rows && split < row_units(a, splits, pps, row);
    }
    return find_dense_unit<NW>(
        a.rows, [&](uint32_t r) { return row_units(a, splits, pps, r); }, unit, row, split);
}

constexpr uint32_t kPageWindow = 1024;   // block-table entries staged in LDS per pass

// PSQ4 workgroups are VALU-bound (nibble expansion, per-block scales), so two
// of them share a CU: a 512-entry window keeps the LDS of one under 80 KB and
// the register budget is 256 per wave. Every other format runs one per CU.
template <int FMT>
constexpr uint32_t page_window() { return FMT == kFmtPsq4 ? 512u : kPageWindow; }
template <int FMT>
constexpr int waves_per_simd() { return FMT == kFmtPsq4 ? 2 : 1; }

// LDS bytes of one pipeline stage of one wave: K and V of a chunk (lane-major
// DMA layout) and, FP8 and PSQ, the k/v scales of its tokens (256 B per
// 16-token half).
template <int FMT, int D>
constexpr int stage_bytes() {
    return 2 * chunk_halves<FMT>() * (16 * code_bytes<FMT, D>() + 128) +
           (FMT != kFmtBf16 ? 2 * chunk_halves<FMT>() * 256 : 0);
}

// kIndep: the 4 waves of a workgroup are 4 independent items, the kv heads
// 4*kv_group + w of one (row, split); they stream the same tokens (adjacent
// head slices of each token row) and need no merge. Otherwise the 4 waves
// share one (row, kv_head, split) item, take its chunks round robin and merge
// through LDS at the end (used when the independent grid cannot fill the GPU).
// PK (PSQ4, q_per_kv <= 8): the score MFMA's 16 columns carry the group's
// heads twice, columns n and n + 8 both head n, and take the two 16-token
// halves of a chunk, so that every lane holds useful scores of one half
// (see consume_pk).
template <int FMT, int D, bool kIndep, int NW, bool PK = false>
__global__ __launch_bounds__(NW * 64, waves_per_simd<FMT>()) void paged_decode_kernel(const DecodeParams p) {
    constexpr uint32_t NT = NW * 64;   // threads of the workgroup
    static_assert(kIndep || NW == kWaves, "the shared-item merge uses 4 waves");
    constexpr int KVB = FMT == kFmtBf16 ? 2 : 1;
    constexpr bool kPsq = fmt_psq<FMT>();
    constexpr int CB = code_bytes<FMT, D>();   // K (V) bytes of one token's head slice
    constexpr int H = chunk_halves<FMT>();
    constexpr int CT = 16 * H;         // tokens per chunk
    constexpr int NL = CB / 64;        // 16 B loads per lane per 16-token half
    constexpr int NS = D / 32;         // MFMA K-steps of the score product
    constexpr int NDB = D / 16;        // 16-dim blocks of the output
    // a 16-token half of K (V) in LDS, padded by 128 B so that the two halves
    // of a chunk fall on opposite halves of the 64 LDS banks (the transposing
    // V reads of one instruction touch both)
    constexpr int HALF_STRIDE = 16 * CB + 128;
    constexpr int KV_BYTES = H * HALF_STRIDE;               // K (or V) of one chunk
    constexpr int SC_BYTES = KVB == 1 ? H * 256 : 0;       // k (or v) scales of one chunk
    constexpr int STAGE = stage_bytes<FMT, D>();
    // Head slices of a multiple of 128 B (kLineLayout): a 16-token half of K
    // (V) sits in LDS as NL 1 KB blocks, block j = tokens 8(j&1)..+7 x bytes
    // [128(j>>1), +128), token row r (of 8) at +128r, its 16 B column c (of 8)
    // at +16(c ^ r): each DMA instruction reads whole 128 B lines and the
    // column reads stay conflict-free. Otherwise block i = bytes [64i, +64)
    // of 16 tokens, lane-major.
    // PSQ4 keeps the lane-major layout: at 128 B per token slice the line
    // layout measured slower for it (4.53 against 4.7 TB/s at b64/32k).
    constexpr bool kLineLayout = CB % 128 == 0 && FMT != kFmtPsq4;
    // PSQ: dwords of block scales per token head (2 bf16 each); the scales of
    // a 16-token half sit dword-major in LDS: dword w of token t at 64w + 4t
    constexpr int SW = D / 64;
    constexpr uint32_t kWin = page_window<FMT>();
    constexpr int kWinBytes = (int)kWin * 4;
    // vector-memory operations of one issue(): K and V DMAs and the scale DMAs
    constexpr int kStepOps = H * (2 * NL + (KVB == 1 ? 2 : 0));
    constexpr uint32_t kStride = kIndep ? CT : NW * CT;   // a wave's chunk stride
    static_assert(NL >= 1 && NS >= 1, "head_dim too small for this kernel");

    extern __shared__ __align__(16) uint8_t lds[];
    __shared__ uint32_t bad_shared;

    const psk_paged_attention_args& a = p.a;
    const uint32_t tid = threadIdx.x;
    const uint32_t lane = tid & 63u;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // uniform: scalar addressing
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
    static_assert(!PK || FMT == kFmtPsq4, "packed columns: PSQ4");
    const uint32_t qn = PK ? (n & 7u) : n;   // this lane's head (column)
    {
        const bool hv = qn < qpk;
        const uint16_t* qrow = static_cast<const uint16_t*>(a.q) + (uint64_t)row * a.q_row_stride +
                               (uint64_t)(kvh * qpk + (hv ? qn : 0u)) * D;
#pragma unroll
        for (int s = 0; s < NS; ++s) {
            if constexpr (FMT == kFmtPsq4) {
                qf[s] = load_q4x2(qrow + s * 32 + (int)g * 4, hv);
            } else {
                const int d0 = (FMT == kFmtBf16 || FMT == kFmtPsq8)
                                   ? s * 32 + (int)g * 8
                                   : (s >> 1) * 64 + (int)g * 16 + (s & 1) * 8;
                qf[s] = load_q8(qrow + d0, hv);
            }
        }
    }
    // PSQ4: the score product runs on the fp8 MFMA with the K codes as the
    // E4M3 bytes of their cb10 values (exact), so no K value is converted.
    // Q goes in as E4M3 hi + lo parts of q * 2^sh (sh = 8 - E for the head's
    // max|q| = m * 2^E, m in [0.5, 1)): hi = RNE(q * 2^sh), lo = RNE(q * 2^sh
    // - hi), which keep q to 2^-8 relative (the residual is exact in fp32);
    // the scores take the factor qinv = 2^-sh. Byte j of an operand is
    // element j of the bf16 operand it replaces (same dims, same order).
    // Each 32-dim block s (one K-step, one K block scale) takes its own power
    // of two: q * 2^(sh + d_s), d_s = E - E_s for the block's max|q| = m_s *
    // 2^E_s, and the block's partial scores the factor qfac[s] = 2^-d_s next
    // to its K scale. A block of small Q elements then keeps 2^-8 relative
    // even where its K block scale is large (a single power of two per head
    // would leave it 2^-17 of the head maximum in absolute terms).
    constexpr bool kQ8 = FMT == kFmtPsq4;
    uint64_t q8h[kQ8 ? NS : 1], q8l[kQ8 ? NS : 1];
    float qinv = 1.0f;
    float qfac[kQ8 ? NS : 1];
    if constexpr (kQ8) {
        float bmax[NS];
        float amax = 0.0f;
#pragma unroll
        for (int s = 0; s < NS; ++s) {
            const u32x4 w = __builtin_bit_cast(u32x4, qf[s]);
            bmax[s] = 0.0f;
#pragma unroll
            for (int k = 0; k < 4; ++k)
                bmax[s] = __builtin_fmaxf(bmax[s],
                                          __builtin_fmaxf(__builtin_fabsf(__uint_as_float(w[k] << 16)),
                                                          __builtin_fabsf(__uint_as_float(w[k] & 0xFFFF0000u))));
            bmax[s] = max_xor32(max_xor16(bmax[s]));   // the head's lanes (n, g = 0..3)
            amax = __builtin_fmaxf(amax, bmax[s]);
        }
        const bool fin = amax > 0.0f && amax <= 3.0e38f;
        const int eh = __builtin_amdgcn_frexp_expf(amax);
        const int sh = fin ? 8 - eh : 0;
        int dsv[NS];
#pragma unroll
        for (int s = 0; s < NS; ++s) {
            dsv[s] = (fin && bmax[s] > 0.0f) ? min(eh - __builtin_amdgcn_frexp_expf(bmax[s]), 120) : 0;
            qfac[s] = __builtin_ldexpf(1.0f, -dsv[s]);
        }
#pragma unroll
        for (int s = 0; s < NS; ++s) {
            const u32x4 w = __builtin_bit_cast(u32x4, qf[s]);
            uint32_t hw[2], lw[2];
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                float y[4], r[4];
#pragma unroll
                for (int t = 0; t < 2; ++t) {
                    y[2 * t] = __builtin_ldexpf(__uint_as_float(w[2 * h + t] << 16), sh + dsv[s]);
                    y[2 * t + 1] = __builtin_ldexpf(__uint_as_float(w[2 * h + t] & 0xFFFF0000u), sh + dsv[s]);
                }
                hw[h] = e4m3x4_rne(y[0], y[1], y[2], y[3]);
                r[0] = y[0] - __builtin_amdgcn_cvt_f32_fp8((int)hw[h], 0);
                r[1] = y[1] - __builtin_amdgcn_cvt_f32_fp8((int)hw[h], 1);
                r[2] = y[2] - __builtin_amdgcn_cvt_f32_fp8((int)hw[h], 2);
                r[3] = y[3] - __builtin_amdgcn_cvt_f32_fp8((int)hw[h], 3);
                lw[h] = e4m3x4_rne(r[0], r[1], r[2], r[3]);
            }
            q8h[s] = (uint64_t)hw[0] | ((uint64_t)hw[1] << 32);
            q8l[s] = (uint64_t)lw[0] | ((uint64_t)lw[1] << 32);
        }
        qinv = __builtin_ldexpf(1.0f, -sh);
    }
    // PK: the Q operands with the columns of the other half zeroed (lanes
    // n < 8 carry half 0's heads, lanes n >= 8 half 1's), so the two halves'
    // score MFMAs accumulate into one result whose column n is the product of
    // lane n's own half
    uint64_t q8m[PK ? 2 : 1][PK ? 2 * NS : 1];
    if constexpr (PK) {
#pragma unroll
        for (int hf = 0; hf < 2; ++hf)
#pragma unroll
            for (int s = 0; s < NS; ++s) {
                const bool mine = (n >> 3) == (uint32_t)hf;
                q8m[hf][2 * s] = mine ? q8h[s] : 0u;
                q8m[hf][2 * s + 1] = mine ? q8l[s] : 0u;
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
    // kLineLayout (FP8): the same (token, bytes) at their line-layout places.
    //   K word i (bytes [64i + 16g, +16) of token n): 2048*(i>>1) + (i odd ? k_line ^ 64 : k_line)
    //   V block db (bytes [16db, +16) of the tr-read token, +8*(n&1)):
    //     v_line + 2048*(db>>3) + (16*(token & 7) ^ 16*(db & 7))
    //   BF16 V block db (tr16 token t = 4g + (n>>2), bytes 32db + 16((n>>1)&1) + 8(n&1)):
    //     v_line + 2048*(db>>2) + (32*(db&3) ^ v_row16)
    //   PSQ8 K (bytes 32s + 8g of token n): 2048*(s>>2) + k_line + (32*(s&3) ^ k_x)
    //   PSQ4 K (bytes 16s + 4g of token n): k_line + (16*s ^ k_x)
    uint32_t k_line = 0, k_x = 0, v_line = 0, v_row16 = 0;
    if constexpr (kLineLayout) {
        const uint32_t r = n & 7u;
        if constexpr (FMT == kFmtPsq8) {
            k_line = 1024u * (n >> 3) + 128u * r + 8u * (g & 1u);
            k_x = (16u * (g >> 1)) ^ (16u * r);
        } else if constexpr (FMT == kFmtPsq4) {
            k_line = 1024u * (n >> 3) + 128u * r + 4u * g;
            k_x = 16u * r;
        } else {
            k_line = 1024u * (n >> 3) + 128u * r + 16u * (g ^ r);
        }
        if constexpr (KVB == 1) {
            const uint32_t j = n >> 1;
            const uint32_t t = 4u * g + (j & 3u);   // token within its half
            v_row16 = 16u * (t & 7u);
            v_line = (j < 4u ? 0u : (uint32_t)HALF_STRIDE) + 1024u * (t >> 3) + 128u * (t & 7u) + 8u * (n & 1u);
        } else {
            const uint32_t t = 4u * g + (n >> 2);
            v_row16 = (16u * ((n >> 1) & 1u)) ^ (16u * (t & 7u));
            v_line = 1024u * (t >> 3) + 128u * (t & 7u) + 8u * (n & 1u);
        }
    }

    float m_run = -INFINITY;   // running max (log2 units), head n
    float l_run = 0.0f;        // partial softmax sum of this lane's tokens
    f32x4 o[NDB];
#pragma unroll
    for (int db = 0; db < NDB; ++db) o[db] = (f32x4){0.f, 0.f, 0.f, 0.f};

    // One pass per window of kWin pages (a single pass unless the
    // split holds more pages than that).
    for (uint32_t wp = pb; wp < pe; wp += kWin) {
        const uint32_t wp_end = min(pe, wp + kWin);
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
                // FP8 scale index; PSQ (token, head) slice index
                const uint64_t si = ((scale_layer + page) * P + off) * a.kv_heads + kvh;
                const uint64_t cbase =
                    kPsq ? si * CB
                         : (layer_base + (uint64_t)page * a.elems_per_page +
                            (uint64_t)off * a.elems_per_token + (uint64_t)kvh * D) * KVB;
                if constexpr (kLineLayout) {
                    // instruction j: tokens 8(j&1) + (lane>>3) of the half, 16 B
                    // column 8(j>>1) + ((lane&7) ^ (lane>>3)); every 8 lanes read
                    // one token's whole 128 B line (non-temporal: read once)
#pragma unroll
                    for (int tg = 0; tg < 2; ++tg) {
                        const uint32_t tau8 = min(c + (uint32_t)hf * 16u + 8u * tg + (lane >> 3), t_last);
                        uint32_t page8 = win[tau8 / P - wp];
                        const bool inv8 = page8 >= a.num_pages;
                        bad |= inv8;
                        page8 = inv8 ? 0u : page8;
                        const uint32_t off8 = tau8 % P;
                        const uint64_t si8 = ((scale_layer + page8) * P + off8) * a.kv_heads + kvh;
                        const uint64_t b8 =
                            (kPsq ? si8 * CB
                                  : (layer_base + (uint64_t)page8 * a.elems_per_page +
                                     (uint64_t)off8 * a.elems_per_token + (uint64_t)kvh * D) * KVB) +
                            16u * ((lane & 7u) ^ (lane >> 3));
#pragma unroll
                        for (int cb = 0; cb < NL / 2; ++cb) {
                            const int j = 2 * cb + tg;
                            load_lds<16, kCpolStream>(p.k_pool + b8 + 128 * cb, st + hf * HALF_STRIDE + j * 1024);
                            load_lds<16, kCpolStream>(p.v_pool + b8 + 128 * cb,
                                                      st + KV_BYTES + hf * HALF_STRIDE + j * 1024);
                        }
                    }
                } else {
                    const uint8_t* ks = p.k_pool + cbase + g * 16;
                    const uint8_t* vs = p.v_pool + cbase + g * 16;
#pragma unroll
                    for (int i = 0; i < NL; ++i) load_lds<16>(ks + i * 64, st + hf * HALF_STRIDE + i * 1024);
#pragma unroll
                    for (int i = 0; i < NL; ++i)
                        load_lds<16>(vs + i * 64, st + KV_BYTES + hf * HALF_STRIDE + i * 1024);
                }
                if constexpr (FMT == kFmtFp8) {
                    load_lds<4>(static_cast<const float*>(p.k_scale) + si, st + 2 * KV_BYTES + hf * 256);
                    load_lds<4>(static_cast<const float*>(p.v_scale) + si,
                                st + 2 * KV_BYTES + SC_BYTES + hf * 256);
                } else if constexpr (kPsq) {
                    // lane (n, g): dword g of token n's block scales (lane
                    // groups past SW repeat a dword into unused LDS)
                    const uint64_t sb = si * (uint64_t)(4 * SW) + 4u * (g % (uint32_t)SW);
                    load_lds<4>(static_cast<const uint8_t*>(p.k_scale) + sb, st + 2 * KV_BYTES + hf * 256);
                    load_lds<4>(static_cast<const uint8_t*>(p.v_scale) + sb,
                                st + 2 * KV_BYTES + SC_BYTES + hf * 256);
                }
            }
        };

        // Scores, online softmax and PV of the chunk at c held in stage st.
        auto consume = [&](uint32_t c, const uint8_t* st) __attribute__((always_inline)) {
            f32x4 sc[H];
#pragma unroll
            for (int hf = 0; hf < H; ++hf) {
                f32x4 acc = {0.f, 0.f, 0.f, 0.f};
                if constexpr (kPsq) {
                    // K-step s = block s: its partial scores times the block's
                    // K scale of each token 4g + r (bf16 -> f32 by shift).
                    const uint8_t* kb = st + hf * HALF_STRIDE;
                    const uint8_t* kscl = st + 2 * KV_BYTES + hf * 256 + 16 * g;
#pragma unroll
                    for (int s = 0; s < NS; ++s) {
                        bf16x8 kf;
                        [[maybe_unused]] long kf8 = 0;
                        if constexpr (FMT == kFmtPsq8) {
                            // bytes 32s + 8g .. +8 of token n
                            const u32x2 w = kLineLayout
                                ? *reinterpret_cast<const u32x2*>(kb + 2048 * (s >> 2) + k_line +
                                                                  ((32u * (s & 3)) ^ k_x))
                                : *reinterpret_cast<const u32x2*>(
                                      kb + 1024 * (s >> 1) + 16 * (16 * (2 * (s & 1) + (int)(g >> 1)) + (int)n) +
                                      8 * (int)(g & 1u));
                            kf = fp8x8_to_bf16x8(w[0], w[1]);
                        } else {
                            // bytes 16s + 4g .. +4 of token n: dims 4g.. (low
                            // nibbles) and 16 + 4g.. (high nibbles) of block s
                            const uint32_t x = kLineLayout
                                ? *reinterpret_cast<const uint32_t*>(kb + k_line + ((16u * s) ^ k_x))
                                : *reinterpret_cast<const uint32_t*>(kb + 256 * s + 16 * n + 4 * g);
                            const uint64_t ka = (uint64_t)psq4_e4m3x4(x, false) |
                                                ((uint64_t)psq4_e4m3x4(x, true) << 32);
                            kf8 = (long)ka;
                        }
                        f32x4 part;
                        if constexpr (kQ8) {
                            part = __builtin_amdgcn_mfma_f32_16x16x32_fp8_fp8(
                                kf8, (long)q8h[s], (f32x4){0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                            part = __builtin_amdgcn_mfma_f32_16x16x32_fp8_fp8(kf8, (long)q8l[s], part, 0, 0, 0);
                        } else {
                            part = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                                kf, qf[s], (f32x4){0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                        }
                        const u32x4 kw = *reinterpret_cast<const u32x4*>(kscl + 64 * (s >> 1));
                        if constexpr (kQ8) part *= qfac[s];
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            const float ksc = __uint_as_float((s & 1) ? (kw[r] & 0xFFFF0000u) : (kw[r] << 16));
                            acc[r] = s == 0 ? part[r] * ksc : __builtin_fmaf(part[r], ksc, acc[r]);
                        }
                    }
                } else {
                    const uint8_t* kb = st + hf * HALF_STRIDE + 16 * lane;
#pragma unroll
                    for (int s = 0; s < NS; ++s) {
                        bf16x8 kf;
                        if constexpr (KVB == 2 && kLineLayout) {
                            kf = *reinterpret_cast<const bf16x8*>(st + hf * HALF_STRIDE + 2048 * (s >> 1) +
                                                                 ((s & 1) ? (k_line ^ 64u) : k_line));
                        } else if constexpr (KVB == 2) {
                            kf = *reinterpret_cast<const bf16x8*>(kb + 1024 * s);
                        } else if constexpr (kLineLayout) {
                            // bytes [64i + 16g, +16) of token n, i = s >> 1
                            const int i = s >> 1;
                            const u32x4 w = *reinterpret_cast<const u32x4*>(
                                st + hf * HALF_STRIDE + 2048 * (i >> 1) + ((i & 1) ? (k_line ^ 64u) : k_line));
                            kf = (s & 1) ? fp8x8_to_bf16x8(w[2], w[3]) : fp8x8_to_bf16x8(w[0], w[1]);
                        } else {
                            const u32x4 w = *reinterpret_cast<const u32x4*>(kb + 1024 * (s >> 1));
                            kf = (s & 1) ? fp8x8_to_bf16x8(w[2], w[3]) : fp8x8_to_bf16x8(w[0], w[1]);
                        }
                        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf, qf[s], acc, 0, 0, 0);
                    }
                }
                sc[hf] = acc;
            }

            // online softmax (log2 units) for head n over tokens 4g + r
            float s2[H][4], vsc[H][4];
            float mx = -INFINITY;
#pragma unroll
            for (int hf = 0; hf < H; ++hf) {
                f32x4 kscale = {1.f, 1.f, 1.f, 1.f}, vscale = {1.f, 1.f, 1.f, 1.f};
                if constexpr (FMT == kFmtFp8) {
                    kscale = *reinterpret_cast<const f32x4*>(st + 2 * KV_BYTES + hf * 256 + 16 * g);
                    vscale = *reinterpret_cast<const f32x4*>(st + 2 * KV_BYTES + SC_BYTES + hf * 256 +
                                                             16 * g);
                }
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const bool ok = c + hf * 16 + 4u * g + (uint32_t)r < te;
                    s2[hf][r] = ok ? sc[hf][r] * (p.scale_log2 * (kQ8 ? qinv : kscale[r])) : -INFINITY;
                    vsc[hf][r] = vscale[r];
                    mx = __builtin_fmaxf(mx, s2[hf][r]);
                }
            }
            mx = max_xor32(max_xor16(mx));   // lane permutes, no LDS round trip
            // m_run is the head's softmax reference. BF16 / FP8 (P as a bf16 hi +
            // lo pair): it moves only when a score exceeds it by more than
            // kLazyMaxSlack (then P <= 2^slack). PSQ (P x V scale as one bf16
            // operand): it is the running maximum, so the largest weight of a
            // row is 1, exact in bf16.
            const bool moved = mx > m_run + (kPsq ? 0.0f : kLazyMaxSlack);
            const float m_new = moved ? mx : m_run;
            const float m_use = m_new == -INFINITY ? 0.0f : m_new;
            const float alpha = moved ? __builtin_amdgcn_exp2f(m_run - m_use) : 1.0f;
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
            // O is rescaled only when some head's reference moved.
            if (__any(moved)) {
#pragma unroll
                for (int db = 0; db < NDB; ++db) o[db] *= alpha;
            }

            // O^T += V^T * P^T. P (v_scale folded in) as hi + lo bf16 pairs:
            // two MFMAs keep ~16 mantissa bits of every weight (V and K are
            // exact in bf16).
            const uint8_t* vb = st + KV_BYTES + tr_off;
            if constexpr (kPsq) {
                // Per block b: P times the block's V scale of each token (the
                // lane's tokens 4g + r of both halves), one bf16 P operand,
                // then the MFMAs of the block's two 16-dim output blocks.
                const uint8_t* vscl = st + 2 * KV_BYTES + SC_BYTES + 16 * g;
#pragma unroll
                for (int b = 0; b < NS; ++b) {
                    const u32x4 w0 = *reinterpret_cast<const u32x4*>(vscl + 64 * (b >> 1));
                    const u32x4 w1 = *reinterpret_cast<const u32x4*>(vscl + 256 + 64 * (b >> 1));
                    float f[8];
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        f[r] = pv[0][r] * __uint_as_float((b & 1) ? (w0[r] & 0xFFFF0000u) : (w0[r] << 16));
                        f[4 + r] = pv[1][r] * __uint_as_float((b & 1) ? (w1[r] & 0xFFFF0000u) : (w1[r] << 16));
                    }
                    u32x4 ph;
#pragma unroll
                    for (int i = 0; i < 4; ++i) ph[i] = pack_bf16x2(f[2 * i], f[2 * i + 1]);
                    const bf16x8 pf = __builtin_bit_cast(bf16x8, ph);
                    if constexpr (FMT == kFmtPsq8) {
#pragma unroll
                        for (int h = 0; h < 2; ++h) {
                            const int db = 2 * b + h;
                            const i32x2 w = kLineLayout
                                ? lds_read_tr8(st + KV_BYTES + v_line + 2048 * (db >> 3) + (v_row16 ^ (16u * (db & 7))))
                                : lds_read_tr8(vb + 256 * db);
                            const bf16x8 vf = fp8x8_to_bf16x8((uint32_t)w[0], (uint32_t)w[1]);
                            o[2 * b + h] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf, pf, o[2 * b + h], 0, 0, 0);
                        }
                    } else {
                        // byte i of block b for 8 tokens: dim i (low nibble)
                        // and dim 16 + i (high nibble)
                        const i32x2 w = kLineLayout
                            ? lds_read_tr8(st + KV_BYTES + v_line + 2048 * (b >> 3) + (v_row16 ^ (16u * (b & 7))))
                            : lds_read_tr8(vb + 256 * b);
                        const bf16x8 vlo = fp8x8_to_bf16x8(psq4_e4m3x4((uint32_t)w[0], false),
                                                           psq4_e4m3x4((uint32_t)w[1], false));
                        const bf16x8 vhi = fp8x8_to_bf16x8(psq4_e4m3x4((uint32_t)w[0], true),
                                                           psq4_e4m3x4((uint32_t)w[1], true));
                        o[2 * b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vlo, pf, o[2 * b], 0, 0, 0);
                        o[2 * b + 1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vhi, pf, o[2 * b + 1], 0, 0, 0);
                    }
                }
            } else if constexpr (KVB == 1) {
                u32x4 ph, pl;
                { const u32x2 t_ = split_bf16x2(pv[0][0], pv[0][1]); ph[0] = t_[0]; pl[0] = t_[1]; }
                { const u32x2 t_ = split_bf16x2(pv[0][2], pv[0][3]); ph[1] = t_[0]; pl[1] = t_[1]; }
                { const u32x2 t_ = split_bf16x2(pv[1][0], pv[1][1]); ph[2] = t_[0]; pl[2] = t_[1]; }
                { const u32x2 t_ = split_bf16x2(pv[1][2], pv[1][3]); ph[3] = t_[0]; pl[3] = t_[1]; }
                const bf16x8 pfh = __builtin_bit_cast(bf16x8, ph);
                const bf16x8 pfl = __builtin_bit_cast(bf16x8, pl);
#pragma unroll
                for (int db = 0; db < NDB; ++db) {
                    i32x2 w;
                    if constexpr (kLineLayout)
                        w = lds_read_tr8(st + KV_BYTES + v_line + 2048 * (db >> 3) + (v_row16 ^ (16u * (db & 7))));
                    else
                        w = lds_read_tr8(vb + 256 * db);
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
                    const i16x4 vf = kLineLayout
                        ? lds_read_tr16(st + KV_BYTES + v_line + 2048 * (db >> 2) + ((32u * (db & 3)) ^ v_row16))
                        : lds_read_tr16(vb + 512 * db);
                    o[db] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(vf, pfh, o[db], 0, 0, 0);
                    o[db] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(vf, pfl, o[db], 0, 0, 0);
                }
            }
        };

        // PK: scores, softmax and PV of the chunk at c with one accumulator
        // per lane. Column n of the score MFMAs is head n & 7 for 16-token
        // half n >> 3: each K-step runs the two halves' K fragments against
        // the same Q operand (heads in columns n and n + 8) and keeps, per
        // lane, the product of its own half, so the per-block K scales, the
        // softmax and the per-block V scales touch 4 useful values per lane
        // instead of 8 with 10 of 16 columns idle. The PV operand of head
        // column n takes its 4 P values of half 0 and lane n + 8's of half 1.
        auto consume_pk = [&](uint32_t c, const uint8_t* st) __attribute__((always_inline)) {
            const uint32_t half = n >> 3;
            const uint8_t* kscl = st + 2 * KV_BYTES + half * 256 + 16 * g;
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int s = 0; s < NS; ++s) {
                f32x4 part = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int hf = 0; hf < H; ++hf) {
                    // bytes 16s + 4g .. +4 of token n: dims 4g.. (low nibbles)
                    // and 16 + 4g.. (high nibbles) of block s
                    const uint32_t x = *reinterpret_cast<const uint32_t*>(st + hf * HALF_STRIDE + 256 * s + 16 * n + 4 * g);
                    const long ka = (long)((uint64_t)psq4_e4m3x4(x, false) | ((uint64_t)psq4_e4m3x4(x, true) << 32));
                    part = __builtin_amdgcn_mfma_f32_16x16x32_fp8_fp8(ka, (long)q8m[hf][2 * s], part, 0, 0, 0);
                    part = __builtin_amdgcn_mfma_f32_16x16x32_fp8_fp8(ka, (long)q8m[hf][2 * s + 1], part, 0, 0, 0);
                }
                const u32x4 kw = *reinterpret_cast<const u32x4*>(kscl + 64 * (s >> 1));
                part *= qfac[s];
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float ksc = __uint_as_float((s & 1) ? (kw[r] & 0xFFFF0000u) : (kw[r] << 16));
                    acc[r] = s == 0 ? part[r] * ksc : __builtin_fmaf(part[r], ksc, acc[r]);
                }
            }
            // online softmax (log2 units) for head n & 7 over tokens 16 half + 4g + r
            float s2[4];
            float mx = -INFINITY;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const bool ok = c + 16u * half + 4u * g + (uint32_t)r < te;
                s2[r] = ok ? acc[r] * (p.scale_log2 * qinv) : -INFINITY;
                mx = __builtin_fmaxf(mx, s2[r]);
            }
            mx = max_xor32(max_xor16(mx));
            mx = __builtin_fmaxf(mx, row_ror8(mx));   // the other half
            const bool moved = mx > m_run;   // the running maximum (PSQ, see consume)
            const float m_new = moved ? mx : m_run;
            const float m_use = m_new == -INFINITY ? 0.0f : m_new;
            const float alpha = moved ? __builtin_amdgcn_exp2f(m_run - m_use) : 1.0f;
            float pv[4], psum = 0.0f;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                pv[r] = __builtin_amdgcn_exp2f(s2[r] - m_use);
                psum += pv[r];
            }
            l_run = l_run * alpha + psum;
            m_run = m_new;
            if (__any(moved)) {
#pragma unroll
                for (int db = 0; db < NDB; ++db) o[db] *= alpha;
            }
            // O^T += V^T P^T per block b: P times the block's V scale of each
            // of the lane's tokens, one bf16 operand (own half, then lane
            // n ^ 8's half; columns 8-15 of O are never written)
            const uint8_t* vscl = st + 2 * KV_BYTES + SC_BYTES + half * 256 + 16 * g;
            const uint8_t* vb = st + KV_BYTES + tr_off;
#pragma unroll
            for (int b = 0; b < NS; ++b) {
                const u32x4 w = *reinterpret_cast<const u32x4*>(vscl + 64 * (b >> 1));
                float f[4];
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    f[r] = pv[r] * __uint_as_float((b & 1) ? (w[r] & 0xFFFF0000u) : (w[r] << 16));
                const uint32_t own0 = pack_bf16x2(f[0], f[1]), own1 = pack_bf16x2(f[2], f[3]);
                const u32x4 ph = {own0, own1, row_ror8(own0), row_ror8(own1)};
                const bf16x8 pf = __builtin_bit_cast(bf16x8, ph);
                // byte i of block b for 8 tokens: dim i (low nibble) and dim
                // 16 + i (high nibble)
                const i32x2 vw = lds_read_tr8(vb + 256 * b);
                const bf16x8 vlo = fp8x8_to_bf16x8(psq4_e4m3x4((uint32_t)vw[0], false),
                                                   psq4_e4m3x4((uint32_t)vw[1], false));
                const bf16x8 vhi = fp8x8_to_bf16x8(psq4_e4m3x4((uint32_t)vw[0], true),
                                                   psq4_e4m3x4((uint32_t)vw[1], true));
                o[2 * b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vlo, pf, o[2 * b], 0, 0, 0);
                o[2 * b + 1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vhi, pf, o[2 * b + 1], 0, 0, 0);
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
            if constexpr (PK)
                consume_pk(c, cur);
            else
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
        const float l_all = sum_xor32(sum_xor16(PK ? l_run + row_ror8(l_run) : l_run));
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
        const float l_all = sum_xor32(sum_xor16(PK ? l_run + row_ror8(l_run) : l_run));
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
// kv_dtype: PSK_KV_*.
size_t decode_workgroup_lds_bytes(uint32_t kv_dtype, uint32_t head_dim) {
    const size_t D = head_dim <= 64 ? 64 : head_dim <= 128 ? 128 : 256;
    const bool bf16 = kv_dtype == PSK_KV_BF16;
    const size_t H = bf16 ? 1 : 2;
    const size_t cb = bf16 ? 2 * D : kv_dtype == PSK_KV_PSQ4_W32 ? D / 2 : D;
    const size_t stage = 2 * H * (16 * cb + 128) + (bf16 ? 0 : 2 * H * 256);
    const size_t win = kv_dtype == PSK_KV_PSQ4_W32 ? page_window<kFmtPsq4>() : kPageWindow;
    return win * 4 + (size_t)kWaves * 2 * stage;
}

namespace {

template <int FMT, int D, bool kIndep, int NW, bool PK = false>
hipError_t launch_decode_t2(const DecodeParams& p, uint64_t grid, hipStream_t stream) {
    const uint32_t qpk = p.a.q_heads / p.a.kv_heads;
    // block-table window + two pipeline stages per wave; the shared-item merge
    // later reuses the same LDS
    const size_t v_bytes = (size_t)page_window<FMT>() * 4 + (size_t)NW * 2 * stage_bytes<FMT, D>();
    const size_t m_bytes = kIndep ? 0 : (size_t)NW * 32 * sizeof(float) +
                                            (size_t)NW * qpk * D * sizeof(float);
    const size_t lds_bytes = v_bytes > m_bytes ? v_bytes : m_bytes;
    if (grid == 0u || grid > 0x7FFFFFFFull) return hipErrorInvalidValue;
    if (lds_bytes > 64u * 1024u) {
        // gfx950 has 160 KB of LDS per CU; raise the per-kernel dynamic limit.
        static std::atomic<uint64_t> lds_ready{0};
        const hipError_t attr =
            allow_full_lds(reinterpret_cast<const void*>(&paged_decode_kernel<FMT, D, kIndep, NW, PK>), lds_ready);
        if (attr != hipSuccess) return attr;
    }
    hipLaunchKernelGGL((paged_decode_kernel<FMT, D, kIndep, NW, PK>), dim3((uint32_t)grid),
                       dim3(NW * 64), lds_bytes, stream, p);
    return hipGetLastError();
}

// Independent waves (one kv head each) when that grid fills at least half of
// the GPU's 256 CUs; otherwise the 4 waves share each (row, kv_head, split)
// item. The split chooser assumes the same rule.
template <int FMT, int D>
hipError_t launch_decode_t(const DecodeParams& p, hipStream_t stream) {
    const uint64_t units = (uint64_t)p.a.rows * p.splits;
    const uint64_t groups = (p.a.kv_heads + kWaves - 1u) / kWaves;
    if constexpr (FMT == kFmtPsq4) {
        if (p.a.q_heads / p.a.kv_heads <= 8u) {
            if (units * groups >= 128u)
                return launch_decode_t2<FMT, D, true, kWaves, true>(p, units * groups, stream);
            return launch_decode_t2<FMT, D, false, kWaves, true>(p, units * p.a.kv_heads, stream);
        }
    }
    if (units * groups >= 128u) return launch_decode_t2<FMT, D, true, kWaves>(p, units * groups, stream);
    return launch_decode_t2<FMT, D, false, kWaves>(p, units * p.a.kv_heads, stream);
}

template <int FMT>
hipError_t launch_decode(const DecodeParams& p, hipStream_t stream) {
    switch (p.a.head_dim) {
        case 256: return launch_decode_t<FMT, 256>(p, stream);
        case 128: return launch_decode_t<FMT, 128>(p, stream);
        case 64:
            if constexpr (FMT != kFmtPsq4) return launch_decode_t<FMT, 64>(p, stream);
            return hipErrorNotSupported;
        case 32:
            if constexpr (FMT == kFmtBf16) return launch_decode_t<kFmtBf16, 32>(p, stream);
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

DecodeParams make(const psk_paged_attention_args& c, const void* k, const void* v, const void* ks,
                  const void* vs, float* partials, uint32_t splits, uint32_t pps) {
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

// PSQ shapes of the MFMA kernel: q_per_kv <= 16, head_dim 128 or 256 (and
// 64 for PSQ8), code pools 16 B aligned, scale pools 4 B aligned. Every
// (token, head) slice is then 16 B aligned (its offset is a multiple of
// head_dim/2 or head_dim bytes).
bool psq_mfma_shape_ok(const psk_paged_attention_args& c, bool psq4, const void* kp, const void* vp,
                       const void* ks, const void* vs) {
    if (c.q_heads / c.kv_heads > (uint32_t)kMaxQPerKV) return false;
    const uint32_t D = c.head_dim;
    if (!(D == 128 || D == 256 || (D == 64 && !psq4))) return false;
    auto al = [](const void* ptr, uintptr_t n) { return reinterpret_cast<uintptr_t>(ptr) % n == 0u; };
    return al(kp, 16) && al(vp, 16) && al(ks, 4) && al(vs, 4);
}

// Validation shared by the PSQ launchers (paged_decode.hip:1597-1609): the
// common checks, both scale pools, head_dim == 32 * blocks_per_head.
hipError_t validate_psq(const psk_paged_attention_args* a, const void* kc, const void* vc,
                        const void* ks, const void* vs, uint32_t blocks_per_head) {
    if (a == nullptr || kc == nullptr || vc == nullptr || ks == nullptr || vs == nullptr)
        return hipErrorInvalidValue;
    const hipError_t e = validate_common(*a);
    if (e != hipSuccess) return e;
    if (a->head_dim != 32u * blocks_per_head) return hipErrorNotSupported;
    return hipSuccess;
}

}  // namespace

// Generic fallbacks for shapes outside the MFMA kernel (page_ops.hip).
hipError_t launch_attention_generic(const psk_paged_attention_args& c, int kvb, const void* k,
                                    const void* v, const float* ks, const float* vs,
                                    hipStream_t stream);
hipError_t launch_attention_generic_psq(const psk_paged_attention_args& c, bool psq4, const void* k,
                                        const void* v, const uint16_t* ks, const uint16_t* vs,
                                        hipStream_t stream);

// PSQ attention of every row straight to the output (partials == nullptr)
// or into split partials.
hipError_t launch_psq(const psk_paged_attention_args& a, bool psq4, const uint8_t* kc,
                      const uint8_t* vc, const uint16_t* ks, const uint16_t* vs, float* partials,
                      uint32_t splits, uint32_t pps, hipStream_t st) {
    if (!psq_mfma_shape_ok(a, psq4, kc, vc, ks, vs)) {
        if (partials != nullptr) return hipErrorNotSupported;
        return launch_attention_generic_psq(a, psq4, kc, vc, ks, vs, st);
    }
    const DecodeParams p = make(a, kc, vc, ks, vs, partials, splits, pps);
    return psq4 ? launch_decode<kFmtPsq4>(p, st) : launch_decode<kFmtPsq8>(p, st);
}

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
    return psk::launch_decode<psk::kFmtBf16>(psk::make(*a, k_pool, v_pool, nullptr, nullptr, nullptr, 1u, 0u), st);
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
    return psk::launch_decode<psk::kFmtFp8>(
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
    return psk::launch_decode<psk::kFmtBf16>(
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
    return psk::launch_decode<psk::kFmtFp8>(psk::make(*a, k_pool, v_pool, k_scale_pool, v_scale_pool, partials,
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

// ------------------------------------------------------------ PSQ KV
extern "C" int psk_attention_paged_psq(const psk_paged_attention_args* a, uint32_t kv_dtype,
                                       const uint8_t* k_code_pool, const uint8_t* v_code_pool,
                                       const uint16_t* k_scale_pool, const uint16_t* v_scale_pool,
                                       uint32_t blocks_per_head, void* stream) {
    if (kv_dtype != PSK_KV_PSQ4_W32 && kv_dtype != PSK_KV_PSQ8_W32) return hipErrorInvalidValue;
    hipError_t e = psk::validate_psq(a, k_code_pool, v_code_pool, k_scale_pool, v_scale_pool,
                                     blocks_per_head);
    if (e != hipSuccess) return e;
    return psk::launch_psq(*a, kv_dtype == PSK_KV_PSQ4_W32, k_code_pool, v_code_pool, k_scale_pool,
                           v_scale_pool, nullptr, 1u, 0u, static_cast<hipStream_t>(stream));
}

extern "C" int psk_attention_paged_psq_split_ex(const psk_paged_attention_args* a, uint32_t kv_dtype,
                                                const uint8_t* k_code_pool,
                                                const uint8_t* v_code_pool,
                                                const uint16_t* k_scale_pool,
                                                const uint16_t* v_scale_pool,
                                                uint32_t blocks_per_head, float* partials,
                                                uint32_t splits, uint32_t pages_per_split,
                                                void* stream) {
    if (kv_dtype != PSK_KV_PSQ4_W32 && kv_dtype != PSK_KV_PSQ8_W32) return hipErrorInvalidValue;
    hipError_t e = psk::validate_psq(a, k_code_pool, v_code_pool, k_scale_pool, v_scale_pool,
                                     blocks_per_head);
    if (e != hipSuccess) return e;
    if (partials == nullptr || splits == 0u || splits > psk::kMaxSplits) return hipErrorInvalidValue;
    return psk::launch_psq(*a, kv_dtype == PSK_KV_PSQ4_W32, k_code_pool, v_code_pool, k_scale_pool,
                           v_scale_pool, partials, splits, pages_per_split,
                           static_cast<hipStream_t>(stream));
}

// The reference's split launchers accept q_per_kv 4 or 6 and 2, 4, 8 or 16
// splits (paged_decode.hip:2109-2116, 2172-2179).
static int psq_split_ref(const psk_paged_attention_args* a, uint32_t kv_dtype, const uint8_t* kc,
                         const uint8_t* vc, const uint16_t* ks, const uint16_t* vs, uint32_t bph,
                         float* partials, uint32_t splits, void* stream) {
    if (a == nullptr) return hipErrorInvalidValue;
    if (a->kv_heads != 0u && a->q_heads % a->kv_heads == 0u) {
        const uint32_t qpk = a->q_heads / a->kv_heads;
        if (qpk != 4u && qpk != 6u) return hipErrorInvalidValue;
    }
    if (splits != 2u && splits != 4u && splits != 8u && splits != 16u) return hipErrorInvalidValue;
    return psk_attention_paged_psq_split_ex(a, kv_dtype, kc, vc, ks, vs, bph, partials, splits, 0u,
                                            stream);
}

extern "C" int psk_attention_paged_psq4(const psk_paged_attention_args* a, const uint8_t* kc,
                                        const uint8_t* vc, const uint16_t* ks, const uint16_t* vs,
                                        uint32_t bph, void* stream) {
    return psk_attention_paged_psq(a, PSK_KV_PSQ4_W32, kc, vc, ks, vs, bph, stream);
}
extern "C" int psk_attention_paged_psq8(const psk_paged_attention_args* a, const uint8_t* kc,
                                        const uint8_t* vc, const uint16_t* ks, const uint16_t* vs,
                                        uint32_t bph, void* stream) {
    return psk_attention_paged_psq(a, PSK_KV_PSQ8_W32, kc, vc, ks, vs, bph, stream);
}
// Prefill rows run as independent decode rows (each sees its own pos + 1
// tokens, the reference's causal rule).
namespace psk {
bool launch_prefill_psq_tiles(const psk_paged_attention_args& a, uint32_t kv_dtype, const void* kc,
                              const void* vc, const void* ks, const void* vs, hipStream_t stream,
                              hipError_t& err);
}  // namespace psk

// PSQ prefill (paged_prefill.hip:461-490,852-880): 16-row tiles of the
// launch (the tile contract of the BF16 / FP8 prefill launchers) on the tile
// kernel; shapes outside it run row by row on the PSQ decode kernel.
static int prefill_psq(const psk_paged_attention_args* a, uint32_t kv_dtype, const uint8_t* kc,
                       const uint8_t* vc, const uint16_t* ks, const uint16_t* vs, uint32_t bph,
                       void* stream) {
    hipError_t e = psk::validate_psq(a, kc, vc, ks, vs, bph);
    if (e != hipSuccess) return e;
    if (psk::launch_prefill_psq_tiles(*a, kv_dtype, kc, vc, ks, vs, static_cast<hipStream_t>(stream), e))
        return e;
    return psk_attention_paged_psq(a, kv_dtype, kc, vc, ks, vs, bph, stream);
}
extern "C" int psk_attention_paged_prefill_psq4(const psk_paged_attention_args* a, const uint8_t* kc,
                                                const uint8_t* vc, const uint16_t* ks,
                                                const uint16_t* vs, uint32_t bph, void* stream) {
    return prefill_psq(a, PSK_KV_PSQ4_W32, kc, vc, ks, vs, bph, stream);
}
extern "C" int psk_attention_paged_prefill_psq8(const psk_paged_attention_args* a, const uint8_t* kc,
                                                const uint8_t* vc, const uint16_t* ks,
                                                const uint16_t* vs, uint32_t bph, void* stream) {
    return prefill_psq(a, PSK_KV_PSQ8_W32, kc, vc, ks, vs, bph, stream);
}
extern "C" int psk_attention_paged_psq4_split(const psk_paged_attention_args* a, const uint8_t* kc,
                                              const uint8_t* vc, const uint16_t* ks,
                                              const uint16_t* vs, uint32_t bph, float* partials,
                                              uint32_t splits, void* stream) {
    return psq_split_ref(a, PSK_KV_PSQ4_W32, kc, vc, ks, vs, bph, partials, splits, stream);
}
extern "C" int psk_attention_paged_psq8_split(const psk_paged_attention_args* a, const uint8_t* kc,
                                              const uint8_t* vc, const uint16_t* ks,
                                              const uint16_t* vs, uint32_t bph, float* partials,
                                              uint32_t splits, void* stream) {
    return psq_split_ref(a, PSK_KV_PSQ8_W32, kc, vc, ks, vs, bph, partials, splits, stream);
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

// The reference's reduce runs one query head per workgroup in this build.
uint32_t paged_attention_split_reduce_qh_per_wg() { return 1u; }

#define PSK_PSQ_ARGS(common, k, v, ks, vs)                                                   \
    C(common), k, v, reinterpret_cast<const uint16_t*>(ks), reinterpret_cast<const uint16_t*>(vs)

hipError_t launch_attention_paged_psq4(const PagedAttentionCommonArgs& common, const uint8_t* k,
                                       const uint8_t* v, const bf16_t* ks, const bf16_t* vs,
                                       uint32_t bph, hipStream_t stream) {
    return static_cast<hipError_t>(
        psk_attention_paged_psq4(PSK_PSQ_ARGS(common, k, v, ks, vs), bph, stream));
}
hipError_t launch_attention_paged_psq8(const PagedAttentionCommonArgs& common, const uint8_t* k,
                                       const uint8_t* v, const bf16_t* ks, const bf16_t* vs,
                                       uint32_t bph, hipStream_t stream) {
    return static_cast<hipError_t>(
        psk_attention_paged_psq8(PSK_PSQ_ARGS(common, k, v, ks, vs), bph, stream));
}
hipError_t launch_attention_paged_prefill_psq4(const PagedAttentionCommonArgs& common,
                                               const uint8_t* k, const uint8_t* v, const bf16_t* ks,
                                               const bf16_t* vs, uint32_t bph, hipStream_t stream) {
    return static_cast<hipError_t>(
        psk_attention_paged_prefill_psq4(PSK_PSQ_ARGS(common, k, v, ks, vs), bph, stream));
}
hipError_t launch_attention_paged_prefill_psq8(const PagedAttentionCommonArgs& common,
                                               const uint8_t* k, const uint8_t* v, const bf16_t* ks,
                                               const bf16_t* vs, uint32_t bph, hipStream_t stream) {
    return static_cast<hipError_t>(
        psk_attention_paged_prefill_psq8(PSK_PSQ_ARGS(common, k, v, ks, vs), bph, stream));
}
hipError_t launch_attention_paged_psq4_split(const PagedAttentionCommonArgs& common, const uint8_t* k,
                                             const uint8_t* v, const bf16_t* ks, const bf16_t* vs,
                                             uint32_t bph, float* partials, uint32_t splits,
                                             hipStream_t stream) {
    return static_cast<hipError_t>(psk_attention_paged_psq4_split(
        PSK_PSQ_ARGS(common, k, v, ks, vs), bph, partials, splits, stream));
}
hipError_t launch_attention_paged_psq8_split(const PagedAttentionCommonArgs& common, const uint8_t* k,
                                             const uint8_t* v, const bf16_t* ks, const bf16_t* vs,
                                             uint32_t bph, float* partials, uint32_t splits,
                                             hipStream_t stream) {
    return static_cast<hipError_t>(psk_attention_paged_psq8_split(
        PSK_PSQ_ARGS(common, k, v, ks, vs), bph, partials, splits, stream));
}
#undef PSK_PSQ_ARGS

hipError_t launch_attention_paged_split_reduce_ex(const PagedAttentionCommonArgs& common,
                                                  const float* partials, uint32_t splits,
                                                  uint32_t pages_per_split, hipStream_t stream) {
    return static_cast<hipError_t>(
        psk_attention_paged_split_reduce_ex(C(common), partials, splits, pages_per_split, stream));
}

}  // namespace ps::kernel

// ------------------------------------------- allocation-free split decode
// FP8 split-K decode plus its combine with the split partials in a
// library-owned device array instead of a caller workspace, for callers that
// cannot allocate device memory (code under HIP graph capture, serving loops,
// harnesses that forbid hipMalloc). Each GPU the library runs on holds its own
// copy of the array for the life of the process. Every call on a GPU shares
// that GPU's array: calls that overlap on one GPU (two streams, two threads)
// race on it. Nothing in it needs clearing: the split kernel writes every
// partial the combine reads.
namespace {

constexpr uint64_t kNoAllocScratchBytes = PSK_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) float scratch[kNoAllocScratchBytes / sizeof(float)];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
float* g_scratch_ptr[kMaxDevices] = {};

// The array's device address on the current device, looked up once per
// device. In host code `scratch` is only a host-side stand-in for the symbol:
// kernels receive the address returned here, never the name.
hipError_t scratch_for_current_device(float** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch_ptr[dev] == nullptr) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        g_scratch_ptr[dev] = static_cast<float*>(p);
    }
    *out = g_scratch_ptr[dev];
    return hipSuccess;
}

}  // namespace

extern "C" int psk_attention_paged_fp8_e4m3_split_noalloc(const psk_paged_attention_args* a,
                                                          const void* k_pool, const void* v_pool,
                                                          const float* k_scale_pool,
                                                          const float* v_scale_pool,
                                                          uint32_t splits, uint32_t pages_per_split,
                                                          void* stream) {
    if (a == nullptr || k_pool == nullptr || v_pool == nullptr || k_scale_pool == nullptr ||
        v_scale_pool == nullptr)
        return hipErrorInvalidValue;
    hipError_t e = psk::validate_common(*a);
    if (e != hipSuccess) return e;
    if (splits == 0u || splits > psk::kMaxSplits) return hipErrorInvalidValue;
    // the partials of this call must fit the array
    if (psk_attention_split_partials_bytes(a->rows, a->q_heads, a->kv_heads, splits) >
        kNoAllocScratchBytes)
        return hipErrorInvalidValue;
    if (!psk::mfma_shape_ok(*a, 1, k_pool, v_pool)) return hipErrorNotSupported;
    float* parts = nullptr;
    e = scratch_for_current_device(&parts);
    if (e != hipSuccess) return e;
    const hipStream_t st = static_cast<hipStream_t>(stream);
    const psk::DecodeParams p =
        psk::make(*a, k_pool, v_pool, k_scale_pool, v_scale_pool, parts, splits, pages_per_split);
    e = psk::launch_decode<psk::kFmtFp8>(p, st);
    if (e != hipSuccess) return e;
    return psk::launch_reduce(p, st);
}
