/*
 * ps_oracle.c — CPU restatement of the PhaseShift qwen35 paged KV-cache path.
 *
 * TEST INFRASTRUCTURE ONLY. This file is the checker the GPU kernels are
 * compared against. Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it; the product library never links or calls it.
 *
 * Every function cites the reference file:line whose behaviour it restates
 * (paths relative to the reference repository root). Pinning of each function
 * (what independent evidence fixes its output) is listed in its comment:
 *   e4m3 encode/decode  pinned by the OCP E4M3 known-answer list
 *                       (tests/unit/test_ocp_e4m3_codec.cpp:54-103), by exhaustive
 *                       comparison with the reference's own e4m3.cpp built under
 *                       oracle/_ref, and by ROCm's hip_fp8.h host converter
 *                       (tests/golden fixtures).
 *   bf16 RNE            pinned exhaustively against the reference's
 *                       f32_to_bf16_rne (oracle/_ref) and against torch's cast.
 *   kv append           pinned by the closed form (byte copy / per-head absmax
 *                       scale) and by the ROCm-converter golden append fixture.
 *   attention           pinned by closed forms: single visible token => V,
 *                       equal keys => mean of V, permutation invariance of pages,
 *                       and against a float64 numpy softmax.
 *   gather / page copy  pinned by the byte-copy closed form (round trips).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define OR_INVALID_PAGE 0xFFFFFFFFu

/* ------------------------------------------------------------------------- */
/* bf16 <-> f32. Restates include/phaseshift/core/memory/types.h:11-21:       */
/* NaN -> 0x7FC0, +-inf kept, otherwise round-to-nearest-even on bit 16.      */
uint16_t or_f32_to_bf16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7F800000u) == 0x7F800000u) {
        if (u & 0x007FFFFFu) return 0x7FC0u;
        return (uint16_t)(u >> 16);
    }
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

float or_bf16_to_f32(uint16_t h) {
    uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

void or_f32_to_bf16_array(const float* in, uint16_t* out, uint64_t n) {
    for (uint64_t i = 0; i < n; ++i) out[i] = or_f32_to_bf16(in[i]);
}

/* ------------------------------------------------------------------------- */
/* OCP FP8 E4M3 (bias 7, no infinities, S.1111.111 = NaN, max 448).           */
/* Decode restates quantization/fpx/e4m3.cpp:45-56:                           */
/*   e == 0 : m * 2^-9 ; else (8 + m) * 2^(e-10) ; 0x7F/0xFF -> NaN.          */
float or_e4m3_decode(uint8_t x) {
    const uint32_t s = x >> 7, e = (x >> 3) & 15u, m = x & 7u;
    if ((x & 0x7Fu) == 0x7Fu) return NAN;
    const float mag = e == 0 ? ldexpf((float)m, -9) : ldexpf((float)(8u + m), (int)e - 10);
    return s ? -mag : mag;
}

/* Encode with the saturating (SATFINITE) semantics the reference uses on the
 * device: e4m3_detail.h:13-15 -> __hip_cvt_float_to_fp8(x, SATFINITE, E4M3),
 * which clamps finite x to [-448, 448] and rounds to nearest, ties to even.
 * Host twin: quantization/fpx/e4m3.cpp:58-99 (+-inf -> +-448, NaN -> 0x7F).
 * Computed here in closed form instead of the reference's grid search:
 *   |x| < 2^-6 : code = rint(|x| * 2^9)            (subnormal quantum 2^-9;
 *                                                    rint(...) == 8 is 2^-6)
 *   else       : E = floor(log2|x|), n = rint(|x| * 2^(3-E)) in [8,16],
 *                n == 16 -> E+1, n = 8; code = (E+7)<<3 | (n-8).
 * rintf rounds half to even in the default rounding mode; the multiplications
 * by powers of two are exact. */
uint8_t or_e4m3_encode(float x) {
    if (isnan(x)) return 0x7Fu;
    const uint8_t sign = signbit(x) ? 0x80u : 0x00u;
    float a = fabsf(x);
    if (a >= 448.0f) return (uint8_t)(sign | 0x7Eu);   /* includes +-inf */
    if (a < 0.015625f) {                                  /* 2^-6 */
        const uint32_t n = (uint32_t)rintf(a * 512.0f);  /* 0..8 */
        return (uint8_t)(sign | n);
    }
    int E;
    frexpf(a, &E);   /* a = f * 2^E, f in [0.5,1) => floor(log2 a) = E-1 */
    E -= 1;
    uint32_t n = (uint32_t)rintf(ldexpf(a, 3 - E));      /* 8..16 */
    if (n == 16u) { n = 8u; E += 1; }
    if (E > 8 || (E == 8 && n > 14u)) return (uint8_t)(sign | 0x7Eu);
    return (uint8_t)(sign | (uint8_t)(((uint32_t)(E + 7) << 3) | (n - 8u)));
}

/* Encodes the float whose bit patterns are start, start+1, ..., start+count-1. */
void or_e4m3_encode_range(uint32_t start_bits, uint32_t count, uint8_t* out) {
    for (uint32_t i = 0; i < count; ++i) {
        const uint32_t b = start_bits + i;
        float f;
        memcpy(&f, &b, 4);
        out[i] = or_e4m3_encode(f);
    }
}

void or_e4m3_encode_array(const float* in, uint8_t* out, uint64_t n) {
    for (uint64_t i = 0; i < n; ++i) out[i] = or_e4m3_encode(in[i]);
}

void or_e4m3_decode_array(const uint8_t* in, float* out, uint64_t n) {
    for (uint64_t i = 0; i < n; ++i) out[i] = or_e4m3_decode(in[i]);
}

/* ------------------------------------------------------------------------- */
/* Argument blocks: same field order and meaning as the reference launcher    */
/* structs (kv_append.h:12-41, paged_attention.h:42-78), host pointers.       */
typedef struct {
    const uint16_t* k_input;
    const uint16_t* v_input;
    uint32_t k_row_stride, v_row_stride;
    const uint32_t* row_sequence_slots;
    const uint32_t* row_positions;
    const uint32_t* block_tables;
    uint32_t block_table_stride, max_sequences, rows, layer, page_tokens, num_pages,
        num_attention_layers, kv_heads, head_dim, elems_per_token, elems_per_page,
        elems_per_layer;
} or_append_args;

/* Destination element base of (row); returns 0 when the optimized reference
 * kernel would skip the row (kv_append.hip:31-55): slot >= max_sequences,
 * logical block >= stride, or page >= num_pages. */
static int or_append_target(const or_append_args* a, uint32_t row, uint64_t* base,
                            uint32_t* page, uint32_t* off) {
    const uint32_t slot = a->row_sequence_slots[row];
    if (slot >= a->max_sequences) return 0;
    const uint32_t pos = a->row_positions[row];
    const uint32_t lb = pos / a->page_tokens;
    *off = pos % a->page_tokens;
    if (lb >= a->block_table_stride) return 0;
    *page = a->block_tables[(uint64_t)slot * a->block_table_stride + lb];
    if (*page >= a->num_pages) return 0;
    *base = (uint64_t)a->layer * a->elems_per_layer + (uint64_t)(*page) * a->elems_per_page +
            (uint64_t)(*off) * a->elems_per_token;
    return 1;
}

/* BF16 append: a byte copy of each head slice into its page slot
 * (kv_append.hip:21-103; correctness twin attention.inc:248-278). */
void or_kv_append_bf16(const or_append_args* a, uint16_t* k_pool, uint16_t* v_pool) {
    for (uint32_t row = 0; row < a->rows; ++row) {
        uint64_t base;
        uint32_t page, off;
        if (!or_append_target(a, row, &base, &page, &off)) continue;
        for (uint32_t h = 0; h < a->kv_heads; ++h) {
            const uint16_t* ks = a->k_input + (uint64_t)row * a->k_row_stride + (uint64_t)h * a->head_dim;
            const uint16_t* vs = a->v_input + (uint64_t)row * a->v_row_stride + (uint64_t)h * a->head_dim;
            const uint64_t dst = base + (uint64_t)h * a->head_dim;
            memcpy(k_pool + dst, ks, (size_t)a->head_dim * 2);
            memcpy(v_pool + dst, vs, (size_t)a->head_dim * 2);
        }
    }
}

/* FP8 append (kv_append.hip:148-272; correctness twin attention.inc:190-247):
 * per (row, head): amax = max |x| (fmaxf, so NaN inputs do not raise it);
 * scale = amax == 0 ? 1 : amax / 448 (fp32 division); code = e4m3(x / scale)
 * (fp32 division, then SATFINITE RNE encode); the scale goes to
 * ((layer*num_pages + page)*page_tokens + off)*kv_heads + h. */
void or_kv_append_fp8(const or_append_args* a, uint8_t* k_pool, uint8_t* v_pool,
                      float* k_scale_pool, float* v_scale_pool) {
    for (uint32_t row = 0; row < a->rows; ++row) {
        uint64_t base;
        uint32_t page, off;
        if (!or_append_target(a, row, &base, &page, &off)) continue;
        for (uint32_t h = 0; h < a->kv_heads; ++h) {
            const uint16_t* ks = a->k_input + (uint64_t)row * a->k_row_stride + (uint64_t)h * a->head_dim;
            const uint16_t* vs = a->v_input + (uint64_t)row * a->v_row_stride + (uint64_t)h * a->head_dim;
            float km = 0.0f, vm = 0.0f;
            for (uint32_t i = 0; i < a->head_dim; ++i) {
                km = fmaxf(km, fabsf(or_bf16_to_f32(ks[i])));
                vm = fmaxf(vm, fabsf(or_bf16_to_f32(vs[i])));
            }
            const float kscale = km == 0.0f ? 1.0f : km / 448.0f;
            const float vscale = vm == 0.0f ? 1.0f : vm / 448.0f;
            const uint64_t si =
                (((uint64_t)a->layer * a->num_pages + page) * a->page_tokens + off) * a->kv_heads + h;
            k_scale_pool[si] = kscale;
            v_scale_pool[si] = vscale;
            const uint64_t dst = base + (uint64_t)h * a->head_dim;
            for (uint32_t i = 0; i < a->head_dim; ++i) {
                k_pool[dst + i] = or_e4m3_encode(or_bf16_to_f32(ks[i]) / kscale);
                v_pool[dst + i] = or_e4m3_encode(or_bf16_to_f32(vs[i]) / vscale);
            }
        }
    }
}

/* ------------------------------------------------------------------------- */
/* Gather: token t of sequence i -> output row seq_token_offsets[i] + t, the  */
/* contiguous [kv_heads*head_dim] slice of the pool at (layer, page, slot).   */
/* Address math of resolve_paged_token (detail/attention_paged_common.h:22-50) */
/* Rows whose slot or page is invalid are left unwritten.                      */
typedef struct {
    const uint32_t* block_tables;
    const uint32_t* seq_slots;
    const uint32_t* seq_token_offsets;
    uint32_t block_table_stride, max_sequences, num_seqs, total_tokens, layer, page_tokens,
        num_pages, kv_heads, head_dim, elems_per_token, elems_per_page, elems_per_layer;
} or_gather_args;

void or_kv_gather(const or_gather_args* a, const uint8_t* pool, uint8_t* out, uint32_t elem_bytes) {
    const uint64_t row_bytes = (uint64_t)a->elems_per_token * elem_bytes;
    for (uint32_t s = 0; s < a->num_seqs; ++s) {
        const uint32_t slot = a->seq_slots[s];
        const uint32_t t0 = a->seq_token_offsets[s], t1 = a->seq_token_offsets[s + 1];
        if (slot >= a->max_sequences) continue;
        for (uint32_t t = 0; t < t1 - t0; ++t) {
            const uint32_t lb = t / a->page_tokens, off = t % a->page_tokens;
            if (lb >= a->block_table_stride) continue;
            const uint32_t page = a->block_tables[(uint64_t)slot * a->block_table_stride + lb];
            if (page >= a->num_pages) continue;
            const uint64_t e = (uint64_t)a->layer * a->elems_per_layer +
                               (uint64_t)page * a->elems_per_page + (uint64_t)off * a->elems_per_token;
            memcpy(out + (uint64_t)(t0 + t) * row_bytes, pool + e * elem_bytes, row_bytes);
        }
    }
}

/* ------------------------------------------------------------------------- */
/* Paged attention, fp32 two-pass softmax per (row, q_head).                 */
/* Restates kernels/correctness/detail/attention.inc:281-524 (bf16 :445-476,  */
/* fp8 :477-516) with the optimized kernels' skip rules                       */
/* (paged_decode.hip:79-97,123-128): slot >= max_sequences or                 */
/* pos+1 > stride*page_tokens -> row skipped; an invalid page on the way ->   */
/* that (row, q_head) output left unwritten.                                  */
/*   bf16: s = scale * sum_i q_i k_i                                          */
/*   fp8 : s = (sum_i q_i dec(k_i)) * k_scale * scale,                        */
/*         acc += (p * v_scale) * dec(v_i)                                    */
/*   out = acc / sum p,  p = exp(s - max s)                                   */
typedef struct {
    const uint16_t* q;
    void* output;
    uint32_t output_dtype; /* 0 bf16, 1 f32 */
    uint32_t q_row_stride, output_row_stride;
    const uint32_t* row_sequence_slots;
    const uint32_t* row_positions;
    const uint32_t* block_tables;
    uint32_t block_table_stride, max_sequences, rows, layer, page_tokens, num_pages,
        num_attention_layers, q_heads, kv_heads, head_dim, elems_per_token, elems_per_page,
        elems_per_layer;
    float scale;
} or_attn_args;

static void or_store(const or_attn_args* a, uint64_t idx, float v) {
    if (a->output_dtype == 1u)
        ((float*)a->output)[idx] = v;
    else
        ((uint16_t*)a->output)[idx] = or_f32_to_bf16(v);
}

/* kv_dtype: 0 bf16 pools (uint16), 1 fp8 pools (uint8) + fp32 scales. */
void or_paged_attention(const or_attn_args* a, uint32_t kv_dtype, const void* k_pool,
                        const void* v_pool, const float* k_scale_pool, const float* v_scale_pool) {
    const uint32_t D = a->head_dim;
    const uint32_t group = a->q_heads / a->kv_heads;
    float* qv = (float*)malloc(sizeof(float) * D);
    float* acc = (float*)malloc(sizeof(float) * D);
    float* kf = (float*)malloc(sizeof(float) * D);
    for (uint32_t row = 0; row < a->rows; ++row) {
        const uint32_t slot = a->row_sequence_slots[row];
        if (slot >= a->max_sequences) continue;
        const uint64_t visible = (uint64_t)a->row_positions[row] + 1u;
        if (visible > (uint64_t)a->block_table_stride * a->page_tokens) continue;
        const uint32_t* bt = a->block_tables + (uint64_t)slot * a->block_table_stride;
        for (uint32_t h = 0; h < a->q_heads; ++h) {
            const uint32_t kvh = h / group;
            const uint16_t* q = a->q + (uint64_t)row * a->q_row_stride + (uint64_t)h * D;
            for (uint32_t i = 0; i < D; ++i) qv[i] = or_bf16_to_f32(q[i]);
            float max_score = -3.402823466e+38f, sum = 0.0f;
            int bad = 0;
            for (int pass = 0; pass < 2 && !bad; ++pass) {
                sum = 0.0f;
                for (uint32_t i = 0; i < D; ++i) acc[i] = 0.0f;
                for (uint32_t p = 0; p < visible; ++p) {
                    const uint32_t lb = p / a->page_tokens, off = p % a->page_tokens;
                    const uint32_t page = bt[lb];
                    if (page >= a->num_pages) { bad = 1; break; }
                    const uint64_t kb = (uint64_t)a->layer * a->elems_per_layer +
                                        (uint64_t)page * a->elems_per_page +
                                        (uint64_t)off * a->elems_per_token + (uint64_t)kvh * D;
                    const uint64_t si =
                        (((uint64_t)a->layer * a->num_pages + page) * a->page_tokens + off) * a->kv_heads + kvh;
                    float sc = 0.0f, vw = 1.0f;
                    if (kv_dtype == 0u) {
                        const uint16_t* k = (const uint16_t*)k_pool + kb;
                        for (uint32_t i = 0; i < D; ++i) sc += qv[i] * or_bf16_to_f32(k[i]);
                        sc *= a->scale;
                    } else {
                        const uint8_t* k = (const uint8_t*)k_pool + kb;
                        for (uint32_t i = 0; i < D; ++i) sc += qv[i] * or_e4m3_decode(k[i]);
                        sc *= k_scale_pool[si] * a->scale;
                        vw = v_scale_pool[si];
                    }
                    if (pass == 0) {
                        if (sc > max_score) max_score = sc;
                    } else {
                        const float pv = expf(sc - max_score);
                        sum += pv;
                        if (kv_dtype == 0u) {
                            const uint16_t* v = (const uint16_t*)v_pool + kb;
                            for (uint32_t i = 0; i < D; ++i) acc[i] += pv * or_bf16_to_f32(v[i]);
                        } else {
                            const uint8_t* v = (const uint8_t*)v_pool + kb;
                            const float w = pv * vw;
                            for (uint32_t i = 0; i < D; ++i) acc[i] += w * or_e4m3_decode(v[i]);
                        }
                    }
                }
            }
            if (bad) continue;
            const uint64_t ob = (uint64_t)row * a->output_row_stride + (uint64_t)h * D;
            for (uint32_t i = 0; i < D; ++i) or_store(a, ob + i, acc[i] / sum);
        }
    }
    free(qv);
    free(acc);
    free(kf);
}

/* ------------------------------------------------------------------------- */
/* Split-K combine (paged_decode.hip:474-555): for each (row, kv_head, qh):   */
/* g = max_s m_s, W_s = exp(m_s - g), out = sum_s W_s A_s / sum_s W_s P_s,    */
/* over the splits s < n_used(row). Partials layout                           */
/* [row][kv_head][split][q_per_kv*(2+256)]: m at [qh], P at [q_per_kv+qh],    */
/* A at [2*q_per_kv + qh*256 + d].                                            */
void or_split_reduce(const or_attn_args* a, const float* partials, uint32_t splits,
                     const uint32_t* n_used) {
    const uint32_t qpk = a->q_heads / a->kv_heads;
    const uint64_t stride = (uint64_t)qpk * (2u + 256u);
    for (uint32_t row = 0; row < a->rows; ++row) {
        if (a->row_sequence_slots[row] >= a->max_sequences) continue;
        const uint32_t nu = n_used[row];
        for (uint32_t kvh = 0; kvh < a->kv_heads; ++kvh) {
            const float* base = partials + ((uint64_t)row * a->kv_heads + kvh) * splits * stride;
            for (uint32_t qh = 0; qh < qpk; ++qh) {
                float g = -3.402823466e+38f;
                for (uint32_t s = 0; s < nu; ++s) g = fmaxf(g, base[s * stride + qh]);
                float tot = 0.0f;
                for (uint32_t s = 0; s < nu; ++s)
                    tot += expf(base[s * stride + qh] - g) * base[s * stride + qpk + qh];
                for (uint32_t d = 0; d < a->head_dim; ++d) {
                    float acc = 0.0f;
                    for (uint32_t s = 0; s < nu; ++s)
                        acc += expf(base[s * stride + qh] - g) * base[s * stride + 2 * qpk + qh * 256 + d];
                    or_store(a, (uint64_t)row * a->output_row_stride +
                                    (uint64_t)(kvh * qpk + qh) * a->head_dim + d,
                             acc / tot);
                }
            }
        }
    }
}

/* ------------------------------------------------------------------------- */
/* Page copy (state/paged_kv_pool.cpp:338-542): per layer, the page body of K */
/* and V (page_tokens*kv_heads*head_dim elements) and, for FP8, the          */
/* page_tokens*kv_heads scales of K and V.                                   */
void or_copy_page(uint8_t* dst_k, uint8_t* dst_v, float* dst_ks, float* dst_vs,
                  const uint8_t* src_k, const uint8_t* src_v, const float* src_ks,
                  const float* src_vs, uint32_t dst_page, uint32_t src_page, uint32_t layers,
                  uint32_t dst_num_pages, uint32_t src_num_pages, uint32_t page_tokens,
                  uint32_t kv_heads, uint32_t head_dim, uint32_t elem_bytes) {
    const uint64_t page_elems = (uint64_t)page_tokens * kv_heads * head_dim;
    const uint64_t page_scales = (uint64_t)page_tokens * kv_heads;
    for (uint32_t l = 0; l < layers; ++l) {
        const uint64_t d = ((uint64_t)l * dst_num_pages + dst_page) * page_elems * elem_bytes;
        const uint64_t s = ((uint64_t)l * src_num_pages + src_page) * page_elems * elem_bytes;
        memcpy(dst_k + d, src_k + s, page_elems * elem_bytes);
        memcpy(dst_v + d, src_v + s, page_elems * elem_bytes);
        if (dst_ks) {
            const uint64_t ds = ((uint64_t)l * dst_num_pages + dst_page) * page_scales;
            const uint64_t ss = ((uint64_t)l * src_num_pages + src_page) * page_scales;
            memcpy(dst_ks + ds, src_ks + ss, page_scales * 4);
            memcpy(dst_vs + ds, src_vs + ss, page_scales * 4);
        }
    }
}

/* ------------------------------------------------------------------------- */
/* PSQ4_W32 / PSQ8_W32 KV (blocks of 32 values, one bf16 scale per block).   */
/* Codec: include/phaseshift/quantization/psq/psq_device.h:13-35 (cb10),     */
/*        psq4_kv.h:9-18 (bf16 round), psq8_kv.h:12-27 (e4m3 codes).         */
/* Append: kernels/optimized/kv_append.hip:276-643; host block encoders       */
/*        psq4_kv.h:20-79, psq8_kv.h:29-83.                                   */

/* bf16 round-to-nearest-even by bit arithmetic, as psq_bf16_round
 * (psq4_kv.h:9-18): no NaN special case. */
float or_psq_bf16_round(float v) {
    uint32_t u;
    memcpy(&u, &v, 4);
    u += 0x7FFFu + ((u >> 16) & 1u);
    u &= 0xFFFF0000u;
    float out;
    memcpy(&out, &u, 4);
    return out;
}

/* cb10 codebook: magnitudes {0,1,2,3,4,6,8,10}, bit 3 = sign. */
float or_cb10_decode(uint8_t code) {
    static const float mag[8] = {0.0f, 1.0f, 2.0f, 3.0f, 4.0f, 6.0f, 8.0f, 10.0f};
    const float m = mag[code & 7u];
    return (code & 8u) ? -m : m;
}

/* a = |x| * inv_scale, thresholds at the midpoints 0.5, 1.5, 2.5, 3.5, 5, 7, 9
 * (comparisons false for NaN -> index 7, as the reference's chain). */
uint8_t or_cb10_encode(float x, float inv_scale) {
    const float a = (x < 0.0f ? -x : x) * inv_scale;
    const uint8_t m = (a <= 0.5f) ? 0u : (a <= 1.5f) ? 1u : (a <= 2.5f) ? 2u : (a <= 3.5f) ? 3u
                    : (a <= 5.0f) ? 4u : (a <= 7.0f) ? 5u : (a <= 9.0f) ? 6u : 7u;
    return (uint8_t)(m | (x < 0.0f ? 8u : 0u));
}

static uint8_t or_psq_code(uint32_t fmt, float x, float s) {
    if (fmt == 4u) return or_cb10_encode(x, 1.0f / s);
    return or_e4m3_encode(x * (1.0f / s));
}

static float or_psq_value(uint32_t fmt, uint8_t c) {
    return fmt == 4u ? or_cb10_decode(c) : or_e4m3_decode(c);
}

/* Sum of v[0..31] in the order of the device kernels' 32-lane xor butterfly
 * (x += shfl_xor(x, o) for o = 16, 8, 4, 2, 1; every lane ends with the same
 * bits, kv_append.hip:293-299,433-439). */
static float or_butterfly32(const float* v) {
    float a[32], b[32];
    for (int i = 0; i < 32; ++i) a[i] = v[i];
    for (int o = 16; o >= 1; o >>= 1) {
        for (int i = 0; i < 32; ++i) b[i] = a[i] + a[i ^ o];
        for (int i = 0; i < 32; ++i) a[i] = b[i];
    }
    return a[0];
}

/* One block of 32 values -> scale (bf16 bits) and 32 codes (unpacked).
 * fmt 4: s0 = bf16(amax * 0.1f), cb10 codes of x * (1/s);
 * fmt 8: s0 = bf16(amax * (1/448)), e4m3 SATFINITE codes of x * (1/s).
 * lsq1: s1 = bf16(sum x q / sum q q) over the decoded codes q, then re-encode;
 * a non-positive s1 gives scale 0 and all-zero codes. The sums follow the
 * device kernels' butterfly order (device_order = 1) or the reference host
 * encoders' sequential loop (device_order = 0). The first scale follows
 * the device kernels (any positive amax; the host encoders also require
 * amax < FLT_MAX, psq4_kv.h:28). */
void or_psq_encode_block(const float* x, uint32_t fmt, uint32_t lsq1, uint32_t device_order,
                         uint16_t* scale_bits, uint8_t* codes) {
    float amax = 0.0f;   /* NaN never compares greater: dropped, as fmaxf on the device */
    for (int i = 0; i < 32; ++i) {
        const float ax = x[i] < 0.0f ? -x[i] : x[i];
        if (ax > amax) amax = ax;
    }
    float s = 0.0f;
    if (amax > 0.0f) s = or_psq_bf16_round(amax * (fmt == 4u ? 0.1f : (1.0f / 448.0f)));
    for (int i = 0; i < 32; ++i) codes[i] = (s > 0.0f) ? or_psq_code(fmt, x[i], s) : 0u;
    if (lsq1) {
        float num[32], den[32];
        for (int i = 0; i < 32; ++i) {
            const float q = or_psq_value(fmt, codes[i]);
            num[i] = x[i] * q;
            den[i] = q * q;
        }
        float sn = 0.0f, sd = 0.0f;
        if (device_order) {
            sn = or_butterfly32(num);
            sd = or_butterfly32(den);
        } else {
            for (int i = 0; i < 32; ++i) { sn += num[i]; sd += den[i]; }
        }
        const float sl = (sd > 0.0f) ? (sn / sd) : 0.0f;
        float s1 = or_psq_bf16_round(sl);
        if (!(s1 > 0.0f)) {
            s1 = 0.0f;
            for (int i = 0; i < 32; ++i) codes[i] = 0u;
        } else {
            for (int i = 0; i < 32; ++i) codes[i] = or_psq_code(fmt, x[i], s1);
        }
        s = s1;
    }
    uint32_t u;
    memcpy(&u, &s, 4);
    *scale_bits = (uint16_t)(u >> 16);
}

/* PSQ append: for each row and kv head, blocks b = 0..head_dim/32-1 of the
 * head slice; block index bi = (((layer*num_pages + page)*page_tokens + off)
 * *kv_heads + h)*blocks_per_head + b; codes at bi*16 (PSQ4, byte j = code[j] |
 * code[j+16] << 4) or bi*32 (PSQ8), bf16 scale at bi. Skip rules as the
 * other appends. */
void or_kv_append_psq(const or_append_args* a, uint32_t fmt, uint32_t lsq1, uint32_t device_order,
                      uint8_t* k_code, uint8_t* v_code, uint16_t* k_scale, uint16_t* v_scale) {
    const uint32_t bph = a->head_dim / 32u;
    const uint32_t cbytes = fmt == 4u ? 16u : 32u;
    for (uint32_t row = 0; row < a->rows; ++row) {
        uint64_t base;
        uint32_t page, off;
        if (!or_append_target(a, row, &base, &page, &off)) continue;
        for (uint32_t h = 0; h < a->kv_heads; ++h) {
            for (int t = 0; t < 2; ++t) {
                const uint16_t* src = (t == 0 ? a->k_input : a->v_input) +
                                      (uint64_t)row * (t == 0 ? a->k_row_stride : a->v_row_stride) +
                                      (uint64_t)h * a->head_dim;
                uint8_t* cp = t == 0 ? k_code : v_code;
                uint16_t* sp = t == 0 ? k_scale : v_scale;
                for (uint32_t b = 0; b < bph; ++b) {
                    const uint64_t bi =
                        ((((uint64_t)a->layer * a->num_pages + page) * a->page_tokens + off) * a->kv_heads + h) * bph + b;
                    float x[32];
                    for (int i = 0; i < 32; ++i) x[i] = or_bf16_to_f32(src[b * 32u + (uint32_t)i]);
                    uint8_t codes[32];
                    or_psq_encode_block(x, fmt, lsq1, device_order, sp + bi, codes);
                    if (fmt == 4u) {
                        for (int j = 0; j < 16; ++j)
                            cp[bi * cbytes + (uint32_t)j] = (uint8_t)((codes[j] & 0xFu) | ((codes[j + 16] & 0xFu) << 4));
                    } else {
                        for (int j = 0; j < 32; ++j) cp[bi * cbytes + (uint32_t)j] = codes[j];
                    }
                }
            }
        }
    }
}

/* Dequantized value d of (block index bi): scale * codebook(code), fp32
 * (paged_decode.hip:1206-1215 psq4_value, :1667-1673 psq8_value). */
static float or_psq_dequant(uint32_t fmt, const uint8_t* code_pool, const uint16_t* scale_pool,
                            uint64_t bi, uint32_t j) {
    const float s = or_bf16_to_f32(scale_pool[bi]);
    uint8_t c;
    if (fmt == 4u) {
        const uint8_t byte = code_pool[bi * 16u + (j & 15u)];
        c = (uint8_t)(j < 16u ? (byte & 0xFu) : (byte >> 4));
    } else {
        c = code_pool[bi * 32u + j];
    }
    return s * or_psq_value(fmt, c);
}

/* Paged attention over PSQ pools: as or_paged_attention with every K and V
 * element dequantized (scale * codebook value, fp32) before the fp32
 * two-pass softmax (paged_decode.hip:1219-1383, 1677-1847). */
void or_paged_attention_psq(const or_attn_args* a, uint32_t fmt, const uint8_t* k_code,
                            const uint8_t* v_code, const uint16_t* k_scale, const uint16_t* v_scale) {
    const uint32_t D = a->head_dim;
    const uint32_t bph = D / 32u;
    const uint32_t group = a->q_heads / a->kv_heads;
    float* qv = (float*)malloc(sizeof(float) * D);
    float* acc = (float*)malloc(sizeof(float) * D);
    for (uint32_t row = 0; row < a->rows; ++row) {
        const uint32_t slot = a->row_sequence_slots[row];
        if (slot >= a->max_sequences) continue;
        const uint64_t visible = (uint64_t)a->row_positions[row] + 1u;
        if (visible > (uint64_t)a->block_table_stride * a->page_tokens) continue;
        const uint32_t* bt = a->block_tables + (uint64_t)slot * a->block_table_stride;
        for (uint32_t h = 0; h < a->q_heads; ++h) {
            const uint32_t kvh = h / group;
            const uint16_t* q = a->q + (uint64_t)row * a->q_row_stride + (uint64_t)h * D;
            for (uint32_t i = 0; i < D; ++i) qv[i] = or_bf16_to_f32(q[i]);
            float max_score = -3.402823466e+38f, sum = 0.0f;
            int bad = 0;
            for (int pass = 0; pass < 2 && !bad; ++pass) {
                sum = 0.0f;
                for (uint32_t i = 0; i < D; ++i) acc[i] = 0.0f;
                for (uint32_t p = 0; p < visible; ++p) {
                    const uint32_t lb = p / a->page_tokens, off = p % a->page_tokens;
                    const uint32_t page = bt[lb];
                    if (page >= a->num_pages) { bad = 1; break; }
                    const uint64_t tb =
                        ((((uint64_t)a->layer * a->num_pages + page) * a->page_tokens + off) * a->kv_heads + kvh) * bph;
                    float sc = 0.0f;
                    for (uint32_t i = 0; i < D; ++i)
                        sc += qv[i] * or_psq_dequant(fmt, k_code, k_scale, tb + i / 32u, i % 32u);
                    sc *= a->scale;
                    if (pass == 0) {
                        if (sc > max_score) max_score = sc;
                    } else {
                        const float pv = expf(sc - max_score);
                        sum += pv;
                        for (uint32_t i = 0; i < D; ++i)
                            acc[i] += pv * or_psq_dequant(fmt, v_code, v_scale, tb + i / 32u, i % 32u);
                    }
                }
            }
            if (bad) continue;
            const uint64_t ob = (uint64_t)row * a->output_row_stride + (uint64_t)h * D;
            for (uint32_t i = 0; i < D; ++i) or_store(a, ob + i, acc[i] / sum);
        }
    }
    free(qv);
    free(acc);
}

void or_psq_bf16_round_array(const float* in, float* out, uint64_t n) {
    for (uint64_t i = 0; i < n; ++i) out[i] = or_psq_bf16_round(in[i]);
}

void or_cb10_encode_array(const float* x, const float* inv, uint8_t* out, uint64_t n) {
    for (uint64_t i = 0; i < n; ++i) out[i] = or_cb10_encode(x[i], inv[i]);
}
