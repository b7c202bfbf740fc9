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
