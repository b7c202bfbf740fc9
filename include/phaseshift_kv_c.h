/*
 * phaseshift_kv_c.h — C-ABI of the MI355X (gfx950) paged KV-cache hot path.
 *
 * Plain C: pointers, sizes, POD structs. No HIP or torch types appear in any
 * signature: a stream is passed as `void*` (a hipStream_t, NULL = default
 * stream) and every entry point returns an `int` that holds a hipError_t value
 * (0 = hipSuccess, 1 = hipErrorInvalidValue, 801 = hipErrorNotSupported).
 *
 * The argument structs are byte-for-byte the reference's launcher structs, so
 * a caller that already fills those can pass their address here unchanged:
 *   psk_kv_append_args      == ps::kernel::KvAppendCommonArgs
 *       (reference include/phaseshift/models/qwen35/kernels/optimized/kv_append.h:12-41,
 *        96 B, asserted :52-72)
 *   psk_paged_attention_args == ps::kernel::PagedAttentionCommonArgs
 *       (reference include/phaseshift/models/qwen35/kernels/optimized/attention/
 *        paged_attention.h:42-78, 112 B, asserted :86-109)
 *
 * Semantics shared by every entry point (reference file:line in brackets):
 *  - KV pool element index: layer*elems_per_layer + page*elems_per_page
 *    + slot*elems_per_token + kv_head*head_dim + d
 *    [state/paged_kv_pool.cpp:64-69, kernels/optimized/kv_append.hip:47-49].
 *  - FP8 scale index: ((layer*num_pages + page)*page_tokens + slot)*kv_heads + kv_head
 *    [kv_append.hip:230-231].
 *  - Block table: uint32 [max_sequences][block_table_stride]; 0xFFFFFFFF = empty
 *    [state/paged_types.h:12]. A page id >= num_pages is invalid.
 *  - Row r attends to positions [0, row_positions[r]] inclusive
 *    [kernels/optimized/attention/paged_decode.hip:86-90].
 *  - Launchers allocate nothing, never synchronise, and only enqueue on `stream`.
 *  - Bad geometry / null pointers -> hipErrorInvalidValue; a shape no kernel
 *    here handles -> hipErrorNotSupported; else the launch status.
 *  - Data errors found on the device are silent: a row whose slot is invalid
 *    is skipped; a row that meets an invalid page leaves its output unwritten.
 */
#ifndef PHASESHIFT_KV_C_H
#define PHASESHIFT_KV_C_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PSK_INVALID_PAGE_ID 0xFFFFFFFFu

/* KVCacheDType values [state/kv_cache_types.h:9-14]. */
#define PSK_KV_BF16 0u
#define PSK_KV_FP8_E4M3 1u
#define PSK_KV_PSQ4_W32 3u
#define PSK_KV_PSQ8_W32 4u

/* PagedAttentionOutputDType values [paged_attention.h:37-40]. */
#define PSK_OUT_BF16 0u
#define PSK_OUT_F32 1u

/* Same layout as ps::kernel::KvAppendCommonArgs (96 B, align 8). */
typedef struct psk_kv_append_args {
    const void* k_input;               /* bf16 [rows][k_row_stride] */
    const void* v_input;               /* bf16 [rows][v_row_stride] */
    uint32_t k_row_stride;             /* elements */
    uint32_t v_row_stride;
    const uint32_t* row_sequence_slots;
    const uint32_t* row_positions;
    const uint32_t* block_tables;
    uint32_t block_table_stride;
    uint32_t max_sequences;
    uint32_t rows;
    uint32_t layer;
    uint32_t page_tokens;
    uint32_t num_pages;
    uint32_t num_attention_layers;
    uint32_t kv_heads;
    uint32_t head_dim;
    uint32_t elems_per_token;
    uint32_t elems_per_page;
    uint32_t elems_per_layer;
} psk_kv_append_args;

/* Same layout as ps::kernel::PagedAttentionCommonArgs (112 B, align 8). */
typedef struct psk_paged_attention_args {
    const void* q;                     /* bf16 [rows][q_row_stride] */
    void* output;                      /* bf16 or f32 [rows][output_row_stride] */
    uint8_t output_dtype;              /* PSK_OUT_BF16 / PSK_OUT_F32 */
    uint32_t q_row_stride;
    uint32_t output_row_stride;
    const uint32_t* row_sequence_slots;
    const uint32_t* row_positions;
    const uint32_t* block_tables;
    uint32_t block_table_stride;
    uint32_t max_sequences;
    uint32_t rows;
    uint32_t layer;
    uint32_t page_tokens;
    uint32_t num_pages;
    uint32_t num_attention_layers;
    uint32_t q_heads;
    uint32_t kv_heads;
    uint32_t head_dim;
    uint32_t elems_per_token;
    uint32_t elems_per_page;
    uint32_t elems_per_layer;
    float scale;
} psk_paged_attention_args;

/* Gather of paged KV back to contiguous [token][kv_heads*head_dim] rows.
 * Sequence i contributes tokens [0, seq_lengths) of slot seq_slots[i], written
 * to output rows [seq_token_offsets[i], seq_token_offsets[i+1]). No reference
 * counterpart: the reference reads pools back on the host in its tests
 * [tests/kernels/optimized/test_kv_append.hip:147-191]. */
typedef struct psk_kv_gather_args {
    const uint32_t* block_tables;
    const uint32_t* seq_slots;         /* [num_seqs] */
    const uint32_t* seq_token_offsets; /* [num_seqs + 1], exclusive prefix sum */
    uint32_t block_table_stride;
    uint32_t max_sequences;
    uint32_t num_seqs;
    uint32_t total_tokens;             /* == seq_token_offsets[num_seqs] */
    uint32_t layer;
    uint32_t page_tokens;
    uint32_t num_pages;
    uint32_t kv_heads;
    uint32_t head_dim;
    uint32_t elems_per_token;
    uint32_t elems_per_page;
    uint32_t elems_per_layer;
} psk_kv_gather_args;

/* One page-copy job: copy page `src_page` of the source pools to page
 * `dst_page` of the destination pools, every layer, K and V (and scales). */
typedef struct psk_page_copy_pair {
    uint32_t dst_page;
    uint32_t src_page;
} psk_page_copy_pair;

typedef struct psk_page_copy_args {
    void* dst_k;
    void* dst_v;
    float* dst_k_scale;                /* FP8: f32 scales; PSQ: bf16 block scales; BF16: NULL */
    float* dst_v_scale;
    const void* src_k;
    const void* src_v;
    const float* src_k_scale;
    const float* src_v_scale;
    const psk_page_copy_pair* pairs;   /* device array [num_pairs] */
    uint32_t num_pairs;
    uint32_t num_layers;
    uint32_t dst_num_pages;
    uint32_t src_num_pages;
    uint32_t page_tokens;
    uint32_t kv_heads;
    uint32_t head_dim;
    uint32_t kv_dtype;                 /* PSK_KV_* (PSQ: head_dim % 32 == 0) */
} psk_page_copy_args;

/* Row metadata descriptor: same layout as ps::runtime::DeviceRequestDescriptor
 * (64 B) [include/phaseshift/runtime/batch/device_batch_context.h:30-49]. */
typedef struct psk_request_descriptor {
    uint32_t slot;                     /* RequestHandle.slot */
    uint32_t generation;               /* RequestHandle.generation */
    uint32_t row_begin;
    uint32_t row_count;
    uint32_t prefix_length;
    uint32_t sequence_length;
    uint32_t output_index;
    uint8_t execution_class;           /* 0 DECODE 1 SPEC_VERIFY 2 PREFILL 3 SPEC_DRAFT */
    uint8_t compute_logits;
    uint8_t output_count;
    uint8_t reserved0;
    uint8_t sampling[32];              /* DeviceSamplingParams, opaque here */
} psk_request_descriptor;

/* ---- KV append [kernels/optimized/kv_append.h:78-97] ---------------------- */
int psk_kv_append_bf16(const psk_kv_append_args* a, void* k_pool, void* v_pool, void* stream);
int psk_kv_append_fp8_e4m3(const psk_kv_append_args* a, void* k_pool, void* v_pool,
                           float* k_scale_pool, float* v_scale_pool, void* stream);

/* KV append of a planned step with its row metadata formed in the same launch
 * [runtime/batch/device_batch_context.hip:69-90 followed by
 * kernels/optimized/kv_append.h:78-97]: row r of the append takes slot and
 * prefix_length + (r - row_begin) of the first request whose rows hold it, and
 * the launch writes them to a->row_sequence_slots / a->row_positions (which
 * must be writable device arrays of a->rows entries) for the step's later
 * launches; rows of no request are skipped and keep their metadata. Same
 * result as psk_prepare_row_metadata followed by psk_kv_append_*, in one
 * launch where the append takes its fast path (head_dim % 8 == 0, 16 B
 * aligned slices), else in those two launches. */
int psk_kv_append_bf16_from_requests(const psk_kv_append_args* a, const psk_request_descriptor* requests,
                                     uint32_t num_requests, void* k_pool, void* v_pool, void* stream);
int psk_kv_append_fp8_e4m3_from_requests(const psk_kv_append_args* a,
                                         const psk_request_descriptor* requests, uint32_t num_requests,
                                         void* k_pool, void* v_pool, float* k_scale_pool,
                                         float* v_scale_pool, void* stream);

/* ---- Paged attention [attention/paged_attention.h:140-201] ---------------- */
int psk_attention_paged_bf16(const psk_paged_attention_args* a, const void* k_pool,
                             const void* v_pool, void* stream);
int psk_attention_paged_fp8_e4m3(const psk_paged_attention_args* a, const void* k_pool,
                                 const void* v_pool, const float* k_scale_pool,
                                 const float* v_scale_pool, void* stream);
int psk_attention_paged_bf16_split(const psk_paged_attention_args* a, const void* k_pool,
                                   const void* v_pool, float* partials, uint32_t splits,
                                   void* stream);
int psk_attention_paged_bf16_split_reduce(const psk_paged_attention_args* a,
                                          const float* partials, uint32_t splits,
                                          void* stream);
/* Additive (no reference counterpart): FP8 split-K decode. pages_per_split = 0
 * splits each row's pages evenly into `splits` parts (the reference BF16 rule,
 * paged_decode.hip:315-320); > 0 gives every split that many pages, so rows of
 * different lengths use different numbers of splits. Partials layout is the
 * BF16 split layout: f32 [rows][kv_heads][splits][q_per_kv*(2+256)]. */
int psk_attention_paged_fp8_e4m3_split(const psk_paged_attention_args* a, const void* k_pool,
                                       const void* v_pool, const float* k_scale_pool,
                                       const float* v_scale_pool, float* partials,
                                       uint32_t splits, uint32_t pages_per_split,
                                       void* stream);
/* No counterpart in the reference. For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): psk_attention_paged_fp8_e4m3_split followed by
 * psk_attention_paged_split_reduce_ex in one call, with the split partials in a
 * library-owned static device array of PSK_NOALLOC_SCRATCH_BYTES per GPU
 * instead of a caller workspace. Calls no hipMalloc/hipFree. Returns
 * hipErrorInvalidValue when the call's partials
 * (psk_attention_split_partials_bytes(rows, q_heads, kv_heads, splits)) exceed
 * PSK_NOALLOC_SCRATCH_BYTES. Every call on one GPU shares that GPU's array:
 * calls that overlap on one GPU (other streams, other threads) race. */
#define PSK_NOALLOC_SCRATCH_BYTES (32ull << 20)
int psk_attention_paged_fp8_e4m3_split_noalloc(const psk_paged_attention_args* a,
                                               const void* k_pool, const void* v_pool,
                                               const float* k_scale_pool,
                                               const float* v_scale_pool, uint32_t splits,
                                               uint32_t pages_per_split, void* stream);
/* Additive: BF16 split with an explicit pages_per_split, and the matching reduce. */
int psk_attention_paged_bf16_split_ex(const psk_paged_attention_args* a, const void* k_pool,
                                      const void* v_pool, float* partials, uint32_t splits,
                                      uint32_t pages_per_split, void* stream);
int psk_attention_paged_split_reduce_ex(const psk_paged_attention_args* a,
                                        const float* partials, uint32_t splits,
                                        uint32_t pages_per_split, void* stream);
/* Bytes of partials the split launchers need. */
uint64_t psk_attention_split_partials_bytes(uint32_t rows, uint32_t q_heads,
                                            uint32_t kv_heads, uint32_t splits);

/* Multi-row tiles (speculative verify blocks, chunked prefill)
 * [attention/paged_prefill.hip:115-459,586-850]: rows [16*t, 16*t+16) of a
 * launch form one tile and belong to the sequence of the tile's first row
 * (the reference's own tile contract, paged_prefill.hip:152-164); rows of
 * another slot are left unwritten. Shapes outside the tile kernel (q_per_kv
 * > 8) run row by row on the decode launcher. */
int psk_attention_paged_prefill_bf16(const psk_paged_attention_args* a, const void* k_pool,
                                     const void* v_pool, void* stream);
int psk_attention_paged_prefill_fp8_e4m3(const psk_paged_attention_args* a,
                                         const void* k_pool, const void* v_pool,
                                         const float* k_scale_pool,
                                         const float* v_scale_pool, void* stream);

/* Additive: split-K over the same tiles; the combine is
 * psk_attention_paged_split_reduce_ex with the same splits / pages_per_split
 * (pages_per_split > 0 is required: the rows of a tile differ in length).
 * kv_dtype: PSK_KV_BF16, PSK_KV_FP8_E4M3 (f32 scale pools), PSK_KV_PSQ4_W32 or
 * PSK_KV_PSQ8_W32 (bf16 block-scale pools, 4 B aligned; head_dim 128 or 256). */
int psk_attention_paged_tile_split(const psk_paged_attention_args* a, uint32_t kv_dtype,
                                   const void* k_pool, const void* v_pool,
                                   const void* k_scale_pool, const void* v_scale_pool,
                                   float* partials, uint32_t splits, uint32_t pages_per_split,
                                   void* stream);

/* ---- PSQ4_W32 / PSQ8_W32 KV ----------------------------------------------
 * Pools [state/kv_cache_types.h:16-46]: blocks of 32 values of one (token,
 * kv head); block index bi = (((layer*num_pages + page)*page_tokens + off)
 * *kv_heads + head)*blocks_per_head + b, b = d/32. Codes at bi*16 (PSQ4:
 * byte j = cb10 code of value j | code of value j+16 << 4) or bi*32 (PSQ8:
 * E4M3 codes); one bf16 scale per block at bi. head_dim must equal
 * 32*blocks_per_head (else hipErrorNotSupported, as the reference). */
/* [kv_append.h:99-123]; estimator 0 = MaxAbs, 1 = Lsq1. */
int psk_kv_append_psq4(const psk_kv_append_args* a, uint8_t* k_code_pool, uint8_t* v_code_pool,
                       uint16_t* k_scale_pool, uint16_t* v_scale_pool,
                       uint32_t blocks_per_head, uint32_t estimator, void* stream);
int psk_kv_append_psq8(const psk_kv_append_args* a, uint8_t* k_code_pool, uint8_t* v_code_pool,
                       uint16_t* k_scale_pool, uint16_t* v_scale_pool,
                       uint32_t blocks_per_head, uint32_t estimator, void* stream);
/* [attention/paged_attention.h:203-225] */
int psk_attention_paged_psq4(const psk_paged_attention_args* a, const uint8_t* k_code_pool,
                             const uint8_t* v_code_pool, const uint16_t* k_scale_pool,
                             const uint16_t* v_scale_pool, uint32_t blocks_per_head,
                             void* stream);
int psk_attention_paged_psq8(const psk_paged_attention_args* a, const uint8_t* k_code_pool,
                             const uint8_t* v_code_pool, const uint16_t* k_scale_pool,
                             const uint16_t* v_scale_pool, uint32_t blocks_per_head,
                             void* stream);
/* [paged_attention.h:227-249]: every row attends to its own pos + 1 tokens. */
int psk_attention_paged_prefill_psq4(const psk_paged_attention_args* a,
                                     const uint8_t* k_code_pool, const uint8_t* v_code_pool,
                                     const uint16_t* k_scale_pool, const uint16_t* v_scale_pool,
                                     uint32_t blocks_per_head, void* stream);
int psk_attention_paged_prefill_psq8(const psk_paged_attention_args* a,
                                     const uint8_t* k_code_pool, const uint8_t* v_code_pool,
                                     const uint16_t* k_scale_pool, const uint16_t* v_scale_pool,
                                     uint32_t blocks_per_head, void* stream);
/* [paged_attention.h:251-283]: q_per_kv 4 or 6, splits 2/4/8/16, as the
 * reference; combine with psk_attention_paged_bf16_split_reduce. */
int psk_attention_paged_psq4_split(const psk_paged_attention_args* a, const uint8_t* k_code_pool,
                                   const uint8_t* v_code_pool, const uint16_t* k_scale_pool,
                                   const uint16_t* v_scale_pool, uint32_t blocks_per_head,
                                   float* partials, uint32_t splits, void* stream);
int psk_attention_paged_psq8_split(const psk_paged_attention_args* a, const uint8_t* k_code_pool,
                                   const uint8_t* v_code_pool, const uint16_t* k_scale_pool,
                                   const uint16_t* v_scale_pool, uint32_t blocks_per_head,
                                   float* partials, uint32_t splits, void* stream);
/* Additive: kv_dtype PSK_KV_PSQ4_W32 / PSK_KV_PSQ8_W32 forms; the split form
 * takes any q_per_kv <= 16, splits <= 1024 and pages_per_split as
 * psk_attention_paged_fp8_e4m3_split (combine: psk_attention_paged_split_reduce_ex). */
int psk_attention_paged_psq(const psk_paged_attention_args* a, uint32_t kv_dtype,
                            const uint8_t* k_code_pool, const uint8_t* v_code_pool,
                            const uint16_t* k_scale_pool, const uint16_t* v_scale_pool,
                            uint32_t blocks_per_head, void* stream);
int psk_attention_paged_psq_split_ex(const psk_paged_attention_args* a, uint32_t kv_dtype,
                                     const uint8_t* k_code_pool, const uint8_t* v_code_pool,
                                     const uint16_t* k_scale_pool, const uint16_t* v_scale_pool,
                                     uint32_t blocks_per_head, float* partials,
                                     uint32_t splits, uint32_t pages_per_split, void* stream);

/* ---- Page-level operations ------------------------------------------------- */
/* elem_bytes: 2 (bf16 pool), 1 (fp8 codes) or 4 (fp32 scale pool, with
 * elems_per_token = kv_heads, elems_per_page = page_tokens*kv_heads). */
int psk_kv_gather(const psk_kv_gather_args* a, const void* pool, void* out,
                  uint32_t elem_bytes, void* stream);
/* Batched prefix-cache / copy-on-write page copy
 * [state/paged_kv_pool.cpp:338-542] in one launch. */
int psk_kv_copy_pages(const psk_page_copy_args* a, void* stream);
/* Fill `count` uint32 words at `dst` with `value` (block-table truncation
 * [state/sequence_slot_pool.cpp:192-232]) without hipMemsetAsync. */
int psk_fill_u32(uint32_t* dst, uint32_t value, uint64_t count, void* stream);
/* Row metadata [runtime/batch/device_batch_context.hip:69-90]: for request i,
 * rows [row_begin, row_begin+row_count) get slot and prefix_length + t. */
int psk_prepare_row_metadata(const psk_request_descriptor* requests, uint32_t num_requests,
                             uint32_t actual_rows, uint32_t* row_sequence_slots,
                             uint32_t* row_positions, void* stream);

/* ---- Host KV state (opaque handles) ----------------------------------------
 * Status codes of these entry points: 0 ok, else one of PSK_ERR_* (message in
 * psk_last_error_message()). Reference: state/paged_kv_pool.cpp,
 * state/sequence_slot_pool.cpp, state/paged_sequence_state.cpp. */
#define PSK_ERR_INVALID_ARGUMENT 1001
#define PSK_ERR_OUT_OF_RANGE 1002
#define PSK_ERR_INVALID_STATE 1003
#define PSK_ERR_INSUFFICIENT_MEMORY 1004
#define PSK_ERR_HIP 1005

typedef struct psk_kv_pool psk_kv_pool;
typedef struct psk_slot_pool psk_slot_pool;
typedef struct psk_sequence psk_sequence;

typedef struct psk_pool_info_t {
    void* k_pool;
    void* v_pool;
    float* k_scale_pool;
    float* v_scale_pool;
    uint32_t num_pages;
    uint32_t page_tokens;
    uint32_t num_layers;
    uint32_t kv_heads;
    uint32_t head_dim;
    uint32_t kv_dtype;
    uint32_t free_pages;
    uint32_t used_pages;
    uint64_t reserved_bytes;
} psk_pool_info_t;

typedef struct psk_sequence_info_t {
    uint32_t slot;
    uint32_t generation;
    uint32_t position;
    uint32_t max_seq_len;
    uint32_t num_blocks;
    uint32_t poisoned;
} psk_sequence_info_t;

const char* psk_last_error_message(void);
/* PagedKVPool::create (paged_kv_pool.cpp:27-194); kv_dtype PSK_KV_*. */
int psk_pool_create(psk_kv_pool** out, uint32_t num_pages, uint32_t page_tokens,
                    uint32_t num_layers, uint32_t kv_heads, uint32_t head_dim, uint32_t kv_dtype);
void psk_pool_destroy(psk_kv_pool* pool);
int psk_pool_info(const psk_kv_pool* pool, psk_pool_info_t* out);
int psk_pool_allocate(psk_kv_pool* pool, uint32_t* page);
int psk_pool_release(psk_kv_pool* pool, uint32_t page);
/* copy_page_from for n (dst, src) pairs, host arrays (paged_kv_pool.cpp:338-542). */
int psk_pool_copy_pages(psk_kv_pool* dst, const psk_kv_pool* src, const uint32_t* dst_pages,
                        const uint32_t* src_pages, uint32_t n, void* stream);
/* SequenceSlotPool (sequence_slot_pool.cpp): device tables [max_sequences][max_blocks]. */
int psk_slot_pool_create(psk_slot_pool** out, uint32_t max_sequences, uint32_t max_blocks,
                         void* stream);
void psk_slot_pool_destroy(psk_slot_pool* slots);
uint32_t* psk_slot_pool_block_tables(const psk_slot_pool* slots);
/* PagedSequenceState and its reserve / rollback / commit
 * (paged_sequence_state.cpp:111-271). */
int psk_sequence_create(psk_sequence** out, psk_slot_pool* slots, psk_kv_pool* pool,
                        uint32_t max_seq_len, void* stream);
int psk_sequence_release(psk_sequence* seq, void* stream);
int psk_sequence_reserve(psk_sequence* seq, uint32_t token_count, void* stream);
int psk_sequence_rollback(psk_sequence* seq, uint32_t old_block_count, void* stream);
int psk_sequence_commit(psk_sequence* seq, uint32_t tokens);
int psk_sequence_info(const psk_sequence* seq, psk_sequence_info_t* out);
uint32_t psk_sequence_block_table(const psk_sequence* seq, uint32_t* out, uint32_t cap);

/* ---- GDN recurrent-state pool [state/gdn_state_pool.h:41-200] ------------
 * Per slot: bf16 conv history [states][conv_history][conv_history_stride]
 * and f32 recurrent state [states][v_heads][head_k][head_v]. The prefix
 * cache copies a sequence's slot (slot id = its sequence slot). */
typedef struct psk_gdn_pool psk_gdn_pool;
typedef struct psk_gdn_layout {
    uint32_t num_gdn_states;
    uint32_t conv_dim;
    uint32_t conv_dim_padded;
    uint32_t conv_history;
    uint32_t conv_history_stride;
    uint32_t num_v_heads;
    uint32_t head_k;
    uint32_t head_v;
} psk_gdn_layout;
typedef struct psk_gdn_pool_info_t {
    void* conv_base;
    void* recurrent_base;
    uint64_t conv_slot_bytes;
    uint64_t recurrent_slot_bytes;
    uint64_t reserved_bytes;
    uint32_t max_sequences;
    uint32_t used_slots;
} psk_gdn_pool_info_t;
/* GdnStatePoolLayout::make [gdn_state_pool.h:52-66]: conv_dim padded to 8. */
int psk_gdn_layout_make(uint32_t gdn_layers, uint32_t conv_dim, uint32_t conv_history,
                        uint32_t num_v_heads, uint32_t head_k, uint32_t head_v,
                        psk_gdn_layout* out);
int psk_gdn_pool_create(psk_gdn_pool** out, uint32_t max_sequences, const psk_gdn_layout* layout);
void psk_gdn_pool_destroy(psk_gdn_pool* pool);
int psk_gdn_pool_info(const psk_gdn_pool* pool, psk_gdn_pool_info_t* out);
int psk_gdn_pool_initialize(psk_gdn_pool* pool, uint32_t slot, void* stream);
int psk_gdn_pool_reset(psk_gdn_pool* pool, uint32_t slot, void* stream);
int psk_gdn_pool_release(psk_gdn_pool* pool, uint32_t slot);
int psk_gdn_pool_copy_slot(psk_gdn_pool* dst, uint32_t dst_slot, const psk_gdn_pool* src,
                           uint32_t src_slot, void* stream);

/* ---- Prefix cache [runtime/prefix_cache.h:24-150, prefix_cache.cpp:84-486] -
 * LRU checkpoints of (KV pages, GDN slot, optional DFlash ring) in cache-owned
 * pools. save/restore move all of a checkpoint's bytes in one batched copy
 * launch. Checkpoints are named by a stable id (0 = none). */
typedef struct psk_prefix_cache psk_prefix_cache;
/* The drafter's DFlash2 context ring [dflash2/context_state.h:15-27]. */
typedef struct psk_dflash_context {
    void* k_ring;
    void* v_ring;
    uint64_t ring_bytes;
    uint32_t length;
    uint32_t next_position;
} psk_dflash_context;
typedef struct psk_prefix_checkpoint_info {
    uint64_t id;                       /* 0: no checkpoint */
    uint64_t last_used;
    uint32_t position;
    uint32_t num_pages;
    uint32_t cache_state_slot;
    uint32_t dflash;
} psk_prefix_checkpoint_info;
typedef struct psk_prefix_cache_stats_t {
    uint64_t lookups, hits, misses, inserts, duplicate_hits, evictions, skipped_too_large;
    uint64_t restored_tokens, saved_tokens, save_d2d_bytes, restore_d2d_bytes, copy_launches;
    uint64_t cache_kv_bytes, cache_gdn_bytes, dflash_ring_bytes;
    uint32_t size, cache_pages, cache_free_pages, cache_free_slots, max_entries, capacity_tokens;
} psk_prefix_cache_stats_t;
int psk_prefix_cache_create(psk_prefix_cache** out, const psk_kv_pool* active_kv,
                            const psk_gdn_pool* active_gdn, uint32_t capacity_tokens,
                            uint32_t max_entries, uint32_t min_prefix_tokens);
void psk_prefix_cache_destroy(psk_prefix_cache* cache);
int psk_prefix_cache_enable_dflash_ring(psk_prefix_cache* cache, uint64_t ring_bytes);
/* Longest cached prefix of tokens[0..n) (strictly shorter if asked); out->id
 * is 0 on a miss. */
int psk_prefix_cache_find_longest(psk_prefix_cache* cache, const int32_t* tokens, uint32_t n,
                                  uint32_t strictly_shorter, psk_prefix_checkpoint_info* out);
int psk_prefix_cache_save(psk_prefix_cache* cache, const psk_sequence* seq,
                          const psk_gdn_pool* gdn, const psk_kv_pool* kv, const int32_t* tokens,
                          uint32_t n, uint32_t prompt_boundary, const psk_dflash_context* dflash,
                          void* stream);
int psk_prefix_cache_restore(psk_prefix_cache* cache, psk_sequence* seq, psk_gdn_pool* gdn,
                             psk_kv_pool* kv, uint64_t checkpoint_id, psk_dflash_context* dflash,
                             void* stream);
int psk_prefix_cache_clear(psk_prefix_cache* cache);
int psk_prefix_cache_stats(const psk_prefix_cache* cache, psk_prefix_cache_stats_t* out);

/* ---- Step planner (paged_attention_dispatch.hip:437-894) -------------------
 * Plans and launches the PAGED_ATTENTION binding of one mixed step. Requests
 * must partition [0, rows) in order (else the whole step is one decode
 * region). PREFILL requests of >= 128 rows (the reference rule) and
 * SPEC_VERIFY requests of >= 8 rows go to one tile launch per class; runs of
 * the other requests go to decode launches. A launch uses split-K when its
 * max_visible_tokens >= 2048 and the partials fit partial_bytes; splits are
 * sized to ~2048 workgroups of >= 16 pages. stream == (void*)~0 plans without
 * launching. */
#define PSK_MAX_PLANNED 16
typedef struct psk_step_request {
    uint32_t row_begin;
    uint32_t row_count;
    uint8_t execution_class;           /* 0 DECODE 1 SPEC_VERIFY 2 PREFILL 3 SPEC_DRAFT */
    uint8_t reserved[3];
    uint32_t max_visible;              /* largest visible length of its rows (prefix + count);
                                          0: unknown, the step's max_visible_tokens is used */
} psk_step_request;

typedef struct psk_planned_kernel {
    uint32_t kind;                     /* 0 decode (split when splits > 1), 1 tile */
    uint32_t row_begin;
    uint32_t rows;
    uint32_t splits;
    uint32_t pages_per_split;
    uint32_t side;                     /* 0: on the caller's stream; 1 / 2: on side lane 1
                                          (decode launches) / 2 (the other tile launches),
                                          concurrent with the step's largest tile launch and
                                          with each other (forked and joined by events on the
                                          caller's stream) */
} psk_planned_kernel;

typedef struct psk_step_plan_t {
    uint32_t count;
    psk_planned_kernel kernels[PSK_MAX_PLANNED];
} psk_step_plan_t;

int psk_paged_attention_step(const psk_paged_attention_args* common, uint32_t kv_dtype,
                             const void* k_pool, const void* v_pool, const void* k_scale_pool,
                             const void* v_scale_pool, const psk_step_request* requests,
                             uint32_t num_requests, uint32_t max_visible_tokens, float* partials,
                             uint64_t partial_bytes, psk_step_plan_t* plan_out, void* stream);

/* HIP-graph capture of planned steps (additive; the reference keys its batch
 * graphs with a plan signature, paged_attention_dispatch.hip:896-908, and
 * captures warm buckets, executor.hip:990-1075). The signature covers the
 * plan's launches (kinds, regions, splits, tile and combine tables), the
 * KV dtype, the argument bytes and the pool / scale / workspace pointers; the
 * contents of those buffers may change between replays. A key's first step
 * launches eagerly, the second captures and launches the graph, later ones
 * replay it. *how: 0 eager, 1 captured, 2 replayed. Least recently used
 * graphs beyond `capacity` keys are destroyed. Not thread-safe; one cache per
 * stream. */
typedef struct psk_step_graph_cache psk_step_graph_cache;
typedef struct psk_step_graph_stats_t {
    uint64_t eager;
    uint64_t captures;
    uint64_t replays;
    uint64_t evictions;
    uint32_t entries;
    uint32_t graphs;
} psk_step_graph_stats_t;
int psk_step_graph_cache_create(psk_step_graph_cache** out, uint32_t capacity);
void psk_step_graph_cache_destroy(psk_step_graph_cache* cache);
int psk_step_graph_cache_stats(const psk_step_graph_cache* cache, psk_step_graph_stats_t* out);
int psk_paged_attention_step_graphed(psk_step_graph_cache* cache,
                                     const psk_paged_attention_args* common, uint32_t kv_dtype,
                                     const void* k_pool, const void* v_pool,
                                     const void* k_scale_pool, const void* v_scale_pool,
                                     const psk_step_request* requests, uint32_t num_requests,
                                     uint32_t max_visible_tokens, float* partials,
                                     uint64_t partial_bytes, psk_step_plan_t* plan_out,
                                     void* stream, uint32_t* how);
/* 64-bit FNV-1a of the plan signature (0 if the step does not plan). */
uint64_t psk_paged_attention_plan_signature(const psk_paged_attention_args* common,
                                            uint32_t kv_dtype, const void* k_pool,
                                            const void* v_pool, const void* k_scale_pool,
                                            const void* v_scale_pool,
                                            const psk_step_request* requests,
                                            uint32_t num_requests, uint32_t max_visible_tokens,
                                            float* partials, uint64_t partial_bytes);

/* Split-K sizing the planner uses for a decode launch (additive, no reference
 * counterpart): the split count and pages per split that finish first under
 * the decode kernel's XCD-aware dispatch on this device. row_visible is an
 * optional host array of the rows' visible lengths (NULL: every row at
 * max_visible_tokens); the partials must fit partial_bytes. *splits == 1:
 * launch unsplit. Uses a->rows, q_heads, kv_heads, head_dim, page_tokens. */
int psk_choose_decode_split(const psk_paged_attention_args* a, uint32_t kv_dtype,
                            const uint32_t* row_visible, uint32_t max_visible_tokens,
                            uint64_t partial_bytes, uint32_t* splits, uint32_t* pages_per_split);

/* ---- Self-test hooks (diagnostics, no reference counterpart) --------------- */
/* Runs the device E4M3 encoder of the append kernel on the floats whose bit
 * patterns are start_bits .. start_bits+count-1 (count % 4 == 0); word i of
 * out_words holds the codes of inputs 4i..4i+3 in bytes 0..3. */
int psk_selftest_e4m3_encode_range(uint32_t start_bits, uint32_t count, uint32_t* out_words,
                                   void* stream);
/* Decodes all 256 E4M3 codes with the device decoder of the attention kernels. */
int psk_selftest_e4m3_decode_all(float* out256, void* stream);

/* ---- Library --------------------------------------------------------------- */
const char* psk_version(void);
/* gfx target the library was built for ("gfx950"). */
const char* psk_build_arch(void);
/* Name of the last error an entry point returned on this thread. */
const char* psk_error_string(int err);

#ifdef __cplusplus
}  /* extern "C" */
#endif

#endif /* PHASESHIFT_KV_C_H */
