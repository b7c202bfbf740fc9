// Page-level kernels of the paged KV path (gfx950, wave64):
//   gather of paged KV to contiguous rows, batched prefix-cache page copy,
//   u32 fill (block-table truncation), row metadata from request descriptors,
//   the generic any-shape attention kernel, and the E4M3 encoder self-test.
#include "device_common.h"
#include "page_ops.h"

#include <phaseshift_kv/paged_attention.h>

#include <cfloat>

namespace psk {
namespace {

// ----------------------------------------------------------------- gather
// One wave per output token row; the row is elems_per_token*elem_bytes
// contiguous bytes in the pool (slot layout [kv_heads][head_dim]), copied with
// 16 B accesses when aligned.
__global__ __launch_bounds__(256) void gather_kernel(const psk_kv_gather_args a, const uint8_t* pool,
                                                     uint8_t* out, uint32_t eb, uint32_t vec16) {
    const uint64_t wave = ((uint64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    const uint32_t lane = threadIdx.x & 63u;
    if (wave >= a.total_tokens) return;
    const uint32_t t = (uint32_t)wave;
    // sequence of token t: last i with seq_token_offsets[i] <= t
    uint32_t lo = 0, hi = a.num_seqs;
    while (hi - lo > 1u) {
        const uint32_t mid = (lo + hi) >> 1;
        if (a.seq_token_offsets[mid] <= t) lo = mid; else hi = mid;
    }
    const uint32_t slot = a.seq_slots[lo];
    if (slot >= a.max_sequences) return;
    const uint32_t pos = t - a.seq_token_offsets[lo];
    const uint32_t lb = pos / a.page_tokens;
    if (lb >= a.block_table_stride) return;
    const uint32_t page = a.block_tables[(uint64_t)slot * a.block_table_stride + lb];
    if (page >= a.num_pages) return;
    const uint64_t src_e = (uint64_t)a.layer * a.elems_per_layer + (uint64_t)page * a.elems_per_page +
                           (uint64_t)(pos % a.page_tokens) * a.elems_per_token;
    const uint64_t bytes = (uint64_t)a.elems_per_token * eb;
    const uint8_t* s = pool + src_e * eb;
    uint8_t* d = out + (uint64_t)t * bytes;
    if (vec16) {
        for (uint64_t o = (uint64_t)lane * 16u; o < bytes; o += 64u * 16u)
            *reinterpret_cast<u32x4*>(d + o) = *reinterpret_cast<const u32x4*>(s + o);
    } else {
        for (uint64_t o = lane; o < bytes; o += 64u) d[o] = s[o];
    }
}

// ------------------------------------------------------------- page copy
// Bytes of one page of one layer: the K (V) body and its scale rows.
//   BF16  P*H*D*2, no scales        FP8   P*H*D, P*H f32 scales
//   PSQ4  P*H*D/2, P*H*D/32 bf16    PSQ8  P*H*D, P*H*D/32 bf16
// (PSQ blocks of a page are contiguous: block index ((layer*num_pages +
// page)*P + off)*H*D/32 + ..., kv_append.hip:368-372.)
__host__ __device__ inline void page_bytes(const psk_page_copy_args& a, uint64_t& body,
                                           uint64_t& scales) {
    const uint64_t th = (uint64_t)a.page_tokens * a.kv_heads;   // (token, head) slices
    switch (a.kv_dtype) {
        case PSK_KV_BF16: body = th * a.head_dim * 2u; scales = 0; break;
        case PSK_KV_FP8_E4M3: body = th * a.head_dim; scales = th * 4u; break;
        case PSK_KV_PSQ4_W32: body = th * a.head_dim / 2u; scales = th * (a.head_dim / 32u) * 2u; break;
        default: body = th * a.head_dim; scales = th * (a.head_dim / 32u) * 2u; break;
    }
}

// grid.x = page pairs * layers * 2 tensors (K, V); every block copies one
// page body and then the page's scale rows of that tensor, with 16 B
// accesses. Copies `bytes` (a multiple of 16) with the workgroup's 256
// threads: each thread issues the loads of a 16 KB round (4 x 16 B per
// thread) before its stores, so several loads are in flight per thread. The
// bytes are moved once: non-temporal loads and stores.
__device__ __forceinline__ void copy16_block(uint8_t* d, const uint8_t* s, uint64_t bytes) {
    constexpr int U = 4;
    constexpr uint64_t kRound = 256u * 16u * U;
    for (uint64_t o0 = (uint64_t)threadIdx.x * 16u; o0 < bytes; o0 += kRound) {
        u32x4 v[U];
#pragma unroll
        for (int j = 0; j < U; ++j) {
            const uint64_t o = o0 + (uint64_t)j * 256u * 16u;
            if (o < bytes) v[j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(s + o));
        }
#pragma unroll
        for (int j = 0; j < U; ++j) {
            const uint64_t o = o0 + (uint64_t)j * 256u * 16u;
            if (o < bytes) __builtin_nontemporal_store(v[j], reinterpret_cast<u32x4*>(d + o));
        }
    }
}

// vec16: d and s 16 B aligned: 16 B accesses over the whole 16 B units,
// bytes for a tail below 16 B; otherwise bytes throughout.
__device__ __forceinline__ void copy_bytes(uint8_t* d, const uint8_t* s, uint64_t bytes, uint32_t vec16) {
    const uint64_t m = vec16 ? bytes & ~(uint64_t)15u : 0u;
    if (m != 0u) copy16_block(d, s, m);
    for (uint64_t o = m + threadIdx.x; o < bytes; o += 256u) d[o] = s[o];
}

// blocks per (page pair, layer): K and V, each body + scale rows
constexpr uint32_t kCopyTensors = 2u;

// tensor 0: K body + K scale rows, 1: V body + V scale rows. Page p of a
// pool starts at p x (body or scale row bytes): 16 B accesses need those
// sizes to be multiples of 16 as well as 16 B aligned pools (vec16).
__device__ __forceinline__ void copy_one(const psk_page_copy_args& a, uint32_t vec16,
                                         uint32_t dst_page, uint32_t src_page, uint32_t layer,
                                         uint32_t tensor) {
    if (dst_page >= a.dst_num_pages || src_page >= a.src_num_pages) return;
    uint64_t body, scales;
    page_bytes(a, body, scales);
    const uint64_t sp = (uint64_t)layer * a.src_num_pages + src_page;
    const uint64_t dp = (uint64_t)layer * a.dst_num_pages + dst_page;
    copy_bytes(static_cast<uint8_t*>(tensor == 0u ? a.dst_k : a.dst_v) + dp * body,
               static_cast<const uint8_t*>(tensor == 0u ? a.src_k : a.src_v) + sp * body, body,
               vec16 && body % 16u == 0u);
    if (scales == 0u) return;
    copy_bytes(reinterpret_cast<uint8_t*>(tensor == 0u ? a.dst_k_scale : a.dst_v_scale) + dp * scales,
               reinterpret_cast<const uint8_t*>(tensor == 0u ? a.src_k_scale : a.src_v_scale) + sp * scales,
               scales, vec16 && scales % 16u == 0u);
}

__global__ __launch_bounds__(256) void copy_pages_kernel(const psk_page_copy_args a,
                                                         uint32_t vec16) {
    const uint32_t rest = blockIdx.x / kCopyTensors;
    const uint32_t pair = rest / a.num_layers;
    if (pair >= a.num_pairs) return;
    copy_one(a, vec16, a.pairs[pair].dst_page, a.pairs[pair].src_page, rest % a.num_layers,
             blockIdx.x % kCopyTensors);
}

// Pairs passed by value in the kernel arguments (host-driven copies: no
// device staging buffer and no ordering hazard on a reused host buffer).
struct InlinePairs {
    psk_page_copy_pair p[kInlinePairs];
};


// ------------------------------------------------------------ copy plan
// One launch for a whole prefix-cache save or restore: up to
// kMaxCopySegments contiguous segments (GDN state slots, DFlash rings), each
// cut into kSegmentBlockBytes per workgroup (blocks [0, seg_blocks)), then
// the KV page pairs above. The segment blocks go first: a launch's tail is
// then the short page blocks.
constexpr uint64_t kSegmentBlockBytes = 16u * 1024u;
struct InlineSegments {
    CopySegment s[kMaxCopySegments];
    uint64_t first_block[kMaxCopySegments + 1];
};

// Pairs inline (kernel arguments) or, when a.pairs is set, from device memory.
__global__ __launch_bounds__(256) void copy_plan_kernel(const psk_page_copy_args a,
                                                        const InlinePairs pairs,
                                                        const InlineSegments segs, uint32_t nseg,
                                                        uint32_t vec16, uint32_t seg_blocks) {
    if (blockIdx.x >= seg_blocks) {
        const uint32_t rest = (blockIdx.x - seg_blocks) / kCopyTensors;
        const uint32_t pair = rest / a.num_layers;
        if (pair >= a.num_pairs) return;
        const psk_page_copy_pair pp = a.pairs != nullptr ? a.pairs[pair] : pairs.p[pair];
        copy_one(a, vec16, pp.dst_page, pp.src_page, rest % a.num_layers,
                 (blockIdx.x - seg_blocks) % kCopyTensors);
        return;
    }
    const uint64_t b = blockIdx.x;
    uint32_t i = 0;
    while (i + 1u < nseg && segs.first_block[i + 1] <= b) ++i;
    if (i >= nseg || b >= segs.first_block[nseg]) return;
    const CopySegment sg = segs.s[i];
    const uint64_t off = (b - segs.first_block[i]) * kSegmentBlockBytes;
    const uint64_t n = min(kSegmentBlockBytes, sg.bytes - off);
    const uint8_t* src = static_cast<const uint8_t*>(sg.src) + off;
    uint8_t* dst = static_cast<uint8_t*>(sg.dst) + off;
    const bool al = ((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst)) & 15u) == 0u;
    copy_bytes(dst, src, n, al ? 1u : 0u);
}

// ------------------------------------------------------------------ fill
__global__ __launch_bounds__(256) void fill_u32_kernel(uint32_t* dst, uint32_t value, uint64_t n) {
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (uint64_t)gridDim.x * blockDim.x)
        dst[i] = value;
}

// --------------------------------------------------------- row metadata
// Restates prepare_batch_descriptor_kernel (device_batch_context.hip:69-90)
// for the two row arrays of the KV path; one thread per (request, row).
__global__ __launch_bounds__(256) void row_metadata_kernel(const psk_request_descriptor* req,
                                                           uint32_t num_requests, uint32_t actual_rows,
                                                           uint32_t* slots, uint32_t* positions) {
    const uint32_t r = blockIdx.y;
    if (r >= num_requests) return;
    const psk_request_descriptor d = req[r];
    for (uint32_t t = blockIdx.x * blockDim.x + threadIdx.x; t < d.row_count;
         t += gridDim.x * blockDim.x) {
        const uint32_t row = d.row_begin + t;
        if (row >= actual_rows) continue;
        slots[row] = d.slot;
        positions[row] = d.prefix_length + t;
    }
}

// -------------------------------------------------- generic attention
// Any head_dim <= 256, any q_per_kv: one wave per (row, q_head), lanes over
// dims (4 per lane), online softmax in fp32, the reference's per-(row, head)
// formulation (paged_decode.hip:47-206, FP8 :970-1140).
template <int KVB>
__global__ __launch_bounds__(256) void generic_attention_kernel(const psk_paged_attention_args a,
                                                                const uint8_t* kp, const uint8_t* vp,
                                                                const float* ksc, const float* vsc) {
    const uint64_t task = ((uint64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    const uint32_t lane = threadIdx.x & 63u;
    if (task >= (uint64_t)a.rows * a.q_heads) return;
    const uint32_t row = (uint32_t)(task / a.q_heads);
    const uint32_t qh = (uint32_t)(task % a.q_heads);
    const uint32_t kvh = qh / (a.q_heads / a.kv_heads);
    const uint32_t slot = a.row_sequence_slots[row];
    if (slot >= a.max_sequences) return;
    const uint64_t vis64 = (uint64_t)a.row_positions[row] + 1u;
    if (vis64 > (uint64_t)a.block_table_stride * a.page_tokens) return;
    const uint32_t visible = (uint32_t)vis64;
    const uint32_t D = a.head_dim;
    const uint32_t* bt = a.block_tables + (uint64_t)slot * a.block_table_stride;
    const uint16_t* q = static_cast<const uint16_t*>(a.q) + (uint64_t)row * a.q_row_stride +
                        (uint64_t)qh * D;
    float qv[4], acc[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t d = lane + 64u * j;
        qv[j] = d < D ? bf16_bits_to_f32(q[d]) : 0.0f;
        acc[j] = 0.0f;
    }
    float m = -INFINITY, l = 0.0f;
    const float sl = a.scale * kLog2e;
    for (uint32_t t = 0; t < visible; ++t) {
        const uint32_t page = bt[t / a.page_tokens];
        if (page >= a.num_pages) return;   // output left unwritten
        const uint64_t e = (uint64_t)a.layer * a.elems_per_layer + (uint64_t)page * a.elems_per_page +
                           (uint64_t)(t % a.page_tokens) * a.elems_per_token + (uint64_t)kvh * D;
        float kf[4], vf[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t d = lane + 64u * j;
            if (d < D) {
                if constexpr (KVB == 2) {
                    kf[j] = bf16_bits_to_f32(reinterpret_cast<const uint16_t*>(kp)[e + d]);
                    vf[j] = bf16_bits_to_f32(reinterpret_cast<const uint16_t*>(vp)[e + d]);
                } else {
                    kf[j] = __builtin_amdgcn_cvt_pk_f32_fp8((uint32_t)kp[e + d], false)[0];
                    vf[j] = __builtin_amdgcn_cvt_pk_f32_fp8((uint32_t)vp[e + d], false)[0];
                }
            } else {
                kf[j] = 0.0f;
                vf[j] = 0.0f;
            }
        }
        float dot = 0.0f;
#pragma unroll
        for (int j = 0; j < 4; ++j) dot += qv[j] * kf[j];
        dot = wave_sum(dot);
        float vw = 1.0f, f = sl;
        if constexpr (KVB == 1) {
            const uint64_t si = (((uint64_t)a.layer * a.num_pages + page) * a.page_tokens +
                                 t % a.page_tokens) * a.kv_heads + kvh;
            f *= ksc[si];
            vw = vsc[si];
        }
        const float s = dot * f;
        const float mn = __builtin_fmaxf(m, s);
        const float alpha = __builtin_amdgcn_exp2f(m - mn);
        const float w = __builtin_amdgcn_exp2f(s - mn);
        l = l * alpha + w;
        m = mn;
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[j] = acc[j] * alpha + (w * vw) * vf[j];
    }
    const uint64_t ob = (uint64_t)row * a.output_row_stride + (uint64_t)qh * D;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t d = lane + 64u * j;
        if (d >= D) continue;
        const float r = acc[j] / l;
        if (a.output_dtype == PSK_OUT_F32)
            static_cast<float*>(a.output)[ob + d] = r;
        else
            static_cast<uint16_t*>(a.output)[ob + d] = f32_to_bf16_bits(r);
    }
}

// PSQ8_W32 / PSQ4_W32 KV, same formulation: every value dequantised as
// bf16 block scale x codebook value in fp32 (paged_decode.hip:1206-1215,
// 1667-1673); block index bi = (token, head) slice * D/32 + d/32.
template <bool kPsq4>
__global__ __launch_bounds__(256) void generic_attention_psq_kernel(
    const psk_paged_attention_args a, const uint8_t* kp, const uint8_t* vp, const uint16_t* ksc,
    const uint16_t* vsc) {
    const uint64_t task = ((uint64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    const uint32_t lane = threadIdx.x & 63u;
    if (task >= (uint64_t)a.rows * a.q_heads) return;
    const uint32_t row = (uint32_t)(task / a.q_heads);
    const uint32_t qh = (uint32_t)(task % a.q_heads);
    const uint32_t kvh = qh / (a.q_heads / a.kv_heads);
    const uint32_t slot = a.row_sequence_slots[row];
    if (slot >= a.max_sequences) return;
    const uint64_t vis64 = (uint64_t)a.row_positions[row] + 1u;
    if (vis64 > (uint64_t)a.block_table_stride * a.page_tokens) return;
    const uint32_t visible = (uint32_t)vis64;
    const uint32_t D = a.head_dim;
    const uint32_t bph = D / 32u;
    const uint32_t* bt = a.block_tables + (uint64_t)slot * a.block_table_stride;
    const uint16_t* q = static_cast<const uint16_t*>(a.q) + (uint64_t)row * a.q_row_stride +
                        (uint64_t)qh * D;
    float qv[4], acc[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t d = lane + 64u * j;
        qv[j] = d < D ? bf16_bits_to_f32(q[d]) : 0.0f;
        acc[j] = 0.0f;
    }
    auto value = [&](const uint8_t* pool, const uint16_t* scl, uint64_t bi, uint32_t j) {
        uint32_t c;
        if constexpr (kPsq4) {
            const uint32_t byte = pool[bi * 16u + (j & 15u)];
            c = j < 16u ? (byte & 0xFu) : (byte >> 4);
            const uint32_t mi = c & 7u;
            const float mag = mi < 5u ? (float)mi : (float)(2u * mi - 4u);   // 0,1,2,3,4,6,8,10
            return bf16_bits_to_f32(scl[bi]) * ((c & 8u) ? -mag : mag);
        } else {
            c = pool[bi * 32u + j];
            return bf16_bits_to_f32(scl[bi]) * __builtin_amdgcn_cvt_pk_f32_fp8(c, false)[0];
        }
    };
    float m = -INFINITY, l = 0.0f;
    const float sl = a.scale * kLog2e;
    for (uint32_t t = 0; t < visible; ++t) {
        const uint32_t page = bt[t / a.page_tokens];
        if (page >= a.num_pages) return;   // output left unwritten
        const uint64_t tb = ((((uint64_t)a.layer * a.num_pages + page) * a.page_tokens +
                              t % a.page_tokens) * a.kv_heads + kvh) * bph;
        float kf[4], vf[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t d = lane + 64u * j;
            kf[j] = d < D ? value(kp, ksc, tb + d / 32u, d % 32u) : 0.0f;
            vf[j] = d < D ? value(vp, vsc, tb + d / 32u, d % 32u) : 0.0f;
        }
        float dot = 0.0f;
#pragma unroll
        for (int j = 0; j < 4; ++j) dot += qv[j] * kf[j];
        dot = wave_sum(dot);
        const float s = dot * sl;
        const float mn = __builtin_fmaxf(m, s);
        const float alpha = __builtin_amdgcn_exp2f(m - mn);
        const float w = __builtin_amdgcn_exp2f(s - mn);
        l = l * alpha + w;
        m = mn;
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[j] = acc[j] * alpha + w * vf[j];
    }
    const uint64_t ob = (uint64_t)row * a.output_row_stride + (uint64_t)qh * D;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t d = lane + 64u * j;
        if (d >= D) continue;
        const float r = acc[j] / l;
        if (a.output_dtype == PSK_OUT_F32)
            static_cast<float*>(a.output)[ob + d] = r;
        else
            static_cast<uint16_t*>(a.output)[ob + d] = f32_to_bf16_bits(r);
    }
}

// ------------------------------------------------- encoder self-test
// Encodes the floats with bit patterns start .. start+count-1 through the same
// e4m3_encode_pair the append kernel uses (pairs land in bytes 0-3 of a word
// exactly as in kv_append_kernel).
__global__ __launch_bounds__(256) void e4m3_selftest_kernel(uint32_t start, uint32_t count,
                                                            uint32_t* out) {
    const uint64_t w = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (w * 4u >= count) return;
    float x[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) x[i] = __uint_as_float(start + (uint32_t)(w * 4u) + (uint32_t)i);
    out[w] = e4m3_encode_pair(x[2], x[3], e4m3_encode_pair(x[0], x[1], 0u, false), true);
}

__global__ __launch_bounds__(256) void e4m3_decode_selftest_kernel(float* out) {
    const uint32_t c = threadIdx.x;
    const uint32_t bf = fp8x2_to_bf16x2(c, false) & 0xFFFFu;
    out[c] = __uint_as_float(bf << 16);
}

}  // namespace

hipError_t launch_attention_generic(const psk_paged_attention_args& c, int kvb, const void* k,
                                    const void* v, const float* ks, const float* vs,
                                    hipStream_t stream) {
    const uint64_t waves = (uint64_t)c.rows * c.q_heads;
    const uint64_t blocks = (waves + 3u) / 4u;
    if (blocks == 0u || blocks > 0x7FFFFFFFull) return hipErrorInvalidValue;
    if (kvb == 2)
        hipLaunchKernelGGL(generic_attention_kernel<2>, dim3((uint32_t)blocks), dim3(256), 0, stream,
                           c, static_cast<const uint8_t*>(k), static_cast<const uint8_t*>(v), ks, vs);
    else
        hipLaunchKernelGGL(generic_attention_kernel<1>, dim3((uint32_t)blocks), dim3(256), 0, stream,
                           c, static_cast<const uint8_t*>(k), static_cast<const uint8_t*>(v), ks, vs);
    return hipGetLastError();
}

hipError_t launch_attention_generic_psq(const psk_paged_attention_args& c, bool psq4, const void* k,
                                        const void* v, const uint16_t* ks, const uint16_t* vs,
                                        hipStream_t stream) {
    const uint64_t waves = (uint64_t)c.rows * c.q_heads;
    const uint64_t blocks = (waves + 3u) / 4u;
    if (blocks == 0u || blocks > 0x7FFFFFFFull) return hipErrorInvalidValue;
    if (psq4)
        hipLaunchKernelGGL(generic_attention_psq_kernel<true>, dim3((uint32_t)blocks), dim3(256), 0,
                           stream, c, static_cast<const uint8_t*>(k), static_cast<const uint8_t*>(v),
                           ks, vs);
    else
        hipLaunchKernelGGL(generic_attention_psq_kernel<false>, dim3((uint32_t)blocks), dim3(256), 0,
                           stream, c, static_cast<const uint8_t*>(k), static_cast<const uint8_t*>(v),
                           ks, vs);
    return hipGetLastError();
}

}  // namespace psk

extern "C" int psk_kv_gather(const psk_kv_gather_args* a, const void* pool, void* out,
                             uint32_t elem_bytes, void* stream) {
    if (a == nullptr || pool == nullptr || out == nullptr) return hipErrorInvalidValue;
    if (elem_bytes != 1u && elem_bytes != 2u && elem_bytes != 4u) return hipErrorInvalidValue;
    if (a->total_tokens == 0u) return hipSuccess;
    if (a->block_tables == nullptr || a->seq_slots == nullptr || a->seq_token_offsets == nullptr ||
        a->num_seqs == 0u || a->page_tokens == 0u || a->elems_per_token == 0u)
        return hipErrorInvalidValue;
    const uint64_t row_bytes = (uint64_t)a->elems_per_token * elem_bytes;
    const uint32_t vec16 = (row_bytes % 16u == 0u) && ((uint64_t)a->elems_per_page * elem_bytes % 16u == 0u) &&
                           ((uint64_t)a->elems_per_layer * elem_bytes % 16u == 0u) &&
                           (reinterpret_cast<uintptr_t>(pool) % 16u == 0u) &&
                           (reinterpret_cast<uintptr_t>(out) % 16u == 0u);
    const uint64_t blocks = ((uint64_t)a->total_tokens + 3u) / 4u;
    hipLaunchKernelGGL(psk::gather_kernel, dim3((uint32_t)blocks), dim3(256), 0,
                       static_cast<hipStream_t>(stream), *a, static_cast<const uint8_t*>(pool),
                       static_cast<uint8_t*>(out), elem_bytes, vec16);
    return hipGetLastError();
}

namespace psk {
namespace {
hipError_t copy_validate(const psk_page_copy_args* a, uint32_t& vec16) {
    if (a == nullptr) return hipErrorInvalidValue;
    if (a->dst_k == nullptr || a->dst_v == nullptr || a->src_k == nullptr || a->src_v == nullptr ||
        a->num_layers == 0u || a->page_tokens == 0u || a->kv_heads == 0u || a->head_dim == 0u)
        return hipErrorInvalidValue;
    const bool psq = a->kv_dtype == PSK_KV_PSQ4_W32 || a->kv_dtype == PSK_KV_PSQ8_W32;
    if (a->kv_dtype != PSK_KV_BF16 && a->kv_dtype != PSK_KV_FP8_E4M3 && !psq)
        return hipErrorInvalidValue;
    if (psq && a->head_dim % 32u != 0u) return hipErrorInvalidValue;
    const bool scaled = a->kv_dtype != PSK_KV_BF16;
    if (scaled && (a->dst_k_scale == nullptr || a->dst_v_scale == nullptr ||
                   a->src_k_scale == nullptr || a->src_v_scale == nullptr))
        return hipErrorInvalidValue;
    auto al = [](const void* p) { return reinterpret_cast<uintptr_t>(p) % 16u == 0u; };
    vec16 = al(a->dst_k) && al(a->dst_v) && al(a->src_k) && al(a->src_v) &&
            (!scaled ||
             (al(a->dst_k_scale) && al(a->dst_v_scale) && al(a->src_k_scale) && al(a->src_v_scale)));
    return hipSuccess;
}
}  // namespace

// Host-array variant used by the C++ pool layer: chunks of kInlinePairs pairs
// go to the kernel by value.
hipError_t copy_pages_host_pairs(const psk_page_copy_args& args, const psk_page_copy_pair* pairs,
                                 uint32_t n, hipStream_t stream) {
    return copy_plan_host(&args, pairs, n, nullptr, 0, stream, nullptr);
}

// Page pairs (kv == nullptr or n == 0: none) and segments in as few launches
// as the inline pair limit allows: the first launch carries every segment and
// the first kInlinePairs pairs.
hipError_t copy_plan_host(const psk_page_copy_args* kv, const psk_page_copy_pair* pairs, uint32_t n,
                          const CopySegment* segs, uint32_t nseg, hipStream_t stream,
                          psk_page_copy_pair* device_pairs) {
    if (nseg > kMaxCopySegments) return hipErrorInvalidValue;
    uint32_t vec16 = 0;
    psk_page_copy_args base{};
    if (kv != nullptr && n > 0) {
        const hipError_t e = copy_validate(kv, vec16);
        if (e != hipSuccess) return e;
        base = *kv;
    } else {
        n = 0;
        base.num_layers = 1;
    }
    InlineSegments is{};
    uint64_t seg_blocks = 0;
    for (uint32_t i = 0; i < nseg; ++i) {
        if (segs[i].bytes != 0 && (segs[i].dst == nullptr || segs[i].src == nullptr))
            return hipErrorInvalidValue;
        is.s[i] = segs[i];
        is.first_block[i] = seg_blocks;
        seg_blocks += (segs[i].bytes + kSegmentBlockBytes - 1) / kSegmentBlockBytes;
    }
    is.first_block[nseg] = seg_blocks;
    if (device_pairs != nullptr && n > kInlinePairs) {
        // one launch: the pair list goes to the caller's device buffer first
        // (a pageable-source copy returns once the data is staged)
        hipError_t e = hipMemcpyAsync(device_pairs, pairs, (size_t)n * sizeof(psk_page_copy_pair),
                                      hipMemcpyHostToDevice, stream);
        if (e != hipSuccess) return e;
        psk_page_copy_args a = base;
        a.num_pairs = n;
        a.pairs = device_pairs;
        const uint64_t page_blocks = (uint64_t)n * a.num_layers * kCopyTensors;
        const uint64_t blocks = page_blocks + seg_blocks;
        if (blocks > 0x7FFFFFFFull) return hipErrorInvalidValue;
        hipLaunchKernelGGL(copy_plan_kernel, dim3((uint32_t)blocks), dim3(256), 0, stream, a,
                           InlinePairs{}, is, nseg, vec16, (uint32_t)seg_blocks);
        return hipGetLastError();
    }
    uint32_t b = 0;
    do {
        psk_page_copy_args a = base;
        a.num_pairs = n - b < kInlinePairs ? n - b : kInlinePairs;
        a.pairs = nullptr;
        InlinePairs ip{};
        for (uint32_t i = 0; i < a.num_pairs; ++i) ip.p[i] = pairs[b + i];
        const uint64_t page_blocks = (uint64_t)a.num_pairs * a.num_layers * kCopyTensors;
        const uint32_t ns = b == 0 ? nseg : 0u;
        const uint64_t blocks = page_blocks + (b == 0 ? seg_blocks : 0u);
        if (blocks > 0x7FFFFFFFull) return hipErrorInvalidValue;
        if (blocks > 0) {
            hipLaunchKernelGGL(copy_plan_kernel, dim3((uint32_t)blocks), dim3(256), 0, stream, a, ip,
                               is, ns, vec16, (uint32_t)(b == 0 ? seg_blocks : 0u));
            const hipError_t le = hipGetLastError();
            if (le != hipSuccess) return le;
        }
        b += a.num_pairs;
    } while (b < n);
    return hipSuccess;
}

// Zero `bytes` (a multiple of 4) at dst without hipMemsetAsync.
hipError_t zero_fill(void* dst, uint64_t bytes, hipStream_t stream) {
    if (bytes % 4u) return hipErrorInvalidValue;
    return static_cast<hipError_t>(psk_fill_u32(static_cast<uint32_t*>(dst), 0u, bytes / 4u, stream));
}

}  // namespace psk

extern "C" int psk_kv_copy_pages(const psk_page_copy_args* a, void* stream) {
    if (a == nullptr) return hipErrorInvalidValue;
    if (a->num_pairs == 0u) return hipSuccess;
    if (a->pairs == nullptr) return hipErrorInvalidValue;
    uint32_t vec16 = 0;
    const hipError_t e = psk::copy_validate(a, vec16);
    if (e != hipSuccess) return e;
    const uint64_t blocks = (uint64_t)a->num_pairs * a->num_layers * psk::kCopyTensors;
    if (blocks > 0x7FFFFFFFull) return hipErrorInvalidValue;
    hipLaunchKernelGGL(psk::copy_pages_kernel, dim3((uint32_t)blocks), dim3(256), 0,
                       static_cast<hipStream_t>(stream), *a, vec16);
    return hipGetLastError();
}

extern "C" int psk_fill_u32(uint32_t* dst, uint32_t value, uint64_t count, void* stream) {
    if (count == 0u) return hipSuccess;
    if (dst == nullptr) return hipErrorInvalidValue;
    uint64_t blocks = (count + 255u) / 256u;
    if (blocks > 4096u) blocks = 4096u;
    hipLaunchKernelGGL(psk::fill_u32_kernel, dim3((uint32_t)blocks), dim3(256), 0,
                       static_cast<hipStream_t>(stream), dst, value, count);
    return hipGetLastError();
}

extern "C" int psk_prepare_row_metadata(const psk_request_descriptor* requests, uint32_t num_requests,
                                        uint32_t actual_rows, uint32_t* row_sequence_slots,
                                        uint32_t* row_positions, void* stream) {
    if (num_requests == 0u) return hipSuccess;
    if (requests == nullptr || row_sequence_slots == nullptr || row_positions == nullptr)
        return hipErrorInvalidValue;
    if (num_requests > 65535u) return hipErrorInvalidValue;
    hipLaunchKernelGGL(psk::row_metadata_kernel, dim3(8, num_requests), dim3(256), 0,
                       static_cast<hipStream_t>(stream), requests, num_requests, actual_rows,
                       row_sequence_slots, row_positions);
    return hipGetLastError();
}

// Self-test hooks: run the device E4M3 encoder / decoder on given inputs.
extern "C" int psk_selftest_e4m3_encode_range(uint32_t start_bits, uint32_t count, uint32_t* out_words,
                                              void* stream) {
    if (out_words == nullptr || count % 4u != 0u) return hipErrorInvalidValue;
    if (count == 0u) return hipSuccess;
    const uint64_t words = count / 4u;
    hipLaunchKernelGGL(psk::e4m3_selftest_kernel, dim3((uint32_t)((words + 255u) / 256u)), dim3(256),
                       0, static_cast<hipStream_t>(stream), start_bits, count, out_words);
    return hipGetLastError();
}

extern "C" int psk_selftest_e4m3_decode_all(float* out256, void* stream) {
    if (out256 == nullptr) return hipErrorInvalidValue;
    hipLaunchKernelGGL(psk::e4m3_decode_selftest_kernel, dim3(1), dim3(256), 0,
                       static_cast<hipStream_t>(stream), out256);
    return hipGetLastError();
}
