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
// Layout of the work: one "head task" = (row, kv_head). A task is handled by
// L = lanes_per_head lanes (a power of two <= 64), each lane owning chunks of
// 8 consecutive elements (16 B of bf16 input); a wave runs 64/L tasks. For
// head_dim 256 that is 32 lanes x 16 B per K and V, i.e. fully coalesced
// 512 B reads and 256 B (FP8) or 512 B (BF16) writes per tensor per task.
#include "device_common.h"

#include <phaseshift_kv/kv_append.h>

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
// wave runs kUnroll groups of 64/L tasks. The kUnroll slot/position loads go
// out first, then all input loads, then the block-table loads (which wait
// only for slot/position), so the HBM reads overlap the lookup chain
// (reference skip rules: kv_append.hip:31-55).
constexpr int kUnroll = 4;

template <bool kFp8>
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
        slot[u] = a.row_sequence_slots[row[u]];
        pos[u] = a.row_positions[row[u]];
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
        kw[u] = *reinterpret_cast<const u32x4*>(ks);
        vw[u] = *reinterpret_cast<const u32x4*>(vs);
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
                *reinterpret_cast<u32x2*>(static_cast<uint8_t*>(p.k_pool) + dst) = kc;
                *reinterpret_cast<u32x2*>(static_cast<uint8_t*>(p.v_pool) + dst) = vc;
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
    const uint64_t waves = fast ? (groups + kUnroll - 1) / kUnroll : groups;
    const uint64_t blocks = (waves + 3) / 4;
    if (blocks > 0x7FFFFFFFull) return hipErrorInvalidValue;
    if (fast)
        hipLaunchKernelGGL(kv_append_fast_kernel<kFp8>, dim3((uint32_t)blocks), dim3(256), 0, stream, p);
    else
        hipLaunchKernelGGL(kv_append_generic_kernel<kFp8>, dim3((uint32_t)blocks), dim3(256), 0, stream,
                           p);
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

}  // namespace ps::kernel
