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

__device__ __forceinline__ bool resolve_row(const psk_kv_append_args& a, uint32_t row,
                                            uint64_t& base, uint32_t& page, uint32_t& off) {
    const uint32_t slot = a.row_sequence_slots[row];
    if (slot >= a.max_sequences) return false;
    const uint32_t pos = a.row_positions[row];
    const uint32_t lb = pos / a.page_tokens;
    off = pos % a.page_tokens;
    if (lb >= a.block_table_stride) return false;
    page = a.block_tables[(uint64_t)slot * a.block_table_stride + lb];
    if (page >= a.num_pages) return false;
    base = (uint64_t)a.layer * a.elems_per_layer + (uint64_t)page * a.elems_per_page +
           (uint64_t)off * a.elems_per_token;
    return true;
}

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

template <bool kFp8>
__global__ __launch_bounds__(256) void kv_append_kernel(const AppendParams p) {
    const psk_kv_append_args& a = p.a;
    const uint32_t L = p.lanes_per_head;
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t wave_global = (blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    const uint32_t tasks_per_wave = 64u >> p.log2_lanes;
    const uint64_t task = (uint64_t)wave_global * tasks_per_wave + (lane >> p.log2_lanes);
    const uint32_t sub = lane & (L - 1u);
    const uint64_t total = (uint64_t)a.rows * a.kv_heads;
    const bool live = task < total;

    uint32_t row = 0, head = 0, page = 0, off = 0;
    uint64_t base = 0;
    bool valid = false;
    if (live) {
        row = (uint32_t)(task / a.kv_heads);
        head = (uint32_t)(task % a.kv_heads);
        valid = resolve_row(a, row, base, page, off);
    }
    const uint32_t D = a.head_dim;
    const bool vec = p.vec_ok != 0u;
    const uint16_t* ks = static_cast<const uint16_t*>(a.k_input) + (uint64_t)row * a.k_row_stride +
                         (uint64_t)head * D;
    const uint16_t* vs = static_cast<const uint16_t*>(a.v_input) + (uint64_t)row * a.v_row_stride +
                         (uint64_t)head * D;
    const uint64_t dst = base + (uint64_t)head * D;

    if constexpr (!kFp8) {
        if (!valid) return;
        uint16_t* kd = static_cast<uint16_t*>(p.k_pool) + dst;
        uint16_t* vd = static_cast<uint16_t*>(p.v_pool) + dst;
        for (uint32_t c = sub; c < p.chunks; c += L) {
            const uint32_t e0 = c * 8u;
            if (vec) {
                const u32x4 kw = *reinterpret_cast<const u32x4*>(ks + e0);
                const u32x4 vw = *reinterpret_cast<const u32x4*>(vs + e0);
                *reinterpret_cast<u32x4*>(kd + e0) = kw;
                *reinterpret_cast<u32x4*>(vd + e0) = vw;
            } else {
                for (uint32_t i = 0; i < 8u && e0 + i < D; ++i) {
                    kd[e0 + i] = ks[e0 + i];
                    vd[e0 + i] = vs[e0 + i];
                }
            }
        }
    } else {
        // Pass 1: per-head absmax over the L lanes of the task. fmaxf ignores
        // NaN, as the reference's fmaxf(k_max, fabsf(kf)) does.
        float kx[8], vx[8];
        float km = 0.0f, vm = 0.0f;
        if (valid) {
            for (uint32_t c = sub; c < p.chunks; c += L) {
                load_chunk(ks, c, D, vec, kx);
                load_chunk(vs, c, D, vec, vx);
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    km = __builtin_fmaxf(km, __builtin_fabsf(kx[i]));
                    vm = __builtin_fmaxf(vm, __builtin_fabsf(vx[i]));
                }
            }
        }
        // Reduce within the L-lane group (groups are aligned lane ranges).
        for (uint32_t o = L >> 1; o >= 1u; o >>= 1) {
            km = __builtin_fmaxf(km, __shfl_xor(km, (int)o, 64));
            vm = __builtin_fmaxf(vm, __shfl_xor(vm, (int)o, 64));
        }
        if (!valid) return;
        const float k_scale = km == 0.0f ? 1.0f : km / kFp8Max;
        const float v_scale = vm == 0.0f ? 1.0f : vm / kFp8Max;
        const float k_rcp = 1.0f / k_scale;
        const float v_rcp = 1.0f / v_scale;
        const bool k_fast = k_scale >= 0x1p-100f && k_scale <= 0x1.fffffep+127f;
        const bool v_fast = v_scale >= 0x1p-100f && v_scale <= 0x1.fffffep+127f;
        if (sub == 0u) {
            const uint64_t si =
                (((uint64_t)a.layer * a.num_pages + page) * a.page_tokens + off) * a.kv_heads + head;
            p.k_scale[si] = k_scale;
            p.v_scale[si] = v_scale;
        }
        uint8_t* kd = static_cast<uint8_t*>(p.k_pool) + dst;
        uint8_t* vd = static_cast<uint8_t*>(p.v_pool) + dst;
        // Pass 2: quantize. With one chunk per lane the values are still in
        // registers; otherwise they are reloaded (cache hits).
        const bool single = p.chunks <= L;
        for (uint32_t c = sub; c < p.chunks; c += L) {
            if (!single) {
                load_chunk(ks, c, D, vec, kx);
                load_chunk(vs, c, D, vec, vx);
            }
            float kq[8], vq[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                kq[i] = div_by_scale(kx[i], k_scale, k_rcp, k_fast);
                vq[i] = div_by_scale(vx[i], v_scale, v_rcp, v_fast);
            }
            u32x2 kc, vc;
            kc[0] = e4m3_encode_pair(kq[2], kq[3], e4m3_encode_pair(kq[0], kq[1], 0u, false), true);
            kc[1] = e4m3_encode_pair(kq[6], kq[7], e4m3_encode_pair(kq[4], kq[5], 0u, false), true);
            vc[0] = e4m3_encode_pair(vq[2], vq[3], e4m3_encode_pair(vq[0], vq[1], 0u, false), true);
            vc[1] = e4m3_encode_pair(vq[6], vq[7], e4m3_encode_pair(vq[4], vq[5], 0u, false), true);
            const uint32_t e0 = c * 8u;
            if (vec) {
                *reinterpret_cast<u32x2*>(kd + e0) = kc;
                *reinterpret_cast<u32x2*>(vd + e0) = vc;
            } else {
                for (uint32_t i = 0; i < 8u && e0 + i < D; ++i) {
                    kd[e0 + i] = (uint8_t)(kc[i >> 2] >> (8u * (i & 3u)));
                    vd[e0 + i] = (uint8_t)(vc[i >> 2] >> (8u * (i & 3u)));
                }
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
    const uint64_t waves = (tasks + tasks_per_wave - 1) / tasks_per_wave;
    const uint64_t blocks = (waves + 3) / 4;
    if (blocks > 0x7FFFFFFFull) return hipErrorInvalidValue;
    hipLaunchKernelGGL(kv_append_kernel<kFp8>, dim3((uint32_t)blocks), dim3(256), 0, stream, p);
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
