// Device helpers shared by the gfx950 kernels of the paged KV path.
// Wave64 throughout: a wavefront is 64 lanes, cross-lane reductions use the
// full width.
#pragma once
#include <hip/hip_runtime.h>
#include <atomic>
#include <cstdint>

namespace psk {

typedef __attribute__((ext_vector_type(2))) float f32x2;
typedef __attribute__((ext_vector_type(4))) float f32x4;
typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2;
typedef __attribute__((ext_vector_type(4))) uint32_t u32x4;
typedef __attribute__((ext_vector_type(2))) uint32_t u32x2;

constexpr int kWave = 64;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kFp8Max = 448.0f;

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h) {
    return __uint_as_float(h << 16);
}

// Round-to-nearest-even f32 -> bf16 bits (NaN -> quiet NaN), as __float2bfloat16.
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
    bf16x2 v = __builtin_convertvector((f32x2){f, 0.0f}, bf16x2);
    return __builtin_bit_cast(uint32_t, v) & 0xFFFFu;
}

__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){a, b}, bf16x2));
}

// a, b -> bf16 pairs hi = bf16(x), lo = bf16(x - hi): hi + lo carries ~16
// mantissa bits of x (RNE at each step).
// Returns {hi, lo}.
__device__ __forceinline__ u32x2 split_bf16x2(float a, float b) {
    const uint32_t hi = pack_bf16x2(a, b);
    const float ah = __uint_as_float(hi << 16), bh = __uint_as_float(hi & 0xFFFF0000u);
    return (u32x2){hi, pack_bf16x2(a - ah, b - bh)};
}

// Two FP8 E4M3 codes (bytes 0/1 or 2/3 of `w`) -> two bf16 (exact: every E4M3
// value is a bf16 value). One v_cvt_scalef32_pk_bf16_fp8 with unit scale.
__device__ __forceinline__ uint32_t fp8x2_to_bf16x2(uint32_t w, bool hi) {
    bf16x2 r = hi ? __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, true)
                  : __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, false);
    return __builtin_bit_cast(uint32_t, r);
}

// 8 FP8 codes in two dwords -> 8 bf16 as one MFMA operand.
__device__ __forceinline__ bf16x8 fp8x8_to_bf16x8(uint32_t w0, uint32_t w1) {
    u32x4 r;
    r[0] = fp8x2_to_bf16x2(w0, false);
    r[1] = fp8x2_to_bf16x2(w0, true);
    r[2] = fp8x2_to_bf16x2(w1, false);
    r[3] = fp8x2_to_bf16x2(w1, true);
    return __builtin_bit_cast(bf16x8, r);
}

// SATFINITE E4M3 encode of two floats into the low 16 bits of the result
// (byte 0 = a, byte 1 = b): clamp finite values to [-448, 448], then the
// hardware round-to-nearest-even conversion. This is what ROCm's
// __hip_cvt_float_to_fp8(x, __HIP_SATFINITE, __HIP_E4M3) lowers to on gfx950,
// the conversion the reference calls (kv_append.hip:144-146).
__device__ __forceinline__ float sat_e4m3(float x) {
    const uint32_t u = __float_as_uint(x);
    return ((u & 0x7F800000u) != 0x7F800000u) ? __builtin_amdgcn_fmed3f(x, kFp8Max, -kFp8Max)
                                              : x;
}
__device__ __forceinline__ uint32_t e4m3_encode_pair(float a, float b, uint32_t old, bool hi) {
    return hi ? __builtin_amdgcn_cvt_pk_fp8_f32(sat_e4m3(a), sat_e4m3(b), old, true)
              : __builtin_amdgcn_cvt_pk_fp8_f32(sat_e4m3(a), sat_e4m3(b), old, false);
}

// x / s with the IEEE-correct result's E4M3 code, given r = 1/s correctly
// rounded: q0 = x*r, rem = fma(-q0, s, x) (exact), q = fma(rem, r, q0).
// Valid when s >= 2^-100 and |x| >= 2^-100; otherwise a true division is used.
// The E4M3 code of the result was checked equal to the code of x/s for every
// finite bf16 pair with |x| <= amax, s = amax/448 (tests/native/div_identity.c).
__device__ __forceinline__ float div_by_scale(float x, float s, float r, bool fast_scale) {
    if (fast_scale && __builtin_fabsf(x) >= 0x1p-100f) {
        const float q0 = x * r;
        const float rem = __builtin_fmaf(-q0, s, x);
        return __builtin_fmaf(rem, r, q0);
    }
    return x / s;
}

typedef __attribute__((ext_vector_type(8))) _Float16 f16x8;
typedef __attribute__((ext_vector_type(2))) _Float16 f16x2;

// 8 FP8 codes in two dwords -> 8 f16 (exact: every E4M3 value is an f16 value).
__device__ __forceinline__ f16x8 fp8x8_to_f16x8(uint32_t w0, uint32_t w1) {
    u32x4 r;
    r[0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w0, 1.0f, false));
    r[1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w0, 1.0f, true));
    r[2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w1, 1.0f, false));
    r[3] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w1, 1.0f, true));
    return __builtin_bit_cast(f16x8, r);
}

// Packs 4 floats into 4 E4M3 bytes (hardware RNE; callers keep |x| <= 448).
__device__ __forceinline__ uint32_t e4m3x4_rne(float a, float b, float c, float d) {
    uint32_t w = (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
    return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(c, d, (int)w, true);
}

// Two floats -> f16 pair (round to nearest even).
__device__ __forceinline__ uint32_t pack_f16x2(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){a, b}, f16x2));
}

// Online softmax with a lazily moved reference: the running reference max
// (log2 units) moves only when a new score exceeds it by more than this, so
// the accumulator rescale is rare; exponentials stay below 2^kLazyMaxSlack.
constexpr float kLazyMaxSlack = 8.0f;

template <int W>
__device__ __forceinline__ float group_max(float x) {
#pragma unroll
    for (int o = W / 2; o >= 1; o >>= 1) x = __builtin_fmaxf(x, __shfl_xor(x, o, 64));
    return x;
}

// Combine x with the value of lane ^ 16 (lane ^ 32) without the LDS crossbar:
// v_permlane16_swap (v_permlane32_swap) with both operands x returns, in its
// two results, x of the lane and of its partner in some order, so a
// symmetric combine of the two is the pairwise reduction.
__device__ __forceinline__ float max_xor16(float x) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __builtin_fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float max_xor32(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __builtin_fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum_xor16(float x) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float sum_xor32(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// The value of lane ^ 8 (within each 16-lane row; DPP row rotate by 8).
__device__ __forceinline__ uint32_t row_ror8(uint32_t x) {
    // every lane of every row is written, so the instruction needs no prior
    // value of its destination (mov_dpp leaves it undefined)
    return (uint32_t)__builtin_amdgcn_mov_dpp((int)x, 0x128, 0xF, 0xF, true);
}
__device__ __forceinline__ float row_ror8(float x) { return __uint_as_float(row_ror8(__float_as_uint(x))); }

// Maximum of x over the 64 lanes without the LDS crossbar: DPP row rotates
// within each 16-lane row, then the permlane swaps across rows.
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t x) {
    x = max(x, (uint32_t)__builtin_amdgcn_mov_dpp((int)x, 0x128, 0xF, 0xF, true));   // row_ror:8
    x = max(x, (uint32_t)__builtin_amdgcn_mov_dpp((int)x, 0x124, 0xF, 0xF, true));   // row_ror:4
    x = max(x, (uint32_t)__builtin_amdgcn_mov_dpp((int)x, 0x122, 0xF, 0xF, true));   // row_ror:2
    x = max(x, (uint32_t)__builtin_amdgcn_mov_dpp((int)x, 0x121, 0xF, 0xF, true));   // row_ror:1
    const auto a = __builtin_amdgcn_permlane16_swap(x, x, false, false);
    x = max(a[0], a[1]);
    const auto b = __builtin_amdgcn_permlane32_swap(x, x, false, false);
    return max(b[0], b[1]);
}

// A wave-uniform float moved to a scalar register.
__device__ __forceinline__ float uniform_f32(float x) {
    return __uint_as_float(__builtin_amdgcn_readfirstlane(__float_as_uint(x)));
}

__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) x += __shfl_xor(x, o, 64);
    return x;
}

__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) x = __builtin_fmaxf(x, __shfl_xor(x, o, 64));
    return x;
}

typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(1))) void global_void_t;

// Global memory straight into LDS (gfx950 LDS DMA, global_load_lds_dword /
// _dwordx4): lane l of the wave writes LDS[dst + BYTES*l] (the instruction's
// immediate offset would be added to both addresses; it is 0 here). `dst`
// must be wave-uniform. The hardware counts these loads in vmcnt and writes
// LDS asynchronously: the data may be read only after s_waitcnt vmcnt.
// CPOL is the cache policy: kCpolStream (the `nt` bit) for bytes read once
// in whole 128 B lines. On MI355X a stream of such 16 B DMAs reaches ~6.8 TB/s
// against ~6.1 TB/s with the default policy; DMAs that read half lines
// (16 rows x 64 B per instruction) are slower with `nt` (~5.9 TB/s), since the
// two halves of a line are no longer served by one L2 fill.
constexpr int kCpolDefault = 0;
constexpr int kCpolStream = 2;
template <int BYTES, int CPOL = kCpolDefault>
__device__ __forceinline__ void load_lds(const void* src, uint8_t* dst) {
    static_assert(BYTES == 4 || BYTES == 16, "DMA width");
    if constexpr (BYTES == 16)
        __builtin_amdgcn_global_load_lds((global_void_t*)src, (lds_void_t*)dst, 16, 0, CPOL);
    else
        __builtin_amdgcn_global_load_lds((global_void_t*)src, (lds_void_t*)dst, 4, 0, CPOL);
}

// Waits until at most N vector-memory operations of this wave are
// outstanding. The memory clobber keeps every load and LDS access on its side.
// The pipelines count their own DMAs into N, so a loop that waits this way
// must issue no other vector-memory operation (register spills to scratch
// included): the kernels' chunk loops are kept free of spills.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// wait_vmcnt<N> followed by a workgroup barrier without memory fences (a
// fenced __syncthreads would also wait for every outstanding load). After it,
// every wave's LDS DMAs older than its last N vector-memory operations have
// landed in LDS.
template <int N>
__device__ __forceinline__ void wait_vmcnt_barrier() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(N) : "memory");
}

// Orders this wave's LDS writes before its later LDS reads by other lanes.
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// KV formats of the attention kernels.
constexpr int kFmtBf16 = 0;   // bf16 values
constexpr int kFmtFp8 = 1;    // E4M3 codes, one f32 scale per (token, kv head)
constexpr int kFmtPsq8 = 2;   // E4M3 codes, one bf16 scale per 32-value block
constexpr int kFmtPsq4 = 3;   // cb10 nibbles, one bf16 scale per 32-value block

template <int FMT>
constexpr bool fmt_psq() { return FMT == kFmtPsq8 || FMT == kFmtPsq4; }
// bytes of one (token, kv head) K (or V) slice
template <int FMT, int D>
constexpr int code_bytes() { return FMT == kFmtBf16 ? 2 * D : FMT == kFmtPsq4 ? D / 2 : D; }

// Q fragment of a PSQ4 K-step: dims d0..d0+3 and d0+16..d0+19 (the low and
// high nibbles of 4 code bytes), zeros past the group.
__device__ __forceinline__ bf16x8 load_q4x2(const uint16_t* q, bool ok) {
    u32x4 r = {0u, 0u, 0u, 0u};
    if (ok) {
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            r[i] = (uint32_t)q[2 * i] | ((uint32_t)q[2 * i + 1] << 16);
            r[2 + i] = (uint32_t)q[16 + 2 * i] | ((uint32_t)q[16 + 2 * i + 1] << 16);
        }
    }
    return __builtin_bit_cast(bf16x8, r);
}

// The E4M3 codes of the cb10 values of 4 PSQ4 code bytes, low nibbles (hi =
// false) or high nibbles: magnitude index -> E4M3 code of {0,1,2,3,4,6,8,10}
// by byte permute, the nibble's sign bit -> bit 7.
__device__ __forceinline__ uint32_t psq4_e4m3x4(uint32_t x, bool hi) {
    const uint32_t idx = (hi ? (x >> 4) : x) & 0x07070707u;
    const uint32_t mag = __builtin_amdgcn_perm(0x52504C48u, 0x44403800u, idx);
    return mag | ((hi ? x : (x << 4)) & 0x80808080u);
}

// Exclusive scan of two counters over the NW waves of the workgroup; tx, ty
// receive the workgroup totals. All NW*64 threads must call it.
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

// Maps a dense unit index to (item, split) over `count` items, item i holding
// units(i) splits (0: the item is skipped). Units are ordered so that the
// workgroups of one launch spread evenly over the XCDs (block b runs on XCD
// b mod 8) and the longest go first: every item's splits but the last
// (item-major), then the last split of every item. Returns false past the
// last unit. All NW*64 threads of the workgroup must call it.
template <int NW, typename UnitsFn>
__device__ bool find_dense_unit(uint32_t count, UnitsFn units, uint32_t unit, uint32_t& item,
                                uint32_t& split) {
    __shared__ uint32_t tmp[2 * NW];
    __shared__ uint32_t found[2];
    const uint32_t tid = threadIdx.x;
    const uint32_t each = (count + NW * 64u - 1u) / (NW * 64u);
    const uint32_t i0 = min(count, tid * each), i1 = min(count, i0 + each);
    uint32_t nf = 0, nl = 0;   // this thread's non-last and last units
    uint32_t u0 = 0;           // units of item i0, kept for the search below
    for (uint32_t i = i0; i < i1; ++i) {
        const uint32_t u = units(i);
        if (i == i0) u0 = u;
        if (u != 0u) { nf += u - 1u; nl += 1u; }
    }
    if (tid == 0) found[0] = 0xFFFFFFFFu;
    uint32_t pf = nf, pl = nl, F, L;
    block_scan2<NW>(pf, pl, F, L, tmp);
    if (unit < F) {
        if (unit >= pf && unit < pf + nf) {
            uint32_t k = unit - pf;
            for (uint32_t i = i0; i < i1; ++i) {
                const uint32_t u = i == i0 ? u0 : units(i);
                if (u > 1u) {
                    if (k < u - 1u) { found[0] = i; found[1] = k; break; }
                    k -= u - 1u;
                }
            }
        }
    } else if (unit - F < L) {
        const uint32_t k0 = unit - F;
        if (k0 >= pl && k0 < pl + nl) {
            uint32_t k = k0 - pl;
            for (uint32_t i = i0; i < i1; ++i) {
                const uint32_t u = i == i0 ? u0 : units(i);
                if (u != 0u) {
                    if (k == 0u) { found[0] = i; found[1] = u - 1u; break; }
                    --k;
                }
            }
        }
    }
    __syncthreads();
    // uniform over the workgroup: scalar registers
    item = __builtin_amdgcn_readfirstlane(found[0]);
    split = __builtin_amdgcn_readfirstlane(found[1]);
    return item != 0xFFFFFFFFu;
}

// Raises kernel fn's dynamic LDS limit to the CU's 160 KB (less 1 KB of
// static LDS) on the current device, once per device: `done` holds one bit per
// device index that is already set up (devices past 63 are set up on every call).
inline hipError_t allow_full_lds(const void* fn, std::atomic<uint64_t>& done) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return hipErrorInvalidDevice;
    const uint64_t bit = dev >= 0 && dev < 64 ? (uint64_t{1} << dev) : 0u;
    if (bit != 0u && (done.load(std::memory_order_acquire) & bit) != 0u) return hipSuccess;
    const hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024 - 1024);
    if (e == hipSuccess && bit != 0u) done.fetch_or(bit, std::memory_order_release);
    return e;
}

}  // namespace psk
