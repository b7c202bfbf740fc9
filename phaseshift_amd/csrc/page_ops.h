// Host entry points of the page-level kernels (page_ops.hip) used by the C++
// state layer (kv_state.cpp, prefix_cache.cpp).
#pragma once
#include <phaseshift_kv_c.h>
#include <hip/hip_runtime.h>

#include <cstdint>

namespace psk {

// A contiguous device-to-device copy of `bytes` bytes.
struct CopySegment {
    void* dst;
    const void* src;
    uint64_t bytes;
};
constexpr uint32_t kMaxCopySegments = 8;
// Page pairs a copy launch carries in its kernel arguments (2 KB).
constexpr uint32_t kInlinePairs = 256;

// Page pairs of `args` (all layers, K, V and scale rows), in launches of up to
// kInlinePairs pairs.
hipError_t copy_pages_host_pairs(const psk_page_copy_args& args, const psk_page_copy_pair* pairs,
                                 uint32_t n, hipStream_t stream);
// Page pairs (kv may be null when n == 0) and up to kMaxCopySegments segments;
// one launch when n <= kInlinePairs or when device_pairs (room for n pairs,
// owned by the caller, reused only after this launch in stream order) is
// given, else one launch per kInlinePairs pairs.
hipError_t copy_plan_host(const psk_page_copy_args* kv, const psk_page_copy_pair* pairs, uint32_t n,
                          const CopySegment* segs, uint32_t nseg, hipStream_t stream,
                          psk_page_copy_pair* device_pairs = nullptr);
// Zero `bytes` (a multiple of 4) with a fill kernel (no hipMemsetAsync).
hipError_t zero_fill(void* dst, uint64_t bytes, hipStream_t stream);

}  // namespace psk
