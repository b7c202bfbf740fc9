// Core value types of the paged KV path, with the reference's names and sizes.
//   bf16_t                    reference include/phaseshift/core/memory/types.h:7-9
//   fp8e4m3_storage_t         reference include/phaseshift/models/qwen35/state/kv_cache_types.h:8-9
//   KVCacheDType              reference kv_cache_types.h:11-16
//   PageId / kInvalidPageId   reference include/phaseshift/models/qwen35/state/paged_types.h:9-15
#pragma once
#include <cstdint>
#include <limits>

namespace ps {

struct alignas(2) bf16_t {
    uint16_t data;
};
static_assert(sizeof(bf16_t) == 2);

namespace qwen35 {

using fp8e4m3_storage_t = unsigned char;
static_assert(sizeof(fp8e4m3_storage_t) == 1);

enum class KVCacheDType : uint8_t {
    BF16 = 0,
    FP8_E4M3 = 1,
    PSQ4_W32 = 3,
    PSQ8_W32 = 4,
};

// PSQ KV estimators (kv_cache_types.h:27-30,42-45); PSQ dtypes are declared
// for signature compatibility, their launchers report hipErrorNotSupported.
enum class Psq4ScaleEstimator : uint8_t { MaxAbs = 0, Lsq1 = 1 };
enum class Psq8ScaleEstimator : uint8_t { MaxAbs = 0, Lsq1 = 1 };

using PageId = uint32_t;
using SequenceSlotId = uint32_t;
inline constexpr PageId kInvalidPageId = std::numeric_limits<PageId>::max();
inline constexpr SequenceSlotId kInvalidSlot = std::numeric_limits<SequenceSlotId>::max();

}  // namespace qwen35
}  // namespace ps
