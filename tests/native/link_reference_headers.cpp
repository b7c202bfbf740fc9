// Compiled against the REFERENCE's own launcher headers (include path of the
// reference tree) and linked against libphaseshift_kv.so: every launcher the
// reference's dispatchers call must resolve to this library with the same
// C++ signature (mangled name). Built and run by tests/test_link_reference.py.
#include <phaseshift/models/qwen35/kernels/optimized/attention/paged_attention.h>
#include <phaseshift/models/qwen35/kernels/optimized/kv_append.h>

#include <cstdio>

int main() {
    using namespace ps::kernel;
    const void* fns[] = {
        reinterpret_cast<const void*>(&launch_kv_append_bf16),
        reinterpret_cast<const void*>(&launch_kv_append_fp8_e4m3),
        reinterpret_cast<const void*>(&launch_kv_append_psq4),
        reinterpret_cast<const void*>(&launch_kv_append_psq8),
        reinterpret_cast<const void*>(&launch_attention_paged_bf16),
        reinterpret_cast<const void*>(&launch_attention_paged_prefill_bf16),
        reinterpret_cast<const void*>(&launch_attention_paged_prefill_fp8_e4m3),
        reinterpret_cast<const void*>(&launch_attention_paged_fp8_e4m3),
        reinterpret_cast<const void*>(&launch_attention_paged_bf16_split),
        reinterpret_cast<const void*>(&launch_attention_paged_bf16_split_reduce),
        reinterpret_cast<const void*>(&launch_attention_paged_psq4),
        reinterpret_cast<const void*>(&launch_attention_paged_psq8),
        reinterpret_cast<const void*>(&launch_attention_paged_prefill_psq4),
        reinterpret_cast<const void*>(&launch_attention_paged_prefill_psq8),
        reinterpret_cast<const void*>(&launch_attention_paged_psq8_split),
        reinterpret_cast<const void*>(&launch_attention_paged_psq4_split),
        reinterpret_cast<const void*>(&paged_attention_split_reduce_qh_per_wg),
    };
    int missing = 0;
    for (const void* f : fns) missing += f == nullptr;
    // Argument validation happens before any device work: a zero-row call
    // returns hipErrorInvalidValue without touching a GPU.
    KvAppendCommonArgs a{};
    const hipError_t e = launch_kv_append_bf16(a, nullptr, nullptr, nullptr);
    PagedAttentionCommonArgs c{};
    const hipError_t e2 = launch_attention_paged_fp8_e4m3(c, nullptr, nullptr, nullptr, nullptr, nullptr);
    std::printf("launchers %zu missing %d kv_append(rows=0)=%d attention(rows=0)=%d\n",
                sizeof(fns) / sizeof(fns[0]), missing, (int)e, (int)e2);
    return (missing == 0 && e == hipErrorInvalidValue && e2 == hipErrorInvalidValue) ? 0 : 1;
}
