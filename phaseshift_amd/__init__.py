"""phaseshift_amd — MI355X (gfx950) paged KV-cache hot path of PhaseShift qwen35.

The product is the HIP library ``libphaseshift_kv.so`` behind the C-ABI of
``include/phaseshift_kv_c.h``. This package loads it with ctypes and offers
torch-tensor helpers (torch provides device memory and streams only). There is
no fallback: if the library is missing, importing the ops raises.
"""
from __future__ import annotations

import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libphaseshift_kv.so")

PSK_INVALID_PAGE_ID = 0xFFFFFFFF
KV_BF16, KV_FP8 = 0, 1
KV_PSQ4, KV_PSQ8 = 3, 4   # KVCacheDType PSQ4_W32 / PSQ8_W32
OUT_BF16, OUT_F32 = 0, 1
HIP_SUCCESS, HIP_INVALID_VALUE, HIP_NOT_SUPPORTED = 0, 1, 801


class KvAppendArgs(C.Structure):
    """psk_kv_append_args == ps::kernel::KvAppendCommonArgs (96 B)."""
    _fields_ = [("k_input", C.c_void_p), ("v_input", C.c_void_p),
                ("k_row_stride", C.c_uint32), ("v_row_stride", C.c_uint32),
                ("row_sequence_slots", C.c_void_p), ("row_positions", C.c_void_p),
                ("block_tables", C.c_void_p)] + [
        (n, C.c_uint32) for n in (
            "block_table_stride", "max_sequences", "rows", "layer", "page_tokens",
            "num_pages", "num_attention_layers", "kv_heads", "head_dim",
            "elems_per_token", "elems_per_page", "elems_per_layer")]


class PagedAttentionArgs(C.Structure):
    """psk_paged_attention_args == ps::kernel::PagedAttentionCommonArgs (112 B)."""
    _fields_ = [("q", C.c_void_p), ("output", C.c_void_p), ("output_dtype", C.c_uint8),
                ("q_row_stride", C.c_uint32), ("output_row_stride", C.c_uint32),
                ("row_sequence_slots", C.c_void_p), ("row_positions", C.c_void_p),
                ("block_tables", C.c_void_p)] + [
        (n, C.c_uint32) for n in (
            "block_table_stride", "max_sequences", "rows", "layer", "page_tokens",
            "num_pages", "num_attention_layers", "q_heads", "kv_heads", "head_dim",
            "elems_per_token", "elems_per_page", "elems_per_layer")] + [("scale", C.c_float)]


class KvGatherArgs(C.Structure):
    _fields_ = [("block_tables", C.c_void_p), ("seq_slots", C.c_void_p),
                ("seq_token_offsets", C.c_void_p)] + [
        (n, C.c_uint32) for n in (
            "block_table_stride", "max_sequences", "num_seqs", "total_tokens", "layer",
            "page_tokens", "num_pages", "kv_heads", "head_dim", "elems_per_token",
            "elems_per_page", "elems_per_layer")]


class PageCopyArgs(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in (
        "dst_k", "dst_v", "dst_k_scale", "dst_v_scale", "src_k", "src_v", "src_k_scale",
        "src_v_scale", "pairs")] + [
        (n, C.c_uint32) for n in (
            "num_pairs", "num_layers", "dst_num_pages", "src_num_pages", "page_tokens",
            "kv_heads", "head_dim", "kv_dtype")]


class PoolInfo(C.Structure):
    _fields_ = [("k_pool", C.c_void_p), ("v_pool", C.c_void_p), ("k_scale_pool", C.c_void_p),
                ("v_scale_pool", C.c_void_p)] + [
        (n, C.c_uint32) for n in ("num_pages", "page_tokens", "num_layers", "kv_heads", "head_dim",
                                  "kv_dtype", "free_pages", "used_pages")] + [
        ("reserved_bytes", C.c_uint64)]


class SequenceInfo(C.Structure):
    _fields_ = [(n, C.c_uint32) for n in ("slot", "generation", "position", "max_seq_len",
                                          "num_blocks", "poisoned")]


class StepRequest(C.Structure):
    _fields_ = [("row_begin", C.c_uint32), ("row_count", C.c_uint32),
                ("execution_class", C.c_uint8), ("reserved", C.c_uint8 * 3),
                ("max_visible", C.c_uint32)]


class PlannedKernel(C.Structure):
    _fields_ = [(n, C.c_uint32) for n in ("kind", "row_begin", "rows", "splits", "pages_per_split",
                                          "side")]


class StepPlan(C.Structure):
    _fields_ = [("count", C.c_uint32), ("kernels", PlannedKernel * 16)]


class GdnLayout(C.Structure):
    """psk_gdn_layout == GdnStatePoolLayout (gdn_state_pool.h:41-50)."""
    _fields_ = [(n, C.c_uint32) for n in ("num_gdn_states", "conv_dim", "conv_dim_padded",
                                          "conv_history", "conv_history_stride", "num_v_heads",
                                          "head_k", "head_v")]


class GdnPoolInfo(C.Structure):
    _fields_ = [("conv_base", C.c_void_p), ("recurrent_base", C.c_void_p),
                ("conv_slot_bytes", C.c_uint64), ("recurrent_slot_bytes", C.c_uint64),
                ("reserved_bytes", C.c_uint64), ("max_sequences", C.c_uint32),
                ("used_slots", C.c_uint32)]


class DFlashContext(C.Structure):
    _fields_ = [("k_ring", C.c_void_p), ("v_ring", C.c_void_p), ("ring_bytes", C.c_uint64),
                ("length", C.c_uint32), ("next_position", C.c_uint32)]


class CheckpointInfo(C.Structure):
    _fields_ = [("id", C.c_uint64), ("last_used", C.c_uint64)] + [
        (n, C.c_uint32) for n in ("position", "num_pages", "cache_state_slot", "dflash")]


class PrefixCacheStats(C.Structure):
    _fields_ = [(n, C.c_uint64) for n in (
        "lookups", "hits", "misses", "inserts", "duplicate_hits", "evictions", "skipped_too_large",
        "restored_tokens", "saved_tokens", "save_d2d_bytes", "restore_d2d_bytes", "copy_launches",
        "cache_kv_bytes", "cache_gdn_bytes", "dflash_ring_bytes")] + [
        (n, C.c_uint32) for n in ("size", "cache_pages", "cache_free_pages", "cache_free_slots",
                                  "max_entries", "capacity_tokens")]


class StepGraphStats(C.Structure):
    _fields_ = [(n, C.c_uint64) for n in ("eager", "captures", "replays", "evictions")] + [
        ("entries", C.c_uint32), ("graphs", C.c_uint32)]


PSK_ERR = {1001: "invalid_argument", 1002: "out_of_range", 1003: "invalid_state",
           1004: "insufficient_memory", 1005: "hip_error"}
PLAN_ONLY = C.c_void_p(~0 & 0xFFFFFFFFFFFFFFFF)


class RequestDescriptor(C.Structure):
    """psk_request_descriptor == ps::runtime::DeviceRequestDescriptor (64 B)."""
    _fields_ = [("slot", C.c_uint32), ("generation", C.c_uint32), ("row_begin", C.c_uint32),
                ("row_count", C.c_uint32), ("prefix_length", C.c_uint32),
                ("sequence_length", C.c_uint32), ("output_index", C.c_uint32),
                ("execution_class", C.c_uint8), ("compute_logits", C.c_uint8),
                ("output_count", C.c_uint8), ("reserved0", C.c_uint8),
                ("sampling", C.c_uint8 * 32)]


assert C.sizeof(KvAppendArgs) == 96
assert C.sizeof(PagedAttentionArgs) == 112
assert PagedAttentionArgs.scale.offset == 108 and PagedAttentionArgs.output_dtype.offset == 16
assert C.sizeof(RequestDescriptor) == 64

_P = C.c_void_p
_U32 = C.c_uint32
# name -> argtypes (restype int unless listed in _RESTYPE)
SIGNATURES = {
    "psk_kv_append_bf16": [_P, _P, _P, _P],
    "psk_kv_append_fp8_e4m3": [_P, _P, _P, _P, _P, _P],
    "psk_kv_append_bf16_from_requests": [_P, _P, _U32, _P, _P, _P],
    "psk_kv_append_fp8_e4m3_from_requests": [_P, _P, _U32, _P, _P, _P, _P, _P],
    "psk_attention_paged_bf16": [_P, _P, _P, _P],
    "psk_attention_paged_fp8_e4m3": [_P, _P, _P, _P, _P, _P],
    "psk_attention_paged_bf16_split": [_P, _P, _P, _P, _U32, _P],
    "psk_attention_paged_bf16_split_reduce": [_P, _P, _U32, _P],
    "psk_attention_paged_fp8_e4m3_split": [_P, _P, _P, _P, _P, _P, _U32, _U32, _P],
    "psk_attention_paged_fp8_e4m3_split_noalloc": [_P, _P, _P, _P, _P, _U32, _U32, _P],
    "psk_attention_paged_bf16_split_ex": [_P, _P, _P, _P, _U32, _U32, _P],
    "psk_attention_paged_split_reduce_ex": [_P, _P, _U32, _U32, _P],
    "psk_attention_split_partials_bytes": [_U32, _U32, _U32, _U32],
    "psk_attention_paged_prefill_bf16": [_P, _P, _P, _P],
    "psk_attention_paged_prefill_fp8_e4m3": [_P, _P, _P, _P, _P, _P],
    "psk_attention_paged_tile_split": [_P, _U32, _P, _P, _P, _P, _P, _U32, _U32, _P],
    "psk_kv_append_psq4": [_P, _P, _P, _P, _P, _U32, _U32, _P],
    "psk_kv_append_psq8": [_P, _P, _P, _P, _P, _U32, _U32, _P],
    "psk_attention_paged_psq4": [_P, _P, _P, _P, _P, _U32, _P],
    "psk_attention_paged_psq8": [_P, _P, _P, _P, _P, _U32, _P],
    "psk_attention_paged_prefill_psq4": [_P, _P, _P, _P, _P, _U32, _P],
    "psk_attention_paged_prefill_psq8": [_P, _P, _P, _P, _P, _U32, _P],
    "psk_attention_paged_psq4_split": [_P, _P, _P, _P, _P, _U32, _P, _U32, _P],
    "psk_attention_paged_psq8_split": [_P, _P, _P, _P, _P, _U32, _P, _U32, _P],
    "psk_attention_paged_psq": [_P, _U32, _P, _P, _P, _P, _U32, _P],
    "psk_attention_paged_psq_split_ex": [_P, _U32, _P, _P, _P, _P, _U32, _P, _U32, _U32, _P],
    "psk_kv_gather": [_P, _P, _P, _U32, _P],
    "psk_kv_copy_pages": [_P, _P],
    "psk_fill_u32": [_P, _U32, C.c_uint64, _P],
    "psk_prepare_row_metadata": [_P, _U32, _U32, _P, _P, _P],
    "psk_last_error_message": [],
    "psk_pool_create": [_P, _U32, _U32, _U32, _U32, _U32, _U32],
    "psk_pool_destroy": [_P],
    "psk_pool_info": [_P, _P],
    "psk_pool_allocate": [_P, _P],
    "psk_pool_release": [_P, _U32],
    "psk_pool_copy_pages": [_P, _P, _P, _P, _U32, _P],
    "psk_slot_pool_create": [_P, _U32, _U32, _P],
    "psk_slot_pool_destroy": [_P],
    "psk_slot_pool_block_tables": [_P],
    "psk_sequence_create": [_P, _P, _P, _U32, _P],
    "psk_sequence_release": [_P, _P],
    "psk_sequence_reserve": [_P, _U32, _P],
    "psk_sequence_rollback": [_P, _U32, _P],
    "psk_sequence_commit": [_P, _U32],
    "psk_sequence_info": [_P, _P],
    "psk_sequence_block_table": [_P, _P, _U32],
    "psk_gdn_layout_make": [_U32, _U32, _U32, _U32, _U32, _U32, _P],
    "psk_gdn_pool_create": [_P, _U32, _P],
    "psk_gdn_pool_destroy": [_P],
    "psk_gdn_pool_info": [_P, _P],
    "psk_gdn_pool_initialize": [_P, _U32, _P],
    "psk_gdn_pool_reset": [_P, _U32, _P],
    "psk_gdn_pool_release": [_P, _U32],
    "psk_gdn_pool_copy_slot": [_P, _U32, _P, _U32, _P],
    "psk_prefix_cache_create": [_P, _P, _P, _U32, _U32, _U32],
    "psk_prefix_cache_destroy": [_P],
    "psk_prefix_cache_enable_dflash_ring": [_P, C.c_uint64],
    "psk_prefix_cache_find_longest": [_P, _P, _U32, _U32, _P],
    "psk_prefix_cache_save": [_P, _P, _P, _P, _P, _U32, _U32, _P, _P],
    "psk_prefix_cache_restore": [_P, _P, _P, _P, C.c_uint64, _P, _P],
    "psk_prefix_cache_clear": [_P],
    "psk_prefix_cache_stats": [_P, _P],
    "psk_paged_attention_step": [_P, _U32, _P, _P, _P, _P, _P, _U32, _U32, _P, C.c_uint64, _P, _P],
    "psk_step_graph_cache_create": [_P, _U32],
    "psk_step_graph_cache_destroy": [_P],
    "psk_step_graph_cache_stats": [_P, _P],
    "psk_paged_attention_step_graphed": [_P, _P, _U32, _P, _P, _P, _P, _P, _U32, _U32, _P,
                                         C.c_uint64, _P, _P, _P],
    "psk_paged_attention_plan_signature": [_P, _U32, _P, _P, _P, _P, _P, _U32, _U32, _P,
                                           C.c_uint64],
    "psk_choose_decode_split": [_P, _U32, _P, _U32, C.c_uint64, _P, _P],
    "psk_selftest_e4m3_encode_range": [_U32, _U32, _P, _P],
    "psk_selftest_e4m3_decode_all": [_P, _P],
    "psk_version": [],
    "psk_build_arch": [],
    "psk_error_string": [C.c_int],
}
_RESTYPE = {
    "psk_last_error_message": C.c_char_p,
    "psk_pool_destroy": None,
    "psk_gdn_pool_destroy": None,
    "psk_prefix_cache_destroy": None,
    "psk_step_graph_cache_destroy": None,
    "psk_paged_attention_plan_signature": C.c_uint64,
    "psk_slot_pool_destroy": None,
    "psk_slot_pool_block_tables": C.c_void_p,
    "psk_sequence_block_table": C.c_uint32,
    "psk_attention_split_partials_bytes": C.c_uint64,
    "psk_version": C.c_char_p,
    "psk_build_arch": C.c_char_p,
    "psk_error_string": C.c_char_p,
}

_lib = None


class _Lib:
    """The C-ABI with a ctypes prototype on every entry point. Only functions
    listed in SIGNATURES are reachable: a call without a prototype would pass
    64-bit device pointers as 32-bit ints."""

    def __init__(self, cdll: C.CDLL):
        self._cdll = cdll
        for name, argt in SIGNATURES.items():
            f = getattr(cdll, name)
            f.argtypes = argt
            f.restype = _RESTYPE.get(name, C.c_int)
            setattr(self, name, f)

    def __getattr__(self, name):
        raise AttributeError(f"{name} has no ctypes prototype in phaseshift_amd.SIGNATURES")


def lib() -> _Lib:
    """The loaded HIP library. Raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"{LIB_PATH} is missing: build it with `python -m phaseshift_amd.build` "
                "(no CPU fallback exists)")
        _lib = _Lib(C.CDLL(LIB_PATH))
    return _lib


class HipError(RuntimeError):
    def __init__(self, fn: str, code: int):
        name = lib().psk_error_string(code).decode()
        super().__init__(f"{fn} returned {code} ({name})")
        self.code = code


def check(fn: str, code: int) -> None:
    if code != HIP_SUCCESS:
        raise HipError(fn, code)


class StateError(RuntimeError):
    """A PSK_ERR_* status of the host-state entry points (reference Status codes)."""

    def __init__(self, fn: str, code: int):
        msg = lib().psk_last_error_message().decode()
        super().__init__(f"{fn}: {PSK_ERR.get(code, code)}: {msg}")
        self.code = code
        self.kind = PSK_ERR.get(code, "hip_error")


def check_state(fn: str, code: int) -> None:
    if code != 0:
        raise StateError(fn, code)
