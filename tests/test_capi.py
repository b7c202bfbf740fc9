"""The C-ABI library loads, exports every entry point include/*.h declares, its
structs have the reference's layout, and launchers reject bad arguments the way
the reference's do (hipErrorInvalidValue) — all without touching a GPU."""
import ctypes as C
import os
import re
import subprocess

import pytest

import phaseshift_amd as P

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_c_symbols():
    names = set()
    for dirpath, _, files in os.walk(os.path.join(ROOT, "include")):
        for f in files:
            if f.endswith(".h"):
                txt = open(os.path.join(dirpath, f)).read()
                names |= set(re.findall(r"^\w[\w\s\*]*?\b(psk_\w+)\s*\(", txt, re.M))
    return names


def exported():
    out = subprocess.run(["nm", "-D", "--defined-only", P.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    return {line.split()[-1] for line in out.splitlines() if line.strip()}


def test_library_exports_every_declared_symbol():
    names = declared_c_symbols()
    assert len(names) >= 20
    missing = names - exported()
    assert not missing, missing
    L = P.lib()
    for n in names:
        getattr(L, n)


def test_every_exported_entry_point_has_a_ctypes_prototype():
    """Without a prototype ctypes passes device pointers as 32-bit ints."""
    exported_c = {s for s in exported() if s.startswith("psk_")}
    assert exported_c <= set(P.SIGNATURES), exported_c - set(P.SIGNATURES)
    assert declared_c_symbols() == exported_c
    with pytest.raises(AttributeError):
        P.lib().psk_not_a_function


def test_reference_cpp_launchers_exported():
    syms = exported()
    for name in ["launch_kv_append_bf16", "launch_kv_append_fp8_e4m3",
                 "launch_attention_paged_bf16", "launch_attention_paged_fp8_e4m3",
                 "launch_attention_paged_bf16_split", "launch_attention_paged_bf16_split_reduce",
                 "launch_attention_paged_prefill_bf16", "launch_attention_paged_prefill_fp8_e4m3"]:
        assert any(f"ps6kernel{len(name)}{name}" in s for s in syms), name


def test_struct_layouts():
    assert C.sizeof(P.KvAppendArgs) == 96
    assert P.KvAppendArgs.block_table_stride.offset == 48
    assert P.KvAppendArgs.elems_per_layer.offset == 92
    assert C.sizeof(P.PagedAttentionArgs) == 112
    assert P.PagedAttentionArgs.output_dtype.offset == 16
    assert P.PagedAttentionArgs.q_row_stride.offset == 20
    assert P.PagedAttentionArgs.rows.offset == 64
    assert P.PagedAttentionArgs.scale.offset == 108
    assert C.sizeof(P.RequestDescriptor) == 64
    assert P.RequestDescriptor.execution_class.offset == 28
    assert P.RequestDescriptor.sampling.offset == 32


def test_invalid_arguments_rejected_without_launch():
    L = P.lib()
    a = P.KvAppendArgs()
    assert L.psk_kv_append_bf16(None, None, None, None) == P.HIP_INVALID_VALUE
    assert L.psk_kv_append_bf16(C.byref(a), None, None, None) == P.HIP_INVALID_VALUE
    a.rows, a.head_dim, a.kv_heads, a.page_tokens, a.block_table_stride, a.num_pages = 1, 8, 1, 16, 1, 1
    assert L.psk_kv_append_fp8_e4m3(C.byref(a), 16, 16, None, None, None) == P.HIP_INVALID_VALUE
    b = P.PagedAttentionArgs()
    assert L.psk_attention_paged_bf16(C.byref(b), 16, 16, None) == P.HIP_INVALID_VALUE
    b.rows, b.head_dim, b.q_heads, b.kv_heads = 1, 300, 4, 4   # head_dim > 256
    b.page_tokens, b.block_table_stride, b.num_pages = 16, 1, 1
    b.q = b.output = b.row_sequence_slots = b.row_positions = b.block_tables = 16
    assert L.psk_attention_paged_fp8_e4m3(C.byref(b), 16, 16, 16, 16, None) == P.HIP_INVALID_VALUE
    b.head_dim, b.q_heads = 256, 6                       # q_heads % kv_heads != 0
    assert L.psk_attention_paged_bf16(C.byref(b), 16, 16, None) == P.HIP_INVALID_VALUE
    b.q_heads = 24
    for splits in (0, 3, 32):   # reference split launcher accepts 2, 4, 8, 16
        assert L.psk_attention_paged_bf16_split(C.byref(b), 16, 16, 16, splits, None) == \
            P.HIP_INVALID_VALUE
    assert L.psk_kv_gather(None, None, None, 2, None) == P.HIP_INVALID_VALUE
    assert L.psk_fill_u32(None, 0, 5, None) == P.HIP_INVALID_VALUE
    assert L.psk_fill_u32(None, 0, 0, None) == P.HIP_SUCCESS
    assert L.psk_attention_split_partials_bytes(64, 24, 4, 16) == 64 * 4 * 16 * 6 * 258 * 4


def test_version_and_arch():
    L = P.lib()
    assert L.psk_build_arch() == b"gfx950"
    assert L.psk_version().startswith(b"phaseshift-kv")
