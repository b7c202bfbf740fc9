"""Torch-tensor front of the C-ABI: fills the argument structs from tensors and
calls the HIP library on the current torch stream.

The geometry and argument meaning are the reference's launcher contract
(include/phaseshift/models/qwen35/kernels/optimized/kv_append.h:12-41,
attention/paged_attention.h:42-78); errors surface as HipError carrying the
hipError_t code the launcher returned (hipErrorInvalidValue on bad geometry or
null pointers, hipErrorNotSupported on shapes no kernel handles).
"""
from __future__ import annotations

import ctypes as C
import math
from dataclasses import dataclass

import torch

from . import (KV_BF16, KV_FP8, KV_PSQ4, KV_PSQ8, OUT_BF16, OUT_F32, KvAppendArgs, KvGatherArgs, PageCopyArgs,
               PagedAttentionArgs, RequestDescriptor, check, lib)


@dataclass(frozen=True)
class PoolGeometry:
    """KV pool geometry: [layers][num_pages][page_tokens][kv_heads][head_dim]
    (reference state/paged_kv_pool.cpp:64-75)."""
    num_layers: int
    num_pages: int
    page_tokens: int
    kv_heads: int
    head_dim: int

    @property
    def elems_per_token(self) -> int:
        return self.kv_heads * self.head_dim

    @property
    def elems_per_page(self) -> int:
        return self.page_tokens * self.elems_per_token

    @property
    def elems_per_layer(self) -> int:
        return self.num_pages * self.elems_per_page

    @property
    def pool_elems(self) -> int:
        return self.num_layers * self.elems_per_layer

    @property
    def scale_elems(self) -> int:
        return self.num_layers * self.num_pages * self.page_tokens * self.kv_heads

    # PSQ pools (kv_cache_types.h:16-46): blocks of 32 values of a (token,
    # head) slice; 16 (PSQ4) or 32 (PSQ8) code bytes and one bf16 scale each.
    @property
    def psq_blocks(self) -> int:
        return self.scale_elems * (self.head_dim // 32)

    def psq_code_bytes(self, fmt: int) -> int:
        return self.psq_blocks * (16 if fmt == 4 else 32)


def _ptr(t) -> int | None:
    return None if t is None else t.data_ptr()


def _stream(stream) -> int | None:
    if stream is None:
        return torch.cuda.current_stream().cuda_stream
    return stream.cuda_stream if hasattr(stream, "cuda_stream") else stream


def _check_u32(*ts):
    for t in ts:
        if t is not None and t.dtype not in (torch.int32, torch.uint32):
            raise TypeError("row metadata and block tables must be 32-bit integer tensors")


def _check_append_input(geom: PoolGeometry, k_in, v_in):
    """The launchers read each input row as kv_heads*head_dim packed bf16 values
    (kv_append.hip:21-49): any other dtype, a non-unit inner stride or a short
    row would be read as garbage codes, so reject them here."""
    width = geom.kv_heads * geom.head_dim
    for name, t in (("k_in", k_in), ("v_in", v_in)):
        if t.dtype not in (torch.bfloat16, torch.int16, torch.uint16):
            raise TypeError(f"{name} must hold bf16 values (bfloat16 or its int16 bits), got {t.dtype}")
        if t.dim() != 2 or t.stride(-1) != 1:
            raise ValueError(f"{name} must be a 2-D [rows, >= kv_heads*head_dim] tensor with unit inner stride")
        if t.shape[1] < width or t.stride(0) < width:
            raise ValueError(f"{name} rows must hold kv_heads*head_dim = {width} values")
    if k_in.shape[0] != v_in.shape[0]:
        raise ValueError("k_in and v_in must have the same number of rows")


def append_args(geom: PoolGeometry, layer: int, k_in, v_in, slots, positions, block_tables,
                max_sequences: int | None = None) -> KvAppendArgs:
    _check_u32(slots, positions, block_tables)
    _check_append_input(geom, k_in, v_in)
    a = KvAppendArgs()
    a.k_input, a.v_input = _ptr(k_in), _ptr(v_in)
    a.k_row_stride, a.v_row_stride = k_in.stride(0), v_in.stride(0)
    a.row_sequence_slots, a.row_positions = _ptr(slots), _ptr(positions)
    a.block_tables = _ptr(block_tables)
    a.block_table_stride = block_tables.shape[1]
    a.max_sequences = block_tables.shape[0] if max_sequences is None else max_sequences
    a.rows = k_in.shape[0]
    a.layer = layer
    a.page_tokens, a.num_pages = geom.page_tokens, geom.num_pages
    a.num_attention_layers = geom.num_layers
    a.kv_heads, a.head_dim = geom.kv_heads, geom.head_dim
    a.elems_per_token, a.elems_per_page = geom.elems_per_token, geom.elems_per_page
    a.elems_per_layer = geom.elems_per_layer
    a._tensors = (k_in, v_in, slots, positions, block_tables)   # see attention_args
    return a


def kv_append(geom: PoolGeometry, layer: int, k_in, v_in, slots, positions, block_tables,
              k_pool, v_pool, k_scale=None, v_scale=None, stream=None,
              max_sequences: int | None = None) -> None:
    """launch_kv_append_bf16 / launch_kv_append_fp8_e4m3 (kv_append.h:78-97)."""
    a = append_args(geom, layer, k_in, v_in, slots, positions, block_tables, max_sequences)
    s = _stream(stream)
    if k_pool.dtype == torch.uint8:
        check("psk_kv_append_fp8_e4m3", lib().psk_kv_append_fp8_e4m3(
            C.byref(a), _ptr(k_pool), _ptr(v_pool), _ptr(k_scale), _ptr(v_scale), s))
    else:
        check("psk_kv_append_bf16", lib().psk_kv_append_bf16(
            C.byref(a), _ptr(k_pool), _ptr(v_pool), s))


def kv_append_from_requests(geom: PoolGeometry, layer: int, k_in, v_in, requests_dev,
                            num_requests: int, slots, positions, block_tables, k_pool, v_pool,
                            k_scale=None, v_scale=None, stream=None,
                            max_sequences: int | None = None) -> None:
    """Row metadata (device_batch_context.hip:69-90) and KV append in one
    launch: slots / positions are written for the rows of the requests
    (requests_dev: uint8 device tensor of num_requests RequestDescriptor)."""
    a = append_args(geom, layer, k_in, v_in, slots, positions, block_tables, max_sequences)
    s = _stream(stream)
    if k_pool.dtype == torch.uint8:
        check("psk_kv_append_fp8_e4m3_from_requests", lib().psk_kv_append_fp8_e4m3_from_requests(
            C.byref(a), _ptr(requests_dev), num_requests, _ptr(k_pool), _ptr(v_pool), _ptr(k_scale),
            _ptr(v_scale), s))
    else:
        check("psk_kv_append_bf16_from_requests", lib().psk_kv_append_bf16_from_requests(
            C.byref(a), _ptr(requests_dev), num_requests, _ptr(k_pool), _ptr(v_pool), s))


def attention_args(geom: PoolGeometry, layer: int, q, out, slots, positions, block_tables,
                   q_heads: int, scale: float | None = None,
                   max_sequences: int | None = None) -> PagedAttentionArgs:
    _check_u32(slots, positions, block_tables)
    a = PagedAttentionArgs()
    a.q, a.output = _ptr(q), _ptr(out)
    a.output_dtype = OUT_F32 if out.dtype == torch.float32 else OUT_BF16
    a.q_row_stride, a.output_row_stride = q.stride(0), out.stride(0)
    a.row_sequence_slots, a.row_positions = _ptr(slots), _ptr(positions)
    a.block_tables = _ptr(block_tables)
    a.block_table_stride = block_tables.shape[1]
    a.max_sequences = block_tables.shape[0] if max_sequences is None else max_sequences
    a.rows = q.shape[0]
    a.layer = layer
    a.page_tokens, a.num_pages = geom.page_tokens, geom.num_pages
    a.num_attention_layers = geom.num_layers
    a.q_heads, a.kv_heads, a.head_dim = q_heads, geom.kv_heads, geom.head_dim
    a.elems_per_token, a.elems_per_page = geom.elems_per_token, geom.elems_per_page
    a.elems_per_layer = geom.elems_per_layer
    a.scale = 1.0 / math.sqrt(geom.head_dim) if scale is None else scale
    # the struct holds raw device pointers: keep the tensors alive with it, so
    # a temporary passed here is not freed and its memory handed to another
    # allocation while launches still read it
    a._tensors = (q, out, slots, positions, block_tables)
    return a


def split_partials_bytes(rows: int, q_heads: int, kv_heads: int, splits: int) -> int:
    return int(lib().psk_attention_split_partials_bytes(rows, q_heads, kv_heads, splits))


def choose_decode_split(rows: int, q_heads: int, kv_heads: int, head_dim: int, page_tokens: int,
                        fp8: bool, visible, partial_bytes: int,
                        kv_dtype: int | None = None) -> tuple[int, int]:
    """(splits, pages_per_split) the step planner would use for a decode launch
    over rows with these visible lengths (host sequence of ints). kv_dtype
    (KV_*) overrides fp8."""
    import numpy as np
    a = PagedAttentionArgs()
    a.rows, a.q_heads, a.kv_heads, a.head_dim, a.page_tokens = rows, q_heads, kv_heads, head_dim, page_tokens
    vis = np.ascontiguousarray(np.asarray(visible, dtype=np.uint32))
    sp, pp = C.c_uint32(0), C.c_uint32(0)
    check("psk_choose_decode_split", lib().psk_choose_decode_split(
        C.byref(a), kv_dtype if kv_dtype is not None else (KV_FP8 if fp8 else KV_BF16),
        vis.ctypes.data, int(vis.max()), partial_bytes,
        C.byref(sp), C.byref(pp)))
    return sp.value, pp.value


def paged_attention(geom: PoolGeometry, layer: int, q, out, slots, positions, block_tables,
                    k_pool, v_pool, q_heads: int, k_scale=None, v_scale=None,
                    scale: float | None = None, splits: int = 1, pages_per_split: int = 0,
                    partials=None, stream=None, max_sequences: int | None = None,
                    kind: str = "decode") -> None:
    """Paged attention. splits == 1: launch_attention_paged_{bf16,fp8_e4m3};
    splits > 1: the split kernel into `partials`, then the combine.
    kind == "prefill": launch_attention_paged_prefill_* (multi-row tiles)."""
    a = attention_args(geom, layer, q, out, slots, positions, block_tables, q_heads, scale,
                       max_sequences)
    s = _stream(stream)
    L = lib()
    fp8 = k_pool.dtype == torch.uint8
    if kind == "prefill":
        if fp8:
            check("prefill_fp8", L.psk_attention_paged_prefill_fp8_e4m3(
                C.byref(a), _ptr(k_pool), _ptr(v_pool), _ptr(k_scale), _ptr(v_scale), s))
        else:
            check("prefill_bf16", L.psk_attention_paged_prefill_bf16(
                C.byref(a), _ptr(k_pool), _ptr(v_pool), s))
        return
    if splits <= 1:
        if fp8:
            check("psk_attention_paged_fp8_e4m3", L.psk_attention_paged_fp8_e4m3(
                C.byref(a), _ptr(k_pool), _ptr(v_pool), _ptr(k_scale), _ptr(v_scale), s))
        else:
            check("psk_attention_paged_bf16", L.psk_attention_paged_bf16(
                C.byref(a), _ptr(k_pool), _ptr(v_pool), s))
        return
    need = split_partials_bytes(q.shape[0], q_heads, geom.kv_heads, splits)
    if partials is None or partials.numel() * partials.element_size() < need:
        raise ValueError(f"partials workspace must hold {need} bytes")
    if fp8:
        check("psk_attention_paged_fp8_e4m3_split", L.psk_attention_paged_fp8_e4m3_split(
            C.byref(a), _ptr(k_pool), _ptr(v_pool), _ptr(k_scale), _ptr(v_scale),
            _ptr(partials), splits, pages_per_split, s))
    else:
        check("psk_attention_paged_bf16_split_ex", L.psk_attention_paged_bf16_split_ex(
            C.byref(a), _ptr(k_pool), _ptr(v_pool), _ptr(partials), splits, pages_per_split, s))
    check("psk_attention_paged_split_reduce_ex", L.psk_attention_paged_split_reduce_ex(
        C.byref(a), _ptr(partials), splits, pages_per_split, s))


def kv_append_psq(geom: PoolGeometry, layer: int, k_in, v_in, slots, positions, block_tables,
                  k_code, v_code, k_scale, v_scale, fmt: int, estimator: int = 0, stream=None,
                  max_sequences: int | None = None) -> None:
    """launch_kv_append_psq4 / launch_kv_append_psq8 (kv_append.h:99-123).
    fmt 4 or 8; estimator 0 = MaxAbs, 1 = Lsq1; scale pools are bf16 bits
    (int16/uint16/bfloat16 tensors)."""
    a = append_args(geom, layer, k_in, v_in, slots, positions, block_tables, max_sequences)
    fn = "psk_kv_append_psq4" if fmt == 4 else "psk_kv_append_psq8"
    check(fn, getattr(lib(), fn)(C.byref(a), _ptr(k_code), _ptr(v_code), _ptr(k_scale),
                                 _ptr(v_scale), geom.head_dim // 32, estimator, _stream(stream)))


def paged_attention_psq(geom: PoolGeometry, layer: int, q, out, slots, positions, block_tables,
                        k_code, v_code, k_scale, v_scale, q_heads: int, fmt: int,
                        scale: float | None = None, splits: int = 1, pages_per_split: int = 0,
                        partials=None, stream=None, max_sequences: int | None = None,
                        kind: str = "decode") -> None:
    """Paged attention over PSQ4/PSQ8 pools (paged_attention.h:202-285).
    splits == 1: launch_attention_paged_psq{4,8} (kind "prefill":
    launch_attention_paged_prefill_psq{4,8}); splits > 1: the split kernel
    into `partials`, then the combine."""
    a = attention_args(geom, layer, q, out, slots, positions, block_tables, q_heads, scale,
                       max_sequences)
    s = _stream(stream)
    L = lib()
    bph = geom.head_dim // 32
    ptrs = (_ptr(k_code), _ptr(v_code), _ptr(k_scale), _ptr(v_scale))
    if splits <= 1:
        fn = f"psk_attention_paged_{'prefill_' if kind == 'prefill' else ''}psq{fmt}"
        check(fn, getattr(L, fn)(C.byref(a), *ptrs, bph, s))
        return
    need = split_partials_bytes(q.shape[0], q_heads, geom.kv_heads, splits)
    if partials is None or partials.numel() * partials.element_size() < need:
        raise ValueError(f"partials workspace must hold {need} bytes")
    check("psk_attention_paged_psq_split_ex", L.psk_attention_paged_psq_split_ex(
        C.byref(a), KV_PSQ4 if fmt == 4 else KV_PSQ8, *ptrs, bph, _ptr(partials), splits,
        pages_per_split, s))
    check("psk_attention_paged_split_reduce_ex", L.psk_attention_paged_split_reduce_ex(
        C.byref(a), _ptr(partials), splits, pages_per_split, s))


def kv_gather(geom: PoolGeometry, layer: int, pool, block_tables, seq_slots, seq_offsets,
              out, elem_bytes: int | None = None, elems_per_token: int | None = None,
              elems_per_page: int | None = None, max_sequences: int | None = None,
              stream=None) -> None:
    """psk_kv_gather: paged pool -> out[token][elems_per_token]."""
    _check_u32(block_tables, seq_slots, seq_offsets)
    a = KvGatherArgs()
    a.block_tables, a.seq_slots, a.seq_token_offsets = (
        _ptr(block_tables), _ptr(seq_slots), _ptr(seq_offsets))
    a.block_table_stride = block_tables.shape[1]
    a.max_sequences = block_tables.shape[0] if max_sequences is None else max_sequences
    a.num_seqs = seq_slots.shape[0]
    a.total_tokens = out.shape[0]
    a.layer = layer
    a.page_tokens, a.num_pages = geom.page_tokens, geom.num_pages
    a.kv_heads, a.head_dim = geom.kv_heads, geom.head_dim
    ept = elems_per_token or geom.elems_per_token
    epp = elems_per_page or geom.page_tokens * ept
    a.elems_per_token, a.elems_per_page = ept, epp
    a.elems_per_layer = epp * geom.num_pages
    eb = elem_bytes or pool.element_size()
    check("psk_kv_gather", lib().psk_kv_gather(C.byref(a), _ptr(pool), _ptr(out), eb,
                                               _stream(stream)))


def copy_pages(geom: PoolGeometry, dst: dict, src: dict, pairs, src_num_pages: int | None = None,
               stream=None) -> None:
    """psk_kv_copy_pages: pairs is an int32 device tensor [n, 2] of (dst_page, src_page)."""
    a = PageCopyArgs()
    a.dst_k, a.dst_v = _ptr(dst["k"]), _ptr(dst["v"])
    a.dst_k_scale, a.dst_v_scale = _ptr(dst.get("k_scale")), _ptr(dst.get("v_scale"))
    a.src_k, a.src_v = _ptr(src["k"]), _ptr(src["v"])
    a.src_k_scale, a.src_v_scale = _ptr(src.get("k_scale")), _ptr(src.get("v_scale"))
    a.pairs = _ptr(pairs)
    a.num_pairs = pairs.shape[0]
    a.num_layers = geom.num_layers
    a.dst_num_pages = geom.num_pages
    a.src_num_pages = geom.num_pages if src_num_pages is None else src_num_pages
    a.page_tokens, a.kv_heads, a.head_dim = geom.page_tokens, geom.kv_heads, geom.head_dim
    a.kv_dtype = KV_FP8 if dst["k"].dtype == torch.uint8 else KV_BF16
    check("psk_kv_copy_pages", lib().psk_kv_copy_pages(C.byref(a), _stream(stream)))


def fill_u32(dst, value: int, stream=None) -> None:
    check("psk_fill_u32", lib().psk_fill_u32(_ptr(dst), value & 0xFFFFFFFF, dst.numel(),
                                             _stream(stream)))


def prepare_row_metadata(requests_dev, num_requests: int, actual_rows: int, slots, positions,
                         stream=None) -> None:
    """requests_dev: uint8 device tensor holding num_requests RequestDescriptor (64 B each)."""
    check("psk_prepare_row_metadata", lib().psk_prepare_row_metadata(
        _ptr(requests_dev), num_requests, actual_rows, _ptr(slots), _ptr(positions),
        _stream(stream)))


def pack_requests(descs: list[dict]) -> bytes:
    arr = (RequestDescriptor * len(descs))()
    for i, d in enumerate(descs):
        for k, v in d.items():
            setattr(arr[i], k, v)
        if "output_index" not in d:
            arr[i].output_index = 0xFFFFFFFF
    return bytes(arr)
