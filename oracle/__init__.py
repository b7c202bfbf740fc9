"""CPU oracle of the paged KV-cache path — TEST INFRASTRUCTURE ONLY.

Python (ctypes + numpy) front of ``ps_oracle.c``. Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg import this
package; the product (``phaseshift_amd``) never does and fails loudly without
its HIP library.

Each wrapper names the C function it calls; the C source cites the reference
file:line each one restates.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libps_oracle.so")
REF_LIB_PATH = os.path.join(HERE, "_ref", "libref_codec.so")

_u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")


def build(force: bool = False) -> None:
    """Compile ps_oracle.c (and oracle/_ref when the reference tree exists)."""
    targets = ["all"]
    if os.path.isdir("/root/reference/src"):
        targets.append("ref")
    args = ["make", "-s", "-C", HERE] + (["-B"] if force else []) + targets
    subprocess.run(args, check=True)


_lib = None
_ref = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        _lib = C.CDLL(LIB_PATH)
        L = _lib
        L.or_f32_to_bf16.restype = C.c_uint16
        L.or_f32_to_bf16.argtypes = [C.c_float]
        L.or_e4m3_encode.restype = C.c_uint8
        L.or_e4m3_encode.argtypes = [C.c_float]
        L.or_e4m3_decode.restype = C.c_float
        L.or_e4m3_decode.argtypes = [C.c_uint8]
        L.or_e4m3_encode_range.argtypes = [C.c_uint32, C.c_uint32, _u8p]
        L.or_e4m3_encode_array.argtypes = [_f32p, _u8p, C.c_uint64]
        L.or_e4m3_decode_array.argtypes = [_u8p, _f32p, C.c_uint64]
        L.or_f32_to_bf16_array.argtypes = [_f32p, _u16p, C.c_uint64]
        for name in ("or_kv_append_bf16", "or_kv_append_fp8", "or_kv_gather",
                     "or_paged_attention", "or_split_reduce", "or_copy_page",
                     "or_kv_append_psq", "or_paged_attention_psq"):
            getattr(L, name).restype = None
        L.or_psq_bf16_round_array.argtypes = [_f32p, _f32p, C.c_uint64]
        L.or_cb10_encode_array.argtypes = [_f32p, _f32p, _u8p, C.c_uint64]
        L.or_cb10_decode.restype = C.c_float
        L.or_cb10_decode.argtypes = [C.c_uint8]
        L.or_psq_encode_block.restype = None
        L.or_psq_encode_block.argtypes = [_f32p, C.c_uint32, C.c_uint32, C.c_uint32, _u16p, _u8p]
    return _lib


def ref_lib():
    """The reference's own e4m3.cpp / f32_to_bf16_rne, or None if not built."""
    global _ref
    if _ref is None and os.path.exists(REF_LIB_PATH):
        _ref = C.CDLL(REF_LIB_PATH)
        _ref.ref_e4m3_encode_range.argtypes = [C.c_uint32, C.c_uint32, _u8p]
        _ref.ref_e4m3_decode_all.argtypes = [_f32p]
        _ref.ref_f32_to_bf16_range.argtypes = [C.c_uint32, C.c_uint32, _u16p]
        _ref.ref_psq4_encode_block.argtypes = [_f32p, C.c_uint32, _f32p, _u8p]
        _ref.ref_psq4_pack_codes.argtypes = [_u8p, _u8p]
        _ref.ref_psq8_encode_block.argtypes = [_f32p, C.c_uint32, _f32p, _u8p]
        _ref.ref_psq_bf16_round_array.argtypes = [_f32p, _f32p, C.c_uint64]
        _ref.ref_cb10_encode_array.argtypes = [_f32p, _f32p, _u8p, C.c_uint64]
        _ref.ref_cb10_code_to_f32.restype = C.c_float
        _ref.ref_cb10_code_to_f32.argtypes = [C.c_uint8]
    return _ref


# --------------------------------------------------------------------- codecs
def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    """or_f32_to_bf16 (types.h:11-21) over an array -> uint16 bit patterns."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().or_f32_to_bf16_array(x.reshape(-1), out.reshape(-1), x.size)
    return out


def bf16_to_f32(h: np.ndarray) -> np.ndarray:
    return (np.asarray(h, np.uint16).astype(np.uint32) << 16).view(np.float32)


def e4m3_encode(x: np.ndarray) -> np.ndarray:
    """or_e4m3_encode (SATFINITE RNE) over an array."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, np.uint8)
    lib().or_e4m3_encode_array(x.reshape(-1), out.reshape(-1), x.size)
    return out


def e4m3_decode(c: np.ndarray) -> np.ndarray:
    c = np.ascontiguousarray(c, dtype=np.uint8)
    out = np.empty(c.shape, np.float32)
    lib().or_e4m3_decode_array(c.reshape(-1), out.reshape(-1), c.size)
    return out


# ---------------------------------------------------------------- PSQ codecs
def psq_bf16_round(x: np.ndarray) -> np.ndarray:
    """or_psq_bf16_round (psq4_kv.h:9-18) over an array."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, np.float32)
    lib().or_psq_bf16_round_array(x.reshape(-1), out.reshape(-1), x.size)
    return out


def cb10_encode(x: np.ndarray, inv_scale) -> np.ndarray:
    """or_cb10_encode (psq_device.h:22-35) elementwise."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    inv = np.ascontiguousarray(np.broadcast_to(np.float32(inv_scale), x.shape), dtype=np.float32)
    out = np.empty(x.shape, np.uint8)
    lib().or_cb10_encode_array(x.reshape(-1), inv.reshape(-1), out.reshape(-1), x.size)
    return out


def cb10_decode(c: np.ndarray) -> np.ndarray:
    L = lib()
    return np.array([L.or_cb10_decode(int(v)) for v in np.asarray(c).reshape(-1)],
                    np.float32).reshape(np.shape(c))


def psq_encode_block(x: np.ndarray, fmt: int, lsq1: bool, device_order: bool = True):
    """or_psq_encode_block: 32 floats -> (bf16 scale bits, 32 unpacked codes)."""
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(32)
    sb = np.zeros(1, np.uint16)
    codes = np.zeros(32, np.uint8)
    lib().or_psq_encode_block(x, fmt, int(lsq1), int(device_order), sb, codes)
    return int(sb[0]), codes


# --------------------------------------------------------------- arg structs
def _p(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


class _AppendArgs(C.Structure):
    _fields_ = [("k_input", C.c_void_p), ("v_input", C.c_void_p),
                ("k_row_stride", C.c_uint32), ("v_row_stride", C.c_uint32),
                ("row_sequence_slots", C.c_void_p), ("row_positions", C.c_void_p),
                ("block_tables", C.c_void_p)] + [
        (n, C.c_uint32) for n in (
            "block_table_stride", "max_sequences", "rows", "layer", "page_tokens",
            "num_pages", "num_attention_layers", "kv_heads", "head_dim",
            "elems_per_token", "elems_per_page", "elems_per_layer")]


class _GatherArgs(C.Structure):
    _fields_ = [("block_tables", C.c_void_p), ("seq_slots", C.c_void_p),
                ("seq_token_offsets", C.c_void_p)] + [
        (n, C.c_uint32) for n in (
            "block_table_stride", "max_sequences", "num_seqs", "total_tokens", "layer",
            "page_tokens", "num_pages", "kv_heads", "head_dim", "elems_per_token",
            "elems_per_page", "elems_per_layer")]


class _AttnArgs(C.Structure):
    _fields_ = [("q", C.c_void_p), ("output", C.c_void_p), ("output_dtype", C.c_uint32),
                ("q_row_stride", C.c_uint32), ("output_row_stride", C.c_uint32),
                ("row_sequence_slots", C.c_void_p), ("row_positions", C.c_void_p),
                ("block_tables", C.c_void_p)] + [
        (n, C.c_uint32) for n in (
            "block_table_stride", "max_sequences", "rows", "layer", "page_tokens",
            "num_pages", "num_attention_layers", "q_heads", "kv_heads", "head_dim",
            "elems_per_token", "elems_per_page", "elems_per_layer")] + [("scale", C.c_float)]


def _u32(a):
    return np.ascontiguousarray(a, dtype=np.uint32)


# ------------------------------------------------------------------ KV append
def kv_append(geom: dict, k_in: np.ndarray, v_in: np.ndarray, slots, positions,
              block_tables: np.ndarray, k_pool: np.ndarray, v_pool: np.ndarray,
              k_scale: np.ndarray | None = None, v_scale: np.ndarray | None = None) -> None:
    """In place: or_kv_append_bf16 (uint16 pools) or or_kv_append_fp8 (uint8 pools).

    geom keys: layer, page_tokens, num_pages, num_attention_layers, kv_heads,
    head_dim, block_table_stride, max_sequences. k_in/v_in: uint16 [rows, stride].
    """
    k_in = np.ascontiguousarray(k_in, np.uint16)
    v_in = np.ascontiguousarray(v_in, np.uint16)
    slots, positions, bt = _u32(slots), _u32(positions), _u32(block_tables)
    a = _AppendArgs()
    a.k_input, a.v_input = _p(k_in), _p(v_in)
    a.k_row_stride, a.v_row_stride = k_in.shape[1], v_in.shape[1]
    a.row_sequence_slots, a.row_positions, a.block_tables = _p(slots), _p(positions), _p(bt)
    a.rows = k_in.shape[0]
    for n in ("block_table_stride", "max_sequences", "layer", "page_tokens", "num_pages",
              "num_attention_layers", "kv_heads", "head_dim"):
        setattr(a, n, geom[n])
    ept = geom["kv_heads"] * geom["head_dim"]
    a.elems_per_token, a.elems_per_page = ept, ept * geom["page_tokens"]
    a.elems_per_layer = a.elems_per_page * geom["num_pages"]
    if k_pool.dtype == np.uint16:
        lib().or_kv_append_bf16(C.byref(a), _p(k_pool), _p(v_pool))
    else:
        lib().or_kv_append_fp8(C.byref(a), _p(k_pool), _p(v_pool), _p(k_scale), _p(v_scale))


def kv_append_psq(geom: dict, k_in: np.ndarray, v_in: np.ndarray, slots, positions,
                  block_tables: np.ndarray, k_code: np.ndarray, v_code: np.ndarray,
                  k_scale: np.ndarray, v_scale: np.ndarray, fmt: int, lsq1: bool,
                  device_order: bool = True) -> None:
    """In place: or_kv_append_psq. Code pools uint8 [blocks*16|32], scale
    pools uint16 (bf16 bits) [blocks]; geom as kv_append."""
    k_in = np.ascontiguousarray(k_in, np.uint16)
    v_in = np.ascontiguousarray(v_in, np.uint16)
    slots, positions, bt = _u32(slots), _u32(positions), _u32(block_tables)
    a = _AppendArgs()
    a.k_input, a.v_input = _p(k_in), _p(v_in)
    a.k_row_stride, a.v_row_stride = k_in.shape[1], v_in.shape[1]
    a.row_sequence_slots, a.row_positions, a.block_tables = _p(slots), _p(positions), _p(bt)
    a.rows = k_in.shape[0]
    for n in ("block_table_stride", "max_sequences", "layer", "page_tokens", "num_pages",
              "num_attention_layers", "kv_heads", "head_dim"):
        setattr(a, n, geom[n])
    lib().or_kv_append_psq(C.byref(a), C.c_uint32(fmt), C.c_uint32(int(lsq1)),
                           C.c_uint32(int(device_order)), _p(k_code), _p(v_code), _p(k_scale),
                           _p(v_scale))


def kv_gather(geom: dict, pool: np.ndarray, block_tables, seq_slots, seq_lengths,
              elems_per_token: int | None = None, elems_per_page: int | None = None,
              out: np.ndarray | None = None) -> np.ndarray:
    """or_kv_gather: pool (any dtype) -> [total_tokens, elems_per_token]."""
    seq_slots = _u32(seq_slots)
    offs = _u32(np.concatenate([[0], np.cumsum(seq_lengths)]))
    bt = _u32(block_tables)
    ept = elems_per_token or geom["kv_heads"] * geom["head_dim"]
    epp = elems_per_page or ept * geom["page_tokens"]
    total = int(offs[-1])
    if out is None:
        out = np.zeros((total, ept), pool.dtype)
    a = _GatherArgs()
    a.block_tables, a.seq_slots, a.seq_token_offsets = _p(bt), _p(seq_slots), _p(offs)
    a.num_seqs, a.total_tokens = len(seq_slots), total
    for n in ("block_table_stride", "max_sequences", "layer", "page_tokens", "num_pages",
              "kv_heads", "head_dim"):
        setattr(a, n, geom[n])
    a.elems_per_token, a.elems_per_page = ept, epp
    a.elems_per_layer = epp * geom["num_pages"]
    lib().or_kv_gather(C.byref(a), _p(np.ascontiguousarray(pool)), _p(out),
                       C.c_uint32(pool.dtype.itemsize))
    return out


# ------------------------------------------------------------------ attention
def paged_attention(geom: dict, q: np.ndarray, slots, positions, block_tables,
                    k_pool, v_pool, k_scale=None, v_scale=None, scale=None,
                    output_dtype: str = "f32", out: np.ndarray | None = None) -> np.ndarray:
    """or_paged_attention: fp32 two-pass softmax. q: uint16 [rows, q_row_stride]."""
    q = np.ascontiguousarray(q, np.uint16)
    rows = q.shape[0]
    H, D = geom["q_heads"], geom["head_dim"]
    if out is None:
        out = np.zeros((rows, H * D), np.float32 if output_dtype == "f32" else np.uint16)
    slots, positions, bt = _u32(slots), _u32(positions), _u32(block_tables)
    a = _AttnArgs()
    a.q, a.output = _p(q), _p(out)
    a.output_dtype = 1 if out.dtype == np.float32 else 0
    a.q_row_stride, a.output_row_stride = q.shape[1], out.shape[1]
    a.row_sequence_slots, a.row_positions, a.block_tables = _p(slots), _p(positions), _p(bt)
    a.rows = rows
    for n in ("block_table_stride", "max_sequences", "layer", "page_tokens", "num_pages",
              "num_attention_layers", "q_heads", "kv_heads", "head_dim"):
        setattr(a, n, geom[n])
    ept = geom["kv_heads"] * D
    a.elems_per_token, a.elems_per_page = ept, ept * geom["page_tokens"]
    a.elems_per_layer = a.elems_per_page * geom["num_pages"]
    a.scale = float(scale if scale is not None else 1.0 / np.sqrt(D))
    fp8 = k_pool.dtype == np.uint8
    lib().or_paged_attention(C.byref(a), C.c_uint32(1 if fp8 else 0),
                             _p(np.ascontiguousarray(k_pool)), _p(np.ascontiguousarray(v_pool)),
                             _p(k_scale), _p(v_scale))
    return out


def paged_attention_psq(geom: dict, q: np.ndarray, slots, positions, block_tables, k_code,
                        v_code, k_scale, v_scale, fmt: int, scale=None,
                        output_dtype: str = "f32", out: np.ndarray | None = None) -> np.ndarray:
    """or_paged_attention_psq: every K/V value dequantised (bf16 block scale x
    codebook value) in fp32, then the two-pass fp32 softmax."""
    q = np.ascontiguousarray(q, np.uint16)
    rows = q.shape[0]
    H, D = geom["q_heads"], geom["head_dim"]
    if out is None:
        out = np.zeros((rows, H * D), np.float32 if output_dtype == "f32" else np.uint16)
    slots, positions, bt = _u32(slots), _u32(positions), _u32(block_tables)
    a = _AttnArgs()
    a.q, a.output = _p(q), _p(out)
    a.output_dtype = 1 if out.dtype == np.float32 else 0
    a.q_row_stride, a.output_row_stride = q.shape[1], out.shape[1]
    a.row_sequence_slots, a.row_positions, a.block_tables = _p(slots), _p(positions), _p(bt)
    a.rows = rows
    for n in ("block_table_stride", "max_sequences", "layer", "page_tokens", "num_pages",
              "num_attention_layers", "q_heads", "kv_heads", "head_dim"):
        setattr(a, n, geom[n])
    a.scale = float(scale if scale is not None else 1.0 / np.sqrt(D))
    lib().or_paged_attention_psq(C.byref(a), C.c_uint32(fmt),
                                 _p(np.ascontiguousarray(k_code)), _p(np.ascontiguousarray(v_code)),
                                 _p(np.ascontiguousarray(k_scale)),
                                 _p(np.ascontiguousarray(v_scale)))
    return out


def split_reduce(geom: dict, partials: np.ndarray, splits: int, n_used, slots,
                 rows: int, output_dtype: str = "f32") -> np.ndarray:
    """or_split_reduce over f32 partials [rows][kv][splits][q_per_kv*(2+256)]."""
    H, D = geom["q_heads"], geom["head_dim"]
    out = np.zeros((rows, H * D), np.float32 if output_dtype == "f32" else np.uint16)
    slots, n_used = _u32(slots), _u32(n_used)
    a = _AttnArgs()
    a.output = _p(out)
    a.output_dtype = 1 if out.dtype == np.float32 else 0
    a.output_row_stride = H * D
    a.row_sequence_slots = _p(slots)
    a.rows = rows
    a.max_sequences = geom["max_sequences"]
    a.q_heads, a.kv_heads, a.head_dim = H, geom["kv_heads"], D
    lib().or_split_reduce(C.byref(a), _p(np.ascontiguousarray(partials, np.float32)),
                          C.c_uint32(splits), _p(n_used))
    return out


def copy_page(dst: dict, src: dict, dst_page: int, src_page: int, geom: dict) -> None:
    """or_copy_page in place; dst/src: dicts of k, v (uint8 views) and k_scale, v_scale."""
    L = lib()
    eb = geom.get("elem_bytes", 1)
    L.or_copy_page(_p(dst["k"]), _p(dst["v"]), _p(dst.get("k_scale")), _p(dst.get("v_scale")),
                   _p(src["k"]), _p(src["v"]), _p(src.get("k_scale")), _p(src.get("v_scale")),
                   C.c_uint32(dst_page), C.c_uint32(src_page), C.c_uint32(geom["layers"]),
                   C.c_uint32(geom["dst_num_pages"]), C.c_uint32(geom["src_num_pages"]),
                   C.c_uint32(geom["page_tokens"]), C.c_uint32(geom["kv_heads"]),
                   C.c_uint32(geom["head_dim"]), C.c_uint32(eb))
