"""Python handles over the host KV state of the C-ABI (PagedKVPool,
SequenceSlotPool, PagedSequenceState) and the step planner.

Reference classes: src/phaseshift/models/qwen35/state/paged_kv_pool.cpp,
sequence_slot_pool.cpp, paged_sequence_state.cpp, and
runtime/paged_attention_dispatch.hip (planner). Errors raise StateError with
the reference's Status category (invalid_argument, out_of_range, ...).
"""
from __future__ import annotations

import ctypes as C

from . import (CheckpointInfo, DFlashContext, GdnLayout, GdnPoolInfo, PrefixCacheStats,
               StepGraphStats,
               KV_BF16, KV_FP8, KV_PSQ4, KV_PSQ8, PLAN_ONLY, PoolInfo, SequenceInfo, StepPlan, StepRequest, check,
               check_state, lib)
from .ops import PoolGeometry, _stream


class KVPool:
    def __init__(self, num_pages, page_tokens, num_layers, kv_heads, head_dim, fp8=True,
                 kv_dtype=None):
        """kv_dtype (KV_BF16, KV_FP8, KV_PSQ4, KV_PSQ8) overrides fp8."""
        self._h = C.c_void_p()
        self.kv_dtype = kv_dtype if kv_dtype is not None else (KV_FP8 if fp8 else KV_BF16)
        check_state("psk_pool_create", lib().psk_pool_create(
            C.byref(self._h), num_pages, page_tokens, num_layers, kv_heads, head_dim,
            self.kv_dtype))
        self.geom = PoolGeometry(num_layers, num_pages, page_tokens, kv_heads, head_dim)
        self.fp8 = self.kv_dtype == KV_FP8

    def close(self):
        if self._h:
            lib().psk_pool_destroy(self._h)
            self._h = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def info(self) -> PoolInfo:
        i = PoolInfo()
        check_state("psk_pool_info", lib().psk_pool_info(self._h, C.byref(i)))
        return i

    def allocate(self) -> int:
        p = C.c_uint32()
        check_state("psk_pool_allocate", lib().psk_pool_allocate(self._h, C.byref(p)))
        return p.value

    def release(self, page: int) -> None:
        check_state("psk_pool_release", lib().psk_pool_release(self._h, page))

    def copy_pages_from(self, src: "KVPool", dst_pages, src_pages, stream=None) -> None:
        n = len(dst_pages)
        d = (C.c_uint32 * n)(*dst_pages)
        s = (C.c_uint32 * n)(*src_pages)
        check_state("psk_pool_copy_pages", lib().psk_pool_copy_pages(
            self._h, src._h, d, s, n, _stream(stream)))

    def tensors(self, torch):
        """Views of the pools as torch tensors (no copy)."""
        i = self.info()
        g = self.geom
        if self.kv_dtype in (KV_PSQ4, KV_PSQ8):
            fmt = 4 if self.kv_dtype == KV_PSQ4 else 8
            nc = g.psq_code_bytes(fmt)
            return {"k": _wrap(torch, i.k_pool, nc, torch.uint8),
                    "v": _wrap(torch, i.v_pool, nc, torch.uint8),
                    "k_scale": _wrap(torch, i.k_scale_pool, g.psq_blocks, torch.int16),
                    "v_scale": _wrap(torch, i.v_scale_pool, g.psq_blocks, torch.int16)}
        n = g.pool_elems
        dt = torch.uint8 if self.fp8 else torch.int16
        out = {"k": _wrap(torch, i.k_pool, n, dt), "v": _wrap(torch, i.v_pool, n, dt)}
        if self.fp8:
            out["k_scale"] = _wrap(torch, i.k_scale_pool, g.scale_elems, torch.float32)
            out["v_scale"] = _wrap(torch, i.v_scale_pool, g.scale_elems, torch.float32)
        return out


def _wrap(torch, ptr, n, dtype):
    """A torch tensor aliasing device memory owned by the library."""
    itemsize = torch.tensor([], dtype=dtype).element_size()

    class _Mem:
        __cuda_array_interface__ = None

    typestr = {torch.uint8: "|u1", torch.int16: "<i2", torch.float32: "<f4",
               torch.int32: "<i4"}[dtype]
    m = _Mem()
    m.__cuda_array_interface__ = {"shape": (n,), "typestr": typestr, "data": (ptr, False),
                                  "version": 3, "strides": (itemsize,)}
    return torch.as_tensor(m, device="cuda")


class SlotPool:
    def __init__(self, max_sequences, max_blocks, stream=None):
        self._h = C.c_void_p()
        check_state("psk_slot_pool_create", lib().psk_slot_pool_create(
            C.byref(self._h), max_sequences, max_blocks, _stream(stream)))
        self.max_sequences, self.max_blocks = max_sequences, max_blocks

    def block_tables(self, torch):
        ptr = lib().psk_slot_pool_block_tables(self._h)
        return _wrap(torch, ptr, self.max_sequences * self.max_blocks, torch.int32).view(
            self.max_sequences, self.max_blocks)

    def close(self):
        if self._h:
            lib().psk_slot_pool_destroy(self._h)
            self._h = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Sequence:
    def __init__(self, slots: SlotPool, pool: KVPool, max_seq_len: int, stream=None):
        self._h = C.c_void_p()
        check_state("psk_sequence_create", lib().psk_sequence_create(
            C.byref(self._h), slots._h, pool._h, max_seq_len, _stream(stream)))

    def info(self) -> SequenceInfo:
        i = SequenceInfo()
        check_state("psk_sequence_info", lib().psk_sequence_info(self._h, C.byref(i)))
        return i

    @property
    def slot(self) -> int:
        return self.info().slot

    @property
    def position(self) -> int:
        return self.info().position

    def block_table(self) -> list[int]:
        n = lib().psk_sequence_block_table(self._h, None, 0)
        buf = (C.c_uint32 * max(n, 1))()
        lib().psk_sequence_block_table(self._h, buf, n)
        return list(buf[:n])

    def reserve(self, tokens: int, stream=None) -> None:
        check_state("psk_sequence_reserve", lib().psk_sequence_reserve(self._h, tokens,
                                                                       _stream(stream)))

    def rollback(self, old_block_count: int, stream=None) -> None:
        check_state("psk_sequence_rollback", lib().psk_sequence_rollback(
            self._h, old_block_count, _stream(stream)))

    def commit(self, tokens: int) -> None:
        check_state("psk_sequence_commit", lib().psk_sequence_commit(self._h, tokens))

    def release(self, stream=None) -> None:
        if self._h:
            h, self._h = self._h, C.c_void_p()
            check_state("psk_sequence_release", lib().psk_sequence_release(h, _stream(stream)))


class GdnPool:
    """GdnStatePool (gdn_state_pool.h:41-200): per-slot bf16 conv history and
    f32 recurrent state."""

    def __init__(self, max_sequences, gdn_layers, conv_dim, conv_history, num_v_heads, head_k,
                 head_v):
        self.layout = GdnLayout()
        check_state("psk_gdn_layout_make", lib().psk_gdn_layout_make(
            gdn_layers, conv_dim, conv_history, num_v_heads, head_k, head_v, C.byref(self.layout)))
        self._h = C.c_void_p()
        check_state("psk_gdn_pool_create", lib().psk_gdn_pool_create(
            C.byref(self._h), max_sequences, C.byref(self.layout)))

    def close(self):
        if self._h:
            lib().psk_gdn_pool_destroy(self._h)
            self._h = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def info(self) -> GdnPoolInfo:
        i = GdnPoolInfo()
        check_state("psk_gdn_pool_info", lib().psk_gdn_pool_info(self._h, C.byref(i)))
        return i

    def initialize(self, slot, stream=None):
        check_state("psk_gdn_pool_initialize", lib().psk_gdn_pool_initialize(
            self._h, slot, _stream(stream)))

    def reset(self, slot, stream=None):
        check_state("psk_gdn_pool_reset", lib().psk_gdn_pool_reset(self._h, slot, _stream(stream)))

    def release(self, slot):
        check_state("psk_gdn_pool_release", lib().psk_gdn_pool_release(self._h, slot))

    def copy_slot_from(self, dst_slot, src: "GdnPool", src_slot, stream=None):
        check_state("psk_gdn_pool_copy_slot", lib().psk_gdn_pool_copy_slot(
            self._h, dst_slot, src._h, src_slot, _stream(stream)))

    def tensors(self, torch):
        """(conv uint8 view, recurrent uint8 view) of the whole pool."""
        i = self.info()
        return (_wrap(torch, i.conv_base, i.conv_slot_bytes * i.max_sequences, torch.uint8),
                _wrap(torch, i.recurrent_base, i.recurrent_slot_bytes * i.max_sequences,
                      torch.uint8))


class PrefixCache:
    """PrefixCache (runtime/prefix_cache.h): LRU checkpoints of KV pages, the
    GDN slot and an optional DFlash ring; one batched copy launch per save or
    restore."""

    def __init__(self, active_kv: KVPool, active_gdn: GdnPool, capacity_tokens, max_entries,
                 min_prefix_tokens=64):
        self._h = C.c_void_p()
        check_state("psk_prefix_cache_create", lib().psk_prefix_cache_create(
            C.byref(self._h), active_kv._h, active_gdn._h, capacity_tokens, max_entries,
            min_prefix_tokens))

    def close(self):
        if self._h:
            lib().psk_prefix_cache_destroy(self._h)
            self._h = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def enable_dflash_ring(self, ring_bytes):
        check_state("psk_prefix_cache_enable_dflash_ring",
                    lib().psk_prefix_cache_enable_dflash_ring(self._h, ring_bytes))

    @staticmethod
    def _tokens(tokens):
        """(pointer, count) of int32 tokens: a C-contiguous int32 numpy array
        is passed as is, anything else converted."""
        import numpy as np
        if not (isinstance(tokens, np.ndarray) and tokens.dtype == np.int32
                and tokens.flags.c_contiguous):
            tokens = np.ascontiguousarray(np.asarray(tokens, dtype=np.int64).astype(np.int32))
        return tokens, tokens.ctypes.data if tokens.size else None, int(tokens.size)

    def find_longest(self, tokens, strictly_shorter=False) -> CheckpointInfo | None:
        keep, t, n = self._tokens(tokens)
        out = CheckpointInfo()
        check_state("psk_prefix_cache_find_longest", lib().psk_prefix_cache_find_longest(
            self._h, t, n, int(strictly_shorter), C.byref(out)))
        return out if out.id != 0 else None

    def save(self, seq: "Sequence", gdn: GdnPool, kv: KVPool, tokens, stream=None,
             prompt_boundary=False, dflash: DFlashContext | None = None):
        keep, t, n = self._tokens(tokens)
        check_state("psk_prefix_cache_save", lib().psk_prefix_cache_save(
            self._h, seq._h, gdn._h, kv._h, t, n, int(prompt_boundary),
            C.byref(dflash) if dflash is not None else None, _stream(stream)))

    def restore(self, seq: "Sequence", gdn: GdnPool, kv: KVPool, checkpoint_id: int, stream=None,
                dflash: DFlashContext | None = None):
        check_state("psk_prefix_cache_restore", lib().psk_prefix_cache_restore(
            self._h, seq._h, gdn._h, kv._h, checkpoint_id,
            C.byref(dflash) if dflash is not None else None, _stream(stream)))

    def clear(self):
        check_state("psk_prefix_cache_clear", lib().psk_prefix_cache_clear(self._h))

    def stats(self) -> PrefixCacheStats:
        s = PrefixCacheStats()
        check_state("psk_prefix_cache_stats", lib().psk_prefix_cache_stats(self._h, C.byref(s)))
        return s


def plan_step(args, kv_dtype: int, requests, max_visible_tokens: int, partial_bytes: int,
              partials_ptr=None, k_pool=None, v_pool=None, k_scale=None, v_scale=None,
              stream=None, launch=False) -> StepPlan:
    """psk_paged_attention_step: plan (and with launch=True run) one step's
    PAGED_ATTENTION binding. requests: list of (row_begin, row_count, exec_class)
    or (row_begin, row_count, exec_class, max_visible)."""
    n = len(requests)
    reqs = (StepRequest * max(n, 1))()
    for i, r in enumerate(requests):
        reqs[i].row_begin, reqs[i].row_count, reqs[i].execution_class = r[0], r[1], r[2]
        reqs[i].max_visible = r[3] if len(r) > 3 else 0
    plan = StepPlan()
    p = lambda t: None if t is None else (t if isinstance(t, int) else t.data_ptr())
    # planning alone only needs a non-null partials pointer to allow split-K
    part = p(partials_ptr) if partials_ptr is not None else (16 if partial_bytes else None)
    rc = lib().psk_paged_attention_step(
        C.byref(args), kv_dtype, p(k_pool), p(v_pool), p(k_scale), p(v_scale), reqs, n,
        max_visible_tokens, part, partial_bytes, C.byref(plan),
        _stream(stream) if launch else PLAN_ONLY)
    check("psk_paged_attention_step", rc)
    return plan


class StepGraphCache:
    """HIP graphs of planned PAGED_ATTENTION steps keyed by the plan signature
    (psk_paged_attention_step_graphed): first sighting eager, second captured,
    then replayed."""

    def __init__(self, capacity=8):
        self._h = C.c_void_p()
        check("psk_step_graph_cache_create", lib().psk_step_graph_cache_create(
            C.byref(self._h), capacity))

    def close(self):
        if self._h:
            lib().psk_step_graph_cache_destroy(self._h)
            self._h = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def step(self, args, kv_dtype, requests, max_visible_tokens, partial_bytes, partials,
             k_pool, v_pool, k_scale=None, v_scale=None, stream=None):
        """Returns (plan, how) with how 0 eager, 1 captured, 2 replayed."""
        n = len(requests)
        reqs = (StepRequest * max(n, 1))()
        for i, r in enumerate(requests):
            reqs[i].row_begin, reqs[i].row_count, reqs[i].execution_class = r[0], r[1], r[2]
            reqs[i].max_visible = r[3] if len(r) > 3 else 0
        plan = StepPlan()
        how = C.c_uint32(99)
        p = lambda t: None if t is None else (t if isinstance(t, int) else t.data_ptr())
        check("psk_paged_attention_step_graphed", lib().psk_paged_attention_step_graphed(
            self._h, C.byref(args), kv_dtype, p(k_pool), p(v_pool), p(k_scale), p(v_scale), reqs,
            n, max_visible_tokens, p(partials), partial_bytes, C.byref(plan), _stream(stream),
            C.byref(how)))
        return plan, how.value

    def stats(self) -> StepGraphStats:
        st = StepGraphStats()
        check("psk_step_graph_cache_stats", lib().psk_step_graph_cache_stats(self._h, C.byref(st)))
        return st


def plan_signature(args, kv_dtype, requests, max_visible_tokens, partial_bytes, partials,
                   k_pool, v_pool, k_scale=None, v_scale=None) -> int:
    n = len(requests)
    reqs = (StepRequest * max(n, 1))()
    for i, r in enumerate(requests):
        reqs[i].row_begin, reqs[i].row_count, reqs[i].execution_class = r[0], r[1], r[2]
        reqs[i].max_visible = r[3] if len(r) > 3 else 0
    p = lambda t: None if t is None else (t if isinstance(t, int) else t.data_ptr())
    return int(lib().psk_paged_attention_plan_signature(
        C.byref(args), kv_dtype, p(k_pool), p(v_pool), p(k_scale), p(v_scale), reqs, n,
        max_visible_tokens, p(partials), partial_bytes))
