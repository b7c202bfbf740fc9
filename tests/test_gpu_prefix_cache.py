"""Prefix cache on the GPU: the reference's own cases
(tests/unit/test_qwen35_prefix_cache.hip: round trip per KV dtype, partial
page, LRU and duplicate, too large and eviction release) plus the DFlash ring,
the GDN pool, and the batched copy (one launch per save / restore). Every check is byte equality against a host
snapshot taken before the save."""
import numpy as np
import pytest
import torch

import phaseshift_amd as P
from phaseshift_amd import state

pytestmark = pytest.mark.gpu

PT, H, D = 16, 4, 256


class Fixture:
    def __init__(self, dev, kv_dtype=P.KV_FP8, pages=64, layers=2, capacity=512, entries=4,
                 min_prefix=16, max_blocks=40):
        self.dev = dev
        self.kv = state.KVPool(pages, PT, layers, H, D, kv_dtype=kv_dtype)
        self.slots = state.SlotPool(8, max_blocks)
        self.gdn = state.GdnPool(8, 3, 100, 3, 2, 16, 16)
        self.cache = state.PrefixCache(self.kv, self.gdn, capacity, entries, min_prefix)
        self.layers = layers
        self.max_seq_len = max_blocks * PT
        gen = torch.Generator(device=dev)
        gen.manual_seed(kv_dtype * 7 + pages)
        for t in self.kv.tensors(torch).values():
            t.copy_(torch.randint(0, 255, t.shape, generator=gen, device=dev).to(t.dtype))
        for t in self.gdn.tensors(torch):
            t.copy_(torch.randint(0, 255, t.shape, generator=gen, device=dev).to(t.dtype))
        torch.cuda.synchronize()

    def sequence(self, tokens):
        s = state.Sequence(self.slots, self.kv, self.max_seq_len)
        self.gdn.initialize(s.slot)
        if tokens:
            s.reserve(tokens)
            s.commit(tokens)
        return s

    def page_bytes(self, pages):
        """Host copy of the given pages of every tensor of the KV pool."""
        out = {}
        for k, t in self.kv.tensors(torch).items():
            a = t.cpu().numpy().reshape(self.layers, self.kv.geom.num_pages, -1)
            out[k] = a[:, list(pages)].copy()
        return out

    def gdn_slot(self, slot):
        i = self.gdn.info()
        conv, rec = (t.cpu().numpy() for t in self.gdn.tensors(torch))
        return (conv[slot * i.conv_slot_bytes:(slot + 1) * i.conv_slot_bytes].copy(),
                rec[slot * i.recurrent_slot_bytes:(slot + 1) * i.recurrent_slot_bytes].copy())


def tokens_of(n, base=1):
    return [base + 3 * i for i in range(n)]


@pytest.mark.parametrize("kv_dtype", [P.KV_BF16, P.KV_FP8, P.KV_PSQ4, P.KV_PSQ8])
def test_roundtrip(dev, kv_dtype):
    fx = Fixture(dev, kv_dtype)
    pos = 64
    seq = fx.sequence(pos)
    pages = seq.block_table()
    want_kv = fx.page_bytes(pages)
    want_gdn = fx.gdn_slot(seq.slot)
    toks = tokens_of(pos)
    fx.cache.save(seq, fx.gdn, fx.kv, toks)
    st = fx.cache.stats()
    assert st.size == 1 and st.inserts == 1 and st.copy_launches == 1
    fx.gdn.release(seq.slot)
    seq.release()
    cp = fx.cache.find_longest(toks + [7, 8])
    assert cp is not None and cp.position == pos and cp.num_pages == pos // PT
    # scribble over the freed pages before the restore reuses them
    for t in fx.kv.tensors(torch).values():
        t.fill_(0)
    restored = fx.sequence(0)
    fx.cache.restore(restored, fx.gdn, fx.kv, cp.id)
    torch.cuda.synchronize()
    assert restored.position == pos and len(restored.block_table()) == pos // PT
    got_kv = fx.page_bytes(restored.block_table())
    for k in want_kv:
        assert np.array_equal(got_kv[k], want_kv[k]), k
    got_gdn = fx.gdn_slot(restored.slot)
    assert np.array_equal(got_gdn[0], want_gdn[0]) and np.array_equal(got_gdn[1], want_gdn[1])
    st = fx.cache.stats()
    assert st.copy_launches == 2 and st.restored_tokens == pos and st.hits == 1


def test_partial_page_and_append_after_restore(dev):
    fx = Fixture(dev)
    partial = 37
    seq = fx.sequence(partial)
    want = fx.page_bytes(seq.block_table())
    fx.cache.save(seq, fx.gdn, fx.kv, tokens_of(partial, 5))
    fx.gdn.release(seq.slot)
    seq.release()
    cp = fx.cache.find_longest(tokens_of(partial, 5))
    restored = fx.sequence(0)
    fx.cache.restore(restored, fx.gdn, fx.kv, cp.id)
    torch.cuda.synchronize()
    assert restored.position == partial and len(restored.block_table()) == 3
    got = fx.page_bytes(restored.block_table())
    for k in want:
        assert np.array_equal(got[k], want[k]), k
    restored.reserve(20)
    restored.commit(20)
    assert restored.position == partial + 20
    assert fx.cache.stats().size == 1     # the cache entry is untouched


def test_lru_and_duplicate(dev):
    fx = Fixture(dev, capacity=2 * 48, entries=2)
    a, b, c = tokens_of(40, 1), tokens_of(40, 1000), tokens_of(40, 2000)
    for toks in (a, b):
        s = fx.sequence(40)
        fx.cache.save(s, fx.gdn, fx.kv, toks)
        fx.gdn.release(s.slot)
        s.release()
    assert fx.cache.stats().size == 2
    assert fx.cache.find_longest(a) is not None          # a is now the most recent
    s = fx.sequence(40)
    fx.cache.save(s, fx.gdn, fx.kv, c)
    assert fx.cache.find_longest(b) is None              # b evicted
    assert fx.cache.find_longest(a) is not None and fx.cache.find_longest(c) is not None
    assert fx.cache.stats().evictions == 1
    before = fx.cache.stats().size
    fx.cache.save(s, fx.gdn, fx.kv, c)                    # duplicate
    st = fx.cache.stats()
    assert st.size == before and st.duplicate_hits == 1
    fx.cache.clear()
    st = fx.cache.stats()
    assert st.size == 0 and st.cache_free_pages == st.cache_pages and st.cache_free_slots == 2
    # strictly shorter lookups skip an exact match
    fx.cache.save(s, fx.gdn, fx.kv, c)
    assert fx.cache.find_longest(c, strictly_shorter=True) is None
    assert fx.cache.find_longest(c + [1]) is not None


def test_too_large_min_prefix_and_eviction_release(dev):
    fx = Fixture(dev, capacity=32, entries=2, min_prefix=16)
    big = fx.sequence(48)                                  # 3 pages > 2 cache pages
    fx.cache.save(big, fx.gdn, fx.kv, tokens_of(48))
    st = fx.cache.stats()
    assert st.size == 0 and st.skipped_too_large == 1 and st.cache_free_pages == 2
    small = fx.sequence(10)                                # below min_prefix_tokens
    fx.cache.save(small, fx.gdn, fx.kv, tokens_of(10))
    assert fx.cache.stats().size == 0 and fx.cache.stats().inserts == 0
    s1 = fx.sequence(32)
    fx.cache.save(s1, fx.gdn, fx.kv, tokens_of(32, 50))
    s2 = fx.sequence(20)
    fx.cache.save(s2, fx.gdn, fx.kv, tokens_of(20, 90))   # needs 2 pages: evicts s1's entry
    st = fx.cache.stats()
    assert st.evictions == 1 and st.size == 1 and st.cache_free_pages == 0
    fx.cache.clear()
    st = fx.cache.stats()
    assert st.cache_free_pages == 2 and st.cache_free_slots == 2
    with pytest.raises(P.StateError):
        fx.cache.save(s1, fx.gdn, fx.kv, tokens_of(31))     # token count != position


def test_dflash_ring_roundtrip(dev):
    fx = Fixture(dev)
    ring_bytes = 3 * 64 * 128 * 2
    fx.cache.enable_dflash_ring(ring_bytes)
    k = torch.randint(0, 255, (ring_bytes,), dtype=torch.uint8, device=dev)
    v = torch.randint(0, 255, (ring_bytes,), dtype=torch.uint8, device=dev)
    ctx = P.DFlashContext(k.data_ptr(), v.data_ptr(), ring_bytes, 17, 81)
    seq = fx.sequence(48)
    fx.cache.save(seq, fx.gdn, fx.kv, tokens_of(48), dflash=ctx)
    torch.cuda.synchronize()
    want_k, want_v = k.cpu().clone(), v.cpu().clone()
    k.zero_()
    v.fill_(3)
    cp = fx.cache.find_longest(tokens_of(48))
    assert cp.dflash == 1
    out = P.DFlashContext(k.data_ptr(), v.data_ptr(), ring_bytes, 0, 0)
    restored = fx.sequence(0)
    fx.cache.restore(restored, fx.gdn, fx.kv, cp.id, dflash=out)
    torch.cuda.synchronize()
    assert torch.equal(k.cpu(), want_k) and torch.equal(v.cpu(), want_v)
    assert out.length == 17 and out.next_position == 81
    assert fx.cache.stats().copy_launches == 2


@pytest.mark.parametrize("npages", [40, 300])
def test_many_pages_one_launch(dev, npages):
    """40 pages (their pairs inline in the launch's arguments) and 300 pages
    (more than the 256 pairs a launch carries: the pair list goes to the
    device first): each save is one copy launch; bytes exact."""
    fx = Fixture(dev, pages=2 * npages + 16, capacity=16 * (npages + 8), entries=2, max_blocks=npages + 8)
    seq = fx.sequence(16 * npages)
    want = fx.page_bytes(seq.block_table())
    want_gdn = fx.gdn_slot(seq.slot)
    fx.cache.save(seq, fx.gdn, fx.kv, tokens_of(16 * npages))
    assert fx.cache.stats().copy_launches == 1
    restored = fx.sequence(0)
    fx.cache.restore(restored, fx.gdn, fx.kv, fx.cache.find_longest(tokens_of(16 * npages)).id)
    torch.cuda.synchronize()
    got = fx.page_bytes(restored.block_table())
    for k in want:
        assert np.array_equal(got[k], want[k]), k
    g = fx.gdn_slot(restored.slot)
    assert np.array_equal(g[0], want_gdn[0]) and np.array_equal(g[1], want_gdn[1])


def test_gdn_pool_initialize_reset_copy(dev):
    gdn = state.GdnPool(4, 3, 100, 3, 2, 16, 16)
    i = gdn.info()
    assert gdn.layout.conv_dim_padded == 104 and i.conv_slot_bytes == 3 * 3 * 104 * 2
    assert i.recurrent_slot_bytes == 3 * 2 * 16 * 16 * 4
    for t in gdn.tensors(torch):
        t.fill_(7)
    gdn.initialize(1)
    torch.cuda.synchronize()
    conv, rec = (t.cpu().numpy() for t in gdn.tensors(torch))
    cs, rs = i.conv_slot_bytes, i.recurrent_slot_bytes
    assert not conv[cs:2 * cs].any() and not rec[rs:2 * rs].any()
    assert (conv[:cs] == 7).all() and (conv[2 * cs:] == 7).all()
    with pytest.raises(P.StateError):
        gdn.initialize(1)
    other = state.GdnPool(2, 3, 100, 3, 2, 16, 16)
    for t in other.tensors(torch):
        t.copy_(torch.arange(t.numel(), device=dev).to(torch.uint8))
    gdn.copy_slot_from(3, other, 1)
    torch.cuda.synchronize()
    conv, rec = (t.cpu().numpy() for t in gdn.tensors(torch))
    oc, orr = (t.cpu().numpy() for t in other.tensors(torch))
    assert np.array_equal(conv[3 * cs:4 * cs], oc[cs:2 * cs])
    assert np.array_equal(rec[3 * rs:4 * rs], orr[rs:2 * rs])
    bad = state.GdnPool(2, 3, 96, 3, 2, 16, 16)
    with pytest.raises(P.StateError):
        gdn.copy_slot_from(0, bad, 0)
    gdn.release(1)
    with pytest.raises(P.StateError):
        gdn.release(1)
