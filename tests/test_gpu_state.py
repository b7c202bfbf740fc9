"""Host KV state on the GPU: pool free list, device block tables, reserve /
rollback (page truncation) / commit, prefix-cache page copy, and the BASELINE
config-5 mixed continuous-batching step end to end (append, CoW copy, planned
attention, verify rollback) against the oracle."""
import math

import numpy as np
import pytest
import torch

import oracle
import phaseshift_amd as P
from phaseshift_amd import ops, state
from tests.kvcase import (INVALID, REL_DECODE, REL_TILE, assert_attention_close, bf16_normal,
                          oracle_attention_parallel, to_dev, to_host)

pytestmark = pytest.mark.gpu


def test_pool_free_list_and_errors(dev):
    pool = state.KVPool(8, 16, 2, 4, 256, fp8=True)
    info = pool.info()
    assert info.free_pages == 8 and info.reserved_bytes == 2 * 2 * 8 * 16 * 4 * 256 + 2 * 2 * 8 * 16 * 4 * 4
    pages = [pool.allocate() for _ in range(8)]
    assert sorted(pages) == list(range(8)) and pages[0] == 7   # LIFO from the back
    with pytest.raises(P.StateError) as e:
        pool.allocate()
    assert e.value.kind == "insufficient_memory"
    pool.release(3)
    with pytest.raises(P.StateError) as e:
        pool.release(3)
    assert e.value.kind == "invalid_argument"
    with pytest.raises(P.StateError):
        pool.release(99)
    assert pool.allocate() == 3


def test_reserve_rollback_commit(dev):
    pool = state.KVPool(64, 16, 1, 4, 256, fp8=True)
    slots = state.SlotPool(4, 20)
    seq = state.Sequence(slots, pool, 300)
    bt = slots.block_tables(torch)
    torch.cuda.synchronize()
    assert np.all(to_host(bt) == INVALID)
    seq.reserve(40)                    # 3 pages
    seq.commit(40)
    seq.reserve(16 * 5 - 40 + 3)       # up to 83 tokens -> 6 pages
    table = seq.block_table()
    assert len(table) == 6 and pool.info().free_pages == 58
    torch.cuda.synchronize()
    dev_row = to_host(bt)[seq.slot]
    assert list(dev_row[:6]) == table and np.all(dev_row[6:] == INVALID)
    # rejected speculative tail: truncate back to ceil(41/16) = 3 pages
    seq.rollback(3)
    torch.cuda.synchronize()
    dev_row = to_host(bt)[seq.slot]
    assert list(dev_row[:3]) == table[:3] and np.all(dev_row[3:] == INVALID)
    assert pool.info().free_pages == 61 and seq.block_table() == table[:3]
    seq.rollback(3)                    # repeated rollback: no-op, no double free
    torch.cuda.synchronize()
    assert pool.info().free_pages == 61 and seq.block_table() == table[:3]
    assert list(to_host(bt)[seq.slot][:3]) == table[:3]
    seq.commit(1)
    assert seq.position == 41
    with pytest.raises(P.StateError) as e:
        seq.rollback(9)
    assert e.value.kind == "out_of_range"
    with pytest.raises(P.StateError) as e:
        seq.reserve(1000)
    assert e.value.kind == "out_of_range"
    seq.release()
    assert pool.info().free_pages == 64


def test_prefix_cache_page_copy(dev):
    """save: active -> cache pages; restore: cache -> fresh active pages
    (prefix_cache.cpp:324-331,426-437); byte-exact K, V and scale rows."""
    L, NP, Pt, H, D = 3, 40, 16, 4, 256
    active = state.KVPool(NP, Pt, L, H, D, fp8=True)
    cache = state.KVPool(NP, Pt, L, H, D, fp8=True)
    at, ct = active.tensors(torch), cache.tensors(torch)
    gen = torch.Generator(device=dev)
    gen.manual_seed(1)
    for t in at.values():
        t.copy_(torch.randint(0, 255, t.shape, generator=gen, device=dev).to(t.dtype))
    src = [active.allocate() for _ in range(32)]
    dst = [cache.allocate() for _ in range(32)]
    cache.copy_pages_from(active, dst, src)
    restored = [active.allocate() for _ in range(5)]
    active.copy_pages_from(cache, restored, dst[:5])
    torch.cuda.synchronize()
    A = {k: to_host(v) for k, v in at.items()}
    Cc = {k: to_host(v) for k, v in ct.items()}
    for k in ("k", "v"):
        a = A[k].reshape(L, NP, -1)
        c = Cc[k].reshape(L, NP, -1)
        assert np.array_equal(c[:, dst], a[:, src])
        assert np.array_equal(a[:, restored], a[:, src[:5]])
    for k in ("k_scale", "v_scale"):
        a = A[k].reshape(L, NP, -1)
        c = Cc[k].reshape(L, NP, -1)
        assert np.array_equal(c[:, dst].view(np.uint32), a[:, src].view(np.uint32))


def test_config5_mixed_step(dev):
    """8 prefill chunks of 512 rows, 48 decode rows, 8 DFlash2
    verify blocks of 16 drafts (causal) with rollback of rejected tails, and a CoW
    restore of 32 shared prefix pages; FP8 KV, 24/4 heads, hd 256, page 16,
    contexts U[2k,16k]."""
    rng = np.random.default_rng(5005)
    QH, H, D, Pt = 24, 4, 256, 16
    n_pre, n_dec, n_ver = 8, 48, 8
    ctx = rng.integers(2048, 16385, n_pre + n_dec + n_ver)
    max_len = int(ctx.max()) + 512 + 16
    need_pages = int(sum(math.ceil((c + 512) / Pt) for c in ctx)) + 64
    pool = state.KVPool(need_pages, Pt, 1, H, D, fp8=True)
    cache = state.KVPool(64, Pt, 1, H, D, fp8=True)
    slots = state.SlotPool(n_pre + n_dec + n_ver + 1, math.ceil(max_len / Pt))
    g = pool.geom
    T = pool.tensors(torch)
    gen = torch.Generator(device=dev)
    gen.manual_seed(5)
    # existing context: random codes / scales (no NaN codes)
    for k in ("k", "v"):
        x = torch.randint(0, 126, T[k].shape, generator=gen, device=dev, dtype=torch.int32)
        T[k].copy_(torch.where(torch.rand(T[k].shape, generator=gen, device=dev) < 0.5, x, x + 128).to(torch.uint8))
    for k in ("k_scale", "v_scale"):
        T[k].copy_(torch.rand(T[k].shape, generator=gen, device=dev) * 0.02 + 1e-3)
    CT = cache.tensors(torch)
    for k in CT:
        CT[k].copy_(T[k][:CT[k].numel()])
    seqs = [state.Sequence(slots, pool, max_len) for _ in range(len(ctx))]
    for s, c in zip(seqs, ctx):
        s.reserve(int(c))
        s.commit(int(c))
    # CoW / prefix restore: sequence 0's first 32 pages come from the cache pool
    cache_pages = [cache.allocate() for _ in range(32)]
    pool.copy_pages_from(cache, seqs[0].block_table()[:32], cache_pages)
    # step layout: decode rows, verify blocks, prefill chunks
    reqs, descs, row = [], [], 0
    for i in range(n_dec):
        s = seqs[n_pre + i]
        reqs.append((row, 1, 0)); descs.append(dict(slot=s.slot, row_begin=row, row_count=1,
                                                    prefix_length=s.position, execution_class=0))
        s.reserve(1); row += 1
    for i in range(n_ver):
        s = seqs[n_pre + n_dec + i]
        reqs.append((row, 16, 1)); descs.append(dict(slot=s.slot, row_begin=row, row_count=16,
                                                     prefix_length=s.position, execution_class=1))
        s.reserve(16); row += 16
    for i in range(n_pre):
        s = seqs[i]
        reqs.append((row, 512, 2)); descs.append(dict(slot=s.slot, row_begin=row, row_count=512,
                                                      prefix_length=s.position, execution_class=2))
        s.reserve(512); row += 512
    rows = row
    assert rows == 4272
    raw = to_dev(np.frombuffer(ops.pack_requests(descs), np.uint8).copy())
    rslots = torch.empty(rows, dtype=torch.int32, device=dev)
    rpos = torch.empty(rows, dtype=torch.int32, device=dev)
    ops.prepare_row_metadata(raw, len(descs), rows, rslots, rpos)
    bt = slots.block_tables(torch)
    torch.cuda.synchronize()
    pool_before = {k: to_host(v).copy() for k, v in T.items()}
    # KV append of every row (fused FP8 quantization)
    kin = bf16_normal(rng, (rows, H * D), 0.01, 20.0)
    vin = bf16_normal(rng, (rows, H * D), 0.01, 20.0)
    ops.kv_append(g, 0, to_dev(kin), to_dev(vin), rslots, rpos, bt, T["k"], T["v"],
                  T["k_scale"], T["v_scale"])
    # planned attention
    q = bf16_normal(rng, (rows, QH * D))
    dq = to_dev(q)
    out = torch.full((rows, QH * D), 7.0, dtype=torch.float32, device=dev)
    a = ops.attention_args(g, 0, dq, out, rslots, rpos, bt, QH)
    part = torch.empty((256 << 20) // 4, dtype=torch.float32, device=dev)
    plan = state.plan_step(a, P.KV_FP8, reqs, int(ctx.max()) + 512, part.numel() * 4,
                           partials_ptr=part, k_pool=T["k"], v_pool=T["v"], k_scale=T["k_scale"],
                           v_scale=T["v_scale"], launch=True)
    assert [k.kind for k in plan.kernels[:plan.count]] == [0, 1, 1]
    torch.cuda.synchronize()
    # ---- append parity (bit-exact) on the host copy of the pool
    h_slots, h_pos, h_bt = to_host(rslots), to_host(rpos), to_host(bt)
    geom = dict(layer=0, page_tokens=Pt, num_pages=g.num_pages, num_attention_layers=1,
                kv_heads=H, head_dim=D, block_table_stride=h_bt.shape[1],
                max_sequences=h_bt.shape[0])
    oracle.kv_append(geom, kin, vin, h_slots, h_pos, h_bt, pool_before["k"], pool_before["v"],
                     pool_before["k_scale"], pool_before["v_scale"])
    for k in ("k", "v"):
        assert np.array_equal(to_host(T[k]), pool_before[k])
    for k in ("k_scale", "v_scale"):
        assert np.array_equal(to_host(T[k]).view(np.uint32), pool_before[k].view(np.uint32))
    # ---- attention parity: every decode and verify row, every 8th row of each
    # prefill chunk, and all 512 rows of the chunk with the shortest context
    pick = list(range(48 + 128))
    shortest = int(np.argmin(ctx[:n_pre]))
    for i in range(n_pre):
        b = 176 + 512 * i
        pick += list(range(b, b + 512)) if i == shortest else list(range(b, b + 512, 8)) + [b + 511]
    pick = np.array(pick)
    og = dict(geom, q_heads=QH)
    want = oracle_attention_parallel(og, q[pick], h_slots[pick], h_pos[pick], h_bt,
                                     pool_before["k"], pool_before["v"], pool_before["k_scale"],
                                     pool_before["v_scale"], 1.0 / 16.0, workers=16)
    got = out.cpu().numpy()[pick]
    err = np.max(np.abs(got - want), axis=1)
    groups = {"decode": err[:48], "verify": err[48:176], "prefill": err[176:]}
    worst = {k: (float(v.max()), int(np.argmax(v))) for k, v in groups.items()}
    print("config5 max-abs error per group (value, index):", worst, "prefill rows checked:", len(pick) - 176)
    bad = np.nonzero(err >= 5e-2)[0]
    print("rows over tolerance:", [(int(pick[i]), float(err[i])) for i in bad[:20]])
    assert np.max(err) < 5e-2
    # decode, verify and prefill rows: FP8 KV, so the FP8 tile bound holds all
    assert_attention_close(got, want, 5e-2, REL_TILE[True], "config5 mixed step")
    # ---- verify rollback: accept a random prefix of each 16-draft block
    # (paged_sequence_state.cpp:189-229; the reference's speculative
    # transaction test, test_qwen35_spec_transaction.hip:170-203: pages
    # released exactly, a repeated rollback is a no-op, the rejected tail is
    # invisible to the next step)
    free_before = pool.info().free_pages
    released = 0
    ver = []
    for i in range(n_ver):
        s = seqs[n_pre + n_dec + i]
        accepted = int(rng.integers(0, 16)) if i else 0   # block 0 rejects every draft
        new_pos = s.position + accepted
        keep = math.ceil(new_pos / Pt)
        old = s.block_table()
        s.rollback(keep)
        released += len(old) - keep
        if accepted:
            s.commit(accepted)
        s.rollback(keep)                  # repeated: no-op, nothing freed twice
        torch.cuda.synchronize()
        dev_row = to_host(bt)[s.slot]
        assert list(dev_row[:keep]) == old[:keep] and np.all(dev_row[keep:len(old)] == INVALID)
        assert s.block_table() == old[:keep] and s.position == new_pos
        ver.append((s, 16 - accepted))
    assert pool.info().free_pages == free_before + released
    assert released > 0
    # next step: one new token per verify sequence at its accepted position.
    # The rejected drafts' K/V stay in the kept pages past that position; the
    # decode must not see them.
    nv = len(ver)
    v_slots = np.array([s.slot for s, _ in ver], np.uint32)
    v_pos = np.array([s.position for s, _ in ver], np.uint32)
    for s, _ in ver:
        s.reserve(1)
    torch.cuda.synchronize()
    h_bt = to_host(bt)
    kin2 = bf16_normal(rng, (nv, H * D), 0.01, 20.0)
    vin2 = bf16_normal(rng, (nv, H * D), 0.01, 20.0)
    ds2, dp2 = to_dev(v_slots), to_dev(v_pos)
    before2 = {k: to_host(v).copy() for k, v in T.items()}
    ops.kv_append(g, 0, to_dev(kin2), to_dev(vin2), ds2, dp2, bt, T["k"], T["v"], T["k_scale"], T["v_scale"])
    oracle.kv_append(dict(geom, block_table_stride=h_bt.shape[1]), kin2, vin2, v_slots, v_pos, h_bt,
                     before2["k"], before2["v"], before2["k_scale"], before2["v_scale"])
    after2 = {k: to_host(v) for k, v in T.items()}
    for k in ("k", "v"):
        assert np.array_equal(after2[k], before2[k])
    q2 = bf16_normal(rng, (nv, QH * D))
    out2 = torch.full((nv, QH * D), 7.0, dtype=torch.float32, device=dev)
    ops.paged_attention(g, 0, to_dev(q2), out2, ds2, dp2, bt, T["k"], T["v"], QH, T["k_scale"], T["v_scale"])
    got2 = out2.cpu().numpy()
    want2 = oracle_attention_parallel(og, q2, v_slots, v_pos, h_bt, after2["k"], after2["v"],
                                      after2["k_scale"], after2["v_scale"], 1.0 / 16.0, workers=8)
    assert_attention_close(got2, want2, 5e-2, REL_DECODE, "config5 decode after rollback")
    # the check has bite: a decode that read the stale tail (the rejected
    # drafts still in the kept page past the new token) would break the bound
    stale = np.array([p_ + min(r - 1, Pt - 1 - p_ % Pt) for p_, (_, r) in zip(v_pos, ver)], np.uint32)
    many = stale >= v_pos + 4
    assert np.any(many)
    seen = oracle_attention_parallel(og, q2[many], v_slots[many], stale[many], h_bt, after2["k"],
                                     after2["v"], after2["k_scale"], after2["v_scale"], 1.0 / 16.0, workers=8)
    row_max = np.abs(want2[many]).max(axis=1)
    assert np.all(np.abs(seen - want2[many]).max(axis=1) > REL_DECODE * row_max + 1e-6)
