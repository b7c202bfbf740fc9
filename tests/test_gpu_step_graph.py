"""HIP-graph capture of planned PAGED_ATTENTION steps: a mixed step (decode rows
with split-K, two verify blocks, one prefill chunk) run eagerly once, captured
once, then replayed; between replays the query and KV contents change in
place and unrelated eager work runs, and every replay must equal an eager
launch of the same step bit for bit (same kernels, same arguments)."""
import numpy as np
import pytest
import torch

import phaseshift_amd as P
from phaseshift_amd import ops, state
from tests.kvcase import paged_layout, to_dev

pytestmark = pytest.mark.gpu

QH, H, D, PT = 24, 4, 256, 16


def mixed_case(dev, kv_dtype, seed):
    rng = np.random.default_rng(seed)
    ctx = [int(x) for x in rng.integers(2200, 3600, 8)]
    lens = ctx + [1016, 1016, 328]
    lay = paged_layout(rng, lens, PT, H, D, spare_pages=2)
    g = ops.PoolGeometry(1, lay.num_pages, PT, H, D)
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    if kv_dtype == P.KV_BF16:
        kp = torch.randn(g.pool_elems, generator=gen, device=dev).to(torch.bfloat16)
        vp = torch.randn(g.pool_elems, generator=gen, device=dev).to(torch.bfloat16)
        ks = vs = None
    elif kv_dtype == P.KV_FP8:
        kp = torch.randint(0, 126, (g.pool_elems,), generator=gen, device=dev).to(torch.uint8)
        vp = torch.randint(0, 126, (g.pool_elems,), generator=gen, device=dev).to(torch.uint8)
        ks = torch.rand(g.scale_elems, generator=gen, device=dev) * 0.02 + 1e-3
        vs = torch.rand(g.scale_elems, generator=gen, device=dev) * 0.02 + 1e-3
    else:
        kp = torch.randint(0, 256, (g.psq_code_bytes(4),), generator=gen, device=dev).to(torch.uint8)
        vp = torch.randint(0, 256, (g.psq_code_bytes(4),), generator=gen, device=dev).to(torch.uint8)
        ks = (torch.rand(g.psq_blocks, generator=gen, device=dev) * 0.2 + 0.02).to(torch.bfloat16)
        vs = (torch.rand(g.psq_blocks, generator=gen, device=dev) * 0.2 + 0.02).to(torch.bfloat16)
    slots = np.array(list(range(8)) + [8] * 16 + [9] * 16 + [10] * 128, np.uint32)
    pos = np.array([c - 1 for c in ctx] + list(range(1000, 1016)) * 2 + list(range(200, 328)),
                   np.uint32)
    reqs = ([(i, 1, 0, ctx[i]) for i in range(8)] + [(8, 16, 1, 1016), (24, 16, 1, 1016),
                                                     (40, 128, 2, 328)])
    rows = len(slots)
    q = torch.randn((rows, QH * D), generator=gen, device=dev).to(torch.bfloat16)
    return g, lay, (kp, vp, ks, vs), to_dev(slots), to_dev(pos), to_dev(lay.block_tables), q, reqs


@pytest.mark.parametrize("kv_dtype", [P.KV_BF16, P.KV_FP8, P.KV_PSQ4])
def test_replays_equal_eager(dev, kv_dtype):
    g, lay, pools, slots, pos, bt, q, reqs = mixed_case(dev, kv_dtype, 5 + kv_dtype)
    rows = q.shape[0]
    maxvis = 3600
    nbytes = 64 << 20
    part = torch.empty(nbytes // 4, dtype=torch.float32, device=dev)
    part_e = torch.empty_like(part)
    out_g = torch.full((rows, QH * D), 7.0, device=dev)
    out_e = torch.full((rows, QH * D), 7.0, device=dev)
    a_g = ops.attention_args(g, 0, q, out_g, slots, pos, bt, QH)
    a_e = ops.attention_args(g, 0, q, out_e, slots, pos, bt, QH)
    cache = state.StepGraphCache(4)
    gen = torch.Generator(device=dev)
    gen.manual_seed(99)
    hows = []
    for it in range(6):
        if it:
            # new step contents in the same buffers
            q.copy_(torch.randn(q.shape, generator=gen, device=dev).to(q.dtype))
            kp = pools[0]
            n = kp.numel() // 4
            if kp.dtype == torch.bfloat16:
                kp[:n].copy_(torch.randn(n, generator=gen, device=dev).to(kp.dtype))
            else:
                kp[:n].copy_(torch.randint(0, 126, (n,), generator=gen, device=dev).to(kp.dtype))
            _ = (torch.randn(1 << 20, device=dev) * 2).sum()   # unrelated eager work
        plan, how = cache.step(a_g, kv_dtype, reqs, maxvis, nbytes, part, *pools)
        hows.append(how)
        state.plan_step(a_e, kv_dtype, reqs, maxvis, nbytes, part_e, *pools, launch=True)
        torch.cuda.synchronize()
        assert torch.equal(out_g, out_e), (it, how)
        assert not torch.any(out_g == 7.0)
    assert hows == [0, 1, 2, 2, 2, 2]
    st = cache.stats()
    assert (st.eager, st.captures, st.replays, st.graphs) == (1, 1, 4, 1)
    if kv_dtype != P.KV_PSQ4:
        assert plan.count >= 2   # decode + tile launches in the graph
    # a different plan (shorter max_visible: no split) is a new key
    sig_a = state.plan_signature(a_g, kv_dtype, reqs, maxvis, nbytes, part, *pools)
    sig_b = state.plan_signature(a_g, kv_dtype, reqs, 2000, nbytes, part, *pools)
    sig_c = state.plan_signature(a_e, kv_dtype, reqs, maxvis, nbytes, part, *pools)
    assert len({sig_a, sig_b, sig_c}) == 3 and 0 not in (sig_a, sig_b, sig_c)
    _, how = cache.step(a_g, kv_dtype, reqs, 1500, nbytes, part, *pools)
    assert how == 0


def test_lru_capacity(dev):
    g, lay, pools, slots, pos, bt, q, reqs = mixed_case(dev, P.KV_FP8, 3)
    rows = q.shape[0]
    nbytes = 64 << 20
    part = torch.empty(nbytes // 4, dtype=torch.float32, device=dev)
    outs = [torch.zeros((rows, QH * D), device=dev) for _ in range(3)]
    cache = state.StepGraphCache(2)
    args = [ops.attention_args(g, 0, q, o, slots, pos, bt, QH) for o in outs]
    for a in args:                    # three keys through a 2-entry cache
        cache.step(a, P.KV_FP8, reqs, 3600, nbytes, part, *pools)
        cache.step(a, P.KV_FP8, reqs, 3600, nbytes, part, *pools)
    st = cache.stats()
    assert st.captures == 3 and st.evictions == 1 and st.entries == 2 and st.graphs == 2
    _, how = cache.step(args[0], P.KV_FP8, reqs, 3600, nbytes, part, *pools)
    assert how == 0                   # evicted: seen again from scratch
    torch.cuda.synchronize()
    assert torch.equal(outs[1], outs[2])


def test_forked_step_replays_equal_eager(dev):
    """A step with >= 1024 tile rows runs its decode launch on a side stream
    (fork and join by events); the captured graph keeps the fork, and every
    replay equals the eager step."""
    rng = np.random.default_rng(17)
    ctx = [int(x) for x in rng.integers(2200, 3000, 6)]
    lens = ctx + [1024 + 700]
    lay = paged_layout(rng, lens, PT, H, D, spare_pages=2)
    g = ops.PoolGeometry(1, lay.num_pages, PT, H, D)
    gen = torch.Generator(device=dev)
    gen.manual_seed(17)
    kp = torch.randint(0, 126, (g.pool_elems,), generator=gen, device=dev).to(torch.uint8)
    vp = torch.randint(0, 126, (g.pool_elems,), generator=gen, device=dev).to(torch.uint8)
    ks = torch.rand(g.scale_elems, generator=gen, device=dev) * 0.02 + 1e-3
    vs = torch.rand(g.scale_elems, generator=gen, device=dev) * 0.02 + 1e-3
    slots = np.array(list(range(6)) + [6] * 1024, np.uint32)
    pos = np.array([c - 1 for c in ctx] + list(range(700, 1724)), np.uint32)
    reqs = [(i, 1, 0, ctx[i]) for i in range(6)] + [(6, 1024, 2, 1724)]
    rows = len(slots)
    q = torch.randn((rows, QH * D), generator=gen, device=dev).to(torch.bfloat16)
    nbytes = 64 << 20
    part = torch.empty(nbytes // 4, dtype=torch.float32, device=dev)
    part_e = torch.empty_like(part)
    out_g = torch.full((rows, QH * D), 7.0, device=dev)
    out_e = torch.full((rows, QH * D), 7.0, device=dev)
    s, p_, bt = to_dev(slots), to_dev(pos), to_dev(lay.block_tables)
    a_g = ops.attention_args(g, 0, q, out_g, s, p_, bt, QH)
    a_e = ops.attention_args(g, 0, q, out_e, s, p_, bt, QH)
    cache = state.StepGraphCache(2)
    hows = []
    for it in range(4):
        if it:
            q.copy_(torch.randn(q.shape, generator=gen, device=dev).to(q.dtype))
            _ = (torch.randn(1 << 20, device=dev) * 2).sum()
        plan, how = cache.step(a_g, P.KV_FP8, reqs, 3000, nbytes, part, kp, vp, ks, vs)
        hows.append(how)
        state.plan_step(a_e, P.KV_FP8, reqs, 3000, nbytes, part_e, kp, vp, ks, vs, launch=True)
        torch.cuda.synchronize()
        assert torch.equal(out_g, out_e), (it, how)
        assert not torch.any(out_g == 7.0)
    assert hows == [0, 1, 2, 2]
    assert [k.side for k in plan.kernels[:plan.count]] == [1, 0]
