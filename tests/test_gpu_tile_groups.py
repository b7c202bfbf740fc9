"""Grouped prefill tiles (GQA groups of 1-8 heads): the step planner puts
consecutive 16-row tiles of one prefill request into groups of eight (one
workgroup, one wave per tile, the group's K/V chunks staged once) and pads a
short last group with empty tiles. Ragged requests (partial groups, a partial
last tile, a chunk at position 0) and split and unsplit launches, every row
against the fp32 oracle."""

import numpy as np
import pytest
import torch

import phaseshift_amd as P
from phaseshift_amd import ops, state
from tests.kvcase import INVALID, REL_TILE, assert_attention_close, bf16_normal, paged_layout, to_dev
from tests.test_gpu_paged_attention import TOL, make_pools, oracle_out

pytestmark = pytest.mark.gpu


def grouped_step(dev, fp8, qh, kvh, D, split):
    rng = np.random.default_rng(qh * 7 + fp8 + 2 * split)
    # (prefix, rows, class): 328 rows = 20 full tiles + 8 (3 groups of 8 tiles,
    # the last padded), 136 rows from position 0 (2 groups, the second one
    # tile and 7 empty), 128 rows (1 full group), decode rows between them
    reqs_spec = [(1500, 328, 2), (900, 1, 0), (0, 136, 2), (2100, 1, 0), (700, 128, 2),
                 (333, 1, 0)]
    lens = [p + n for p, n, _ in reqs_spec]
    lay = paged_layout(rng, lens, 16, kvh, D, spare_pages=2)
    kp, vp, ks, vs = make_pools(lay, fp8, 11 + qh, dev)
    slots, pos, reqs, row = [], [], [], 0
    for s, (p, n, cls) in enumerate(reqs_spec):
        slots += [s] * n
        pos += list(range(p, p + n))
        reqs.append((row, n, cls, p + n))
        row += n
    slots, pos = np.array(slots, np.uint32), np.array(pos, np.uint32)
    q = bf16_normal(rng, (row, qh * D))
    g = ops.PoolGeometry(1, lay.num_pages, 16, kvh, D)
    out = torch.full((row, qh * D), 7.0, dtype=torch.float32, device=dev)
    a = ops.attention_args(g, 0, to_dev(q), out, to_dev(slots), to_dev(pos),
                           to_dev(lay.block_tables), qh)
    nbytes = (64 << 20) if split else 0
    part = torch.empty(max(nbytes, 4) // 4, dtype=torch.float32, device=dev) if split else None
    maxvis = max(lens)
    kvd = P.KV_FP8 if fp8 else P.KV_BF16
    plan = state.plan_step(a, kvd, reqs, maxvis, nbytes, partials_ptr=part, k_pool=kp,
                           v_pool=vp, k_scale=ks, v_scale=vs, launch=True)
    torch.cuda.synchronize()
    want = oracle_out(lay, qh, q, slots, pos, lay.block_tables, kp, vp, ks, vs)
    return plan, out.cpu().numpy(), want


@pytest.mark.parametrize("fp8", [False, True])
@pytest.mark.parametrize("qh,kvh", [(24, 4), (20, 4)])   # 6 heads per group; 5 (a half-empty head part)
@pytest.mark.parametrize("split", [False, True])
def test_grouped_prefill_vs_oracle(dev, fp8, qh, kvh, split):
    plan, got, want = grouped_step(dev, fp8, qh, kvh, 256, split)
    kinds = [k.kind for k in plan.kernels[:plan.count]]
    assert kinds.count(1) == 1                      # one tile launch for the three prefill requests
    tile = [k for k in plan.kernels[:plan.count] if k.kind == 1][0]
    assert (tile.splits > 1) == split
    assert not np.any(got == 7.0)
    err = np.max(np.abs(got - want), axis=1)
    nan_rows = np.nonzero(np.isnan(got).any(axis=1))[0]
    nan_heads = sorted(set(np.nonzero(np.isnan(got.reshape(got.shape[0], qh, -1)).any(axis=2))[1].tolist()))
    assert np.max(err) < TOL[fp8], (int(np.argmax(err)), float(np.max(err)), len(nan_rows),
                                    nan_rows[:8].tolist(), nan_heads,
                                    [(k.kind, k.row_begin, k.rows, k.splits, k.pages_per_split, k.side)
                                     for k in plan.kernels[:plan.count]])
    assert_attention_close(got, want, TOL[fp8], REL_TILE[fp8], f"grouped prefill fp8={fp8} {qh}/{kvh} split={split}")


@pytest.mark.parametrize("qh,fp8,split", [(4, True, False), (8, False, True), (12, True, True),
                                           (16, True, False), (28, False, False), (32, True, True)])
def test_grouped_prefill_other_group_sizes(dev, qh, fp8, split):
    """Grouped launches for GQA groups of 1-8 heads (4 kv heads): head pairs,
    the second head of an odd group's last pair computed on zero Q and never
    written."""
    plan, got, want = grouped_step(dev, fp8, qh, 4, 256, split)
    tile = [k for k in plan.kernels[:plan.count] if k.kind == 1]
    assert len(tile) == 1 and (tile[0].splits > 1) == split
    assert not np.any(got == 7.0)
    assert_attention_close(got, want, TOL[fp8], REL_TILE[fp8], f"grouped prefill {qh}/4 fp8={fp8} split={split}")


def test_grouped_prefill_d128(dev):
    """head_dim 128 through the same grouped path."""
    rng = np.random.default_rng(3)
    lens = [400 + 200]
    lay = paged_layout(rng, lens, 16, 2, 128, spare_pages=2)
    kp, vp, ks, vs = make_pools(lay, True, 5, dev)
    slots = np.zeros(200, np.uint32)
    pos = np.arange(400, 600, dtype=np.uint32)
    q = bf16_normal(rng, (200, 12 * 128))
    g = ops.PoolGeometry(1, lay.num_pages, 16, 2, 128)
    out = torch.full((200, 12 * 128), 7.0, dtype=torch.float32, device=dev)
    a = ops.attention_args(g, 0, to_dev(q), out, to_dev(slots), to_dev(pos),
                           to_dev(lay.block_tables), 12)
    state.plan_step(a, P.KV_FP8, [(0, 200, 2, 600)], 600, 0, k_pool=kp, v_pool=vp, k_scale=ks,
                    v_scale=vs, launch=True)
    torch.cuda.synchronize()
    want = oracle_out(lay, 12, q, slots, pos, lay.block_tables, kp, vp, ks, vs)
    assert_attention_close(out.cpu().numpy(), want, TOL[True], REL_TILE[True], "test_gpu_tile_groups 1")


@pytest.mark.parametrize("fp8", [False, True])
def test_grouped_and_verify_tiles_page24(dev, fp8):
    """Page size 24 (not a multiple of 16): a 16-token half can straddle two
    pages, so every lane looks up its own page in both the grouped (prefill)
    and the six-wave (verify) tile kernels."""
    rng = np.random.default_rng(24 + fp8)
    spec = [(900, 200, 2), (1300, 16, 1), (40, 1, 0), (500, 136, 2)]
    lens = [p + n for p, n, _ in spec]
    P_ = 24
    lay = paged_layout(rng, lens, P_, 4, 256, spare_pages=2)
    kp, vp, ks, vs = make_pools(lay, fp8, 77 + fp8, dev)
    slots, pos, reqs, row = [], [], [], 0
    for s, (p, n, cls) in enumerate(spec):
        slots += [s] * n
        pos += list(range(p, p + n))
        reqs.append((row, n, cls, p + n))
        row += n
    slots, pos = np.array(slots, np.uint32), np.array(pos, np.uint32)
    q = bf16_normal(rng, (row, 24 * 256))
    g = ops.PoolGeometry(1, lay.num_pages, P_, 4, 256)
    out = torch.full((row, 24 * 256), 7.0, dtype=torch.float32, device=dev)
    a = ops.attention_args(g, 0, to_dev(q), out, to_dev(slots), to_dev(pos),
                           to_dev(lay.block_tables), 24)
    part = torch.empty((64 << 20) // 4, dtype=torch.float32, device=dev)
    plan = state.plan_step(a, P.KV_FP8 if fp8 else P.KV_BF16, reqs, max(lens), 64 << 20,
                           partials_ptr=part, k_pool=kp, v_pool=vp, k_scale=ks, v_scale=vs,
                           launch=True)
    torch.cuda.synchronize()
    assert [k.kind for k in plan.kernels[:plan.count]].count(1) == 2   # verify + prefill tiles
    want = oracle_out(lay, 24, q, slots, pos, lay.block_tables, kp, vp, ks, vs)
    got = out.cpu().numpy()
    assert not np.any(got == 7.0)
    assert_attention_close(got, want, TOL[fp8], REL_TILE[fp8], "test_gpu_tile_groups 2")


def invalid_page_step(dev, kvd, split, seed, pools_fn, oracle_fn):
    """A step whose first prefill request meets an invalid page (every row of
    it sees the page): its rows stay unwritten, split or not (a split that
    meets the page marks its partials and the combine skips the row), while
    the decode row, the verify block and the other prefill request are exact."""
    rng = np.random.default_rng(seed)
    spec = [(3000, 160, 2), (40, 1, 0), (2500, 96, 2), (700, 16, 1)]
    lens = [p + n for p, n, _ in spec]
    lay = paged_layout(rng, lens, 16, 4, 256, spare_pages=2)
    pools = pools_fn(lay)
    bt = lay.block_tables.copy()
    bt[0, 10] = INVALID
    slots, pos, reqs, row = [], [], [], 0
    for s, (p, n, cls) in enumerate(spec):
        slots += [s] * n
        pos += list(range(p, p + n))
        reqs.append((row, n, cls, p + n))
        row += n
    slots, pos = np.array(slots, np.uint32), np.array(pos, np.uint32)
    q = bf16_normal(rng, (row, 24 * 256))
    g = ops.PoolGeometry(1, lay.num_pages, 16, 4, 256)
    out = torch.full((row, 24 * 256), 7.0, dtype=torch.float32, device=dev)
    a = ops.attention_args(g, 0, to_dev(q), out, to_dev(slots), to_dev(pos), to_dev(bt), 24)
    nbytes = (64 << 20) if split else 0
    part = torch.empty(max(nbytes, 4) // 4, dtype=torch.float32, device=dev) if split else None
    plan = state.plan_step(a, kvd, reqs, max(lens), nbytes, part, *pools, launch=True)
    torch.cuda.synchronize()
    pre = max((k for k in plan.kernels[:plan.count] if k.kind == 1), key=lambda k: k.rows)
    assert (pre.splits > 1) == split
    got = out.cpu().numpy()
    assert np.all(got[:160] == 7.0)
    want = oracle_fn(lay, q[160:], slots[160:], pos[160:], bt, pools)
    return got[160:], want


@pytest.mark.parametrize("fp8", [False, True])
@pytest.mark.parametrize("split", [False, True])
def test_invalid_page_leaves_prefill_rows_unwritten(dev, fp8, split):
    got, want = invalid_page_step(
        dev, P.KV_FP8 if fp8 else P.KV_BF16, split, 31 + fp8 + 2 * split,
        lambda lay: make_pools(lay, fp8, 31 + fp8, dev),
        lambda lay, q, s, p, bt, pools: oracle_out(lay, 24, q, s, p, bt, *pools))
    assert not np.any(got == 7.0)
    assert_attention_close(got, want, TOL[fp8], REL_TILE[fp8], f"test_gpu_tile_groups 3 {(fp8, split)}")
