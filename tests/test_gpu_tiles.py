"""Multi-row tile kernel (verify blocks, chunked prefill) vs the fp32 oracle:
causal rows of one sequence, ragged tiles, GQA groups of 1..8, split-K with the
shared combine, and the tile contract (rows of another slot left unwritten)."""
import ctypes as C
import math

import numpy as np
import pytest
import torch

import phaseshift_amd as P
from phaseshift_amd import ops
from tests.kvcase import (REL_BF16_OUT, REL_TILE, assert_attention_close, bf16_normal,
                          oracle_attention_parallel, paged_layout, to_dev, to_host)
from tests.test_gpu_paged_attention import TOL, make_pools, oracle_out

pytestmark = pytest.mark.gpu


def tile_case(seed, prefix, chunk, qh, kvh, D, fp8, dev, P_=16, extra_seqs=()):
    rng = np.random.default_rng(seed)
    lens = [prefix + chunk] + list(extra_seqs)
    lay = paged_layout(rng, lens, P_, kvh, D, spare_pages=2)
    kp, vp, ks, vs = make_pools(lay, fp8, seed, dev)
    slots = np.array([0] * chunk, np.uint32)
    pos = np.arange(prefix, prefix + chunk, dtype=np.uint32)
    q = bf16_normal(rng, (chunk, qh * D))
    return lay, kp, vp, ks, vs, q, slots, pos


def run_tile(lay, qh, q, slots, pos, kp, vp, ks, vs, splits=1, pps=0, out_dtype=torch.float32):
    g = ops.PoolGeometry(lay.num_layers, lay.num_pages, lay.page_tokens, lay.kv_heads, lay.head_dim)
    rows = q.shape[0]
    out = torch.full((rows, qh * lay.head_dim), 7.0, dtype=out_dtype, device=kp.device)
    dq, ds, dp, dbt = to_dev(q), to_dev(slots), to_dev(pos), to_dev(lay.block_tables)
    a = ops.attention_args(g, 0, dq, out, ds, dp, dbt, qh)
    L = P.lib()
    fp8 = kp.dtype == torch.uint8
    p = lambda t: None if t is None else t.data_ptr()
    if splits == 1:
        fn = L.psk_attention_paged_prefill_fp8_e4m3 if fp8 else L.psk_attention_paged_prefill_bf16
        args = (C.byref(a), p(kp), p(vp)) + ((p(ks), p(vs)) if fp8 else ()) + (None,)
        P.check("prefill", fn(*args))
    else:
        nb = ops.split_partials_bytes(rows, qh, lay.kv_heads, splits)
        part = torch.empty(nb // 4, dtype=torch.float32, device=kp.device)
        P.check("tile_split", L.psk_attention_paged_tile_split(
            C.byref(a), P.KV_FP8 if fp8 else P.KV_BF16, p(kp), p(vp), p(ks), p(vs),
            part.data_ptr(), splits, pps, None))
        P.check("reduce", L.psk_attention_paged_split_reduce_ex(C.byref(a), part.data_ptr(),
                                                                 splits, pps, None))
    torch.cuda.synchronize()
    return out.float().cpu().numpy()


@pytest.mark.parametrize("fp8", [False, True])
@pytest.mark.parametrize("qh,kvh,D,prefix,chunk", [
    (24, 4, 256, 2000, 16),    # DFlash2 verify block: 16 drafts
    (24, 4, 256, 700, 512),    # chunked prefill, 512-row chunk
    (24, 4, 256, 0, 37),       # first chunk of a sequence, ragged last tile
    (8, 4, 128, 130, 50),      # GQA 2
    (16, 2, 64, 64, 33),       # GQA 8 (largest tile group)
    (32, 4, 256, 600, 40),     # GQA 8 at head_dim 256 (8 one-head waves)
    (4, 4, 128, 90, 20),       # MHA
])
def test_tile_vs_oracle(dev, fp8, qh, kvh, D, prefix, chunk):
    lay, kp, vp, ks, vs, q, slots, pos = tile_case(qh + D + chunk, prefix, chunk, qh, kvh, D, fp8, dev)
    want = oracle_out(lay, qh, q, slots, pos, lay.block_tables, kp, vp, ks, vs)
    got = run_tile(lay, qh, q, slots, pos, kp, vp, ks, vs)
    assert_attention_close(got, want, TOL[fp8], REL_TILE[fp8], "test_gpu_tiles 1")
    if prefix + chunk >= 512:
        got_s = run_tile(lay, qh, q, slots, pos, kp, vp, ks, vs, splits=8, pps=8)
        assert_attention_close(got_s, want, TOL[fp8], REL_TILE[fp8], "test_gpu_tiles 2")


def test_tile_bf16_output_and_page64(dev):
    lay, kp, vp, ks, vs, q, slots, pos = tile_case(9, 3000, 40, 24, 4, 256, True, dev, P_=64)
    want = oracle_out(lay, 24, q, slots, pos, lay.block_tables, kp, vp, ks, vs)
    got = run_tile(lay, 24, q, slots, pos, kp, vp, ks, vs, out_dtype=torch.bfloat16)
    assert_attention_close(got, want, 5e-2, REL_TILE[True] + REL_BF16_OUT, "test_gpu_tiles 3")


def test_tile_rows_of_other_sequence_left_unwritten(dev):
    """The tile contract: rows of a tile whose slot differs from the tile's first
    row are not computed (paged_prefill.hip:152-164 assumes one sequence)."""
    lay, kp, vp, ks, vs, q, slots, pos = tile_case(3, 100, 16, 24, 4, 256, True, dev,
                                                   extra_seqs=[50])
    slots = slots.copy()
    pos = pos.copy()
    slots[10:] = 1
    pos[10:] = np.arange(40, 46)
    got = run_tile(lay, 24, q, slots, pos, kp, vp, ks, vs)
    assert np.all(got[10:] == 7.0)
    want = oracle_out(lay, 24, q[:10], slots[:10], pos[:10], lay.block_tables, kp, vp, ks, vs)
    assert_attention_close(got[:10], want, 5e-2, REL_TILE[True], "test_gpu_tiles 4")


@pytest.mark.parametrize("fp8", [False, True])
@pytest.mark.parametrize("splits,pps", [(64, 16), (5, 120), (13, 79)])
def test_split_tiles_of_uneven_lengths(dev, fp8, splits, pps):
    """Split ungrouped tiles run as dense (tile, split) units, longest first:
    16-row blocks over contexts from 40 to 9000 tokens leave most of the
    (tile, split) grid empty. Also covered: a tile whose rows name no valid
    sequence (skipped, rows untouched) and a tile whose last rows belong to
    another sequence: the tile kernel leaves their partials alone and the
    combine then writes those rows from partials nobody produced, so they are
    not compared (the unsplit contract is
    test_tile_rows_of_other_sequence_left_unwritten)."""
    qh, kvh, D = 24, 4, 256
    rng = np.random.default_rng(41 + splits)
    prefixes = [9000, 40, 3000, 900, 6000]
    lens = [p_ + 16 for p_ in prefixes]
    lay = paged_layout(rng, lens, 16, kvh, D, spare_pages=2)
    kp, vp, ks, vs = make_pools(lay, fp8, 77, dev)
    slots = np.concatenate([np.full(16, i, np.uint32) for i in range(len(lens))])
    pos = np.concatenate([np.arange(p_, p_ + 16, dtype=np.uint32) for p_ in prefixes])
    slots[16:32] = 1000           # tile 1: no valid sequence
    slots[16 * 3 + 12:16 * 4] = 2  # tile 3: last 4 rows of another sequence
    pos[16 * 3 + 12:16 * 4] = np.arange(10, 14)
    q = bf16_normal(rng, (len(slots), qh * D))
    got = run_tile(lay, qh, q, slots, pos, kp, vp, ks, vs, splits=splits, pps=pps)
    assert np.all(got[16:32] == 7.0)
    cmp = np.ones(len(slots), bool)
    cmp[16:32] = False
    cmp[16 * 3 + 12:16 * 4] = False
    want = oracle_out(lay, qh, q[cmp], slots[cmp], pos[cmp], lay.block_tables, kp, vp, ks, vs)
    assert_attention_close(got[cmp], want, TOL[fp8], REL_TILE[fp8], f"uneven tiles {splits}/{pps}")


@pytest.mark.parametrize("fp8", [False, True])
def test_split_tiles_beyond_the_dense_limit(dev, fp8):
    """A split tile launch with more tiles x splits than the dense numbering
    takes (70 implicit tiles x 16 splits = 1120 > 1024) runs on the plain
    (tile, kv head, split) grid: a 1120-row chunk after a 200-token prefix,
    8 pages per split, every row against the oracle."""
    lay, kp, vp, ks, vs, q, slots, pos = tile_case(91, 200, 1120, 24, 4, 256, fp8, dev)
    want = oracle_out(lay, 24, q, slots, pos, lay.block_tables, kp, vp, ks, vs)
    got = run_tile(lay, 24, q, slots, pos, kp, vp, ks, vs, splits=16, pps=8)
    assert_attention_close(got, want, TOL[fp8], REL_TILE[fp8], "tiles beyond the dense limit")
