"""psk_attention_paged_fp8_e4m3_split_noalloc (allocation-free split decode:
partials in the library's static device array) against the caller-workspace
path (psk_attention_paged_fp8_e4m3_split + psk_attention_paged_split_reduce_ex)
on the same inputs, through the C-ABI: bit-identical outputs on two calls in a
row, the second with a smaller input (fewer rows, shorter contexts, fewer
splits), and a clear error when the partials would not fit the array."""
import ctypes as C

import numpy as np
import pytest
import torch

from phaseshift_amd import lib, ops
from tests.test_gpu_paged_attention import case, oracle_out, run_gpu

pytestmark = pytest.mark.gpu

SCRATCH = 32 << 20


def noalloc(lay, q, slots, pos, kp, vp, ks, vs, splits, pps, dev):
    g = ops.PoolGeometry(lay.num_layers, lay.num_pages, lay.page_tokens, lay.kv_heads,
                         lay.head_dim)
    from tests.kvcase import to_dev
    dq = to_dev(q)
    out = torch.full((q.shape[0], 24 * lay.head_dim), 7.0, dtype=torch.float32, device=dev)
    a = ops.attention_args(g, 0, dq, out, to_dev(np.asarray(slots, np.uint32)),
                           to_dev(np.asarray(pos, np.uint32)), to_dev(lay.block_tables), 24)
    rc = lib().psk_attention_paged_fp8_e4m3_split_noalloc(
        C.byref(a), kp.data_ptr(), vp.data_ptr(), ks.data_ptr(), vs.data_ptr(), splits, pps,
        torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    return rc, out.cpu().numpy()


def test_noalloc_matches_workspace_path_twice(dev):
    big = [int(x) for x in np.random.default_rng(1).integers(3000, 40000, 40)]
    small = [int(x) for x in np.random.default_rng(2).integers(100, 5000, 7)]
    cases = []
    for lens, splits, pps in ((big, 12, 0), (small, 4, 24)):
        _, lay, kp, vp, ks, vs, q, slots, pos = case(len(lens) * 7 + splits, lens, 24, 4, 256, 16,
                                                     True, dev)
        assert ops.split_partials_bytes(len(lens), 24, 4, splits) <= SCRATCH
        cases.append((lay, kp, vp, ks, vs, q, slots, pos, splits, pps))
    # two allocation-free calls in a row, the second smaller: it reuses the
    # array the first one filled
    got = []
    for lay, kp, vp, ks, vs, q, slots, pos, splits, pps in cases:
        rc, out = noalloc(lay, q, slots, pos, kp, vp, ks, vs, splits, pps, dev)
        assert rc == 0
        got.append(out)
    for (lay, kp, vp, ks, vs, q, slots, pos, splits, pps), out in zip(cases, got):
        want = run_gpu(lay, 24, q, slots, pos, lay.block_tables, kp, vp, ks, vs, splits=splits,
                       pages_per_split=pps)
        assert np.array_equal(out, want), (q.shape[0], splits)
        assert not np.any(out == 7.0)
    # and the oracle on the small case
    ref = oracle_out(lay, 24, q, slots, pos, lay.block_tables, kp, vp, ks, vs)
    assert np.max(np.abs(got[1] - ref)) < 5e-2


def test_noalloc_rejects_partials_beyond_the_array(dev):
    lens = [4096] * 64
    _, lay, kp, vp, ks, vs, q, slots, pos = case(5, lens, 24, 4, 256, 16, True, dev)
    too_many = 1 + SCRATCH // ops.split_partials_bytes(64, 24, 4, 1)
    assert ops.split_partials_bytes(64, 24, 4, too_many) > SCRATCH
    rc, got = noalloc(lay, q, slots, pos, kp, vp, ks, vs, too_many, 0, dev)
    assert rc == 1                       # hipErrorInvalidValue, nothing launched
    assert np.all(got == 7.0)
