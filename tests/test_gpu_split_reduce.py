"""The split-K combine kernel on synthetic partials, against the oracle's
restatement of the reference combine (paged_decode.hip:474-555; the
reference's own exactness test sweeps rows {1,2,4,8} x splits {2,4,8,16} x
head_dim {128,256} with extreme running maxima,
test_paged_attention_split_reduce_exact.hip:144-190). Here the per-split
maxima spread over +-80 (so some splits' weights underflow to zero), the
number of used splits varies per row with its visible length, a NaN maximum
(a split that met an invalid page) leaves that (row, head) output unwritten,
and rows of an invalid slot stay unwritten."""
import ctypes as C

import numpy as np
import pytest
import torch

import oracle
import phaseshift_amd as P
from phaseshift_amd import ops
from tests.kvcase import to_dev

pytestmark = pytest.mark.gpu

HEAD_LIMIT = 256   # the partial layout reserves 256 dims per head


def reduce_case(rows, splits, D, seed, qh=8, kvh=2, page=16, pps=3):
    rng = np.random.default_rng(seed)
    qpk = qh // kvh
    # visible lengths giving 1..splits used splits of pps pages each
    vis = rng.integers(1, splits * pps * page + 1, rows)
    vis[0] = splits * pps * page            # every split used
    if rows > 1:
        vis[1] = 1                          # one split
    pages = int(((vis + page - 1) // page).max())
    stride = qpk * (2 + HEAD_LIMIT)
    part = np.zeros((rows, kvh, splits, stride), np.float32)
    part[..., :qpk] = rng.uniform(-80.0, 80.0, (rows, kvh, splits, qpk))          # m (natural log)
    part[..., qpk:2 * qpk] = rng.uniform(0.5, 40.0, (rows, kvh, splits, qpk))     # l
    part[..., 2 * qpk:] = rng.standard_normal((rows, kvh, splits, qpk * HEAD_LIMIT)) * 3.0  # A
    n_used = np.minimum(splits, (((vis + page - 1) // page) + pps - 1) // pps).astype(np.uint32)
    slots = np.arange(rows, dtype=np.uint32)
    return dict(qh=qh, kvh=kvh, page=page, pps=pps, vis=vis, pages=pages, part=part,
                n_used=n_used, slots=slots, D=D)


def run_reduce(dev, c, splits, slots=None):
    rows, D, qh = len(c["vis"]), c["D"], c["qh"]
    g = ops.PoolGeometry(1, c["pages"] * rows + 1, c["page"], c["kvh"], D)
    q = torch.zeros((rows, qh * D), dtype=torch.bfloat16, device=dev)
    out = torch.full((rows, qh * D), 7.0, dtype=torch.float32, device=dev)
    bt = np.arange(rows * c["pages"], dtype=np.uint32).reshape(rows, c["pages"])
    sl = c["slots"] if slots is None else slots
    a = ops.attention_args(g, 0, q, out, to_dev(sl), to_dev((c["vis"] - 1).astype(np.uint32)),
                           to_dev(bt), qh)
    part = torch.from_numpy(c["part"]).to(dev)
    st = torch.cuda.current_stream().cuda_stream
    P.check("reduce", P.lib().psk_attention_paged_split_reduce_ex(C.byref(a), part.data_ptr(), splits,
                                                                   c["pps"], st))
    torch.cuda.synchronize()
    return out.cpu().numpy()


def oracle_reduce(c, splits, slots=None):
    rows = len(c["vis"])
    geom = dict(q_heads=c["qh"], kv_heads=c["kvh"], head_dim=c["D"], max_sequences=rows)
    return oracle.split_reduce(geom, c["part"], splits, c["n_used"],
                               c["slots"] if slots is None else slots, rows)


@pytest.mark.parametrize("D", [128, 256])
@pytest.mark.parametrize("splits", [2, 4, 8, 16])
@pytest.mark.parametrize("rows", [1, 2, 4, 8])
def test_split_reduce_vs_oracle(dev, rows, splits, D):
    c = reduce_case(rows, splits, D, 1000 * rows + 10 * splits + D)
    got = run_reduce(dev, c, splits)
    want = oracle_reduce(c, splits)
    # exp through exp2 on the device: a few ulp per weight
    np.testing.assert_allclose(got, want, rtol=2e-5, atol=2e-5 * np.abs(want).max())


def test_split_reduce_nan_split_and_invalid_slot_leave_rows_unwritten(dev):
    splits, D, rows = 8, 256, 4
    c = reduce_case(rows, splits, D, 77)
    c["vis"][:] = splits * c["pps"] * c["page"]          # every split used
    c["n_used"][:] = splits
    c["part"][2, 1, 5, 3] = np.nan                       # row 2, kv head 1, split 5, head 3
    slots = c["slots"].copy()
    slots[3] = 1000                                      # invalid slot
    got = run_reduce(dev, c, splits, slots)
    want = oracle_reduce(c, splits, slots)
    qpk = c["qh"] // c["kvh"]
    for r in (0, 1):
        np.testing.assert_allclose(got[r], want[r], rtol=2e-5, atol=2e-5 * np.abs(want[r]).max())
    # the NaN split's (row, kv head, head) output stays at the sentinel, the
    # row's other heads are combined
    h = 1 * qpk + 3
    assert np.all(got[2, h * D:(h + 1) * D] == 7.0)
    other = np.ones(c["qh"], bool)
    other[h] = False
    for hh in np.nonzero(other)[0]:
        w = want[2, hh * D:(hh + 1) * D]
        np.testing.assert_allclose(got[2, hh * D:(hh + 1) * D], w, rtol=2e-5, atol=2e-5 * np.abs(w).max())
    assert np.all(got[3] == 7.0)
