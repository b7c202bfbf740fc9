"""Split decode with many more (row, split) units than CUs: short units (8, 4,
3 and 1 pages; a one-page unit is shorter than a 32-token chunk), 15000-20000
units per launch, ragged row lengths, invalid pages inside single units, BF16
and FP8, all against the fp32 oracle."""
import numpy as np
import pytest

from tests.kvcase import INVALID, REL_DECODE, assert_attention_close
from tests.test_gpu_paged_attention import TOL, case, oracle_out, run_gpu

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("fp8", [False, True])
def test_many_short_units(dev, fp8):
    rng = np.random.default_rng(31 + fp8)
    lens = [int(x) for x in np.exp(rng.uniform(np.log(1500), np.log(40000), 24))]
    _, lay, kp, vp, ks, vs, q, slots, pos = case(41 + fp8, lens, 24, 4, 256, 16, fp8, dev)
    pps = 8
    splits = max((l + 16 * pps - 1) // (16 * pps) for l in lens)
    assert 24 * splits > 256                # more units than CUs
    got = run_gpu(lay, 24, q, slots, pos, lay.block_tables, kp, vp, ks, vs, splits=splits,
                  pages_per_split=pps)
    want = oracle_out(lay, 24, q, slots, pos, lay.block_tables, kp, vp, ks, vs)
    assert_attention_close(got, want, TOL[fp8], REL_DECODE, "test_gpu_decode_many_units 1")


def test_many_units_long_rows(dev):
    """24 rows x 40k tokens at 4 and 3 pages per split: 15000 and 20016 units."""
    lens = [40000 - 37 * i for i in range(24)]
    _, lay, kp, vp, ks, vs, q, slots, pos = case(43, lens, 24, 4, 256, 16, True, dev)
    want = oracle_out(lay, 24, q, slots, pos, lay.block_tables, kp, vp, ks, vs)
    for pps in (4, 3):
        splits = (max(lens) + 16 * pps - 1) // (16 * pps)
        assert splits <= 1024
        got = run_gpu(lay, 24, q, slots, pos, lay.block_tables, kp, vp, ks, vs, splits=splits,
                      pages_per_split=pps)
        assert_attention_close(got, want, TOL[True], REL_DECODE, f"test_gpu_decode_many_units 2 {pps}")


def test_one_page_units_with_invalid_pages(dev):
    """Units of one page; an invalid page in one unit of row 2 and one of row 9
    leaves exactly those rows unwritten, the rows around them exact."""
    lens = [700 + 13 * i for i in range(12)]
    _, lay, kp, vp, ks, vs, q, slots, pos = case(44, lens, 24, 4, 256, 16, True, dev)
    bt = lay.block_tables.copy()
    bt[2, 30] = INVALID
    bt[9, 0] = 1 << 30
    splits = max((l + 15) // 16 for l in lens)
    got = run_gpu(lay, 24, q, slots, pos, bt, kp, vp, ks, vs, splits=splits, pages_per_split=1)
    assert np.all(got[2] == 7.0) and np.all(got[9] == 7.0)
    keep = [i for i in range(12) if i not in (2, 9)]
    want = oracle_out(lay, 24, q[keep], slots[keep], pos[keep], bt, kp, vp, ks, vs)
    assert_attention_close(got[keep], want, TOL[True], REL_DECODE, "test_gpu_decode_many_units 3")
