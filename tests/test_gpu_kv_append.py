"""KV append on the GPU vs the oracle: bit-exact pools and scales.

Cases: BASELINE config 1 (BF16, 2 KV heads, hd 128, page 16, lengths
{7,33,64,100}, 64-page seeded permutation) with sentinel bytes
(FP8, 4 KV heads, hd 256, 128 rows at U[0,32k) positions, 1% x20 outliers); the
ROCm-converter golden fixture; the reference test's geometries
(test_kv_append.hip:562-637: kvh4 hd256 page16 layers 2/4, hd64 page4); ragged
head_dim (no vector path); skip rules; a 2^16-row round trip."""
import os

import numpy as np
import pytest
import torch

import oracle
from phaseshift_amd import ops
from tests.kvcase import INVALID, bf16_normal, paged_layout, to_dev, to_host

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


def geom_of(lay):
    return ops.PoolGeometry(lay.num_layers, lay.num_pages, lay.page_tokens, lay.kv_heads,
                            lay.head_dim)


def run_both(lay, layer, k, v, slots, pos, bt, fp8, sentinel=0x3F):
    g = geom_of(lay)
    og = dict(lay.geom, layer=layer, block_table_stride=bt.shape[1], max_sequences=bt.shape[0])
    if fp8:
        kp = np.full(lay.pool_elems, sentinel, np.uint8)
        ks = np.full(lay.scale_elems, -1.0, np.float32)
    else:
        kp = np.full(lay.pool_elems, sentinel * 0x101, np.uint16)
        ks = None
    vp, vs = kp.copy(), (None if ks is None else ks.copy())
    dk, dv = to_dev(kp), to_dev(vp)
    dks = to_dev(ks) if fp8 else None
    dvs = to_dev(vs) if fp8 else None
    ops.kv_append(g, layer, to_dev(k), to_dev(v), to_dev(np.asarray(slots, np.uint32)),
                  to_dev(np.asarray(pos, np.uint32)), to_dev(bt), dk, dv, dks, dvs)
    torch.cuda.synchronize()
    oracle.kv_append(og, k, v, slots, pos, bt, kp, vp, ks, vs)
    assert np.array_equal(to_host(dk), kp)
    assert np.array_equal(to_host(dv), vp)
    if fp8:
        assert np.array_equal(to_host(dks).view(np.uint32), ks.view(np.uint32))
        assert np.array_equal(to_host(dvs).view(np.uint32), vs.view(np.uint32))
    return kp


def test_config1_bf16_append_bitexact_with_sentinels(dev):
    rng = np.random.default_rng(101)
    lens = [7, 33, 64, 100]
    lay = paged_layout(rng, lens, 16, 2, 128, spare_pages=64 - 15)
    slots = np.repeat(np.arange(4), lens).astype(np.uint32)
    pos = np.concatenate([np.arange(n) for n in lens]).astype(np.uint32)
    k, v = bf16_normal(rng, (len(pos), 256)), bf16_normal(rng, (len(pos), 256))
    run_both(lay, 0, k, v, slots, pos, lay.block_tables, fp8=False)


def test_config2_fp8_append_bitexact(dev):
    rng = np.random.default_rng(202)
    rows, H, D, P = 128, 4, 256, 16
    pos = rng.integers(0, 32768, rows).astype(np.uint32)
    # each sequence has the page of its append position mapped (the decode
    # step's newly reserved page); the rest of its 2048-entry table is empty
    lay = paged_layout(rng, [P] * rows, P, H, D, spare_pages=16)
    bt = np.full((rows, 2048), INVALID, np.uint32)
    bt[np.arange(rows), pos // P] = lay.block_tables[:, 0]
    k = bf16_normal(rng, (rows, H * D), 0.01, 20.0)
    v = bf16_normal(rng, (rows, H * D), 0.01, 20.0)
    run_both(lay, 0, k, v, np.arange(rows, dtype=np.uint32), pos, bt, fp8=True)


def test_fp8_append_matches_rocm_golden_fixture(dev):
    R, H, D = 128, 4, 256
    k = np.fromfile(f"{GOLDEN}/fp8_append_k_in.bf16", np.uint16).reshape(R, H * D)
    v = np.fromfile(f"{GOLDEN}/fp8_append_v_in.bf16", np.uint16).reshape(R, H * D)
    g = ops.PoolGeometry(1, R, 16, H, D)
    bt = to_dev(np.arange(R, dtype=np.uint32).reshape(R, 1))
    kp = torch.zeros(R * 16 * H * D, dtype=torch.uint8, device=dev)
    vp = torch.zeros_like(kp)
    ks = torch.zeros(R * 16 * H, dtype=torch.float32, device=dev)
    vs = torch.zeros_like(ks)
    ops.kv_append(g, 0, to_dev(k), to_dev(v), to_dev(np.arange(R, dtype=np.uint32)),
                  to_dev(np.zeros(R, np.uint32)), bt, kp, vp, ks, vs)
    torch.cuda.synchronize()
    for t, pool, sc in (("k", kp, ks), ("v", vp, vs)):
        codes = np.fromfile(f"{GOLDEN}/fp8_append_{t}_codes.u8", np.uint8).reshape(R, H, D)
        scale = np.fromfile(f"{GOLDEN}/fp8_append_{t}_scale.f32", np.float32).reshape(R, H)
        got = to_host(pool).reshape(R, 16, H, D)[:, 0]
        assert np.array_equal(got, codes)
        assert np.array_equal(to_host(sc).reshape(R, 16, H)[:, 0].view(np.uint32),
                              scale.view(np.uint32))


@pytest.mark.parametrize("fp8", [False, True])
@pytest.mark.parametrize("layers,layer,H,D,P,rows", [(2, 1, 4, 256, 16, 8), (4, 3, 4, 256, 16, 4),
                                                     (1, 0, 4, 256, 16, 1), (1, 0, 2, 64, 4, 37),
                                                     (2, 1, 3, 100, 5, 19), (1, 0, 1, 520, 16, 9)])
def test_reference_geometries_and_ragged(dev, fp8, layers, layer, H, D, P, rows):
    rng = np.random.default_rng(layers * 100 + D + rows)
    lens = [rows + 3, rows // 2 + 1]
    lay = paged_layout(rng, lens, P, H, D, num_layers=layers, spare_pages=5)
    # distinct (slot, position) targets, as in a real step
    pairs = [(s, p) for s in range(2) for p in range(lens[s])]
    pick = rng.choice(len(pairs), rows, replace=False)
    slots = np.array([pairs[i][0] for i in pick], np.uint32)
    pos = np.array([pairs[i][1] for i in pick], np.uint32)
    k = bf16_normal(rng, (rows, H * D + 8), 0.05, 30.0)   # row stride > kv_heads*head_dim
    v = bf16_normal(rng, (rows, H * D + 8), 0.05, 30.0)
    k[0, :D] = 0   # all-zero head -> scale 1.0
    run_both(lay, layer, k, v, slots, pos, lay.block_tables, fp8)


@pytest.mark.parametrize("fp8", [False, True])
def test_invalid_rows_are_skipped(dev, fp8):
    rng = np.random.default_rng(9)
    lay = paged_layout(rng, [64, 64], 16, 4, 256, spare_pages=2)
    bt = lay.block_tables.copy()
    bt[1, 2] = INVALID
    bt[0, 3] = 10_000   # page id >= num_pages
    slots = np.array([0, 7, 1, 0, 1, 0], np.uint32)          # slot 7 >= max_sequences
    pos = np.array([1, 2, 40, 50, 1 << 20, 63], np.uint32)   # 1<<20: block past the table
    k, v = bf16_normal(rng, (6, 1024)), bf16_normal(rng, (6, 1024))
    run_both(lay, 0, k, v, slots, pos, bt, fp8)


def test_large_append_round_trip(dev):
    """2^16 decode rows (FP8, config-2 shape): bit-exact vs the oracle on every row."""
    rng = np.random.default_rng(77)
    rows, H, D, P = 1 << 16, 4, 256, 16
    seqs = rows // P                      # every sequence fills one page, all 16 slots
    lay = paged_layout(rng, [P] * seqs, P, H, D)
    slots = np.repeat(np.arange(seqs), P).astype(np.uint32)
    pos = np.tile(np.arange(P), seqs).astype(np.uint32)
    perm = rng.permutation(rows)          # rows in random order
    k = bf16_normal(rng, (rows, H * D), 0.01, 20.0)
    v = bf16_normal(rng, (rows, H * D), 0.01, 20.0)
    run_both(lay, 0, k, v, slots[perm], pos[perm], lay.block_tables, fp8=True)


@pytest.mark.parametrize("fp8", [False, True])
def test_append_overwrites_positions(dev, fp8):
    """A second append to positions already written replaces their K/V (and
    FP8 scales) and leaves the rest of the pool as the first append wrote it
    (the reference test's overwrite case, test_qwen35_mtp_kv_cache.hip:146-229):
    two launches against the oracle applied in the same order."""
    rng = np.random.default_rng(404)
    lens = [40, 17]
    lay = paged_layout(rng, lens, 16, 4, 256, spare_pages=2)
    g = geom_of(lay)
    og = dict(lay.geom, layer=0, block_table_stride=lay.block_tables.shape[1],
              max_sequences=lay.block_tables.shape[0])
    slots = np.repeat(np.arange(2), lens).astype(np.uint32)
    pos = np.concatenate([np.arange(n) for n in lens]).astype(np.uint32)
    k, v = bf16_normal(rng, (len(pos), 1024)), bf16_normal(rng, (len(pos), 1024))
    # second launch: positions 15, 16 (a page boundary) and 39 of sequence 0,
    # position 0 of sequence 1
    slots2 = np.array([0, 0, 0, 1], np.uint32)
    pos2 = np.array([15, 16, 39, 0], np.uint32)
    k2, v2 = bf16_normal(rng, (4, 1024)), bf16_normal(rng, (4, 1024))
    if fp8:
        kp = np.full(lay.pool_elems, 0x3F, np.uint8)
        ks = np.full(lay.scale_elems, -1.0, np.float32)
    else:
        kp = np.full(lay.pool_elems, 0x3F3F, np.uint16)
        ks = None
    vp, vs = kp.copy(), (None if ks is None else ks.copy())
    dk, dv = to_dev(kp), to_dev(vp)
    dks, dvs = (to_dev(ks), to_dev(vs)) if fp8 else (None, None)
    bt = to_dev(lay.block_tables)
    for kk, vv, ss, pp in ((k, v, slots, pos), (k2, v2, slots2, pos2)):
        ops.kv_append(g, 0, to_dev(kk), to_dev(vv), to_dev(ss), to_dev(pp), bt, dk, dv, dks, dvs)
        oracle.kv_append(og, kk, vv, ss, pp, lay.block_tables, kp, vp, ks, vs)
    torch.cuda.synchronize()
    assert np.array_equal(to_host(dk), kp)
    assert np.array_equal(to_host(dv), vp)
    if fp8:
        assert np.array_equal(to_host(dks).view(np.uint32), ks.view(np.uint32))
        assert np.array_equal(to_host(dvs).view(np.uint32), vs.view(np.uint32))
    # and the second launch did change the pool
    kp1 = np.full_like(kp, 0x3F if fp8 else 0x3F3F)
    vp1 = kp1.copy()
    ks1 = None if ks is None else np.full_like(ks, -1.0)
    vs1 = None if vs is None else ks1.copy()
    oracle.kv_append(og, k, v, slots, pos, lay.block_tables, kp1, vp1, ks1, vs1)
    assert not np.array_equal(kp1, kp)   # the second launch changed the pool


@pytest.mark.parametrize("fp8", [False, True])
@pytest.mark.parametrize("kvh,D", [(4, 256), (2, 128), (3, 100)])
def test_append_from_requests_equals_metadata_then_append(dev, fp8, kvh, D):
    """psk_kv_append_*_from_requests (row metadata and append in one launch)
    against psk_prepare_row_metadata followed by psk_kv_append_*: the same
    pool bytes, scales, slots and positions, bit for bit, and both against the
    oracle's append. 150 requests (more than one 64-descriptor pass), given
    out of row order: decode rows, a 16-row verify block, prefill chunks of
    40 rows, and two rows (between requests) that no request covers, whose
    slot/position entries must stay untouched and which are not appended.
    head_dim 100 takes the two-launch route (no fast path)."""
    rng = np.random.default_rng(7 + D + kvh + fp8)
    spec = [(1, 0)] * 140 + [(16, 1)] + [(40, 2)] * 9
    lens, descs, row = [], [], 0
    gaps = {60, 145}
    for i, (cnt, cls) in enumerate(spec):
        if i in gaps:
            row += 1
        prefix = int(rng.integers(0, 300))
        lens.append(prefix + cnt)
        descs.append(dict(slot=i, row_begin=row, row_count=cnt, prefix_length=prefix, execution_class=cls))
        row += cnt
    rows = row
    lay = paged_layout(rng, lens, 16, kvh, D, spare_pages=3)
    order = rng.permutation(len(descs))
    raw = to_dev(np.frombuffer(ops.pack_requests([descs[i] for i in order]), np.uint8).copy())
    g = geom_of(lay)
    k, v = bf16_normal(rng, (rows, kvh * D), 0.01), bf16_normal(rng, (rows, kvh * D), 0.01)
    dk_in, dv_in, bt = to_dev(k), to_dev(v), to_dev(lay.block_tables)

    def pools():
        if fp8:
            return (to_dev(np.full(lay.pool_elems, 0x3F, np.uint8)), to_dev(np.full(lay.pool_elems, 0x3F, np.uint8)),
                    to_dev(np.full(lay.scale_elems, -1.0, np.float32)),
                    to_dev(np.full(lay.scale_elems, -1.0, np.float32)))
        return (to_dev(np.full(lay.pool_elems, 0x3F3F, np.uint16)),
                to_dev(np.full(lay.pool_elems, 0x3F3F, np.uint16)), None, None)

    sentinel = np.full(rows, 0xABCD1234, np.uint32)
    s1, p1 = to_dev(sentinel), to_dev(sentinel)
    a1 = pools()
    ops.prepare_row_metadata(raw, len(descs), rows, s1, p1)
    ops.kv_append(g, 0, dk_in, dv_in, s1, p1, bt, *a1)
    s2, p2 = to_dev(sentinel), to_dev(sentinel)
    a2 = pools()
    ops.kv_append_from_requests(g, 0, dk_in, dv_in, raw, len(descs), s2, p2, bt, *a2)
    torch.cuda.synchronize()
    assert np.array_equal(to_host(s1), to_host(s2)) and np.array_equal(to_host(p1), to_host(p2))
    hs, hp = to_host(s2), to_host(p2)
    gap_rows = np.nonzero(hs == 0xABCD1234)[0]
    assert len(gap_rows) == 2 and np.all(hp[gap_rows] == 0xABCD1234)
    for t1, t2 in zip(a1, a2):
        if t1 is not None:
            assert np.array_equal(to_host(t1).view(np.uint8), to_host(t2).view(np.uint8))
    # and the oracle's append over the covered rows
    covered = np.nonzero(hs != 0xABCD1234)[0]
    og = dict(lay.geom, block_table_stride=lay.block_tables.shape[1], max_sequences=lay.block_tables.shape[0])
    kp = np.full(lay.pool_elems, 0x3F if fp8 else 0x3F3F, np.uint8 if fp8 else np.uint16)
    vp = kp.copy()
    ks = np.full(lay.scale_elems, -1.0, np.float32) if fp8 else None
    vs = None if ks is None else ks.copy()
    oracle.kv_append(og, k[covered], v[covered], hs[covered], hp[covered], lay.block_tables, kp, vp, ks, vs)
    assert np.array_equal(to_host(a2[0]), kp) and np.array_equal(to_host(a2[1]), vp)
    if fp8:
        assert np.array_equal(to_host(a2[2]).view(np.uint32), ks.view(np.uint32))
