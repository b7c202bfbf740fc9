"""Paged-attention decode / split-K / verify tiles on the GPU vs the fp32 oracle.

Tolerances (north star): max-abs 2e-2 for BF16 KV, 5e-2 for FP8 KV, against the
oracle's fp32 two-pass softmax on the same (dequantized) KV.
Cases: the reference test's geometries (test_paged_attention.hip:585-743: GQA
8/4 hd64, MHA hd128, GQA 8/2 hd32, long visible 4097/8192/32768 at hd256 page64),
BASELINE config 3 (BF16, batch 32, 24/4 heads, hd256, ctx U[1k,32k]) and config 4
(FP8, batch 64, ctx log-U[4k,64k], split-K + combine), verify blocks (consecutive
positions of one sequence), and the edge rules (one visible token, invalid slot,
invalid page, empty splits).
Every comparison also holds each row to 1% of its own largest oracle output
(assert_attention_close), and peaked-softmax cases at 32k context give the
outputs a size the bounds bite on."""
import math

import numpy as np
import pytest
import torch

import oracle
from phaseshift_amd import ops
from tests.kvcase import (INVALID, REL_BF16_OUT, REL_DECODE, REL_TILE, assert_attention_close,
                          bf16_normal, oracle_attention_parallel, paged_layout, random_fp8_codes, to_dev, to_host)

pytestmark = pytest.mark.gpu

TOL = {False: 2e-2, True: 5e-2}


def close(got, want, fp8, what="", tile=False, bf16_out=False):
    rel = REL_TILE[fp8] if tile else REL_DECODE
    if bf16_out:
        rel += REL_BF16_OUT
    assert_attention_close(got, want, TOL[fp8], rel, what)


def make_pools(lay, fp8, seed, dev):
    """Pools filled on the device (seeded), plus host copies for the oracle."""
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    n = lay.pool_elems
    if fp8:
        kp = torch.randint(0, 256, (n,), generator=gen, device=dev, dtype=torch.int32)
        vp = torch.randint(0, 256, (n,), generator=gen, device=dev, dtype=torch.int32)
        # no NaN codes (0x7F / 0xFF)
        kp = torch.where((kp & 0x7F) == 0x7F, kp ^ 1, kp).to(torch.uint8)
        vp = torch.where((vp & 0x7F) == 0x7F, vp ^ 1, vp).to(torch.uint8)
        ks = torch.rand(lay.scale_elems, generator=gen, device=dev) * 0.02 + 0.001
        vs = torch.rand(lay.scale_elems, generator=gen, device=dev) * 0.02 + 0.001
    else:
        kp = torch.randn(n, generator=gen, device=dev).to(torch.bfloat16).view(torch.int16)
        vp = torch.randn(n, generator=gen, device=dev).to(torch.bfloat16).view(torch.int16)
        ks = vs = None
    return kp, vp, ks, vs


def host(t):
    return None if t is None else to_host(t)


def run_gpu(lay, q_heads, q, slots, pos, bt, kp, vp, ks, vs, out_dtype=torch.float32, splits=1,
            pages_per_split=0, kind="decode", out=None, q_pad=0, out_pad=0, layer=0):
    """q_pad / out_pad > 0: Q and the output are column slices of wider row-major
    buffers, so q_row_stride and output_row_stride exceed q_heads * head_dim
    (the strided views paged_attention_dispatch.hip:415-416 passes). The pad
    columns of the output must come back untouched (7.0)."""
    g = ops.PoolGeometry(lay.num_layers, lay.num_pages, lay.page_tokens, lay.kv_heads,
                         lay.head_dim)
    rows = q.shape[0]
    width = q_heads * lay.head_dim
    if q_pad:
        qw = np.zeros((rows, width + q_pad), np.uint16)
        qw[:, :width] = q
        qw[:, width:] = 0x7FC0                   # NaN: must never be read
        dq = to_dev(qw)[:, :width]
    else:
        dq = to_dev(q)
    full = None
    if out is None:
        full = torch.full((rows, width + out_pad), 7.0, dtype=out_dtype, device=kp.device)
        out = full[:, :width]
    partials = None
    if splits > 1:
        nbytes = ops.split_partials_bytes(rows, q_heads, lay.kv_heads, splits)
        partials = torch.empty(nbytes // 4, dtype=torch.float32, device=kp.device)
    ops.paged_attention(g, layer, dq, out, to_dev(np.asarray(slots, np.uint32)),
                        to_dev(np.asarray(pos, np.uint32)), to_dev(bt), kp, vp, q_heads,
                        ks, vs, splits=splits, pages_per_split=pages_per_split,
                        partials=partials, kind=kind)
    torch.cuda.synchronize()
    if full is not None and out_pad:
        assert torch.all(full[:, width:] == 7.0), "output pad columns were written"
    return out.float().cpu().numpy() if out.dtype != torch.float32 else out.cpu().numpy()


def oracle_out(lay, q_heads, q, slots, pos, bt, kp, vp, ks, vs, workers=8, layer=0):
    g = dict(lay.geom, q_heads=q_heads, block_table_stride=bt.shape[1], max_sequences=bt.shape[0],
             layer=layer)
    return oracle_attention_parallel(g, q, slots, pos, bt, host(kp), host(vp), host(ks), host(vs),
                                     1.0 / math.sqrt(lay.head_dim), workers=workers)


def case(seed, lens, q_heads, kv_heads, D, P, fp8, dev, spare=2):
    rng = np.random.default_rng(seed)
    lay = paged_layout(rng, lens, P, kv_heads, D, spare_pages=spare)
    kp, vp, ks, vs = make_pools(lay, fp8, seed, dev)
    q = bf16_normal(rng, (len(lens), q_heads * D))
    slots = np.arange(len(lens), dtype=np.uint32)
    pos = np.asarray(lens, np.uint32) - 1
    return rng, lay, kp, vp, ks, vs, q, slots, pos


@pytest.mark.parametrize("fp8", [False, True])
@pytest.mark.parametrize("qh,kvh,D,P,lens", [
    (8, 4, 64, 16, [1, 5, 16, 17, 100]),      # GQA 8/4 hd64
    (4, 4, 128, 16, [3, 31, 33, 64]),         # MHA hd128
    (8, 2, 32, 16, [2, 15, 47]),              # GQA 8/2 hd32
    (24, 4, 256, 64, [4097, 8192, 32768]),    # long visible, page 64
    (24, 4, 256, 16, [1, 2, 31, 32, 33, 1000]),
    (16, 1, 256, 16, [300, 7]),               # q_per_kv 16 (one full MFMA N block)
    (20, 1, 64, 16, [70]),                    # q_per_kv 20: generic kernel
    (6, 2, 96, 8, [50, 9]),                   # head_dim 96: generic kernel
])
def test_reference_geometries(dev, fp8, qh, kvh, D, P, lens):
    _, lay, kp, vp, ks, vs, q, slots, pos = case(qh * 31 + D + P, lens, qh, kvh, D, P, fp8, dev)
    bt = lay.block_tables
    want = oracle_out(lay, qh, q, slots, pos, bt, kp, vp, ks, vs)
    got = run_gpu(lay, qh, q, slots, pos, bt, kp, vp, ks, vs)
    close(got, want, fp8, f"geom qh{qh} kv{kvh} D{D} P{P} fp8={fp8}")
    if D in (64, 128, 256) and qh // kvh <= 16 and max(lens) > 64:
        for splits, pps in ((4, 0), (16, 0), (3, 2), (64, 1)):
            got_s = run_gpu(lay, qh, q, slots, pos, bt, kp, vp, ks, vs, splits=splits,
                            pages_per_split=pps)
            close(got_s, want, fp8, f"geom qh{qh} D{D} fp8={fp8} split {splits}/{pps}")


def test_config3_bf16_decode(dev):
    """batch 32, 24/4 heads, hd256, page 16, ctx U[1k,32k], bf16 out."""
    rng = np.random.default_rng(303)
    lens = rng.integers(1024, 32769, 32)
    _, lay, kp, vp, ks, vs, q, slots, pos = case(303, lens, 24, 4, 256, 16, False, dev)
    want = oracle_out(lay, 24, q, slots, pos, lay.block_tables, kp, vp, ks, vs)
    for splits in (1, 16):
        got = run_gpu(lay, 24, q, slots, pos, lay.block_tables, kp, vp, ks, vs,
                      out_dtype=torch.bfloat16, splits=splits)
        close(got, want, False, f"config3 splits {splits}", bf16_out=True)


def test_config4_fp8_split_decode(dev):
    """batch 64, FP8 KV, ctx log-U[4k,64k], split-K + combine.
    Every one of the 64 rows is checked against the oracle (about 3 GB of KV,
    threaded oracle), for three split layouts."""
    rng = np.random.default_rng(404)
    lens = np.exp(rng.uniform(np.log(4096), np.log(65536), 64)).astype(np.int64)
    _, lay, kp, vp, ks, vs, q, slots, pos = case(404, lens, 24, 4, 256, 16, True, dev)
    bt = lay.block_tables
    a = run_gpu(lay, 24, q, slots, pos, bt, kp, vp, ks, vs, splits=16)
    b = run_gpu(lay, 24, q, slots, pos, bt, kp, vp, ks, vs, splits=64, pages_per_split=64)
    c = run_gpu(lay, 24, q, slots, pos, bt, kp, vp, ks, vs, splits=1)
    want = oracle_out(lay, 24, q, slots, pos, bt, kp, vp, ks, vs, workers=16)
    for name, got in (("splits16", a), ("pps64", b), ("unsplit", c)):
        close(got, want, True, f"config4 {name}")


@pytest.mark.parametrize("fp8", [False, True])
def test_verify_block_rows_are_causal(dev, fp8):
    """DFlash2 verify block: 16 rows of one sequence at positions prefix..prefix+15
    (device_batch_context.hip:73-78); each row attends to [0, its position]."""
    rng = np.random.default_rng(55 + fp8)
    prefix = 2000
    lay = paged_layout(rng, [prefix + 16, 500], 16, 4, 256, spare_pages=3)
    kp, vp, ks, vs = make_pools(lay, fp8, 55, dev)
    rows = 16 + 1
    slots = np.array([0] * 16 + [1], np.uint32)
    pos = np.array(list(range(prefix, prefix + 16)) + [499], np.uint32)
    q = bf16_normal(rng, (rows, 24 * 256))
    want = oracle_out(lay, 24, q, slots, pos, lay.block_tables, kp, vp, ks, vs)
    for kind in ("decode", "prefill"):
        got = run_gpu(lay, 24, q, slots, pos, lay.block_tables, kp, vp, ks, vs, kind=kind)
        close(got, want, fp8, f"verify block {kind} fp8={fp8}", tile=kind == "prefill")


def test_single_visible_token_outputs_v(dev):
    _, lay, kp, vp, ks, vs, q, slots, pos = case(8, [1, 1], 24, 4, 256, 16, False, dev)
    got = run_gpu(lay, 24, q, slots, pos, lay.block_tables, kp, vp, ks, vs)
    V = to_host(vp).reshape(lay.num_pages, 16, 4, 256)
    for r in range(2):
        v0 = oracle.bf16_to_f32(V[lay.block_tables[r, 0], 0])     # [4, 256]
        want = np.repeat(v0, 6, axis=0).reshape(-1)
        # one visible token: its softmax weight is exactly 1
        assert np.array_equal(got[r], want)


@pytest.mark.parametrize("splits", [1, 8])
def test_invalid_slot_and_page_leave_output_unwritten(dev, splits):
    _, lay, kp, vp, ks, vs, q, slots, pos = case(12, [600, 600, 600, 600], 24, 4, 256, 16, True,
                                                 dev)
    bt = lay.block_tables.copy()
    bt[1, 20] = INVALID
    bt[2, 3] = 1 << 30
    slots = slots.copy()
    slots[3] = 1000
    got = run_gpu(lay, 24, q, slots, pos, bt, kp, vp, ks, vs, splits=splits)
    assert np.all(got[1] == 7.0) and np.all(got[2] == 7.0) and np.all(got[3] == 7.0)
    want = oracle_out(lay, 24, q[:1], slots[:1], pos[:1], bt, kp, vp, ks, vs)
    close(got[:1], want, True, "invalid slot/page, valid row")


def test_position_past_table_skips_row(dev):
    _, lay, kp, vp, ks, vs, q, slots, pos = case(13, [40, 40], 8, 4, 64, 16, False, dev)
    pos = pos.copy()
    pos[1] = 16 * lay.block_tables.shape[1]     # visible = stride*P + 1 > capacity
    got = run_gpu(lay, 8, q, slots, pos, lay.block_tables, kp, vp, ks, vs)
    assert np.all(got[1] == 7.0) and not np.all(got[0] == 7.0)


@pytest.mark.parametrize("fp8", [False, True])
def test_unsplit_independent_waves(dev, fp8):
    """>= 256 rows unsplit: the 4 waves of a workgroup are the 4 kv heads of one
    row and each writes its heads' output straight from registers."""
    rng = np.random.default_rng(71 + fp8)
    lens = rng.integers(1, 200, 300)
    _, lay, kp, vp, ks, vs, q, slots, pos = case(71 + fp8, lens, 24, 4, 256, 16, fp8, dev)
    want = oracle_out(lay, 24, q, slots, pos, lay.block_tables, kp, vp, ks, vs)
    got = run_gpu(lay, 24, q, slots, pos, lay.block_tables, kp, vp, ks, vs)
    close(got, want, fp8, f"unsplit independent fp8={fp8}")


@pytest.mark.parametrize("fp8", [False, True])
def test_independent_waves_partial_head_group(dev, fp8):
    """kv_heads = 6: the second group of each row has 2 of 4 waves active."""
    rng = np.random.default_rng(81 + fp8)
    lens = rng.integers(1, 90, 260)
    _, lay, kp, vp, ks, vs, q, slots, pos = case(81 + fp8, lens, 12, 6, 64, 16, fp8, dev)
    want = oracle_out(lay, 12, q, slots, pos, lay.block_tables, kp, vp, ks, vs)
    for splits, pps in ((1, 0), (3, 2)):
        got = run_gpu(lay, 12, q, slots, pos, lay.block_tables, kp, vp, ks, vs, splits=splits,
                      pages_per_split=pps)
        close(got, want, fp8, f"partial head group fp8={fp8} {splits}/{pps}")


def test_split_window_passes(dev):
    """Splits of more than 1024 pages stage the block table in several passes."""
    rng = np.random.default_rng(91)
    lens = np.array([40000, 20000, 17000, 1500] * 64)[:256]
    _, lay, kp, vp, ks, vs, q, slots, pos = case(91, lens[:4], 24, 4, 256, 16, True, dev)
    # 4 distinct rows replicated: 256 rows share 4 block tables
    bt = lay.block_tables
    reps = 64
    slots_r = np.tile(slots, reps)
    pos_r = np.tile(pos, reps)
    q_r = np.tile(q, (reps, 1))
    ref = run_gpu(lay, 24, q_r[:4], slots_r[:4], pos_r[:4], bt, kp, vp, ks, vs, splits=1)
    want = oracle_out(lay, 24, q[:4], slots[:4], pos[:4], bt, kp, vp, ks, vs)
    close(ref, want, True, "window passes unsplit")
    got = run_gpu(lay, 24, q_r, slots_r, pos_r, bt, kp, vp, ks, vs, splits=2, pages_per_split=1100)
    close(got, np.tile(want, (reps, 1)), True, "window passes split")


def test_invalid_page_independent_split(dev):
    """Invalid pages under the independent-wave split kernel (>= 256 units)."""
    _, lay, kp, vp, ks, vs, q, slots, pos = case(14, [600] * 8, 24, 4, 256, 16, True, dev)
    bt = lay.block_tables.copy()
    bt[1, 20] = INVALID
    bt[5, 3] = 1 << 30
    got = run_gpu(lay, 24, q, slots, pos, bt, kp, vp, ks, vs, splits=38, pages_per_split=1)
    assert np.all(got[1] == 7.0) and np.all(got[5] == 7.0)
    keep = [0, 2, 3, 4, 6, 7]
    want = oracle_out(lay, 24, q[keep], slots[keep], pos[keep], bt, kp, vp, ks, vs)
    close(got[keep], want, True, "invalid page independent split")


def peaked_case(seed, fp8, lens, qh=24, kvh=4, D=256, P=16, target_std=4.0):
    """Pools of well-scaled values (BF16 N(0,1); FP8 codes of magnitude 2^-2..3.75
    with scales in [0.25, 0.5]) and Q scaled by a power of two so the scores
    scale*q.k have a standard deviation near target_std: the softmax of a 32k
    row then puts most of its weight on a few tokens, and outputs are O(1)."""
    rng = np.random.default_rng(seed)
    lay = paged_layout(rng, lens, P, kvh, D, spare_pages=2)
    n = lay.pool_elems
    if fp8:
        def codes():
            e = rng.integers(5, 9, n, dtype=np.uint8)
            m = rng.integers(0, 8, n, dtype=np.uint8)
            s = rng.integers(0, 2, n, dtype=np.uint8)
            return (s << 7) | (e << 3) | m
        kp, vp = codes(), codes()
        ks = rng.uniform(0.25, 0.5, lay.scale_elems).astype(np.float32)
        vs = rng.uniform(0.25, 0.5, lay.scale_elems).astype(np.float32)
    else:
        kp, vp = bf16_normal(rng, n), bf16_normal(rng, n)
        ks = vs = None
    q0 = bf16_normal(rng, (len(lens), qh * D))
    # empirical score spread of row 0, head 0 over its first 128 pages
    bt = lay.block_tables[0]
    ept = kvh * D
    K, sc = [], []
    for p in bt[:128]:
        blk = kp[int(p) * P * ept:(int(p) + 1) * P * ept].reshape(P, kvh, D)[:, 0, :]
        K.append(oracle.e4m3_decode(blk) if fp8 else oracle.bf16_to_f32(blk))
        if fp8:
            sc.append(ks[(int(p) * P + np.arange(P)) * kvh])
    K = np.concatenate(K).astype(np.float64)
    if fp8:
        K *= np.concatenate(sc)[:, None]
    s = K @ oracle.bf16_to_f32(q0[0, :D]).astype(np.float64) / math.sqrt(D)
    factor = 2.0 ** round(math.log2(target_std / s.std()))
    q = oracle.f32_to_bf16(oracle.bf16_to_f32(q0) * np.float32(factor))
    return (lay, to_dev(kp), to_dev(vp), None if ks is None else to_dev(ks),
            None if vs is None else to_dev(vs), q)


@pytest.mark.parametrize("fp8", [False, True])
def test_peaked_softmax_32k(dev, fp8):
    """Scores with std ~4 at 32k context: decode (unsplit, reference split rule,
    chooser-size splits) and a 16-row verify tile at the end of a 32k row, all
    held to the oracle per row. The oracle outputs here reach O(1), so a kernel
    that drops or misweights tokens fails the bounds."""
    lens = [32768, 32768, 30001, 32768]
    lay, kp, vp, ks, vs, q = peaked_case(900 + fp8, fp8, lens)
    bt = lay.block_tables
    slots = np.arange(3, dtype=np.uint32)
    pos = np.asarray(lens[:3], np.uint32) - 1
    want = oracle_out(lay, 24, q[:3], slots, pos, bt, kp, vp, ks, vs)
    assert np.abs(want).max(axis=1).min() > 0.5    # the case is peaked
    for splits, pps in ((1, 0), (16, 0), (8, 256), (64, 32)):
        got = run_gpu(lay, 24, q[:3], slots, pos, bt, kp, vp, ks, vs, splits=splits,
                      pages_per_split=pps)
        close(got, want, fp8, f"peaked32k fp8={fp8} {splits}/{pps}")
    # verify block: 16 rows of slot 3 at positions 32752..32767
    rng = np.random.default_rng(77)
    qv = q[rng.integers(0, 4, 16)].copy()
    vslots = np.full(16, 3, np.uint32)
    vpos = np.arange(32752, 32768, dtype=np.uint32)
    want_v = oracle_out(lay, 24, qv, vslots, vpos, bt, kp, vp, ks, vs)
    for kind in ("decode", "prefill"):
        got = run_gpu(lay, 24, qv, vslots, vpos, bt, kp, vp, ks, vs, kind=kind)
        close(got, want_v, fp8, f"peaked32k verify {kind} fp8={fp8}", tile=kind == "prefill")


@pytest.mark.parametrize("fp8", [False, True])
def test_padded_q_and_output_strides(dev, fp8):
    """q_row_stride and output_row_stride larger than q_heads*head_dim: Q rows
    and output rows are column slices of wider buffers (the reference resolves
    both strides from tensor views, paged_attention_dispatch.hip:415-416). The
    pad columns of Q hold NaN and those of the output must stay untouched, on
    the decode, split-K and tile paths, for f32 and bf16 output."""
    lens = [3000, 700, 17, 2500]
    _, lay, kp, vp, ks, vs, q, slots, pos = case(611 + fp8, lens, 24, 4, 256, 16, fp8, dev)
    bt = lay.block_tables
    want = oracle_out(lay, 24, q, slots, pos, bt, kp, vp, ks, vs)
    for out_dtype in (torch.float32, torch.bfloat16):
        for splits, pps in ((1, 0), (4, 0), (5, 16)):
            got = run_gpu(lay, 24, q, slots, pos, bt, kp, vp, ks, vs, out_dtype=out_dtype,
                          splits=splits, pages_per_split=pps, q_pad=64, out_pad=40)
            close(got, want, fp8, f"padded fp8={fp8} {out_dtype} {splits}/{pps}",
                  bf16_out=out_dtype == torch.bfloat16)
    # a verify block through the tile path with the same padding
    vrows = 16
    vslots = np.zeros(vrows, np.uint32)
    vpos = np.arange(lens[0] - vrows, lens[0], dtype=np.uint32)
    qv = bf16_normal(np.random.default_rng(5), (vrows, 24 * 256))
    want_v = oracle_out(lay, 24, qv, vslots, vpos, bt, kp, vp, ks, vs)
    got = run_gpu(lay, 24, qv, vslots, vpos, bt, kp, vp, ks, vs, kind="prefill", q_pad=128,
                  out_pad=8)
    close(got, want_v, fp8, f"padded tile fp8={fp8}", tile=True)


@pytest.mark.parametrize("fp8", [False, True])
def test_layer_offset_in_multi_layer_pool(dev, fp8):
    """Pools of 3 attention layers, attention on layer 2 (and layer 1): every
    kernel adds the layer's offset to K/V and scale addresses (reference
    paged_kv_pool.cpp:64-75: [layers][pages][page_tokens][kv_heads][head_dim]).
    Decode unsplit and split, and a verify block on the tile kernel, each
    against the oracle on the same layer; the other layers hold different
    random values, so a wrong offset reads the wrong layer."""
    rng = np.random.default_rng(321 + fp8)
    lens = [2100, 600, 37]
    lay = paged_layout(rng, lens + [1200 + 16], 16, 4, 256, num_layers=3, spare_pages=2)
    kp, vp, ks, vs = make_pools(lay, fp8, 321 + fp8, dev)
    bt = lay.block_tables
    q = bf16_normal(rng, (3, 24 * 256))
    slots = np.arange(3, dtype=np.uint32)
    pos = np.asarray(lens, np.uint32) - 1
    vslots = np.full(16, 3, np.uint32)
    vpos = np.arange(1200, 1216, dtype=np.uint32)
    qv = bf16_normal(rng, (16, 24 * 256))
    for layer in (2, 1):
        want = oracle_out(lay, 24, q, slots, pos, bt, kp, vp, ks, vs, layer=layer)
        for splits, pps in ((1, 0), (4, 0), (7, 16)):
            got = run_gpu(lay, 24, q, slots, pos, bt, kp, vp, ks, vs, splits=splits,
                          pages_per_split=pps, layer=layer)
            close(got, want, fp8, f"layer {layer} fp8={fp8} {splits}/{pps}")
        want_v = oracle_out(lay, 24, qv, vslots, vpos, bt, kp, vp, ks, vs, layer=layer)
        got = run_gpu(lay, 24, qv, vslots, vpos, bt, kp, vp, ks, vs, kind="prefill", layer=layer)
        close(got, want_v, fp8, f"layer {layer} tile fp8={fp8}", tile=True)
