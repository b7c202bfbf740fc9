"""Gather, batched page copy, u32 fill (truncation) and row metadata on the GPU,
bit-exact against the oracle / closed forms."""
import numpy as np
import pytest
import torch

import oracle
from phaseshift_amd import ops
from tests.kvcase import INVALID, bf16_normal, paged_layout, random_fp8_codes, to_dev, to_host

pytestmark = pytest.mark.gpu


def test_config1_gather_inverts_append(dev):
    """append 204 rows (BF16, 2 heads, hd128), gather back to
    contiguous [seq, token, head, dim]: bit-exact with the appended input."""
    rng = np.random.default_rng(1)
    lens = [7, 33, 64, 100]
    lay = paged_layout(rng, lens, 16, 2, 128, spare_pages=64 - 15)
    g = ops.PoolGeometry(1, 64, 16, 2, 128)
    slots = np.repeat(np.arange(4), lens).astype(np.uint32)
    pos = np.concatenate([np.arange(n) for n in lens]).astype(np.uint32)
    k = bf16_normal(rng, (len(pos), 256))
    v = bf16_normal(rng, (len(pos), 256))
    kp = torch.zeros(lay.pool_elems, dtype=torch.int16, device=dev)
    vp = torch.zeros_like(kp)
    bt = to_dev(lay.block_tables)
    ops.kv_append(g, 0, to_dev(k), to_dev(v), to_dev(slots), to_dev(pos), bt, kp, vp)
    offs = to_dev(np.concatenate([[0], np.cumsum(lens)]).astype(np.uint32))
    for pool, src in ((kp, k), (vp, v)):
        out = torch.zeros((len(pos), 256), dtype=torch.int16, device=dev)
        ops.kv_gather(g, 0, pool, bt, to_dev(np.arange(4, dtype=np.uint32)), offs, out)
        torch.cuda.synchronize()
        assert np.array_equal(to_host(out), src)
        want = oracle.kv_gather(lay.geom, to_host(pool), lay.block_tables, np.arange(4), lens)
        assert np.array_equal(to_host(out), want)


def test_fp8_gather_codes_and_scales(dev):
    rng = np.random.default_rng(2)
    lens = [50, 3, 129]
    lay = paged_layout(rng, lens, 16, 4, 256, num_layers=2, spare_pages=4)
    g = ops.PoolGeometry(2, lay.num_pages, 16, 4, 256)
    codes = random_fp8_codes(rng, lay.pool_elems)
    scales = rng.random(lay.scale_elems).astype(np.float32)
    bt = to_dev(lay.block_tables)
    offs_np = np.concatenate([[0], np.cumsum(lens)]).astype(np.uint32)
    seq = to_dev(np.arange(3, dtype=np.uint32))
    out = torch.zeros((sum(lens), 1024), dtype=torch.uint8, device=dev)
    ops.kv_gather(g, 1, to_dev(codes), bt, seq, to_dev(offs_np), out)
    sout = torch.zeros((sum(lens), 4), dtype=torch.float32, device=dev)
    ops.kv_gather(g, 1, to_dev(scales), bt, seq, to_dev(offs_np), sout, elem_bytes=4,
                  elems_per_token=4, elems_per_page=64)
    torch.cuda.synchronize()
    geom = dict(lay.geom, layer=1)
    assert np.array_equal(to_host(out), oracle.kv_gather(geom, codes, lay.block_tables,
                                                         np.arange(3), lens))
    assert np.array_equal(to_host(sout), oracle.kv_gather(geom, scales, lay.block_tables,
                                                          np.arange(3), lens, 4, 64))


@pytest.mark.parametrize("fp8", [False, True])
@pytest.mark.parametrize("P,H,D", [(16, 4, 256), (7, 3, 100)])
def test_batched_page_copy(dev, fp8, P, H, D):
    """32 prefix pages copied between two pools (prefix-cache save), every layer,
    K, V and the FP8 scale rows (paged_kv_pool.cpp:338-542). Page 7 x 3 heads
    x 100: page bodies (2100 / 4200 B) and scale rows (84 B) that are not
    multiples of 16 B, so pages after the first start unaligned."""
    rng = np.random.default_rng(3 + fp8 + P)
    L, NS, ND = 3, 80, 64
    eb = 1 if fp8 else 2
    src = {k: random_fp8_codes(rng, L * NS * P * H * D * eb) for k in "kv"}
    dst = {k: random_fp8_codes(rng, L * ND * P * H * D * eb) for k in "kv"}
    if fp8:
        src.update({k + "_scale": rng.random(L * NS * P * H).astype(np.float32) for k in "kv"})
        dst.update({k + "_scale": rng.random(L * ND * P * H).astype(np.float32) for k in "kv"})
    pairs = np.stack([rng.permutation(ND)[:32], rng.permutation(NS)[:32]], 1).astype(np.uint32)
    dd = {k: to_dev(v) for k, v in dst.items()}
    if not fp8:
        dd = {k: v.view(torch.int16) if k in "kv" else v for k, v in dd.items()}
    sd = {k: to_dev(v) for k, v in src.items()}
    if not fp8:
        sd = {k: v.view(torch.int16) if k in "kv" else v for k, v in sd.items()}
    ops.copy_pages(ops.PoolGeometry(L, ND, P, H, D), dd, sd, to_dev(pairs), src_num_pages=NS)
    torch.cuda.synchronize()
    for dp, sp in pairs:
        oracle.copy_page(dst, src, int(dp), int(sp), dict(layers=L, dst_num_pages=ND,
                                                          src_num_pages=NS, page_tokens=P,
                                                          kv_heads=H, head_dim=D, elem_bytes=eb))
    for k in dst:
        got = to_host(dd[k])
        assert np.array_equal(got.view(np.uint8) if k in "kv" else got, dst[k]), k


def test_fill_u32_truncates_block_table(dev):
    bt = torch.arange(64 * 100, dtype=torch.int32, device=dev).view(64, 100)
    ops.fill_u32(bt[7, 30:], INVALID)
    torch.cuda.synchronize()
    h = to_host(bt)
    assert np.all(h[7, 30:] == INVALID) and np.array_equal(h[7, :30], np.arange(700, 730))
    assert np.array_equal(h[8], np.arange(800, 900))


def test_row_metadata(dev):
    descs = [dict(slot=5, row_begin=0, row_count=3, prefix_length=100),
             dict(slot=2, row_begin=3, row_count=16, prefix_length=2000, execution_class=1),
             dict(slot=9, row_begin=19, row_count=600, prefix_length=0, execution_class=2)]
    raw = np.frombuffer(ops.pack_requests(descs), np.uint8)
    slots = torch.full((619,), -1, dtype=torch.int32, device=dev)
    pos = torch.full((619,), -1, dtype=torch.int32, device=dev)
    ops.prepare_row_metadata(to_dev(raw), 3, 619, slots, pos)
    torch.cuda.synchronize()
    want_s = np.array([5] * 3 + [2] * 16 + [9] * 600)
    want_p = np.concatenate([100 + np.arange(3), 2000 + np.arange(16), np.arange(600)])
    assert np.array_equal(slots.cpu().numpy(), want_s)
    assert np.array_equal(pos.cpu().numpy(), want_p)
