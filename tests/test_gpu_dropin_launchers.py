"""The reference-signature launchers themselves, driven with data.

The reference dispatchers (kv_append_dispatch.hip:247-275,
paged_attention_dispatch.hip:790-894) bind the C++ entry points
`ps::kernel::launch_*` declared in kv_append.h:78-125 and
paged_attention.h:140-285. These tests call exactly those symbols, by their
Itanium-mangled names, with the reference ABI (the argument struct by const
reference, i.e. by address; hipStream_t last), and compare with the CPU oracle:
bit-exact for appends, the north-star attention tolerances plus a per-row 1%
bound for attention. The PSQ launchers are also held bit-identical to the
plain C-ABI (`psk_*`) entry points on the same inputs.

Covered: launch_kv_append_{bf16,fp8_e4m3,psq4,psq8},
launch_attention_paged_{bf16,fp8_e4m3} (the FP8 route an unmodified
dispatcher takes: unsplit), launch_attention_paged_bf16_split (16 splits, the
reference's fixed count) + launch_attention_paged_bf16_split_reduce,
launch_attention_paged_fp8_e4m3_split + launch_attention_paged_split_reduce_ex,
launch_attention_paged_prefill_{bf16,fp8_e4m3} on a verify block and a
128-row prefill chunk, launch_attention_paged_{,prefill_}psq{4,8} and
launch_attention_paged_psq{4,8}_split."""
import ctypes as C
import math

import numpy as np
import pytest
import torch

import oracle
import phaseshift_amd
from phaseshift_amd import ops
from tests.kvcase import (INVALID, REL_BF16_OUT, REL_DECODE, REL_TILE, assert_attention_close,
                          bf16_normal, oracle_attention_parallel, oracle_attention_psq_parallel, paged_layout, to_dev, to_host)

pytestmark = pytest.mark.gpu

_P, _U32 = C.c_void_p, C.c_uint32
# mangled name -> argtypes (every launcher returns hipError_t, an int)
MANGLED = {
    "launch_kv_append_bf16":
        ("_ZN2ps6kernel21launch_kv_append_bf16ERKNS0_18KvAppendCommonArgsEPNS_6bf16_tES5_P12ihipStream_t",
         [_P, _P, _P, _P]),
    "launch_kv_append_fp8_e4m3":
        ("_ZN2ps6kernel25launch_kv_append_fp8_e4m3ERKNS0_18KvAppendCommonArgsEPhS4_PfS5_P12ihipStream_t",
         [_P, _P, _P, _P, _P, _P]),
    "launch_kv_append_psq4":
        ("_ZN2ps6kernel21launch_kv_append_psq4ERKNS0_18KvAppendCommonArgsEPhS4_PNS_6bf16_tES6_jNS_6qwen3518Psq4ScaleEstimatorEP12ihipStream_t",
         [_P, _P, _P, _P, _P, _U32, C.c_int, _P]),
    "launch_kv_append_psq8":
        ("_ZN2ps6kernel21launch_kv_append_psq8ERKNS0_18KvAppendCommonArgsEPhS4_PNS_6bf16_tES6_jNS_6qwen3518Psq8ScaleEstimatorEP12ihipStream_t",
         [_P, _P, _P, _P, _P, _U32, C.c_int, _P]),
    "launch_attention_paged_bf16":
        ("_ZN2ps6kernel27launch_attention_paged_bf16ERKNS0_24PagedAttentionCommonArgsEPKNS_6bf16_tES6_P12ihipStream_t",
         [_P, _P, _P, _P]),
    "launch_attention_paged_fp8_e4m3":
        ("_ZN2ps6kernel31launch_attention_paged_fp8_e4m3ERKNS0_24PagedAttentionCommonArgsEPKhS5_PKfS7_P12ihipStream_t",
         [_P, _P, _P, _P, _P, _P]),
    "launch_attention_paged_bf16_split":
        ("_ZN2ps6kernel33launch_attention_paged_bf16_splitERKNS0_24PagedAttentionCommonArgsEPKNS_6bf16_tES6_PfjP12ihipStream_t",
         [_P, _P, _P, _P, _U32, _P]),
    "launch_attention_paged_bf16_split_reduce":
        ("_ZN2ps6kernel40launch_attention_paged_bf16_split_reduceERKNS0_24PagedAttentionCommonArgsEPKfjP12ihipStream_t",
         [_P, _P, _U32, _P]),
    "launch_attention_paged_fp8_e4m3_split":
        ("_ZN2ps6kernel37launch_attention_paged_fp8_e4m3_splitERKNS0_24PagedAttentionCommonArgsEPKhS5_PKfS7_PfjjP12ihipStream_t",
         [_P, _P, _P, _P, _P, _P, _U32, _U32, _P]),
    "launch_attention_paged_split_reduce_ex":
        ("_ZN2ps6kernel38launch_attention_paged_split_reduce_exERKNS0_24PagedAttentionCommonArgsEPKfjjP12ihipStream_t",
         [_P, _P, _U32, _U32, _P]),
    "launch_attention_paged_prefill_bf16":
        ("_ZN2ps6kernel35launch_attention_paged_prefill_bf16ERKNS0_24PagedAttentionCommonArgsEPKNS_6bf16_tES6_P12ihipStream_t",
         [_P, _P, _P, _P]),
    "launch_attention_paged_prefill_fp8_e4m3":
        ("_ZN2ps6kernel39launch_attention_paged_prefill_fp8_e4m3ERKNS0_24PagedAttentionCommonArgsEPKhS5_PKfS7_P12ihipStream_t",
         [_P, _P, _P, _P, _P, _P]),
    "launch_attention_paged_psq4":
        ("_ZN2ps6kernel27launch_attention_paged_psq4ERKNS0_24PagedAttentionCommonArgsEPKhS5_PKNS_6bf16_tES8_jP12ihipStream_t",
         [_P, _P, _P, _P, _P, _U32, _P]),
    "launch_attention_paged_psq8":
        ("_ZN2ps6kernel27launch_attention_paged_psq8ERKNS0_24PagedAttentionCommonArgsEPKhS5_PKNS_6bf16_tES8_jP12ihipStream_t",
         [_P, _P, _P, _P, _P, _U32, _P]),
    "launch_attention_paged_prefill_psq4":
        ("_ZN2ps6kernel35launch_attention_paged_prefill_psq4ERKNS0_24PagedAttentionCommonArgsEPKhS5_PKNS_6bf16_tES8_jP12ihipStream_t",
         [_P, _P, _P, _P, _P, _U32, _P]),
    "launch_attention_paged_prefill_psq8":
        ("_ZN2ps6kernel35launch_attention_paged_prefill_psq8ERKNS0_24PagedAttentionCommonArgsEPKhS5_PKNS_6bf16_tES8_jP12ihipStream_t",
         [_P, _P, _P, _P, _P, _U32, _P]),
    "launch_attention_paged_psq4_split":
        ("_ZN2ps6kernel33launch_attention_paged_psq4_splitERKNS0_24PagedAttentionCommonArgsEPKhS5_PKNS_6bf16_tES8_jPfjP12ihipStream_t",
         [_P, _P, _P, _P, _P, _U32, _P, _U32, _P]),
    "launch_attention_paged_psq8_split":
        ("_ZN2ps6kernel33launch_attention_paged_psq8_splitERKNS0_24PagedAttentionCommonArgsEPKhS5_PKNS_6bf16_tES8_jPfjP12ihipStream_t",
         [_P, _P, _P, _P, _P, _U32, _P, _U32, _P]),
}


@pytest.fixture(scope="module")
def ref_api(dev):
    """The reference-signature launchers of the built library, by mangled name."""
    cdll = C.CDLL(phaseshift_amd.LIB_PATH)
    fns = {}
    for name, (sym, argt) in MANGLED.items():
        f = getattr(cdll, sym)
        f.argtypes, f.restype = argt, C.c_int
        fns[name] = f
    return fns


def call(ref_api, name, *args):
    rc = ref_api[name](*args, torch.cuda.current_stream().cuda_stream)
    assert rc == 0, (name, rc)


def ptr(t):
    return None if t is None else t.data_ptr()


def geom_of(lay):
    return ops.PoolGeometry(lay.num_layers, lay.num_pages, lay.page_tokens, lay.kv_heads,
                            lay.head_dim)


# ------------------------------------------------------------------ append
@pytest.mark.parametrize("fp8", [False, True])
def test_append_launchers_bitexact(dev, ref_api, fp8):
    """launch_kv_append_{bf16,fp8_e4m3}: BASELINE config 1 (BF16, 2 kv heads, hd 128,
    lengths {7,33,64,100}) and config 2 (FP8, 4 kv heads, hd 256, 128 rows at
    U[0,32k), 1% x20 outliers), pools pre-filled with sentinels."""
    rng = np.random.default_rng(1701 + fp8)
    if fp8:
        rows, H, D = 128, 4, 256
        pos = rng.integers(0, 32768, rows).astype(np.uint32)
        lay = paged_layout(rng, [16] * rows, 16, H, D, spare_pages=16)
        bt = np.full((rows, 2048), INVALID, np.uint32)
        bt[np.arange(rows), pos // 16] = lay.block_tables[:, 0]
        slots = np.arange(rows, dtype=np.uint32)
        k = bf16_normal(rng, (rows, H * D), 0.01, 20.0)
        v = bf16_normal(rng, (rows, H * D), 0.01, 20.0)
    else:
        lens = [7, 33, 64, 100]
        lay = paged_layout(rng, lens, 16, 2, 128, spare_pages=64 - 15)
        bt = lay.block_tables
        slots = np.repeat(np.arange(4), lens).astype(np.uint32)
        pos = np.concatenate([np.arange(n) for n in lens]).astype(np.uint32)
        k, v = bf16_normal(rng, (len(pos), 256)), bf16_normal(rng, (len(pos), 256))
    g = geom_of(lay)
    dk_in, dv_in, dsl, dpos, dbt = to_dev(k), to_dev(v), to_dev(slots), to_dev(pos), to_dev(bt)
    a = ops.append_args(g, 0, dk_in, dv_in, dsl, dpos, dbt)
    if fp8:
        kp = np.full(lay.pool_elems, 0x3F, np.uint8)
        ks = np.full(lay.scale_elems, -1.0, np.float32)
    else:
        kp = np.full(lay.pool_elems, 0x3F3F, np.uint16)
        ks = None
    vp, vs = kp.copy(), (None if ks is None else ks.copy())
    dk, dv = to_dev(kp), to_dev(vp)
    if fp8:
        dks, dvs = to_dev(ks), to_dev(vs)
        call(ref_api, "launch_kv_append_fp8_e4m3", C.addressof(a), ptr(dk), ptr(dv), ptr(dks),
             ptr(dvs))
    else:
        call(ref_api, "launch_kv_append_bf16", C.addressof(a), ptr(dk), ptr(dv))
    torch.cuda.synchronize()
    og = dict(lay.geom, block_table_stride=bt.shape[1], max_sequences=bt.shape[0])
    oracle.kv_append(og, k, v, slots, pos, bt, kp, vp, ks, vs)
    assert np.array_equal(to_host(dk), kp) and np.array_equal(to_host(dv), vp)
    if fp8:
        assert np.array_equal(to_host(dks).view(np.uint32), ks.view(np.uint32))
        assert np.array_equal(to_host(dvs).view(np.uint32), vs.view(np.uint32))


# --------------------------------------------------------------- attention
def attention_case(fp8, seed, dev):
    """6 decode rows over 1k-9k tokens, then one 16-row verify block and one
    128-row prefill chunk, each of its own sequence (24/4 heads, hd 256, page 16)."""
    rng = np.random.default_rng(seed)
    dec = [int(x) for x in rng.integers(1024, 9000, 6)]
    lens = dec + [3000 + 16, 2000 + 128]
    lay = paged_layout(rng, lens, 16, 4, 256, spare_pages=2)
    n = lay.pool_elems
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    if fp8:
        kp = torch.randint(0, 256, (n,), generator=gen, device=dev, dtype=torch.int32)
        vp = torch.randint(0, 256, (n,), generator=gen, device=dev, dtype=torch.int32)
        kp = torch.where((kp & 0x7F) == 0x7F, kp ^ 1, kp).to(torch.uint8)
        vp = torch.where((vp & 0x7F) == 0x7F, vp ^ 1, vp).to(torch.uint8)
        ks = torch.rand(lay.scale_elems, generator=gen, device=dev) * 0.02 + 0.001
        vs = torch.rand(lay.scale_elems, generator=gen, device=dev) * 0.02 + 0.001
    else:
        kp = torch.randn(n, generator=gen, device=dev).to(torch.bfloat16).view(torch.int16)
        vp = torch.randn(n, generator=gen, device=dev).to(torch.bfloat16).view(torch.int16)
        ks = vs = None
    slots = np.array(list(range(6)) + [6] * 16 + [7] * 128, np.uint32)
    pos = np.array([x - 1 for x in dec] + list(range(3000, 3016)) + list(range(2000, 2128)),
                   np.uint32)
    q = bf16_normal(rng, (len(slots), 24 * 256))
    return lay, kp, vp, ks, vs, q, slots, pos


def oracle_of(lay, q, slots, pos, kp, vp, ks, vs):
    g = dict(lay.geom, q_heads=24)
    h = lambda t: None if t is None else to_host(t)
    return oracle_attention_parallel(g, q, slots, pos, lay.block_tables, h(kp), h(vp), h(ks), h(vs),
                                     1.0 / 16)


def region(lay, q, slots, pos, lo, hi, dev, out_dtype=torch.float32):
    """Argument struct of rows [lo, hi) plus its output tensor (kept alive)."""
    g = geom_of(lay)
    dq = to_dev(q[lo:hi])
    out = torch.full((hi - lo, 24 * 256), 7.0, dtype=out_dtype, device=dev)
    a = ops.attention_args(g, 0, dq, out, to_dev(slots[lo:hi]), to_dev(pos[lo:hi]),
                           to_dev(lay.block_tables), 24)
    return a, out


def result(out):
    torch.cuda.synchronize()
    return out.float().cpu().numpy()


@pytest.mark.parametrize("fp8", [False, True])
def test_attention_launchers(dev, ref_api, fp8):
    lay, kp, vp, ks, vs, q, slots, pos = attention_case(fp8, 2024 + fp8, dev)
    want = oracle_of(lay, q, slots, pos, kp, vp, ks, vs)
    tol = 5e-2 if fp8 else 2e-2
    pools = (ptr(kp), ptr(vp)) + ((ptr(ks), ptr(vs)) if fp8 else ())
    dec = slice(0, 6)
    # unsplit decode: what the reference dispatcher launches for FP8, and for BF16
    # below 2048 visible tokens
    for out_dtype in (torch.float32, torch.bfloat16):
        a, out = region(lay, q, slots, pos, 0, 6, dev, out_dtype)
        call(ref_api, "launch_attention_paged_fp8_e4m3" if fp8 else "launch_attention_paged_bf16",
             C.addressof(a), *pools)
        rel = REL_DECODE + (REL_BF16_OUT if out_dtype == torch.bfloat16 else 0.0)
        assert_attention_close(result(out), want[dec], tol, rel, f"unsplit {out_dtype}")
    # split-K: BF16 at the reference's 16 splits + its reduce; FP8 additive split + reduce_ex
    rows = 6
    nbytes = ops.split_partials_bytes(rows, 24, 4, 16)
    part = torch.empty(nbytes // 4, dtype=torch.float32, device=dev)
    a, out = region(lay, q, slots, pos, 0, 6, dev)
    if fp8:
        call(ref_api, "launch_attention_paged_fp8_e4m3_split", C.addressof(a), *pools, ptr(part), 16, 0)
        call(ref_api, "launch_attention_paged_split_reduce_ex", C.addressof(a), ptr(part), 16, 0)
    else:
        call(ref_api, "launch_attention_paged_bf16_split", C.addressof(a), *pools, ptr(part), 16)
        call(ref_api, "launch_attention_paged_bf16_split_reduce", C.addressof(a), ptr(part), 16)
    assert_attention_close(result(out), want[dec], tol, REL_DECODE, "split16")
    # multi-row tiles: the verify block (16 rows) and the prefill chunk (128 rows)
    name = "launch_attention_paged_prefill_fp8_e4m3" if fp8 else "launch_attention_paged_prefill_bf16"
    for lo, hi in ((6, 22), (22, 150)):
        a, out = region(lay, q, slots, pos, lo, hi, dev)
        call(ref_api, name, C.addressof(a), *pools)
        assert_attention_close(result(out), want[lo:hi], tol, REL_TILE[fp8], f"prefill rows {lo}:{hi}")


def test_launchers_reject_bad_geometry(dev, ref_api):
    """hipErrorInvalidValue (1) on null pools and rows == 0, as the reference."""
    lay, kp, vp, ks, vs, q, slots, pos = attention_case(False, 7, dev)
    a, out = region(lay, q, slots, pos, 0, 6, dev)
    s = torch.cuda.current_stream().cuda_stream
    assert ref_api["launch_attention_paged_bf16"](C.addressof(a), None, ptr(vp), s) == 1
    a.rows = 0
    assert ref_api["launch_attention_paged_bf16"](C.addressof(a), ptr(kp), ptr(vp), s) == 1
    torch.cuda.synchronize()
    assert torch.all(out == 7.0)


# --------------------------------------------------------------------- PSQ
@pytest.mark.parametrize("fmt", [4, 8])
def test_psq_launchers_match_capi_and_oracle(dev, ref_api, fmt):
    """launch_kv_append_psq{4,8} (both estimators) bit-identical to psk_kv_append_psq*;
    launch_attention_paged_{,prefill_}psq* and the split launcher against the
    oracle over the appended pools, and bit-identical to the psk_* calls."""
    rng = np.random.default_rng(31 + fmt)
    dec = [int(x) for x in rng.integers(300, 2500, 4)]
    lens = dec + [1000 + 16]
    lay = paged_layout(rng, lens, 16, 4, 256, spare_pages=1)
    g = geom_of(lay)
    slots = np.concatenate([np.full(n, i, np.uint32) for i, n in enumerate(lens)])
    pos = np.concatenate([np.arange(n, dtype=np.uint32) for n in lens])
    # no outliers here: outputs stay O(1), where the north-star max-abs bound
    # bites (append with outliers is held bit-exact in test_gpu_psq.py)
    k_in = bf16_normal(rng, (len(pos), 1024))
    v_in = bf16_normal(rng, (len(pos), 1024))
    dk_in, dv_in, dsl, dpos, dbt = (to_dev(k_in), to_dev(v_in), to_dev(slots), to_dev(pos),
                                    to_dev(lay.block_tables))
    nb, cb = g.psq_blocks, g.psq_code_bytes(fmt)

    def pools():
        return (torch.zeros(cb, dtype=torch.uint8, device=dev), torch.zeros(cb, dtype=torch.uint8, device=dev),
                torch.zeros(nb, dtype=torch.int16, device=dev), torch.zeros(nb, dtype=torch.int16, device=dev))

    name = f"launch_kv_append_psq{fmt}"
    for est in (0, 1):
        ref_p, capi_p = pools(), pools()
        a = ops.append_args(g, 0, dk_in, dv_in, dsl, dpos, dbt)
        call(ref_api, name, C.addressof(a), *map(ptr, ref_p), 8, est)
        ops.kv_append_psq(g, 0, dk_in, dv_in, dsl, dpos, dbt, *capi_p, fmt, est)
        torch.cuda.synchronize()
        for x, y in zip(ref_p, capi_p):
            assert torch.equal(x, y), (fmt, est)
    kc, vc, ks, vs = ref_p          # LSQ1 pools
    h = [to_host(t) for t in ref_p]
    # decode rows: the last token of each of the 4 sequences; verify: slot 4's 16 rows
    qs = bf16_normal(rng, (4 + 16, 24 * 256))
    rs = np.array(list(range(4)) + [4] * 16, np.uint32)
    rp = np.array([n - 1 for n in dec] + list(range(1000, 1016)), np.uint32)
    og = dict(lay.geom, q_heads=24)
    want = oracle_attention_psq_parallel(og, qs, rs, rp, lay.block_tables, *h, fmt, 1.0 / 16)
    P = (ptr(kc), ptr(vc), ptr(ks), ptr(vs), 8)

    def args(lo, hi):
        dq = to_dev(qs[lo:hi])
        out = torch.full((hi - lo, 24 * 256), 7.0, dtype=torch.float32, device=dev)
        return ops.attention_args(g, 0, dq, out, to_dev(rs[lo:hi]), to_dev(rp[lo:hi]), dbt, 24), out, dq

    a, out, dq = args(0, 4)
    call(ref_api, f"launch_attention_paged_psq{fmt}", C.addressof(a), *P)
    got = result(out)
    assert_attention_close(got, want[:4], 5e-2, 1e-2, f"psq{fmt} unsplit")
    out2 = torch.full_like(out, 7.0)
    ops.paged_attention_psq(g, 0, dq, out2, to_dev(rs[:4]), to_dev(rp[:4]), dbt, kc, vc, ks, vs,
                            24, fmt)
    assert np.array_equal(result(out2), got)
    # the reference split launcher (q_per_kv 4 or 6, 2/4/8/16 splits) + reduce
    part = torch.empty(ops.split_partials_bytes(4, 24, 4, 8) // 4, dtype=torch.float32, device=dev)
    a, out, _ = args(0, 4)
    call(ref_api, f"launch_attention_paged_psq{fmt}_split", C.addressof(a), *P, ptr(part), 8)
    # the reference follows a PSQ split with the bf16 reduce (paged_attention_dispatch.hip:811-832)
    call(ref_api, "launch_attention_paged_bf16_split_reduce", C.addressof(a), ptr(part), 8)
    assert_attention_close(result(out), want[:4], 5e-2, 1e-2, f"psq{fmt} split8")
    a, out, _ = args(4, 20)
    call(ref_api, f"launch_attention_paged_prefill_psq{fmt}", C.addressof(a), *P)
    assert_attention_close(result(out), want[4:], 5e-2, 1e-2, f"psq{fmt} verify tile")
