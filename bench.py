"""Benchmark of the paged KV-cache hot path on one MI355X.

Metric: paged decode-attention HBM GB/s (% of the 8 TB/s peak)
plus KV-append tokens/s, 1 GPU.

Workload of `value` (one "step" = one decode pass over one batch): FP8 E4M3 KV
paged decode, batch 64, every row at context 32768, 24 query / 4 KV heads,
head_dim 256, page 16, split-K + combine — the north-star point. Inputs are
synthetic (seeded random codes/scales/queries) and resident in HBM before the
timed region. Algorithmic bytes per step = sum over rows of ctx * 2080.25 B
(K+V codes 2*4*256, K+V scales 2*4*4, 1/16 of a 4 B block-table entry) plus
the query rows (24*256*2 B each).

Extra lines inside the same JSON object: BASELINE config 4 (log-uniform
contexts) and config 3 (BF16 KV), and KV append at config 2 (128 rows) and at
2^16 rows, each with kernel times from HIP events on the launch stream.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBPS = 8000.0
BYTES_PER_TOKEN_FP8 = 2 * 4 * 256 + 2 * 4 * 4 + 4 / 16      # 2080.25
BYTES_PER_TOKEN_BF16 = 2 * 4 * 256 * 2 + 4 / 16              # 4096.25
APPEND_BYTES_PER_ROW_FP8 = 2 * 4 * 256 * 2 + 8 + 4 + 2 * 4 * 256 + 2 * 4 * 4   # 6188
# PSQ: per (token, kv head) K and V codes (hd/2 or hd bytes) + hd/32 bf16 block scales
BYTES_PER_TOKEN_PSQ = {4: 2 * 4 * (128 + 16) + 4 / 16, 8: 2 * 4 * (256 + 16) + 4 / 16}
APPEND_BYTES_PER_ROW_PSQ = {f: 2 * 4 * 256 * 2 + 8 + 4 + BYTES_PER_TOKEN_PSQ[f] - 4 / 16 for f in (4, 8)}
# HBM bytes per main-line decode launch measured with rocprofv3 --pmc on this
# kernel (FETCH_SIZE 2,131,849 KiB x 2.0 calibration + WRITE_SIZE 6,206 KiB).
DECODE_TRAFFIC_BYTES = 2131849 * 1024 * 2 + 6206 * 1024
# Untimed warm-up runs at least `--warmup` steps and at least this long, so the
# GPU clocks have ramped before a timed loop starts.
WARM_MIN_S = 0.2


def warm(torch, fn, steps):
    """Runs fn() at least `steps` times and for at least WARM_MIN_S seconds."""
    t0 = time.perf_counter()
    n = 0
    while n < steps or time.perf_counter() - t0 < WARM_MIN_S:
        fn()
        n += 1
        if n % 16 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--only", default="", help="comma list: main,cfg4,cfg3,append,cfg5,prefill,psq,prefix,graph,loop,dropin")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="run only a plain 1 GiB device-to-device copy (5 times), the reference "
                         "kernel for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE")
    return ap.parse_args()


class Timer:
    """HIP-event timing on the stream the kernels are launched on."""

    def __init__(self, torch):
        self.torch = torch
        self.s = torch.cuda.Event(enable_timing=True)
        self.e = torch.cuda.Event(enable_timing=True)

    def __enter__(self):
        self.s.record()
        return self

    def __exit__(self, *a):
        self.e.record()

    def ms(self):
        self.e.synchronize()
        return self.s.elapsed_time(self.e)


def decode_setup(torch, ops, lens, fp8, seed, dev):
    rows = len(lens)
    P, H, D, QH = 16, 4, 256, 24
    rng = np.random.default_rng(seed)
    need = [(int(n) + P - 1) // P for n in lens]
    num_pages = sum(need)
    stride = max(need)
    perm = torch.from_numpy(rng.permutation(num_pages).astype(np.int32))
    bt = torch.full((rows, stride), -1, dtype=torch.int32)
    k = 0
    for r, n in enumerate(need):
        bt[r, :n] = perm[k:k + n]
        k += n
    g = ops.PoolGeometry(1, num_pages, P, H, D)
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    if fp8:
        kp = torch.randint(0, 126, (g.pool_elems,), generator=gen, device=dev,
                           dtype=torch.int32).to(torch.uint8)
        vp = torch.randint(0, 126, (g.pool_elems,), generator=gen, device=dev,
                           dtype=torch.int32).to(torch.uint8)
        ks = torch.rand(g.scale_elems, generator=gen, device=dev) * 0.02 + 1e-3
        vs = torch.rand(g.scale_elems, generator=gen, device=dev) * 0.02 + 1e-3
    else:
        kp = torch.randn(g.pool_elems, generator=gen, device=dev).to(torch.bfloat16).view(torch.int16)
        vp = torch.randn(g.pool_elems, generator=gen, device=dev).to(torch.bfloat16).view(torch.int16)
        ks = vs = None
    q = torch.randn((rows, QH * D), generator=gen, device=dev).to(torch.bfloat16).view(torch.int16)
    out = torch.empty((rows, QH * D), dtype=torch.bfloat16, device=dev)
    slots = torch.arange(rows, dtype=torch.int32, device=dev)
    pos = torch.tensor(np.asarray(lens) - 1, dtype=torch.int32, device=dev)
    return dict(g=g, kp=kp, vp=vp, ks=ks, vs=vs, q=q, out=out, slots=slots, pos=pos,
                bt=bt.to(dev), lens=np.asarray(lens), fp8=fp8, QH=QH)


def choose_splits(ops, lens, fp8, kv_heads=4, q_heads=24, head_dim=256, page_tokens=16):
    """The step planner's split choice for these rows (psk_choose_decode_split)."""
    return ops.choose_decode_split(len(lens), q_heads, kv_heads, head_dim, page_tokens, fp8,
                                   lens, 1 << 40)


def run_decode(torch, ops, st, steps, warmup, dev, splits=None, pps=None):
    """Returns (step_ms, split_kernel_ms, reduce_ms, bytes)."""
    import ctypes as C
    from phaseshift_amd import lib, check
    g, lens = st["g"], st["lens"]
    if splits is None:
        splits, pps = choose_splits(ops, lens, st["fp8"])
    rows = len(lens)
    a = ops.attention_args(g, 0, st["q"], st["out"], st["slots"], st["pos"], st["bt"], st["QH"])
    nbytes = ops.split_partials_bytes(rows, st["QH"], g.kv_heads, splits)
    partials = torch.empty(nbytes // 4, dtype=torch.float32, device=dev)
    L = lib()
    s = torch.cuda.current_stream().cuda_stream
    kp, vp = st["kp"].data_ptr(), st["vp"].data_ptr()

    def split_launch():
        if st["fp8"]:
            check("split", L.psk_attention_paged_fp8_e4m3_split(
                C.byref(a), kp, vp, st["ks"].data_ptr(), st["vs"].data_ptr(),
                partials.data_ptr(), splits, pps, s))
        else:
            check("split", L.psk_attention_paged_bf16_split_ex(
                C.byref(a), kp, vp, partials.data_ptr(), splits, pps, s))

    def reduce_launch():
        check("reduce", L.psk_attention_paged_split_reduce_ex(C.byref(a), partials.data_ptr(),
                                                              splits, pps, s))

    def step():
        split_launch()
        reduce_launch()

    warm(torch, step, warmup)
    # step time: K back-to-back steps
    t = Timer(torch)
    with t:
        for _ in range(steps):
            split_launch()
            reduce_launch()
    step_ms = t.ms() / steps
    # per-kernel durations: HIP events on the launch stream around `steps`
    # back-to-back launches of that kernel alone (amortizes the event gaps)
    warm(torch, split_launch, 1)
    t1 = Timer(torch)
    with t1:
        for _ in range(steps):
            split_launch()
    t2 = Timer(torch)
    with t2:
        for _ in range(steps):
            reduce_launch()
    per_tok = BYTES_PER_TOKEN_FP8 if st["fp8"] else BYTES_PER_TOKEN_BF16
    nbytes_alg = float(lens.sum()) * per_tok + rows * st["QH"] * 256 * 2
    return step_ms, t1.ms() / steps, t2.ms() / steps, nbytes_alg, splits, pps


def run_append(torch, ops, rows, steps, warmup, dev, seed=7, graph=False, mode="append"):
    """mode "append": the KV append alone; "meta_append": the row metadata of
    `rows` one-row decode requests, then the append (two launches); "fused":
    both in one launch (psk_kv_append_fp8_e4m3_from_requests)."""
    H, D, P = 4, 256, 16
    rng = np.random.default_rng(seed)
    seqs = max(1, rows // P)
    g = ops.PoolGeometry(1, seqs + 16, P, H, D)
    bt = torch.from_numpy(rng.permutation(seqs + 16)[:seqs].astype(np.int32).reshape(seqs, 1)).to(dev)
    slots = torch.from_numpy(np.repeat(np.arange(seqs), P)[:rows].astype(np.int32)).to(dev)
    pos = torch.from_numpy(np.tile(np.arange(P), seqs)[:rows].astype(np.int32)).to(dev)
    perm = torch.from_numpy(rng.permutation(rows)).to(dev)
    slots, pos = slots[perm].contiguous(), pos[perm].contiguous()
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    k = torch.randn((rows, H * D), generator=gen, device=dev).to(torch.bfloat16).view(torch.int16)
    v = torch.randn((rows, H * D), generator=gen, device=dev).to(torch.bfloat16).view(torch.int16)
    kp = torch.empty(g.pool_elems, dtype=torch.uint8, device=dev)
    vp = torch.empty_like(kp)
    ks = torch.empty(g.scale_elems, dtype=torch.float32, device=dev)
    vs = torch.empty_like(ks)

    if mode != "append":
        hs, hp = slots.cpu().numpy(), pos.cpu().numpy()
        descs = [dict(slot=int(hs[r]), row_begin=r, row_count=1, prefix_length=int(hp[r]),
                      execution_class=0) for r in range(rows)]
        raw = torch.from_numpy(np.frombuffer(ops.pack_requests(descs), np.uint8).copy()).to(dev)
        slots = torch.empty_like(slots)
        pos = torch.empty_like(pos)

    def launch():
        if mode == "fused":
            ops.kv_append_from_requests(g, 0, k, v, raw, rows, slots, pos, bt, kp, vp, ks, vs)
            return
        if mode == "meta_append":
            ops.prepare_row_metadata(raw, rows, rows, slots, pos)
        ops.kv_append(g, 0, k, v, slots, pos, bt, kp, vp, ks, vs)

    warm(torch, launch, warmup)
    t = Timer(torch)
    with t:
        for _ in range(steps):
            launch()
    ms = t.ms() / steps
    if not graph:
        return ms, rows * APPEND_BYTES_PER_ROW_FP8
    # the same launches captured back to back in one HIP graph and replayed:
    # the GPU-side cost per append without the host's per-launch work
    n = 100
    s = torch.cuda.Stream()
    cg = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        launch()                      # first use outside the capture
        torch.cuda.synchronize()
        with torch.cuda.graph(cg, stream=s):
            for _ in range(n):
                launch()
    torch.cuda.synchronize()
    for _ in range(3):
        cg.replay()
    torch.cuda.synchronize()
    t = Timer(torch)
    with t:
        for _ in range(steps):
            cg.replay()
    return ms, rows * APPEND_BYTES_PER_ROW_FP8, t.ms() / (steps * n)


def run_fp8_prefill(torch, ops, steps, warmup, dev):
    """Config 5's 8 prefill chunks of 512 causal rows (contexts U[2k, 16k]
    before each chunk, seed 5005, FP8 KV, 24/4 heads, hd 256, page 16) alone:
    through the step planner (grouped tiles, one launch) and through the
    reference's prefill launcher (implicit 16-row tiles, one launch)."""
    from phaseshift_amd import KV_FP8, state
    QH, H, D, P = 24, 4, 256, 16
    rng = np.random.default_rng(5005)
    pre = rng.integers(2048, 16385, 8)
    lens = pre + 512
    need = (lens + P - 1) // P
    g = ops.PoolGeometry(1, int(need.sum()), P, H, D)
    perm = rng.permutation(int(need.sum())).astype(np.int32)
    bt = np.full((8, int(need.max())), -1, np.int32)
    o_ = 0
    for r, n in enumerate(need):
        bt[r, :n] = perm[o_:o_ + n]
        o_ += n
    gen = torch.Generator(device=dev)
    gen.manual_seed(5)
    kp = torch.randint(0, 126, (g.pool_elems,), generator=gen, device=dev, dtype=torch.int32).to(torch.uint8)
    vp = torch.randint(0, 126, (g.pool_elems,), generator=gen, device=dev, dtype=torch.int32).to(torch.uint8)
    ks = torch.rand(g.scale_elems, generator=gen, device=dev) * 0.02 + 1e-3
    vs = torch.rand(g.scale_elems, generator=gen, device=dev) * 0.02 + 1e-3
    rows = 8 * 512
    q = torch.randn((rows, QH * D), generator=gen, device=dev).to(torch.bfloat16).view(torch.int16)
    out = torch.empty((rows, QH * D), dtype=torch.bfloat16, device=dev)
    slots = torch.from_numpy(np.repeat(np.arange(8), 512).astype(np.int32)).to(dev)
    pos = torch.from_numpy(np.concatenate([np.arange(p0, p0 + 512) for p0 in pre]).astype(np.int32)).to(dev)
    btd = torch.from_numpy(bt).to(dev)
    flops = float(sum(int(p0) * 512 + 512 * 513 // 2 for p0 in pre)) * QH * D * 4
    a = ops.attention_args(g, 0, q, out, slots, pos, btd, QH)
    reqs = [(512 * i, 512, 2, int(lens[i])) for i in range(8)]
    part = torch.empty((64 << 20) // 4, dtype=torch.float32, device=dev)
    t_ms = {}
    for kind, reps in (("planner", steps), ("prefill", max(2, steps // 2))):
        def launch():
            if kind == "planner":
                state.plan_step(a, KV_FP8, reqs, int(lens.max()), part.numel() * 4, part, kp, vp, ks, vs,
                                launch=True)
            else:
                ops.paged_attention(g, 0, q, out, slots, pos, btd, kp, vp, QH, ks, vs, kind="prefill")

        warm(torch, launch, warmup)
        t = Timer(torch)
        with t:
            for _ in range(reps):
                launch()
        t_ms[kind] = t.ms() / reps
    tflops = flops / (t_ms["planner"] * 1e-3) / 1e12
    return dict(rows=rows, tile_ms=round(t_ms["planner"], 4), tile_tflops=round(tflops, 1),
                frac_of_mfma_peak=round(tflops / 2500.0, 4),
                reference_launcher_ms=round(t_ms["prefill"], 4), flops=flops)


def run_psq(torch, ops, steps, warmup, dev):
    """PSQ4_W32 / PSQ8_W32 KV: decode at the north-star shape (batch 64, ctx
    32768, 24/4 heads, hd256, page 16; planner-chosen split + combine) and the
    append of 2^16 rows (MaxAbs and LSQ1)."""
    import ctypes as C
    from phaseshift_amd import KV_PSQ4, KV_PSQ8, check, lib, state
    L = lib()
    s = torch.cuda.current_stream().cuda_stream
    res = {}
    rows, ctx, QH, H, D, P = 64, 32768, 24, 4, 256, 16
    for fmt in (4, 8):
        pages = rows * ctx // P
        g = ops.PoolGeometry(1, pages, P, H, D)
        gen = torch.Generator(device=dev)
        gen.manual_seed(fmt)
        nb, cb = g.psq_blocks, g.psq_code_bytes(fmt)
        kc = torch.randint(0, 126, (cb,), generator=gen, device=dev, dtype=torch.int32).to(torch.uint8)
        vc = torch.randint(0, 126, (cb,), generator=gen, device=dev, dtype=torch.int32).to(torch.uint8)
        ks = (torch.rand(nb, generator=gen, device=dev) * 0.01 + 1e-3).to(torch.bfloat16)
        vs = (torch.rand(nb, generator=gen, device=dev) * 0.01 + 1e-3).to(torch.bfloat16)
        perm = torch.randperm(pages, generator=torch.Generator().manual_seed(fmt)).to(torch.int32)
        bt = perm.view(rows, ctx // P).to(dev)
        q = torch.randn((rows, QH * D), generator=gen, device=dev).to(torch.bfloat16)
        out = torch.empty((rows, QH * D), dtype=torch.bfloat16, device=dev)
        slots = torch.arange(rows, dtype=torch.int32, device=dev)
        pos = torch.full((rows,), ctx - 1, dtype=torch.int32, device=dev)
        kvd = KV_PSQ4 if fmt == 4 else KV_PSQ8
        splits, pps = ops.choose_decode_split(rows, QH, H, D, P, False, [ctx] * rows, 1 << 40,
                                              kv_dtype=kvd)
        a = ops.attention_args(g, 0, q, out, slots, pos, bt, QH)
        part = torch.empty(ops.split_partials_bytes(rows, QH, H, splits) // 4, device=dev)
        ptrs = (kc.data_ptr(), vc.data_ptr(), ks.data_ptr(), vs.data_ptr())

        def split_launch():
            check("psq split", L.psk_attention_paged_psq_split_ex(
                C.byref(a), kvd, *ptrs, D // 32, part.data_ptr(), splits, pps, s))

        def reduce_launch():
            check("reduce", L.psk_attention_paged_split_reduce_ex(C.byref(a), part.data_ptr(),
                                                                  splits, pps, s))

        def step():
            split_launch()
            reduce_launch()

        warm(torch, step, warmup)
        t = Timer(torch)
        with t:
            for _ in range(steps):
                step()
        step_ms = t.ms() / steps
        t1 = Timer(torch)
        with t1:
            for _ in range(steps):
                split_launch()
        k_ms = t1.ms() / steps
        nbytes = rows * ctx * BYTES_PER_TOKEN_PSQ[fmt] + rows * QH * D * 2
        res[f"psq{fmt}_decode_b64_ctx32k"] = dict(
            GBps=round(nbytes / (step_ms * 1e-3) / 1e9, 1), ms_per_step=round(step_ms, 4),
            split_kernel_ms=round(k_ms, 4),
            kernel_GBps=round(nbytes / (k_ms * 1e-3) / 1e9, 1),
            frac_of_peak=round(nbytes / (step_ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4),
            tokens_per_s=round(rows * ctx / (step_ms * 1e-3), 1),
            bytes_per_step=nbytes, splits=splits, pages_per_split=pps)
        del kc, vc, ks, vs, part
        torch.cuda.empty_cache()

        # append: 2^16 rows, one page-slot each (as the FP8 append line)
        arows = 1 << 16
        seqs = arows // P
        ga = ops.PoolGeometry(1, seqs + 16, P, H, D)
        rng = np.random.default_rng(7)
        abt = torch.from_numpy(rng.permutation(seqs + 16)[:seqs].astype(np.int32).reshape(seqs, 1)).to(dev)
        aslots = torch.from_numpy(np.repeat(np.arange(seqs), P).astype(np.int32)).to(dev)
        apos = torch.from_numpy(np.tile(np.arange(P), seqs).astype(np.int32)).to(dev)
        prm = torch.from_numpy(rng.permutation(arows)).to(dev)
        aslots, apos = aslots[prm].contiguous(), apos[prm].contiguous()
        kin = torch.randn((arows, H * D), generator=gen, device=dev).to(torch.bfloat16)
        vin = torch.randn((arows, H * D), generator=gen, device=dev).to(torch.bfloat16)
        akc = torch.empty(ga.psq_code_bytes(fmt), dtype=torch.uint8, device=dev)
        avc = torch.empty_like(akc)
        aks = torch.empty(ga.psq_blocks, dtype=torch.int16, device=dev)
        avs = torch.empty_like(aks)
        for est, name in ((0, "maxabs"), (1, "lsq1")):
            def launch():
                ops.kv_append_psq(ga, 0, kin, vin, aslots, apos, abt, akc, avc, aks, avs, fmt, est)

            warm(torch, launch, warmup)
            t = Timer(torch)
            with t:
                for _ in range(steps):
                    launch()
            ms = t.ms() / steps
            nb_ = arows * APPEND_BYTES_PER_ROW_PSQ[fmt]
            res[f"psq{fmt}_append_{name}_rows_{arows}"] = dict(
                tokens_per_s=round(arows / (ms * 1e-3), 1), kernel_ms=round(ms, 5),
                GBps=round(nb_ / (ms * 1e-3) / 1e9, 1),
                frac_of_peak=round(nb_ / (ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4))
        del kin, vin, akc, avc, aks, avs
        torch.cuda.empty_cache()

        # prefill: config 5's 8 chunks of 512 causal rows (contexts U[2k, 16k]
        # before the chunk) through the step planner (grouped PSQ tiles), the
        # reference's prefill launcher (implicit 16-row tiles, one head per
        # wave) and the PSQ decode kernel (the row-by-row path tiles replace)
        rng = np.random.default_rng(5005)
        pre = rng.integers(2048, 16385, 8)
        lens = pre + 512
        need = (lens + P - 1) // P
        gp = ops.PoolGeometry(1, int(need.sum()), P, H, D)
        stride = int(need.max())
        perm = rng.permutation(int(need.sum())).astype(np.int32)
        btp = np.full((8, stride), -1, np.int32)
        o_ = 0
        for r, n in enumerate(need):
            btp[r, :n] = perm[o_:o_ + n]
            o_ += n
        nb, cb = gp.psq_blocks, gp.psq_code_bytes(fmt)
        kc = torch.randint(0, 126, (cb,), generator=gen, device=dev, dtype=torch.int32).to(torch.uint8)
        vc = torch.randint(0, 126, (cb,), generator=gen, device=dev, dtype=torch.int32).to(torch.uint8)
        ks = (torch.rand(nb, generator=gen, device=dev) * 0.01 + 1e-3).to(torch.bfloat16)
        vs = (torch.rand(nb, generator=gen, device=dev) * 0.01 + 1e-3).to(torch.bfloat16)
        prow = 8 * 512
        q = torch.randn((prow, QH * D), generator=gen, device=dev).to(torch.bfloat16)
        out = torch.empty((prow, QH * D), dtype=torch.bfloat16, device=dev)
        pslots = torch.from_numpy(np.repeat(np.arange(8), 512).astype(np.int32)).to(dev)
        ppos = torch.from_numpy(np.concatenate([np.arange(p0, p0 + 512) for p0 in pre]).astype(np.int32)).to(dev)
        btd = torch.from_numpy(btp).to(dev)
        flops = float(sum(int(p0) * 512 + 512 * 513 // 2 for p0 in pre)) * QH * D * 4
        pt = {}
        pa = ops.attention_args(gp, 0, q, out, pslots, ppos, btd, QH)
        preqs = [(512 * i, 512, 2, int(lens[i])) for i in range(8)]
        ppart = torch.empty((64 << 20) // 4, dtype=torch.float32, device=dev)
        for kind, reps in (("planner", steps), ("prefill", max(2, steps // 4)), ("decode", 2)):
            def launch():
                if kind == "planner":
                    state.plan_step(pa, KV_PSQ4 if fmt == 4 else KV_PSQ8, preqs, int(lens.max()),
                                    ppart.numel() * 4, ppart, kc, vc, ks, vs, launch=True)
                else:
                    ops.paged_attention_psq(gp, 0, q, out, pslots, ppos, btd, kc, vc, ks, vs, QH, fmt,
                                            kind=kind)

            warm(torch, launch, 1 if kind == "decode" else warmup)
            t = Timer(torch)
            with t:
                for _ in range(reps):
                    launch()
            pt[kind] = t.ms() / reps
        res[f"psq{fmt}_prefill_cfg5_chunks"] = dict(
            rows=prow, tile_ms=round(pt["planner"], 4),
            tile_tflops=round(flops / (pt["planner"] * 1e-3) / 1e12, 1),
            reference_launcher_ms=round(pt["prefill"], 4), decode_path_ms=round(pt["decode"], 4),
            speedup=round(pt["decode"] / pt["planner"], 2))
        del kc, vc, ks, vs, q, out, ppart
        torch.cuda.empty_cache()
    return res


def run_prefix_cache(torch, steps, warmup, dev):
    """Prefix-cache save and restore of a 4096-token prefix: FP8 KV, 6
    attention layers x 4 kv heads x hd 256, page 16 (256 pages), plus the GDN
    slot of the reference's qwen35-0.8B layout (18 states, conv 6144 x 3,
    16 x 128 x 128 recurrent). Each is one batched copy launch (up to 256 pages)."""
    from phaseshift_amd import state
    L, P, H, D, tokens = 6, 16, 4, 256, 4096
    kv = state.KVPool(2 * tokens // P + 8, P, L, H, D, fp8=True)
    slots = state.SlotPool(4, tokens // P)
    gdn = state.GdnPool(4, 18, 6144, 3, 16, 128, 128)
    cache = state.PrefixCache(kv, gdn, tokens, 2, 64)
    seq = state.Sequence(slots, kv, tokens)
    gdn.initialize(seq.slot)
    seq.reserve(tokens)
    seq.commit(tokens)
    toks = np.arange(tokens, dtype=np.int32)
    gi = gdn.info()
    moved = (tokens // P) * L * 2 * (P * H * D + P * H * 4) + gi.conv_slot_bytes + gi.recurrent_slot_bytes
    save_ms, restore_ms = [], []

    save_gpu, restore_gpu = [], []

    def gpu_us(fn):
        # the stream held busy while the host enqueues: the events then time
        # the GPU work of the call alone (pair-list upload + copy launch)
        torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        torch.cuda._sleep(1_000_000)
        e0.record()
        fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e3

    def once(record):
        cache.clear()
        t = Timer(torch)
        with t:
            cache.save(seq, gdn, kv, toks)
        r = state.Sequence(slots, kv, tokens)
        gdn.initialize(r.slot)
        cid = cache.find_longest(toks).id
        t2 = Timer(torch)
        with t2:
            cache.restore(r, gdn, kv, cid)
        if record:
            save_ms.append(t.ms())
            restore_ms.append(t2.ms())
        gdn.release(r.slot)
        r.release()
        if record:
            cache.clear()
            save_gpu.append(gpu_us(lambda: cache.save(seq, gdn, kv, toks)))
            r = state.Sequence(slots, kv, tokens)
            gdn.initialize(r.slot)
            cid = cache.find_longest(toks).id
            restore_gpu.append(gpu_us(lambda: cache.restore(r, gdn, kv, cid)))
            gdn.release(r.slot)
            r.release()

    for _ in range(max(warmup, 3)):
        once(False)
    for _ in range(steps):
        once(True)
    st = cache.stats()
    s_ms, r_ms = float(np.median(save_ms)), float(np.median(restore_ms))
    res = dict(prefix_tokens=tokens, pages=tokens // P, layers=L, copied_bytes=moved,
               save_ms=round(s_ms, 4), restore_ms=round(r_ms, 4),
               save_GBps_read_plus_write=round(2 * moved / (s_ms * 1e-3) / 1e9, 1),
               restore_GBps_read_plus_write=round(2 * moved / (r_ms * 1e-3) / 1e9, 1),
               save_gpu_us=round(float(np.median(save_gpu)), 2),
               restore_gpu_us=round(float(np.median(restore_gpu)), 2),
               save_gpu_GBps_read_plus_write=round(2 * moved / (float(np.median(save_gpu)) * 1e-6) / 1e9, 1),
               launches_per_save=int(st.copy_launches // max(1, 2 * (steps + max(warmup, 3)) + 2 * steps)),
               reference_copies_per_save=(tokens // P) * L * 4 + 4)
    # the page copy alone, kernel time: the same per-block copy (page body and
    # scale rows of K or V per workgroup) over the sequence's 256 pages x 6
    # layers into the pool's free pages, 20 back-to-back launches
    from phaseshift_amd import ops
    T = kv.tensors(torch)
    src_pages = seq.block_table()
    used = set(src_pages)
    dst_pages = [pg for pg in range(kv.geom.num_pages) if pg not in used][:len(src_pages)]
    pairs = torch.tensor(list(zip(dst_pages, src_pages)), dtype=torch.int32, device=dev)
    kv_bytes = len(src_pages) * L * 2 * (P * H * D + P * H * 4)

    def cp():
        ops.copy_pages(kv.geom, T, T, pairs)

    warm(torch, cp, warmup)
    t = Timer(torch)
    with t:
        for _ in range(20):
            cp()
    k_ms = t.ms() / 20
    res["page_copy_kernel"] = dict(pages=len(src_pages), layers=L, bytes_read=kv_bytes, us=round(k_ms * 1e3, 2),
                                   GBps_read_plus_write=round(2 * kv_bytes / (k_ms * 1e-3) / 1e9, 1),
                                   frac_of_peak=round(2 * kv_bytes / (k_ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4))
    gdn.release(seq.slot)
    seq.release()
    cache.close()
    del st
    return res


def run_step_graph(torch, ops, steps, warmup, dev):
    """Planned PAGED_ATTENTION steps with FP8 KV launched eagerly
    (psk_paged_attention_step: plan + launches) and as a captured HIP graph
    (psk_paged_attention_step_graphed: plan + signature + one graph launch).
    "mixed": 8 decode rows at 2.2k-3.6k tokens (split-K + combine), two 16-row
    verify blocks, a 128-row prefill chunk. "verify32": 32 verify blocks of 16
    rows at 1k context, whose split tiles need one combine launch per block
    (34 launches a step). GPU time per step (events around back-to-back steps)
    and host time to enqueue a step."""
    import time
    from phaseshift_amd import KV_FP8, state
    QH, H, D, P = 24, 4, 256, 16

    def workload(kind, seed):
        rng = np.random.default_rng(seed)
        if kind == "mixed":
            ctx = [int(x) for x in rng.integers(2200, 3600, 8)]
            lens = ctx + [1016, 1016, 328]
            slot_l = list(range(8)) + [8] * 16 + [9] * 16 + [10] * 128
            pos_l = [c - 1 for c in ctx] + list(range(1000, 1016)) * 2 + list(range(200, 328))
            reqs = [(i, 1, 0, ctx[i]) for i in range(8)] + [(8, 16, 1, 1016), (24, 16, 1, 1016),
                                                            (40, 128, 2, 328)]
            maxvis = 3600
        else:
            lens = [1016] * 32
            slot_l = [b for b in range(32) for _ in range(16)]
            pos_l = list(range(1000, 1016)) * 32
            reqs = [(16 * b, 16, 1, 1016) for b in range(32)]
            maxvis = 2048
        need = [(n + P - 1) // P for n in lens]
        pages = sum(need) + 2
        perm = rng.permutation(pages).astype(np.int32)
        bt = np.full((len(lens), max(need)), -1, np.int32)
        k = 0
        for r, n in enumerate(need):
            bt[r, :n] = perm[k:k + n]
            k += n
        g = ops.PoolGeometry(1, pages, P, H, D)
        gen = torch.Generator(device=dev)
        gen.manual_seed(seed)
        pools = (torch.randint(0, 126, (g.pool_elems,), generator=gen, device=dev).to(torch.uint8),
                 torch.randint(0, 126, (g.pool_elems,), generator=gen, device=dev).to(torch.uint8),
                 torch.rand(g.scale_elems, generator=gen, device=dev) * 0.02 + 1e-3,
                 torch.rand(g.scale_elems, generator=gen, device=dev) * 0.02 + 1e-3)
        slots = torch.tensor(slot_l, dtype=torch.int32, device=dev)
        pos = torch.tensor(pos_l, dtype=torch.int32, device=dev)
        rows = slots.numel()
        q = torch.randn((rows, QH * D), generator=gen, device=dev).to(torch.bfloat16)
        out = torch.empty((rows, QH * D), dtype=torch.float32, device=dev)
        a = ops.attention_args(g, 0, q, out, slots, pos, torch.from_numpy(bt).to(dev), QH)
        return a, pools, reqs, maxvis, (q, out, slots, pos)

    res = {}
    nbytes = 64 << 20
    part = torch.empty(nbytes // 4, dtype=torch.float32, device=dev)
    for kind in ("mixed", "verify32"):
        a, pools, reqs, maxvis, keep = workload(kind, 5)
        cache = state.StepGraphCache(4)

        def eager():
            state.plan_step(a, KV_FP8, reqs, maxvis, nbytes, part, *pools, launch=True)

        def graphed():
            cache.step(a, KV_FP8, reqs, maxvis, nbytes, part, *pools)

        r = {}
        for name, fn in (("eager", eager), ("graph", graphed)):
            warm(torch, fn, max(warmup, 3))
            t = Timer(torch)
            h0 = time.perf_counter()
            with t:
                for _ in range(steps):
                    fn()
            host_ms = (time.perf_counter() - h0) * 1e3 / steps
            r[name + "_gpu_ms_per_step"] = round(t.ms() / steps, 4)
            r[name + "_host_ms_per_step"] = round(host_ms, 4)
        plan, how = cache.step(a, KV_FP8, reqs, maxvis, nbytes, part, *pools)
        torch.cuda.synchronize()
        r.update(planned_kernels=int(plan.count), replayed=bool(how == 2),
                 gpu_speedup=round(r["eager_gpu_ms_per_step"] / r["graph_gpu_ms_per_step"], 3))
        res[kind] = r
        cache.close()
    return res


def run_dropin_unpatched(torch, ops, steps, warmup, dev):
    """What an unmodified PhaseShift dispatcher gets when it links this library:
    it calls the reference-signature launchers (ps::kernel::launch_*, by their
    mangled names) the way paged_attention_dispatch.hip:437-477,790-894 does —
    FP8 KV unsplit (its plan admits no FP8 split) at the north-star batch 64 x
    32k, and BF16 at its fixed 16 splits + the bf16 reduce at BASELINE config 3.
    Kernel times from HIP events on the launch stream."""
    import ctypes as C
    import phaseshift_amd
    cdll = C.CDLL(phaseshift_amd.LIB_PATH)
    P, U = C.c_void_p, C.c_uint32
    fp8_fn = cdll["_ZN2ps6kernel31launch_attention_paged_fp8_e4m3ERKNS0_24PagedAttentionCommonArgs"
                  "EPKhS5_PKfS7_P12ihipStream_t"]
    fp8_fn.argtypes, fp8_fn.restype = [P] * 6, C.c_int
    sp_fn = cdll["_ZN2ps6kernel33launch_attention_paged_bf16_splitERKNS0_24PagedAttentionCommonArgs"
                 "EPKNS_6bf16_tES6_PfjP12ihipStream_t"]
    sp_fn.argtypes, sp_fn.restype = [P, P, P, P, U, P], C.c_int
    rd_fn = cdll["_ZN2ps6kernel40launch_attention_paged_bf16_split_reduceERKNS0_24PagedAttentionCommonArgs"
                 "EPKfjP12ihipStream_t"]
    rd_fn.argtypes, rd_fn.restype = [P, P, U, P], C.c_int
    s = torch.cuda.current_stream().cuda_stream
    res = {}

    def timed(fn):
        warm(torch, fn, warmup)
        t = Timer(torch)
        with t:
            for _ in range(steps):
                fn()
        return t.ms() / steps

    st = decode_setup(torch, ops, [32768] * 64, True, 11, dev)
    a = ops.attention_args(st["g"], 0, st["q"], st["out"], st["slots"], st["pos"], st["bt"], st["QH"])
    ptrs = (st["kp"].data_ptr(), st["vp"].data_ptr(), st["ks"].data_ptr(), st["vs"].data_ptr())

    def fp8_unsplit():
        assert fp8_fn(C.addressof(a), *ptrs, s) == 0

    ms = timed(fp8_unsplit)
    nb = 64 * 32768 * BYTES_PER_TOKEN_FP8 + 64 * 24 * 256 * 2
    res["fp8_unsplit_b64_ctx32k"] = dict(kernel_ms=round(ms, 4), GBps=round(nb / (ms * 1e-3) / 1e9, 1),
                                         frac_of_peak=round(nb / (ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4))
    del st, a
    torch.cuda.empty_cache()
    rng = np.random.default_rng(303)
    lens = rng.integers(1024, 32769, 32)
    st = decode_setup(torch, ops, lens, False, 303, dev)
    a = ops.attention_args(st["g"], 0, st["q"], st["out"], st["slots"], st["pos"], st["bt"], st["QH"])
    part = torch.empty(ops.split_partials_bytes(32, 24, 4, 16) // 4, dtype=torch.float32, device=dev)
    kp, vp = st["kp"].data_ptr(), st["vp"].data_ptr()

    def split16():
        assert sp_fn(C.addressof(a), kp, vp, part.data_ptr(), 16, s) == 0

    def reduce16():
        assert rd_fn(C.addressof(a), part.data_ptr(), 16, s) == 0

    step_ms = timed(lambda: (split16(), reduce16()))
    k_ms = timed(split16)
    nb = float(lens.sum()) * BYTES_PER_TOKEN_BF16 + 32 * 24 * 256 * 2
    res["bf16_split16_cfg3"] = dict(ms_per_step=round(step_ms, 4), split_kernel_ms=round(k_ms, 4),
                                    GBps=round(nb / (step_ms * 1e-3) / 1e9, 1),
                                    frac_of_peak=round(nb / (step_ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4))
    del st, a, part
    torch.cuda.empty_cache()
    return res


def run_decode_loop(torch, ops, dev, n_steps=64):
    """Continuous decode at BASELINE config 4 (64 rows, FP8, ctx log-U[4k,64k]):
    n_steps consecutive steps through psk_paged_attention_step (plan + split
    launch + combine), every row's position advancing by one token per step and
    each request carrying its row's visible length, as a serving loop sees
    them. Host time is the C-ABI call alone (request arrays are built before
    the loop); GPU time is HIP events around the whole loop. The device
    positions advance by a small fill between steps, outside both figures'
    planning but inside the GPU time."""
    import ctypes as C
    from phaseshift_amd import KV_FP8, StepPlan, StepRequest, check, lib
    from phaseshift_amd.ops import _stream
    rng = np.random.default_rng(404)
    lens = np.exp(rng.uniform(np.log(4096), np.log(65536), 64)).astype(np.int64)
    st = decode_setup(torch, ops, lens + n_steps + 1, True, 404, dev)
    rows = len(lens)
    pos = torch.tensor(lens - 1, dtype=torch.int32, device=dev)
    a = ops.attention_args(st["g"], 0, st["q"], st["out"], st["slots"], pos, st["bt"], st["QH"])
    pbytes = 64 << 20
    part = torch.empty(pbytes // 4, dtype=torch.float32, device=dev)
    L = lib()
    s = _stream(None)
    ptrs = (st["kp"].data_ptr(), st["vp"].data_ptr(), st["ks"].data_ptr(), st["vs"].data_ptr())
    one = torch.ones(rows, dtype=torch.int32, device=dev)
    req_sets = []
    for i in range(n_steps + 1):
        rq = (StepRequest * rows)()
        for r in range(rows):
            rq[r].row_begin, rq[r].row_count, rq[r].execution_class = r, 1, 0
            rq[r].max_visible = int(lens[r]) + i
        req_sets.append((rq, int(lens.max()) + i))
    plan = StepPlan()

    def step(i):
        rq, mv = req_sets[i]
        h0 = time.perf_counter_ns()
        check("psk_paged_attention_step", L.psk_paged_attention_step(
            C.byref(a), KV_FP8, *ptrs, rq, rows, mv, part.data_ptr(), pbytes, C.byref(plan), s))
        h = time.perf_counter_ns() - h0
        pos.add_(one)
        return h

    # the first plan of the batch (cold: the chooser simulates)
    cold_us = step(0) / 1e3
    torch.cuda.synchronize()
    t = Timer(torch)
    host = []
    with t:
        for i in range(1, n_steps + 1):
            host.append(step(i))
    gpu_ms = t.ms() / n_steps
    host_us = np.asarray(host, np.float64) / 1e3
    splits = [int(plan.kernels[0].splits), int(plan.kernels[0].pages_per_split)]
    del st
    torch.cuda.empty_cache()
    return dict(steps=n_steps, host_us_per_step_mean=round(float(host_us.mean()), 2),
                host_us_per_step_p50=round(float(np.median(host_us)), 2),
                host_us_per_step_max=round(float(host_us.max()), 2),
                first_plan_host_us=round(cold_us, 1), gpu_ms_per_step=round(gpu_ms, 4),
                last_plan_splits_pages=splits)


def run_mixed_step(torch, ops, steps, warmup, dev):
    """BASELINE config 5, one continuous-batching step on the device: row
    metadata from the request descriptors, KV append (fused FP8 quantization) of
    all 4272 rows, the planned PAGED_ATTENTION launches (48 decode rows, 8 verify
    blocks of 16 causal drafts on the tile kernel, 8 prefill chunks of 512 rows
    on the tile kernel) and the CoW restore of 32 prefix pages. Contexts
    U[2k,16k], FP8 KV, 24/4 heads, hd 256, page 16. Rollback (page truncation)
    changes the step's work, so it is timed once on its own."""
    from phaseshift_amd import KV_FP8, state
    rng = np.random.default_rng(5005)
    QH, H, D, Pt = 24, 4, 256, 16
    n_pre, n_dec, n_ver = 8, 48, 8
    ctx = rng.integers(2048, 16385, n_pre + n_dec + n_ver)
    max_len = int(ctx.max()) + 512 + 16
    need_pages = int(sum(math.ceil((c + 512) / Pt) for c in ctx)) + 64
    pool = state.KVPool(need_pages, Pt, 1, H, D, fp8=True)
    cache = state.KVPool(64, Pt, 1, H, D, fp8=True)
    slots = state.SlotPool(n_pre + n_dec + n_ver + 1, math.ceil(max_len / Pt))
    g = pool.geom
    T = pool.tensors(torch)
    gen = torch.Generator(device=dev)
    gen.manual_seed(5)
    for k in ("k", "v"):
        T[k].copy_(torch.randint(0, 126, T[k].shape, generator=gen, device=dev,
                                 dtype=torch.int32).to(torch.uint8))
    for k in ("k_scale", "v_scale"):
        T[k].copy_(torch.rand(T[k].shape, generator=gen, device=dev) * 0.02 + 1e-3)
    seqs = [state.Sequence(slots, pool, max_len) for _ in range(len(ctx))]
    for sq, c in zip(seqs, ctx):
        sq.reserve(int(c))
        sq.commit(int(c))
    cache_pages = [cache.allocate() for _ in range(32)]
    dst_pages = seqs[0].block_table()[:32]
    reqs, descs, row = [], [], 0
    layout = [(n_pre + i, 1, 0) for i in range(n_dec)] + \
             [(n_pre + n_dec + i, 16, 1) for i in range(n_ver)] + [(i, 512, 2) for i in range(n_pre)]
    visible = []
    for si, cnt, cls in layout:
        sq = seqs[si]
        reqs.append((row, cnt, cls, sq.position + cnt))
        descs.append(dict(slot=sq.slot, row_begin=row, row_count=cnt, prefix_length=sq.position,
                          execution_class=cls))
        visible += [sq.position + j + 1 for j in range(cnt)]
        sq.reserve(cnt)
        row += cnt
    rows = row
    raw = torch.from_numpy(np.frombuffer(ops.pack_requests(descs), np.uint8).copy()).to(dev)
    rslots = torch.empty(rows, dtype=torch.int32, device=dev)
    rpos = torch.empty(rows, dtype=torch.int32, device=dev)
    bt = slots.block_tables(torch)
    kin = torch.randn((rows, H * D), generator=gen, device=dev).to(torch.bfloat16).view(torch.int16)
    vin = torch.randn((rows, H * D), generator=gen, device=dev).to(torch.bfloat16).view(torch.int16)
    q = torch.randn((rows, QH * D), generator=gen, device=dev).to(torch.bfloat16).view(torch.int16)
    out = torch.empty((rows, QH * D), dtype=torch.bfloat16, device=dev)
    a = ops.attention_args(g, 0, q, out, rslots, rpos, bt, QH)
    part = torch.empty((256 << 20) // 4, dtype=torch.float32, device=dev)
    maxvis = int(ctx.max()) + 512

    def append():
        ops.kv_append(g, 0, kin, vin, rslots, rpos, bt, T["k"], T["v"], T["k_scale"],
                      T["v_scale"])

    def attend():
        return state.plan_step(a, KV_FP8, reqs, maxvis, part.numel() * 4, partials_ptr=part,
                               k_pool=T["k"], v_pool=T["v"], k_scale=T["k_scale"],
                               v_scale=T["v_scale"], launch=True)

    def cow():
        pool.copy_pages_from(cache, dst_pages, cache_pages)

    def meta_append():
        # the step's row metadata formed inside the append launch
        ops.kv_append_from_requests(g, 0, kin, vin, raw, len(descs), rslots, rpos, bt, T["k"], T["v"],
                                    T["k_scale"], T["v_scale"])

    def step():
        meta_append()
        attend()
        cow()

    warm(torch, step, warmup)
    plan = attend()
    t = Timer(torch)
    with t:
        for _ in range(steps):
            step()
    step_ms = t.ms() / steps
    parts = {}
    for name, fn in (("metadata_and_append", meta_append), ("append", append), ("attention", attend),
                     ("cow_copy", cow)):
        tt = Timer(torch)
        with tt:
            for _ in range(steps):
                fn()
        parts[name] = round(tt.ms() / steps, 4)
    parts["rollback_8_blocks"] = time_rollback(torch, seqs[n_pre + n_dec:], rng, Pt)
    vis = np.asarray(visible, np.float64)
    flops = float((vis * QH * D * 4).sum())
    kinds = [(int(k.kind), int(k.rows), int(k.splits)) for k in plan.kernels[:plan.count]]
    return dict(ms_per_step=round(step_ms, 4), rows=rows,
                tokens_per_s=round(rows / (step_ms * 1e-3), 1), parts_ms=parts,
                attention_tflops=round(flops / (parts["attention"] * 1e-3) / 1e12, 2),
                attention_flops=flops, plan=kinds)


def time_rollback(torch, ver_seqs, rng, page_tokens, warmup=5, reps=40):
    """Rollback (page truncation) of the verify blocks' rejected tails, each
    block keeping a seeded accepted prefix; the 16-draft reservation is
    re-made before every repetition. Host: the time of the rollback calls
    themselves (free-list updates plus the enqueue of each block-table clear).
    GPU: HIP events around the clears, with the stream held busy while the
    host enqueues them, so the events see only the clears' own execution."""
    keeps = [math.ceil((sq.position + int(rng.integers(0, 17))) / page_tokens) for sq in ver_seqs]
    host_us, gpu_us = [], []
    released = 0
    for r in range(warmup + reps):
        for sq in ver_seqs:
            sq.reserve(16)
        torch.cuda.synchronize()
        released = sum(len(sq.block_table()) - keep for sq, keep in zip(ver_seqs, keeps))
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        torch.cuda._sleep(1_000_000)
        e0.record()
        t0 = time.perf_counter()
        for sq, keep in zip(ver_seqs, keeps):
            sq.rollback(keep)
        t1 = time.perf_counter()
        e1.record()
        torch.cuda.synchronize()
        if r >= warmup:
            host_us.append((t1 - t0) * 1e6)
            gpu_us.append(e0.elapsed_time(e1) * 1e3)
    return dict(blocks=len(ver_seqs), reps=reps,
                host_us_median=round(float(np.median(host_us)), 2),
                host_us_p90=round(float(np.percentile(host_us, 90)), 2),
                gpu_us_median=round(float(np.median(gpu_us)), 2), pages_released_per_rep=released)


def cpu_baseline(lens_row, seconds_cap=30.0):
    """Scalar C oracle on a bounded sample of the same workload: FP8 decode of
    whole rows at context 32768, single-threaded and on a thread pool over rows
    (the C call releases the GIL), each for ~10 s of wall time. The thread
    count is the host's CPU count read at run time, capped at 16 (one GPU's
    share of the box)."""
    import concurrent.futures as cf
    import oracle
    P, H, D, QH = 16, 4, 256, 24
    ctx = int(lens_row)
    rng = np.random.default_rng(5)
    need = (ctx + P - 1) // P
    num_pages = need
    bt = rng.permutation(num_pages).astype(np.uint32).reshape(1, need)
    n = num_pages * P * H * D
    kp = rng.integers(0, 126, n, dtype=np.uint8)
    vp = rng.integers(0, 126, n, dtype=np.uint8)
    ks = rng.uniform(1e-3, 2e-2, num_pages * P * H).astype(np.float32)
    vs = rng.uniform(1e-3, 2e-2, num_pages * P * H).astype(np.float32)
    geom = dict(layer=0, page_tokens=P, num_pages=num_pages, num_attention_layers=1,
                kv_heads=H, head_dim=D, block_table_stride=need, max_sequences=1, q_heads=QH)
    q = oracle.f32_to_bf16(rng.standard_normal((1, QH * D)).astype(np.float32))

    def one_row():
        oracle.paged_attention(geom, q, [0], [ctx - 1], bt, kp, vp, ks, vs, 1 / 16)

    def timed(threads):
        budget = min(10.0, seconds_cap)
        done, t0 = 0, time.perf_counter()
        if threads == 1:
            while time.perf_counter() - t0 < budget:
                one_row()
                done += 1
        else:
            with cf.ThreadPoolExecutor(threads) as ex:
                while time.perf_counter() - t0 < budget:
                    list(ex.map(lambda _: one_row(), range(threads)))
                    done += threads
        el = time.perf_counter() - t0
        return done, el, done * ctx * BYTES_PER_TOKEN_FP8 / el / 1e9

    host_cpus = os.cpu_count() or 1
    threads = max(1, min(16, host_cpus))
    d1, e1, g1 = timed(1)
    dn, en, gn = timed(threads) if threads > 1 else (d1, e1, g1)
    return dict(value=round(gn, 4), unit="GB/s", cores=threads, kind="port",
                single_thread_GBps=round(g1, 4), host_cpus=host_cpus,
                sample=f"FP8 decode of whole rows at ctx {ctx}, 24q/4kv, hd256, scalar C oracle "
                       f"(two-pass fp32 softmax, gcc -O2): {dn} rows on {threads} threads in "
                       f"{en:.1f} s; {d1} rows on 1 thread in {e1:.1f} s")


def cpu_baseline_append(rows=1 << 16, budget_s=5.0):
    """Scalar C oracle of the FP8 KV append (or_kv_append_fp8, the restatement
    of kv_append.hip:127-272) on the 2^16-row workload of the GPU append line
    (4 kv heads, hd 256, page 16, rows scattered over 4096 sequences), single
    threaded and on a thread pool over row chunks (rows of distinct (slot,
    position) write disjoint pool entries), each for about budget_s seconds."""
    import concurrent.futures as cf
    import oracle
    H, D, P = 4, 256, 16
    rng = np.random.default_rng(7)
    seqs = max(1, rows // P)
    num_pages = seqs + 16
    bt = rng.permutation(num_pages)[:seqs].astype(np.uint32).reshape(seqs, 1)
    perm = rng.permutation(rows)
    slots = np.repeat(np.arange(seqs), P)[:rows].astype(np.uint32)[perm]
    pos = np.tile(np.arange(P), seqs)[:rows].astype(np.uint32)[perm]
    k = oracle.f32_to_bf16(rng.standard_normal((rows, H * D), dtype=np.float32))
    v = oracle.f32_to_bf16(rng.standard_normal((rows, H * D), dtype=np.float32))
    n = num_pages * P * H * D
    kp, vp = np.zeros(n, np.uint8), np.zeros(n, np.uint8)
    ks, vs = np.zeros(n // D, np.float32), np.zeros(n // D, np.float32)
    geom = dict(layer=0, page_tokens=P, num_pages=num_pages, num_attention_layers=1, kv_heads=H,
                head_dim=D, block_table_stride=1, max_sequences=seqs)

    def chunk(a, b):
        oracle.kv_append(geom, k[a:b], v[a:b], slots[a:b], pos[a:b], bt, kp, vp, ks, vs)

    def timed(threads):
        done, t0 = 0, time.perf_counter()
        bounds = np.linspace(0, rows, threads * 4 + 1).astype(int)
        while time.perf_counter() - t0 < budget_s:
            if threads == 1:
                chunk(0, rows)
            else:
                with cf.ThreadPoolExecutor(threads) as ex:
                    list(ex.map(lambda i: chunk(bounds[i], bounds[i + 1]), range(len(bounds) - 1)))
            done += rows
        el = time.perf_counter() - t0
        return done, el, done / el

    threads = max(1, min(16, os.cpu_count() or 1))
    d1, e1, t1 = timed(1)
    dn, en, tn = timed(threads) if threads > 1 else (d1, e1, t1)
    return dict(tokens_per_s=round(tn, 1), GBps=round(tn * APPEND_BYTES_PER_ROW_FP8 / 1e9, 4),
                cores=threads, single_thread_tokens_per_s=round(t1, 1), kind="port",
                sample=f"FP8 append of {rows} rows (4 kv heads, hd 256), scalar C oracle (gcc -O2): "
                       f"{dn} rows on {threads} threads in {en:.1f} s; {d1} rows on 1 thread in "
                       f"{e1:.1f} s")


def main():
    args = parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build measures one GPU only (the KV path needs no collective: "
              "it shards by KV head or batch row, each GPU running these kernels on its own "
              "pool); run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    import torch
    from phaseshift_amd import ops
    dev = torch.device("cuda:0")
    if args.copy_calibration:
        src = torch.ones(1 << 28, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes": src.numel() * 4, "launches": 5}))
        return
    only = set(args.only.split(",")) if args.only else {"main", "cfg4", "cfg3", "append", "cfg5", "prefill",
                                                     "psq", "prefix", "graph", "loop", "dropin"}
    extra = {}

    # ---- main: north-star point, FP8 batch 64 @ 32k
    st = decode_setup(torch, ops, [32768] * 64, True, 11, dev)
    torch.cuda.synchronize()
    step_ms, k_ms, r_ms, nbytes, splits, pps = run_decode(torch, ops, st, args.steps, args.warmup,
                                                          dev)
    value = nbytes / (step_ms * 1e-3) / 1e9
    achieved = nbytes / (k_ms * 1e-3) / 1e9
    del st
    torch.cuda.empty_cache()

    if "cfg4" in only:
        rng = np.random.default_rng(404)
        lens = np.exp(rng.uniform(np.log(4096), np.log(65536), 64)).astype(np.int64)
        st = decode_setup(torch, ops, lens, True, 404, dev)
        s_ms, k4, r4, nb4, sp4, pp4 = run_decode(torch, ops, st, args.steps, args.warmup, dev)
        extra["cfg4_fp8_decode_loguniform"] = dict(
            GBps=round(nb4 / (s_ms * 1e-3) / 1e9, 1), ms_per_step=round(s_ms, 4),
            split_kernel_ms=round(k4, 4), reduce_ms=round(r4, 4), splits=sp4, pages_per_split=pp4,
            frac_of_peak=round(nb4 / (s_ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4))
        del st
        torch.cuda.empty_cache()
    if "cfg3" in only:
        rng = np.random.default_rng(303)
        lens = rng.integers(1024, 32769, 32)
        st = decode_setup(torch, ops, lens, False, 303, dev)
        s_ms, k3, r3, nb3, sp3, pp3 = run_decode(torch, ops, st, args.steps, args.warmup, dev)
        extra["cfg3_bf16_decode"] = dict(
            GBps=round(nb3 / (s_ms * 1e-3) / 1e9, 1), ms_per_step=round(s_ms, 4),
            split_kernel_ms=round(k3, 4), reduce_ms=round(r3, 4), splits=sp3, pages_per_split=pp3,
            frac_of_peak=round(nb3 / (s_ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4))
        del st
        torch.cuda.empty_cache()
    if "append" in only:
        ap = {}
        for rows in (128, 1 << 16):
            ms, nb = run_append(torch, ops, rows, args.steps, args.warmup, dev)
            ap[f"rows_{rows}"] = dict(tokens_per_s=round(rows / (ms * 1e-3), 1),
                                      kernel_ms=round(ms, 5),
                                      GBps=round(nb / (ms * 1e-3) / 1e9, 1),
                                      frac_of_peak=round(nb / (ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4))
        # config 2 at decode batch size is launch-bound: the same append
        # replayed from a captured graph shows its GPU-side cost per launch
        _, nb, gms = run_append(torch, ops, 128, args.steps, args.warmup, dev, graph=True)
        ap["rows_128_graph_replay"] = dict(tokens_per_s=round(128 / (gms * 1e-3), 1),
                                           ms_per_append=round(gms, 5),
                                           GBps=round(nb / (gms * 1e-3) / 1e9, 1))
        # a planned step's row metadata + append: two launches, or one
        # (metadata formed inside the append), graph-replayed
        both = {}
        for mode in ("meta_append", "fused"):
            _, _, gm = run_append(torch, ops, 128, args.steps, args.warmup, dev, graph=True, mode=mode)
            both[mode + "_us"] = round(gm * 1e3, 3)
        ap["rows_128_metadata_and_append_graph_replay"] = both
        # the row sweep 2^12 .. 2^17: where the append leaves the launch-bound
        # regime for the HBM-bound one
        sweep = {}
        for lg in range(12, 18):
            ms, nb = run_append(torch, ops, 1 << lg, args.steps, args.warmup, dev)
            sweep[f"rows_2^{lg}"] = dict(kernel_ms=round(ms, 5), tokens_per_s=round((1 << lg) / (ms * 1e-3), 1),
                                         frac_of_peak=round(nb / (ms * 1e-3) / 1e9 / HBM_PEAK_GBPS, 4))
        ap["row_sweep"] = sweep
        extra["kv_append_fp8"] = ap

    if "psq" in only:
        extra["psq_kv"] = run_psq(torch, ops, args.steps, args.warmup, dev)

    if "prefix" in only:
        extra["prefix_cache_fp8"] = run_prefix_cache(torch, args.steps, args.warmup, dev)

    if "graph" in only:
        extra["step_graph_fp8"] = run_step_graph(torch, ops, args.steps, args.warmup, dev)

    if "dropin" in only:
        extra["dropin_unpatched_dispatcher"] = run_dropin_unpatched(torch, ops, args.steps,
                                                                    args.warmup, dev)

    if "loop" in only:
        extra["cfg4_decode_loop_planned"] = run_decode_loop(torch, ops, dev)

    if "prefill" in only:
        extra["cfg5_prefill_chunks_fp8"] = run_fp8_prefill(torch, ops, max(5, args.steps // 2),
                                                           args.warmup, dev)
    if "cfg5" in only:
        extra["cfg5_mixed_step"] = run_mixed_step(torch, ops, max(5, args.steps // 2),
                                                  args.warmup, dev)
        torch.cuda.empty_cache()

    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(32768)
        cpu["kv_append_fp8"] = cpu_baseline_append()
    line = {
        "metric": "paged decode-attn HBM GB/s (% of 8 TB/s peak) + KV-append tokens/s, 1 GPU",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "warmup_min_s": WARM_MIN_S,
        "ms_per_step": round(step_ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8_e4m3 KV, bf16 Q, fp32 accumulate",
        "data": "synthetic (seeded random FP8 codes/scales and bf16 queries)",
        "config": {"workload": "paged decode, FP8 E4M3 KV, batch 64, ctx 32768 each, 24 q / 4 kv "
                               "heads, head_dim 256, page 16, split-K + combine",
                   "splits": splits, "pages_per_split": pps, "frac_of_peak":
                       round(value / HBM_PEAK_GBPS, 4)},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBPS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBPS, 4),
                     "traffic": DECODE_TRAFFIC_BYTES,
                     "traffic_source": "profiles/paged_decode_fp8_b64_ctx32k.md (rocprofv3 --pmc "
                                       "FETCH_SIZE x2.0 + WRITE_SIZE x1.0 per dispatch)",
                     "kernel": "paged_decode_kernel<1,256> (FP8 split)",
                     "kernel_ms": round(k_ms, 5), "reduce_ms": round(r_ms, 5),
                     "bytes_per_launch": nbytes},
        "cpu_baseline": cpu,
    }
    line.update(extra)
    print(json.dumps(line))


if __name__ == "__main__":
    main()
