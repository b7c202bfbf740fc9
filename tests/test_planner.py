"""Step planner (host logic, no GPU): region rules of the reference
(paged_attention_dispatch.hip:705-788) plus the tile routing of verify blocks
and the split sizing. Runs the C-ABI in plan-only mode."""
import numpy as np
import pytest
import phaseshift_amd as P
from phaseshift_amd import state


def args(rows, qh=24, kvh=4, hd=256, page=16):
    a = P.PagedAttentionArgs()
    a.rows, a.q_heads, a.kv_heads, a.head_dim, a.page_tokens = rows, qh, kvh, hd, page
    return a


def kernels(plan):
    return [(k.kind, k.row_begin, k.rows, k.splits, k.pages_per_split)
            for k in plan.kernels[:plan.count]]


def test_config5_mixed_step_layout():
    reqs = ([(i, 1, 0) for i in range(48)] + [(48 + 16 * i, 16, 1) for i in range(8)] +
            [(176 + 512 * i, 512, 2) for i in range(8)])
    plan = state.plan_step(args(4272), P.KV_FP8, reqs, 16384, 256 << 20)
    ks = kernels(plan)
    assert ks[0][:3] == (0, 0, 48)               # decode rows, split-K
    assert ks[0][3] > 1
    assert ks[1][:3] == (1, 48, 128)             # 8 verify blocks -> one tile launch
    assert ks[1][3] > 1                          # few tiles -> split-K
    assert ks[2][:3] == (1, 176, 4096)           # 8 prefill chunks -> one tile launch
    assert plan.count == 3


def test_short_context_does_not_split_and_reference_threshold():
    plan = state.plan_step(args(64), P.KV_FP8, [(i, 1, 0) for i in range(64)], 2047, 1 << 30)
    assert kernels(plan) == [(0, 0, 64, 1, 0)]
    plan = state.plan_step(args(64), P.KV_FP8, [(i, 1, 0) for i in range(64)], 2048, 1 << 30)
    assert kernels(plan)[0][3] > 1


def test_no_workspace_means_no_split():
    plan = state.plan_step(args(64), P.KV_BF16, [(i, 1, 0) for i in range(64)], 32768, 0)
    assert kernels(plan) == [(0, 0, 64, 1, 0)]


def test_split_respects_workspace_cap():
    cap = 32 << 20   # the reference's 32 MiB partial workspace (program_executor.h:21)
    plan = state.plan_step(args(64), P.KV_FP8, [(i, 1, 0) for i in range(64)], 65536, cap)
    k = plan.kernels[0]
    need = 64 * 4 * k.splits * 6 * 258 * 4
    assert k.splits > 1 and need <= cap
    assert k.splits * k.pages_per_split >= 65536 // 16


def test_small_prefill_and_small_verify_stay_on_decode():
    reqs = [(0, 4, 1), (4, 100, 2), (104, 1, 0)]   # 4-row verify, 100-row prefill chunk
    plan = state.plan_step(args(105), P.KV_BF16, reqs, 4096, 1 << 30)
    ks = kernels(plan)
    assert len(ks) == 1 and ks[0][:3] == (0, 0, 105)


def test_gapped_requests_fall_back_to_one_decode_region():
    plan = state.plan_step(args(40), P.KV_FP8, [(0, 8, 0), (16, 24, 1)], 100, 0)
    assert kernels(plan) == [(0, 0, 40, 1, 0)]


def test_decode_runs_between_tiles():
    reqs = [(0, 2, 0), (2, 16, 1), (18, 3, 0), (21, 128, 2), (149, 1, 0)]
    plan = state.plan_step(args(150), P.KV_FP8, reqs, 1000, 0)
    ks = kernels(plan)
    assert [(k[0], k[1], k[2]) for k in ks] == [(0, 0, 2), (0, 18, 3), (0, 149, 1),
                                                 (1, 2, 16), (1, 21, 128)]


def test_prefill_tiles_unsplit_when_they_fill_the_gpu():
    """256 prefill tiles x 4 kv heads already fill every tile slot: no split
    (and no combine pass); 8 verify blocks alone get split-K."""
    reqs = [(512 * i, 512, 2, 9000 + 512) for i in range(8)]
    ks = kernels(state.plan_step(args(4096), P.KV_FP8, reqs, 16384, 256 << 20))
    assert ks == [(1, 0, 4096, 1, 0)]
    reqs = [(16 * i, 16, 1, 9000) for i in range(8)]
    ks = kernels(state.plan_step(args(128), P.KV_FP8, reqs, 16384, 256 << 20))
    assert ks[0][:3] == (1, 0, 128) and ks[0][3] > 1


def test_request_lengths_shape_the_decode_split():
    """Rows announced as short (max_visible per request) need fewer splits than
    rows assumed at the step's max_visible_tokens."""
    unknown = [(i, 1, 0) for i in range(48)]
    short = [(i, 1, 0, 3000) for i in range(48)]
    a = kernels(state.plan_step(args(48), P.KV_FP8, unknown, 65536, 1 << 30))[0]
    b = kernels(state.plan_step(args(48), P.KV_FP8, short, 65536, 1 << 30))[0]
    assert a[3] > 1 and b[3] >= 1
    assert b[3] * b[4] < a[3] * a[4] or b[4] < a[4]


def test_choose_decode_split_export():
    """psk_choose_decode_split: the north-star workload splits (B=64 x 32k FP8
    on 256 CUs), every split holds >= 16 pages, and the cap is honoured."""
    from phaseshift_amd import ops
    sp, pp = ops.choose_decode_split(64, 24, 4, 256, 16, True, [32768] * 64, 1 << 40)
    assert sp > 1 and pp >= 16 and sp * pp >= 2048
    cap = 64 * 4 * 2 * 6 * 258 * 4
    sp, pp = ops.choose_decode_split(64, 24, 4, 256, 16, True, [32768] * 64, cap)
    assert sp <= 2
    sp, pp = ops.choose_decode_split(64, 24, 4, 256, 16, True, [1000] * 64, 1 << 40)
    assert sp == 1   # below the reference's 2048-token split threshold


def test_psq_steps_use_tiles_where_the_tile_kernel_covers_them():
    """PSQ pools at head_dim 256: the config-5 request mix plans like FP8 (decode
    rows, one verify tile launch, one prefill tile launch); at head_dim 64 (outside the PSQ tile kernel) every row is a
    decode row."""
    reqs = ([(i, 1, 0) for i in range(48)] + [(48 + 16 * i, 16, 1) for i in range(8)] +
            [(176 + 512 * i, 512, 2) for i in range(8)])
    for dt in (P.KV_PSQ4, P.KV_PSQ8):
        plan = state.plan_step(args(4272), dt, reqs, 16384, 256 << 20)
        ks = kernels(plan)
        assert [k[:3] for k in ks] == [(0, 0, 48), (1, 48, 128), (1, 176, 4096)]
        plan = state.plan_step(args(4272, hd=64), dt, reqs, 16384, 256 << 20)
        assert [k[:3] for k in kernels(plan)] == [(0, 0, 4272)]
        plan = state.plan_step(args(64), dt, [(i, 1, 0) for i in range(64)], 32768, 1 << 30)
        assert kernels(plan)[0][3] > 1


def test_psq_choose_decode_split_and_unknown_dtype():
    from phaseshift_amd import ops
    import pytest
    for dt in (P.KV_PSQ4, P.KV_PSQ8):
        sp, pp = ops.choose_decode_split(64, 24, 4, 256, 16, False, [32768] * 64, 1 << 40,
                                         kv_dtype=dt)
        assert sp > 1 and sp * pp >= 2048
    with pytest.raises(P.HipError):
        ops.choose_decode_split(64, 24, 4, 256, 16, False, [32768] * 64, 1 << 40, kv_dtype=2)


def test_other_launches_beside_the_largest_tile_launch():
    """In a step with a tile launch of >= 1024 rows, every other launch (decode,
    the verify tile launch) goes to the side stream when the split-K
    workspace holds the large launch's partials and, after them, the largest
    side launch's; otherwise the step stays in order."""
    reqs = ([(i, 1, 0) for i in range(48)] + [(48 + 16 * i, 16, 1) for i in range(8)] +
            [(176 + 512 * i, 512, 2) for i in range(8)])
    plan = state.plan_step(args(4272), P.KV_FP8, reqs, 16384, 256 << 20)
    ks = plan.kernels[:plan.count]
    # decode on side lane 1, the verify tile launch on lane 2 (each its own workspace region)
    assert [(k.kind, k.side) for k in ks] == [(0, 1), (1, 2), (1, 0)]
    # small tile steps (largest tile launch under 1024 rows) and decode-only steps never fork
    small = [(i, 1, 0) for i in range(8)] + [(8, 16, 1), (24, 128, 2)]
    plan = state.plan_step(args(152), P.KV_FP8, small, 16384, 256 << 20)
    assert [k.side for k in plan.kernels[:plan.count]] == [0, 0, 0]
    plan = state.plan_step(args(64), P.KV_FP8, [(i, 1, 0) for i in range(64)], 32768, 256 << 20)
    assert [k.side for k in plan.kernels[:plan.count]] == [0]
    # for any workspace: side launches sit after the large launch's partials
    # (one 1024-row prefill chunk beside 48 decode rows: the chunk splits too)
    reqs = [(i, 1, 0) for i in range(48)] + [(48, 1024, 2)]
    forked = ordered = 0
    # (caps around 76 MB hold the chunk's 3-split partials but not the decode's beside them)
    for cap in [1 << 20, 16 << 20, 64 << 20, 256 << 20] + [(70 + 2 * i) << 20 for i in range(8)]:
        plan = state.plan_step(args(1072), P.KV_FP8, reqs, 16384, cap)
        ks = plan.kernels[:plan.count]
        need = [k.rows * 4 * k.splits * 6 * 258 * 4 if k.splits > 1 else 0 for k in ks]
        main = max(range(len(ks)), key=lambda i: ks[i].rows if ks[i].kind == 1 else -1)
        side = max(n for i, n in enumerate(need) if i != main)
        at = ((need[main] + 255) // 256) * 256
        if ks[0].side:
            forked += 1
            assert all(k.side for i, k in enumerate(ks) if i != main) and not ks[main].side
            assert side == 0 or at + side <= cap
        else:
            ordered += 1
            assert not any(k.side for k in ks)
            assert at + side > cap
    assert forked and ordered


def test_verify_split_fills_one_round_of_units():
    """Split verify tiles run as dense (tile, split) units; the planner sizes
    the split from each block's own context so that the units of config 5's
    8 verify blocks (contexts 3.7k-15.4k, 4 kv heads) fit one round of one
    6-wave workgroup per CU (256 CUs) while still splitting."""
    import math
    rng = np.random.default_rng(5005)
    ctx = rng.integers(2048, 16385, 64)
    vis = [int(c) + 16 for c in ctx[56:]]
    reqs = [(16 * i, 16, 1, v) for i, v in enumerate(vis)]
    plan = state.plan_step(args(128), P.KV_FP8, reqs, int(ctx.max()) + 512, 256 << 20)
    k = plan.kernels[0]
    assert plan.count == 1 and k.kind == 1 and k.splits > 1
    units = sum(math.ceil(math.ceil(v / 16) / k.pages_per_split) for v in vis) * 4
    assert 128 < units <= 256, (k.splits, k.pages_per_split, units)


def test_side_lanes_fall_back_to_one_lane():
    """Config-5 shape: the decode launch on side lane 1 and the verify launch
    on lane 2 when the workspace holds both partial regions; both on lane 1,
    sharing one region, when it holds only the larger of them."""
    reqs = ([(i, 1, 0) for i in range(48)] + [(48 + 16 * i, 16, 1) for i in range(8)] +
            [(176 + 512 * i, 512, 2) for i in range(8)])

    def plan_at(cap):
        ks = state.plan_step(args(4272), P.KV_FP8, reqs, 16384, cap).kernels
        ks = [ks[i] for i in range(3)]
        need = [k.rows * 4 * k.splits * 6 * 258 * 4 if k.splits > 1 else 0 for k in ks]
        return [(k.kind, k.side, k.splits) for k in ks], need

    both, need = plan_at(256 << 20)
    assert [(k, s) for k, s, _ in both] == [(0, 1), (1, 2), (1, 0)], both
    assert need[0] > 0 and need[1] > 0 and need[2] == 0
    # room for the larger region only (the regions start 256-byte aligned)
    one, need1 = plan_at(max(need[0], need[1]) + 1024)
    assert need1 == need and [s for _, _, s in one] == [s for _, _, s in both]
    assert [(k, s) for k, s, _ in one] == [(0, 1), (1, 1), (1, 0)], one


def test_args_keep_their_tensors_alive():
    """The argument structs hold raw device pointers; they keep the tensors
    they point into alive (a temporary passed in must not be freed and its
    memory reused while the struct is still launched)."""
    import gc
    import weakref
    import torch
    from phaseshift_amd import ops
    g = ops.PoolGeometry(1, 8, 16, 4, 64)
    q = torch.zeros((3, 8 * 64), dtype=torch.bfloat16)
    ref = weakref.ref(q)
    a = ops.attention_args(g, 0, q, torch.zeros((3, 8 * 64)), torch.zeros(3, dtype=torch.int32),
                           torch.zeros(3, dtype=torch.int32), torch.zeros((2, 4), dtype=torch.int32), 8)
    del q
    gc.collect()
    assert ref() is not None and a.q == ref().data_ptr()
    k = torch.zeros((3, 4 * 64), dtype=torch.bfloat16)
    ref_k = weakref.ref(k)
    b = ops.append_args(g, 0, k, torch.zeros_like(k), torch.zeros(3, dtype=torch.int32),
                        torch.zeros(3, dtype=torch.int32), torch.zeros((2, 4), dtype=torch.int32))
    del k
    gc.collect()
    assert ref_k() is not None and b.k_input == ref_k().data_ptr()


def test_split_chooser_against_measured_sweep():
    """psk_choose_decode_split on the bench workloads picks a split whose measured
    kernel time (one MI355X, tests/measured/decode_split_times_mi355x.json, written on one
    MI355X box by a working sweep script that is not part of the library) is within 5% of the fastest measured split."""
    import json
    import os
    import numpy as np
    from phaseshift_amd import ops
    path = os.path.join(os.path.dirname(__file__), "measured", "decode_split_times_mi355x.json")
    times = json.load(open(path))
    rng = np.random.default_rng(404)
    cfg4 = np.exp(rng.uniform(np.log(4096), np.log(65536), 64)).astype(np.int64)
    cfg3 = np.random.default_rng(303).integers(1024, 32769, 32)
    cases = [("cfg4_fp8_loguniform_seed404", cfg4, True),
             ("cfg3_bf16_uniform_seed303", cfg3, False),
             ("main_fp8_b64_ctx32k", np.array([32768] * 64), True)]
    for name, lens, fp8 in cases:
        measured = {int(k): v for k, v in times[name].items()}
        sp, pp = ops.choose_decode_split(len(lens), 24, 4, 256, 16, fp8, [int(x) for x in lens], 1 << 40)
        assert pp in measured, (name, sp, pp)
        best = min(measured.values())
        assert measured[pp] <= 1.05 * best, (name, pp, measured[pp], best)


def test_append_rejects_inputs_it_would_misread():
    """kv_append / kv_append_psq read each input row as kv_heads*head_dim packed
    bf16 values: float32, transposed or short inputs are rejected up front."""
    import torch
    from phaseshift_amd import ops
    g = ops.PoolGeometry(1, 8, 16, 4, 64)
    i32 = lambda *s: torch.zeros(s, dtype=torch.int32)
    good = torch.zeros((3, 4 * 64), dtype=torch.bfloat16)
    ops.append_args(g, 0, good, good, i32(3), i32(3), i32(2, 4))
    for bad, exc in ((torch.zeros((3, 256)), TypeError),
                     (torch.zeros((256, 3), dtype=torch.bfloat16).t(), ValueError),
                     (torch.zeros((3, 255), dtype=torch.bfloat16), ValueError),
                     (torch.zeros((4, 256), dtype=torch.bfloat16), ValueError)):
        with pytest.raises(exc):
            ops.append_args(g, 0, good, bad, i32(3), i32(3), i32(2, 4))


def _fresh_split(*args, **kw):
    """psk_choose_decode_split in a new thread: its plan memo is thread-local,
    so this is a computation from scratch."""
    import threading
    from phaseshift_amd import ops
    out = []
    t = threading.Thread(target=lambda: out.append(ops.choose_decode_split(*args, **kw)))
    t.start()
    t.join()
    return out[0]


def test_split_memo_reuse_rules():
    """The chooser's per-thread plan memo: identical inputs give the fresh
    answer in any A, B, A order; a plan is reused across small page drifts
    only while it stays valid (no row needs more splits, the unit count is
    unchanged, the total drift is at most 1/64 of the pages); any other input
    change (partials workspace, a long jump, the batch shape) recomputes."""
    from phaseshift_amd import ops
    rng = np.random.default_rng(404)
    A = [int(x) for x in np.exp(rng.uniform(np.log(4096), np.log(65536), 64))]
    B = [32768] * 64
    args = lambda v, pb=64 << 20: (64, 24, 4, 256, 16, True, v, pb)
    fa, fb = _fresh_split(*args(A)), _fresh_split(*args(B))
    assert fa != fb
    for v, want in ((A, fa), (B, fb), (A, fa), (B, fb)):
        assert ops.choose_decode_split(*args(v)) == want
    # one row grows by one page (16 tokens): the memo answers with A's plan
    A1 = list(A)
    A1[3] += 16
    assert ops.choose_decode_split(*args(A1)) == fa
    sp, pp = fa
    # a row pushed past sp * pp pages would need more splits: recomputed
    A2 = list(A)
    A2[0] = sp * pp * 16 + 1
    assert ops.choose_decode_split(*args(A2)) == _fresh_split(*args(A2))
    # drift above 1/64 of the pages: recomputed
    A3 = [x + 400 for x in A]
    assert ops.choose_decode_split(*args(A3)) == _fresh_split(*args(A3))
    # a different partials workspace: recomputed
    assert ops.choose_decode_split(*args(A, 8 << 20)) == _fresh_split(*args(A, 8 << 20))
    # a unit-count change (a row crossing a multiple of the split size)
    A4 = list(A)
    r = int(np.argmax([(-(-x // 16)) % pp for x in A]))   # row nearest its next boundary
    A4[r] = (-(-A[r] // 16) // pp + 1) * pp * 16 + 1
    if (-(-A4[r] // 16) + pp - 1) // pp <= sp:
        assert ops.choose_decode_split(*args(A4)) == _fresh_split(*args(A4))
