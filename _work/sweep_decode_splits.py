"""Measures the decode split kernel at every distinct pages_per_split of the bench
workloads on one GPU and writes decode_split_times_mi355x.json beside this file.

Run on an MI355X from the repository root:
    python tests/measured/sweep_decode_splits.py
The file it writes is the fixture of tests/test_planner.py::test_split_chooser_against_measured_sweep
(kernel milliseconds per pages_per_split, HIP events over 10 launches after 3 warm-ups).
"""
import json
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)


def main():
    import torch
    import bench
    from phaseshift_amd import ops
    dev = torch.device("cuda:0")
    rng = np.random.default_rng(404)
    cfg4 = np.exp(rng.uniform(np.log(4096), np.log(65536), 64)).astype(np.int64)
    cfg3 = np.random.default_rng(303).integers(1024, 32769, 32)
    main_lens = np.array([32768] * 64)
    out = {"note": "decode split-kernel time (ms) per pages_per_split on one MI355X "
                   "(tests/measured/sweep_decode_splits.py)"}
    for name, lens, fp8, seed, min_per in [("cfg4_fp8_loguniform_seed404", cfg4, True, 404, 24),
                                           ("cfg3_bf16_uniform_seed303", cfg3, False, 404, 24),
                                           ("main_fp8_b64_ctx32k", main_lens, True, 404, 32)]:
        st = bench.decode_setup(torch, ops, lens, fp8, seed, dev)
        maxp = (int(lens.max()) + 15) // 16
        pers = sorted(set((maxp + s - 1) // s for s in range(2, maxp // 16)))
        res = {}
        for pps in [p for p in pers if p >= min_per]:
            splits = (maxp + pps - 1) // pps
            _, k_ms, _, _, _, _ = bench.run_decode(torch, ops, st, 10, 3, dev, splits=splits, pps=pps)
            res[str(pps)] = round(k_ms, 4)
            print(name, pps, res[str(pps)], flush=True)
        out[name] = res
        del st
        torch.cuda.empty_cache()
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "decode_split_times_mi355x.json")
    with open(path, "w") as f:
        json.dump(out, f, indent=0)


if __name__ == "__main__":
    main()
