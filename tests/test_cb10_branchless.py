"""The PSQ4 append kernel's branch-free cb10 code (a 3-bit lookup of
min(ceil((|x| * inv) * 2), 19), inv = 1/s) equals the reference's comparison
chain (psq_device.h:22-31): exhaustively for every non-negative float bit
pattern (NaNs and +inf included), for every positive bf16 scale (subnormals
included) over a spread of x, and for 2^26 random (x, bf16 scale) pairs, on the
CPU (IEEE fminf/ceilf and one rounding per multiply are the device's v_min,
v_ceil and v_mul)."""
import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)


def test_cb10_branchless_exhaustive(tmp_path):
    exe = tmp_path / "cb10_branchless"
    subprocess.run(["gcc", "-O2", "-fopenmp", "-ffp-contract=off", "-fno-fast-math", "-std=c11",
                    os.path.join(HERE, "native", "cb10_branchless.c"),
                    os.path.join(ROOT, "oracle", "ps_oracle.c"), "-o", str(exe), "-lm"],
                   check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=600,
                       env=dict(os.environ, OMP_NUM_THREADS=os.environ.get("OMP_NUM_THREADS", "8")))
    assert r.returncode == 0, r.stdout + r.stderr
    assert "mismatches 0" in r.stdout
