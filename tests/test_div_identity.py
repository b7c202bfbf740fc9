"""The FP8 append kernel's reciprocal+FMA division gives the same E4M3 code as
the IEEE division x / scale the reference performs (kv_append.hip:249-250), for
every finite bf16 input pair. Exhaustive, on the CPU (IEEE fma == v_fma_f32)."""
import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)


def test_division_identity_exhaustive(tmp_path):
    exe = tmp_path / "div_identity"
    subprocess.run(["gcc", "-O2", "-fopenmp", "-ffp-contract=off", "-std=c11",
                    os.path.join(HERE, "native", "div_identity.c"),
                    os.path.join(ROOT, "oracle", "ps_oracle.c"), "-o", str(exe), "-lm"],
                   check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=600,
                       env=dict(os.environ, OMP_NUM_THREADS=os.environ.get("OMP_NUM_THREADS", "8")))
    assert r.returncode == 0, r.stdout + r.stderr
    assert "code_mismatches 0" in r.stdout
