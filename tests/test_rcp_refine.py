"""The PSQ append kernel's reciprocal of a bf16 block scale (hardware
reciprocal, within one ulp, refined by two FMAs) is the correctly rounded
1/s for every bf16 s in [2^-126, 2^126], whichever float within one ulp the
hardware returns. Exhaustive, on the CPU (IEEE fmaf == v_fma_f32)."""
import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))


def test_rcp_refine_exhaustive(tmp_path):
    exe = tmp_path / "rcp_refine"
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-std=c11",
                    os.path.join(HERE, "native", "rcp_refine.c"), "-o", str(exe), "-lm"], check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "mismatches 0" in r.stdout
