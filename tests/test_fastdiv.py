"""The launch-time integer division of the PSQ append kernel
(phaseshift_amd/csrc/fastdiv.h: multiply-high, subtract, two shifts) equals
n / d for every divisor 1..4096 and 2^k +- 1 over edge and random 32-bit
numerators, on the CPU."""
import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)


def test_fastdiv_matches_division(tmp_path):
    exe = tmp_path / "fastdiv_check"
    subprocess.run(["g++", "-O2", "-std=c++17", "-I", os.path.join(ROOT, "phaseshift_amd", "csrc"),
                    os.path.join(HERE, "native", "fastdiv_check.cpp"), "-o", str(exe)], check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "mismatches 0" in r.stdout
