"""Link-level drop-in: a program compiled against the reference's own launcher
headers (kv_append.h, attention/paged_attention.h, read in place from the
reference tree) links against libphaseshift_kv.so and gets the reference's
error behaviour for invalid arguments. Skipped where the reference is absent."""
import os
import subprocess

import pytest

import phaseshift_amd as P

REF = "/root/reference"
HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.mark.skipif(not os.path.isdir(os.path.join(REF, "include")), reason="no reference tree")
def test_reference_headers_link_against_library(tmp_path):
    exe = tmp_path / "link_ref"
    lib_dir = os.path.dirname(P.LIB_PATH)
    subprocess.run(["/opt/rocm/bin/hipcc", "-std=c++20", "-O1", f"-I{REF}/include",
                    os.path.join(HERE, "native", "link_reference_headers.cpp"),
                    f"-L{lib_dir}", "-lphaseshift_kv", f"-Wl,-rpath,{lib_dir}", "-o", str(exe)],
                   check=True, capture_output=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "missing 0" in r.stdout
