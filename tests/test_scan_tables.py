"""CPU check of the host work splits (maxsim_amd/csrc/scan_tables.cpp,
score_tables.cpp): compiled with g++ against the library sources and run over
random ragged corpora, in both scan partition modes and for documents and
candidate targets of the generalized scorer."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.mark.skipif(shutil.which("g++") is None, reason="g++ not available")
def test_scan_tables_cover_every_token_once_per_document(tmp_path):
    exe = tmp_path / "scan_tables_check"
    src = os.path.join(ROOT, "tests", "cpp", "scan_tables_check.cpp")
    libs = [os.path.join(ROOT, "maxsim_amd", "csrc", f) for f in ("scan_tables.cpp", "score_tables.cpp")]
    subprocess.run(["g++", "-std=c++17", "-O1", "-I", os.path.join(ROOT, "maxsim_amd", "csrc"),
                    "-I", "/opt/rocm/include", "-D__HIP_PLATFORM_AMD__", src, *libs, "-o", str(exe)],
                   check=True, capture_output=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout
    assert out.strip() == "ok"
