"""The chunk index of the multi-tensor kernels (csrc/kernels/mta_index.h),
compiled for the host and checked block by block against bisection of the
chunk prefix table."""
import os
import subprocess

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_bucket_index_matches_bisection(tmp_path):
    exe = tmp_path / "test_mta_index"
    subprocess.run(["g++", "-O2", "-std=c++17", "-I", os.path.join(ROOT, "torch-supa_amd", "csrc", "kernels"),
                    os.path.join(ROOT, "tests", "cpp", "test_mta_index.cpp"), "-o", str(exe)], check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    assert r.stdout.startswith("OK")
