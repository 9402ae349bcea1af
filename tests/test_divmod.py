"""The magic-number divider of the strided kernels (csrc/kernels/divmod.h),
compiled for the host and checked against exact division by brute force."""
import os
import subprocess

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_fastdiv_matches_exact_division(tmp_path):
    exe = tmp_path / "test_divmod"
    subprocess.run(["g++", "-O2", "-std=c++17", "-I", os.path.join(ROOT, "torch-supa_amd", "csrc", "kernels"),
                    os.path.join(ROOT, "tests", "cpp", "test_divmod.cpp"), "-o", str(exe)], check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True)
    assert r.returncode == 0, r.stdout + r.stderr
    assert r.stdout.startswith("OK")
