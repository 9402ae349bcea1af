"""Host-side C++ of the path built for the CPU and checked by brute force, and
the same programs built with AddressSanitizer and UndefinedBehaviorSanitizer
(g++ on host sources only; no GPU code is built with a sanitizer):

* csrc/kernels/divmod.h      -- magic-number division vs exact division
* csrc/kernels/mta_index.h   -- multi-tensor chunk index vs bisection
* csrc/kernels/split32.h     -- the 2^31-element split, with the limit lowered
                                to 1..1000, vs brute-force enumeration
* csrc/host/planner.cpp      -- broadcast / layout / coalescing plans vs
                                brute-force enumeration, mismatches rejected
"""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
KERNELS = os.path.join(ROOT, "torch-supa_amd", "csrc", "kernels")
HOST = os.path.join(ROOT, "torch-supa_amd", "csrc", "host")
INCLUDE = os.path.join(ROOT, "include")
CPP = os.path.join(ROOT, "tests", "cpp")

PROGRAMS = {
    "divmod": (["test_divmod.cpp"], []),
    "mta_index": (["test_mta_index.cpp"], []),
    "split32": (["test_split32.cpp"], []),
    "planner": (["test_planner_fuzz.cpp"], [os.path.join(HOST, "planner.cpp")]),
}
SANITIZE = ["-fsanitize=address,undefined", "-fno-sanitize-recover=all", "-fno-omit-frame-pointer", "-g"]


def _build_and_run(tmp_path, name, flags):
    srcs, extra = PROGRAMS[name]
    exe = tmp_path / f"test_{name}"
    cmd = ["g++", "-std=c++17", *flags, "-I", KERNELS, "-I", HOST, "-I", INCLUDE,
           *[os.path.join(CPP, s) for s in srcs], *extra, "-o", str(exe)]
    subprocess.run(cmd, check=True)
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0", UBSAN_OPTIONS="print_stacktrace=1")
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=600, env=env)
    assert r.returncode == 0, r.stdout + r.stderr
    assert r.stdout.startswith("OK"), r.stdout


@pytest.mark.parametrize("name", ["split32", "planner"])
def test_brute_force(tmp_path, name):
    _build_and_run(tmp_path, name, ["-O2"])


@pytest.mark.parametrize("name", sorted(PROGRAMS))
def test_sanitized(tmp_path, name):
    _build_and_run(tmp_path, name, ["-O1", *SANITIZE])
