"""In-tree build of the two shared libraries of the package.

* ``torch_supa/libsupa_amd_kernels.so`` -- the gfx950 HIP kernels behind the
  C ABI declared in ``include/supa_amd.h`` (no torch dependency).
* ``torch_supa/_C<ext>`` -- the PyTorch PrivateUse1 backend (runtime,
  planner, operator registrations, Python bindings), linked to the kernels.

Usage: ``python torch-supa_amd/build.py [--jobs N] [--incremental]``.
Every translation unit is compiled on each call unless ``--incremental`` is
given (then only sources newer than their object are rebuilt).
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import subprocess
import sys
import sysconfig

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)
PKG = os.path.join(HERE, "torch_supa")
BUILD = os.path.join(HERE, "_build")
KERNEL_DIR = os.path.join(HERE, "csrc", "kernels")
HOST_DIR = os.path.join(HERE, "csrc", "host")
INCLUDE = os.path.join(REPO, "include")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HIPCC = os.path.join(ROCM, "bin", "hipcc")
ARCH = "gfx950"

KERNELS_SO = os.path.join(PKG, "libsupa_amd_kernels.so")
EXT_SUFFIX = sysconfig.get_config_var("EXT_SUFFIX") or ".so"
C_SO = os.path.join(PKG, "_C" + EXT_SUFFIX)

HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-std=c++20", "-O3", "-fPIC",
    # bit-reproducible float math: no implicit contraction into fma
    "-ffp-contract=off",
    # no packed fp32 VALU instructions
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # without packed fp32 the SLP vectorizer's <2 x float> groups gain nothing,
    # and some (f16 negation in the two-row broadcast kernel) fail instruction
    # selection
    "-fno-slp-vectorize",
    "-I", INCLUDE, "-I", KERNEL_DIR,
]


def _torch_paths():
    import torch
    from torch.utils import cpp_extension as ce

    inc = ce.include_paths()
    libdir = os.path.join(os.path.dirname(torch.__file__), "lib")
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    return inc, libdir, abi


def _run(cmd):
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if r.returncode != 0:
        raise RuntimeError("build step failed:\n" + " ".join(cmd) + "\n" + r.stdout[-8000:])
    return r.stdout


def _stale(src, obj, deps):
    if not os.path.exists(obj):
        return True
    t = os.path.getmtime(obj)
    return any(os.path.getmtime(p) > t for p in [src] + deps)


def build(jobs: int | None = None, incremental: bool = False, verbose: bool = True) -> None:
    os.makedirs(os.path.join(BUILD, "kernels"), exist_ok=True)
    os.makedirs(os.path.join(BUILD, "host"), exist_ok=True)
    jobs = jobs or min(16, os.cpu_count() or 4)
    inc, torch_lib, abi = _torch_paths()
    py_inc = sysconfig.get_paths()["include"]

    kdeps = [os.path.join(KERNEL_DIR, f) for f in os.listdir(KERNEL_DIR) if f.endswith(".h")]
    kdeps.append(os.path.join(INCLUDE, "supa_amd.h"))
    hdeps = [os.path.join(HOST_DIR, f) for f in os.listdir(HOST_DIR) if f.endswith(".h")]
    hdeps.append(os.path.join(INCLUDE, "supa_amd.h"))

    jobs_list = []
    kobjs = []
    for f in sorted(os.listdir(KERNEL_DIR)):
        if not f.endswith(".hip"):
            continue
        src = os.path.join(KERNEL_DIR, f)
        obj = os.path.join(BUILD, "kernels", f[:-4] + ".o")
        kobjs.append(obj)
        if not incremental or _stale(src, obj, kdeps):
            jobs_list.append([HIPCC, *HIP_FLAGS, "-c", src, "-o", obj])
    host_flags = [
        "-std=c++17", "-O2", "-fPIC", "-Wall", "-Wno-unused-parameter", "-Wno-sign-compare",
        "-D__HIP_PLATFORM_AMD__", "-DTORCH_EXTENSION_NAME=_C", "-DTORCH_API_INCLUDE_EXTENSION_H",
        f"-D_GLIBCXX_USE_CXX11_ABI={abi}", "-I", py_inc, "-I", os.path.join(ROCM, "include"),
        "-I", INCLUDE, "-I", HOST_DIR,
    ]
    for p in inc:
        host_flags += ["-isystem", p]
    hobjs = []
    for f in sorted(os.listdir(HOST_DIR)):
        if not f.endswith(".cpp"):
            continue
        src = os.path.join(HOST_DIR, f)
        obj = os.path.join(BUILD, "host", f[:-4] + ".o")
        hobjs.append(obj)
        if not incremental or _stale(src, obj, hdeps):
            jobs_list.append(["g++", *host_flags, "-c", src, "-o", obj])

    if verbose and jobs_list:
        print(f"[torch_supa build] compiling {len(jobs_list)} translation units with {jobs} jobs", flush=True)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        futs = [ex.submit(_run, c) for c in jobs_list]
        for fu in futs:
            fu.result()

    # kernels: shared library against torch's HIP runtime (same SONAME as
    # /opt/rocm's, so one runtime is loaded whichever comes first)
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", KERNELS_SO + ".tmp", *kobjs,
          "-L", torch_lib, "-lamdhip64", f"-Wl,-rpath,{torch_lib}"])
    os.replace(KERNELS_SO + ".tmp", KERNELS_SO)
    _run(["g++", "-shared", "-o", C_SO + ".tmp", *hobjs, "-L", PKG, "-lsupa_amd_kernels",
          "-L", torch_lib, "-lc10", "-ltorch", "-ltorch_cpu", "-ltorch_python", "-lamdhip64",
          "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{torch_lib}"])
    os.replace(C_SO + ".tmp", C_SO)
    if verbose:
        print(f"[torch_supa build] wrote {os.path.relpath(KERNELS_SO, REPO)} and {os.path.relpath(C_SO, REPO)}",
              flush=True)


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=None)
    ap.add_argument("--incremental", action="store_true")
    a = ap.parse_args(argv)
    build(a.jobs, a.incremental)


if __name__ == "__main__":
    main()
