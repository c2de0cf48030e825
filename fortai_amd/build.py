"""Build the gfx950 backend library in-tree (no JIT cache, so it travels).

``libfortai_hip.so`` is compiled by hipcc for gfx950 only, with
multiply/add contraction off (the kernels write every fused multiply-add they
intend explicitly), and packed-fp32 instruction selection disabled.
"""

from __future__ import annotations

import glob
import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "lib", "libfortai_hip.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

HIP_FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-shared", "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def build_library(verbose: bool = False, jobs: int = 0) -> str:
    """Each source is compiled to its own object in parallel (no relocatable
    device code: no kernel or device symbol crosses a source file), then
    linked into the shared library."""
    from concurrent.futures import ThreadPoolExecutor
    os.makedirs(os.path.dirname(LIB), exist_ok=True)
    objdir = os.path.join(os.path.dirname(LIB), "obj")
    os.makedirs(objdir, exist_ok=True)
    sources = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    compile_flags = [f for f in HIP_FLAGS if f != "-shared"]

    def compile_one(src):
        obj = os.path.join(objdir, os.path.basename(src).replace(".hip", ".o"))
        res = subprocess.run([HIPCC, *compile_flags, "-c", src, "-o", obj], capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"hipcc failed on {os.path.basename(src)}:\n" + res.stderr)
        if verbose and res.stderr:
            print(res.stderr)
        return obj

    jobs = jobs or min(len(sources), max(1, (os.cpu_count() or 1)), 8)
    with ThreadPoolExecutor(jobs) as pool:
        objs = list(pool.map(compile_one, sources))
    tmp = LIB + ".tmp"
    res = subprocess.run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", *objs, "-o", tmp],
                         capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError("hipcc link failed:\n" + res.stderr)
    os.replace(tmp, LIB)
    return LIB


FORTRAN = os.path.join(HERE, "fortran")
FC = os.environ.get("FC_AMD", "/opt/rocm/bin/amdflang")
SMOKE = os.path.join(HERE, "lib", "hip_abi_smoke")


def build_fortran(verbose: bool = False) -> str:
    """Compile the iso_c_binding module (fortai_backend_hip) with its
    standalone status module and link the Fortran ABI smoke program against
    libfortai_hip.so (rpath to this directory)."""
    out = os.path.join(HERE, "lib", "fortran")
    os.makedirs(out, exist_ok=True)
    sources = ["fortai_status.f90", "fortai_backend_hip.f90", "fortai_backend_cuda_on_hip.f90"]
    objs = []
    for name in sources:
        obj = os.path.join(out, name.replace(".f90", ".o"))
        cmd = [FC, "-O2", "-c", os.path.join(FORTRAN, name), "-o", obj, "-J", out]
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"{FC} failed on {name}:\n" + res.stderr)
        objs.append(obj)
    cmd = [FC, "-O2", os.path.join(FORTRAN, "hip_abi_smoke.f90"), *objs[:2], "-I", out, "-J", out,
           "-L", os.path.dirname(LIB), "-lfortai_hip", "-Wl,-rpath,$ORIGIN", "-o", SMOKE]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"{FC} failed linking hip_abi_smoke:\n" + res.stderr)
    if verbose and res.stderr:
        print(res.stderr)
    return SMOKE


def build(verbose: bool = False) -> None:
    build_library(verbose)
    build_fortran(verbose)
