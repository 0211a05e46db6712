"""Build the crbq HIP library in-tree: crb_amd/libcrbq.so (gfx950 only).

    python -m crb_amd.build            # or: from crb_amd.build import build

Each .hip source is compiled with hipcc for gfx950 and linked into one
shared library exporting the C ABI declared in include/crbq.h.  Packed fp32
instructions are disabled (-packed-fp32-ops) and floating-point contraction
is off so the elementwise arithmetic rounds exactly like the reference's
separate torch ops.
"""
from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
OBJ = os.path.join(HERE, "_obj")
LIB = os.path.join(HERE, "libcrbq.so")
SOURCES = ["capi.hip", "gemm_f32.hip", "hessian.hip", "chol.hip", "block.hip", "packed.hip"]

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = [
    "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result",
    "-I", os.path.join(ROOT, "include"),
]


def _compile(src: str) -> str:
    obj = os.path.join(OBJ, src.replace(".hip", ".o"))
    cmd = [HIPCC, *FLAGS, "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src}:\n{r.stdout}\n{r.stderr}")
    return obj


def build(verbose: bool = False) -> str:
    """Compile every source and link libcrbq.so.  Always rebuilds."""
    os.makedirs(OBJ, exist_ok=True)
    with ThreadPoolExecutor(max_workers=min(len(SOURCES), os.cpu_count() or 4)) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = LIB + ".tmp"
    cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", *objs, "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print("built", LIB)
    return LIB


def asan_runtime() -> str | None:
    """The ROCm toolchain's shared AddressSanitizer runtime (to preload into
    a process that loads an ASan build), or None."""
    base = os.path.join(os.path.dirname(os.path.dirname(os.path.realpath(HIPCC))), "llvm", "lib",
                        "clang")
    if not os.path.isdir(base):
        base = "/opt/rocm/llvm/lib/clang"
    if not os.path.isdir(base):
        return None
    for ver in sorted(os.listdir(base), reverse=True):
        p = os.path.join(base, ver, "lib", "linux", "libclang_rt.asan-x86_64.so")
        if os.path.exists(p):
            return p
    return None


def build_host_asan(out_dir: str) -> str:
    """The same library with its host code built with AddressSanitizer
    (-Xarch_host: the gfx950 code is unchanged), for checks of the C ABI's
    host side (argument validation, workspace carving, pointer arrays).  It
    links the shared ASan runtime, which the loading process must preload
    (asan_runtime()).  Not the product library: written to out_dir."""
    objdir = os.path.join(out_dir, "obj")
    os.makedirs(objdir, exist_ok=True)
    flags = [f for f in FLAGS if f != "-O3"] + [
        "-O1", "-g", "-Xarch_host", "-fsanitize=address", "-Xarch_host", "-shared-libasan",
        "-Xarch_host", "-fno-omit-frame-pointer"]

    def one(src: str) -> str:
        obj = os.path.join(objdir, src.replace(".hip", ".o"))
        r = subprocess.run([HIPCC, *flags, "-c", os.path.join(CSRC, src), "-o", obj],
                           capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"hipcc failed on {src}:\n{r.stdout}\n{r.stderr}")
        return obj

    with ThreadPoolExecutor(max_workers=min(len(SOURCES), os.cpu_count() or 4)) as ex:
        objs = list(ex.map(one, SOURCES))
    lib = os.path.join(out_dir, "libcrbq_asan.so")
    link = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC"]
    link += ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-shared-libasan"]
    r = subprocess.run([*link, *objs, "-o", lib], capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    return lib


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
