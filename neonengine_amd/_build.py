"""Builds libneon_gptoss.so in-tree with hipcc for gfx950.

Run as ``python -m neonengine_amd._build`` or through __graft_entry__.build().
The shared library is placed next to this file so it travels with the tree.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "libneon_gptoss.so")
SOURCES = ["neon_kernels.hip", "neon_prefill.hip", "neon_mx.hip", "neon_engine.hip"]

HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    # no packed-fp32 instructions: some of their forms have given silent wrong
    # results on this hardware pool
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # every fused multiply-add on the decode path is written out explicitly
    # (the CPU oracle mirrors the exact operation sequence)
    "-ffp-contract=off",
    # LDS holds only what a kernel declares: no compiler-promoted private
    # arrays in LDS
    "-mllvm", "--disable-promote-alloca-to-lds",
    "-Wall",
    "-Wno-unused-function",
]

# every kernel is hand-written: the library links the HIP runtime only
LINK_LIBS: list = []


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build the gfx950 kernels)")


def build(verbose: bool = False) -> str:
    objs = []
    tmp_dir = os.path.join(HERE, "_build")
    os.makedirs(tmp_dir, exist_ok=True)
    procs = []
    for src in SOURCES:
        obj = os.path.join(tmp_dir, src.replace(".hip", ".o"))
        cmd = [hipcc()] + [f for f in HIPCC_FLAGS if f != "-shared"] + [
            "-I", os.path.join(ROOT, "include"), "-c", os.path.join(CSRC, src), "-o", obj]
        procs.append((cmd, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT)))
        objs.append(obj)
    for cmd, p in procs:
        out, _ = p.communicate()
        text = "\n".join(l for l in out.decode(errors="replace").splitlines()
                         if "packed-fp32-ops" not in l)
        if verbose and text.strip():
            print(text)
        if p.returncode != 0:
            raise RuntimeError(f"hipcc failed ({p.returncode}): {' '.join(cmd)}\n{text}")
    tmp = LIB + ".tmp"
    cmd = [hipcc(), "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp] + objs + LINK_LIBS
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT)
    if r.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{r.stdout.decode(errors='replace')}")
    os.replace(tmp, LIB)
    return LIB


# Host sanitizers for the library's host code (argument validation, config
# checks, context set-up: all in neon_engine.hip); the device code is
# unchanged.  Each -fsanitize= is a host-only flag.
SANITIZE_HOST = ["-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fsanitize=undefined",
                 "-Xarch_host", "-fno-sanitize-recover=undefined", "-Xarch_host", "-g",
                 "-Xarch_host", "-fno-omit-frame-pointer"]
ASAN_DIR = os.path.join(HERE, "_asan")
ASAN_LIB = os.path.join(ASAN_DIR, "libneon_gptoss.so")


def build_sanitized(verbose: bool = False) -> str:
    """neonengine_amd/_asan/libneon_gptoss.so: neon_engine.hip recompiled with
    the host sanitizers, linked with the regular objects of build()."""
    os.makedirs(ASAN_DIR, exist_ok=True)
    obj = os.path.join(ASAN_DIR, "neon_engine.o")
    cmd = [hipcc()] + [f for f in HIPCC_FLAGS if f != "-shared"] + SANITIZE_HOST + [
        "-I", os.path.join(ROOT, "include"), "-c", os.path.join(CSRC, "neon_engine.hip"), "-o", obj]
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed: {' '.join(cmd)}\n{r.stdout.decode(errors='replace')}")
    others = [os.path.join(HERE, "_build", s.replace(".hip", ".o")) for s in SOURCES
              if s != "neon_engine.hip"]
    tmp = ASAN_LIB + ".tmp"
    cmd = [hipcc(), "--offload-arch=gfx950", "-shared", "-fPIC", "-Xarch_host", "-fsanitize=address",
           "-Xarch_host", "-fsanitize=undefined", "-Xarch_host", "-shared-libasan", "-o", tmp,
           obj] + others + LINK_LIBS
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT)
    if r.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{r.stdout.decode(errors='replace')}")
    os.replace(tmp, ASAN_LIB)
    return ASAN_LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
    if "--sanitize" in sys.argv:
        print(build_sanitized(verbose="-v" in sys.argv))
