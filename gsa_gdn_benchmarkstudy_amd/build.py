"""Build libgsa_hip.so (the gfx950 kernels and their C ABI) in-tree with hipcc.

Usage: ``python -m gsa_gdn_benchmarkstudy_amd.build`` or ``build_library()``.
Every call recompiles; objects go to ``_build/`` beside this file and the
library to ``libgsa_hip.so`` in this package directory.

For kernel work, ``python -m gsa_gdn_benchmarkstudy_amd.build --dense-src COPY.hip
--out LIB.so`` builds a separate library with ``dense_attn.hip`` replaced by a
copy (objects under ``_build/variant/``), to be timed against the default build
with ``python -m gsa_gdn_benchmarkstudy_amd.attn_ab``.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(PKG_DIR, "csrc")
BUILD_DIR = os.path.join(PKG_DIR, "_build")
LIB_PATH = os.path.join(PKG_DIR, "libgsa_hip.so")
ARCH = "gfx950"

HIP_SOURCES = ("indexer.hip", "topk_select.hip", "sparse_attn.hip", "dense_attn.hip", "proj_fused.hip")
CXX_SOURCES = ("abi.cpp",)

# Packed fp32 VALU forms are disabled in device code: the compiler would
# otherwise form v_pk_{add,mul,fma}_f32 from ordinary float code.
DEVICE_FLAGS = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
COMMON_FLAGS = ["-O3", "-std=c++20", "-fPIC", "-Wall", "-Wno-unused-function"]
# The indexer's MFMA results feed VALU epilogues directly: keep them in arch
# VGPRs instead of AGPRs (saves a v_accvgpr_read per result element).
FILE_FLAGS = {"indexer.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=true"]}


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass reports the device-only feature flag as unknown: drop that line
    err = "\n".join(l for l in res.stderr.splitlines() if "packed-fp32-ops" not in l)
    if res.returncode != 0:
        raise RuntimeError(f"command failed ({res.returncode}): {' '.join(cmd)}\n{err}")
    if verbose and err.strip():
        print(err, file=sys.stderr)


def build_library(verbose: bool = False, jobs: int = 4, overrides=None, out: str = None) -> str:
    """Compile every source for gfx950 and link libgsa_hip.so; returns its path.
    `overrides` maps a source name (e.g. "dense_attn.hip") to the path of a copy
    to compile in its place; with overrides the objects go to _build/variant/ and
    the library to `out`, so the default build is left alone."""
    overrides = dict(overrides or {})
    unknown = set(overrides) - set(HIP_SOURCES + CXX_SOURCES)
    if unknown:
        raise ValueError(f"unknown sources to override: {sorted(unknown)}")
    if overrides and not out:
        raise ValueError("a build with overridden sources needs an output path")
    cc = hipcc()
    bdir = os.path.join(BUILD_DIR, "variant") if overrides else BUILD_DIR
    os.makedirs(bdir, exist_ok=True)
    jobs_list = []
    objs = []
    for src in HIP_SOURCES + CXX_SOURCES:
        obj = os.path.join(bdir, os.path.splitext(src)[0] + ".o")
        path = os.path.abspath(overrides.get(src, os.path.join(CSRC, src)))
        cmd = [cc, f"--offload-arch={ARCH}", *COMMON_FLAGS, f"-I{CSRC}", "-c", path, "-o", obj]
        if src.endswith(".hip"):
            cmd[2:2] = DEVICE_FLAGS + FILE_FLAGS.get(src, [])
        else:
            cmd = [cc, *COMMON_FLAGS, "-x", "c++", "-c", path, "-o", obj]
        jobs_list.append(cmd)
        objs.append(obj)
    with ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        list(ex.map(lambda c: _run(c, verbose), jobs_list))
    dst = os.path.abspath(out) if out else LIB_PATH
    tmp = dst + ".tmp"
    _run([cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs], verbose)
    os.replace(tmp, dst)
    return dst


if __name__ == "__main__":
    import argparse

    ap = argparse.ArgumentParser(description="build libgsa_hip.so for gfx950")
    ap.add_argument("-v", "--verbose", action="store_true")
    ap.add_argument("--dense-src", help="a copy of dense_attn.hip to build in its place (needs --out)")
    ap.add_argument("--out", help="library path for a build with a replaced source")
    a = ap.parse_args()
    ov = {"dense_attn.hip": a.dense_src} if a.dense_src else None
    print(build_library(verbose=a.verbose, overrides=ov, out=a.out))
