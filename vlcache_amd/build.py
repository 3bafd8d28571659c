"""Build the gfx950 kernel library ``vlcache_amd/_vlcache_hip.so`` in-tree.

The library is plain ``hipcc`` output with a C ABI (``include/vlc_capi.h``); it
links no torch C++ symbols, so it loads next to any torch build through ctypes.

Usage: ``python -m vlcache_amd.build`` (or ``vlcache_amd.build.build()``).
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
import tempfile

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
REPO_DIR = os.path.dirname(PKG_DIR)
CSRC = os.path.join(PKG_DIR, "csrc")
INCLUDE = os.path.join(REPO_DIR, "include")
LIB_NAME = "_vlcache_hip.so"
LIB_PATH = os.path.join(PKG_DIR, LIB_NAME)
ARCH = "gfx950"

HIP_SOURCES = ["store_kvcache.hip", "rope_store_kv.hip", "rerotate_kv.hip", "varlen_attn.hip", "decode_attn.hip",
               "vision_rope.hip", "norm_act.hip", "linear_skinny.hip"]
HOST_SOURCES = ["attn_plan.cpp", "capi.cpp"]

# Device flags: gfx950 only; packed-fp32 instructions are disabled for all HIP code.
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-fvisibility=hidden",
    "-mcode-object-version=5",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]
HOST_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-fvisibility=hidden", "-Wall", "-Wextra"]


def _hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found: the gfx950 kernel library cannot be built")
    return path


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass warns that it does not know the packed-fp32 feature: harmless.
    err = "\n".join(
        line for line in proc.stderr.splitlines() if "packed-fp32-ops" not in line
    ).strip()
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{err}")
    if err:
        print(err, file=sys.stderr)


def build(verbose: bool = False) -> str:
    """Compile every source and link the shared library; returns its path."""
    hipcc = _hipcc()
    incs = [f"-I{INCLUDE}", f"-I{CSRC}"]
    with tempfile.TemporaryDirectory(prefix="vlc_build_") as tmp:
        objs = []
        for src in HIP_SOURCES:
            obj = os.path.join(tmp, src + ".o")
            cmd = [hipcc, *HIP_FLAGS, *incs, "-c", os.path.join(CSRC, src), "-o", obj]
            if verbose:
                print(" ".join(cmd))
            _run(cmd)
            objs.append(obj)
        cxx = shutil.which("g++") or "g++"
        for src in HOST_SOURCES:
            obj = os.path.join(tmp, src + ".o")
            cmd = [cxx, *HOST_FLAGS, *incs, "-c", os.path.join(CSRC, src), "-o", obj]
            if verbose:
                print(" ".join(cmd))
            _run(cmd)
            objs.append(obj)
        tmp_lib = os.path.join(tmp, LIB_NAME)
        cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp_lib]
        if verbose:
            print(" ".join(cmd))
        _run(cmd)
        # Replace atomically so a process that already mapped the old file keeps it intact.
        staged = LIB_PATH + ".tmp"
        shutil.copyfile(tmp_lib, staged)
        os.replace(staged, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
