"""Build libflashmlp.so (the gfx950 HIP kernels and their C ABI) in-tree with hipcc.

    python -m flashmlp_amd.build          # writes flashmlp_amd/libflashmlp.so

The library is a plain shared object: host code calls it through include/flashmlp.h
(ctypes from Python). Cross-compiles on a machine without a GPU. The MFMA-ceiling
measurement kernel (fmlp_ceiling.hip, used by bench.py only) goes into its own
libfmlp_ceiling.so.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libflashmlp.so"
SOURCES = ["fmlp_fwd.hip", "fmlp_bwd.hip", "fmlp_gen.hip", "fmlp_scratch.hip", "fmlp_abi.cpp"]
CEILING_SRC = "fmlp_ceiling.hip"
CEILING_LIB = PKG / "libfmlp_ceiling.so"
ARCH = os.environ.get("FLASHMLP_ARCH", "gfx950")

# Packed fp32 VALU forms are disabled for every device pass.
DEVICE_FLAGS = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
COMMON = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}", "-fvisibility=hidden",
          f"-I{ROOT / 'include'}", f"-I{CSRC}", "-Wno-unused-command-line-argument"]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: set HIPCC or install ROCm")


def _compile(src: str, verbose: bool) -> Path:
    obj = BUILD / (src.rsplit(".", 1)[0] + ".o")
    cmd = [_hipcc(), *COMMON, *DEVICE_FLAGS, "-x", "hip", "-c", str(CSRC / src), "-o", str(obj)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    out = "\n".join(l for l in (res.stdout + res.stderr).splitlines()
                    if "packed-fp32-ops" not in l and l.strip())
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{out}")
    if verbose and out:
        print(out, flush=True)
    return obj


def _link(objs, lib: Path, verbose: bool) -> None:
    tmp = lib.with_suffix(".so.tmp")
    cmd = [_hipcc(), "-shared", "-fPIC", f"--offload-arch={ARCH}", *[str(o) for o in objs], "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}{res.stderr}")
    os.replace(tmp, lib)


def build(verbose: bool = False) -> Path:
    """Compile every source and link flashmlp_amd/libflashmlp.so (and the measurement-only
    libfmlp_ceiling.so). Always rebuilds."""
    BUILD.mkdir(exist_ok=True)
    srcs = SOURCES + [CEILING_SRC]
    with ThreadPoolExecutor(max_workers=len(srcs)) as ex:
        objs = list(ex.map(lambda s: _compile(s, verbose), srcs))
    _link(objs[:len(SOURCES)], LIB, verbose)
    _link(objs[len(SOURCES):], CEILING_LIB, verbose)
    return LIB


if __name__ == "__main__":
    p = build(verbose="-v" in sys.argv)
    print(p)
