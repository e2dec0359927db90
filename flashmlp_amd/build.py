"""Build libflashmlp.so (the gfx950 HIP kernels and their C ABI) in-tree with hipcc.

    python -m flashmlp_amd.build          # writes flashmlp_amd/libflashmlp.so

The library is a plain shared object: host code calls it through include/flashmlp.h
(ctypes from Python). Cross-compiles on a machine without a GPU. The MFMA-ceiling
measurement kernel (fmlp_ceiling.hip, used by bench.py only) goes into its own
libfmlp_ceiling.so. _fmlp_fast.so (fmlp_py.cpp, host C++ built with the system compiler
against torch's headers and libflashmlp.so) is the Python wrappers' per-call fast path over
the same C ABI.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
import sysconfig
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
FAST_SRC = "fmlp_py.cpp"
FAST_LIB = PKG / "_fmlp_fast.so"
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


def _run(cmd, what: str, verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"{what} failed:\n{res.stdout}{res.stderr}")


def _fast_flags():
    import torch
    import torch.utils.cpp_extension as ce

    rocm_inc = Path(_hipcc()).resolve().parent.parent / "include"
    inc = [*ce.include_paths(), str(rocm_inc), sysconfig.get_paths()["include"], str(ROOT / "include")]
    defs = [f"-D_GLIBCXX_USE_CXX11_ABI={int(torch.compiled_with_cxx11_abi())}", "-D__HIP_PLATFORM_AMD__"]
    return [*defs, *[f"-I{p}" for p in inc]], ce.library_paths()


def _compile_fast(verbose: bool) -> Path:
    obj = BUILD / "fmlp_py.o"
    cflags, _ = _fast_flags()
    cxx = os.environ.get("CXX", "g++")
    _run([cxx, "-O2", "-std=c++17", "-fPIC", "-fvisibility=hidden", *cflags, "-c", str(CSRC / FAST_SRC), "-o",
          str(obj)], "compiling fmlp_py.cpp", verbose)
    return obj


def _link_fast(obj: Path, verbose: bool) -> None:
    _, libdirs = _fast_flags()
    cxx = os.environ.get("CXX", "g++")
    tmp = FAST_LIB.with_suffix(".so.tmp")
    _run([cxx, "-shared", "-fPIC", str(obj), "-o", str(tmp), f"-L{PKG}", "-lflashmlp", *[f"-L{p}" for p in libdirs],
          "-lc10", "-lc10_hip", "-ltorch_cpu", "-ltorch_python", "-Wl,-rpath,$ORIGIN",
          *[f"-Wl,-rpath,{p}" for p in libdirs]], "linking _fmlp_fast.so", verbose)
    os.replace(tmp, FAST_LIB)


def build(verbose: bool = False) -> Path:
    """Compile every source and link flashmlp_amd/libflashmlp.so (and the measurement-only
    libfmlp_ceiling.so, and the wrappers' fast path _fmlp_fast.so). Always rebuilds."""
    BUILD.mkdir(exist_ok=True)
    srcs = SOURCES + [CEILING_SRC]
    with ThreadPoolExecutor(max_workers=len(srcs) + 1) as ex:
        fast = ex.submit(_compile_fast, verbose)
        objs = list(ex.map(lambda s: _compile(s, verbose), srcs))
        fast_obj = fast.result()
    _link(objs[:len(SOURCES)], LIB, verbose)
    _link(objs[len(SOURCES):], CEILING_LIB, verbose)
    _link_fast(fast_obj, verbose)
    return LIB


if __name__ == "__main__":
    p = build(verbose="-v" in sys.argv)
    print(p)
