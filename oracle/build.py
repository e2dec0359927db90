"""Build and load the fp64 C brute force (oracle/brute.c -> oracle/_build/libfmlp_brute.so).

Test infrastructure only. The reference (Python + Triton) has no C sources, so there is no
oracle/_ref build: the reference path is restated in reference.py instead.
"""
from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
SRC = HERE / "brute.c"
OUT = HERE / "_build" / "libfmlp_brute.so"


def build() -> Path:
    OUT.parent.mkdir(exist_ok=True)
    cmd = ["gcc", "-O2", "-fPIC", "-shared", "-fno-fast-math", str(SRC), "-o", str(OUT), "-lm"]
    subprocess.run(cmd, check=True)
    return OUT


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not OUT.exists() or OUT.stat().st_mtime < SRC.stat().st_mtime:
            build()
        L = ctypes.CDLL(str(OUT))
        dp = np.ctypeslib.ndpointer(dtype=np.float64, flags="C_CONTIGUOUS")
        i = ctypes.c_int
        L.brute_fwd.argtypes = [dp, dp, dp, dp, i, i, i, i, i]
        L.brute_fwd.restype = None
        L.brute_bwd.argtypes = [dp, dp, dp, dp, dp, dp, dp, i, i, i, i, i]
        L.brute_bwd.restype = None
        _lib = L
    return _lib


ACT = {"": 0, "silu": 1, "leaky_relu": 2, "sigmoid": 3}


def brute_fwd(x, w1, w2, activation=""):
    x, w1, w2 = (np.ascontiguousarray(np.asarray(t, dtype=np.float64)) for t in (x, w1, w2))
    H, B, D = x.shape
    E = w1.shape[2]
    o = np.empty((H, B, D))
    lib().brute_fwd(x, w1, w2, o, H, B, D, E, ACT.get(activation, 0))
    return o


def brute_bwd(x, w1, w2, do, activation=""):
    x, w1, w2, do = (np.ascontiguousarray(np.asarray(t, dtype=np.float64)) for t in (x, w1, w2, do))
    H, B, D = x.shape
    E = w1.shape[2]
    dx = np.empty((H, B, D))
    dw1 = np.empty((H, D, E))
    dw2 = np.empty((H, E, D))
    lib().brute_bwd(x, w1, w2, do, dx, dw1, dw2, H, B, D, E, ACT.get(activation, 0))
    return dx, dw1, dw2
