"""The C ABI library (libflashmlp.so) loads, exports every symbol include/flashmlp.h declares,
and rejects out-of-contract arguments on the host, before any GPU work (runs without a GPU).
"""
import ctypes
import re
import subprocess
from pathlib import Path

import pytest

from flashmlp_amd import _lib

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "flashmlp.h"

OK, INVALID, UNSUPPORTED, HIPERR, WORKSPACE = 0, 1, 2, 3, 4


def declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(fmlp_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def L():
    if not _lib.LIB_PATH.exists():
        pytest.skip("libflashmlp.so not built (python -m flashmlp_amd.build)")
    return _lib.lib()


def test_header_declares_expected_entry_points():
    names = declared_functions()
    assert names == sorted(_lib.SIGNATURES), names


def test_library_exports_every_declared_symbol(L):
    out = subprocess.run(["nm", "-D", "--defined-only", str(_lib.LIB_PATH)], capture_output=True, text=True,
                         check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if line.strip()}
    for name in declared_functions():
        assert name in exported, name
        assert getattr(L, name) is not None


def test_version_and_status_strings(L):
    assert L.fmlp_abi_version() == 4
    assert L.fmlp_status_string(OK) == b"ok"
    for st in (INVALID, UNSUPPORTED, HIPERR, WORKSPACE):
        assert L.fmlp_status_string(st) not in (b"ok", b"unknown status")
    assert L.fmlp_status_string(99) == b"unknown status"


def test_activation_names_mirror_reference(L):
    # flashmlp.py:140-147: unknown strings fall through to linear
    assert L.fmlp_act_from_name(b"silu") == 1
    assert L.fmlp_act_from_name(b"leaky_relu") == 2
    assert L.fmlp_act_from_name(b"sigmoid") == 3
    assert L.fmlp_act_from_name(b"") == 0
    assert L.fmlp_act_from_name(b"gelu") == 0
    assert L.fmlp_act_from_name(None) == 0


def test_shape_support(L):
    assert L.fmlp_shape_supported(32, 16384, 128, 1024, 1) == 1
    assert L.fmlp_shape_supported(8, 4097, 64, 2048, 0) == 1
    assert L.fmlp_shape_supported(1, 1, 64, 8, 1) == 1
    assert L.fmlp_shape_supported(2, 8, 96, 64, 1) == 0   # D not a power of two
    assert L.fmlp_shape_supported(2, 8, 512, 64, 1) == 0  # D above 256
    for D in (16, 32, 256):                                # the generic kernels' D
        assert L.fmlp_shape_supported(2, 8, D, 64, 1) == 1
    assert L.fmlp_shape_supported(2, 8, 64, 12, 1) == 1   # any E (generic kernels when E % 8 != 0)
    assert L.fmlp_shape_supported(2, 8, 64, 0, 1) == 0    # E = 0
    assert L.fmlp_shape_supported(2, 8, 64, 64, 2) == 1   # fp32 io
    assert L.fmlp_shape_supported(2, 8, 64, 64, 3) == 0   # no such dtype
    # the fp32-output flag is accepted on every io dtype and nothing else
    assert L.fmlp_shape_supported(2, 8, 64, 64, 1 | _lib.FMLP_OUT_F32) == 1
    assert L.fmlp_shape_supported(2, 8, 64, 64, 0 | _lib.FMLP_OUT_F32) == 1
    assert L.fmlp_shape_supported(2, 8, 64, 64, 2 | _lib.FMLP_OUT_F32) == 1
    assert L.fmlp_shape_supported(2, 8, 64, 64, 3 | _lib.FMLP_OUT_F32) == 0
    # so is the backward's hi/lo dW flag, alone or with the fp32-output flag; unknown bits are not
    assert L.fmlp_shape_supported(2, 8, 64, 64, 1 | _lib.FMLP_DW_HILO) == 1
    assert L.fmlp_shape_supported(2, 8, 64, 64, 0 | _lib.FMLP_DW_HILO | _lib.FMLP_OUT_F32) == 1
    assert L.fmlp_shape_supported(2, 8, 64, 64, 1 | _lib.FMLP_BWD_RECOMPUTE) == 1
    assert L.fmlp_shape_supported(2, 8, 64, 64, 1 | _lib.FMLP_BWD_STORE_DZ) == 1
    assert L.fmlp_shape_supported(2, 8, 64, 64, 1 | _lib.FMLP_BWD_STORE_DZ | _lib.FMLP_BWD_RECOMPUTE) == 0
    assert L.fmlp_shape_supported(2, 8, 64, 64, 1 | _lib.FMLP_BWD_NO_DX | _lib.FMLP_BWD_NO_DW) == 1
    assert L.fmlp_shape_supported(2, 8, 64, 64, 1 | 0x4000) == 0  # an unknown flag bit
    assert L.fmlp_shape_supported(-1, 8, 64, 64, 1) == 0


def test_shape_tuned(L):
    # the tuned gfx950 kernels: 16-bit io, D in {64, 128}, E % 8 == 0
    assert L.fmlp_shape_tuned(128, 1024, 1) == 1 and L.fmlp_shape_tuned(64, 2048, 0) == 1
    assert L.fmlp_shape_tuned(128, 1024, 1 | _lib.FMLP_OUT_F32 | _lib.FMLP_DW_HILO) == 1
    assert L.fmlp_shape_tuned(32, 1024, 1) == 0 and L.fmlp_shape_tuned(256, 1024, 1) == 0
    assert L.fmlp_shape_tuned(128, 1020, 1) == 0 and L.fmlp_shape_tuned(128, 1024, 2) == 0


# Every call below carries fake device addresses: each must be rejected (or be a no-op)
# before any kernel launch, so the file is safe to run on a machine with a GPU.
def _fwd(L, x=0x1000, w1=0x1000, w2=0x1000, o=0x1000, H=2, B=8, D=64, E=64, dtype=1, act=1):
    return L.fmlp_fwd(x, w1, w2, o, H, B, D, E, dtype, act, None)


def test_forward_argument_validation(L):
    assert _fwd(L, dtype=1 | _lib.FMLP_DW_HILO) == INVALID  # a backward-only flag
    assert _fwd(L, dtype=1 | _lib.FMLP_BWD_RECOMPUTE) == INVALID  # a backward-only flag
    assert _fwd(L, dtype=1 | _lib.FMLP_BWD_STORE_DZ) == INVALID  # a backward-only flag
    assert _fwd(L, D=96) == UNSUPPORTED
    assert b"D=96" in L.fmlp_last_error()
    assert _fwd(L, E=0) == UNSUPPORTED
    assert _fwd(L, dtype=5) == UNSUPPORTED
    assert _fwd(L, act=7) == INVALID
    assert _fwd(L, H=-2) == INVALID
    assert _fwd(L, x=None) == INVALID
    assert b"x is NULL" in L.fmlp_last_error()
    assert _fwd(L, w2=0x1001) == INVALID  # not aligned to its 2-byte elements
    assert b"aligned" in L.fmlp_last_error()
    assert _fwd(L, dtype=2, w1=0x1002) == INVALID  # fp32 elements need 4-byte alignment
    # strided entry point: NULL or negative strides are rejected
    s3 = (ctypes.c_int64 * 3)(512, 64, 1)
    neg = (ctypes.c_int64 * 3)(512, -64, 1)
    assert L.fmlp_fwd_strided(0x1000, 0x1000, 0x1000, 0x1000, 2, 8, 64, 64, None, s3, s3, 1, 1, None) == INVALID
    assert L.fmlp_fwd_strided(0x1000, 0x1000, 0x1000, 0x1000, 2, 8, 64, 64, neg, s3, s3, 1, 1, None) == INVALID
    assert b"negative" in L.fmlp_last_error()
    assert L.fmlp_fwd_strided(0x1000, 0x1000, 0x1000, 0x1000, 2, 8, 96, 64, s3, s3, s3, 1, 1, None) == UNSUPPORTED
    # nothing to do: no pointers needed, no GPU touched
    assert _fwd(L, x=None, o=None, B=0) == OK
    assert L.fmlp_last_error() == b""


def test_backward_argument_validation(L):
    p = 0x2000

    def bwd(**kw):
        a = dict(x=p, w1=p, w2=p, do=p, dx=p, dw1=p, dw2=p, H=2, B=8, D=128, E=64, dtype=1, act=2, ws=None, nws=0)
        a.update(kw)
        return L.fmlp_bwd(a["x"], a["w1"], a["w2"], a["do"], a["dx"], a["dw1"], a["dw2"], a["H"], a["B"], a["D"],
                          a["E"], a["dtype"], a["act"], a["ws"], a["nws"], None)

    assert bwd(D=96) == UNSUPPORTED
    assert bwd(dw1=None) == INVALID
    assert b"dw1" in L.fmlp_last_error()
    assert bwd(do=0x2003) == INVALID
    # fp32 outputs (FMLP_OUT_F32) need 4-byte aligned output pointers
    assert bwd(dx=0x2002, dtype=1 | _lib.FMLP_OUT_F32) == INVALID
    # the tuned path's workspace rule: a split shape with no workspace is rejected (without a
    # GPU the CU-count query fails first)
    assert bwd(H=2, B=8192, D=128, E=128) in (WORKSPACE, HIPERR)
    assert bwd(act=-1) == INVALID
    assert bwd(H=0, x=None, do=None, dx=None) == OK
    # FMLP_BWD_NO_DX / FMLP_BWD_NO_DW: the unwanted outputs may be NULL (the argument checks pass;
    # without a GPU the CU-count query fails next), the wanted ones may not; both: nothing to do
    assert bwd(dx=None, dtype=1 | _lib.FMLP_BWD_NO_DX) in (OK, HIPERR)
    assert bwd(dw1=None, dw2=None, dtype=1 | _lib.FMLP_BWD_NO_DW) in (OK, HIPERR)
    assert bwd(dx=None, dtype=1 | _lib.FMLP_BWD_NO_DW) == INVALID
    assert bwd(dx=None, dw1=None, dw2=None, dtype=1 | _lib.FMLP_BWD_NO_DX | _lib.FMLP_BWD_NO_DW) == OK
    assert _fwd(L, dtype=1 | _lib.FMLP_BWD_NO_DX) == INVALID  # a backward-only flag


def test_workspace_query_is_zero_for_invalid_shapes(L):
    assert L.fmlp_bwd_workspace_bytes(2, 8, 96, 64, 1) == 0
    # the backward-form query answers 0 for rejected arguments (and for the generic kernels)
    assert L.fmlp_bwd_stores_dz(2, 8, 96, 64, 1, 1) == 0
    assert L.fmlp_bwd_stores_dz(2, 8, 64, 64, 1, -1) == 0
    assert L.fmlp_bwd_stores_dz(2, 8, 64, 64, 1 | _lib.FMLP_BWD_RECOMPUTE | _lib.FMLP_BWD_STORE_DZ, 1) == 0
    assert L.fmlp_bwd_stores_dz(2, 8, 64, 64, _lib.FMLP_DTYPE_F32, 1) == 0


def test_last_error_is_thread_local(L):
    import threading

    assert _fwd(L, D=96) == UNSUPPORTED
    seen = []
    t = threading.Thread(target=lambda: seen.append(L.fmlp_last_error()))
    t.start()
    t.join()
    assert seen == [b""]
    assert b"D=96" in L.fmlp_last_error()


def test_ceiling_library_exports_its_entry_point():
    """The measurement-only MFMA-ceiling library (bench.py --workload mfma_ceiling) is built
    beside libflashmlp.so and exports its one launcher."""
    lib = ROOT / "flashmlp_amd" / "libfmlp_ceiling.so"
    if not lib.exists():
        pytest.skip("libfmlp_ceiling.so not built (python -m flashmlp_amd.build)")
    out = subprocess.run(["nm", "-D", "--defined-only", str(lib)], capture_output=True, text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if line.strip()}
    assert "fmlp_ceiling_mfma" in exported and "fmlp_ceiling_mix" in exported
    assert "fmlp_ceiling_act_mix" in exported
    ctypes.CDLL(str(lib))  # loads without a GPU
