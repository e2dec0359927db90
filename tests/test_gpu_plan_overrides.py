"""The library's plan overrides (environment variables read once per process: FMLP_BWD_UNIFIED,
FMLP_BWD_DZ, FMLP_BWD_NS / FMLP_BWD_ORDER, FMLP_BWD_ET / FMLP_BWD_DXES / FMLP_BWD_DXSPLIT,
FMLP_DXG_TP, FMLP_FWD_SPLIT / FMLP_FWD_T64 / FMLP_FWD_XS / FMLP_FWD_OCC, FMLP_DW256_NS) select
other kernel forms, splits and orders than the plan's estimate. Each override set runs a fixed
set of shapes (tests/override_child.py: D 32 to 256, fp16 / bf16 / fp32, ragged B, every
activation, the recompute form and the accuracy mode) in a child process of its own, one after
another, against the CPU oracle at the bars of tests/test_gpu_random_shapes.py. No counterpart
in the reference, which has no such switches.
"""
import os
import subprocess
import sys

import pytest

pytestmark = pytest.mark.gpu

CHILD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "override_child.py")
OVERRIDES = [
    {},
    {"FMLP_BWD_UNIFIED": "0"},
    {"FMLP_BWD_DZ": "1"},
    {"FMLP_BWD_DZ": "1", "FMLP_DXG_TP": "1"},
    {"FMLP_BWD_DZ": "0"},
    {"FMLP_BWD_NS": "4", "FMLP_BWD_ORDER": "2"},
    {"FMLP_BWD_ET": "128", "FMLP_BWD_DXES": "1", "FMLP_BWD_DXSPLIT": "0"},
    {"FMLP_FWD_SPLIT": "0", "FMLP_FWD_T64": "0", "FMLP_FWD_XS": "0", "FMLP_FWD_OCC": "2"},
    {"FMLP_FWD_SPLIT": "1"},
    {"FMLP_DW256_NS": "1"},
]


@pytest.mark.parametrize("override", OVERRIDES, ids=lambda o: ",".join(f"{k}={v}" for k, v in o.items()) or "none")
def test_override_keeps_parity(override):
    env = {k: v for k, v in os.environ.items() if not k.startswith("FMLP_")}
    env.update(override)
    print(f"[overrides] {override or 'none'}", flush=True)
    r = subprocess.run([sys.executable, "-u", CHILD], env=env, capture_output=True, text=True, timeout=180)
    print(r.stdout[-4000:], flush=True)
    assert r.returncode == 0, f"{override}: exit {r.returncode}\n{r.stdout[-3000:]}\n{r.stderr[-3000:]}"
