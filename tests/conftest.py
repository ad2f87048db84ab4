import json
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "oracle"))
sys.path.insert(0, os.path.join(ROOT, "tests", "golden"))

import __graft_entry__  # noqa: E402

pkg = __graft_entry__.load_package()
from smol_genius_amd import synth  # noqa: E402,F401

GOLDEN = os.path.join(ROOT, "tests", "golden")

# Parity bar for the HIP path against the CPU oracle on fp32 outputs:
# every element satisfies |gpu - cpu| <= ATOL + RTOL * |cpu|.
ATOL = 2e-3
RTOL = 1e-2


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs on the GPU box)")


@pytest.fixture(scope="session")
def oracle():
    from oracle import Oracle
    o = Oracle()
    o.set_threads(min(os.cpu_count() or 1, 16))
    return o


@pytest.fixture(scope="session")
def golden():
    with open(os.path.join(GOLDEN, "ref_attention.json")) as f:
        meta = json.load(f)
    data = np.load(os.path.join(GOLDEN, "ref_attention.npz"))
    return meta, data


def parity_report(gpu, cpu):
    gpu = np.asarray(gpu, np.float64)
    cpu = np.asarray(cpu, np.float64)
    d = np.abs(gpu - cpu)
    ratio = float((d / (ATOL + RTOL * np.abs(cpu))).max()) if d.size else 0.0
    return dict(max_abs=float(d.max()) if d.size else 0.0, ratio=ratio,
                finite=bool(np.isfinite(gpu).all()))


def assert_parity(gpu, cpu, what=""):
    r = parity_report(gpu, cpu)
    print("parity %-40s max_abs %.3e ratio %.3f" % (what, r["max_abs"], r["ratio"]), flush=True)
    assert r["finite"], "%s: non-finite output" % what
    assert r["ratio"] <= 1.0, "%s: |gpu-cpu| exceeds %g + %g|cpu| (max_abs %.3e, ratio %.3f)" % (
        what, ATOL, RTOL, r["max_abs"], r["ratio"])
    return r
