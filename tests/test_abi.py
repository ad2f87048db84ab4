"""The C-ABI library loads and exports every entry point declared in include/*.h.

No computation runs here (this suite also runs where there is no GPU); the
host-only table builder is checked against the oracle, and without a GPU the
library reports SMOL_ATTN_ERR_NO_GPU instead of computing anything on the CPU.
"""
import ctypes
import os
import re
import subprocess

import numpy as np
import pytest

from conftest import ROOT, pkg  # noqa: F401

INCLUDE = os.path.join(ROOT, "include")
DECL = re.compile(r"SMOL_(?:ATTN|KERNELS)_API\s+[\w\s\*]*?\b(\w+)\s*\(", re.S)


def declared():
    names = []
    for f in sorted(os.listdir(INCLUDE)):
        if f.endswith(".h"):
            with open(os.path.join(INCLUDE, f)) as fh:
                text = "\n".join(l for l in fh.read().splitlines() if not l.lstrip().startswith("#"))
                names += DECL.findall(text)
    return names


def test_library_exports_every_declared_symbol():
    from smol_genius_amd import smol_attn as sa
    lib = sa.load()
    names = declared()
    assert len(names) >= 30
    out = subprocess.run(["nm", "-D", "--defined-only", sa.LIB_PATH], capture_output=True, text=True).stdout
    exported = {l.split()[-1] for l in out.splitlines() if " T " in l}
    missing = [n for n in names if n not in exported]
    assert not missing, missing
    for n in names:
        assert getattr(lib, n) is not None
    # the Python mirror binds exactly the declared set
    assert sorted(n for n, _, _ in sa.SIGNATURES) == sorted(names)
    # nothing else leaks out of the library with default visibility
    extra = sorted(e for e in exported if e.startswith("smol_") and e not in names)
    assert not extra, extra


def test_version_string():
    from smol_genius_amd import smol_attn as sa
    assert b"gfx950" in sa.load().smol_attn_version()


def test_host_rope_table_matches_oracle(oracle):
    from smol_genius_amd import smol_attn as sa
    for hd, theta, rt in [(128, 1e6, 0), (256, 1e4, 1), (72, 1e4, 0), (64, 1e6, 1)]:
        c, s = sa.rope_fill_host(0, 8300, hd, theta, rt)
        oc, os_ = oracle.fill_rope_table(0, 8300, hd, theta, rt == 1)
        np.testing.assert_array_equal(c, oc)
        np.testing.assert_array_equal(s, os_)
        c2, s2 = sa.rope_fill_host(4000, 5, hd, theta, rt)
        np.testing.assert_array_equal(c2, oc[4000:4005])


def test_no_gpu_means_no_compute():
    torch = pytest.importorskip("torch")
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    from smol_genius_amd import smol_attn as sa
    lib = sa.load()
    assert lib.smol_attn_device_count() == -5
    h = ctypes.c_void_p()
    assert lib.smol_attn_ctx_create(0, None, ctypes.byref(h)) == -5
    assert b"no HIP device" in lib.smol_attn_last_error()
    with pytest.raises(sa.SmolAttnError):
        sa.Context(0, stream=0)
