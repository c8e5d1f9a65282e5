"""The multi-workgroup fast kernel against the oracle and against the general
kernel, on the BASELINE.json configurations: both paths must meet the parity
bar, and the fast path must finish the rows of the benchmark configurations
itself (rows it defers are finished by the general kernel)."""

import pytest
import torch

from tests import parity as PY
from tests import workloads as W

pytestmark = pytest.mark.gpu


def _paths(w, dev, rows=None, lp=False):
    fast = PY.run_workload(w, dev, path="auto")
    gen = PY.run_workload(w, dev, path="generic")
    rf = PY.check_rows(w, fast, rows=rows, lp=lp)
    rg = PY.check_rows(w, gen, rows=rows, lp=lp)
    nfast = int((fast.row_path.cpu() == 0).sum())
    same = int((fast.tokens == gen.tokens).sum())
    print(f"{w.name}: fast-path rows {nfast}/{w.B}; tokens equal to the general kernel {same}/{w.B}; "
          f"fast {rf}; general {rg}", flush=True)
    return fast, gen, nfast


def test_paths_c2(dev):
    w = W.c2()
    fast, gen, nfast = _paths(w, dev)
    assert nfast == w.B


def test_paths_c1(dev):
    for g in (False, True):
        w = W.c1(greedy=g)
        fast, gen, nfast = _paths(w, dev)
        assert nfast == 1


@pytest.mark.parametrize("B", [16, 256])
@pytest.mark.parametrize("flat", [False, True])
def test_paths_c3(dev, flat, B):
    """c3 stays on the fast path (at B=256 the launch shape the benchmark
    times).  In its flat variant the cut and draw bins hold thousands of
    logits, which the row-group kernel's second histogram level resolves: at
    most 8 of 256 rows (3 %) may be left to the general kernel."""
    w = W.c3(B=B, flat=flat)
    fast, gen, nfast = _paths(w, dev)
    if not flat:
        assert nfast == w.B
    else:
        assert w.B - nfast <= max(1, (8 * w.B) // 256), f"{w.B - nfast} rows deferred"


def test_hardware_exp2_is_monotone(dev):
    """The row-group kernel finds a histogram region's logits by a search over
    x, which needs exp2(fma(x, c, -ref)) non-decreasing in x: the device's
    hardware exp2 must not decrease anywhere over the fp32 inputs."""
    import ctypes
    from lps import _lib
    v = ctypes.c_ulonglong(12345)
    assert _lib.load().lps_selftest_exp2_monotone(ctypes.byref(v)) == 0
    assert v.value == 0, f"{v.value} decreasing steps"


def test_paths_c5(dev):
    w = W.c5(B=32)
    fast, gen, nfast = _paths(w, dev, lp=True)
    assert nfast == w.B


def test_fast_small_and_ragged(dev):
    """Vocabularies below one chunk, exactly one chunk, ragged last chunk, scalar loads."""
    from tests.test_gpu_parity import _small
    for V in (5, 777, 8192, 8193, 20011):
        for dt in (torch.float32, torch.bfloat16):
            w = _small(V, 16, dt, seed=V)
            out = PY.run_workload(w, dev)
            PY.check_rows(w, out)
