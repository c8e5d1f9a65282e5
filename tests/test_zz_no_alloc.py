"""lps_sample_noalloc (the entry point that allocates nothing, using the
library's static per-GPU workspace) against lps_sample with a caller
workspace: identical outputs on two calls in a row, the second on a smaller
batch, and both against the CPU oracle; batches beyond the static workspace
are refused with LPS_ENOALLOC_CAPACITY before anything is launched."""

import ctypes

import pytest
import torch

from tests import parity as PY
from tests import workloads as W

pytestmark = pytest.mark.gpu

FIELDS = ("tokens", "status", "row_path", "kept_cut", "kept_ties", "kept_count", "chosen_logprob", "top_logprobs",
          "top_ids")


def _same(a, b, what):
    for f in FIELDS:
        x, y = getattr(a, f, None), getattr(b, f, None)
        if x is None and y is None:
            continue
        assert x is not None and y is not None, f"{what}: {f} missing on one side"
        assert torch.equal(x.cpu(), y.cpu()), f"{what}: {f} differs between lps_sample_noalloc and lps_sample"


def _pair(w, dev):
    ref = PY.run_workload(w, dev)                 # lps_sample, caller workspace
    out = PY.run_workload(w, dev, noalloc=True)   # lps_sample_noalloc, static workspace
    return ref, out


def test_noalloc_equals_lps_sample_two_calls(dev):
    # first call: the c2 batch at full size (64 rows, V = 151936, bf16, mixed parameters)
    w1 = W.c2()
    print("noalloc call 1: c2 B=64 V=151936 bf16", flush=True)
    ref1, out1 = _pair(w1, dev)
    _same(out1, ref1, "call 1 (c2)")
    assert int((out1.row_path.cpu() == 0).sum()) == w1.B   # the multi-workgroup kernel used the static workspace
    PY.check_rows(w1, out1)
    # second call, smaller: fp32 nucleus rows of a shorter vocabulary and 8 rows
    w2 = W.c3(B=8, V=40000)
    print("noalloc call 2: c3-shaped B=8 V=40000 fp32", flush=True)
    ref2, out2 = _pair(w2, dev)
    _same(out2, ref2, "call 2 (c3, smaller)")
    PY.check_rows(w2, out2)
    # and the first shape again: nothing of the smaller call's state leaks into it
    out3 = PY.run_workload(w1, dev, noalloc=True)
    _same(out3, ref1, "call 3 (c2 again)")


def test_noalloc_logprobs_rows(dev):
    w = W.c5(B=16)
    print("noalloc logprobs: c5-shaped B=16 fp16", flush=True)
    ref, out = _pair(w, dev)
    _same(out, ref, "c5 logprobs")
    PY.check_rows(w, out, lp=True)


def test_noalloc_refuses_batches_beyond_its_workspace(dev):
    from lps import _lib
    from lps import SamplingParams, sample_rows
    lib = _lib.load()
    V = 151936
    R = 1
    while lib.lps_workspace_bytes(R, V, 0) <= _lib.LPS_NOALLOC_WORKSPACE_BYTES:
        R += 1
    print(f"noalloc capacity: {R - 1} rows at V={V}; refusing {R}", flush=True)
    x = torch.zeros((R, V), dtype=torch.bfloat16, device=dev)
    p = SamplingParams.build(R, dev, temperature=1.0)
    with pytest.raises(ValueError, match="lps_sample_noalloc"):
        sample_rows(x, p, torch.rand(R, device=dev), noalloc=True)
    # the direct C call returns the code and launches nothing
    a = _lib.SampleArgs()
    a.logits = x.data_ptr()
    a.dtype = _lib.LPS_DTYPE_BF16
    a.num_rows = R
    a.vocab = V
    a.rows_inner = 1
    a.stride_outer = V
    a.tokens = torch.empty(R, dtype=torch.int64, device=dev).data_ptr()
    a.uniforms = torch.rand(R, device=dev).data_ptr()
    assert lib.lps_sample_noalloc(ctypes.byref(a), None) == _lib.LPS_ENOALLOC_CAPACITY
