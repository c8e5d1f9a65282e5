"""Legality masks, the packed form of the reference's logit constraints
(constraints.py:53-80: ``LogitConstraint.apply_to_logits`` sets illegal ids to
-inf, then sampling proceeds on the masked logits).

Sampling with a mask must equal sampling on the logits with the illegal ids
written as -inf, bit for bit, on every path (fused kernel, split kernels,
general kernel), and the masked rows must meet the oracle."""

import copy

import pytest
import torch

from tests import parity as PY
from tests import workloads as W

pytestmark = pytest.mark.gpu

FIELDS = ("tokens", "status", "row_path", "kept_cut", "kept_ties", "kept_count", "chosen_logprob",
          "top_logprobs", "top_ids")


def _mask(B, V, seed, frac=0.7, few=5):
    g = torch.Generator().manual_seed(seed)
    m = torch.rand((B, V), generator=g) < frac
    m[0] = True                                                       # every id legal
    if B > 1:                                                         # a few legal ids
        m[1] = False
        m[1, torch.randperm(V, generator=g)[:few]] = True
    if B > 2:
        m[2] = torch.rand(V, generator=g) < 0.02                      # sparse
    if B > 3:
        m[3, :] = True                                                # the row's argmax illegal
    return m


def _masked(w, m):
    w2 = copy.copy(w)
    x = w.logits.clone()
    x[~m] = float("-inf")
    w2.logits = x
    return w2


def _same(a, b, what):
    for f in FIELDS:
        x, y = getattr(a, f, None), getattr(b, f, None)
        if x is None and y is None:
            continue
        x, y = x.cpu(), y.cpu()
        if x.is_floating_point():
            assert torch.equal(torch.nan_to_num(x, nan=7.0), torch.nan_to_num(y, nan=7.0)), f"{what}: {f} differs"
        else:
            assert torch.equal(x, y), f"{what}: {f} differs"


def _case(name):
    if name == "c2":
        return W.c2(B=16)
    if name == "c5":
        return W.c5(B=32)
    from tests.test_gpu_parity import _small
    V = {"small_vec": 1000, "small_scalar": 4099}[name]
    return _small(V, 24, torch.float32, seed=V + 3)


@pytest.mark.parametrize("path", ["auto", "generic"])
@pytest.mark.parametrize("name", ["c2", "c5", "small_vec", "small_scalar"])
def test_mask_equals_masked_logits(dev, name, path):
    w = _case(name)
    # (c5 returns the top-20 logprobs: keep at least 20 legal ids per row, so that
    # no -inf ties enter the top-20 list, whose order the oracle leaves open)
    m = _mask(w.B, w.V, seed=len(name) * 31 + w.V, few=25 if name == "c5" else 5)
    if name == "c2" or name == "c5":
        m[3, int(w.logits[3].float().argmax())] = False
    wm = _masked(w, m)
    a = PY.run_workload(w, dev, path=path, allowed=m.to(dev))
    b = PY.run_workload(wm, dev, path=path)
    _same(a, b, f"{name}/{path}")
    rep = PY.check_rows(wm, a, lp=w.logprobs)
    nfast = int((a.row_path.cpu() == 0).sum())
    print(f"{name}/{path}: {rep}; fast-path rows {nfast}/{w.B}", flush=True)
    legal = m.to(a.tokens.device)
    t = a.tokens
    ok = (t < 0) | legal.gather(1, t.clamp(min=0).view(-1, 1)).view(-1)
    assert bool(ok.all()), "an illegal id was sampled"


def test_mask_split_kernels(dev):
    """128 c2 rows with legality masks: more than one resident round of
    row-group workgroups on 256 CUs, so the top-k and greedy rows take the
    streaming kernel and the nucleus rows the row-group kernel at 104 logits
    per thread (three chunks per row)."""
    w = W.c2(B=128)
    m = _mask(w.B, w.V, seed=5)
    wm = _masked(w, m)
    a = PY.run_workload(w, dev, allowed=m.to(dev))
    b = PY.run_workload(wm, dev)
    _same(a, b, "c2 B=128 split")
    rep = PY.check_rows(wm, a)
    print(f"c2 B=128 masked: {rep}", flush=True)


def test_mask_packed_bits_and_query(dev):
    """Packed int32 bits (pack_allowed) and bool masks agree; the query
    probability of an illegal id is 0."""
    from lps import SamplingParams, pack_allowed, sample_rows
    w = W.c2(B=8)
    m = _mask(w.B, w.V, seed=9)
    p = SamplingParams(w.temperature.to(dev), w.top_k.to(dev), w.top_p.to(dev), w.min_p.to(dev),
                       w.typical_p.to(dev), w.rep.to(dev), w.pres.to(dev), w.freq.to(dev))
    x = w.logits.to(dev)
    q = torch.tensor([int((~m[i]).nonzero()[0]) if (~m[i]).any() else 0 for i in range(w.B)], dtype=torch.int64)
    kw = dict(histories=w.histories.to(dev), history_lengths=w.hist_len.to(dev), kept_set=True,
              query_tokens=q.to(dev))
    a = sample_rows(x, p, w.uniforms.to(dev), allowed=m.to(dev), **kw)
    b = sample_rows(x, p, w.uniforms.to(dev), allowed=pack_allowed(m.to(dev)), **kw)
    torch.cuda.synchronize(dev)
    _same(a, b, "bool vs packed")
    qp = a.query_prob.cpu()
    for i in range(w.B):
        if not bool(m[i].all()):
            assert float(qp[i]) == 0.0, f"row {i}: illegal query id has probability {float(qp[i])}"
