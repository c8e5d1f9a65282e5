"""Long token histories on every kernel, against the CPU oracle.

The reference penalises any ``generated_tokens`` list (``sampling.py:120-137``:
the ids are filtered to [0, V) and made unique with ``torch.unique``), so no
history may make a row fail.  Each history here holds 4096 ids: more than
2000 distinct in-range ids, one id repeated 300 times, repeats of the others
and a few ids outside [0, V).  The rows mix the repetition penalty with
presence / frequency penalties (whose frequency term counts every occurrence),
and greedy, top-k and nucleus rows.

* row-group kernel: B = 16 at V = 151936 (one resident round of 4-chunk rows);
* streaming kernel: B = 288 greedy / top-k rows (more than one resident round);
* general kernel: the same rows with LPS_FLAG_GENERIC.
Every row must finish on the kernel named, with status 0, and match the
oracle row by row."""

import numpy as np
import pytest
import torch

from lps import _lib
from tests import parity as PY
from tests import workloads as W
from tests.test_gpu_stream import _deferral_reasons

pytestmark = pytest.mark.gpu

H = 4096


def _history(rng, V, H=H, distinct=2400, hot_repeats=300):
    """H ids: `distinct` distinct in-range ids, one of them repeated
    `hot_repeats` times, Zipf-like repeats of the others, and 8 ids outside
    [0, V); shuffled."""
    ids = rng.choice(V, size=distinct, replace=False).astype(np.int64)
    hot = ids[0]
    rest = H - distinct - (hot_repeats - 1) - 8
    assert rest >= 0
    w = 1.0 / np.arange(1, distinct + 1) ** 1.1
    extra = rng.choice(ids, size=rest, p=w / w.sum())
    bad = np.array([-1, -7, V, V + 3, -100000, V + 100000, -2, V + 1])
    h = np.concatenate([ids, np.full(hot_repeats - 1, hot), extra, bad])
    rng.shuffle(h)
    return h.astype(np.int32)


def _workload(B, V, dtype, seed, kinds="mixed"):
    g = torch.Generator().manual_seed(seed)
    rng = np.random.default_rng(seed)
    x = (torch.randn((B, V), generator=g) * 2.5).to(dtype)
    hist = torch.from_numpy(np.stack([_history(rng, V) for _ in range(B)]))
    i = torch.arange(B)
    T = torch.where(i % 5 == 0, torch.tensor(0.0), 0.6 + 0.8 * torch.rand((B,), generator=g))
    k = torch.tensor([0, 20, 50, 100], dtype=torch.int32)[i % 4]
    if kinds == "topk":
        k = torch.where(k == 0, torch.tensor(40, dtype=torch.int32), k)
    p = torch.where(i % 3 == 0, torch.tensor(1.0), torch.tensor(0.9))
    # penalty mixes: repetition only; presence + frequency; all three
    rep = torch.tensor([1.2, 1.0, 1.1])[i % 3].float()
    pres = torch.tensor([0.0, 0.5, 0.4])[i % 3].float()
    freq = torch.tensor([0.0, 0.3, 0.05])[i % 3].float()
    f = lambda v: torch.full((B,), v, dtype=torch.float32)
    return W.Workload("long_history", x, T.float(), k, p.float(), f(0.0), f(1.0), rep, pres, freq, hist,
                      torch.full((B,), H, dtype=torch.int32), torch.rand((B,), generator=g))


# deferral reason codes that concern the history: the streaming kernel's list
# or counts (14), the row-group kernel's 16-bit counts (RF_HISTORY: 2 + (2 << 4))
HISTORY_REASONS = {14, 2 + (2 << 4)}


def _check(w, out, dev, expect_path, max_other=0):
    """Status 0 on every row; every row on the expected kernel, except at most
    `max_other` rows deferred for a reason other than the history (a wave's
    candidate segment or the pool past capacity on tie-heavy data); the oracle
    row by row."""
    st = out.status.cpu()
    assert not (st & _lib.LPS_ROW_HISTORY_OVERFLOW).any()
    assert (st == 0).all(), f"row status {st.tolist()}"
    path = out.row_path.cpu()
    off = (path != expect_path).nonzero().flatten().tolist()
    reasons = _deferral_reasons(out, dev, w.B) if expect_path == 0 else {}
    print(f"{w.name} B={w.B} V={w.V} {w.logits.dtype}: rows off the kernel {off}, reasons {reasons}", flush=True)
    assert not (set(reasons.values()) & HISTORY_REASONS), f"history deferrals {reasons}"
    assert len(off) <= max_other, f"rows off the expected kernel: {off} ({reasons})"
    rep = PY.check_rows(w, out)
    print(f"{w.name} B={w.B} V={w.V} {w.logits.dtype}: {rep}", flush=True)


def test_history_shape():
    """The histories hold what the test promises (checked on the CPU side of a GPU test module)."""
    rng = np.random.default_rng(0)
    V = 151936
    h = _history(rng, V)
    inr = h[(h >= 0) & (h < V)]
    vals, cnt = np.unique(inr, return_counts=True)
    assert h.size == 4096 and vals.size >= 2000 and cnt.max() >= 300 and (h < 0).any() and (h >= V).any()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_long_history_rowgroup(dev, dtype):
    """B = 16 rows of V = 151936 (four chunks per row) on the row-group kernel."""
    w = _workload(16, W.V_QWEN3, dtype, seed=101)
    out = PY.run_workload(w, dev, row_kind_hint=0)
    _check(w, out, dev, 0)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_long_history_streaming(dev, dtype):
    """B = 288 greedy and top-k rows of V = 32768: more than one resident round,
    so the streaming kernel takes every row (the row-kind hint launches it alone)."""
    w = _workload(288, 32768, dtype, seed=202, kinds="topk")
    out = PY.run_workload(w, dev, row_kind_hint=_lib.LPS_FLAG_ROWS_TOPK)
    _check(w, out, dev, 0, max_other=3)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_long_history_general(dev, dtype):
    """The same rows on the general kernel (LPS_FLAG_GENERIC)."""
    w = _workload(16, W.V_QWEN3, dtype, seed=101)
    out = PY.run_workload(w, dev, path="generic")
    _check(w, out, dev, 1)


def test_streaming_more_distinct_ids_than_its_list(dev):
    """A history with more distinct ids than the streaming kernel's list (4096)
    sends the row to the general kernel, which counts any history: the row is
    sampled, exactly."""
    B, V = 272, 16384
    w = _workload(B, V, torch.bfloat16, seed=303, kinds="topk")
    rng = np.random.default_rng(7)
    wide = np.stack([np.concatenate([rng.permutation(V)[:5000], rng.integers(0, V, size=1000)]).astype(np.int32)
                     for _ in range(2)])
    hist = torch.zeros((B, 6000), dtype=torch.int32)
    hist[:, :H] = w.histories
    hist[:2] = torch.from_numpy(wide)
    w.histories = hist
    w.hist_len = torch.full((B,), H, dtype=torch.int32)
    w.hist_len[:2] = 6000
    out = PY.run_workload(w, dev, row_kind_hint=_lib.LPS_FLAG_ROWS_TOPK)
    path = out.row_path.cpu()
    reasons = _deferral_reasons(out, dev, B)
    print(f"wide histories: reasons {reasons}", flush=True)
    assert reasons.get(0) == 14 and reasons.get(1) == 14
    assert int(path[2:].sum()) <= 3
    assert (out.status.cpu() == 0).all()
    PY.check_rows(w, out, rows=list(range(8)))
