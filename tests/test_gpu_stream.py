"""The streaming kernel (one workgroup per greedy / top-k row, for batches whose
row-group grid exceeds one resident round) against the CPU oracle, through the
C ABI; and the row-kind hints, which choose the launched kernels but never the
result (a row that breaks a hint is sampled by the general kernel)."""

import numpy as np
import pytest
import torch

from lps import _lib, row_kind_flags
from tests import parity as PY
from tests import workloads as W

pytestmark = pytest.mark.gpu

TOPK = _lib.LPS_FLAG_ROWS_TOPK
NUC = _lib.LPS_FLAG_ROWS_NUCLEUS


def _print(msg):
    print(msg, flush=True)


def _deferral_reasons(out, dev, B):
    """Reason codes of the rows the fast kernels deferred (the workspace's
    status words, LPS_ROW_DEFERRED | reason << 8), by row."""
    from lps import batch
    ws = batch._WS[(dev.index, torch.cuda.current_stream(dev).cuda_stream)]
    st = ws[131072:131072 + 4 * B].view(torch.int32).cpu()
    rows = (out.row_path.cpu() != 0).nonzero().flatten().tolist()
    return {r: int(st[r]) >> 8 for r in rows}


def _big(B, V, dtype, seed, kinds="mixed", H=48, logprobs=False, n_top=0):
    """B rows over a small vocabulary (one chunk per row, so B > 256 makes the
    grid larger than one resident round): ties, penalties with out-of-range
    and repeated history ids, and, by kinds, greedy / top-k / nucleus rows."""
    g = torch.Generator().manual_seed(seed)
    rng = np.random.default_rng(seed)
    x = torch.randn((B, V), generator=g) * 2.5
    x[::7] = torch.round(x[::7] * 2)                                    # ties
    x = x.to(dtype)
    T = torch.from_numpy(rng.choice([0.0, 0.6, 1.0, 1.4], size=B).astype(np.float32))
    k = torch.from_numpy(rng.choice([1, 20, 40, 63, 64, 65, 100, 128], size=B).astype(np.int32))
    if kinds == "mixed":
        k = torch.where(torch.arange(B) % 5 == 0, torch.zeros_like(k), k)
        T = torch.where(torch.arange(B) % 10 == 0, torch.ones_like(T), T)
    elif kinds == "nucleus":
        k = torch.zeros_like(k)
        T = torch.where(T > 0, T, torch.ones_like(T))
    p = torch.from_numpy(rng.choice([1.0, 0.9, 0.5], size=B).astype(np.float32))
    f = lambda v: torch.full((B,), v, dtype=torch.float32)
    hist = torch.from_numpy(rng.integers(-3, V + 3, size=(B, H)).astype(np.int32))
    hist[:, : H // 4] = hist[:, H // 4: H // 2]                          # repeated ids (frequency counts)
    hl = torch.from_numpy(rng.integers(0, H + 1, size=B).astype(np.int32))
    return W.Workload("big", x, T, k, p, f(0.0), f(1.0), f(1.2), f(0.4), f(0.25), hist, hl,
                      torch.rand((B,), generator=g), logprobs=logprobs, n_top=n_top)


def test_c5_full_size_every_row(dev):
    """c5 at its own size (B=512 fp16, greedy and top-k 40 / top-p 0.92 rows,
    repetition penalty over 1024 ids, chosen and top-20 logprobs) with the hint
    Sampler.sample_token passes: the streaming kernel alone; every row against
    the oracle, logprobs included."""
    w = W.c5()
    assert row_kind_flags(w.temperature, w.top_k) == TOPK
    out = PY.run_workload(w, dev)
    assert (out.row_path.cpu() == 0).all()
    rep = PY.check_rows(w, out, lp=True)
    _print(f"c5 B=512 streaming kernel: {rep}")


@pytest.mark.parametrize("hint", [0, TOPK, NUC])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32, torch.float16])
def test_large_mixed_batch_any_hint(dev, dtype, hint):
    """A mixed batch larger than one resident round: greedy and top-k rows on
    the streaming kernel, nucleus / pure rows on the row-group kernel (hint 0);
    a hint that misjudges rows changes only the path (general kernel), never
    the result."""
    B, V = 320, 4096
    w = _big(B, V, dtype, seed=17 + int(dtype == torch.float32))
    out = PY.run_workload(w, dev, row_kind_hint=hint)
    PY.check_rows(w, out)
    path = out.row_path.cpu()
    topk_rows = ~(w.temperature > 0) | (w.top_k > 0)
    plain = torch.arange(B) % 7 != 0      # tie-heavy rows may overflow a wave's segment and defer
    _print(f"{dtype} hint {hint}: deferred rows and reasons {_deferral_reasons(out, dev, B)}")
    if hint == 0:
        assert (path[plain] == 0).all()
    elif hint == TOPK:
        assert (path[topk_rows & plain] == 0).all() and (path[~topk_rows] == 1).all()
    _print(f"{dtype} hint {hint}: general-kernel rows {int(path.sum())}/{B}")


@pytest.mark.parametrize("B", [263, 301])
def test_large_mixed_batch_ragged_group(dev, B):
    """A mixed batch past one resident round whose size is not a multiple of 8:
    the streaming kernel places groups of 8 rows skewed over the XCDs and the
    last, partial group as is; every row against the oracle, every plain row
    on a fast kernel."""
    V = 4096
    w = _big(B, V, torch.bfloat16, seed=B)
    out = PY.run_workload(w, dev)
    rep = PY.check_rows(w, out)
    path = out.row_path.cpu()
    plain = torch.arange(B) % 7 != 0      # tie-heavy rows may overflow a wave's segment and defer
    _print(f"B={B}: {rep}; general-kernel rows {int(path.sum())}/{B}")
    assert (path[plain] == 0).all()


def test_mixed_batch_on_both_kernels(dev):
    """c2's mixed rows at B=700 (V=151936 bf16): past 8 resident rounds of
    row-group workgroups, so the greedy and top-k rows stream and the nucleus
    rows take the row-group kernel (which skips the streamed rows); every row
    on a fast kernel, every seventh row against the oracle."""
    w = W.c2(B=700)
    out = PY.run_workload(w, dev)
    rows = list(range(0, w.B, 7))
    rep = PY.check_rows(w, out, rows=rows)
    path = out.row_path.cpu()
    _print(f"c2 B=700: {rep}; general-kernel rows {int(path.sum())}/{w.B}")
    assert int((path == 1).sum()) <= 3, path.nonzero().flatten().tolist()


@pytest.mark.parametrize("kinds", ["mixed", "nucleus"])
def test_batch_past_the_launch_row_limit(dev, kinds):
    """1100 rows: more than one row-group launch takes (1024 rows), so the
    batch runs as blocks of rows, each its own launch over the same workspace
    (row counters and epochs carried from block to block); every row against
    the oracle, every plain row on a fast kernel."""
    B, V = 1100, 4096
    w = _big(B, V, torch.bfloat16, seed=1100 + len(kinds), kinds=kinds)
    out = PY.run_workload(w, dev)
    rep = PY.check_rows(w, out)
    path = out.row_path.cpu()
    plain = torch.arange(B) % 7 != 0      # tie-heavy rows may overflow a wave's segment and defer
    _print(f"B={B} {kinds}: {rep}; general-kernel rows {int(path.sum())}/{B}")
    assert (path[plain] == 0).all()


@pytest.mark.parametrize("hint", [0, _lib.LPS_FLAG_ROWS_BASIC_FILTERS])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_large_batch_every_filter(dev, dtype, hint):
    """A batch larger than one resident round whose rows use every filter:
    greedy and top-k rows (the streaming kernel), top-p, min-p without top-k
    (alone and after top-p), typical-p alone and after top-p, and top_k past
    the lists (the row-group kernel's extra-features build), in one launch.
    Without a hint every row finishes on a fast kernel (tie-heavy rows aside);
    with a wrong LPS_FLAG_ROWS_BASIC_FILTERS hint the min-p / typical-p /
    large-top-k rows take the general kernel.  Every row matches the oracle."""
    B, V = 320, 4096
    w = _big(B, V, dtype, seed=29 + int(dtype == torch.float16))
    i = torch.arange(B)
    kind = i % 8
    T = torch.where(kind == 0, torch.tensor(0.0), torch.tensor(0.8))
    k = torch.tensor([0, 40, 0, 0, 0, 0, 0, 600], dtype=torch.int32)[kind]
    p = torch.tensor([1.0, 0.9, 0.9, 1.0, 0.8, 1.0, 0.9, 1.0])[kind]
    mp = torch.tensor([0.0, 0.0, 0.0, 0.05, 0.1, 0.0, 0.0, 0.0])[kind]
    tp = torch.tensor([1.0, 1.0, 1.0, 1.0, 1.0, 0.5, 0.7, 1.0])[kind]
    w.temperature, w.top_k, w.top_p, w.min_p, w.typical_p = T, k, p, mp, tp
    out = PY.run_workload(w, dev, row_kind_hint=hint)
    PY.check_rows(w, out)
    path = out.row_path.cpu()
    plain = i % 7 != 0      # tie-heavy rows may overflow a wave's segment and defer
    extra = (kind >= 3)
    reasons = _deferral_reasons(out, dev, B)
    _print(f"{dtype} hint {hint}: {len(reasons)} deferred rows, reasons {sorted(set(reasons.values()))}")
    if hint == 0:
        assert (path[plain] == 0).all()
    else:
        assert (path[extra] == 1).all() and (path[plain & ~extra] == 0).all()


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_large_topk_batch_logprobs(dev, dtype):
    """Greedy and top-k rows only (k up to the streaming kernel's 128, and past
    it), with chosen and top-N logprobs, penalties and ties."""
    B, V = 300, 6000
    w = _big(B, V, dtype, seed=23, kinds="topk", logprobs=True, n_top=20)
    w.top_k[5] = 129          # past the streaming kernel's k': the row-group kernel's row
    w.temperature[5] = 0.8
    out = PY.run_workload(w, dev)
    rep = PY.check_rows(w, out, lp=True)
    plain = torch.arange(B) % 7 != 0      # tie-heavy rows may overflow a wave's segment and defer
    _print(f"{dtype}: deferred rows and reasons {_deferral_reasons(out, dev, B)}")
    # row 5 (k' = 129) is the row-group kernel's, which the batch's row-kind
    # hint (every row greedy or top-k) does not launch: the general kernel's
    assert int(out.row_path[5]) == 1
    plain[5] = False
    assert (out.row_path.cpu()[plain] == 0).all()
    _print(f"{dtype} top-k batch: {rep}; general-kernel rows {int(out.row_path.sum())}/{B}")


def test_large_batch_legality_mask(dev):
    """Legality bits on the streaming kernel equal -inf logits, bit for bit,
    and both match the oracle."""
    B, V = 288, 8192
    w = _big(B, V, torch.bfloat16, seed=31, kinds="topk", logprobs=True, n_top=8)
    g = torch.Generator().manual_seed(2)
    legal = torch.rand((B, V), generator=g) < 0.7
    legal[:, 0] = True
    a = PY.run_workload(w, dev, allowed=legal.to(dev))
    wm = W.Workload(**{**w.__dict__, "logits": w.logits.masked_fill(~legal, float("-inf"))})
    b = PY.run_workload(wm, dev)
    assert torch.equal(a.tokens, b.tokens)
    assert torch.equal(a.kept_count, b.kept_count)
    assert torch.equal(a.chosen_logprob, b.chosen_logprob)
    PY.check_rows(wm, a, lp=True)


def test_large_batch_nonfinite_rows(dev):
    """NaN / +inf / all -inf rows on the streaming kernel: sampling rows report
    the reference's rejection, greedy rows take torch.argmax's first NaN."""
    B, V = 272, 4096
    w = _big(B, V, torch.float32, seed=41, kinds="topk")
    x = w.logits.clone()
    x[3, 100] = float("nan"); w.temperature[3] = 0.9; w.top_k[3] = 20
    x[4, 7] = float("inf"); w.temperature[4] = 0.9; w.top_k[4] = 20
    x[5] = float("-inf"); w.temperature[5] = 0.9; w.top_k[5] = 20
    x[6, 50] = float("nan"); x[6, 30] = float("nan"); w.temperature[6] = 0.0
    w.logits = x
    out = PY.run_workload(w, dev)
    st = out.status.cpu()
    tok = out.tokens.cpu()
    assert st[3] == _lib.LPS_ROW_NONFINITE and tok[3] == -1
    assert st[4] == _lib.LPS_ROW_NONFINITE and tok[4] == -1
    assert st[5] == _lib.LPS_ROW_EMPTY and tok[5] == -1
    assert st[6] == 0 and tok[6] == 30
    ok = [i for i in range(B) if i not in (3, 4, 5, 6)]
    PY.check_rows(w, out, rows=ok)


def _peaked(B, V, dtype, seed, H=48, logprobs=False, top_k=0):
    """B nucleus rows of heavy-tailed logits (Student-t(3) x 2: a few logits
    hold almost all of the mass), with penalties over history ids; every fifth
    row flat (N(0, 0.1^2): its kept set is most of the row)."""
    g = torch.Generator().manual_seed(seed)
    rng = np.random.default_rng(seed)
    x = torch.from_numpy(rng.standard_t(3, size=(B, V)).astype(np.float32) * 2.0)
    flat = torch.arange(B) % 5 == 0
    x[flat] = torch.randn((int(flat.sum()), V), generator=g) * 0.1
    x = x.to(dtype)
    T = torch.from_numpy(rng.choice([0.7, 1.0, 1.3], size=B).astype(np.float32))
    p = torch.from_numpy(rng.choice([0.5, 0.9, 0.95, 0.99], size=B).astype(np.float32))
    f = lambda v: torch.full((B,), v, dtype=torch.float32)
    hist = torch.from_numpy(rng.integers(-3, V + 3, size=(B, H)).astype(np.int32))
    hist[:, : H // 4] = hist[:, H // 4: H // 2]
    hl = torch.from_numpy(rng.integers(0, H + 1, size=B).astype(np.int32))
    k = torch.full((B,), top_k, dtype=torch.int32)
    return W.Workload("peaked", x, T, k, p, f(0.0), f(1.0), f(1.2), f(0.4),
                      f(0.25), hist, hl, torch.rand((B,), generator=g), logprobs=logprobs, n_top=8 if top_k else 0)


@pytest.mark.parametrize("hint", [0, NUC])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_large_nucleus_batch(dev, dtype, hint):
    """Nucleus rows of a batch larger than one resident round (the row-group
    kernel, in rounds): heavy-tailed rows whose scaled logits reach ~100, where
    the chosen logprob must be computed in the same arithmetic as the row's
    mass, and flat rows; every row against the oracle, with the chosen
    logprob."""
    B, V = 288, 8192
    w = _peaked(B, V, dtype, seed=53 + int(dtype == torch.bfloat16), logprobs=True)
    out = PY.run_workload(w, dev, row_kind_hint=hint)
    rep = PY.check_rows(w, out, lp=True)
    path = out.row_path.cpu()
    _print(f"{dtype} hint {hint}: nucleus batch {rep}; general-kernel rows {int(path.sum())}/{B} "
           f"{_deferral_reasons(out, dev, B)}")
    assert (path[torch.arange(B) % 5 != 0] == 0).all()


def test_large_nucleus_batch_mask(dev):
    """Heavy-tailed nucleus rows of a large batch: legality bits equal -inf
    logits bit for bit, and both match the oracle."""
    B, V = 272, 8192
    w = _peaked(B, V, torch.bfloat16, seed=61)
    g = torch.Generator().manual_seed(5)
    legal = torch.rand((B, V), generator=g) < 0.8
    legal[:, 0] = True
    a = PY.run_workload(w, dev, allowed=legal.to(dev))
    wm = W.Workload(**{**w.__dict__, "logits": w.logits.masked_fill(~legal, float("-inf"))})
    b = PY.run_workload(wm, dev)
    assert torch.equal(a.tokens, b.tokens)
    assert torch.equal(a.kept_count, b.kept_count)
    PY.check_rows(wm, a)


@pytest.mark.parametrize("B", [24, 288])
def test_heavy_tailed_topk_logprobs(dev, B):
    """Top-k rows of heavy-tailed logits with chosen and top-N logprobs: on
    the row-group kernel (B = 24) and the streaming kernel (B = 288)."""
    w = _peaked(B, 8192, torch.float32, seed=71, logprobs=True, top_k=20)
    out = PY.run_workload(w, dev)
    rep = PY.check_rows(w, out, lp=True)
    _print(f"heavy-tailed top-k B={B}: {rep}")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_chi_square_draws_streaming_kernel(dev, dtype):
    """1e6 draws of one full-vocabulary top-k row (top_k 40, then top-p 0.9 on
    the top-k set: sampling.py:139-185, draw :84-85) on the streaming kernel
    alone (the top-k hint launches no row-group kernel, and no row may fall to
    the general kernel), against the fp64 kept law, in each input dtype.  The
    kept set is 28 of 64 spikes spread over the row (values 12 + k/16, exact in
    every dtype), so the candidates come from every wave."""
    from scipy.stats import chisquare
    from lps import SamplingParams, sample_rows
    from oracle import reference_semantics as O
    g = torch.Generator().manual_seed(19)
    V, N = 151936, 1_000_000
    row = torch.randn((1, V), generator=g)
    spikes = torch.linspace(53, V - 71, 64).long()
    row[0, spikes] = 12.0 + torch.arange(64, dtype=torch.float32) / 16
    row = row.to(dtype)
    r = O.sample_row(row[0], O.RowParams(temperature=1.0, top_k=40, top_p=0.9), [], 0.5)
    kept = r.kept
    # closed form: within the 40 largest spikes, the 27 largest hold 0.88790 of
    # their mass and 28 hold 0.90011, so top-p keeps the 28 largest
    assert np.array_equal(np.nonzero(kept)[0], spikes[36:].numpy())
    x = row.to(dev).expand(N, V)                          # stride 0 over rows
    p = SamplingParams.build(N, dev, temperature=1.0, top_k=40, top_p=0.9)
    u = torch.rand(N, device=dev, generator=torch.Generator(device=dev).manual_seed(7))
    out = sample_rows(x, p, u, row_kind_hint=TOPK)
    assert int(out.row_path.ne(0).sum().item()) == 0
    assert int(out.status.ne(0).sum().item()) == 0
    counts = torch.bincount(out.tokens, minlength=V).cpu().numpy()
    assert counts[~kept].sum() == 0
    stat, pval = chisquare(counts[kept], r.probs64[kept] * N)
    _print(f"chi-square 1e6 draws, streaming kernel, V={V} {dtype}: kept={int(kept.sum())} stat={stat:.1f} p={pval:.3g}")
    assert pval > 1e-4
