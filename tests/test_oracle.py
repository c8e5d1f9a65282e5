"""Pins the CPU oracle (oracle/reference_semantics.py) against brute force,
closed forms, library routines and the reference's own known-answer tests.
A plausible slip (a dropped term, a wrong sign or index, a transposed
operand, an unstable tie order) fails at least one check here."""

import math

import numpy as np
import pytest
import torch

from oracle import reference_semantics as O


def _np32(x):
    return np.asarray(x, dtype=np.float32)


# ------------------------------------------------------------- penalties --


def test_repetition_penalty_brute_force():
    """sampling.py:108-137: each distinct in-range id once; x>0 divides, else multiplies."""
    rng = np.random.default_rng(0)
    V = 40
    x = torch.from_numpy(rng.normal(0, 2, size=(3, V)).astype(np.float32))
    x[0, 5] = 0.0
    hist = [5, 7, 7, 7, -3, 40, 39, 12, 5, 1000]
    pen = 1.3
    got = O.apply_repetition_penalty(x, hist, pen)
    want = x.numpy().copy()
    for d in sorted(set(h for h in hist if 0 <= h < V)):
        for b in range(3):
            v = want[b, d]
            want[b, d] = np.float32(v / np.float32(pen)) if v > 0 else np.float32(v * np.float32(pen))
    assert np.array_equal(got.numpy(), want)
    # ids outside [0, V) change nothing; duplicates are applied once
    once = O.apply_repetition_penalty(x, [7], pen)
    assert torch.equal(O.apply_repetition_penalty(x, [7, 7, 7], pen), once)
    assert torch.equal(O.apply_repetition_penalty(x, [-1, V, V + 5], pen), x)
    assert torch.equal(O.apply_repetition_penalty(x, [], pen), x)
    assert torch.equal(O.apply_repetition_penalty(x, [3], 1.0), x)


def test_presence_frequency_closed_form():
    rng = np.random.default_rng(1)
    V = 30
    x = torch.from_numpy(rng.normal(0, 3, size=(1, V)).astype(np.float32))
    hist = [1, 1, 1, 4, 9, 9, 29, -1, 30]
    got = O.apply_presence_frequency(x, hist, 0.5, 0.3)
    want = x.numpy().copy()
    cnt = {}
    for h in hist:
        if 0 <= h < V:
            cnt[h] = cnt.get(h, 0) + 1
    for d, c in cnt.items():
        want[0, d] = np.float32(np.float32(want[0, d] - np.float32(np.float32(c) * np.float32(0.3))) - np.float32(0.5))
    assert np.array_equal(got.numpy(), want)
    # presence only / frequency only
    assert torch.equal(O.apply_presence_frequency(x, hist, 0.0, 0.0), x)
    g2 = O.apply_presence_frequency(x, [2, 2], 0.0, 1.0)
    assert g2[0, 2].item() == np.float32(x[0, 2].item() - 2.0)


def test_temperature_is_correctly_rounded_division():
    """Parity rule 2: x / T equals IEEE fp32 division, not a reciprocal multiply."""
    rng = np.random.default_rng(2)
    x = rng.normal(0, 5, size=100000).astype(np.float32)
    for T in (0.7, 0.3, 1.1, 0.8333):
        got = (torch.from_numpy(x) / T).numpy()
        assert np.array_equal(got, x / np.float32(T))
    recip = x * (np.float32(1.0) / np.float32(0.7))
    assert not np.array_equal(recip, x / np.float32(0.7))


# ---------------------------------------------------------------- top-k --


def test_top_k_brute_force_with_ties():
    rng = np.random.default_rng(3)
    for trial in range(50):
        V = int(rng.integers(1, 60))
        x = rng.integers(-4, 5, size=V).astype(np.float32)   # many ties
        k = int(rng.integers(0, V + 3))
        got = O.apply_top_k(torch.from_numpy(x).reshape(1, -1), k).numpy().reshape(-1)
        if k <= 0:
            assert np.array_equal(got, x)
            continue
        kth = np.sort(x)[::-1][min(k, V) - 1]
        want = np.where(x >= kth, x, -np.inf)
        assert np.array_equal(got, want)
        assert np.sum(np.isfinite(got)) >= min(k, V)


# ---------------------------------------------------------------- top-p --


def _top_p_brute(x, p):
    """Keep sorted position j iff j == 0 or exclusive prefix mass <= p, with a
    stable descending order (lower index first) and fp64 masses."""
    V = x.size
    order = sorted(range(V), key=lambda i: (-x[i], i))
    e = np.exp(x.astype(np.float64) - x.max())
    Z = e.sum()
    keep = np.zeros(V, bool)
    acc = 0.0
    for j, i in enumerate(order):
        if j == 0 or acc / Z <= p:
            keep[i] = True
        acc += e[i]
    return keep


def test_top_p_brute_force():
    rng = np.random.default_rng(4)
    mism = 0
    for trial in range(300):
        V = int(rng.integers(1, 40))
        x = (rng.normal(0, 2, size=V)).astype(np.float32)
        if trial % 3 == 0:
            x = np.round(x).astype(np.float32)             # ties
        p = float(rng.uniform(0.05, 0.99))
        got = np.isfinite(O.apply_top_p(torch.from_numpy(x).reshape(1, -1), p).numpy().reshape(-1))
        want = _top_p_brute(x, p)
        if not np.array_equal(got, want):
            # only a boundary-ambiguous decision may differ
            assert O.top_p_band(torch.from_numpy(x), p, int(got.sum()), int(want.sum()), eps=1e-6)
            mism += 1
    assert mism <= 3


def test_top_p_ties_lower_index_first_and_edges():
    x = torch.tensor([[1.0, 3.0, 3.0, 3.0, 0.0]])
    # masses e^0 (x3) dominate: p small keeps only the first of the tied maxima
    kept = torch.isfinite(O.apply_top_p(x, 0.1)).reshape(-1).tolist()
    assert kept == [False, True, False, False, False]
    kept = torch.isfinite(O.apply_top_p(x, 0.4)).reshape(-1).tolist()
    assert kept == [False, True, True, False, False]
    assert torch.equal(O.apply_top_p(x, 1.0), x)                          # p >= 1: no-op
    assert torch.isfinite(O.apply_top_p(x, 0.0)).sum().item() == 1        # p <= 0: argmax only
    assert torch.isfinite(O.apply_top_p(x, -1.0)).reshape(-1).tolist()[1]


# ------------------------------------------------------- min-p, typical --


def test_min_p_closed_form():
    x = torch.tensor([[0.0, -1.0, -2.0, -3.0, 1.0]])
    got = torch.isfinite(O.apply_min_p(x, 0.3)).reshape(-1).numpy()
    e = np.exp(x.numpy().reshape(-1) - 1.0)
    assert np.array_equal(got, e >= 0.3)
    assert torch.equal(O.apply_min_p(x, 0.0), x)


def test_typical_p_closed_form_and_nan_fallback():
    rng = np.random.default_rng(5)
    x = torch.from_numpy(rng.normal(0, 1, size=(1, 50)).astype(np.float32))
    got = torch.isfinite(O.apply_typical_p(x, 0.9)).reshape(-1).numpy()
    p = np.exp(x.numpy().reshape(-1).astype(np.float64))
    p /= p.sum()
    H = -(p * np.log(p)).sum()
    want = -np.log(p) <= np.exp(H) * 0.9
    assert np.array_equal(got, want)
    # a row holding -inf: entropy NaN -> only the argmax survives (sampling.py:231-234)
    y = x.clone()
    y[0, 3] = float("-inf")
    kept = torch.isfinite(O.apply_typical_p(y, 0.9)).reshape(-1)
    assert kept.sum().item() == 1 and kept[int(torch.argmax(y))]


# ------------------------------------------------------------------ draw --


def test_inverse_cdf_draw_brute_force():
    # ids walked by z descending, ties lower index first: 2, 3, 6, 0, 5 (-inf last)
    z = torch.tensor([0.0, float("-inf"), 1.0, 0.5, float("-inf"), -0.3, 0.5])
    vals = z.tolist()
    order = sorted(range(len(vals)), key=lambda i: (-vals[i], i))
    assert order[:5] == [2, 3, 6, 0, 5]
    e = [math.exp(vals[i] - 1.0) if math.isfinite(vals[i]) else 0.0 for i in order]
    tot = sum(e)
    for u in np.linspace(0, 0.999999, 97):
        j = O.draw_inverse_cdf(z, float(u))
        acc, want = 0.0, None
        for pos, i in enumerate(order):
            acc += e[pos] / tot
            if want is None and u < acc:
                want = i
        assert j == want and math.isfinite(z[j].item()), (u, j, want)
    assert O.draw_inverse_cdf(z, 0.0) == 2          # the largest z first
    assert O.draw_inverse_cdf(z, 0.99999) == 5       # the smallest finite z last


def test_inverse_cdf_draw_chi_square():
    from scipy.stats import chisquare
    rng = np.random.default_rng(6)
    z = torch.from_numpy(rng.normal(0, 1, size=12).astype(np.float32))
    e = np.exp(z.double().numpy() - z.max().item())
    probs = e / e.sum()
    n = 100000
    us = rng.random(n)
    counts = np.zeros(12)
    for u in us:
        counts[O.draw_inverse_cdf(z, float(u))] += 1
    stat, pval = chisquare(counts, probs * n)
    assert pval > 1e-4


def test_multinomial_matches_inverse_cdf_distribution():
    """torch.multinomial (reference draw) and the inverse CDF sample the same law."""
    from scipy.stats import chisquare
    g = torch.Generator().manual_seed(7)
    z = torch.randn(8, generator=g)
    probs = torch.softmax(z, -1)
    draws = torch.multinomial(probs.expand(20000, -1).contiguous(), 1, replacement=True, generator=g).reshape(-1)
    counts = np.bincount(draws.numpy(), minlength=8)
    stat, pval = chisquare(counts, probs.double().numpy() * counts.sum())
    assert pval > 1e-4


# -------------------------------------------------------------- logprobs --


def test_logprobs_library():
    g = torch.Generator().manual_seed(8)
    z = torch.round(torch.randn(100, generator=g) * 3)    # ties
    chosen, vals, ids = O.logprobs_row(z, 17, 20)
    lp = torch.log_softmax(z.double(), -1)
    assert chosen == lp[17].item()
    # closed form, with an exactly rounded sum
    zz = z.double().tolist()
    assert abs(chosen - (zz[17] - math.log(math.fsum(math.exp(v) for v in zz)))) < 1e-12
    order = torch.sort(z, descending=True, stable=True).indices[:20].tolist()
    assert ids.tolist() == order
    assert np.array_equal(vals, lp[order].numpy().astype(np.float32))


def test_entropy_closed_form():
    assert abs(O.entropy_row(torch.zeros(64)) - math.log(64)) < 1e-5


# ------------------------------------------------------------ one row ----


def test_sample_row_greedy_after_penalty():
    x = torch.tensor([1.0, 5.0, 4.9, -2.0])
    p = O.RowParams(temperature=0.0, repetition_penalty=2.0)
    r = O.sample_row(x, p, history=[1], u=0.3)
    assert r.greedy and r.token == 2          # 5/2 = 2.5 < 4.9
    r = O.sample_row(torch.tensor([3.0, 3.0, 1.0]), O.RowParams(temperature=0.0), [], 0.1)
    assert r.token == 0                       # first index on ties


def test_sample_row_errors():
    r = O.sample_row(torch.tensor([float("nan"), 1.0]), O.RowParams(temperature=1.0), [], 0.5)
    assert r.error == "nonfinite"
    r = O.sample_row(torch.tensor([float("-inf"), float("-inf")]), O.RowParams(temperature=1.0), [], 0.5)
    assert r.error == "nonfinite"


# ----------------------------------------------------------- speculative --


def test_verify_drafts_matches_python_loop():
    """Restates test_kernels_low_level.py:439-454 (seeded)."""
    g = torch.Generator().manual_seed(9)
    K, V = 64, 16
    tp = torch.softmax(torch.randn(K, V, generator=g), dim=-1)
    dp = torch.rand(K, generator=g) * 0.5 + 0.1
    dt = torch.randint(0, V, (K,), generator=g)
    u = torch.rand(K, generator=g)
    out = O.verify_drafts_ref(tp, dp, dt, u)
    assert out.dtype == torch.int8 and out.shape == (K,)
    for i in range(K):
        p = tp[i, dt[i]].item()
        q = max(dp[i].item(), 1e-9)
        assert int(out[i]) == (1 if u[i].item() < min(p / q, 1.0) else 0)


def _one_hot_logits(seq_next, V):
    x = torch.full((V,), -1e9)
    x[seq_next % V] = 1e9
    return x


def test_spec_verify_greedy_toy_models():
    """test_speculative_decoding.py:70-121: with one-hot toy LMs and T=0, a
    perfect draft is fully accepted (plus the bonus) and a bad draft is
    rejected at position 0 with the target argmax as replacement."""
    V, B, k = 32, 3, 4
    last = torch.tensor([3, 10, 31])
    tgt = torch.stack([torch.stack([_one_hot_logits(int(last[b]) + 1 + i, V) for i in range(k + 1)]) for b in range(B)])
    good = torch.stack([torch.stack([_one_hot_logits(int(last[b]) + 1 + i, V) for i in range(k)]) for b in range(B)])
    toks = torch.stack([torch.tensor([(int(last[b]) + 1 + i) % V for i in range(k)]) for b in range(B)])
    ua, ur = torch.rand(B, k), torch.rand(B, k + 1)
    n, out, bits, P, Q = O.spec_verify_ref(tgt, good, toks, ua, ur, 0.0)
    assert n.tolist() == [k] * B
    assert out[:, :k].tolist() == toks.tolist()
    assert out[:, k].tolist() == [(int(last[b]) + 1 + k) % V for b in range(B)]
    bad = torch.stack([torch.tensor([(int(last[b]) + 13 + i) % V for i in range(k)]) for b in range(B)])
    n, out, bits, P, Q = O.spec_verify_ref(tgt, good, bad, ua, ur, 0.0)
    assert n.tolist() == [0] * B
    assert out[:, 0].tolist() == [(int(last[b]) + 1) % V for b in range(B)]
    assert (out[:, 1:] == -1).all()


def test_spec_verify_accept_rule_matches_verify_drafts():
    g = torch.Generator().manual_seed(10)
    B, k, V = 6, 3, 50
    tgt = torch.randn(B, k + 1, V, generator=g)
    drf = tgt[:, :k] + 0.5 * torch.randn(B, k, V, generator=g)
    toks = torch.randint(0, V, (B, k), generator=g)
    ua, ur = torch.rand(B, k, generator=g), torch.rand(B, k + 1, generator=g)
    n, out, bits, P, Q = O.spec_verify_ref(tgt, drf, toks, ua, ur, 0.8, 1.0)
    tp = torch.softmax(tgt[:, :k] / 0.8, -1).reshape(B * k, V)
    dp = torch.softmax(drf / 0.8, -1).reshape(B * k, V)
    q = dp.gather(-1, toks.reshape(-1, 1)).reshape(-1)
    ref = O.verify_drafts_ref(tp, q, toks.reshape(-1), ua.reshape(-1)).reshape(B, k)
    assert torch.equal(bits, ref)
    for b in range(B):
        j = int(n[b])
        assert j == (k if bits[b].all() else int(torch.nonzero(bits[b] == 0)[0]))


def test_mirostat_v2_closed_form():
    # uniform logits over V: H = ln V, every id ties at the k-th value (top-k keeps all)
    V, tau, eta = 8, 5.0, 0.1
    x = torch.zeros(1, V)
    tok, prev, k = O.mirostat_v2_ref(x, 1.0, tau, eta, None, 0.99)
    H = math.log(V)
    assert abs(prev - (H - eta * (H - tau))) < 1e-6
    assert k == max(1, int(math.exp(prev)))
    assert tok == 7  # inverse CDF of u = 0.99 over 8 equal masses
    # two-level distribution: entropy from an explicit loop, k from the update rule
    x = torch.tensor([[3.0, 3.0, 0.0, 0.0, 0.0, -1.0]])
    T = 0.5
    p = torch.softmax(x / T, -1).double().reshape(-1).tolist()
    H = -sum(pi * math.log(pi) for pi in p)
    tok, prev, k = O.mirostat_v2_ref(x, T, 0.2, 0.5, 0.9, 0.3)
    assert abs(prev - (0.9 - 0.5 * (H - 0.2))) < 1e-6
    assert k == max(1, int(math.exp(prev))) and k == 1
    assert tok == 0  # k = 1 keeps the first maximum (lower index wins the tie)
    # non-positive running estimate: no top-k, a plain draw
    tok, prev, k = O.mirostat_v2_ref(x, T, 0.0, 1.0, 0.1, 0.999999)
    assert prev <= 0 and k == 0 and tok == 5


def test_top_p_truth_brute_force():
    # fp64 keep rule by an explicit loop over every id, ties lower-index-first
    g = torch.Generator().manual_seed(21)
    for trial in range(40):
        V = int(torch.randint(1, 12, (1,), generator=g))
        z = torch.round(torch.randn(V, generator=g) * 2) / 2  # repeated values
        if trial % 5 == 0:
            z[int(torch.randint(0, V, (1,), generator=g))] = float("-inf")
        p = float(torch.rand(1, generator=g)) * 0.999  # p >= 1 turns the filter off
        vals = [float(v) for v in z]
        m = max(vals)
        w = [math.exp(v - m) if v != float("-inf") else 0.0 for v in vals]
        tot = sum(w)
        idx = sorted(range(V), key=lambda i: (-vals[i], i))
        n, run = 0, 0.0
        for pos, i in enumerate(idx):
            if pos == 0 or run / tot <= p:
                n += 1
            else:
                break
            run += w[i]
        order, excl, n_truth = O.top_p_truth(z, p)
        assert list(order) == idx
        assert n_truth == n, (trial, vals, p)


def test_top_p_reference_cum_invariants():
    g = torch.Generator().manual_seed(22)
    z = torch.randn(4000, generator=g) * 3
    ref = O.top_p_reference_cum(z)
    _, excl, _ = O.top_p_truth(z, 0.9)
    assert ref[0] == 0.0                                    # exclusive: nothing precedes the maximum
    p0 = float(torch.softmax(z.double(), 0).max())
    assert abs(ref[1] - p0) < 1e-6                          # then the largest probability
    assert np.all(np.diff(ref) >= 0)                        # descending order gives a non-decreasing prefix
    assert np.max(np.abs(ref - excl)) < 4000 * 2.0 ** -24   # fp32 accumulation of the fp64 truth
    assert np.max(np.abs(ref - excl)) > 0                   # and it is the fp32 one, not the truth


def test_top_p_band_known_cases():
    # four equal masses: exclusive prefixes 0, 1/4, 1/2, 3/4 in stable order
    z = torch.zeros(4)
    _, excl, n = O.top_p_truth(z, 0.5)
    assert n == 3 and np.allclose(excl, [0.0, 0.25, 0.5, 0.75])
    # counts 2 and 3 differ only at position 2, whose prefix is exactly top_p
    assert O.top_p_band(z, 0.5, 3, 2, 2e-6)
    assert O.top_p_band(z, 0.5 + 1e-6, 2, 3, 2e-6)
    assert not O.top_p_band(z, 0.5 + 1e-5, 2, 3, 2e-6)
    # counts 3 and 4 differ at position 3 (prefix 3/4, far from 0.5)
    assert not O.top_p_band(z, 0.5, 3, 4, 2e-6)
    # a span of two positions is in the band only if both are
    assert not O.top_p_band(z, 0.5, 2, 4, 2e-6)
    assert O.top_p_band(z, 0.5, 3, 3, 0.0)


def test_top_p_reference_rounding_known_cases():
    # three equal masses: fp32 softmax rounds 1/3 up to 0.33333334, so the
    # reference's prefix at position 1 lies above the fp64 truth 1/3
    z = torch.zeros(3)
    ref = O.top_p_reference_cum(z)
    _, excl, n_truth = O.top_p_truth(z, 1.0 / 3.0)
    assert n_truth == 2
    assert ref[1] > excl[1] and abs(ref[1] - excl[1]) < 1e-7
    # with top_p = 1/3 the reference's fp32 compare drops position 1 (count 1);
    # the difference is explained by its rounding, even with no slack
    assert O.top_p_reference_rounding(z, 1.0 / 3.0, 2, 1, eps=0.0)
    # at top_p = 0.3 position 1 is 0.033 away from top_p: not rounding
    assert not O.top_p_reference_rounding(z, 0.3, 2, 1, eps=0.0)
    # equal counts are always explained
    assert O.top_p_reference_rounding(z, 0.3, 1, 1, eps=0.0)


def _lev_case():
    tgt = torch.tensor([[[1.0, 0.2, -0.5, 0.9], [0.0, 0.0, 0.0, 0.0]]])
    drf = torch.tensor([[[0.1, 1.5, -0.2, 0.3]]])
    return tgt, drf


def test_leviathan_residual_brute_force():
    """speculative.py:150-157 computes the textbook residual max(p - q, 0) (and
    then resamples the target instead); the oracle's "leviathan" branch draws
    from the normalised residual by inverse CDF in vocabulary order."""
    tgt, drf = _lev_case()
    p = torch.softmax(tgt[0, 0].double(), -1)
    q = torch.softmax(drf[0, 0].double(), -1)
    t = int(torch.argmax(q - p))                       # q > p there: a likely reject
    r = [max(float(p[i] - q[i]), 0.0) for i in range(4)]
    for u in np.linspace(0.0, 0.999, 41):
        # brute force: walk the ids, accumulating the residual
        acc, want = 0.0, None
        for i in range(4):
            acc += r[i] / sum(r)
            if want is None and u < acc:
                want = i
        n, tok, bits, _, _ = O.spec_verify_ref(tgt, drf, torch.tensor([[t]]), torch.tensor([[0.9999]]),
                                               torch.tensor([[float(u), 0.5]]), 1.0, 1.0, "leviathan")
        assert int(n[0]) == 0 and int(bits[0, 0]) == 0
        assert int(tok[0, 0]) == want, (u, int(tok[0, 0]), want)
        assert r[int(tok[0, 0])] > 0.0


def test_leviathan_first_token_law_is_target():
    """Speculative sampling with the residual max(p - q, 0) emits its first
    token with the target law p exactly (Leviathan et al. 2023, Theorem 1).
    The oracle's accept rule and residual branch, integrated over the draft
    token and both uniforms on a fine grid, must give p."""
    tgt, drf = _lev_case()
    p = torch.softmax(tgt[0, 0], -1).double().numpy()
    q = torch.softmax(drf[0, 0], -1).double().numpy()
    grid = (np.arange(400) + 0.5) / 400
    law = np.zeros(4)
    for t in range(4):
        n_acc = 0
        for ua in grid:
            n, tok, bits, _, _ = O.spec_verify_ref(tgt, drf, torch.tensor([[t]]), torch.tensor([[float(ua)]]),
                                                   torch.tensor([[0.5, 0.5]]), 1.0, 1.0, "leviathan")
            n_acc += int(n[0])
        acc = n_acc / grid.size
        law[t] += q[t] * acc
        res = np.zeros(4)
        for ur in grid:
            _, tok, _, _, _ = O.spec_verify_ref(tgt, drf, torch.tensor([[t]]), torch.tensor([[1.0]]),
                                                torch.tensor([[float(ur), 0.5]]), 1.0, 1.0, "leviathan")
            res[int(tok[0, 0])] += 1.0 / grid.size
        law += q[t] * (1.0 - acc) * res
    assert np.abs(law - p).max() < 6e-3, (law, p)
