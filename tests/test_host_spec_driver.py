"""The oracle's speculative-decoding driver loops (``spec_decode_ref``,
``mtp_decode_ref``: ``speculative.py:68-178, 206-280``), pinned on the CPU.

1. The reference's own driver tests, restated against the oracle
   (``testing/unit/test_speculative_decoding.py:59-217``).
2. Greedy speculative decoding equals greedy decoding of the target alone,
   on random trigram models, for several draft lengths.
3. With T > 0 the first emitted token follows the law the reference's rule
   implies: draft ``d ~ q`` kept with probability ``min(1, p/q)``, else a
   replacement from ``p`` (``:150-157``), i.e.
   ``P(x) = min(p(x), q(x)) + (1 - sum_y min(p(y), q(y))) p(x)``
   (chi-square over many uniforms).  The MTP loop's first token is the main
   model's draw, ``P(x) = p(x)``.
"""

import math

import numpy as np
import pytest
import torch

from oracle import reference_semantics as O
from tests import spec_toys as Y


def _rand_uniforms(seed, width):
    g = torch.Generator().manual_seed(seed)

    def f(r):
        u = torch.rand(width, generator=g)
        return u
    return f


def _split(k):
    def wrap(f):
        def g(r):
            u = f(r)
            return u[:k], u[k: 2 * k], u[2 * k:]
        return g
    return wrap


def _greedy_target_decode(model, prompt, n):
    ref = prompt.clone()
    for _ in range(n):
        nxt = model(ref)[:, -1, :].argmax(dim=-1, keepdim=True)
        ref = torch.cat([ref, nxt], dim=1)
    return ref[:, prompt.shape[1]:]


# -- 1. the reference's own cases ---------------------------------------------
def test_ref_case_perfect_draft_matches_target_greedy():
    prompt = torch.tensor([[3]])
    out, rounds, calls, acc = O.spec_decode_ref(Y.greedy_target, Y.greedy_target, prompt, 10, 4, 0.0, None,
                                                _split(4)(_rand_uniforms(0, 13)))
    assert torch.equal(out[:, :10], _greedy_target_decode(Y.greedy_target, prompt, 10))
    out, rounds, calls, acc = O.spec_decode_ref(Y.greedy_target, Y.greedy_target, torch.tensor([[1]]), 20, 4, 0.0,
                                                None, _split(4)(_rand_uniforms(1, 13)))
    assert calls <= 6 and acc >= 16
    assert out.shape[1] >= 20


def test_ref_case_bad_draft_still_correct():
    prompt = torch.tensor([[2]])
    out, rounds, calls, acc = O.spec_decode_ref(Y.greedy_target, Y.greedy_bad_draft, prompt, 5, 4, 0.0, None,
                                                _split(4)(_rand_uniforms(2, 13)))
    assert torch.equal(out[:, :5], _greedy_target_decode(Y.greedy_target, prompt, 5))
    assert acc == 0


def test_ref_case_eos_stops_early():
    out, *_ = O.spec_decode_ref(Y.greedy_target, Y.greedy_target, torch.tensor([[5]]), 20, 4, 0.0, 6,
                                _split(4)(_rand_uniforms(3, 13)))
    assert int(out[0, 0]) == 6 and out.shape[1] <= 4


def _mtp_u(seed):
    f = _rand_uniforms(seed, 3)

    def g(r):
        u = f(r)
        return float(u[0]), float(u[1]), float(u[2])
    return g


def test_ref_case_mtp_perfect_head():
    main = Y.ToyMain()
    prompt = torch.tensor([[7]])
    out, rounds, calls, acc = O.mtp_decode_ref(main, Y.toy_mtp_head, prompt, 10, 0.0, None, _mtp_u(4))
    assert rounds <= 6
    assert torch.equal(out[:, :10], _greedy_target_decode(Y.greedy_target, prompt, 10))


def test_ref_case_mtp_eos():
    out, *_ = O.mtp_decode_ref(Y.ToyMain(), Y.toy_mtp_head, torch.tensor([[7]]), 20, 0.0, 8, _mtp_u(5))
    assert int(out[0, 0]) == 8 and out.shape[1] <= 1


# -- 2. greedy speculative decoding == target greedy --------------------------
@pytest.mark.parametrize("k", [1, 3, 5])
@pytest.mark.parametrize("seed", [0, 1])
def test_greedy_spec_equals_target_greedy(k, seed):
    V = 48
    target = Y.Trigram(V, seed)
    draft = Y.Trigram(V, seed + 100, base=target, noise=1.5)
    prompt = torch.tensor([[seed % V, (seed * 7 + 3) % V]])
    out, rounds, calls, acc = O.spec_decode_ref(target, draft, prompt, 17, k, 0.0, None,
                                                _split(k)(_rand_uniforms(seed, 3 * k + 1)))
    assert torch.equal(out[:, :17], _greedy_target_decode(target, prompt, 17))
    assert calls == rounds and 0 <= acc <= rounds * k


def test_greedy_mtp_equals_main_greedy():
    V = 40
    main = Y.TrigramMain(V, 3)
    out, *_ = O.mtp_decode_ref(main, Y.TrigramMTP(V, 3), torch.tensor([[1, 2]]), 15, 0.0, None, _mtp_u(6))
    assert torch.equal(out[:, :15], _greedy_target_decode(main.lm, torch.tensor([[1, 2]]), 15))


# -- 3. the first token's law with T > 0 --------------------------------------
def _chi2_ok(counts, probs, n):
    exp = probs * n
    keep = exp >= 5
    stat = float((((counts - exp) ** 2) / np.maximum(exp, 1e-12))[keep].sum())
    df = int(keep.sum()) - 1
    # 99.9 % quantile of chi-square by the Wilson-Hilferty approximation
    z = 3.09
    q = df * (1 - 2 / (9 * df) + z * math.sqrt(2 / (9 * df))) ** 3
    return stat < q, stat, q


def test_first_token_law_two_model():
    V, T, k, N = 12, 0.9, 2, 6000
    target = Y.Trigram(V, 11, scale=1.0)
    draft = Y.Trigram(V, 12, base=target, noise=1.0)
    prompt = torch.tensor([[4, 9]])
    p = torch.softmax(target(prompt)[0, -1].double() / T, -1).numpy()
    q = torch.softmax(draft(prompt)[0, -1].double() / T, -1).numpy()
    law = np.minimum(p, q) + (1 - np.minimum(p, q).sum()) * p
    g = torch.Generator().manual_seed(99)
    counts = np.zeros(V)
    for _ in range(N):
        u = torch.rand(3 * k + 1, generator=g)
        out, *_ = O.spec_decode_ref(target, draft, prompt, 1, k, T, None,
                                    lambda r, u=u: (u[:k], u[k: 2 * k], u[2 * k:]))
        counts[int(out[0, 0])] += 1
    ok, stat, q999 = _chi2_ok(counts, law, N)
    assert ok, f"chi2 {stat:.1f} >= {q999:.1f}"
    # and the law is not the target's own (the check has power here)
    ok2, _, _ = _chi2_ok(counts, p, N)
    assert not ok2 or np.abs(law - p).max() < 0.01


def test_first_token_law_mtp():
    V, T, N = 10, 1.1, 4000
    main = Y.TrigramMain(V, 21)
    prompt = torch.tensor([[3, 5]])
    p = torch.softmax(main.lm(prompt)[0, -1].double() / T, -1).numpy()
    g = torch.Generator().manual_seed(7)
    counts = np.zeros(V)
    for _ in range(N):
        u = torch.rand(3, generator=g)
        out, *_ = O.mtp_decode_ref(main, Y.TrigramMTP(V, 21), prompt, 1, T, None,
                                   lambda r, u=u: (float(u[0]), float(u[1]), float(u[2])))
        counts[int(out[0, 0])] += 1
    ok, stat, q999 = _chi2_ok(counts, p, N)
    assert ok, f"chi2 {stat:.1f} >= {q999:.1f}"
