"""GPU parity of the HIP sampler against the CPU oracle, through the C ABI
(``lps.sample_rows`` -> ``lps_sample``), on the seeded BASELINE.json
configurations and the reference's edge cases."""

import math

import numpy as np
import pytest
import torch

from oracle import reference_semantics as O
from tests import parity as PY
from tests import workloads as W

pytestmark = pytest.mark.gpu


def _print(msg):
    print(msg, flush=True)


def test_c1_single_row_sampling_and_greedy(dev):
    for greedy in (False, True):
        w = W.c1(greedy=greedy)
        out = PY.run_workload(w, dev)
        rep = PY.check_rows(w, out)
        _print(f"c1 greedy={greedy}: {rep}")


def test_c2_mixed_params_bf16_full_size(dev):
    w = W.c2()
    out = PY.run_workload(w, dev)
    rep = PY.check_rows(w, out)
    _print(f"c2: {rep}")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_c2_rows_past_one_round(dev, dtype):
    """c2's rows at B=96 (16-bit): more chunk workgroups than one resident
    round at 80 logits per thread, so the row-group kernel runs 104 per
    thread (three chunks per row) for the nucleus rows while the top-k rows
    stream; every row against the oracle."""
    w = W.c2(B=96)
    w.logits = w.logits.to(dtype)
    out = PY.run_workload(w, dev)
    rep = PY.check_rows(w, out)
    paths = out.row_path.cpu()
    _print(f"c2 B=96 {dtype}: {rep}; general-kernel rows {int((paths == 1).sum())}")
    assert int((paths == 1).sum()) <= 2, paths.tolist()


@pytest.mark.parametrize("B", [16, 256])
@pytest.mark.parametrize("flat", [False, True])
def test_c3_nucleus_fp32(dev, flat, B):
    """c3 at B=16 and at its own size B=256 (the launch shape of the benchmark),
    every row against the oracle's top-p rule (sampling.py:158-185)."""
    w = W.c3(B=B, flat=flat)
    out = PY.run_workload(w, dev)
    rep = PY.check_rows(w, out)
    nfast = int((out.row_path.cpu() == 0).sum())
    _print(f"c3 flat={flat} B={B}: {rep}; fast-path rows {nfast}/{B}; "
           f"kept_counts={out.kept_count.cpu().tolist()[:6]}")


def test_c5_logprobs_fp16_subset(dev):
    w = W.c5(B=32)
    out = PY.run_workload(w, dev)
    rep = PY.check_rows(w, out, lp=True)
    _print(f"c5 subset: {rep}")


def test_c5_full_size_properties(dev):
    """B=512 fp16 with logprobs at full size: size-independent properties."""
    w = W.c5()
    out = PY.run_workload(w, dev)
    tok = out.tokens.cpu()
    assert (out.status.cpu() == 0).all()
    assert ((tok >= 0) & (tok < w.V)).all()
    lp = out.chosen_logprob.cpu()
    tl = out.top_logprobs.cpu()
    ti = out.top_ids.cpu()
    assert (lp <= 1e-6).all() and (tl <= 1e-6).all()
    assert (tl[:, :-1] >= tl[:, 1:]).all()                 # sorted descending
    greedy = w.temperature <= 0
    assert torch.equal(ti[greedy, 0], tok[greedy])          # greedy token = top-1 id
    assert torch.allclose(lp[greedy], tl[greedy, 0])
    assert (lp[~greedy] <= tl[~greedy, 0] + 1e-6).all()
    # sampled rows draw inside their top-40 (top_k = 40, ties aside)
    cnt = out.kept_count.cpu()
    assert (cnt[~greedy] >= 1).all() and (cnt[~greedy] <= 60).all()
    # a few full-size rows against the oracle
    PY.check_rows(w, out, rows=[0, 1, 257, 511], lp=True)


def test_determinism_repeat(dev):
    w = W.c2(B=16)
    a = PY.run_workload(w, dev)
    b = PY.run_workload(w, dev)
    assert torch.equal(a.tokens, b.tokens)
    assert torch.equal(a.kept_cut, b.kept_cut) and torch.equal(a.kept_ties, b.kept_ties)


def _small(V, B, dtype, seed, **over):
    g = torch.Generator().manual_seed(seed)
    rng = np.random.default_rng(seed)
    x = torch.randn((B, V), generator=g) * 2
    if seed % 3 == 0:
        x = torch.round(x * 2)             # ties
    x = x.to(dtype)
    f = lambda v, dt=torch.float32: torch.full((B,), v, dtype=dt)
    T = torch.from_numpy(rng.choice([0.0, 0.5, 1.0, 1.7, -1.0], size=B).astype(np.float32))
    k = torch.from_numpy(rng.choice([0, 1, 3, V, V + 5], size=B).astype(np.int32))
    p = torch.from_numpy(rng.choice([1.0, 0.9, 0.5, 0.0, -0.5], size=B).astype(np.float32))
    H = 12
    hist = torch.from_numpy(rng.integers(-3, V + 3, size=(B, H)).astype(np.int32))
    hl = torch.from_numpy(rng.integers(0, H + 1, size=B).astype(np.int32))
    w = W.Workload("small", x, T, k, p, f(0.0), f(1.0), f(1.3), f(0.2), f(0.1), hist, hl, torch.rand((B,), generator=g))
    for kk, vv in over.items():
        setattr(w, kk, vv)
    return w


@pytest.mark.parametrize("V", [1, 7, 64, 1000, 4099])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_small_vocab_mixed_params(dev, V, dtype):
    """Scalar (V % 8 != 0) and vector paths, ties, every filter edge, penalties
    with out-of-range and empty histories."""
    # (the 16-bit V = 64 cases run the same inputs as tests/test_hostemu.py's
    # bounds-checked host build of the kernels, which finds them in bounds)
    w = _small(V, 24, dtype, seed=V + int(dtype == torch.bfloat16) * 7)
    out = PY.run_workload(w, dev)
    PY.check_rows(w, out)


@pytest.mark.parametrize("what", ["min_p", "typical", "typical_noinf"])
def test_min_p_typical(dev, what):
    B, V = 16, 512
    w = _small(V, B, torch.float32, seed=11)
    w.temperature = torch.full((B,), 0.8)
    if what == "min_p":
        w.min_p = torch.linspace(0.01, 0.9, B)
    elif what == "typical":
        w.typical_p = torch.full((B,), 0.7)           # with top-k / top-p active -> argmax fallback
    else:
        w.typical_p = torch.linspace(0.2, 0.99, B)
        w.top_k = torch.zeros(B, dtype=torch.int32)
        w.top_p = torch.ones(B)
    out = PY.run_workload(w, dev)
    PY.check_rows(w, out)


def test_strided_rows_engine_view(dev):
    """logits[:, -1, :] of a [B, T, V] tensor (qwen3_engine.py:528)."""
    g = torch.Generator().manual_seed(12)
    B, T, V = 8, 3, 5000
    big = (torch.randn((B, T, V), generator=g) * 2).to(dev)
    view = big[:, -1, :]
    from lps import SamplingParams, sample_rows
    u = torch.rand(B, generator=g)
    p = SamplingParams.build(B, dev, temperature=0.9, top_k=30, top_p=0.9)
    out = sample_rows(view, p, u.to(dev), kept_set=True)
    ref = sample_rows(view.contiguous(), p, u.to(dev), kept_set=True)
    assert torch.equal(out.tokens, ref.tokens)
    w = W.Workload("strided", view.cpu().contiguous(), torch.full((B,), 0.9), torch.full((B,), 30, dtype=torch.int32),
                   torch.full((B,), 0.9), torch.zeros(B), torch.ones(B), torch.ones(B), torch.zeros(B), torch.zeros(B),
                   None, None, u)
    PY.check_rows(w, out)


def test_nonfinite_rows_report_status(dev):
    from lps import SamplingParams, sample_rows, Sampler
    V = 300
    x = torch.randn(4, V)
    x[0, 5] = float("nan")
    x[1, :] = float("-inf")
    x[2, 7] = float("inf")
    x[3, 9] = float("nan")
    p = SamplingParams.build(4, dev, temperature=torch.tensor([1.0, 1.0, 1.0, 0.0]))
    out = sample_rows(x.to(dev), p, torch.rand(4).to(dev))
    st = out.status.cpu().tolist()
    assert st[0] == 1 and st[1] == 2 and st[2] == 1 and st[3] == 0
    assert out.tokens.cpu().tolist()[:3] == [-1, -1, -1]
    assert out.tokens.cpu().tolist()[3] == 9              # torch.argmax returns the NaN index
    with pytest.raises(RuntimeError):
        Sampler().sample_token(x[:1].to(dev), {"temperature": 1.0})


def test_chi_square_one_million_draws(dev):
    """North-star distribution test: 1e6 draws of one row vs the fp64 kept law."""
    from scipy.stats import chisquare
    from lps import SamplingParams, sample_rows
    g = torch.Generator().manual_seed(13)
    V, N = 96, 1_000_000
    row = torch.randn((1, V), generator=g) * 1.5
    params = O.RowParams(temperature=0.7, top_k=40, top_p=0.9)
    r = O.sample_row(row[0], params, [], 0.5)
    x = row.to(dev).expand(N, V)                          # stride 0 over rows
    p = SamplingParams.build(N, dev, temperature=0.7, top_k=40, top_p=0.9)
    u = torch.rand(N, device=dev)
    out = sample_rows(x, p, u)
    counts = torch.bincount(out.tokens, minlength=V).cpu().numpy()
    kept = r.kept
    assert counts[~kept].sum() == 0
    stat, pval = chisquare(counts[kept], r.probs64[kept] * N)
    _print(f"chi-square 1e6 draws: kept={int(kept.sum())} stat={stat:.1f} p={pval:.3g}")
    assert pval > 1e-4


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_chi_square_draws_across_chunks(dev, dtype):
    """1e6 draws of one full-vocabulary nucleus row (sampling.py:84-85 draw over
    the top-p set of :158-185) vs the fp64 kept law, in each input dtype.  The
    kept set is spikes spread over the whole row (values 12 + k/16, exact in
    every dtype), so each draw crosses the row-group kernel's chunks: the
    chunks' candidate lists, the merged regions and the draw's rescan.  Every
    row must stay on the fast kernel (no deferral)."""
    from scipy.stats import chisquare
    from lps import SamplingParams, sample_rows
    g = torch.Generator().manual_seed(17)
    V, N = 151936, 1_000_000
    row = torch.randn((1, V), generator=g)
    spikes = torch.linspace(97, V - 101, 64).long()
    row[0, spikes] = 12.0 + torch.arange(64, dtype=torch.float32) / 16
    row = row.to(dtype)
    params = O.RowParams(temperature=1.0, top_k=0, top_p=0.9)
    r = O.sample_row(row[0], params, [], 0.5)
    kept = r.kept
    # closed form: the 34 largest spikes hold 0.89535 of the row's mass and 35
    # hold 0.90270, so top-p keeps the 35 largest (the first past 0.9 kept)
    assert np.array_equal(np.nonzero(kept)[0], spikes[29:].numpy())
    x = row.to(dev).expand(N, V)                          # stride 0 over rows
    p = SamplingParams.build(N, dev, temperature=1.0, top_p=0.9)
    u = torch.rand(N, device=dev, generator=torch.Generator(device=dev).manual_seed(5))
    out = sample_rows(x, p, u)
    assert int(out.row_path.ne(0).sum().item()) == 0
    assert int(out.status.ne(0).sum().item()) == 0
    counts = torch.bincount(out.tokens, minlength=V).cpu().numpy()
    assert counts[~kept].sum() == 0
    stat, pval = chisquare(counts[kept], r.probs64[kept] * N)
    _print(f"chi-square 1e6 draws, V={V} {dtype}: kept={int(kept.sum())} stat={stat:.1f} p={pval:.3g}")
    assert pval > 1e-4


def test_sampler_drop_in_matches_oracle(dev):
    """Sampler.sample_token with the reference call shape: one override dict and
    one shared history for the whole batch (sampling.py:51-85)."""
    from lps import Sampler, SamplingConfig
    g = torch.Generator().manual_seed(14)
    B, V = 6, 3000
    x = torch.randn((B, V), generator=g) * 2
    hist = [5, 9, 9, 2999, 3000, -1]
    u = torch.rand(B, generator=g)
    s = Sampler(SamplingConfig(temperature=0.8, top_k=20, top_p=0.85, repetition_penalty=1.2))
    tok = s.sample_token(x.to(dev), None, hist, uniforms=u.to(dev)).cpu()
    for i in range(B):
        r = O.sample_row(x[i], O.RowParams(0.8, 20, 0.85, repetition_penalty=1.2), hist, float(u[i]))
        assert PY.draw_ok(r.z, r.kept, float(u[i]), int(tok[i]))
    tg = s.sample_token(x.to(dev), {"temperature": 0.0}, hist).cpu()
    for i in range(B):
        assert int(tg[i]) == O.sample_row(x[i], O.RowParams(0.0, repetition_penalty=1.2), hist).token


def _mirostat_kept(x_row, T, k):
    z = (x_row.float() / T).reshape(1, -1)
    return O.apply_top_k(z, k).reshape(-1) if k > 0 else z.reshape(-1)


def test_mirostat_entropy(dev):
    """sampling.py:240-279: the entropy update and the drawn token, against
    mirostat_v2_ref (the token through its interval of the kept-set CDF)."""
    from lps import Sampler
    g = torch.Generator().manual_seed(15)
    x = torch.randn((1, 2000), generator=g) * 2
    s = Sampler()
    for u in (0.3, 0.01, 0.97):
        tok, prev = s.sample_mirostat_v2(x.to(dev), {"temperature": 0.9}, None, uniforms=torch.tensor([u], device=dev))
        ref_tok, ref_prev, k = O.mirostat_v2_ref(x[0], 0.9, 5.0, 0.1, None, u)
        assert abs(prev - ref_prev) < 1e-4
        z = _mirostat_kept(x[0], 0.9, k)
        kept = torch.isfinite(z).numpy()
        assert PY.draw_ok(z, kept, u, int(tok)), (u, int(tok), ref_tok, k)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_entropy_on_the_row_group_kernel(dev, dtype):
    """The entropy output of pure rows with the draw skipped (the first call
    of sample_mirostat_v2, sampling.py:240-279), and of nucleus rows that
    draw, at c2's shape (B = 64, V = 151936: four chunks per row, chunk
    references up to several octaves apart): every row finishes on the
    row-group kernel, H of softmax(x / T) within 2e-5 of the fp64 value, and
    the nucleus rows' draws still match the oracle."""
    from lps import SamplingParams, sample_rows
    w = W.c2()
    x = w.logits.to(dtype)
    B = w.B
    T = w.temperature.clamp(min=0.3)
    params = SamplingParams.build(B, dev, temperature=T.to(dev))
    out = sample_rows(x.to(dev), params, None, entropy=True, skip_draw=True)
    assert (out.row_path.cpu() == 0).all(), out.row_path.cpu().tolist()
    H = out.entropy.cpu().double()
    z = x.double() / T.double().view(-1, 1)
    href = -(torch.softmax(z, 1) * torch.log_softmax(z, 1)).sum(1)
    err = (H - href).abs() / href.abs().clamp(min=1.0)
    assert float(err.max()) <= 2e-5, (int(err.argmax()), float(H[err.argmax()]), float(href[err.argmax()]))
    # nucleus rows that also draw, with the entropy asked for
    wn = W.c2()
    wn.logits = x
    wn.temperature = T
    wn.top_k = torch.zeros(B, dtype=torch.int32)
    wn.histories = wn.hist_len = None   # (the entropy is of the penalised logits: compare unpenalised rows)
    outn = PY.run_workload(wn, dev, entropy=True)
    assert (outn.row_path.cpu() == 0).all(), outn.row_path.cpu().tolist()
    Hn = outn.entropy.cpu().double()
    assert float(((Hn - href).abs() / href.abs().clamp(min=1.0)).max()) <= 2e-5
    PY.check_rows(wn, outn)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_min_p_on_the_row_group_kernel(dev, dtype):
    """min-p without top-k (sampling.py:187-205) at c2's shape (B = 64, V =
    151936: four chunks per row, with c2's penalties), alone and after top-p,
    min_p from 1e-3 to 1; and typical-p after top-p / min-p, which keeps the
    argmax (sampling.py:231-234).  The row-group kernel takes these rows
    (region 1 covers the bins that can hold the min-p boundary and the
    finaliser applies the general kernel's test to the sorted candidates):
    at most 2 of the 64 are deferred, and every kept set and draw equals the
    oracle's."""
    from tests.test_gpu_stream import _deferral_reasons
    w = W.c2_minp(dtype)
    B = w.B
    out = PY.run_workload(w, dev)
    off = (out.row_path.cpu() != 0).nonzero().flatten().tolist()
    print(f"min-p rows {dtype}: off the row-group kernel {off}, reasons {_deferral_reasons(out, dev, B)}", flush=True)
    assert len(off) <= 2
    rep = PY.check_rows(w, out)
    print(f"min-p rows {dtype}: {rep}", flush=True)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_typical_p_full_rows_on_the_row_group_kernel(dev, dtype):
    """Typical-p without top-k / top-p / min-p (sampling.py:207-238) at c2's
    shape (four chunks per row, c2's penalties): the cut z - zmax >= lnZ -
    exp(H) typical_p from the row's entropy over the chunks, rows whose cut
    keeps every logit (run as pure rows), rows whose cut keeps nothing and rows
    holding -inf (the argmax).  At most 2 of the 64 rows are deferred; kept sets
    and draws equal the oracle's."""
    from tests.test_gpu_stream import _deferral_reasons
    w = W.c2_typical(dtype)
    B = w.B
    out = PY.run_workload(w, dev)
    off = (out.row_path.cpu() != 0).nonzero().flatten().tolist()
    print(f"typical rows {dtype}: off the row-group kernel {off}, reasons {_deferral_reasons(out, dev, B)}",
          flush=True)
    assert len(off) <= 2
    rep = PY.check_rows(w, out)
    print(f"typical rows {dtype}: {rep}", flush=True)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_top_k_past_the_lists_on_the_row_group_kernel(dev, dtype):
    """top_k from 257 to V - 1 without top-p (sampling.py:139-156) at c2's
    shape (four chunks per row, c2's penalties): the k-th largest located by
    the chunks' merged byte counts, its bin's elements as candidates, every
    tie of the k-th value kept; typical-p after it keeps the argmax.  Every
    row with k <= 5000 stays on the row-group kernel; rows whose k-th largest
    lies in dense bins (k = 20000: counts saturate, candidates overflow) or
    under the histogram (k = V - 1) are deferred to the general kernel.  Kept
    sets and draws equal the oracle's."""
    from tests.test_gpu_stream import _deferral_reasons
    w = W.c2_bigk(dtype)
    B = w.B
    w.top_k[3::7] = 20000
    w.top_k[4::7] = 151935
    out = PY.run_workload(w, dev)
    off = (out.row_path.cpu() != 0).nonzero().flatten().tolist()
    print(f"large top-k rows {dtype}: off the row-group kernel {off}, reasons {_deferral_reasons(out, dev, B)}",
          flush=True)
    assert not set(off) & set((w.top_k <= 5000).nonzero().flatten().tolist())
    rep = PY.check_rows(w, out)
    print(f"large top-k rows {dtype}: {rep}", flush=True)


def test_mirostat_long_low_entropy_loop(dev):
    """A peaked row (entropy below tau) makes prev grow every step, so
    k = int(exp(prev)) passes the vocabulary size; the reference's top-k
    clamps it (sampling.py:151) and sampling goes on.  60 steps against the
    oracle, token by token through the CDF interval."""
    from lps import Sampler
    g = torch.Generator().manual_seed(16)
    V = 500
    x = torch.randn((1, V), generator=g) * 6
    s = Sampler()
    prev = rprev = None
    ks = []
    for step in range(60):
        u = float(torch.rand((), generator=g))
        tok, prev = s.sample_mirostat_v2(x.to(dev), {"temperature": 1.0, "mirostat_eta": 0.5}, prev,
                                         uniforms=torch.tensor([u], device=dev))
        _, rprev, k = O.mirostat_v2_ref(x[0], 1.0, 5.0, 0.5, rprev, u)
        assert abs(prev - rprev) < 1e-3 * max(1.0, abs(rprev)), (step, prev, rprev)
        z = _mirostat_kept(x[0], 1.0, min(k, V))
        assert PY.draw_ok(z, torch.isfinite(z).numpy(), u, int(tok)), (step, int(tok), k)
        ks.append(k)
    assert max(ks) > V


# ------------------------------------------------------------ speculative --


def test_verify_drafts_batched_exact(dev):
    from lps import verify_drafts_batched
    g = torch.Generator().manual_seed(16)
    K, V = 300, 777
    tp = torch.softmax(torch.randn(K, V, generator=g), -1)
    q = torch.rand(K, generator=g) * 0.01
    q[:5] = 0.0
    t = torch.randint(0, V, (K,), generator=g)
    u = torch.rand(K, generator=g) * 0.02
    ref = O.verify_drafts_ref(tp, q, t, u)
    big = torch.zeros(K, 2 * V)
    big[:, ::2] = tp                                   # strided target_probs (stride_v = 2)
    got = verify_drafts_batched(big[:, ::2].to(dev), q.to(dev), t.to(dev), u.to(dev)).cpu()
    assert got.dtype == torch.int8 and torch.equal(got, ref)
    assert 0 < int(ref.sum()) < K


def _check_spec(sw, out, residual="target"):
    n_ref, tok_ref, bits_ref, P_ref, Q_ref = O.spec_verify_ref(sw.target, sw.draft, sw.draft_tokens, sw.u_accept,
                                                               sw.u_resample, sw.temperature, sw.top_p, residual)
    P = out.p_target.cpu()
    Q = out.q_draft.cpu()
    bits = out.accept.cpu()
    n = out.n_accepted.cpu()
    tok = out.tokens.cpu()
    B, k = sw.draft_tokens.shape
    amb = 0
    for b in range(B):
        for i in range(k):
            for a, r in ((P[b, i], P_ref[b, i]), (Q[b, i], Q_ref[b, i])):
                assert abs(float(a) - float(r)) <= 1e-5 * abs(float(r)) + 1e-7, (b, i, float(a), float(r))
            if int(bits[b, i]) != int(bits_ref[b, i]):
                ratio = min(float(P_ref[b, i]) / max(float(Q_ref[b, i]), 1e-9), 1.0)
                assert abs(float(sw.u_accept[b, i]) - ratio) < 1e-5
                amb += 1
        j = k if bits[b].all() else int(torch.nonzero(bits[b] == 0)[0])
        assert int(n[b]) == j
        assert tok[b, :j].tolist() == sw.draft_tokens[b, :j].tolist()
        assert (tok[b, j + 1:] == -1).all()
        if sw.temperature <= 0:
            assert int(tok[b, j]) == int(torch.argmax(sw.target[b, j]))
        elif residual == "target" and int(n[b]) == int(n_ref[b]):
            zj = sw.target[b, j] / sw.temperature
            z = O.apply_top_p(zj.reshape(1, -1), sw.top_p).reshape(-1)
            kept = torch.isfinite(z).numpy()
            u, t = float(sw.u_resample[b, j]), int(tok[b, j])
            if not PY.draw_ok(zj, kept, u, t):
                # a top-p boundary row: the kernel keeps the fp64-exact set, which may
                # differ from the fp32 restatement within the band (parity rule 4)
                order, _, n_truth = O.top_p_truth(zj, sw.top_p)
                kt = np.zeros(kept.size, dtype=bool)
                kt[order[:n_truth]] = True
                assert O.top_p_band(zj, sw.top_p, int(kept.sum()), n_truth, PY.TOP_P_EPS), (b, j)
                assert PY.draw_ok(zj, kt, u, t), (b, j, t)
    return amb


def test_c4_spec_verify_full_size(dev):
    from lps import spec_verify
    sw = W.c4()
    out = spec_verify(sw.target.to(dev), sw.draft.to(dev), sw.draft_tokens.to(dev), sw.u_accept.to(dev),
                      sw.u_resample.to(dev), sw.temperature, sw.top_p)
    torch.cuda.synchronize()
    assert (out.status.cpu() == 0).all()
    amb = _check_spec(sw, out)
    _print(f"c4 spec: accepted={out.n_accepted.cpu().tolist()} ambiguous={amb}")


def test_spec_verify_greedy_and_leviathan(dev):
    from lps import spec_verify
    sw = W.c4(B=8, V=4000, temperature=0.0)
    out = spec_verify(sw.target.to(dev), sw.draft.to(dev), sw.draft_tokens.to(dev), sw.u_accept.to(dev),
                      sw.u_resample.to(dev), 0.0, 1.0)
    torch.cuda.synchronize()
    _check_spec(sw, out)
    sw = W.c4(B=8, V=4000, temperature=1.0, top_p=0.9)
    out = spec_verify(sw.target.to(dev), sw.draft.to(dev), sw.draft_tokens.to(dev), sw.u_accept.to(dev),
                      sw.u_resample.to(dev), 1.0, 0.9, residual="leviathan")
    torch.cuda.synchronize()
    _check_spec(sw, out, residual="leviathan")
    tok = out.tokens.cpu()
    n = out.n_accepted.cpu()
    n_ref, tok_ref, _, _, _ = O.spec_verify_ref(sw.target, sw.draft, sw.draft_tokens, sw.u_accept, sw.u_resample,
                                                1.0, 0.9, "leviathan")
    checked = 0
    for b in range(8):
        j = int(n[b])
        if j < 4:
            tp = O.spec_probs_row(sw.target[b, j], 1.0, 0.9).double()
            dp = O.spec_probs_row(sw.draft[b, j], 1.0, 0.9).double()
            t = int(tok[b, j])
            assert float(tp[t] - dp[t]) > -1e-6   # drawn where p > q
            if j == int(n_ref[b]):
                # the draw against the oracle's residual law norm(max(p - q, 0)),
                # through its CDF interval in vocabulary order
                r = torch.clamp(tp - dp, min=0.0)
                cum = torch.cumsum(r, 0) / r.sum()
                lo = float(cum[t - 1]) if t > 0 else 0.0
                u = float(sw.u_resample[b, j])
                assert lo - 1e-6 <= u < float(cum[t]) + 1e-6, (b, j, t, int(tok_ref[b, j]), u)
                checked += 1
    assert checked > 0


def test_query_token_outside_vocab_has_zero_probability(dev):
    """A query (draft) id >= V on nucleus, pure and top-k rows: probability 0,
    no logit read past the row (the accept rule then rejects, as
    verify_drafts_kernel does for such ids)."""
    from lps import SamplingParams, sample_rows
    g = torch.Generator().manual_seed(31)
    B, V = 6, 20000
    x = (torch.randn((B, V), generator=g) * 2).to(dev)
    T = torch.tensor([1.0, 0.8, 1.0, 0.7, 1.0, 0.9])
    k = torch.tensor([0, 0, 0, 0, 40, 40], dtype=torch.int32)
    p = torch.tensor([0.9, 0.95, 1.0, 1.0, 0.9, 1.0])
    q = torch.tensor([V, V + 7, V, 2**40, V, V + 1], dtype=torch.int64)
    params = SamplingParams.build(B, dev, temperature=T.to(dev), top_k=k.to(dev), top_p=p.to(dev))
    u = torch.rand(B, generator=g).to(dev)
    a = sample_rows(x, params, u, query_tokens=q.to(dev))
    ok = sample_rows(x, params, u, query_tokens=torch.zeros(B, dtype=torch.int64, device=dev))
    torch.cuda.synchronize(dev)
    assert (a.query_prob.cpu() == 0).all()
    assert torch.equal(a.tokens, ok.tokens)
    assert (a.status.cpu() == 0).all()


@pytest.mark.parametrize("residual", ["target", "leviathan"])
def test_spec_verify_first_token_law(dev, residual):
    """The law of the first emitted token of one-draft speculative verification
    (speculative.py:119-174: accept the draft d ~ q with probability
    min(1, p(d) / q(d)), else resample), 1e6 requests, chi-square against its
    closed form: with the reference's resample from the target p
    (speculative.py:150-157) it is min(p, q) + (1 - sum min(p, q)) p; with the
    residual norm(max(p - q, 0)) it is p itself (the speculative sampling
    theorem)."""
    from scipy.stats import chisquare
    from lps import spec_verify
    g = torch.Generator().manual_seed(23)
    V, N = 4000, 1_000_000
    tgt = torch.randn((1, 2, V), generator=g) * 2.0
    drf = tgt[:, :1, :] + torch.randn((1, 1, V), generator=g) * 1.0
    p = torch.softmax(tgt[0, 0].double(), 0).numpy()
    q = torch.softmax(drf[0, 0].double(), 0).numpy()
    rng = np.random.default_rng(29)
    draft_tokens = torch.from_numpy(rng.choice(V, size=(N, 1), p=q))
    ua = torch.from_numpy(rng.random((N, 1), dtype=np.float32))
    ur = torch.from_numpy(rng.random((N, 2), dtype=np.float32))
    out = spec_verify(tgt.to(dev).expand(N, 2, V), drf.to(dev).expand(N, 1, V), draft_tokens.to(dev),
                      ua.to(dev), ur.to(dev), 1.0, 1.0, residual=residual)
    torch.cuda.synchronize()
    assert int(out.status.ne(0).sum().item()) == 0
    first = out.tokens[:, 0].cpu().numpy()
    m = np.minimum(p, q)
    law = p if residual == "leviathan" else m + (1.0 - m.sum()) * p
    counts = np.bincount(first, minlength=V).astype(np.float64)
    exp = law * N
    big = exp >= 20.0                                  # pooled tail below 20 expected draws
    f_obs = np.append(counts[big], counts[~big].sum())
    f_exp = np.append(exp[big], exp[~big].sum())
    stat, pval = chisquare(f_obs, f_exp)
    # the other residual's law is rejected (the test tells the two rules apart)
    other = m + (1.0 - m.sum()) * p if residual == "leviathan" else p
    o_exp = np.append(other[big] * N, other[~big].sum() * N)
    _, p_other = chisquare(f_obs, o_exp * (f_obs.sum() / o_exp.sum()))
    _print(f"spec verify first-token law ({residual}): bins={int(big.sum())}+1 stat={stat:.1f} p={pval:.3g}; "
           f"other law p={p_other:.3g}")
    assert pval > 1e-4 and p_other < 1e-6
