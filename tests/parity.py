"""Parity checks of GPU sampler outputs against the CPU oracle, shared by the GPU
tests, ``__graft_entry__.smoke()`` and the bench's self-check.

Bars:
* greedy tokens, top-k kept sets: bit-exact;
* top-p kept sets: the GPU's kept set equals the fp64-exact keep rule except
  decisions within ``TOP_P_EPS`` of top_p; against the reference restatement
  (fp32 softmax + fp32 cumsum) it is bit-exact except where the reference's
  own rounding at a position exceeds that position's distance to top_p
  (counted and reported as reference-rounding rows);
* draws: the GPU token's interval of the fp64 kept-set CDF in sorted order
  (z descending, ties lower index first) contains the uniform, up to
  ``DRAW_EPS`` (inverse CDF over the same kept set);
* logprobs / probabilities: |gpu - ref| <= LP_RTOL * |ref| + LP_ATOL.
"""

from __future__ import annotations

import numpy as np
import torch

from oracle import reference_semantics as O

TOP_P_EPS = 2e-6
DRAW_EPS = 2e-6
LP_RTOL = 1e-5
LP_ATOL = 2e-6


def gpu_kept_mask(z: torch.Tensor, cut: float, ties: int) -> np.ndarray:
    """Rebuild the kept set from the kernel's (cut, ties) descriptor over the
    oracle's bit-identical scaled logits z."""
    zz = z.numpy()
    c = np.float32(cut)
    gt = zz > c
    eq = zz == c
    if ties < 0:
        return (gt | eq) & np.isfinite(zz)
    rank = np.cumsum(eq) - 1
    return (gt | (eq & (rank < ties))) & np.isfinite(zz)


def row_params(w, i) -> O.RowParams:
    return O.RowParams(temperature=float(w.temperature[i]), top_k=int(w.top_k[i]), top_p=float(w.top_p[i]),
                       min_p=float(w.min_p[i]), typical_p=float(w.typical_p[i]),
                       repetition_penalty=float(w.rep[i]), presence_penalty=float(w.pres[i]),
                       frequency_penalty=float(w.freq[i]))


def draw_ok(z: torch.Tensor, kept: np.ndarray, u: float, tok: int, eps: float = DRAW_EPS) -> bool:
    """The uniform lies in the token's interval of the fp64 kept-set CDF in
    sorted order (z descending, ties lower index first), up to ``eps``."""
    if tok < 0 or tok >= kept.size or not kept[tok]:
        return False
    zz = z.double().numpy()
    m = zz[kept].max()
    e = np.where(kept, np.exp(np.where(kept, zz, m) - m), 0.0)
    Z = e.sum()
    zt = zz[tok]
    before = (zz > zt) | ((zz == zt) & (np.arange(zz.size) < tok))
    lo = e[before & kept].sum() / Z
    hi = lo + e[tok] / Z
    return lo - eps <= u < hi + eps


class RowReport:
    def __init__(self):
        self.rows = 0
        self.band_keep = 0
        self.band_draw = 0
        self.exact_tokens = 0

    def __repr__(self):
        return (f"rows={self.rows} exact_tokens={self.exact_tokens} ref_rounding_rows={self.band_keep} "
                f"draw_band_rows={self.band_draw}")


def check_rows(w, out, rows=None, report: RowReport = None, lp=False) -> RowReport:
    """Compare GPU outputs of workload ``w`` with the oracle row by row."""
    report = report or RowReport()
    rows = range(w.B) if rows is None else rows
    tok = out.tokens.cpu()
    st = out.status.cpu()
    cut = out.kept_cut.cpu() if out.kept_cut is not None else None
    ties = out.kept_ties.cpu() if out.kept_ties is not None else None
    cnt = out.kept_count.cpu() if out.kept_count is not None else None
    for i in rows:
        p = row_params(w, i)
        r = O.sample_row(w.logits[i], p, w.row_history(i), float(w.uniforms[i]))
        report.rows += 1
        assert int(st[i]) == 0, f"row {i}: status {int(st[i])}"
        if r.greedy:
            assert int(tok[i]) == r.token, f"row {i}: greedy {int(tok[i])} != {r.token}"
            report.exact_tokens += 1
        else:
            assert cut is not None
            gk = gpu_kept_mask(r.z, float(cut[i]), int(ties[i]))
            assert int(cnt[i]) == int(gk.sum()), f"row {i}: kept_count {int(cnt[i])} vs mask {int(gk.sum())}"
            if not np.array_equal(gk, r.kept):
                # only top-p boundary decisions may differ
                assert p.min_p <= 0 and p.typical_p >= 1, f"row {i}: kept set differs"
                zk = O.apply_top_k(r.z.reshape(1, -1), p.top_k).reshape(-1)
                _, _, n_truth = O.top_p_truth(zk, p.top_p)
                ng, no = int(gk.sum()), int(r.kept.sum())
                assert O.top_p_band(zk, p.top_p, ng, n_truth, TOP_P_EPS), \
                    f"row {i}: kept {ng} vs fp64 truth {n_truth} outside the band"
                assert O.top_p_reference_rounding(zk, p.top_p, ng, no, TOP_P_EPS), \
                    f"row {i}: kept {ng} vs reference {no} not explained by reference rounding"
                report.band_keep += 1
            t = int(tok[i])
            assert draw_ok(r.z, gk, float(w.uniforms[i]), t), f"row {i}: draw {t} not at u={float(w.uniforms[i])}"
            if t == r.token:
                report.exact_tokens += 1
            else:
                report.band_draw += 1
        if lp and out.chosen_logprob is not None:
            zpre = r.z
            ch, vals, ids = O.logprobs_row(zpre, int(tok[i]), w.n_top)
            g = float(out.chosen_logprob[i])
            assert abs(g - ch) <= LP_RTOL * abs(ch) + LP_ATOL, f"row {i}: logprob {g} vs {ch}"
            if w.n_top:
                gi = out.top_ids[i].cpu().numpy()
                gv = out.top_logprobs[i].cpu().numpy()
                assert np.array_equal(gi, ids), f"row {i}: top ids differ"
                assert np.all(np.abs(gv - vals) <= LP_RTOL * np.abs(vals) + LP_ATOL), f"row {i}: top logprobs"
    return report


def run_workload(w, dev, path="auto", **kw):
    from lps import SamplingParams, row_kind_flags, sample_rows
    kw.setdefault("row_kind_hint", row_kind_flags(w.temperature, w.top_k, w.min_p, w.typical_p))
    p = SamplingParams(w.temperature.to(dev), w.top_k.to(dev), w.top_p.to(dev), w.min_p.to(dev),
                       w.typical_p.to(dev), w.rep.to(dev), w.pres.to(dev), w.freq.to(dev))
    hist = w.histories.to(dev) if w.histories is not None else None
    hl = w.hist_len.to(dev) if w.hist_len is not None else None
    out = sample_rows(w.logits.to(dev), p, w.uniforms.to(dev), histories=hist, history_lengths=hl,
                      logprobs=w.logprobs, top_logprobs=w.n_top, kept_set=True, path=path, **kw)
    torch.cuda.synchronize(dev)
    return out
