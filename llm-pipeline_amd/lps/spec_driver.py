"""Speculative-decoding drivers over a batch of requests.

The reference's drivers (``src/llm_pipeline/inference/speculative.py``) run one
request at a time in Python:

* ``speculative_decode`` (``:68-178``): ``k`` draft steps, one target forward,
  then an accept loop that reads every decision back with ``.item()``;
* ``mtp_speculative_decode`` (``:206-280``): the main model's next token, an
  MTP-head draft, a second main pass that verifies it.

Here the same loops advance ``B`` requests together.  Every draft step samples
all rows in one ``lps_sample`` launch; every round verifies all rows in one
``lps_spec_verify`` launch (accept / reject / replacement or bonus, on the GPU);
the host reads back only how many tokens each row emitted.  Requests leave the
batch as they finish (``eos`` or ``max_new_tokens``).  ``speculative_decode``
and ``mtp_speculative_decode`` keep the reference signatures (``[1, T]``
prompts) on top of the batched loops.

Model callables follow the reference's contract: full-sequence forwards,
``forward(tokens [b, L]) -> logits [b, L, V]`` (the MTP main model also returns
``hidden [b, L, H]``), causal, so right padding does not change the logits of
real positions.  A callable may keep its own KV cache keyed by the prefix.

Randomness: each round takes its uniforms from ``uniforms(round, rows)`` when
given (``rows``: the int64 request indices still active, on the host), else
from ``torch.rand`` on the prompts' device (``generator`` optional).  Two-model
rounds take ``3k + 1`` uniforms per row (``k`` draft draws, ``k`` accept tests,
``k + 1`` replacement / bonus draws); MTP rounds take 3 (next token, draft,
accept test).  Draws are inverse CDFs in sorted order (scaled logit descending,
ties lower index first), as ``lps_sample``
defines them; the reference's ``torch.multinomial`` / ``torch.rand`` draw from
the same distributions.
"""

from __future__ import annotations

from typing import Callable, List, Optional, Sequence, Tuple, Union

import torch

from . import _device as D
from .batch import SamplingParams, row_kind_flags, sample_rows
from .speculative import SpecDecStats, spec_verify

Prompts = Union[torch.Tensor, Sequence[torch.Tensor]]


def _prompt_list(prompts: Prompts) -> List[torch.Tensor]:
    if isinstance(prompts, torch.Tensor):
        if prompts.dim() != 2:
            raise ValueError(f"prompts must be [B, T] or a list of 1-D tensors; got {tuple(prompts.shape)}")
        rows = [prompts[i] for i in range(prompts.shape[0])]
    else:
        rows = list(prompts)
    if not rows:
        raise ValueError("no prompts")
    out = []
    for p in rows:
        D.require_device(p, "prompt")
        if p.dim() != 1 or p.numel() < 1:
            raise ValueError("each prompt must be a non-empty 1-D token tensor")
        out.append(p.to(torch.int64))
    dev = out[0].device
    if any(p.device != dev for p in out):
        raise ValueError("prompts must share one device")
    return out


def _padded(seqs: List[torch.Tensor], extra: int, pad_token_id: int) -> Tuple[torch.Tensor, torch.Tensor]:
    """``[b, max_len + extra]`` right-padded tokens and the lengths ``[b]``."""
    dev = seqs[0].device
    lens = torch.tensor([s.numel() for s in seqs], dtype=torch.int64)
    x = torch.full((len(seqs), int(lens.max()) + extra), pad_token_id, dtype=torch.int64, device=dev)
    for i, s in enumerate(seqs):
        x[i, : s.numel()] = s
    return x, lens.to(dev)


def _plain_params(n: int, temperature: float, dev) -> SamplingParams:
    """``softmax(logits / T)`` with nothing filtered (``speculative.py:50-57``);
    ``T <= 0`` samples the argmax."""
    return SamplingParams.build(n, dev, temperature=max(float(temperature), 0.0), top_k=0, top_p=1.0)


def _plain_hint(temperature: float) -> int:
    """The row-kind hint of ``_plain_params`` rows (every row alike)."""
    return row_kind_flags(max(float(temperature), 0.0), 0, 0.0, 1.0)


def _round_uniforms(uniforms, generator, rnd: int, rows: List[int], width: int, dev) -> torch.Tensor:
    if uniforms is not None:
        u = torch.as_tensor(uniforms(rnd, torch.tensor(rows, dtype=torch.int64)), dtype=torch.float32)
        if tuple(u.shape) != (len(rows), width):
            raise ValueError(f"uniforms(round, rows) must return [{len(rows)}, {width}]; got {tuple(u.shape)}")
        return u.to(dev)
    return torch.rand((len(rows), width), device=dev, generator=generator)


def _logits_on(x: torch.Tensor, dev) -> torch.Tensor:
    return x if x.device == dev else x.to(dev)


def speculative_decode_batched(target_forward: Callable[[torch.Tensor], torch.Tensor],
                               draft_forward: Callable[[torch.Tensor], torch.Tensor], prompts: Prompts,
                               max_new_tokens: int, k: int = 4, temperature: float = 1.0,
                               eos_token_id: Optional[int] = None, pad_token_id: int = 0, *,
                               uniforms=None, generator: Optional[torch.Generator] = None,
                               ) -> Tuple[List[torch.Tensor], List[SpecDecStats]]:
    """Two-model speculative decoding (``speculative.py:68-178``) for ``B``
    requests at once.  Returns each request's generated tokens (``int64 [n_i]``,
    prompt excluded) and its ``SpecDecStats``.  Per request the loop is the
    reference's: it runs while fewer than ``max_new_tokens`` tokens are emitted
    and may overshoot within the last round; an accepted ``eos`` ends the
    request right after it.

    The sequences live in one device buffer; per round the host reads back
    only each active request's emitted count, its stop flag and its accepted
    count (one small copy)."""
    if k < 1:
        raise ValueError("k must be >= 1")
    seqs = _prompt_list(prompts)
    dev = seqs[0].device
    B = len(seqs)
    plen = [s.numel() for s in seqs]
    cap = max(plen) + max(int(max_new_tokens), 0) + 2 * k + 2
    buf = torch.full((B, cap), pad_token_id, dtype=torch.int64, device=dev)
    for i, s in enumerate(seqs):
        buf[i, : plen[i]] = s
    lens = list(plen)                                   # host copy of every request's length
    rounds = [0] * B
    calls = [0] * B
    accepted = [0] * B
    active = list(range(B))
    kk = torch.arange(k + 1, device=dev)
    rnd = 0
    idx = None
    idx_rows: List[int] = []
    while True:
        rows = [i for i in active if lens[i] - plen[i] < max_new_tokens]
        if not rows:
            break
        A = len(rows)
        if rows != idx_rows:
            idx_rows = rows
            idx = torch.tensor(rows, dtype=torch.int64, device=dev)
        u = _round_uniforms(uniforms, generator, rnd, rows, 3 * k + 1, dev)
        rnd += 1
        for i in rows:
            rounds[i] += 1
            calls[i] += 1
        L = max(lens[i] for i in rows)
        ld = torch.tensor([lens[i] for i in rows], dtype=torch.int64, device=dev)
        x = buf[idx, : L + k]                                                  # [A, L + k]
        x = torch.where(torch.arange(L + k, device=dev).unsqueeze(0) < ld.unsqueeze(1), x, pad_token_id)
        ar = torch.arange(A, device=dev)
        params = _plain_params(A, temperature, dev)
        hint = _plain_hint(temperature)
        d_all = None                                                          # [A, k, V] draft rows
        d_tok = torch.empty((A, k), dtype=torch.int64, device=dev)
        for s in range(k):
            logits = _logits_on(draft_forward(x[:, : L + s]), dev)
            if d_all is None:
                d_all = torch.empty((A, k, logits.shape[-1]), dtype=logits.dtype, device=dev)
            d_all[:, s] = logits[ar, ld - 1 + s]
            d_tok[:, s] = sample_rows(d_all[:, s], params, u[:, s].contiguous(), row_kind_hint=hint).tokens
            x[ar, ld + s] = d_tok[:, s]
        t_logits = _logits_on(target_forward(x), dev)
        t_rows = t_logits[ar.unsqueeze(1), (ld - 1).unsqueeze(1) + kk.unsqueeze(0)]   # [A, k+1, V]
        if d_all.dtype != t_rows.dtype:
            d_all = d_all.to(t_rows.dtype)
        res = spec_verify(t_rows, d_all, d_tok, u[:, k: 2 * k].contiguous(), u[:, 2 * k:].contiguous(), temperature)
        n_acc = res.n_accepted.to(torch.int64)
        toks = res.tokens                                                     # [A, k+1], -1 past the emitted
        n_emit = n_acc + 1
        stop = torch.zeros((A,), dtype=torch.bool, device=dev)
        acc_add = n_acc
        if eos_token_id is not None:
            hit = (toks == eos_token_id) & (kk.unsqueeze(0) <= n_acc.unsqueeze(1))
            stop = hit.any(dim=1)
            first = torch.argmax(hit.to(torch.int32), dim=1)
            n_emit = torch.where(stop, first + 1, n_emit)
            acc_add = torch.where(stop & (first < n_acc), first + 1, n_acc)
        # every slot of the round is written; only the first n_emit count
        buf[idx.unsqueeze(1), ld.unsqueeze(1) + kk.unsqueeze(0)] = toks
        back = torch.stack([n_emit, stop.to(torch.int64), acc_add], dim=1).cpu().tolist()
        still = []
        for a, i in enumerate(rows):
            ne, st, ad = back[a]
            lens[i] += int(ne)
            accepted[i] += int(ad)
            if not st:
                still.append(i)
        active = still
    outs = [buf[i, plen[i]: lens[i]].clone() for i in range(B)]
    return outs, [SpecDecStats(rounds[i], calls[i], accepted[i]) for i in range(B)]


def speculative_decode(target_forward: Callable[[torch.Tensor], torch.Tensor],
                       draft_forward: Callable[[torch.Tensor], torch.Tensor], prompt_ids: torch.Tensor,
                       max_new_tokens: int, k: int = 4, temperature: float = 1.0,
                       eos_token_id: Optional[int] = None, *, uniforms=None,
                       generator: Optional[torch.Generator] = None) -> Tuple[torch.Tensor, SpecDecStats]:
    """The reference signature (``speculative.py:68-76``): ``prompt_ids [1, T]``
    on a ROCm device; returns ``(generated [1, n], stats)``."""
    if prompt_ids.dim() != 2 or prompt_ids.shape[0] != 1:
        raise ValueError(f"prompt_ids must be shape [1, T]; got {tuple(prompt_ids.shape)}")
    outs, stats = speculative_decode_batched(target_forward, draft_forward, prompt_ids, max_new_tokens, k,
                                             temperature, eos_token_id, uniforms=uniforms, generator=generator)
    return outs[0].unsqueeze(0), stats[0]


def mtp_speculative_decode_batched(main_forward_with_hidden: Callable[[torch.Tensor], Tuple[torch.Tensor, torch.Tensor]],
                                   mtp_head: Callable[[torch.Tensor, torch.Tensor], torch.Tensor], prompts: Prompts,
                                   max_new_tokens: int, temperature: float = 1.0,
                                   eos_token_id: Optional[int] = None, pad_token_id: int = 0, *,
                                   uniforms=None, generator: Optional[torch.Generator] = None,
                                   ) -> Tuple[List[torch.Tensor], List[SpecDecStats]]:
    """MTP speculative decoding (``speculative.py:206-280``) for ``B``
    requests at once: per round one main forward, one MTP-head call and, for
    the requests still running, one verifying main forward; the draft is
    verified with ``lps_spec_verify`` (``k = 1``, no replacement token)."""
    seqs = _prompt_list(prompts)
    dev = seqs[0].device
    plen = [s.numel() for s in seqs]
    B = len(seqs)
    rounds = [0] * B
    calls = [0] * B
    accepted = [0] * B
    active = list(range(B))
    rnd = 0
    while True:
        rows = [i for i in active if seqs[i].numel() - plen[i] < max_new_tokens]
        if not rows:
            break
        A = len(rows)
        u = _round_uniforms(uniforms, generator, rnd, rows, 3, dev)
        rnd += 1
        for i in rows:
            rounds[i] += 1
            calls[i] += 1
        x, lens = _padded([seqs[i] for i in rows], 2, pad_token_id)   # room for x_next and the draft
        ar = torch.arange(A, device=dev)
        params = _plain_params(A, temperature, dev)
        hint = _plain_hint(temperature)
        logits, hidden = main_forward_with_hidden(x[:, : int(lens.max())])
        logits = _logits_on(logits, dev)
        x_next = sample_rows(logits[ar, lens - 1], params, u[:, 0].contiguous(), row_kind_hint=hint).tokens
        h_last = hidden[ar.to(hidden.device), (lens - 1).to(hidden.device)].unsqueeze(1)
        mtp_logits = _logits_on(mtp_head(h_last, x_next.to(hidden.device).unsqueeze(-1)), dev)     # [A, 1, V]
        x_draft = sample_rows(mtp_logits[:, 0], params, u[:, 1].contiguous(), row_kind_hint=hint).tokens
        x[ar, lens] = x_next
        nxt = x_next.cpu().tolist()
        verify = []
        for a, i in enumerate(rows):
            accepted[i] += 1
            seqs[i] = torch.cat([seqs[i], x_next[a: a + 1]])
            if eos_token_id is not None and nxt[a] == eos_token_id:
                continue
            if seqs[i].numel() - plen[i] >= max_new_tokens:
                continue
            verify.append(a)
        still = []
        if verify:
            va = torch.tensor(verify, dtype=torch.int64, device=dev)
            xv = x[va]
            lv = lens[va] + 1                                            # sequence with x_next
            xv[torch.arange(len(verify), device=dev), lv] = x_draft[va]
            v_logits, _ = main_forward_with_hidden(xv[:, : int(lv.max()) + 1])
            v_logits = _logits_on(v_logits, dev)
            av = torch.arange(len(verify), device=dev)
            pos = (lv - 1).unsqueeze(1) + torch.arange(2, device=dev).unsqueeze(0)
            t_rows = v_logits[av.unsqueeze(1), pos]                      # [n, 2, V]: the draft position, then past it
            d_rows = mtp_logits[va]                                       # [n, 1, V]
            if d_rows.dtype != t_rows.dtype:
                d_rows = d_rows.to(t_rows.dtype)
            res = spec_verify(t_rows, d_rows, x_draft[va].unsqueeze(1), u[va, 2:3].contiguous(),
                              torch.full((len(verify), 2), 0.5, device=dev), temperature)
            acc = res.n_accepted.cpu().tolist()
            drafts = x_draft[va].cpu().tolist()
            for b, a in enumerate(verify):
                i = rows[a]
                calls[i] += 1
                if int(acc[b]) == 1:
                    seqs[i] = torch.cat([seqs[i], x_draft[a: a + 1]])
                    accepted[i] += 1
                    if eos_token_id is not None and drafts[b] == eos_token_id:
                        continue
                still.append(i)
        active = still
    outs = [seqs[i][plen[i]:] for i in range(B)]
    return outs, [SpecDecStats(rounds[i], calls[i], accepted[i]) for i in range(B)]


def mtp_speculative_decode(main_forward_with_hidden: Callable[[torch.Tensor], Tuple[torch.Tensor, torch.Tensor]],
                           mtp_head: Callable[[torch.Tensor, torch.Tensor], torch.Tensor], prompt_ids: torch.Tensor,
                           max_new_tokens: int, temperature: float = 1.0, eos_token_id: Optional[int] = None, *,
                           uniforms=None, generator: Optional[torch.Generator] = None,
                           ) -> Tuple[torch.Tensor, SpecDecStats]:
    """The reference signature (``speculative.py:206-214``): ``prompt_ids
    [1, T]`` on a ROCm device; returns ``(generated [1, n], stats)``."""
    if prompt_ids.dim() != 2 or prompt_ids.shape[0] != 1:
        raise ValueError(f"prompt_ids must be shape [1, T]; got {tuple(prompt_ids.shape)}")
    outs, stats = mtp_speculative_decode_batched(main_forward_with_hidden, mtp_head, prompt_ids, max_new_tokens,
                                                 temperature, eos_token_id, uniforms=uniforms, generator=generator)
    return outs[0].unsqueeze(0), stats[0]
