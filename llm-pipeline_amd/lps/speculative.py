"""Speculative-decoding verification on the GPU.

* ``verify_drafts_batched`` keeps the signature of
  ``src/llm_pipeline/inference/speculative_kernel.py:24-58``:
  ``accept[i] = rand_uniform[i] < min(p_i / max(q_i, 1e-9), 1)`` as int8.
* ``spec_verify`` is the accept / reject / resample block of
  ``src/llm_pipeline/inference/speculative.py:119-174`` for a batch of
  requests, from full-vocabulary target and draft logits, in one stream-ordered
  sequence of launches with no host synchronisation.
"""

from __future__ import annotations

import ctypes
import threading
from dataclasses import dataclass
from typing import Optional

import torch

from . import _device as D
from . import _lib

_WS_LOCK = threading.Lock()
_WS = {}


def _spec_workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    """Zero-filled scratch for ``lps_spec_verify``, cached per (device,
    stream): every launch leaves it ready for the next, and launches on one
    stream never overlap."""
    key = (device.index, torch.cuda.current_stream(device).cuda_stream)
    with _WS_LOCK:
        t = _WS.get(key)
        if t is None or t.numel() < nbytes:
            t = torch.zeros((max(nbytes, 1 << 20),), dtype=torch.uint8, device=device)
            _WS[key] = t
        return t


def verify_drafts_batched(target_probs: torch.Tensor, draft_probs: torch.Tensor, draft_tokens: torch.Tensor,
                          rand_uniform: torch.Tensor) -> torch.Tensor:
    """Per-position accept (1) / reject (0) decisions, ``int8 [K]``.

    ``target_probs [K, V]`` may be strided; ``draft_probs`` holds ``q(t_i)``,
    ``draft_tokens`` the drafted ids and ``rand_uniform`` pre-sampled
    uniforms.  All K positions are decided, as in the reference."""
    D.require_device(target_probs, "target_probs")
    if target_probs.dim() != 2:
        raise ValueError("target_probs must be [K, V]")
    K, V = target_probs.shape
    dev = target_probs.device
    dt = D.dtype_code(target_probs)
    q = draft_probs.to(device=dev, dtype=torch.float32).reshape(-1).contiguous()
    t = draft_tokens.to(device=dev, dtype=torch.int64).reshape(-1).contiguous()
    u = rand_uniform.to(device=dev, dtype=torch.float32).reshape(-1).contiguous()
    if q.numel() != K or t.numel() != K or u.numel() != K:
        raise ValueError("draft_probs, draft_tokens and rand_uniform must have K elements")
    out = torch.empty((K,), dtype=torch.int8, device=dev)
    with torch.cuda.device(dev):
        rc = _lib.load().lps_verify_drafts(D.ptr(target_probs), dt, K, V, target_probs.stride(0),
                                           target_probs.stride(1), D.ptr(q), D.ptr(t), D.ptr(u), D.ptr(out),
                                           D.stream_of(dev))
    _lib.check(rc, "lps_verify_drafts")
    return out


@dataclass
class SpecVerifyOutput:
    n_accepted: torch.Tensor   # int32 [B]
    tokens: torch.Tensor       # int64 [B, k+1]: accepted drafts, then the replacement/bonus, then -1
    accept: torch.Tensor       # int8 [B, k]
    p_target: torch.Tensor     # float32 [B, k]: target probability of each draft token
    q_draft: torch.Tensor      # float32 [B, k]: draft probability of each draft token
    status: torch.Tensor       # int32 [B*(2k+1)]: per-row LPS_ROW_* bits (target rows, then draft rows)


def spec_verify(target_logits: torch.Tensor, draft_logits: torch.Tensor, draft_tokens: torch.Tensor,
                u_accept: torch.Tensor, u_resample: torch.Tensor, temperature: float, top_p: float = 1.0,
                residual: str = "target") -> SpecVerifyOutput:
    """Batched accept / reject / resample.

    ``target_logits [B, k+1, V]``, ``draft_logits [B, k, V]`` (same dtype,
    vocabulary dimension contiguous), ``draft_tokens [B, k]``, ``u_accept
    [B, k]``, ``u_resample [B, k+1]``.  Both distributions are
    ``softmax(top_p(logits / T))``; ``T <= 0`` is greedy.  ``residual`` picks
    the replacement distribution at the first rejection: ``"target"`` (the
    reference, ``speculative.py:150-157``) or ``"leviathan"``
    (``norm(max(p - q, 0))``)."""
    D.require_device(target_logits, "target_logits")
    D.require_device(draft_logits, "draft_logits")
    if target_logits.dim() != 3 or draft_logits.dim() != 3:
        raise ValueError("target_logits must be [B, k+1, V] and draft_logits [B, k, V]")
    B, k1, V = target_logits.shape
    k = k1 - 1
    if k < 1 or tuple(draft_logits.shape) != (B, k, V):
        raise ValueError(f"shape mismatch: target {tuple(target_logits.shape)}, draft {tuple(draft_logits.shape)}")
    if draft_logits.dtype != target_logits.dtype:
        raise TypeError("target and draft logits must share a dtype")
    if residual not in ("target", "leviathan"):
        raise ValueError("residual must be 'target' or 'leviathan'")
    if target_logits.stride(-1) != 1:
        target_logits = target_logits.contiguous()
    if draft_logits.stride(-1) != 1:
        draft_logits = draft_logits.contiguous()
    dev = target_logits.device
    dt = D.dtype_code(target_logits)
    tok = draft_tokens.to(device=dev, dtype=torch.int64).reshape(B, k).contiguous()
    ua = u_accept.to(device=dev, dtype=torch.float32).reshape(B, k).contiguous()
    ur = u_resample.to(device=dev, dtype=torch.float32).reshape(B, k1).contiguous()
    lib = _lib.load()
    ws_bytes = lib.lps_spec_workspace_bytes(B, k, V)
    ws = _spec_workspace(dev, ws_bytes)
    out = SpecVerifyOutput(
        torch.empty((B,), dtype=torch.int32, device=dev),
        torch.empty((B, k1), dtype=torch.int64, device=dev),
        torch.empty((B, k), dtype=torch.int8, device=dev),
        torch.empty((B, k), dtype=torch.float32, device=dev),
        torch.empty((B, k), dtype=torch.float32, device=dev),
        torch.empty((B * (2 * k + 1),), dtype=torch.int32, device=dev),
    )
    a = _lib.SpecArgs()
    a.target_logits = D.ptr(target_logits)
    a.target_stride_b = target_logits.stride(0)
    a.target_stride_k = target_logits.stride(1)
    a.draft_logits = D.ptr(draft_logits)
    a.draft_stride_b = draft_logits.stride(0)
    a.draft_stride_k = draft_logits.stride(1)
    a.dtype = dt
    a.batch = B
    a.k = k
    a.vocab = V
    a.temperature = float(temperature)
    a.top_p = float(top_p)
    a.residual = _lib.LPS_RESIDUAL_TARGET if residual == "target" else _lib.LPS_RESIDUAL_LEVIATHAN
    a.draft_tokens = D.ptr(tok)
    a.u_accept = D.ptr(ua)
    a.u_resample = D.ptr(ur)
    a.n_accepted = D.ptr(out.n_accepted)
    a.tokens = D.ptr(out.tokens)
    a.accept = D.ptr(out.accept)
    a.p_target = D.ptr(out.p_target)
    a.q_draft = D.ptr(out.q_draft)
    a.row_status = D.ptr(out.status)
    a.workspace = D.ptr(ws)
    a.workspace_bytes = ws.numel()
    with torch.cuda.device(dev):
        rc = lib.lps_spec_verify(ctypes.byref(a), D.stream_of(dev))
    _lib.check(rc, "lps_spec_verify")
    return out


class SpecDecStats:
    """Counters of a speculative run (``speculative.py:181-198``)."""

    def __init__(self, rounds: int, target_calls: int, accepted: int):
        self.rounds = rounds
        self.target_calls = target_calls
        self.accepted = accepted

    def acceptance_rate(self) -> float:
        if self.rounds == 0:
            return 0.0
        return self.accepted / (self.rounds * 1.0)

    def __repr__(self) -> str:
        return f"SpecDecStats(rounds={self.rounds}, target_calls={self.target_calls}, accepted={self.accepted})"
