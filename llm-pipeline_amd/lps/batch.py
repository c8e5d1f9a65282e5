"""Batched, per-row sampling on the GPU: one ``lps_sample`` launch for a whole
decode batch with heterogeneous parameters.

The reference applies per-request parameters by calling the scalar sampler
once per row (``src/llm_pipeline/inference/continuous_batching.py:394-401``);
``sample_rows`` gives the same per-row result in one launch.
"""

from __future__ import annotations

import ctypes
import threading
from dataclasses import dataclass, fields
from typing import Iterable, Optional, Sequence

import torch

from . import _device as D
from . import _lib


@dataclass
class SamplingParams:
    """Per-row sampling parameters as device tensors of length ``B``.

    Field meanings follow ``SamplingConfig`` (reference ``sampling.py:10-37``):
    ``temperature <= 0`` is greedy, ``top_k <= 0`` and ``top_p >= 1`` are off,
    ``min_p <= 0`` and ``typical_p >= 1`` are off, ``repetition_penalty == 1``
    and zero presence / frequency penalties are off."""

    temperature: torch.Tensor
    top_k: torch.Tensor
    top_p: torch.Tensor
    min_p: torch.Tensor
    typical_p: torch.Tensor
    repetition_penalty: torch.Tensor
    presence_penalty: torch.Tensor
    frequency_penalty: torch.Tensor

    @classmethod
    def build(cls, B: int, device, temperature=1.0, top_k=0, top_p=1.0, min_p=0.0, typical_p=1.0,
              repetition_penalty=1.0, presence_penalty=0.0, frequency_penalty=0.0) -> "SamplingParams":
        """Scalars broadcast to every row; tensors are taken per row."""
        return cls(D.as_f32(temperature, B, device), D.as_i32(top_k, B, device), D.as_f32(top_p, B, device),
                   D.as_f32(min_p, B, device), D.as_f32(typical_p, B, device),
                   D.as_f32(repetition_penalty, B, device), D.as_f32(presence_penalty, B, device),
                   D.as_f32(frequency_penalty, B, device))

    @classmethod
    def from_configs(cls, configs: Sequence, device) -> "SamplingParams":
        """Tensorise a list of ``SamplingConfig`` objects (one per row)."""
        cols = {f.name: [] for f in fields(cls)}
        for c in configs:
            for name in cols:
                cols[name].append(getattr(c, name, 0.0 if "penalty" in name and name != "repetition_penalty" else 1.0))
        return cls(
            torch.tensor(cols["temperature"], dtype=torch.float32, device=device),
            torch.tensor([int(v) for v in cols["top_k"]], dtype=torch.int32, device=device),
            torch.tensor(cols["top_p"], dtype=torch.float32, device=device),
            torch.tensor(cols["min_p"], dtype=torch.float32, device=device),
            torch.tensor(cols["typical_p"], dtype=torch.float32, device=device),
            torch.tensor(cols["repetition_penalty"], dtype=torch.float32, device=device),
            torch.tensor(cols["presence_penalty"], dtype=torch.float32, device=device),
            torch.tensor(cols["frequency_penalty"], dtype=torch.float32, device=device),
        )


# the row-group kernel's largest top_k / top-N taken from its candidate lists
FAST_KMAX = 256

_WS_LOCK = threading.Lock()
_WS = {}


def workspace_for(device: torch.device, nbytes: int) -> torch.Tensor:
    """Zero-filled scratch for the fast kernel, cached per (device, stream).
    Every launch leaves it ready for the next, so it is filled only when it is
    created; launches on one stream never overlap, so they may share it."""
    dev = torch.device(device)
    key = (dev.index, torch.cuda.current_stream(dev).cuda_stream)
    with _WS_LOCK:
        t = _WS.get(key)
        if t is None or t.numel() < nbytes:
            t = torch.zeros((max(nbytes, 1 << 20),), dtype=torch.uint8, device=dev)
            _WS[key] = t
        return t


@dataclass
class SampleOutput:
    tokens: torch.Tensor                       # int64 [B]
    status: torch.Tensor                       # int32 [B], LPS_ROW_* bits
    chosen_logprob: Optional[torch.Tensor] = None   # float32 [B]
    top_logprobs: Optional[torch.Tensor] = None     # float32 [B, n]
    top_ids: Optional[torch.Tensor] = None          # int64 [B, n]
    query_prob: Optional[torch.Tensor] = None       # float32 [B]
    entropy: Optional[torch.Tensor] = None          # float32 [B]
    kept_cut: Optional[torch.Tensor] = None         # float32 [B]: scaled logit at the cut
    kept_ties: Optional[torch.Tensor] = None        # int32 [B]: kept ids at the cut (-1 = all)
    kept_count: Optional[torch.Tensor] = None       # int32 [B]
    row_path: Optional[torch.Tensor] = None         # int32 [B]: 0 fast kernel, 1 general kernel


def row_kind_flags(temperature, top_k, min_p=None, typical_p=None) -> int:
    """Row-kind hint flags for ``lps_sample`` from host-side per-row
    parameters (scalars, sequences or CPU tensors): ``LPS_FLAG_ROWS_TOPK`` when
    every row is greedy (temperature <= 0) or has top_k > 0,
    ``LPS_FLAG_ROWS_NUCLEUS`` when none is; ``LPS_FLAG_ROWS_BASIC_FILTERS``
    when ``min_p`` and ``typical_p`` are given and no row has min_p > 0,
    typical_p < 1 or top_k > 256.  Nothing is hinted from device tensors,
    whose values the host does not hold.  The hints only choose which kernels
    (and which build of the row-group kernel) a launch runs; a row that breaks
    one is still sampled exactly, by the general kernel."""
    def host(v):
        if isinstance(v, torch.Tensor):
            return v.reshape(-1) if v.device.type == "cpu" else None
        return torch.as_tensor(v).reshape(-1)
    flags = 0
    if min_p is not None and typical_p is not None:
        mp, tp, kk = host(min_p), host(typical_p), host(top_k)
        if mp is not None and tp is not None and kk is not None and not bool((mp.float() > 0).any()) \
                and not bool((tp.float() < 1).any()) and not bool((kk.long() > FAST_KMAX).any()):
            flags |= _lib.LPS_FLAG_ROWS_BASIC_FILTERS
    T, k = host(temperature), host(top_k)
    if T is None or k is None:
        return flags
    n = max(T.numel(), k.numel())
    if n == 0:
        return flags
    T = T.float().expand(n) if T.numel() == 1 else T.float()
    k = k.long().expand(n) if k.numel() == 1 else k.long()
    if T.numel() != n or k.numel() != n:
        return flags
    topk_row = ~(T > 0) | (k > 0)
    if bool(topk_row.all()):
        return flags | _lib.LPS_FLAG_ROWS_TOPK
    if not bool(topk_row.any()):
        return flags | _lib.LPS_FLAG_ROWS_NUCLEUS
    return flags


def pad_histories(histories: Iterable[Sequence[int]], device) -> tuple:
    """Per-row token lists -> padded ``int32 [B, H]`` and lengths ``int32 [B]``."""
    hs = [list(h) for h in histories]
    H = max([len(h) for h in hs] + [1])
    buf = torch.zeros((len(hs), H), dtype=torch.int32)
    lens = torch.zeros((len(hs),), dtype=torch.int32)
    for i, h in enumerate(hs):
        if h:
            buf[i, : len(h)] = torch.tensor(h, dtype=torch.int32)
        lens[i] = len(h)
    return buf.to(device), lens.to(device)


def pack_allowed(legal: torch.Tensor) -> torch.Tensor:
    """Pack a boolean legality mask ``[B, V]`` (True = legal) into the ABI's
    bit rows: ``int32 [B, ceil(V / 32)]`` whose bit ``i & 31`` of word
    ``i >> 5`` is id ``i`` (the words are read as unsigned)."""
    if legal.dim() != 2 or legal.dtype != torch.bool:
        raise ValueError("legal must be a bool tensor [B, V]")
    B, V = legal.shape
    W = (V + 31) // 32
    bits = torch.zeros((B, W * 32), dtype=torch.int64, device=legal.device)
    bits[:, :V] = legal.to(torch.int64)
    weights = torch.pow(2, torch.arange(32, device=legal.device, dtype=torch.int64))
    words = (bits.view(B, W, 32) * weights).sum(-1)
    words = torch.where(words >= 2 ** 31, words - 2 ** 32, words)  # two's complement for int32 storage
    return words.to(torch.int32).contiguous()


def allowed_from_constraint(constraint, generated_ids, tokenizer, vocab_size: int, device) -> torch.Tensor:
    """Legality bits ``int32 [1, ceil(V / 32)]`` of a reference ``LogitConstraint``
    (``constraints.py:53-80``): the constraint's own legality mask for the
    decoded prefix, which already allows every id when none is legal."""
    prefix_text = tokenizer.decode(list(generated_ids))
    legal = constraint._compute_legality_mask(prefix_text, vocab_size, tokenizer)
    return pack_allowed(legal.reshape(1, -1).to(device))


def sample_rows(logits: torch.Tensor, params: SamplingParams, uniforms: Optional[torch.Tensor] = None, *,
                histories: Optional[torch.Tensor] = None, history_lengths: Optional[torch.Tensor] = None,
                logprobs: bool = False, top_logprobs: int = 0, entropy: bool = False,
                query_tokens: Optional[torch.Tensor] = None, skip_draw: bool = False, kept_set: bool = False,
                path: str = "auto", generator: Optional[torch.Generator] = None,
                allowed: Optional[torch.Tensor] = None, append_history: bool = False,
                noalloc: bool = False, row_kind_hint: int = 0) -> SampleOutput:
    """Sample one token per row of ``logits [B, V]`` (rows may be strided, the
    vocabulary dimension must be contiguous).  Asynchronous: nothing is
    synchronised and ``status`` is returned as a device tensor.

    ``path``: ``"auto"`` runs the multi-workgroup kernels (a row they cannot
    finish exactly is sampled by the general kernel launched after them;
    ``row_path`` reports which); ``"generic"`` runs only the general
    one-workgroup-per-row kernel.

    ``allowed``: the rows' legality masks, as a bool ``[B, V]`` tensor (True =
    legal) or as packed bits ``int32 [B, W]`` (``pack_allowed``); illegal ids
    count as -inf logits, as the reference's ``LogitConstraint`` masks them
    (``constraints.py:53-80``).

    ``append_history``: the kernel also appends each row's sampled token to
    its history row in place (``histories[r, history_lengths[r]]``, then
    ``history_lengths[r] += 1``, when the row has room), so the next step's
    penalties see it without a host round trip.  ``histories`` and
    ``history_lengths`` must then be int32 device tensors used as they are
    (row-contiguous histories, contiguous lengths).

    ``row_kind_hint``: ``row_kind_flags(...)`` of the rows' host-side
    parameters, when the caller has them; it only selects the kernels a large
    batch launches (a row that breaks it is still sampled exactly).

    ``noalloc``: launch through ``lps_sample_noalloc``, which uses the
    library's own per-GPU workspace instead of a caller one and allocates
    nothing (for batches up to ``LPS_NOALLOC_WORKSPACE_BYTES`` of workspace;
    larger ones raise ``ValueError``).  Calls that overlap in time on one GPU
    must not both use it."""
    if path not in ("auto", "generic"):
        raise ValueError("path must be 'auto' or 'generic'")
    D.require_device(logits, "logits")
    if logits.dim() != 2:
        raise ValueError(f"logits must be [B, V]; got {tuple(logits.shape)}")
    if logits.stride(-1) != 1:
        logits = logits.contiguous()
    B, V = logits.shape
    dev = logits.device
    dt = D.dtype_code(logits)
    if not 0 <= top_logprobs <= _lib.LPS_MAX_TOP_LOGPROBS:
        raise ValueError(f"top_logprobs must be in [0, {_lib.LPS_MAX_TOP_LOGPROBS}]")
    if uniforms is None and not skip_draw:
        uniforms = torch.rand((B,), device=dev, dtype=torch.float32, generator=generator)
    if uniforms is not None:
        uniforms = uniforms.to(device=dev, dtype=torch.float32).reshape(-1).contiguous()
        if uniforms.numel() != B:
            raise ValueError("uniforms must hold one value per row")
    tokens = torch.empty((B,), dtype=torch.int64, device=dev)
    status = torch.empty((B,), dtype=torch.int32, device=dev)
    out = SampleOutput(tokens, status)
    out.row_path = torch.empty((B,), dtype=torch.int32, device=dev)
    if logprobs:
        out.chosen_logprob = torch.empty((B,), dtype=torch.float32, device=dev)
    if top_logprobs:
        out.top_logprobs = torch.empty((B, top_logprobs), dtype=torch.float32, device=dev)
        out.top_ids = torch.empty((B, top_logprobs), dtype=torch.int64, device=dev)
    if entropy:
        out.entropy = torch.empty((B,), dtype=torch.float32, device=dev)
    if kept_set:
        out.kept_cut = torch.empty((B,), dtype=torch.float32, device=dev)
        out.kept_ties = torch.empty((B,), dtype=torch.int32, device=dev)
        out.kept_count = torch.empty((B,), dtype=torch.int32, device=dev)
    if query_tokens is not None:
        query_tokens = query_tokens.to(device=dev, dtype=torch.int64).reshape(-1).contiguous()
        out.query_prob = torch.empty((B,), dtype=torch.float32, device=dev)
    if append_history:
        if histories is None or history_lengths is None:
            raise ValueError("append_history needs histories and history_lengths")
        if (histories.dtype != torch.int32 or histories.device != dev or histories.dim() != 2
                or histories.stride(1) != 1 or history_lengths.dtype != torch.int32
                or history_lengths.device != dev or not history_lengths.is_contiguous()):
            raise ValueError("append_history writes the histories in place: they must be int32 tensors on "
                             "the logits' device (row-contiguous [B, H], contiguous lengths [B])")
    if histories is not None:
        histories = histories.to(device=dev, dtype=torch.int32)
        if histories.dim() != 2 or histories.shape[0] != B:
            raise ValueError("histories must be int32 [B, H]")
        if histories.stride(1) != 1:
            histories = histories.contiguous()
        if history_lengths is None:
            history_lengths = torch.full((B,), histories.shape[1], dtype=torch.int32, device=dev)
        history_lengths = history_lengths.to(device=dev, dtype=torch.int32).contiguous()
    if allowed is not None:
        if allowed.dtype == torch.bool:
            if tuple(allowed.shape) != (B, V):
                raise ValueError(f"allowed must be bool [{B}, {V}]; got {tuple(allowed.shape)}")
            allowed = pack_allowed(allowed.to(dev))
        else:
            allowed = allowed.to(device=dev, dtype=torch.int32)
            if allowed.dim() != 2 or allowed.shape[0] != B or allowed.shape[1] < (V + 31) // 32:
                raise ValueError(f"allowed bits must be int32 [{B}, >= {(V + 31) // 32}]")
            allowed = allowed.contiguous()
    p = params
    a = _lib.SampleArgs()
    a.logits = D.ptr(logits)
    a.dtype = dt
    a.num_rows = B
    a.vocab = V
    a.rows_inner = 1
    a.stride_outer = logits.stride(0)
    a.stride_inner = 0
    a.temperature = D.ptr(p.temperature)
    a.top_k = D.ptr(p.top_k)
    a.top_p = D.ptr(p.top_p)
    a.min_p = D.ptr(p.min_p)
    a.typical_p = D.ptr(p.typical_p)
    a.repetition_penalty = D.ptr(p.repetition_penalty)
    a.presence_penalty = D.ptr(p.presence_penalty)
    a.frequency_penalty = D.ptr(p.frequency_penalty)
    a.history = D.ptr(histories)
    a.history_stride = histories.stride(0) if histories is not None else 0
    a.history_len = D.ptr(history_lengths) if histories is not None else 0
    a.uniforms = D.ptr(uniforms)
    a.query_tokens = D.ptr(query_tokens)
    a.query_inner = 1 if query_tokens is not None else 0
    a.query_prob = D.ptr(out.query_prob)
    a.tokens = D.ptr(tokens)
    a.chosen_logprob = D.ptr(out.chosen_logprob)
    a.top_logprobs = D.ptr(out.top_logprobs)
    a.top_ids = D.ptr(out.top_ids)
    a.n_top = top_logprobs
    a.entropy = D.ptr(out.entropy)
    a.row_status = D.ptr(status)
    a.skip_draw = 1 if skip_draw else 0
    a.kept_cut = D.ptr(out.kept_cut)
    a.kept_ties = D.ptr(out.kept_ties)
    a.kept_count = D.ptr(out.kept_count)
    a.row_path = D.ptr(out.row_path)
    hints = _lib.LPS_FLAG_ROWS_TOPK | _lib.LPS_FLAG_ROWS_NUCLEUS | _lib.LPS_FLAG_ROWS_BASIC_FILTERS
    if row_kind_hint & ~hints:
        raise ValueError("row_kind_hint takes LPS_FLAG_ROWS_TOPK / LPS_FLAG_ROWS_NUCLEUS / "
                         "LPS_FLAG_ROWS_BASIC_FILTERS only")
    a.flags = ((0 if path == "auto" else _lib.LPS_FLAG_GENERIC) | (_lib.LPS_FLAG_APPEND_HISTORY if append_history else 0)
               | row_kind_hint)
    if noalloc:
        a.workspace = 0
        a.workspace_bytes = 0
    else:
        ws_bytes = _lib.load().lps_workspace_bytes(B, V, a.flags)
        ws = workspace_for(dev, ws_bytes) if ws_bytes else None
        a.workspace = D.ptr(ws)
        a.workspace_bytes = ws.numel() if ws is not None else 0
    a.allowed = D.ptr(allowed)
    a.allowed_stride = allowed.stride(0) if allowed is not None else 0
    entry = "lps_sample_noalloc" if noalloc else "lps_sample"
    with torch.cuda.device(dev):
        rc = getattr(_lib.load(), entry)(ctypes.byref(a), D.stream_of(dev))
    _lib.check(rc, entry)
    return out


def raise_on_status(status: torch.Tensor) -> None:
    """Raise what the reference raises for rows the kernel could not sample
    (``torch.multinomial`` rejects NaN / inf / empty distributions)."""
    bad = int(status.ne(0).any().item())
    if not bad:
        return
    raise RuntimeError("probability tensor contains either `inf`, `nan` or element < 0")
