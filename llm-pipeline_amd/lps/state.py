"""Device-resident per-request sampling state for a continuous batcher.

The reference batcher samples row by row with each request's kwargs
(``continuous_batching.py:394-401``: ``sample_token(logits[i:i+1], kwargs)``),
reads every token back with ``.item()`` and appends it to a host list
(``:404``); the repetition-penalty input of ``sample_token``
(``generated_tokens``, ``sampling.py:125``) is never passed there, so the
penalty never fires (``qwen3_engine.py:537`` and ``batching.py:346-351`` carry
the same unused plumbing).

``SamplerState`` keeps the per-request parameters and token histories on the
GPU.  One ``lps_sample`` launch samples every active row with its own
parameters, and the kernel appends each sampled token to its row's history in
place (``LPS_FLAG_APPEND_HISTORY``), so the next step's penalties see it with
no host round trip and no per-row synchronisation.  Row ``i`` of the state is
row ``i`` of the step's logits; ``remove`` compacts the state when the batcher
drops finished requests.
"""

from __future__ import annotations

import dataclasses
from typing import Any, Dict, Iterable, Optional, Sequence

import torch

from .batch import SampleOutput, SamplingParams, sample_rows
from .sampling import SamplingConfig

_PARAM_FIELDS = [f.name for f in dataclasses.fields(SamplingParams)]


class SamplerState:
    """Per-request sampling parameters and token histories of up to
    ``max_rows`` active requests, resident on ``device``.

    ``history_capacity`` bounds the tokens kept per request (its history row);
    a full row keeps its first ``history_capacity`` tokens.  ``base_config``
    is the default ``SamplingConfig``, which per-request kwargs override as the
    reference's ``_merge_config`` does (``sampling.py:87-106``: unknown keys
    raise ``TypeError``)."""

    def __init__(self, max_rows: int, vocab_size: int, history_capacity: int, device,
                 base_config: Optional[SamplingConfig] = None):
        if max_rows < 1 or history_capacity < 1:
            raise ValueError("max_rows and history_capacity must be positive")
        self.device = torch.device(device)
        self.vocab_size = int(vocab_size)
        self.max_rows = int(max_rows)
        self.capacity = int(history_capacity)
        self.base_config = base_config or SamplingConfig()
        self.params = SamplingParams.build(self.max_rows, self.device)
        self.histories = torch.zeros((self.max_rows, self.capacity), dtype=torch.int32, device=self.device)
        self.history_lengths = torch.zeros((self.max_rows,), dtype=torch.int32, device=self.device)
        self.n = 0

    # -- requests -----------------------------------------------------------
    def config_for(self, kwargs: Optional[Dict[str, Any]]) -> SamplingConfig:
        """The request's config: the base config updated with its kwargs."""
        d = dataclasses.asdict(self.base_config)
        if kwargs:
            d.update(kwargs)
        return SamplingConfig(**d)

    def add(self, kwargs: Optional[Dict[str, Any]] = None, history: Optional[Sequence[int]] = None) -> int:
        """Append a request as the last active row; returns its row index.
        ``history`` seeds its token history (for example tokens generated
        before a preemption); it is truncated to the capacity."""
        if self.n >= self.max_rows:
            raise RuntimeError(f"SamplerState is full ({self.max_rows} rows)")
        cfg = self.config_for(kwargs)
        i = self.n
        for name in _PARAM_FIELDS:
            v = getattr(cfg, name)
            getattr(self.params, name)[i] = int(v) if name == "top_k" else float(v)
        h = list(history or [])[: self.capacity]
        if h:
            self.histories[i, : len(h)] = torch.tensor(h, dtype=torch.int32, device=self.device)
        self.history_lengths[i] = len(h)
        self.n += 1
        return i

    def remove(self, rows: Iterable[int]) -> None:
        """Drop rows (finished requests) and close the gaps, keeping the order
        of the remaining rows, as the batcher compacts its batch."""
        drop = set(int(r) for r in rows)
        if any(r < 0 or r >= self.n for r in drop):
            raise IndexError("row out of range")
        keep = [i for i in range(self.n) if i not in drop]
        k = len(keep)
        if k < self.n and k > 0:
            idx = torch.tensor(keep, dtype=torch.int64, device=self.device)
            for name in _PARAM_FIELDS:
                t = getattr(self.params, name)
                t[:k] = t.index_select(0, idx)
            self.histories[:k] = self.histories.index_select(0, idx)
            self.history_lengths[:k] = self.history_lengths.index_select(0, idx)
        self.n = k

    # -- sampling -----------------------------------------------------------
    def _view(self) -> SamplingParams:
        return SamplingParams(*[getattr(self.params, name)[: self.n] for name in _PARAM_FIELDS])

    def sample(self, logits: torch.Tensor, uniforms: Optional[torch.Tensor] = None,
               generator: Optional[torch.Generator] = None, **kw) -> SampleOutput:
        """Sample one token for every active row from ``logits [n, V]`` (one
        launch, no synchronisation); each sampled token is appended to its
        row's history on the device.  Extra keywords go to ``sample_rows``
        (``logprobs``, ``top_logprobs``, ``allowed``, ...)."""
        if logits.dim() != 2 or logits.shape[0] != self.n or logits.shape[1] != self.vocab_size:
            raise ValueError(f"logits must be [{self.n}, {self.vocab_size}]; got {tuple(logits.shape)}")
        return sample_rows(logits, self._view(), uniforms, histories=self.histories[: self.n],
                           history_lengths=self.history_lengths[: self.n], append_history=True,
                           generator=generator, **kw)

    def history(self, row: int) -> list:
        """Row ``row``'s token history (reads it back: synchronises)."""
        n = int(self.history_lengths[row])
        return self.histories[row, :n].tolist()
