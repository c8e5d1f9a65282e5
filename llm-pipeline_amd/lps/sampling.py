"""Drop-in ``Sampler`` / ``SamplingConfig`` for the llm-pipeline inference engine.

Interface of ``src/llm_pipeline/inference/sampling.py`` kept verbatim:
``Sampler(config)``, ``.config``, ``sample_token(logits, config_override,
generated_tokens)`` (``:51-85``), ``_merge_config`` (``:87-106``, unknown keys
raise ``TypeError``), ``sample_mirostat_v2`` (``:240-279``) and
``get_sampling_info`` (``:281-293``).  Every call runs the HIP kernels of
``liblps.so`` on the logits' device; there is no CPU path.

Additive, default-neutral extensions: ``presence_penalty``,
``frequency_penalty``, ``logprobs`` and ``top_logprobs`` config fields, and
keyword-only ``uniforms`` / ``params`` / ``histories`` / ``history_lengths``
arguments to ``sample_token``.
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Any, Dict, List, Optional

import torch

from . import _device as D
from .batch import SamplingParams, pad_histories, raise_on_status, row_kind_flags, sample_rows


@dataclass
class SamplingConfig:
    """Reference fields (``sampling.py:10-37``) plus the build's extensions."""

    temperature: float = 1.0
    top_k: int = 50
    top_p: float = 0.9
    repetition_penalty: float = 1.0
    typical_p: float = 1.0
    min_p: float = 0.0
    mirostat_tau: float = 5.0
    mirostat_eta: float = 0.1
    do_sample: bool = True
    pad_token_id: Optional[int] = None
    eos_token_id: Optional[int] = None
    presence_penalty: float = 0.0
    frequency_penalty: float = 0.0
    logprobs: bool = False
    top_logprobs: int = 0


_CONFIG_KEYS = (
    "temperature", "top_k", "top_p", "repetition_penalty", "typical_p", "min_p", "mirostat_tau",
    "mirostat_eta", "do_sample", "pad_token_id", "eos_token_id", "presence_penalty", "frequency_penalty",
    "logprobs", "top_logprobs",
)


class Sampler:
    """Centralised logits -> token sampler on MI355X."""

    def __init__(self, config: Optional[SamplingConfig] = None):
        self.config = config or SamplingConfig()
        self.last_output = None

    def sample_token(self, logits: torch.Tensor, config_override: Optional[Dict[str, Any]] = None,
                     generated_tokens: Optional[List[int]] = None, *, uniforms: Optional[torch.Tensor] = None,
                     params: Optional[SamplingParams] = None, histories: Optional[torch.Tensor] = None,
                     history_lengths: Optional[torch.Tensor] = None, generator: Optional[torch.Generator] = None,
                     allowed: Optional[torch.Tensor] = None, strict: Optional[bool] = None) -> torch.Tensor:
        """Sample next token ids ``int64 [B]`` from ``logits [B, V]``.

        As in the reference, ``generated_tokens`` is one history applied to
        every row and the repetition penalty fires only when it is non-empty
        and the penalty differs from 1.  ``params`` (per-row
        ``SamplingParams``) and ``histories`` (padded ``int32 [B, H]``)
        replace the shared values row by row.  ``uniforms`` (``[B]`` in
        [0, 1)) drive the inverse-CDF draw; when omitted they come from
        ``torch.rand`` on the logits' device.  ``allowed`` (bool ``[B, V]`` or
        packed ``int32`` bits) masks illegal ids to -inf, as a reference
        ``LogitConstraint`` applied to the logits first would.

        ``strict`` raises the reference's ``RuntimeError`` for rows
        ``torch.multinomial`` would reject (NaN / +inf / all -inf); reading the
        row status synchronises the stream once, as the engine's ``.item()``
        after every call does anyway (``qwen3_engine.py:412-420``).  The
        default (``None``) checks unless the stream is being captured into a
        graph, where the call stays stream-ordered; ``False`` never checks
        (tokens of rejected rows are -1 and ``last_output.status`` holds the
        reason)."""
        config = self._merge_config(config_override)
        D.require_device(logits, "logits")
        if logits.dim() != 2:
            raise ValueError(f"logits must be [batch_size, vocab_size]; got {tuple(logits.shape)}")
        B = logits.shape[0]
        dev = logits.device
        hint = 0
        if params is None:
            hint = row_kind_flags(config.temperature, config.top_k, config.min_p, config.typical_p)
            params = SamplingParams.build(
                B, dev, temperature=config.temperature, top_k=config.top_k, top_p=config.top_p,
                min_p=config.min_p, typical_p=config.typical_p, repetition_penalty=config.repetition_penalty,
                presence_penalty=config.presence_penalty, frequency_penalty=config.frequency_penalty)
        if histories is None and generated_tokens:
            h = torch.tensor(list(generated_tokens), dtype=torch.int32)
            histories = h.reshape(1, -1).expand(B, -1).to(dev)
            history_lengths = torch.full((B,), h.numel(), dtype=torch.int32, device=dev)
        out = sample_rows(logits, params, uniforms, histories=histories, history_lengths=history_lengths,
                          logprobs=bool(config.logprobs), top_logprobs=int(config.top_logprobs),
                          generator=generator, allowed=allowed, row_kind_hint=hint)
        self.last_output = out
        if strict is None:
            strict = not torch.cuda.is_current_stream_capturing()
        if strict:
            raise_on_status(out.status)
        return out.tokens

    def _merge_config(self, config_override: Optional[Dict[str, Any]]) -> SamplingConfig:
        """``sampling.py:87-106``: copy, ``update``, rebuild; unknown keys raise
        ``TypeError`` from the dataclass constructor."""
        if not config_override:
            return self.config
        d = {k: getattr(self.config, k) for k in _CONFIG_KEYS}
        d.update(config_override)
        return SamplingConfig(**d)

    def sample_mirostat_v2(self, logits: torch.Tensor, config_override: Optional[Dict[str, Any]] = None,
                           previous_entropy: Optional[float] = None, *,
                           uniforms: Optional[torch.Tensor] = None) -> tuple:
        """``sampling.py:240-279``: entropy of ``softmax(logits / T)`` (logits
        unscaled when ``T <= 0``), ``prev -= eta * (H - tau)``, top-k with
        ``k = max(1, int(exp(prev)))`` when ``prev > 0``, then a draw.  Like the
        reference (``.item()`` on the entropy) it takes a single row."""
        config = self._merge_config(config_override)
        D.require_device(logits, "logits")
        B = logits.shape[0]
        dev = logits.device
        T = config.temperature if config.temperature > 0 else 1.0
        stats = sample_rows(logits, SamplingParams.build(B, dev, temperature=T), None, entropy=True,
                            skip_draw=True)
        current = float(stats.entropy.reshape(-1)[0].item())
        if previous_entropy is None:
            previous_entropy = current
        previous_entropy -= config.mirostat_eta * (current - config.mirostat_tau)
        k = max(1, int(math.exp(previous_entropy))) if previous_entropy > 0 else 0
        # the reference's _apply_top_k clamps k to the vocabulary (sampling.py:151)
        k = min(k, logits.shape[-1])
        out = sample_rows(logits, SamplingParams.build(B, dev, temperature=T, top_k=k), uniforms,
                          row_kind_hint=row_kind_flags(T, k, 0.0, 1.0))
        raise_on_status(out.status)
        return out.tokens, previous_entropy

    def get_sampling_info(self) -> Dict[str, Any]:
        """``sampling.py:281-293``."""
        return {
            "temperature": self.config.temperature,
            "top_k": self.config.top_k,
            "top_p": self.config.top_p,
            "repetition_penalty": self.config.repetition_penalty,
            "typical_p": self.config.typical_p,
            "min_p": self.config.min_p,
            "mirostat_tau": self.config.mirostat_tau,
            "mirostat_eta": self.config.mirostat_eta,
            "do_sample": self.config.do_sample,
        }


__all__ = ["Sampler", "SamplingConfig", "pad_histories"]
