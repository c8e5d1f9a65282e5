"""lps: MI355X-native token sampler, a drop-in for the logits -> token path of
the llm-pipeline inference engine (``llm_pipeline.inference`` exports
``Sampler``, ``SamplingConfig`` and ``verify_drafts_batched``,
``src/llm_pipeline/inference/__init__.py:4,17,37-38``)."""

from .batch import (SampleOutput, SamplingParams, allowed_from_constraint, pack_allowed, pad_histories,
                    raise_on_status, row_kind_flags, sample_rows)
from .sampling import Sampler, SamplingConfig
from .speculative import SpecDecStats, SpecVerifyOutput, spec_verify, verify_drafts_batched
from .lmhead import lm_head
from .softmax import fused_softmax, fused_softmax_triton
from .spec_driver import (mtp_speculative_decode, mtp_speculative_decode_batched, speculative_decode,
                          speculative_decode_batched)
from .state import SamplerState

__all__ = [
    "Sampler",
    "SamplingConfig",
    "SamplingParams",
    "SampleOutput",
    "sample_rows",
    "row_kind_flags",
    "pack_allowed",
    "allowed_from_constraint",
    "SamplerState",
    "fused_softmax",
    "fused_softmax_triton",
    "pad_histories",
    "raise_on_status",
    "verify_drafts_batched",
    "spec_verify",
    "lm_head",
    "speculative_decode",
    "speculative_decode_batched",
    "mtp_speculative_decode",
    "mtp_speculative_decode_batched",
    "SpecVerifyOutput",
    "SpecDecStats",
]
