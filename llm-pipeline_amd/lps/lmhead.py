"""The LM-head projection with the softmax-statistics epilogue on the GPU.

The reference's logits producer is ``self.lm_head(hidden_states)``
(``models/qwen3/custom_builder.py:415``, ``models/qwen3_5/model.py:263``), an
``nn.Linear`` without bias.  ``lm_head`` computes the same projection with the
``lps_lm_head`` MFMA kernel and, while the tile is in registers, each row's
``(max, sum(exp(v - max)))`` over every block of 128 vocabulary columns, so a
softmax of the logits (``fused_softmax(logits, row_stats=stats)``) needs one
streaming pass instead of a statistics pass first."""

from __future__ import annotations

import ctypes
from typing import Optional, Tuple, Union

import torch

from . import _device as D
from . import _lib


def lm_head(hidden: torch.Tensor, weight: torch.Tensor, out_dtype: Optional[torch.dtype] = None,
            return_stats: bool = False) -> Union[torch.Tensor, Tuple[torch.Tensor, torch.Tensor]]:
    """``hidden [..., H] @ weight[V, H].T`` -> logits ``[..., V]`` (fp32
    accumulation, stored in ``out_dtype``, default the input dtype).  Inputs:
    bf16 or fp16, the same dtype, ``H`` a multiple of 16.  ``return_stats``
    also returns ``[..., ceil(V / 128), 2]`` float32 block statistics
    ``(max, sum(exp(v - max)))`` of the stored logits."""
    D.require_device(hidden, "hidden")
    D.require_device(weight, "weight")
    if weight.dim() != 2 or hidden.shape[-1] != weight.shape[1]:
        raise ValueError(f"hidden [..., H] and weight [V, H] expected; got {tuple(hidden.shape)}, {tuple(weight.shape)}")
    if hidden.dtype != weight.dtype or hidden.dtype not in (torch.bfloat16, torch.float16):
        raise TypeError("hidden and weight must both be bfloat16 or both float16")
    V, H = weight.shape
    lead = hidden.shape[:-1]
    x = hidden.reshape(-1, H)
    if x.stride(-1) != 1 or (x.shape[0] > 1 and x.stride(0) % 8) or x.data_ptr() % 16:
        x = x.contiguous()
    w = weight
    if w.stride(-1) != 1 or w.stride(0) % 8 or w.data_ptr() % 16:
        w = w.contiguous()
    M = x.shape[0]
    od = out_dtype or hidden.dtype
    out = torch.empty((M, V), dtype=od, device=hidden.device)
    G = (V + _lib.LMHEAD_BLOCK_COLS - 1) // _lib.LMHEAD_BLOCK_COLS
    stats = torch.empty((M, G, 2), dtype=torch.float32, device=hidden.device) if return_stats else None
    a = _lib.LmHeadArgs()
    a.x, a.w, a.out = x.data_ptr(), w.data_ptr(), out.data_ptr()
    a.stats = D.ptr(stats)
    a.dtype = D.dtype_code(x)
    a.out_dtype = D.dtype_code(out)
    a.rows, a.vocab, a.hidden = M, V, H
    a.x_stride = x.stride(0) if M > 1 else H
    a.w_stride = w.stride(0)
    a.out_stride = V
    if M:
        with torch.cuda.device(hidden.device):
            rc = _lib.load().lps_lm_head(ctypes.byref(a), D.stream_of(hidden.device))
        _lib.check(rc, "lps_lm_head")
    out = out.reshape(*lead, V)
    if return_stats:
        return out, stats.reshape(*lead, G, 2)
    return out
