"""Row softmax with an optional causal mask on the GPU: a drop-in for the
reference's ``fused_softmax_triton`` (``quantization/kernels/triton_softmax.py:65-102``),
computed by the ``lps_softmax`` HIP kernel.

Semantics follow the reference's torch restatement (``:105-113``): positions
``j > (row % T) + row_offset`` are ``-inf`` when ``causal`` (``T`` = the size of
the second-to-last axis), softmax in fp32 over the last axis, result in the
input dtype."""

from __future__ import annotations

import ctypes
import threading
from typing import Optional, Tuple, Union

import torch

from . import _device as D
from . import _lib

_WS_LOCK = threading.Lock()
_WS = {}


def _workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    """Zero-filled scratch for split rows, cached per (device, stream): every
    launch leaves it zeroed, and launches on one stream never overlap."""
    key = (device.index, torch.cuda.current_stream(device).cuda_stream)
    with _WS_LOCK:
        t = _WS.get(key)
        if t is None or t.numel() < nbytes:
            t = torch.zeros((max(nbytes, 1 << 16),), dtype=torch.uint8, device=device)
            _WS[key] = t
        return t


def fused_softmax(x: torch.Tensor, causal: bool = False, row_offset: int = 0,
                  return_lse: bool = False, row_stats: Optional[torch.Tensor] = None,
                  stats_cols: int = 128) -> Union[torch.Tensor, Tuple[torch.Tensor, torch.Tensor]]:
    """Softmax over the last axis of ``x [..., n_cols]`` (fp32 / bf16 / fp16 on
    a ROCm device).  ``return_lse`` also returns each row's log-sum-exp of the
    masked values (fp32, shape ``x.shape[:-1]``; -inf for an all -inf row).
    ``row_stats [..., ceil(n_cols / stats_cols), 2]`` (float32 ``(max, sum(exp(v
    - max)))`` per block of ``stats_cols`` columns, as ``lm_head(...,
    return_stats=True)`` returns them) makes the softmax one streaming pass."""
    D.require_device(x, "x")
    if x.dim() < 1:
        raise ValueError("x must have at least one axis")
    shape = x.shape
    n_cols = shape[-1]
    if x.stride(-1) != 1:
        x = x.contiguous()
    x2 = x.reshape(-1, n_cols)
    rows = x2.shape[0]
    out = torch.empty((rows, n_cols), dtype=x.dtype, device=x.device)
    lse = torch.empty((rows,), dtype=torch.float32, device=x.device) if return_lse else None
    a = _lib.SoftmaxArgs()
    a.x = x2.data_ptr()
    a.out = out.data_ptr()
    a.dtype = D.dtype_code(x2)
    a.rows = rows
    a.cols = n_cols
    a.x_stride = x2.stride(0) if rows > 1 else n_cols
    a.out_stride = n_cols
    a.causal = 1 if causal else 0
    a.seq_len = shape[-2] if x.dim() >= 2 else 1
    a.row_offset = int(row_offset)
    a.row_lse = D.ptr(lse)
    if row_stats is not None:
        if causal:
            raise ValueError("row_stats cannot be combined with causal")
        nst = (n_cols + stats_cols - 1) // stats_cols
        st = row_stats.reshape(-1, nst, 2)
        if st.shape[0] != rows or st.dtype != torch.float32 or st.device != x.device:
            raise ValueError(f"row_stats must be float32 [..., {nst}, 2] on the device of x")
        st = st.contiguous()
        a.row_stats = st.data_ptr()
        a.stats_stride = 2 * nst
        a.stats_cols = stats_cols
    if rows:
        lib = _lib.load()
        nb = lib.lps_softmax_workspace_bytes(rows, n_cols, a.dtype)
        with torch.cuda.device(x.device):
            if nb:
                ws = _workspace(x.device, nb)
                a.workspace = ws.data_ptr()
                a.workspace_bytes = ws.numel()
            rc = lib.lps_softmax(ctypes.byref(a), D.stream_of(x.device))
        _lib.check(rc, "lps_softmax")
    out = out.reshape(shape)
    if return_lse:
        return out, lse.reshape(shape[:-1])
    return out


# the reference's name
fused_softmax_triton = fused_softmax
