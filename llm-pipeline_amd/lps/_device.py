"""Device-tensor plumbing shared by the sampler entry points: dtype codes,
pointers, the current HIP stream and per-row parameter tensors."""

from __future__ import annotations

import torch

from . import _lib

_DTYPES = {
    torch.float32: _lib.LPS_DTYPE_F32,
    torch.bfloat16: _lib.LPS_DTYPE_BF16,
    torch.float16: _lib.LPS_DTYPE_F16,
}


def require_device(t: torch.Tensor, name: str) -> None:
    """The sampler runs only on the GPU; there is no CPU path."""
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a torch.Tensor")
    if t.device.type != "cuda":
        raise RuntimeError(f"lps samples on a ROCm device; {name} is on {t.device}")


def dtype_code(t: torch.Tensor) -> int:
    try:
        return _DTYPES[t.dtype]
    except KeyError:
        raise TypeError(f"unsupported logits dtype {t.dtype}; expected float32, bfloat16 or float16") from None


def ptr(t) -> int:
    return 0 if t is None else int(t.data_ptr())


def stream_of(device: torch.device) -> int:
    return int(torch.cuda.current_stream(device).cuda_stream)


def as_f32(v, B: int, device) -> torch.Tensor:
    if isinstance(v, torch.Tensor):
        t = v.to(device=device, dtype=torch.float32).reshape(-1)
        if t.numel() == 1 and B != 1:
            t = t.expand(B)
        return t.contiguous()
    return torch.full((B,), float(v), dtype=torch.float32, device=device)


def as_i32(v, B: int, device) -> torch.Tensor:
    if isinstance(v, torch.Tensor):
        t = v.to(device=device, dtype=torch.int32).reshape(-1)
        if t.numel() == 1 and B != 1:
            t = t.expand(B)
        return t.contiguous()
    return torch.full((B,), int(v), dtype=torch.int32, device=device)
