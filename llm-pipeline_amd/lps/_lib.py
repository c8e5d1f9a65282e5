"""ctypes binding of ``liblps.so`` (the C ABI declared in ``include/lps.h``).

The library is built in-tree by ``lps.build.build()``.  There is no fallback:
if the shared library is missing, importing the sampler entry points raises.
"""

from __future__ import annotations

import ctypes
import os
import threading

LIB_NAME = "liblps.so"
LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)

LPS_OK = 0
LPS_EINVAL = 1
LPS_EUNSUPPORTED_DTYPE = 2
LPS_ELAUNCH = 3
LPS_EWORKSPACE = 4
LPS_ENOALLOC_CAPACITY = 5

# lps_sample_noalloc's per-GPU workspace (include/lps.h)
LPS_NOALLOC_WORKSPACE_BYTES = 16 << 20

LPS_DTYPE_F32 = 0
LPS_DTYPE_BF16 = 1
LPS_DTYPE_F16 = 2

LPS_ROW_NONFINITE = 1
LPS_ROW_EMPTY = 2
LPS_ROW_HISTORY_OVERFLOW = 4   # never set since ABI version 2 (histories of any size)
LPS_ABI_VERSION = 2

LPS_MAX_TOP_LOGPROBS = 64

LPS_FLAG_GENERIC = 1
LPS_FLAG_APPEND_HISTORY = 2
LPS_FLAG_ROWS_TOPK = 4
LPS_FLAG_ROWS_NUCLEUS = 8
LPS_FLAG_ROWS_BASIC_FILTERS = 16

LPS_RESIDUAL_TARGET = 0
LPS_RESIDUAL_LEVIATHAN = 1

_vp = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_f32 = ctypes.c_float


class SampleArgs(ctypes.Structure):
    """Mirror of ``lps_sample_args`` (field order and types as in lps.h)."""

    _fields_ = [
        ("logits", _vp), ("dtype", _i32), ("num_rows", _i32), ("vocab", _i32), ("rows_inner", _i32),
        ("stride_outer", _i64), ("stride_inner", _i64),
        ("temperature", _vp), ("top_k", _vp), ("top_p", _vp), ("min_p", _vp), ("typical_p", _vp),
        ("repetition_penalty", _vp), ("presence_penalty", _vp), ("frequency_penalty", _vp),
        ("history", _vp), ("history_stride", _i64), ("history_len", _vp),
        ("uniforms", _vp),
        ("query_tokens", _vp), ("query_inner", _i32), ("query_prob", _vp),
        ("tokens", _vp), ("chosen_logprob", _vp), ("top_logprobs", _vp), ("top_ids", _vp), ("n_top", _i32),
        ("entropy", _vp), ("row_status", _vp), ("skip_draw", _i32),
        ("kept_cut", _vp), ("kept_ties", _vp), ("kept_count", _vp),
        ("row_path", _vp),
        ("flags", _i32),
        ("workspace", _vp), ("workspace_bytes", ctypes.c_size_t),
        ("allowed", _vp), ("allowed_stride", _i64),
    ]


class LmHeadArgs(ctypes.Structure):
    """Mirror of ``lps_lm_head_args``."""

    _fields_ = [
        ("x", _vp), ("w", _vp), ("out", _vp), ("stats", _vp), ("dtype", _i32), ("out_dtype", _i32),
        ("rows", _i32), ("vocab", _i32), ("hidden", _i32), ("x_stride", _i64), ("w_stride", _i64),
        ("out_stride", _i64),
    ]


LMHEAD_BLOCK_COLS = 128


class SoftmaxArgs(ctypes.Structure):
    """Mirror of ``lps_softmax_args``."""

    _fields_ = [
        ("x", _vp), ("out", _vp), ("dtype", _i32), ("rows", _i32), ("cols", _i32),
        ("x_stride", _i64), ("out_stride", _i64), ("causal", _i32), ("seq_len", _i32), ("row_offset", _i32),
        ("row_lse", _vp), ("workspace", _vp), ("workspace_bytes", ctypes.c_size_t),
        ("row_stats", _vp), ("stats_stride", _i64), ("stats_cols", _i32),
    ]


class SpecArgs(ctypes.Structure):
    """Mirror of ``lps_spec_args``."""

    _fields_ = [
        ("target_logits", _vp), ("target_stride_b", _i64), ("target_stride_k", _i64),
        ("draft_logits", _vp), ("draft_stride_b", _i64), ("draft_stride_k", _i64),
        ("dtype", _i32), ("batch", _i32), ("k", _i32), ("vocab", _i32),
        ("temperature", _f32), ("top_p", _f32), ("residual", _i32),
        ("draft_tokens", _vp), ("u_accept", _vp), ("u_resample", _vp),
        ("n_accepted", _vp), ("tokens", _vp), ("accept", _vp), ("p_target", _vp), ("q_draft", _vp),
        ("row_status", _vp), ("workspace", _vp), ("workspace_bytes", ctypes.c_size_t),
    ]


# Every symbol include/lps.h declares, with its ctypes signature.
SIGNATURES = {
    "lps_version": (_i32, []),
    "lps_status_string": (ctypes.c_char_p, [_i32]),
    "lps_workspace_bytes": (ctypes.c_size_t, [_i32, _i32, _i32]),
    "lps_spec_workspace_bytes": (ctypes.c_size_t, [_i32, _i32, _i32]),
    "lps_sample": (_i32, [ctypes.POINTER(SampleArgs), _vp]),
    "lps_sample_noalloc": (_i32, [ctypes.POINTER(SampleArgs), _vp]),
    "lps_spec_verify": (_i32, [ctypes.POINTER(SpecArgs), _vp]),
    "lps_verify_drafts": (_i32, [_vp, _i32, _i64, _i64, _i64, _i64, _vp, _vp, _vp, _vp, _vp]),
    "lps_softmax": (_i32, [ctypes.c_void_p, _vp]),
    "lps_softmax_workspace_bytes": (ctypes.c_size_t, [_i32, _i32, _i32]),
    "lps_lm_head": (_i32, [ctypes.c_void_p, _vp]),
    "lps_selftest_exp2_monotone": (_i32, [ctypes.POINTER(ctypes.c_ulonglong)]),
}

_lib = None
_lock = threading.Lock()


def load(path: str = LIB_PATH) -> ctypes.CDLL:
    """Load (once) and type the shared library; raises if it is not built."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(path):
            raise RuntimeError(
                f"lps native library not found at {path}; build it with "
                "`python -c 'import __graft_entry__ as g; g.build()'` (hipcc --offload-arch=gfx950)")
        lib = ctypes.CDLL(path)
        for name, (res, argt) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = argt
        if lib.lps_version() != LPS_ABI_VERSION:
            raise RuntimeError(f"lps ABI version mismatch: {lib.lps_version()}")
        _lib = lib
        return lib


def check(rc: int, what: str) -> None:
    """Map an ABI return code onto the exception the reference raises."""
    if rc == LPS_OK:
        return
    msg = f"{what}: {load().lps_status_string(rc).decode()}"
    if rc == LPS_EUNSUPPORTED_DTYPE:
        raise TypeError(msg)
    if rc in (LPS_EINVAL, LPS_EWORKSPACE, LPS_ENOALLOC_CAPACITY):
        raise ValueError(msg)
    raise RuntimeError(msg)
