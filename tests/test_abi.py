"""CPU checks of the C ABI and the host layer: the library loads, exports every
function include/lps.h declares, the ctypes structs match the C layout, and
argument errors are reported without touching a GPU."""

import ctypes
import os
import re
import subprocess
import tempfile

import pytest
import torch

from tests.conftest import REPO

HEADER = os.path.join(REPO, "include", "lps.h")


@pytest.fixture(scope="module")
def lib():
    from lps import _lib
    if not os.path.exists(_lib.LIB_PATH):
        from lps import build
        build.build()
    return _lib.load()


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*[A-Za-z_][\w\s\*]*?\b(lps_\w+)\s*\(", text, flags=re.M)))


def test_header_declares_expected_entry_points():
    from lps import _lib
    assert declared_functions() == sorted(_lib.SIGNATURES)


def test_library_exports_every_declared_symbol(lib):
    for name in declared_functions():
        assert hasattr(lib, name), name
    out = subprocess.run(["nm", "-D", "--defined-only", lib._name], capture_output=True, text=True).stdout
    exported = set(re.findall(r"\bT (lps_\w+)", out))
    assert set(declared_functions()) <= exported


def test_version_and_status_strings(lib):
    ver = int(re.search(r"#define LPS_ABI_VERSION (\d+)", open(HEADER).read()).group(1))
    assert lib.lps_version() == ver
    assert lib.lps_status_string(0) == b"ok"
    assert lib.lps_status_string(2) == b"unsupported logits dtype"
    assert lib.lps_status_string(99) == b"unknown status"


def _c_layout(struct, fields):
    src = "#include <stddef.h>\n#include <stdio.h>\n#include \"lps.h\"\nint main(void){\n"
    src += f'printf("%zu\\n", sizeof({struct}));\n'
    for f in fields:
        src += f'printf("%zu\\n", offsetof({struct}, {f}));\n'
    src += "return 0;}\n"
    with tempfile.TemporaryDirectory() as d:
        c = os.path.join(d, "l.c")
        open(c, "w").write(src)
        exe = os.path.join(d, "l")
        subprocess.run(["gcc", "-std=c99", "-I", os.path.join(REPO, "include"), c, "-o", exe], check=True)
        vals = [int(v) for v in subprocess.run([exe], capture_output=True, text=True, check=True).stdout.split()]
    return vals[0], vals[1:]


@pytest.mark.parametrize("cname,pyname", [("lps_sample_args", "SampleArgs"), ("lps_spec_args", "SpecArgs"),
                                         ("lps_softmax_args", "SoftmaxArgs"), ("lps_lm_head_args", "LmHeadArgs")])
def test_struct_layout_matches_c(cname, pyname):
    from lps import _lib
    py = getattr(_lib, pyname)
    names = [f[0] for f in py._fields_]
    size, offs = _c_layout(cname, names)
    assert ctypes.sizeof(py) == size
    assert [getattr(py, n).offset for n in names] == offs


def _args(**kw):
    from lps import _lib
    a = _lib.SampleArgs()
    a.logits = 0x1000
    a.dtype = 0
    a.num_rows = 4
    a.vocab = 100
    a.rows_inner = 1
    a.stride_outer = 100
    a.tokens = 0x2000
    a.uniforms = 0x3000
    for k, v in kw.items():
        setattr(a, k, v)
    return a


@pytest.mark.parametrize("kw,code", [
    (dict(dtype=7), 2),
    (dict(vocab=0), 1),
    (dict(vocab=1 << 19), 1),
    (dict(rows_inner=0), 1),
    (dict(logits=0), 1),
    (dict(tokens=0), 1),
    (dict(n_top=65, top_logprobs=0x4000), 1),
    (dict(n_top=3), 1),
    (dict(uniforms=0), 1),
    (dict(history=0x5000), 1),
    (dict(stride_outer=-1), 1),
    (dict(allowed=0x6000, allowed_stride=3), 1),      # V=100 needs 4 words per row
    (dict(num_rows=0), 0),
])
def test_sample_argument_errors(lib, kw, code):
    """Invalid arguments are rejected on the host before any launch."""
    a = _args(**kw)
    assert lib.lps_sample(ctypes.byref(a), None) == code
    assert lib.lps_sample(None, None) == 1


def test_spec_argument_errors(lib):
    from lps import _lib
    a = _lib.SpecArgs()
    a.batch, a.k, a.vocab, a.dtype = 2, 0, 10, 0
    assert lib.lps_spec_verify(ctypes.byref(a), None) == 1            # k < 1
    a.k = 3
    a.target_logits = a.draft_logits = a.draft_tokens = a.u_accept = a.u_resample = 0x1000
    a.n_accepted = a.tokens = 0x2000
    assert lib.lps_spec_verify(ctypes.byref(a), None) == 4            # no workspace
    a.workspace = 0x3000
    a.workspace_bytes = lib.lps_spec_workspace_bytes(2, 3, 10) - 1
    assert lib.lps_spec_verify(ctypes.byref(a), None) == 4            # too small
    a.residual = 5
    assert lib.lps_spec_verify(ctypes.byref(a), None) == 1
    a.dtype = 9
    assert lib.lps_spec_verify(ctypes.byref(a), None) == 2
    a.batch = 0
    a.dtype = 0
    a.residual = 0
    assert lib.lps_spec_verify(ctypes.byref(a), None) == 0
    assert lib.lps_spec_workspace_bytes(0, 3, 10) == 0
    assert lib.lps_spec_workspace_bytes(32, 4, 151936) > 0
    assert lib.lps_verify_drafts(None, 0, 0, 10, 10, 1, None, None, None, None, None) == 0
    assert lib.lps_verify_drafts(None, 0, 4, 10, 10, 1, None, None, None, None, None) == 1
    assert lib.lps_verify_drafts(None, 3, 4, 10, 10, 1, None, None, None, None, None) == 2


# ------------------------------------------------------------ host layer --


def test_merge_config_unknown_key_raises_type_error():
    from lps import Sampler, SamplingConfig
    s = Sampler(SamplingConfig(temperature=0.5))
    with pytest.raises(TypeError):
        s._merge_config({"no_such_key": 1})
    c = s._merge_config({"top_k": 7})
    assert c.top_k == 7 and c.temperature == 0.5
    assert s._merge_config(None) is s.config
    assert s.get_sampling_info()["temperature"] == 0.5
    assert set(s.get_sampling_info()) == {"temperature", "top_k", "top_p", "repetition_penalty", "typical_p",
                                          "min_p", "mirostat_tau", "mirostat_eta", "do_sample"}


def test_cpu_tensors_are_refused_not_sampled_on_cpu():
    """No CPU fallback: the product raises instead of sampling on the host."""
    from lps import Sampler, sample_rows, SamplingParams, verify_drafts_batched
    x = torch.randn(2, 16)
    with pytest.raises(RuntimeError, match="ROCm device"):
        Sampler().sample_token(x)
    with pytest.raises(RuntimeError, match="ROCm device"):
        sample_rows(x, SamplingParams.build(2, "cpu"))
    with pytest.raises(RuntimeError, match="ROCm device"):
        verify_drafts_batched(torch.rand(4, 8), torch.rand(4), torch.zeros(4, dtype=torch.long), torch.rand(4))


def test_sampling_params_and_histories_host():
    from lps import SamplingParams, pad_histories, SamplingConfig
    p = SamplingParams.build(3, "cpu", temperature=torch.tensor([0.1, 0.2, 0.3]), top_k=5)
    assert p.temperature.dtype == torch.float32 and p.top_k.tolist() == [5, 5, 5]
    q = SamplingParams.from_configs([SamplingConfig(top_k=3), SamplingConfig(temperature=0.0, top_p=0.5)], "cpu")
    assert q.top_k.tolist() == [3, 50] and q.temperature.tolist() == [1.0, 0.0]
    assert q.presence_penalty.tolist() == [0.0, 0.0]
    h, n = pad_histories([[1, 2, 3], [], [7]], "cpu")
    assert h.shape == (3, 3) and n.tolist() == [3, 0, 1] and h[2, 0].item() == 7


def test_row_kind_flags():
    """Row-kind hints from host-side parameters; nothing is hinted from values
    the host does not hold, and no min-p / typical-p hint without both."""
    from lps import _lib, row_kind_flags
    TOPK, NUC, NMT = _lib.LPS_FLAG_ROWS_TOPK, _lib.LPS_FLAG_ROWS_NUCLEUS, _lib.LPS_FLAG_ROWS_BASIC_FILTERS
    assert row_kind_flags([0.0, 1.0], [0, 5]) == TOPK
    assert row_kind_flags(1.0, 0) == NUC
    assert row_kind_flags([0.0, 1.0], [0, 0]) == 0
    assert row_kind_flags(1.0, 0, 0.0, 1.0) == NUC | NMT
    assert row_kind_flags(torch.tensor([0.0, 0.7]), torch.tensor([0, 9]), [0.0, 0.0], [1.0, 1.0]) == TOPK | NMT
    assert row_kind_flags(1.0, 0, [0.0, 0.05], 1.0) == NUC
    assert row_kind_flags(1.0, 0, 0.0, [1.0, 0.9]) == NUC
    assert row_kind_flags(1.0, 0, 0.0) == NUC
    assert row_kind_flags(1.0, [5, 300], 0.0, 1.0) == TOPK
    assert _lib.LPS_FLAG_ROWS_BASIC_FILTERS == 16


def test_lm_head_argument_errors(lib):
    """Argument checks of lps_lm_head happen before any launch (no GPU)."""
    from lps import _lib
    a = _lib.LmHeadArgs()
    a.dtype, a.out_dtype, a.rows, a.vocab, a.hidden = 0, 0, 4, 100, 64
    assert lib.lps_lm_head(ctypes.byref(a), None) == 2                # fp32 inputs are not supported
    a.dtype = 1
    a.hidden = 40
    assert lib.lps_lm_head(ctypes.byref(a), None) == 1                # hidden not a multiple of 16
    a.hidden = 64
    assert lib.lps_lm_head(ctypes.byref(a), None) == 1                # null pointers
    a.x, a.w, a.out = 0x1000, 0x2000, 0x3000
    a.x_stride, a.w_stride, a.out_stride = 60, 64, 100
    assert lib.lps_lm_head(ctypes.byref(a), None) == 1                # x_stride < hidden
    a.x_stride = 68
    assert lib.lps_lm_head(ctypes.byref(a), None) == 1                # stride not a multiple of 8
    a.x = 0x1004
    a.x_stride = 64
    assert lib.lps_lm_head(ctypes.byref(a), None) == 1                # misaligned rows
    a.rows = 0
    assert lib.lps_lm_head(ctypes.byref(a), None) == 0
    assert lib.lps_lm_head(None, None) == 1
