"""Row softmax (lps_softmax), the drop-in for the reference's
fused_softmax_triton (quantization/kernels/triton_softmax.py:65-102): the
reference's own two tests (testing/unit/test_kernels_low_level.py:138-157), then
dtypes, vocabulary-length rows, causal masks with a row offset, strided rows,
the log-sum-exp output and non-finite rows, against torch's softmax in fp32."""

import math

import pytest
import torch

from lps import fused_softmax, fused_softmax_triton

pytestmark = pytest.mark.gpu


def _ref(x, causal=False, row_offset=0):
    """The reference's torch restatement (triton_softmax.py:105-113)."""
    if causal:
        n_rows = x.shape[-2] if x.dim() >= 2 else 1
        n_cols = x.shape[-1]
        row_idx = torch.arange(n_rows, device=x.device).unsqueeze(-1) + row_offset
        col_idx = torch.arange(n_cols, device=x.device).unsqueeze(0)
        x = x.masked_fill(col_idx > row_idx, float("-inf"))
    return torch.softmax(x.float(), dim=-1).to(x.dtype)


def test_reference_no_mask_matches_torch(dev):
    x = torch.randn(3, 4, 16) * 2.0
    out = fused_softmax_triton(x.to(dev), causal=False)
    torch.testing.assert_close(out.cpu(), torch.softmax(x.float(), dim=-1).to(x.dtype), atol=1e-5, rtol=1e-5)


def test_reference_causal_mask_blocks_future_positions(dev):
    T = 4
    out = fused_softmax_triton(torch.zeros(T, T, device=dev), causal=True).cpu()
    for i in range(T):
        for j in range(T):
            if j <= i:
                assert abs(out[i, j].item() - 1.0 / (i + 1)) < 1e-5
            else:
                assert out[i, j].item() == 0


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("shape", [(64, 151936), (5, 7, 1000), (9, 4099), (2, 3, 1)])
def test_softmax_dtypes_and_shapes(dev, dtype, shape):
    g = torch.Generator().manual_seed(sum(shape))
    x = (torch.randn(shape, generator=g) * 3.0).to(dtype)
    out = fused_softmax(x.to(dev)).cpu()
    # fp64 reference: torch's own fp32 CPU softmax of a 151936-column row is
    # 1.3e-5 away from it (its fp32 row sum), more than the kernel's 2e-6
    ref = torch.softmax(x.double(), dim=-1)
    tol = {torch.float32: 2e-6, torch.bfloat16: 2 ** -8, torch.float16: 2 ** -10}[dtype]
    torch.testing.assert_close(out.double(), ref, atol=1e-7, rtol=tol)
    assert out.dtype == dtype
    s = out.float().sum(-1)                                        # 16-bit outputs carry their rounding
    assert torch.allclose(s, torch.ones_like(s), atol={torch.float32: 1e-5, torch.bfloat16: 2 ** -6,
                                                       torch.float16: 2 ** -8}[dtype])


@pytest.mark.parametrize("row_offset", [0, 3, -2])
def test_softmax_causal_offset_3d(dev, row_offset):
    g = torch.Generator().manual_seed(4)
    x = torch.randn(2, 6, 11, generator=g)
    out = fused_softmax(x.to(dev), causal=True, row_offset=row_offset).cpu()
    ref = _ref(x, causal=True, row_offset=row_offset)
    assert torch.equal(torch.isnan(out), torch.isnan(ref))        # rows fully masked: NaN, as torch
    torch.testing.assert_close(torch.nan_to_num(out), torch.nan_to_num(ref), atol=1e-6, rtol=2e-6)


def test_softmax_strided_rows_and_lse(dev):
    g = torch.Generator().manual_seed(5)
    big = torch.randn(16, 40000, generator=g).to(dev)
    x = big[:, :32768]                                             # rows of a wider buffer
    out, lse = fused_softmax(x, return_lse=True)
    ref = torch.softmax(x.float().cpu(), dim=-1)
    torch.testing.assert_close(out.cpu(), ref, atol=1e-8, rtol=2e-6)
    torch.testing.assert_close(lse.cpu(), torch.logsumexp(x.cpu(), dim=-1), atol=1e-5, rtol=1e-6)


def test_softmax_non_finite_rows_match_torch(dev):
    x = torch.randn(4, 300)
    x[0, 5] = float("nan")
    x[1, 7] = float("inf")
    x[2] = float("-inf")
    out = fused_softmax(x.to(dev)).cpu()
    ref = torch.softmax(x, dim=-1)
    assert torch.equal(torch.isnan(out), torch.isnan(ref))
    torch.testing.assert_close(out[3], ref[3], atol=1e-8, rtol=2e-6)


# ---------------------------------------------------------------------------
# The kernel paths: one wave per row (<= 2048 fp32 / 4096 16-bit columns), one
# register-resident workgroup per row (<= 8192 / 16384), rows split over G
# workgroups that exchange (max, sum) records, and the three-pass kernel
# (unaligned rows, no workspace, in-place split rows).
# ---------------------------------------------------------------------------
def _check(out, x, causal=False, row_offset=0, dtype=None):
    """out against the fp64 softmax of x (masked as the reference masks)."""
    dtype = dtype or x.dtype
    xd = x.double()
    if causal:
        n_rows, n_cols = x.shape[-2], x.shape[-1]
        row_idx = torch.arange(n_rows).unsqueeze(-1) + row_offset
        xd = xd.masked_fill(torch.arange(n_cols).unsqueeze(0) > row_idx, float("-inf"))
    ref = torch.softmax(xd, dim=-1)
    tol = {torch.float32: 2e-6, torch.bfloat16: 2 ** -8, torch.float16: 2 ** -10}[dtype]
    o = out.cpu().double()
    assert torch.equal(torch.isnan(o), torch.isnan(ref))
    torch.testing.assert_close(torch.nan_to_num(o), torch.nan_to_num(ref), atol=1e-7, rtol=tol)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("shape", [(3, 100000), (1, 151936), (7, 12288), (33, 2048), (4, 520), (16, 4096)])
def test_softmax_paths(dev, dtype, shape):
    g = torch.Generator().manual_seed(shape[1] + 7)
    x = (torch.randn(shape, generator=g) * 4.0).to(dtype)
    out, lse = fused_softmax(x.to(dev), return_lse=True)
    _check(out, x)
    torch.testing.assert_close(lse.cpu().double(), torch.logsumexp(x.double(), dim=-1), atol=2e-5, rtol=1e-6)


@pytest.mark.parametrize("cols", [150001, 16385, 4099, 2050])
def test_softmax_ragged_tail_aligned_rows(dev, cols):
    """Rows of a wider buffer (16-byte aligned starts) whose length is not a
    whole number of 16-byte vectors: the last vector is read and written
    element by element, and nothing past the row is touched."""
    g = torch.Generator().manual_seed(cols)
    big = (torch.randn(6, 151944 if cols > 16384 else 16392, generator=g) * 3.0).to(torch.bfloat16).to(dev)
    x = big[:, :cols]
    out = torch.full((6, big.shape[1]), 7.0, dtype=torch.bfloat16, device=dev)
    o = out[:, :cols]
    res = fused_softmax(x)
    o.copy_(res)
    _check(res, x.cpu())
    assert bool((out[:, cols:] == 7.0).all())


@pytest.mark.parametrize("row_offset", [0, 20000, -5])
def test_softmax_causal_split_rows(dev, row_offset):
    """Causal masks over split rows: whole chunks past the mask, chunks cut by it."""
    g = torch.Generator().manual_seed(abs(row_offset) + 3)
    x = torch.randn(2, 5, 40000, generator=g) * 3.0
    out = fused_softmax(x.to(dev), causal=True, row_offset=row_offset)
    _check(out, x, causal=True, row_offset=row_offset)


@pytest.mark.parametrize("cols", [1000, 151936])
def test_softmax_non_finite_in_chunks(dev, cols):
    """A NaN or +inf in one chunk makes its row NaN; a chunk (or row) of -inf
    contributes nothing (an all -inf row is NaN, log-sum-exp -inf)."""
    x = torch.randn(6, cols)
    x[0, cols - 3] = float("nan")                 # last chunk
    x[1, 2] = float("inf")                        # first chunk
    x[2, : cols // 2] = float("-inf")             # -inf chunks, finite rest
    x[3] = float("-inf")
    x[4, 1:] = float("-inf")                      # one finite value: probability 1
    out, lse = fused_softmax(x.to(dev), return_lse=True)
    ref = torch.softmax(x.double(), dim=-1)
    o = out.cpu().double()
    assert torch.equal(torch.isnan(o), torch.isnan(ref))
    torch.testing.assert_close(torch.nan_to_num(o), torch.nan_to_num(ref), atol=1e-7, rtol=2e-6)
    rl = torch.logsumexp(x.double(), dim=-1)
    l = lse.cpu().double()
    assert math.isinf(float(l[3])) and float(l[3]) < 0
    torch.testing.assert_close(l[[2, 4, 5]], rl[[2, 4, 5]], atol=2e-5, rtol=1e-6)


def test_softmax_in_place_and_without_workspace(dev):
    """An in-place call of split rows and a call with no workspace both take
    the three-pass kernel; the result is the same softmax."""
    import ctypes
    from lps import _lib
    from lps import _device as D
    g = torch.Generator().manual_seed(12)
    x = torch.randn(4, 151936, generator=g) * 3.0
    xd = x.to(dev)
    a = _lib.SoftmaxArgs()
    a.x = xd.data_ptr()
    a.out = xd.data_ptr()                          # in place
    a.dtype = D.dtype_code(xd)
    a.rows, a.cols = 4, 151936
    a.x_stride = a.out_stride = 151936
    a.seq_len = 1
    lib = _lib.load()
    ws = torch.zeros(lib.lps_softmax_workspace_bytes(4, 151936, a.dtype), dtype=torch.uint8, device=dev)
    a.workspace, a.workspace_bytes = ws.data_ptr(), ws.numel()
    _lib.check(lib.lps_softmax(ctypes.byref(a), D.stream_of(dev)), "lps_softmax")
    _check(xd, x)
    xd2 = x.to(dev)
    out = torch.empty_like(xd2)
    b = _lib.SoftmaxArgs.from_buffer_copy(a)
    b.x, b.out = xd2.data_ptr(), out.data_ptr()
    b.workspace, b.workspace_bytes = None, 0       # no workspace
    _lib.check(lib.lps_softmax(ctypes.byref(b), D.stream_of(dev)), "lps_softmax")
    _check(out, x)


def test_softmax_graph_replays(dev):
    """Split rows captured in a graph: every replay, with new inputs and eager
    work in between, equals the eager result, and the workspace ends zeroed."""
    g = torch.Generator().manual_seed(21)
    x = (torch.randn(16, 151936, generator=g) * 3.0).to(torch.bfloat16).to(dev)
    out = torch.empty_like(x)
    fused_softmax(x)                               # workspace created outside the capture
    torch.cuda.synchronize(dev)
    graph = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream(dev)
    s.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(s):
        fused_softmax(x)
        torch.cuda.synchronize(dev)
        with torch.cuda.graph(graph, stream=s):
            out.copy_(fused_softmax(x))
    torch.cuda.synchronize(dev)
    for rep in range(4):
        xn = (torch.randn(16, 151936, generator=g) * (2.0 + rep)).to(torch.bfloat16)
        x.copy_(xn.to(dev))
        torch.cuda.synchronize(dev)
        graph.replay()
        torch.cuda.synchronize(dev)
        eager = fused_softmax(x)
        torch.cuda.synchronize(dev)
        assert torch.equal(out, eager), f"replay {rep}"
        _check(out, xn)
    from lps import softmax as SM
    assert all(int(t.count_nonzero()) == 0 for t in SM._WS.values()), "records left in a workspace"


def test_softmax_workspace_reuse_across_layouts(dev):
    """Split calls of different shapes and dtypes share one workspace (record
    and counter regions of one call overlap those of the next): each result
    is right and the workspace is all zeros after every call."""
    from lps import softmax as SM
    g = torch.Generator().manual_seed(33)
    for shape, dtype in [((64, 151936), torch.float32), ((64, 151936), torch.bfloat16), ((3, 100000), torch.float32),
                         ((16, 151936), torch.float16), ((64, 151936), torch.float32)]:
        x = (torch.randn(shape, generator=g) * 3.0).to(dtype)
        out = fused_softmax(x.to(dev))
        torch.cuda.synchronize(dev)
        _check(out, x)
        for t in SM._WS.values():
            assert int(t.count_nonzero()) == 0, f"{shape} {dtype}: records left in the workspace"
