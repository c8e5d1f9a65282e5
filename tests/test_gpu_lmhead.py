"""LM-head projection with the statistics epilogue (``lps_lm_head``), the
logits producer ``logits = lm_head(hidden)`` of ``models/qwen3/custom_builder.py:415``
and ``models/qwen3_5/model.py:263`` (``nn.Linear`` without bias).

Logits: against the projection in fp64 (on the CPU for small shapes, in fp32
on the GPU for the c2 shape), within one rounding of the output dtype plus the
fp32 accumulation error.  Statistics: recomputed in fp64 from the stored
logits, block by block (the max exactly, the sum within 1e-6 relative).  Then
the softmax from the statistics against the softmax of the logits."""

import pytest
import torch

from lps import fused_softmax, lm_head

pytestmark = pytest.mark.gpu

ULP = {torch.bfloat16: 2 ** -8, torch.float16: 2 ** -11, torch.float32: 2 ** -23}


def _ref(x, w):
    return x.double() @ w.double().T


def _check_logits(out, ref, H, scale):
    rel = ULP[out.dtype]
    # fp32 accumulation over H products of size ~scale^2: a few ulp of fp32 each
    acc = 1e-6 * (H ** 0.5) * scale * scale + 1e-30
    err = (out.double().cpu() - ref.cpu()).abs()
    bound = rel * ref.cpu().abs() + acc
    assert bool((err <= bound).all()), f"max err {float(err.max())}, at {int(torch.argmax(err - bound))}"


def _check_stats(out, stats):
    M, V = out.shape
    G = (V + 127) // 128
    v = out.double().cpu()
    pad = torch.full((M, G * 128 - V), float("-inf"), dtype=torch.float64)
    blocks = torch.cat([v, pad], dim=1).reshape(M, G, 128)
    mx = blocks.max(dim=2).values
    s = torch.exp(blocks - mx.unsqueeze(-1)).sum(dim=2)
    st = stats.double().cpu()
    assert torch.equal(st[..., 0], mx.to(torch.float32).double()), "block max differs"
    torch.testing.assert_close(st[..., 1], s, rtol=2e-6, atol=0)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("out_dtype", [None, torch.float32])
@pytest.mark.parametrize("M,V,H", [(5, 1000, 64), (70, 300, 128), (1, 129, 16), (64, 4099, 256), (130, 2000, 48)])
def test_lm_head_small(dev, dtype, out_dtype, M, V, H):
    g = torch.Generator().manual_seed(M * 7 + V + H)
    x = (torch.randn((M, H), generator=g)).to(dtype)
    w = (torch.randn((V, H), generator=g) * 0.5).to(dtype)
    out, stats = lm_head(x.to(dev), w.to(dev), out_dtype=out_dtype, return_stats=True)
    assert out.dtype == (out_dtype or dtype) and tuple(out.shape) == (M, V)
    _check_logits(out, _ref(x, w), H, 1.0)
    _check_stats(out, stats)


def test_lm_head_c2_shape(dev):
    """The c2 decode shape: 64 rows, H = 4096, V = 151936 (a Qwen3-8B head)."""
    g = torch.Generator(device=dev).manual_seed(1)
    M, V, H = 64, 151936, 4096
    x = torch.randn((M, H), generator=g, device=dev).to(torch.bfloat16)
    w = (torch.randn((V, H), generator=g, device=dev) * 0.02).to(torch.bfloat16)
    out, stats = lm_head(x, w, return_stats=True)
    ref = x.float() @ w.float().T                  # fp32 on the GPU as the reference
    err = (out.float() - ref).abs()
    bound = 2 ** -8 * ref.abs() + 1e-6 * (H ** 0.5) * 0.02 * 4
    assert bool((err <= bound).all()), f"max err {float(err.max())}"
    _check_stats(out[:8], stats[:8])


def test_lm_head_batched_leading_dims_and_strided_weight(dev):
    g = torch.Generator().manual_seed(3)
    x = torch.randn((2, 3, 64), generator=g).to(torch.bfloat16)
    wbig = torch.randn((500, 80), generator=g).to(torch.bfloat16)
    w = wbig[:, :64]                                # rows of a wider buffer (stride 80)
    out = lm_head(x.to(dev), w.to(dev))
    assert tuple(out.shape) == (2, 3, 500)
    _check_logits(out.reshape(6, 500), _ref(x.reshape(6, 64), w), 64, 1.0)


def test_softmax_from_stats_equals_softmax(dev):
    """fused_softmax(logits, row_stats=stats) is the softmax of the stored logits."""
    g = torch.Generator().manual_seed(5)
    M, V, H = 16, 151936, 128
    x = torch.randn((M, H), generator=g).to(torch.bfloat16).to(dev)
    w = (torch.randn((V, H), generator=g) * 0.3).to(torch.bfloat16).to(dev)
    logits, stats = lm_head(x, w, return_stats=True)
    p = fused_softmax(logits, row_stats=stats)
    ref = torch.softmax(logits.double().cpu(), dim=-1)
    torch.testing.assert_close(p.double().cpu(), ref, atol=1e-7, rtol=2 ** -8)
    p2, lse = fused_softmax(logits, row_stats=stats, return_lse=True)
    torch.testing.assert_close(lse.double().cpu(), torch.logsumexp(logits.double().cpu(), dim=-1), atol=2e-5, rtol=1e-6)
