"""Seeded synthetic inputs of the BASELINE.json configurations (c1..c5),
generated on the CPU so the GPU and the oracle see identical bits.  Sizes are
parameters so parity tests can shrink V / B while keeping each config's
distribution."""

from __future__ import annotations

from dataclasses import dataclass
from typing import List, Optional

import numpy as np
import torch

V_QWEN3 = 151936


@dataclass
class Workload:
    name: str
    logits: torch.Tensor            # CPU tensor [B, V] in the config dtype
    temperature: torch.Tensor       # f32 [B]
    top_k: torch.Tensor             # i32 [B]
    top_p: torch.Tensor             # f32 [B]
    min_p: torch.Tensor
    typical_p: torch.Tensor
    rep: torch.Tensor
    pres: torch.Tensor
    freq: torch.Tensor
    histories: Optional[torch.Tensor]   # i32 [B, H]
    hist_len: Optional[torch.Tensor]    # i32 [B]
    uniforms: torch.Tensor          # f32 [B]
    logprobs: bool = False
    n_top: int = 0

    @property
    def B(self):
        return self.logits.shape[0]

    @property
    def V(self):
        return self.logits.shape[1]

    def row_history(self, i) -> List[int]:
        if self.histories is None:
            return []
        return [int(v) for v in self.histories[i, : int(self.hist_len[i])]]


def _full(B, v, dtype=torch.float32):
    return torch.full((B,), v, dtype=dtype)


def c1(V=V_QWEN3, seed=1, greedy=False, dtype=torch.float32) -> Workload:
    """B=1 fp32 N(0, 2^2) (or rounded to dtype); rep 1.1 over 64 uniform ids;
    T 0.7, k 50, p 0.9."""
    g = torch.Generator().manual_seed(seed)
    B = 1
    x = (torch.randn((B, V), generator=g) * 2.0).to(dtype)
    hist = torch.randint(0, V, (B, 64), generator=g, dtype=torch.int32)
    return Workload("c1", x, _full(B, 0.0 if greedy else 0.7), _full(B, 50, torch.int32), _full(B, 0.9),
                    _full(B, 0.0), _full(B, 1.0), _full(B, 1.1), _full(B, 0.0), _full(B, 0.0), hist,
                    _full(B, 64, torch.int32), torch.rand((B,), generator=g))


def zipf_ids(rng, n, V, s=1.1):
    ids = rng.zipf(s, size=n * 4)
    ids = ids[ids <= V][:n] - 1
    while ids.size < n:
        more = rng.zipf(s, size=n)
        ids = np.concatenate([ids, more[more <= V] - 1])[:n]
    return ids.astype(np.int32)


def c2(B=64, V=V_QWEN3, seed=2, H=512) -> Workload:
    """B=64 bf16 N(0, 3^2) + 3 spikes at +12; T ~ U[0.3, 1.2]; k in {0,20,50,100};
    p ~ U[0.8, 1.0]; presence 0.5, frequency 0.3 over 512 Zipf(1.1) ids per row."""
    g = torch.Generator().manual_seed(seed)
    rng = np.random.default_rng(seed)
    x = torch.randn((B, V), generator=g) * 3.0
    for i in range(B):
        sp = torch.randperm(V, generator=g)[:3]
        x[i, sp] = 12.0
    x = x.to(torch.bfloat16)
    T = 0.3 + 0.9 * torch.rand((B,), generator=g)
    kk = torch.tensor([0, 20, 50, 100], dtype=torch.int32)[torch.randint(0, 4, (B,), generator=g)]
    p = 0.8 + 0.2 * torch.rand((B,), generator=g)
    hist = torch.from_numpy(np.stack([zipf_ids(rng, H, V) for _ in range(B)]))
    return Workload("c2", x, T, kk, p, _full(B, 0.0), _full(B, 1.0), _full(B, 1.0), _full(B, 0.5),
                    _full(B, 0.3), hist, _full(B, H, torch.int32), torch.rand((B,), generator=g))


def c2_minp(dtype=torch.bfloat16) -> Workload:
    """c2's rows and penalties with min-p instead of top-k: top_k 0, T clamped to
    >= 0.3, min_p cycling 1e-3 / 0.02 / 0.05 / 0.1 / 0.3 / 1 / 0.05 / 0.2, top_p
    cycling 1 / 0.9 / 1 / 0.5 / 0.95, typical_p 0.6 on every ninth row (after
    top-p / min-p: the argmax)."""
    w = c2()
    w.name = "c2_minp"
    w.logits = w.logits.to(dtype)
    B = w.B
    i = torch.arange(B)
    w.top_k = torch.zeros(B, dtype=torch.int32)
    w.temperature = w.temperature.clamp(min=0.3)
    w.min_p = torch.tensor([0.001, 0.02, 0.05, 0.1, 0.3, 1.0, 0.05, 0.2])[i % 8]
    w.top_p = torch.tensor([1.0, 0.9, 1.0, 0.5, 0.95])[i % 5]
    w.typical_p = torch.where(i % 9 == 4, torch.tensor(0.6), torch.tensor(1.0))
    return w


def c2_typical(dtype=torch.bfloat16) -> Workload:
    """c2's rows and penalties with typical-p alone: top_k 0, top_p 1, T cycling
    0.3 / 0.6 / 1 / 1.5, typical_p cycling 0.2 / 0.5 / 0.9 / 0.99 / 0.7 / 0.01 /
    0.95 / 0.3 / 0.05; row 5 holds a -inf logit.  The rows' cuts fall inside
    the histogram, under it, under every logit (all kept) and above the
    maximum (the argmax)."""
    w = c2()
    w.name = "c2_typical"
    B = w.B
    i = torch.arange(B)
    w.top_k = torch.zeros(B, dtype=torch.int32)
    w.top_p = torch.ones(B)
    w.temperature = torch.tensor([0.3, 0.6, 1.0, 1.5])[i % 4]
    w.typical_p = torch.tensor([0.2, 0.5, 0.9, 0.99, 0.7, 0.01, 0.95, 0.3, 0.05])[i % 9]
    x = w.logits.to(dtype).clone()
    x[5, 1000] = float("-inf")
    w.logits = x
    return w


def c2_bigk(dtype=torch.bfloat16) -> Workload:
    """c2's rows and penalties with top_k past the fast lists and no top-p
    (the shape of a Mirostat draw at high k): top_k cycling 300 / 1000 / 5000
    / 700 / 3000 / 257 / 2048, top_p 1, T clamped to >= 0.3, typical_p 0.7 on
    every eleventh row (the argmax after top-k)."""
    w = c2()
    w.name = "c2_bigk"
    w.logits = w.logits.to(dtype)
    B = w.B
    i = torch.arange(B)
    w.top_k = torch.tensor([300, 1000, 5000, 700, 3000, 257, 2048], dtype=torch.int32)[i % 7]
    w.top_p = torch.ones(B)
    w.temperature = w.temperature.clamp(min=0.3)
    w.typical_p = torch.where(i % 11 == 5, torch.tensor(0.7), torch.tensor(1.0))
    return w


def c3(B=256, V=V_QWEN3, seed=3, flat=False) -> Workload:
    """B=256 fp32 Student-t(3)*2 (or flat N(0, 0.1^2)); top_p 0.95, T 1, no penalties."""
    g = torch.Generator().manual_seed(seed)
    rng = np.random.default_rng(seed)
    if flat:
        x = torch.randn((B, V), generator=g) * 0.1
    else:
        x = torch.from_numpy(rng.standard_t(3, size=(B, V)).astype(np.float32) * 2.0)
    return Workload("c3f" if flat else "c3", x, _full(B, 1.0), _full(B, 0, torch.int32), _full(B, 0.95),
                    _full(B, 0.0), _full(B, 1.0), _full(B, 1.0), _full(B, 0.0), _full(B, 0.0), None, None,
                    torch.rand((B,), generator=g))


def c5(B=512, V=V_QWEN3, seed=5, H=1024) -> Workload:
    """B=512 fp16 N(0, 2.5^2); half greedy, half T 0.9 / k 40 / p 0.92; rep 1.05 over
    1024 ids per row; chosen logprob + top-20 logprobs."""
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn((B, V), generator=g) * 2.5).to(torch.float16)
    greedy = torch.arange(B) % 2 == 0
    T = torch.where(greedy, torch.tensor(0.0), torch.tensor(0.9))
    kk = torch.where(greedy, torch.tensor(0), torch.tensor(40)).to(torch.int32)
    p = torch.where(greedy, torch.tensor(1.0), torch.tensor(0.92))
    hist = torch.randint(0, V, (B, H), generator=g, dtype=torch.int32)
    return Workload("c5", x, T, kk, p, _full(B, 0.0), _full(B, 1.0), _full(B, 1.05), _full(B, 0.0),
                    _full(B, 0.0), hist, _full(B, H, torch.int32), torch.rand((B,), generator=g),
                    logprobs=True, n_top=20)


@dataclass
class SpecWorkload:
    target: torch.Tensor     # [B, k+1, V] f32
    draft: torch.Tensor      # [B, k, V] f32
    draft_tokens: torch.Tensor
    u_accept: torch.Tensor
    u_resample: torch.Tensor
    temperature: float
    top_p: float


def c4(B=32, k=4, V=V_QWEN3, seed=4, temperature=0.8, top_p=0.95) -> SpecWorkload:
    """Target [32, 5, V] fp32; draft = target[:, :k] + N(0, 0.5^2); draft tokens
    sampled from the draft distribution with a seed; T 0.8, top_p 0.95."""
    g = torch.Generator().manual_seed(seed)
    tgt = torch.randn((B, k + 1, V), generator=g) * 2.0
    drf = tgt[:, :k, :] + torch.randn((B, k, V), generator=g) * 0.5
    probs = torch.softmax(drf / max(temperature, 1e-6), dim=-1).reshape(B * k, V)
    toks = torch.multinomial(probs, 1, generator=g).reshape(B, k)
    return SpecWorkload(tgt, drf, toks, torch.rand((B, k), generator=g), torch.rand((B, k + 1), generator=g),
                        temperature, top_p)
