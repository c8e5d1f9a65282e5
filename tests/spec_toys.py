"""Toy language models for the speculative-driver tests (CPU or GPU).

The first group restates the reference's own toy models
(``testing/unit/test_speculative_decoding.py:24-51, 166-192``), built on the
input's device.  The second group are random bigram / trigram tables whose
logits are gathers and one elementwise add, so CPU and GPU give the same bits.
"""

from __future__ import annotations

import torch

VOCAB = 32


def greedy_target(seq: torch.Tensor) -> torch.Tensor:
    """Predicts ``(last + 1) % VOCAB`` at every position (``:24-36``)."""
    B, T = seq.shape
    logits = torch.full((B, T, VOCAB), -1e9, device=seq.device)
    logits.scatter_(-1, ((seq + 1) % VOCAB).unsqueeze(-1), 1e9)
    return logits


def greedy_bad_draft(seq: torch.Tensor) -> torch.Tensor:
    """Predicts ``(last + 13) % VOCAB``: every draft is rejected (``:43-51``)."""
    B, T = seq.shape
    logits = torch.full((B, T, VOCAB), -1e9, device=seq.device)
    logits.scatter_(-1, ((seq + 13) % VOCAB).unsqueeze(-1), 1e9)
    return logits


class ToyMain:
    """``greedy_target`` plus a hidden state per position (``:166-183``)."""

    HIDDEN = 8

    def __init__(self, device="cpu"):
        g = torch.Generator().manual_seed(0)
        self.embed = torch.randn((VOCAB, self.HIDDEN), generator=g).to(device)

    def __call__(self, seq: torch.Tensor):
        return greedy_target(seq), self.embed.to(seq.device)[seq]


def toy_mtp_head(hidden: torch.Tensor, next_ids: torch.Tensor) -> torch.Tensor:
    """Predicts ``(next + 1) % VOCAB``: a perfect MTP draft (``:186-192``)."""
    B, T = next_ids.shape
    logits = torch.full((B, T, VOCAB), -1e9, device=next_ids.device)
    logits.scatter_(-1, ((next_ids + 1) % VOCAB).unsqueeze(-1), 1e9)
    return logits


class Trigram:
    """``logits[t] = E[x_t] + F[x_{t-1}]`` (``F`` term 0 at t = 0): causal,
    random, identical bits on every device."""

    def __init__(self, V: int, seed: int, scale: float = 2.0, base=None, noise: float = 0.0, device="cpu"):
        g = torch.Generator().manual_seed(seed)
        if base is None:
            self.E = torch.randn((V, V), generator=g) * scale
            self.F = torch.randn((V, V), generator=g) * (scale / 2)
        else:                                   # a draft: the base model plus noise
            self.E = base.E.cpu() + torch.randn((V, V), generator=g) * noise
            self.F = base.F.cpu() + torch.randn((V, V), generator=g) * noise
        self.E, self.F = self.E.to(device), self.F.to(device)

    def to(self, device) -> "Trigram":
        t = Trigram.__new__(Trigram)
        t.E, t.F = self.E.to(device), self.F.to(device)
        return t

    def __call__(self, seq: torch.Tensor) -> torch.Tensor:
        E, F = self.E.to(seq.device), self.F.to(seq.device)
        out = E[seq]
        prev = torch.zeros_like(out)
        prev[:, 1:] = F[seq[:, :-1]]
        return out + prev


class TrigramMain:
    """Main model for MTP tests: ``Trigram`` logits and ``hidden = H[x_t]``."""

    def __init__(self, V: int, seed: int, device="cpu"):
        self.lm = Trigram(V, seed, device=device)
        g = torch.Generator().manual_seed(seed + 1)
        self.H = torch.randn((V, 4), generator=g).to(device)

    def __call__(self, seq: torch.Tensor):
        return self.lm(seq), self.H.to(seq.device)[seq]


class TrigramMTP:
    """MTP head: ``G[next] + hidden[..., 0]`` (one elementwise add)."""

    def __init__(self, V: int, seed: int, device="cpu"):
        g = torch.Generator().manual_seed(seed + 2)
        self.G = (torch.randn((V, V), generator=g) * 2.0).to(device)

    def __call__(self, hidden: torch.Tensor, next_ids: torch.Tensor) -> torch.Tensor:
        return self.G.to(next_ids.device)[next_ids] + hidden[..., :1]


def uniform_table(n_rows: int, n_rounds: int, width: int, seed: int) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    return torch.rand((n_rows, n_rounds, width), generator=g)
