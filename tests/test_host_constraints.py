"""Host side of the legality masks: bit packing and the adaptor for the
reference's constraint objects (constraints.py:53-80), on the CPU."""

import numpy as np
import torch

from lps import allowed_from_constraint, pack_allowed


def test_pack_allowed_bits_brute_force():
    g = torch.Generator().manual_seed(0)
    for V in (1, 31, 32, 33, 1000, 4099):
        m = torch.rand((3, V), generator=g) < 0.4
        words = pack_allowed(m).numpy().view(np.uint32)
        assert words.shape == (3, (V + 31) // 32)
        for r in range(3):
            for i in range(V):
                assert bool((words[r, i >> 5] >> (i & 31)) & 1) == bool(m[r, i]), (V, r, i)
            # padding bits past V stay clear
            for i in range(V, words.shape[1] * 32):
                assert not (words[r, i >> 5] >> (i & 31)) & 1


class _Tok:
    def __init__(self, table):
        self.table = table

    def decode(self, ids):
        return "".join(self.table[i] for i in ids)


class _DigitsOnly:
    """The reference protocol's mask builder (constraints.py:63-80): every id
    whose text keeps the prefix all digits; all ids when none is."""

    def _compute_legality_mask(self, prefix_text, vocab_size, tokenizer):
        legal = torch.zeros(vocab_size, dtype=torch.bool)
        for t in range(vocab_size):
            legal[t] = (prefix_text + tokenizer.decode([t])).isdigit()
        if not legal.any():
            legal[:] = True
        return legal


def test_allowed_from_constraint():
    table = ["1", "a", "22", "b", "3x", "4"]
    tok = _Tok(table)
    bits = allowed_from_constraint(_DigitsOnly(), [0], tok, len(table), "cpu").numpy().view(np.uint32)
    assert bits.shape == (1, 1)
    assert int(bits[0, 0]) == 0b100101     # ids 0, 2, 5
