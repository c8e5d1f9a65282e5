"""Batched speculative-decoding drivers on the GPU (``lps.spec_driver``) against
the oracle's restatement of the reference loops (``speculative.py:68-178,
206-280``), request by request, with the same uniforms: every generated token
and every counter must be equal.  Then the reference's own driver tests
(``testing/unit/test_speculative_decoding.py:59-217``) through the B = 1
signatures."""

import pytest
import torch

from lps import (SpecDecStats, mtp_speculative_decode, mtp_speculative_decode_batched, speculative_decode,
                 speculative_decode_batched)
from oracle import reference_semantics as O
from tests import spec_toys as Y

pytestmark = pytest.mark.gpu


def _prompts(B, V, seed):
    g = torch.Generator().manual_seed(seed)
    return [torch.randint(0, V, (int(torch.randint(1, 6, (1,), generator=g)),), generator=g) for _ in range(B)]


@pytest.mark.parametrize("temperature", [0.0, 0.7, 1.3])
@pytest.mark.parametrize("k", [1, 4])
@pytest.mark.parametrize("eos", [None, 5])
def test_two_model_batched_equals_oracle(dev, temperature, k, eos):
    V, B, n_new = 256, 6, 14
    target = Y.Trigram(V, 1, scale=1.5)
    draft = Y.Trigram(V, 2, base=target, noise=0.8)
    tgt_d, drf_d = target.to(dev), draft.to(dev)
    prompts = _prompts(B, V, seed=k * 10 + int(temperature * 10))
    table = Y.uniform_table(B, 64, 3 * k + 1, seed=7 + k)
    outs, stats = speculative_decode_batched(tgt_d, drf_d, [p.to(dev) for p in prompts], n_new, k, temperature,
                                             eos_token_id=eos, uniforms=lambda r, rows: table[rows, r])
    for i in range(B):
        ref, rounds, calls, acc = O.spec_decode_ref(
            target, draft, prompts[i].unsqueeze(0), n_new, k, temperature, eos,
            lambda r, i=i: (table[i, r, :k], table[i, r, k: 2 * k], table[i, r, 2 * k:]))
        got = outs[i].cpu()
        assert torch.equal(got, ref[0]), f"row {i}: {got.tolist()} vs {ref[0].tolist()}"
        assert (stats[i].rounds, stats[i].target_calls, stats[i].accepted) == (rounds, calls, acc), f"row {i}"


@pytest.mark.parametrize("temperature", [0.0, 0.9])
@pytest.mark.parametrize("eos", [None, 3])
def test_mtp_batched_equals_oracle(dev, temperature, eos):
    V, B, n_new = 128, 5, 11
    main, head = Y.TrigramMain(V, 4), Y.TrigramMTP(V, 4)
    main_d, head_d = Y.TrigramMain(V, 4, device=dev), Y.TrigramMTP(V, 4, device=dev)
    prompts = _prompts(B, V, seed=31)
    table = Y.uniform_table(B, 64, 3, seed=9)
    outs, stats = mtp_speculative_decode_batched(main_d, head_d, [p.to(dev) for p in prompts], n_new, temperature,
                                                 eos_token_id=eos, uniforms=lambda r, rows: table[rows, r])
    for i in range(B):
        ref, rounds, calls, acc = O.mtp_decode_ref(
            main, head, prompts[i].unsqueeze(0), n_new, temperature, eos,
            lambda r, i=i: (float(table[i, r, 0]), float(table[i, r, 1]), float(table[i, r, 2])))
        got = outs[i].cpu()
        assert torch.equal(got, ref[0]), f"row {i}: {got.tolist()} vs {ref[0].tolist()}"
        assert (stats[i].rounds, stats[i].target_calls, stats[i].accepted) == (rounds, calls, acc), f"row {i}"


def test_batched_rows_independent_of_batch(dev):
    """A request's tokens do not depend on the other requests in the batch."""
    V, k = 200, 3
    target = Y.Trigram(V, 5).to(dev)
    draft = Y.Trigram(V, 6, base=Y.Trigram(V, 5), noise=1.0).to(dev)
    prompts = [p.to(dev) for p in _prompts(4, V, seed=2)]
    table = Y.uniform_table(4, 64, 3 * k + 1, seed=3)
    outs, _ = speculative_decode_batched(target, draft, prompts, 12, k, 0.8, uniforms=lambda r, rows: table[rows, r])
    for i in range(4):
        one, _ = speculative_decode(target, draft, prompts[i].unsqueeze(0), 12, k, 0.8,
                                    uniforms=lambda r, rows, i=i: table[[i], r])
        assert torch.equal(one[0], outs[i])


# -- the reference's own driver tests, through the B = 1 signatures ------------
def _greedy(model, prompt, n):
    ref = prompt.clone()
    for _ in range(n):
        ref = torch.cat([ref, model(ref)[:, -1, :].argmax(dim=-1, keepdim=True)], dim=1)
    return ref[:, prompt.shape[1]:]


def test_reference_shape_and_length(dev):
    out, stats = speculative_decode(Y.greedy_target, Y.greedy_target, torch.tensor([[5, 7]], device=dev),
                                    max_new_tokens=8, k=4, temperature=0.0)
    assert out.dim() == 2 and out.shape[0] == 1 and out.shape[1] >= 8
    assert isinstance(stats, SpecDecStats)


def test_reference_perfect_draft(dev):
    prompt = torch.tensor([[3]], device=dev)
    out, _ = speculative_decode(Y.greedy_target, Y.greedy_target, prompt, max_new_tokens=10, k=4, temperature=0.0)
    assert torch.equal(out[:, :10], _greedy(Y.greedy_target, prompt, 10))
    _, stats = speculative_decode(Y.greedy_target, Y.greedy_target, torch.tensor([[1]], device=dev),
                                  max_new_tokens=20, k=4, temperature=0.0)
    assert stats.target_calls <= 6 and stats.accepted >= 16


def test_reference_bad_draft(dev):
    prompt = torch.tensor([[2]], device=dev)
    out, stats = speculative_decode(Y.greedy_target, Y.greedy_bad_draft, prompt, max_new_tokens=5, k=4,
                                    temperature=0.0)
    assert torch.equal(out[:, :5], _greedy(Y.greedy_target, prompt, 5))
    assert stats.accepted == 0


def test_reference_invalid_prompt(dev):
    with pytest.raises(ValueError, match="prompt_ids"):
        speculative_decode(Y.greedy_target, Y.greedy_target, torch.tensor([1, 2, 3], device=dev),
                           max_new_tokens=4, k=2)


def test_reference_eos(dev):
    out, _ = speculative_decode(Y.greedy_target, Y.greedy_target, torch.tensor([[5]], device=dev),
                                max_new_tokens=20, k=4, temperature=0.0, eos_token_id=6)
    assert int(out[0, 0]) == 6 and out.shape[1] <= 4


def test_reference_mtp(dev):
    main = Y.ToyMain(dev)
    prompt = torch.tensor([[7]], device=dev)
    out, stats = mtp_speculative_decode(main, Y.toy_mtp_head, prompt, max_new_tokens=10, temperature=0.0)
    assert stats.rounds <= 6
    assert torch.equal(out[:, :10], _greedy(Y.greedy_target, prompt, 10))
    out, _ = mtp_speculative_decode(main, Y.toy_mtp_head, prompt, max_new_tokens=20, temperature=0.0,
                                    eos_token_id=8)
    assert int(out[0, 0]) == 8 and out.shape[1] <= 1
