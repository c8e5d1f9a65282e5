"""Device-resident sampler state (LPS_FLAG_APPEND_HISTORY): one launch per step
samples every active row and the kernel appends each token to its row's
history.  Every step must equal the host-managed loop the reference batcher
implies (sample, read the tokens back, append them to host lists, pass the
lists back as histories: continuous_batching.py:394-404, sampling.py:125), on
the fast and general paths, through request removal and a full history row."""

import pytest
import torch

from lps import SamplerState, SamplingParams, pad_histories, sample_rows
from tests import parity as PY
from tests import workloads as W

pytestmark = pytest.mark.gpu


def _oracle_step(x, kws, st, host, u, out):
    """Every row of one batcher step against the oracle's sample_row on the
    host-kept histories (continuous_batching.py:394-404: one
    sample_token(logits[i:i+1], kwargs_i) per row, generated_tokens as the
    history, sampling.py:125)."""
    n = len(kws)
    cfgs = [st.config_for(k) for k in kws]
    col = lambda f, dt=torch.float32: torch.tensor([getattr(c, f) for c in cfgs], dtype=dt)
    H = max(1, max(len(h) for h in host))
    hist = torch.zeros((n, H), dtype=torch.int32)
    for i, h in enumerate(host):
        hist[i, :len(h)] = torch.tensor(h, dtype=torch.int32)
    w = W.Workload("state", x.cpu(), col("temperature"), col("top_k", torch.int32), col("top_p"), col("min_p"),
                   col("typical_p"), col("repetition_penalty"), col("presence_penalty"), col("frequency_penalty"),
                   hist, torch.tensor([len(h) for h in host], dtype=torch.int32), u.cpu())
    return PY.check_rows(w, out)


def _kwargs(B, seed):
    g = torch.Generator().manual_seed(seed)
    out = []
    for i in range(B):
        kw = dict(temperature=float(0.3 + 0.9 * torch.rand((), generator=g)),
                  top_k=int([0, 20, 50][i % 3]), top_p=float(0.8 + 0.2 * torch.rand((), generator=g)),
                  repetition_penalty=1.1, presence_penalty=0.5, frequency_penalty=0.3)
        if i == 1:
            kw["temperature"] = 0.0                 # greedy
        out.append(kw)
    return out


def _params(st, kws, dev):
    cfgs = [st.config_for(k) for k in kws]
    return SamplingParams.from_configs(cfgs, dev)


@pytest.mark.parametrize("path", ["auto", "generic"])
def test_state_steps_equal_host_loop(dev, path):
    B, V, cap, steps = 12, 151936, 64, 6
    st = SamplerState(B, V, cap, dev)
    kws = _kwargs(B, 3)
    g = torch.Generator().manual_seed(7)
    host = []
    for kw in kws:
        seed = torch.randint(0, 200, (5,), generator=g).tolist()   # small ids: repeats across rows and steps
        st.add(kw, history=seed)
        host.append(list(seed))
    for s in range(steps):
        if s == 3:                                  # two requests finish: the batcher compacts its rows
            for r in (7, 2):
                del kws[r]
                del host[r]
            st.remove([2, 7])
        n = len(kws)
        x = (torch.randn((n, V), generator=g) * 3.0).to(torch.bfloat16)
        x[:, :200] += 4.0                           # the history ids are likely picks
        x = x.to(dev)
        u = torch.rand((n,), generator=g).to(dev)
        out = st.sample(x, u, path=path, kept_set=True)
        rep = _oracle_step(x, kws, st, host, u, out)
        print(f"step {s} ({path}): {rep}", flush=True)
        hist, hl = pad_histories(host, dev)
        ref = sample_rows(x, _params(st, kws, dev), u, histories=hist, history_lengths=hl, path=path)
        torch.cuda.synchronize(dev)
        t, tr = out.tokens.cpu(), ref.tokens.cpu()
        assert torch.equal(t, tr), f"step {s}: {t.tolist()} vs {tr.tolist()}"
        for i in range(n):
            if int(tr[i]) >= 0 and len(host[i]) < cap:
                host[i].append(int(tr[i]))
    for i in range(len(host)):
        assert st.history(i) == host[i], f"row {i}"


def test_state_full_history_row_is_kept(dev):
    V, cap = 4096, 7
    st = SamplerState(2, V, cap, dev)
    st.add({"temperature": 0.0}, history=[1, 2, 3, 4, 5])
    st.add({"temperature": 1.0, "top_k": 0, "top_p": 1.0}, history=[])
    g = torch.Generator().manual_seed(1)
    seen = [[1, 2, 3, 4, 5], []]
    for s in range(4):
        x = torch.randn((2, V), generator=g).to(dev)
        out = st.sample(x, torch.rand((2,), generator=g).to(dev))
        t = out.tokens.cpu().tolist()
        for i in range(2):
            if len(seen[i]) < cap:
                seen[i].append(t[i])
    assert st.history(0) == seen[0] and len(seen[0]) == cap
    assert st.history(1) == seen[1] and len(seen[1]) == 4
