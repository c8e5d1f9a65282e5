"""The kernels' index math under host sanitizers (CPU, no GPU).

``tests/hostemu`` compiles the unchanged C ABI and kernels
(``llm-pipeline_amd/csrc/lps.hip``) for x86 with clang, over a host emulation
of the HIP subset they use, with AddressSanitizer and UndefinedBehaviorSanitizer
(array bounds included).  Every LDS array is a bounds-checked array, every
input and output is its own heap allocation of exactly its size, and the
workspace is allocated at ``lps_workspace_bytes``.  A run that reads or writes
out of bounds stops with the sanitizer's report; a run that finishes must also
match the CPU oracle row by row (the same bar as the GPU parity tests).

The emulation runs a launch's blocks one at a time, so it covers launches
whose blocks never wait for one another: row-group plans of one chunk per row
(these include the 16-bit V = 64 rows of ``test_small_vocab_mixed_params``),
and the general kernel.
"""

import hashlib
import os
import shutil
import struct
import subprocess
from types import SimpleNamespace

import numpy as np
import pytest
import torch

from tests import parity as PY
from tests import workloads as W
from tests.test_gpu_parity import _small

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)
EMU = os.path.join(HERE, "hostemu")
BUILD = os.path.join(EMU, "_build")
CLANG = "/opt/rocm/llvm/bin/clang++"
SOURCES = [os.path.join(EMU, "run_case.cpp"), os.path.join(EMU, "shim", "hip", "hip_runtime.h"),
           os.path.join(REPO, "include", "lps.h")]
CSRC = os.path.join(REPO, "llm-pipeline_amd", "csrc")

DT = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}


def _sources():
    files = list(SOURCES) + sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith((".h", ".hip")))
    h = hashlib.sha256()
    for p in files:
        h.update(open(p, "rb").read())
    return h.hexdigest()[:16]


@pytest.fixture(scope="session")
def run_case():
    if not os.path.exists(CLANG):
        pytest.skip("no ROCm clang++ for the host build")
    os.makedirs(BUILD, exist_ok=True)
    exe = os.path.join(BUILD, f"run_case_{_sources()}")
    if not os.path.exists(exe):
        for old in os.listdir(BUILD):
            if old.startswith("run_case_"):
                os.remove(os.path.join(BUILD, old))
        cmd = [CLANG, "-std=c++20", "-O0", "-g1", "-ffp-contract=off",
               "-fsanitize=address,undefined", "-fsanitize=bounds", "-fno-sanitize-recover=all",
               "-I", os.path.join(EMU, "shim"), "-I", os.path.join(REPO, "include"), "-I", CSRC,
               "-x", "c++", os.path.join(EMU, "run_case.cpp"), "-o", exe + ".tmp", "-lpthread"]
        r = subprocess.run(cmd, capture_output=True, text=True)
        assert r.returncode == 0, r.stderr[-4000:]
        shutil.move(exe + ".tmp", exe)
    return exe


def _run(exe, w, tmp_path, flags=0, workspace=True, logprobs=False, n_top=0, entropy=False, skip_draw=False):
    """One lps_sample call of workload w under the sanitizers; its outputs as a
    SampleOutput-like namespace of CPU tensors."""
    B, V = w.B, w.V
    H = 0 if w.histories is None else int(w.histories.shape[1])
    inp, out = tmp_path / "in.bin", tmp_path / "out.bin"
    with open(inp, "wb") as f:
        f.write(struct.pack("<16i", 0x4C505345, DT[w.logits.dtype], B, V, H, n_top, flags, int(workspace),
                            int(logprobs), int(entropy), int(skip_draw), 0, 0, 0, 0, 0))
        f.write(w.logits.contiguous().view(torch.int16 if w.logits.dtype != torch.float32 else torch.int32)
                .numpy().tobytes())
        for a, dt in ((w.temperature, np.float32), (w.top_k, np.int32), (w.top_p, np.float32),
                      (w.min_p, np.float32), (w.typical_p, np.float32), (w.rep, np.float32),
                      (w.pres, np.float32), (w.freq, np.float32)):
            f.write(a.numpy().astype(dt).tobytes())
        if H:
            f.write(w.histories.numpy().astype(np.int32).tobytes())
            f.write(w.hist_len.numpy().astype(np.int32).tobytes())
        f.write(w.uniforms.numpy().astype(np.float32).tobytes())
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:abort_on_error=1",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")
    r = subprocess.run([exe, str(inp), str(out)], capture_output=True, text=True, timeout=600, env=env)
    assert r.returncode == 0, f"host run failed ({r.returncode}):\n{r.stderr[-6000:]}"
    b = open(out, "rb").read()
    o = 0

    def take(dt, n):
        nonlocal o
        a = np.frombuffer(b, dtype=dt, count=n, offset=o).copy()
        o += a.nbytes
        return torch.from_numpy(a)

    res = SimpleNamespace()
    res.tokens = take(np.int64, B)
    res.status = take(np.int32, B)
    res.kept_cut = take(np.float32, B)
    res.kept_ties = take(np.int32, B)
    res.kept_count = take(np.int32, B)
    res.row_path = take(np.int32, B)
    res.chosen_logprob = take(np.float32, B) if logprobs else None
    res.top_logprobs = take(np.float32, B * n_top).reshape(B, n_top) if n_top else None
    res.top_ids = take(np.int64, B * n_top).reshape(B, n_top) if n_top else None
    res.entropy = take(np.float32, B) if entropy else None
    # deferral reasons by row (rows the fast kernels deferred)
    wst = take(np.int32, B)
    res.reasons = {i: int(wst[i]) >> 8 for i in range(B) if int(res.row_path[i]) != 0}
    assert o == len(b)
    return res


@pytest.mark.parametrize("hint", [0, 16])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_v64_mixed_params(run_case, tmp_path, dtype, hint):
    """The inputs of test_small_vocab_mixed_params at V = 64 (16-byte vector
    rows, one chunk): the row-group kernel at G = 1, then the general kernel on
    the rows it defers (top_k beyond V, top_p <= 0, T < 1e-4 ...); both builds
    of the row-group kernel (hint 16, LPS_FLAG_ROWS_BASIC_FILTERS: the one
    without the min-p / typical-p code).  In bounds, and equal to the oracle."""
    w = _small(64, 24, dtype, seed=64 + int(dtype == torch.bfloat16) * 7)
    out = _run(run_case, w, tmp_path, flags=hint)
    PY.check_rows(w, out)


@pytest.mark.parametrize("hint", [0, 16])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_v64_deferred_rows(run_case, tmp_path, dtype, hint):
    """16-bit V = 64 rows with top_k 300 (past V: every id kept, a row without
    top-k), min-p without top-k and typical-p after top-p, which the row-group
    kernel finishes itself.  With hint 16 (LPS_FLAG_ROWS_BASIC_FILTERS,
    wrong for the min-p / typical-p rows) the row-group kernel runs without
    the min-p / typical-p code and defers those rows to the general kernel
    launched after it (16-byte vector loads): still sampled exactly."""
    w = _small(64, 24, dtype, seed=71)
    i = torch.arange(24)
    w.top_k = torch.where(i % 4 == 1, torch.tensor(300, dtype=torch.int32), w.top_k)
    w.min_p = torch.where(i % 4 == 2, torch.tensor(0.05), w.min_p)
    w.typical_p = torch.where(i % 4 == 3, torch.tensor(0.8), w.typical_p)
    w.top_k = torch.where(i % 4 >= 2, torch.tensor(0, dtype=torch.int32), w.top_k)
    w.temperature = torch.where(i % 4 != 0, torch.tensor(0.9), w.temperature)
    out = _run(run_case, w, tmp_path, flags=hint)
    print("paths", out.row_path.tolist(), out.reasons)
    assert (out.row_path[i % 4 <= 1] == 0).all()
    assert (out.row_path[(i % 4 == 3) & (w.top_p >= 1)] == 1).all()
    if hint:
        assert (out.row_path[i % 4 >= 2] == 1).all()
    PY.check_rows(w, out)


@pytest.mark.parametrize("V", [7, 1000, 4099])
def test_small_vocab_scalar_rows(run_case, tmp_path, V):
    """Rows read element by element (V % 8 != 0) and a ragged vector row."""
    w = _small(V, 16, torch.bfloat16, seed=V + 7)
    PY.check_rows(w, _run(run_case, w, tmp_path))


def test_general_kernel_only(run_case, tmp_path):
    """LPS_FLAG_GENERIC: the general kernel for every row, with penalties over
    histories that span several count windows (V = 20000 > 8192 ids)."""
    w = _small(20000, 8, torch.float32, seed=5)
    rng = np.random.default_rng(5)
    w.histories = torch.from_numpy(rng.integers(-5, 20005, size=(8, 600)).astype(np.int32))
    w.hist_len = torch.tensor([0, 1, 17, 600, 599, 300, 600, 5], dtype=torch.int32)
    out = _run(run_case, w, tmp_path, flags=1, workspace=False)
    assert (out.row_path == 1).all()
    PY.check_rows(w, out)


def test_logprobs_one_chunk(run_case, tmp_path):
    """Chosen and top-N logprobs on one-chunk rows (row-group kernel), and on
    rows it defers (general kernel)."""
    w = _small(2048, 12, torch.float16, seed=9)
    w.n_top = 8
    w.logprobs = True
    out = _run(run_case, w, tmp_path, logprobs=True, n_top=8)
    PY.check_rows(w, out, lp=True)


def _flat(V, B, dtype, sigma, seed):
    """Flat rows (N(0, sigma^2) logits: thousands in one histogram bin), top_p
    0.95 and 1 (pure), T 1, no penalties."""
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn((B, V), generator=g) * sigma).to(dtype)
    f = lambda v, dt=torch.float32: torch.full((B,), v, dtype=dt)
    p = torch.tensor([0.95, 1.0, 0.6, 0.95])[torch.arange(B) % 4]
    return W.Workload("flat", x, f(1.0), f(0, torch.int32), p, f(0.0), f(1.0), f(1.0), f(0.0), f(0.0), None,
                      None, torch.rand((B,), generator=g))


def test_flat_rows_second_level(run_case, tmp_path):
    """Flat fp32 rows of one chunk: the cut and draw bins hold thousands of
    logits, more than the lists take, so the row-group kernel refines them
    with its second histogram level (fine bins of the region bins), in
    bounds; every row finishes there and matches the oracle."""
    w = _flat(12288, 8, torch.float32, 0.01, seed=11)
    out = _run(run_case, w, tmp_path)
    assert (out.row_path == 0).all(), out.reasons
    PY.check_rows(w, out)


def test_flat_rows_second_level_16bit(run_case, tmp_path):
    """Flat bf16 rows of one chunk (12288 logits: 24 per thread, the plan of
    16-bit batches of at most 12 rows): with 8 mantissa bits the logits tie in large
    groups; rows the second level resolves finish on the row-group kernel, the
    others are deferred; all match the oracle."""
    w = _flat(12288, 4, torch.bfloat16, 0.02, seed=12)
    out = _run(run_case, w, tmp_path)
    PY.check_rows(w, out)


def test_sixteen_bit_rows_past_32(run_case, tmp_path):
    """33 bf16 rows of 40960 logits: past 32 rows the plan holds 80 logits per
    thread, one chunk per row here; c2's mixed parameters and penalties, in
    bounds and equal to the oracle."""
    w = W.c2(B=33, V=40960, H=64)
    out = _run(run_case, w, tmp_path)
    assert (out.row_path == 0).all(), out.reasons
    PY.check_rows(w, out)


def test_entropy_pure_rows(run_case, tmp_path):
    """The entropy output (the first call of sample_mirostat_v2: pure rows,
    draw skipped) on one-chunk rows of the row-group kernel, and on rows with a
    penalty and non-finite values: H of softmax(x / T) within 2e-5 of the
    fp64 value; NaN where the row has no finite distribution."""
    B, V = 6, 12288
    g = torch.Generator().manual_seed(21)
    x = torch.randn((B, V), generator=g) * torch.tensor([2.0, 0.3, 6.0, 1.0, 2.0, 1.0]).view(-1, 1)
    x[4, 17] = float("nan")
    x[5] = float("-inf")
    f = lambda v, dt=torch.float32: torch.full((B,), v, dtype=dt)
    T = torch.tensor([1.0, 0.7, 1.3, 1.0, 1.0, 1.0])
    w = W.Workload("entropy", x, T, f(0, torch.int32), f(1.0), f(0.0), f(1.0), f(1.0), f(0.0), f(0.0), None,
                   None, torch.rand((B,), generator=g))
    out = _run(run_case, w, tmp_path, entropy=True, skip_draw=True)
    assert (out.row_path[:4] == 0).all(), (out.row_path.tolist(), out.reasons)
    for i in range(4):
        z = x[i].double() / float(T[i])
        p = torch.softmax(z, 0)
        h = float(-(p * torch.log_softmax(z, 0)).sum())
        assert abs(float(out.entropy[i]) - h) <= 2e-5 * max(1.0, abs(h)), (i, float(out.entropy[i]), h)
    assert np.isnan(float(out.entropy[4])) and np.isnan(float(out.entropy[5]))


def _minp_rows(V, dtype, seed):
    """Rows without top-k that the row-group kernel takes with min-p: N(0,
    sigma^2) logits (sigma 1, 2.5, 4: flatter to peaked), min_p from 1e-3 to
    1, alone (top_p 1) and after top_p 0.9 / 0.5 / 0, T 0.7 to 1.3; and
    typical-p after top-p / min-p (the argmax)."""
    B = 24
    g = torch.Generator().manual_seed(seed)
    i = torch.arange(B)
    sig = torch.tensor([1.0, 2.5, 4.0])[i % 3]
    x = (torch.randn((B, V), generator=g) * sig.view(-1, 1)).to(dtype)
    f = lambda v, dt=torch.float32: torch.full((B,), v, dtype=dt)
    T = torch.tensor([0.7, 1.0, 1.3, 1.0])[i % 4]
    mp = torch.tensor([0.001, 0.02, 0.1, 0.5, 1.0, 0.05])[i % 6]
    p = torch.tensor([1.0, 0.9, 1.0, 0.5, 0.0, 1.0, 0.9, 1.0])[i % 8]
    typ = torch.where(i % 7 == 3, torch.tensor(0.7), torch.tensor(1.0))
    return W.Workload("minp", x, T, f(0, torch.int32), p, mp, typ, f(1.0), f(0.0), f(0.0), None, None,
                      torch.rand((B,), generator=g))


@pytest.mark.parametrize("dtype,V", [(torch.float32, 12288), (torch.bfloat16, 20480), (torch.float16, 20480)])
def test_min_p_rows(run_case, tmp_path, dtype, V):
    """min-p without top-k on one-chunk rows of the row-group kernel (region 1
    covers the bins that can hold the min-p boundary; the finaliser applies the
    general kernel's test exactly), with and without top-p, and typical-p after
    them (the argmax): in bounds, and the kept sets and draws equal the
    oracle's.  Rows whose region is crowded are deferred (reason 2 + RF_WIDE)."""
    w = _minp_rows(V, dtype, seed=31 + V)
    out = _run(run_case, w, tmp_path)
    off = [i for i in range(w.B) if int(out.row_path[i]) != 0]
    print("rows off the row-group kernel:", off, out.reasons)
    assert len(off) <= 4, (off, out.reasons)
    PY.check_rows(w, out)


@pytest.mark.parametrize("dtype,V", [(torch.float32, 12288), (torch.bfloat16, 12288)])
def test_typical_p_full_rows(run_case, tmp_path, dtype, V):
    """Typical-p without top-k / top-p / min-p (sampling.py:207-238) on
    one-chunk rows of the row-group kernel: the cut z - zmax >= lnZ - exp(H)
    typical_p from the row's entropy, located like a min-p boundary when it
    lies in the histogram, counted by the chunks when it lies under it; rows
    whose cut keeps every logit run as pure rows; rows holding -inf (NaN
    entropy) and rows whose cut keeps nothing keep only the argmax.  In
    bounds, kept sets and draws equal to the oracle's."""
    B = 16
    g = torch.Generator().manual_seed(41 + V)
    i = torch.arange(B)
    sig = torch.tensor([1.0, 2.5, 4.0, 0.5])[i % 4]
    x = torch.randn((B, V), generator=g) * sig.view(-1, 1)
    x[3, 100] = float("-inf")
    x[7, :5] = float("-inf")
    # rows 12-15: N(0, 3^2) with three spikes at +9, T 0.6: the cut lies under
    # the histogram (mass ratio < 2^-31) but above the least logits
    x[12:] = torch.randn((4, V), generator=g) * 3.0
    x[12:, :3] = 9.0
    x = x.to(dtype)
    f = lambda v, dt=torch.float32: torch.full((B,), v, dtype=dt)
    T = torch.tensor([1.0, 0.7, 1.3, 1.0])[(i // 4) % 4]
    T[12:] = torch.tensor([0.6, 0.7, 0.7, 0.65])
    typ = torch.tensor([0.2, 0.5, 0.9, 0.99, 0.7, 0.01, 0.95, 0.3])[i % 8]
    typ[12:] = torch.tensor([0.9, 0.8, 0.9, 0.85])
    w = W.Workload("typical", x, T, f(0, torch.int32), f(1.0), f(0.0), typ, f(1.0), f(0.0), f(0.0), None, None,
                   torch.rand((B,), generator=g))
    # (the cut under the histogram with dropped logits, inside it, and keeping
    # everything are present; rows 3 and 7 hold -inf and keep the argmax)
    kinds = set()
    for r in range(B):
        z = x[r].double() / float(T[r])
        if torch.isinf(z).any():
            continue
        d = z - z.max()
        e = torch.exp(d)
        lnZ = torch.log(e.sum())
        H = lnZ - (e * d).sum() / e.sum()
        dmin = float(lnZ - torch.exp(H) * float(typ[r]))
        kinds.add("argmax" if dmin > 0 else "all" if float(d.min()) >= dmin else
                  "low" if dmin < np.log(2.0 ** -31) else "cut")
    assert {"all", "low", "cut"} <= kinds, kinds
    out = _run(run_case, w, tmp_path)
    off = [r for r in range(B) if int(out.row_path[r]) != 0]
    print("rows off the row-group kernel:", off, out.reasons)
    assert len(off) <= 2, (off, out.reasons)
    PY.check_rows(w, out)


def test_typical_p_rows_shorter_than_a_chunk(run_case, tmp_path):
    """Typical-p on full rows of V = 512 with penalties (the inputs of
    test_min_p_typical's typical_noinf case): the chunk's slots past its
    vectors hold -inf, which must not count as the row's -inf logits (that
    would keep only the argmax); kept sets equal the oracle's.  (Rows of
    several chunks have such slots in every chunk: the GPU test at c2's shape
    covers them.)"""
    B, V = 16, 512
    w = _small(V, B, torch.float32, seed=11)
    w.temperature = torch.full((B,), 0.8)
    w.typical_p = torch.linspace(0.2, 0.99, B)
    w.top_k = torch.zeros(B, dtype=torch.int32)
    w.top_p = torch.ones(B)
    out = _run(run_case, w, tmp_path)
    assert (out.row_path == 0).all(), out.reasons
    PY.check_rows(w, out)


@pytest.mark.parametrize("dtype,V", [(torch.float32, 12288), (torch.bfloat16, 12288)])
def test_top_k_past_the_lists(run_case, tmp_path, dtype, V):
    """top_k from 257 to V - 1 without top-p / min-p (sampling.py:139-156; the
    Mirostat draw's shape) on one-chunk rows of the row-group kernel: the
    chunks' byte counts locate the bin of the k-th largest logit, whose
    elements are region 1's candidates; every tie of the k-th value is kept;
    typical-p after it keeps the argmax.  In bounds; rows whose counts
    saturate near the cut are deferred (at most a quarter here); kept sets
    and draws equal the oracle's."""
    B = 16
    g = torch.Generator().manual_seed(51 + V)
    i = torch.arange(B)
    sig = torch.tensor([1.0, 2.5, 4.0, 0.5])[i % 4]
    x = (torch.randn((B, V), generator=g) * sig.view(-1, 1)).to(dtype)
    f = lambda v, dt=torch.float32: torch.full((B,), v, dtype=dt)
    k = torch.tensor([257, 300, 1000, 4000, V - 1, 512, 2048, 777], dtype=torch.int32)[i % 8]
    T = torch.tensor([1.0, 0.7, 1.3, 1.0])[(i // 4) % 4]
    typ = torch.where(i == 13, torch.tensor(0.8), torch.tensor(1.0))
    w = W.Workload("bigk", x, T, k, f(1.0), f(0.0), typ, f(1.0), f(0.0), f(0.0), None, None,
                   torch.rand((B,), generator=g))
    out = _run(run_case, w, tmp_path)
    off = [r for r in range(B) if int(out.row_path[r]) != 0]
    print("rows off the row-group kernel:", off, out.reasons)
    assert len(off) <= B // 4, (off, out.reasons)
    PY.check_rows(w, out)
