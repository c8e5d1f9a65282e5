#!/usr/bin/env python3
"""Benchmark of the lps token sampler on one MI355X.

A step is one ``lps_sample`` launch over one batch of synthetic logits, the
BASELINE.json configuration the metric is quoted on (c2: B=64, V=151936 bf16,
heterogeneous per-row parameters, presence/frequency penalties over 512-id
histories).  Inputs are resident in HBM before timing; launches rotate over
>= 2 x 256 MB of distinct logits buffers so the MALL cannot serve the reads,
and are replayed from a HIP graph so host overhead does not gap the GPU.

Prints ONE JSON line (rank 0, N=1) with the roofline of the sampling launch
(algorithmic bytes per launch / average launch time, against 8 TB/s) and the
CPU baseline (the oracle's op-for-op torch-CPU restatement of the reference
sampler, row by row, timed on this host's cores).  One ``lps_sample`` launch is
the row-group kernel plus the filtered general-kernel launch for deferred rows;
the launch time covers both (the filter launch is ~1-2 us when no row is
deferred), so the roofline is that of the dominant row-group kernel measured
with the short filter launch included.  Exactly ``--steps`` launches are
timed: whole replays of a captured graph, then one graph of the remainder.

``--config c4`` times ``lps_spec_verify`` (speculative-decoding verification,
32 requests, k = 4, fp32) the same way.
"""

from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import statistics
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
for _p in (os.path.join(REPO, "llm-pipeline_amd"), REPO):
    if _p not in sys.path:
        sys.path.insert(0, _p)

PEAK_HBM_GBS = 8000.0
MALL_BYTES = 256 << 20
METRIC = "sampled rows/sec at B=64,V=151936 bf16; achieved HBM GB/s vs peak"


def alg_bytes(w, n_out_extra=0) -> int:
    """Algorithmic bytes of one call: logits once, histories, per-row params
    (6 x 4 B), uniforms, token outputs, plus any logprob outputs."""
    B, V = w.B, w.V
    b = B * V * w.logits.element_size()
    if w.histories is not None:
        b += int(w.hist_len.sum()) * 4
    b += B * 24 + B * 4 + B * 8 + n_out_extra
    return b


def build_args(w, dev, logits_dev, out, lib_mod):
    from lps import _lib
    import torch
    a = _lib.SampleArgs()
    a.logits = logits_dev.data_ptr()
    a.dtype = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}[logits_dev.dtype]
    a.num_rows = w.B
    a.vocab = w.V
    a.rows_inner = 1
    a.stride_outer = logits_dev.stride(0)
    for name, t in out["params"].items():
        setattr(a, name, t.data_ptr())
    if out.get("hist") is not None:
        a.history = out["hist"].data_ptr()
        a.history_stride = out["hist"].stride(0)
        a.history_len = out["hl"].data_ptr()
    a.uniforms = out["u"].data_ptr()
    a.tokens = out["tokens"].data_ptr()
    a.row_status = out["status"].data_ptr()
    if w.logprobs:
        a.chosen_logprob = out["lp"].data_ptr()
    if w.n_top:
        a.top_logprobs = out["tl"].data_ptr()
        a.top_ids = out["ti"].data_ptr()
        a.n_top = w.n_top
    a.flags = out.get("flags", 0)
    if out.get("allowed") is not None:
        a.allowed = out["allowed"].data_ptr()
        a.allowed_stride = out["allowed"].stride(0)
    if out.get("ws") is not None:
        a.workspace = out["ws"].data_ptr()
        a.workspace_bytes = out["ws"].numel()
    return a


def fast_path_kernel(w, flags: int = 0) -> str:
    """The kernels lps_sample runs for the rows it can finish exactly (the
    launch plan of lps.hip): the row-group kernel (chunks of a row on one XCD,
    the last to arrive finalising the row) when the batch's chunk grid fits
    one resident round of the 256 CUs; for larger batches the streaming kernel
    (one workgroup per greedy / top-k row) and the row-group kernel for the
    other rows, one of them skipped by a row-kind hint."""
    import math
    from lps import _lib
    fp32 = w.logits.element_size() == 4
    vpe = 4 if fp32 else 8
    nvec = w.V // vpe
    ne = 24 if (fp32 and w.B <= 16 and math.ceil(nvec / (512 * 6)) <= 16) else 80
    G = math.ceil(nvec / (512 * (ne // vpe)))
    big = math.ceil(w.B / 8) * 8 * G > 256 and w.V <= 163840
    if not big or flags & _lib.LPS_FLAG_ROWS_NUCLEUS:
        return "rowgroup_kernel"
    if flags & _lib.LPS_FLAG_ROWS_TOPK:
        return "stream_kernel"
    return "stream_kernel + rowgroup_kernel"


def timed_replays(launch, K, Wm, nbuf, use_graph=True):
    """Exactly K timed launches (after Wm untimed ones), bracketed by HIP events
    on the launching stream: whole replays of a graph of ``per_graph``
    launches, then one graph of the remainder.  Returns ms per launch."""
    import torch
    if not use_graph:
        for i in range(Wm):
            launch(i)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for i in range(K):
            launch(i)
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / K
    per_graph = min(K, nbuf * max(1, 64 // nbuf))
    full, rem = divmod(K, per_graph)

    def capture(n):
        gr = torch.cuda.CUDAGraph()
        with torch.cuda.graph(gr):
            for i in range(n):
                launch(i)
        return gr

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for i in range(2):
            launch(i)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g_full = capture(per_graph)
    g_rem = capture(rem) if rem else None
    for _ in range(max(1, math.ceil(Wm / per_graph))):
        g_full.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(full):
        g_full.replay()
    if g_rem is not None:
        g_rem.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / K


def hbm_traffic(kernel: str, config: str):
    """HBM bytes per launch of the sampling kernels for a workload, as measured by
    rocprofv3 FETCH_SIZE + WRITE_SIZE passes and scaled by the same counters on a
    plain copy of known size (profiles/<kernel>_<config>_hbm_traffic.md,
    line 'traffic_bytes_per_launch: N'); None when no such measurement exists."""
    path = os.path.join(REPO, "profiles", f"{kernel}_{config}_hbm_traffic.md")
    try:
        with open(path) as f:
            for line in f:
                if line.strip().startswith("traffic_bytes_per_launch:"):
                    return int(line.split(":", 1)[1].strip().replace(",", ""))
    except OSError:
        return None
    return None


def copy_calibration(nbytes: int = 256 << 20, reps: int = 4):
    """A plain device-to-device copy of known size, for scaling the HBM byte
    counters (FETCH_SIZE / WRITE_SIZE read nbytes each per copy when exact)."""
    import torch
    dev = torch.device("cuda:0")
    src = torch.randint(0, 255, (nbytes,), dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(reps):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes": nbytes, "copies": reps}), flush=True)


def host_cpu():
    """The host CPU the baseline ran on: model name, os.cpu_count(), the
    cores this process may run on, and the thread share it uses (the box's
    OMP_NUM_THREADS share when set: the GPU box gives one GPU's jobs 16 of its
    host's cores, whatever os.cpu_count() reports)."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        affinity = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        affinity = os.cpu_count() or 1
    share = int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or affinity
    return {"cpu_model": model, "os_cpu_count": os.cpu_count(), "affinity_cores": affinity,
            "threads_used": max(1, min(share, affinity))}


def cpu_baseline(w, max_rows=None, repeats=3, dev=None):
    """Reference-as-written sampler (oracle restatement), one call per row with
    that row's parameters and history (continuous_batching.py:394-401)."""
    import torch
    from oracle import reference_semantics as O
    from tests import parity as PY
    hc = host_cpu()
    threads = hc["threads_used"]
    torch.set_num_threads(threads)
    rows = list(range(w.B if max_rows is None else min(w.B, max_rows)))
    x32 = w.logits.float()
    g = torch.Generator().manual_seed(0)

    def one_pass():
        for i in rows:
            O.reference_sample_token(x32[i:i + 1], PY.row_params(w, i), w.row_history(i), generator=g)

    one_pass()
    ts = []
    for _ in range(repeats):
        t0 = time.perf_counter()
        one_pass()
        ts.append(time.perf_counter() - t0)
    t = statistics.median(ts)
    out = {"value": round(len(rows) / t, 2), "unit": "rows/s", "cores": threads, "kind": "port", "host": hc,
           "sample": f"{len(rows)} rows of the {w.name} batch x {repeats} repeats (median), fp32-upcast logits, "
                     f"torch-CPU restatement of sampling.py:51-85 with torch.multinomial"}
    if dev is not None:
        # the same rows through the GPU path, checked against the restatement:
        # exact tokens, and the rows whose top-p cut or draw sits in the fp32
        # band where the reference's rounding and the exact cut may differ
        res = PY.run_workload(w, dev)
        rep = PY.check_rows(w, res, rows=rows, lp=bool(w.logprobs))
        out["parity"] = {"rows_checked": rep.rows, "exact_tokens": rep.exact_tokens,
                         "band_keep_rows": rep.band_keep, "band_draw_rows": rep.band_draw}
    return out


def engine_step(args):
    """One decode step of the c2 batch (B=64, V=151936 bf16, mixed parameters,
    512-id histories) through ``SamplerState``: one ``lps_sample`` launch that
    also appends every token to its row's history on the GPU.  Against it, the
    reference batcher's loop (``continuous_batching.py:394-404``): one
    ``sample_token`` per row with its kwargs, each token read back with
    ``.item()`` -- here run with this build's sampler and the rows' histories
    passed as the reference would pass ``generated_tokens``."""
    import torch
    from lps import SamplerState, Sampler
    from tests import workloads as W

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    w = W.c2()
    B, V = w.B, w.V
    H = int(w.histories.shape[1])
    st = SamplerState(B, V, H + args.steps + args.warmup + 8, dev)
    kws = []
    for i in range(B):
        kw = dict(temperature=float(w.temperature[i]), top_k=int(w.top_k[i]), top_p=float(w.top_p[i]),
                  presence_penalty=float(w.pres[i]), frequency_penalty=float(w.freq[i]))
        kws.append(kw)
        st.add(kw, history=w.histories[i, : int(w.hist_len[i])].tolist())
    x = w.logits.to(dev)
    us = torch.rand((args.steps + args.warmup, B), device=dev)
    for s in range(args.warmup):
        st.sample(x, us[s])
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record()
    for s in range(args.steps):
        st.sample(x, us[args.warmup + s])
    e1.record()
    torch.cuda.synchronize()
    wall_state = (time.perf_counter() - t0) / args.steps * 1e3
    gpu_state = e0.elapsed_time(e1) / args.steps

    sampler = Sampler()
    hists = [w.histories[i, : int(w.hist_len[i])].tolist() for i in range(B)]
    nref = min(args.steps, 20)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for s in range(nref):
        for i in range(B):
            t = sampler.sample_token(x[i:i + 1], kws[i], generated_tokens=hists[i], strict=False)
            hists[i].append(int(t.item()))
    torch.cuda.synchronize()
    wall_rows = (time.perf_counter() - t0) / nref * 1e3
    print(json.dumps({
        "metric": "decode step of the c2 batch: device-resident SamplerState vs the per-row loop",
        "value": round(B / (wall_state / 1e3), 1), "unit": "rows/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(wall_state, 6), "higher_is_better": True,
        "state_step_gpu_ms": round(gpu_state, 6),
        "per_row_loop_ms_per_step": round(wall_rows, 3),
        "per_row_loop_steps_timed": nref,
        "speedup": round(wall_rows / wall_state, 1),
        "data": "synthetic", "config": {"workload": "c2 rows with their parameters and 512-id histories, "
                                                    "one token appended per row per step"},
    }), flush=True)


SOFTMAX_WORKLOADS = {
    # name: (rows, cols, dtype, causal, seq_len, description)
    "logits": (64, 151936, "bfloat16", False, 1,
               "LM-head softmax producer: the c2 logits, 64 x 151936 bf16, probabilities out in bf16"),
    "attn": (32 * 2048, 2048, "bfloat16", True, 2048,
             "causal attention probabilities: 32 heads x 2048 queries x 2048 keys bf16, row_offset 0"),
}


def softmax_bench(args):
    """Row softmax (``lps_softmax``, the drop-in for the reference's
    ``fused_softmax_triton``) over one workload: every launch reads one input
    buffer and writes one output buffer, rotated over >= 2 x 256 MB, replayed
    from a HIP graph.  Algorithmic bytes: the visible (unmasked) input read
    once plus the whole output written once."""
    import torch
    from lps import _lib
    from lps import _device as D
    from lps import softmax as SM

    rows, cols, dts, causal, seq_len, desc = SOFTMAX_WORKLOADS[args.softmax]
    dtype = getattr(torch, dts)
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    lib = _lib.load()
    es = torch.tensor([], dtype=dtype).element_size()
    nb_in = rows * cols * es
    nbuf = max(2, math.ceil(2 * MALL_BYTES / nb_in))
    g = torch.Generator().manual_seed(5)
    x0 = (torch.randn((rows, cols), generator=g) * 3.0).to(dtype).to(dev)
    xs = [x0] + [x0.roll(i, dims=1) for i in range(1, nbuf)]
    outs = [torch.empty_like(x0) for _ in range(nbuf)]
    wsb = lib.lps_softmax_workspace_bytes(rows, cols, D.dtype_code(x0))
    ws = torch.zeros((max(wsb, 1),), dtype=torch.uint8, device=dev)
    arglist = []
    for x, o in zip(xs, outs):
        a = _lib.SoftmaxArgs()
        a.x, a.out, a.dtype, a.rows, a.cols = x.data_ptr(), o.data_ptr(), D.dtype_code(x), rows, cols
        a.x_stride = a.out_stride = cols
        a.causal, a.seq_len, a.row_offset = int(causal), seq_len, 0
        a.workspace, a.workspace_bytes = (ws.data_ptr(), ws.numel()) if wsb else (None, 0)
        arglist.append(a)

    def launch(i):
        rc = lib.lps_softmax(ctypes.byref(arglist[i % nbuf]), torch.cuda.current_stream().cuda_stream)
        if rc != 0:
            raise RuntimeError(f"lps_softmax failed: {rc}")

    # self-check of the timed configuration: the first rows against torch in fp64
    launch(0)
    torch.cuda.synchronize()
    chk = x0[:4].double().cpu()
    if causal:
        chk = chk.masked_fill(torch.arange(cols).unsqueeze(0) > torch.arange(4).unsqueeze(1), float("-inf"))
    ref = torch.softmax(chk, dim=-1)
    err = float(((outs[0][:4].double().cpu() - ref).abs() - 2 ** -8 * ref.abs()).max())
    assert err <= 1e-6, f"softmax self-check failed ({err})"

    per_graph = nbuf * max(1, 64 // nbuf)
    graph = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for i in range(2):
            launch(i)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    with torch.cuda.graph(graph):
        for i in range(per_graph):
            launch(i)
    for _ in range(max(1, math.ceil(args.warmup / per_graph))):
        graph.replay()
    torch.cuda.synchronize()
    reps = max(1, math.ceil(args.steps / per_graph))
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        graph.replay()
    e1.record()
    torch.cuda.synchronize()
    steps = reps * per_graph
    ms_step = e0.elapsed_time(e1) / steps
    assert all(int(t.count_nonzero()) == 0 for t in [ws]), "workspace not left zeroed"

    visible = sum(min(cols, (r % seq_len) + 1) for r in range(rows)) if causal else rows * cols
    abytes = visible * es + rows * cols * es
    gbs = abytes / (ms_step / 1e3) / 1e9
    plan = "softmax_wave_kernel" if cols <= (2048 if es == 4 else 4096) else (
        "softmax_chunk_kernel (rows split over workgroups)" if wsb else "softmax_chunk_kernel")

    cpu = None
    if not args.no_cpu_baseline:
        threads = host_cpu()["threads_used"]
        torch.set_num_threads(threads)
        n = rows if not causal else 2048
        xc = x0[:n].cpu()

        def ref_cpu():
            xm = xc
            if causal:
                xm = xc.masked_fill(torch.arange(cols).unsqueeze(0) > torch.arange(n).unsqueeze(1), float("-inf"))
            return torch.softmax(xm.float(), dim=-1).to(dtype)

        ref_cpu()   # thread pool and allocator warm
        ts = []
        for _ in range(10):
            t0 = time.perf_counter()
            ref_cpu()
            ts.append(time.perf_counter() - t0)
        t = statistics.median(ts)
        cpu_vis = visible if not causal else sum(min(cols, (r % seq_len) + 1) for r in range(n))
        cpu_bytes = cpu_vis * es + n * cols * es
        cpu = {"value": round(cpu_bytes / t / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port", "host": host_cpu(),
               "sample": f"{n} rows of the workload, torch-CPU restatement of triton_softmax.py:105-113 "
                         f"(masked_fill, softmax in fp32, cast back), median of 10 after one warm-up call"}

    print(json.dumps({
        "metric": f"row softmax achieved HBM GB/s ({args.softmax})",
        "value": round(gbs, 1), "unit": "GB/s", "n_gpus": 1, "steps": steps, "warmup": args.warmup,
        "ms_per_step": round(ms_step, 6), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32", "data": "synthetic",
        "rows_per_s": round(rows / (ms_step / 1e3), 1),
        "config": {"workload": desc, "rows": rows, "cols": cols, "input_dtype": dts, "causal": causal,
                   "buffers_rotated": nbuf, "hip_graph": True, "algorithmic_bytes_per_call": abytes,
                   "kernel": plan},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(gbs / PEAK_HBM_GBS, 4),
                     "traffic": hbm_traffic("softmax", args.softmax)},
        "cpu_baseline": cpu,
    }), flush=True)


def spec_driver_bench(args):
    """Batched two-model speculative decoding (``speculative_decode_batched``,
    the batched form of ``speculative.py:68-178``) at c2's shape: 64 requests,
    V = 151936 bf16, k = 4, T = 1.  The forwards cost nothing (each request's
    target logits are a fixed random row, the draft's the same row plus noise,
    at every position), so the time is the driver's own: k draft-sampling
    launches, the gathers, one ``lps_spec_verify`` launch and one read-back per
    round.  Reported: generated tokens/s and ms per round; the CPU baseline is
    the oracle's restatement of the reference loop, one request, two rounds."""
    import torch
    from lps import speculative_decode_batched

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    B, V, k, T = 64, 151936, 4, 1.0
    g = torch.Generator(device=dev).manual_seed(3)
    tgt = (torch.randn((B, V), generator=g, device=dev) * 3.0).to(torch.bfloat16)
    drf = (tgt.float() + torch.randn((B, V), generator=g, device=dev) * 0.7).to(torch.bfloat16)

    class Fixed:
        def __init__(self, tbl):
            self.tbl = tbl

        def __call__(self, x):
            b, L = x.shape
            return self.tbl[:b].unsqueeze(1).expand(b, L, V)

    prompts = torch.randint(0, V, (B, 8), device=dev)
    ug = torch.Generator(device=dev).manual_seed(5)
    speculative_decode_batched(Fixed(tgt), Fixed(drf), prompts, 10, k, T, generator=ug)   # warm-up
    torch.cuda.synchronize()
    n_new = max(20, args.steps // 10)
    t0 = time.perf_counter()
    outs, stats = speculative_decode_batched(Fixed(tgt), Fixed(drf), prompts, n_new, k, T, generator=ug)
    torch.cuda.synchronize()
    dt = time.perf_counter() - t0
    tokens = sum(int(o.numel()) for o in outs)
    rounds = max(s.rounds for s in stats)
    acc = sum(s.accepted for s in stats) / max(1, sum(s.rounds for s in stats))

    cpu = None
    if not args.no_cpu_baseline:
        from oracle import reference_semantics as O
        tc, dc = tgt[:1].float().cpu(), drf[:1].float().cpu()
        fc = lambda tbl: (lambda x: tbl.unsqueeze(1).expand(x.shape[0], x.shape[1], V))
        gu = torch.Generator().manual_seed(1)
        t1 = time.perf_counter()
        out, r_cpu, _, _ = O.spec_decode_ref(fc(tc), fc(dc), prompts[:1].cpu(), 2 * (k + 1), k, T, None,
                                             lambda r: (torch.rand(k, generator=gu), torch.rand(k, generator=gu),
                                                        torch.rand(k + 1, generator=gu)))
        tcpu = time.perf_counter() - t1
        cpu = {"value": round(out.numel() / tcpu, 2), "unit": "tokens/s", "cores": torch.get_num_threads(),
               "kind": "port", "host": host_cpu(), "sample": f"one request, {r_cpu} rounds of the oracle's restatement of "
                                          f"speculative.py:68-178 (fp32 CPU, same synthetic logits)"}
    print(json.dumps({
        "metric": "batched speculative decoding, generated tokens/s (driver and sampling only)",
        "value": round(tokens / dt, 1), "unit": "tokens/s", "n_gpus": 1, "steps": rounds, "warmup": 1,
        "ms_per_step": round(dt / rounds * 1e3, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "accepted_per_round": round(acc, 3),
        "config": {"workload": "64 requests, V=151936 bf16, k=4, T=1; forwards are fixed random rows (target) "
                               "and the same rows plus N(0, 0.7^2) noise (draft)",
                   "rounds": rounds, "generated_tokens": tokens},
        "cpu_baseline": cpu,
    }), flush=True)


def lm_head_bench(args):
    """LM-head projection with the statistics epilogue (``lps_lm_head``) at the
    c2 decode shape of a Qwen3-8B head: 64 rows, H = 4096, V = 151936, bf16.
    Timed from HIP graphs of back-to-back launches.  Algorithmic bytes: the
    weight, the hidden rows, the logits and the block statistics, each once.
    Beside it: ``torch.matmul`` (hipBLASLt) on the same operands, and the
    softmax producer both ways (projection + statistics + one-pass softmax, vs
    projection + the two-pass softmax)."""
    import torch
    from lps import _device as D
    from lps import _lib, fused_softmax, lm_head

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    M, H, V = 64, 4096, 151936
    g = torch.Generator(device=dev).manual_seed(2)
    x = torch.randn((M, H), generator=g, device=dev).to(torch.bfloat16)
    w = (torch.randn((V, H), generator=g, device=dev) * 0.02).to(torch.bfloat16)
    G = (V + 127) // 128
    out = torch.empty((M, V), dtype=torch.bfloat16, device=dev)
    stats = torch.empty((M, G, 2), dtype=torch.float32, device=dev)
    lib = _lib.load()
    a = _lib.LmHeadArgs()
    a.x, a.w, a.out, a.stats = x.data_ptr(), w.data_ptr(), out.data_ptr(), stats.data_ptr()
    a.dtype = a.out_dtype = D.dtype_code(x)
    a.rows, a.vocab, a.hidden = M, V, H
    a.x_stride, a.w_stride, a.out_stride = H, H, V

    def ours():
        rc = lib.lps_lm_head(ctypes.byref(a), torch.cuda.current_stream().cuda_stream)
        if rc != 0:
            raise RuntimeError(f"lps_lm_head failed: {rc}")

    # self-check on a few rows against fp32 torch
    ours()
    torch.cuda.synchronize()
    ref = x[:4].float() @ w.float().T
    assert float(((out[:4].float() - ref).abs() - 2 ** -8 * ref.abs()).max()) < 1e-3, "lm_head self-check failed"

    def graph_of(fn, reps):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        gr = torch.cuda.CUDAGraph()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            fn()
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        with torch.cuda.graph(gr):
            for _ in range(reps):
                fn()
        gr.replay()
        torch.cuda.synchronize()
        return gr

    logits = torch.empty_like(out)

    def fused_pipeline():
        lo, st = lm_head(x, w, return_stats=True)
        fused_softmax(lo, row_stats=st)

    def plain_pipeline():
        torch.matmul(x, w.T, out=logits)
        fused_softmax(logits)

    # the candidates are replayed in turn, round after round (the GPU's state
    # drifts over a long run of one kernel); medians over the rounds
    reps = 10
    rounds = max(5, min(40, args.steps // 50))
    graphs = {"ours": graph_of(ours, reps), "blas": graph_of(lambda: torch.matmul(x, w.T, out=out), reps),
              "fused": graph_of(fused_pipeline, reps), "plain": graph_of(plain_pipeline, reps)}
    times = {k: [] for k in graphs}
    for _ in range(rounds):
        for k, gr in graphs.items():
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            gr.replay()
            e1.record()
            torch.cuda.synchronize()
            times[k].append(e0.elapsed_time(e1) / reps)
    t_ours, t_blas = statistics.median(times["ours"]), statistics.median(times["blas"])
    t_fused, t_plain = statistics.median(times["fused"]), statistics.median(times["plain"])
    abytes = V * H * 2 + M * H * 2 + M * V * 2 + M * G * 8
    gbs = abytes / (t_ours / 1e3) / 1e9

    cpu = None
    if not args.no_cpu_baseline:
        vs = 16384
        xc, wc = x[:8].float().cpu(), w[:vs].float().cpu()
        torch.matmul(xc, wc.T)
        ts = []
        for _ in range(5):
            t0 = time.perf_counter()
            torch.matmul(xc, wc.T)
            ts.append(time.perf_counter() - t0)
        t = statistics.median(ts)
        cb = vs * H * 2 + 8 * H * 2 + 8 * vs * 2
        cpu = {"value": round(cb / t / 1e9, 3), "unit": "GB/s", "cores": torch.get_num_threads(), "kind": "port", "host": host_cpu(),
               "sample": f"8 rows x {vs} vocabulary rows of the workload, torch-CPU fp32 matmul (the reference's "
                         f"nn.Linear on the CPU), bf16-equivalent bytes, median of 5"}
    print(json.dumps({
        "metric": "LM-head projection + softmax statistics, achieved HBM GB/s (64 x 4096 -> 151936 bf16)",
        "value": round(gbs, 1), "unit": "GB/s", "n_gpus": 1, "steps": reps * rounds, "warmup": 4,
        "ms_per_step": round(t_ours, 5), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16 in, f32 accumulate", "data": "synthetic",
        "torch_matmul_ms": round(t_blas, 5),
        "softmax_producer_ms": {"lm_head+stats -> one-pass softmax": round(t_fused, 5),
                                "torch.matmul -> two-pass softmax": round(t_plain, 5)},
        "config": {"workload": "c2 decode rows through a Qwen3-8B-shaped head: x [64, 4096] bf16, "
                               "w [151936, 4096] bf16 (random), logits bf16 + 128-column block statistics",
                   "algorithmic_bytes_per_call": abytes, "kernel": "lmhead_kernel<bf16, bf16>"},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(gbs / PEAK_HBM_GBS, 4), "traffic": hbm_traffic("lmhead", "c2")},
        "cpu_baseline": cpu,
    }), flush=True)


def spec_bench(args):
    """c4: speculative-decoding verification (``lps_spec_verify``, the drop-in
    for ``speculative.py:119-174``): 32 requests, k = 4, target logits
    [32, 5, 151936] and draft logits [32, 4, 151936] fp32, T 0.8, top_p 0.95.
    A step is one launch: both distributions' top-p filters and softmaxes, the
    accept tests, and the replacement or bonus draw of every request.
    Algorithmic bytes: both logits tensors once, the drafts and uniforms, and
    the outputs."""
    import torch
    from lps import _device as D
    from lps import _lib
    from tests import workloads as W

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    sw = W.c4()
    B, k1, V = sw.target.shape
    k = k1 - 1
    tgt0, drf0 = sw.target.to(dev), sw.draft.to(dev)
    nb = (tgt0.numel() + drf0.numel()) * 4
    nbuf = max(2, math.ceil(2 * MALL_BYTES / nb))
    tgts = [tgt0] + [tgt0.clone() for _ in range(nbuf - 1)]
    drfs = [drf0] + [drf0.clone() for _ in range(nbuf - 1)]
    tok = sw.draft_tokens.to(dev, torch.int64).contiguous()
    ua = sw.u_accept.to(dev, torch.float32).contiguous()
    ur = sw.u_resample.to(dev, torch.float32).contiguous()
    lib = _lib.load()
    ws = torch.zeros((max(lib.lps_spec_workspace_bytes(B, k, V), 1),), dtype=torch.uint8, device=dev)
    n_acc = torch.empty((B,), dtype=torch.int32, device=dev)
    toks = torch.empty((B, k1), dtype=torch.int64, device=dev)
    acc = torch.empty((B, k), dtype=torch.int8, device=dev)
    pt = torch.empty((B, k), dtype=torch.float32, device=dev)
    qd = torch.empty((B, k), dtype=torch.float32, device=dev)
    st = torch.empty((B * (2 * k + 1),), dtype=torch.int32, device=dev)
    arglist = []
    for t, d in zip(tgts, drfs):
        a = _lib.SpecArgs()
        a.target_logits, a.target_stride_b, a.target_stride_k = t.data_ptr(), t.stride(0), t.stride(1)
        a.draft_logits, a.draft_stride_b, a.draft_stride_k = d.data_ptr(), d.stride(0), d.stride(1)
        a.dtype, a.batch, a.k, a.vocab = D.dtype_code(t), B, k, V
        a.temperature, a.top_p = float(sw.temperature), float(sw.top_p)
        a.residual = _lib.LPS_RESIDUAL_TARGET
        a.draft_tokens, a.u_accept, a.u_resample = tok.data_ptr(), ua.data_ptr(), ur.data_ptr()
        a.n_accepted, a.tokens, a.accept = n_acc.data_ptr(), toks.data_ptr(), acc.data_ptr()
        a.p_target, a.q_draft, a.row_status = pt.data_ptr(), qd.data_ptr(), st.data_ptr()
        a.workspace, a.workspace_bytes = ws.data_ptr(), ws.numel()
        arglist.append(a)

    def launch(i):
        rc = lib.lps_spec_verify(ctypes.byref(arglist[i % nbuf]), torch.cuda.current_stream().cuda_stream)
        if rc != 0:
            raise RuntimeError(f"lps_spec_verify failed: {rc}")

    launch(0)
    torch.cuda.synchronize()
    assert int(st.ne(0).sum()) == 0, "row status errors"
    ms_step = timed_replays(launch, args.steps, args.warmup, nbuf, not args.no_graph)
    abytes = nb + B * k * (8 + 4) + B * k1 * 4 + B * 4 + B * k1 * 8 + B * k * (1 + 4 + 4) + B * (2 * k + 1) * 4
    gbs = abytes / (ms_step / 1e3) / 1e9

    cpu = None
    if not args.no_cpu_baseline:
        from oracle import reference_semantics as O
        threads = host_cpu()["threads_used"]
        torch.set_num_threads(threads)
        nr = 8
        args_ref = (sw.target[:nr], sw.draft[:nr], sw.draft_tokens[:nr], sw.u_accept[:nr], sw.u_resample[:nr],
                    sw.temperature, sw.top_p)
        n_ref = O.spec_verify_ref(*args_ref)[0]
        ts = []
        for _ in range(3):
            t0 = time.perf_counter()
            O.spec_verify_ref(*args_ref)
            ts.append(time.perf_counter() - t0)
        t = statistics.median(ts)
        # agreement of the timed launch with the restatement on the sampled requests
        # (an accept test within 1e-5 of its uniform may go either way)
        same = int((n_acc[:nr].cpu() == n_ref).sum())
        cpu = {"value": round(nr / t, 2), "unit": "requests/s", "cores": threads, "kind": "port", "host": host_cpu(),
               "sample": f"{nr} of the 32 requests x 3 repeats (median): the oracle's torch-CPU restatement of "
                         f"speculative.py:119-174 (top-p, softmax, accept tests, resample) on the same logits",
               "parity": {"requests_checked": nr, "n_accepted_equal": same}}
    print(json.dumps({
        "metric": "speculative verification, requests/sec (c4: B=32, k=4, V=151936 fp32)",
        "value": round(B / (ms_step / 1e3), 1), "unit": "requests/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_step, 6), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": "c4: target [32, 5, 151936] fp32, draft = target[:, :4] + N(0, 0.5^2), draft tokens "
                               "sampled from the draft, T 0.8, top_p 0.95, reference residual",
                   "logits_buffers_rotated": nbuf, "hip_graph": not args.no_graph,
                   "algorithmic_bytes_per_call": abytes, "kernel": "rowgroup_kernel (target and draft rows) + "
                                                                  "spec verify kernels"},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(gbs / PEAK_HBM_GBS, 4), "traffic": hbm_traffic("spec_verify", "c4")},
        "cpu_baseline": cpu,
    }), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--config", default="c2", choices=["c1", "c1g", "c1h", "c2", "c2m", "c2t", "c2k", "c3", "c3f", "c4", "c5"])
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-graph", action="store_true")
    ap.add_argument("--generic", action="store_true", help="time the general one-workgroup-per-row kernel")
    ap.add_argument("--allowed-frac", type=float, default=None,
                    help="add a random legality mask with this fraction of legal ids per row")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a plain 256 MB device copy (counter calibration for rocprofv3 --pmc)")
    ap.add_argument("--engine-step", action="store_true",
                    help="time a decode step of the c2 batch through SamplerState (device-resident parameters "
                         "and histories, one launch) against the reference batcher's per-row loop")
    ap.add_argument("--softmax", choices=sorted(SOFTMAX_WORKLOADS), default=None,
                    help="time the row softmax (lps_softmax) on a workload instead of the sampler")
    ap.add_argument("--spec-driver", action="store_true",
                    help="time the batched speculative-decoding driver (zero-cost synthetic forwards)")
    ap.add_argument("--lm-head", action="store_true",
                    help="time the LM-head projection with the softmax statistics epilogue")
    args = ap.parse_args()
    if args.lm_head:
        lm_head_bench(args)
        return
    if args.spec_driver:
        spec_driver_bench(args)
        return
    if args.softmax:
        if args.gpus != 1:
            print("bench.py runs on one GPU only", file=sys.stderr)
            sys.exit(2)
        softmax_bench(args)
        return
    if args.copy_calibration:
        copy_calibration()
        return
    if args.engine_step:
        engine_step(args)
        return
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (asked for --gpus {args.gpus}); the sampler shards rows across "
              f"GPUs with no exchange, which this single-GPU build does not launch.", file=sys.stderr)
        sys.exit(2)
    if args.config == "c4":
        spec_bench(args)
        return

    import torch
    from lps import _lib
    from tests import workloads as W

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    make = {"c1": lambda: W.c1(), "c1g": lambda: W.c1(greedy=True), "c1h": lambda: W.c1(dtype=torch.bfloat16), "c2": lambda: W.c2(), "c2m": lambda: W.c2_minp(), "c2t": lambda: W.c2_typical(), "c2k": lambda: W.c2_bigk(),
            "c3": lambda: W.c3(), "c3f": lambda: W.c3(flat=True), "c5": lambda: W.c5()}[args.config]
    w = make()
    lib = _lib.load()

    # device inputs; rotate distinct logits buffers over >= 2 x MALL
    x = w.logits.to(dev)
    nbuf = max(2, math.ceil(2 * MALL_BYTES / (x.numel() * x.element_size())))
    bufs = [x] + [x.clone() for _ in range(nbuf - 1)]
    B = w.B
    io = {
        "params": {
            "temperature": w.temperature.to(dev), "top_k": w.top_k.to(dev), "top_p": w.top_p.to(dev),
            "min_p": w.min_p.to(dev), "typical_p": w.typical_p.to(dev), "repetition_penalty": w.rep.to(dev),
            "presence_penalty": w.pres.to(dev), "frequency_penalty": w.freq.to(dev),
        },
        "hist": w.histories.to(dev) if w.histories is not None else None,
        "hl": w.hist_len.to(dev) if w.hist_len is not None else None,
        "u": w.uniforms.to(dev),
        "tokens": torch.empty(B, dtype=torch.int64, device=dev),
        "status": torch.empty(B, dtype=torch.int32, device=dev),
        "lp": torch.empty(B, dtype=torch.float32, device=dev),
        "tl": torch.empty((B, max(w.n_top, 1)), dtype=torch.float32, device=dev),
        "ti": torch.empty((B, max(w.n_top, 1)), dtype=torch.int64, device=dev),
    }
    # row-kind hint from the host-side parameters (as Sampler.sample_token
    # passes it): a large batch launches only the kernels its rows need
    from lps import row_kind_flags
    io["flags"] = (_lib.LPS_FLAG_GENERIC if args.generic
                   else row_kind_flags(w.temperature, w.top_k, w.min_p, w.typical_p))
    if args.allowed_frac is not None:
        from lps import pack_allowed
        gm = torch.Generator().manual_seed(11)
        io["allowed"] = pack_allowed((torch.rand((B, w.V), generator=gm) < args.allowed_frac).to(dev))
    wsb = lib.lps_workspace_bytes(B, w.V, io["flags"])
    io["ws"] = torch.zeros((max(wsb, 1),), dtype=torch.uint8, device=dev) if wsb else None
    arglist = [build_args(w, dev, b, io, lib) for b in bufs]
    extra = (B * 4 + B * w.n_top * 12) if w.logprobs else 0
    if io.get("allowed") is not None:
        extra += B * ((w.V + 31) // 32) * 4  # the legality bits, read once
    abytes = alg_bytes(w, extra)

    def launch(i):
        rc = lib.lps_sample(ctypes.byref(arglist[i % nbuf]), torch.cuda.current_stream().cuda_stream)
        if rc != 0:
            raise RuntimeError(f"lps_sample failed: {rc}")

    # the timed configuration must run clean (every row status 0); the rows the
    # row-group kernel deferred to the general kernel are counted
    launch(0)
    torch.cuda.synchronize()
    assert int(io["status"].ne(0).sum()) == 0, "row status errors"
    rp = torch.full((B,), -1, dtype=torch.int32, device=dev)
    a_chk = build_args(w, dev, bufs[0], io, lib)
    a_chk.row_path = rp.data_ptr()
    rc = lib.lps_sample(ctypes.byref(a_chk), torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert rc == 0 and int(io["status"].ne(0).sum()) == 0, "row status errors"
    deferred = int(rp.ne(0).sum())

    K, Wm = args.steps, args.warmup
    use_graph = not args.no_graph
    ms_step = timed_replays(launch, K, Wm, nbuf, use_graph)
    steps = K
    rows_s = B / (ms_step / 1e3)
    gbs = abytes / (ms_step / 1e3) / 1e9
    assert int(io["status"].ne(0).sum()) == 0

    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(w, max_rows=64 if B > 64 else None, dev=dev)

    cfg = {"workload": {"c1": "c1: B=1, V=151936 fp32, rep 1.1 over 64 ids, T 0.7, top_k 50, top_p 0.9",
                        "c1g": "c1 greedy: B=1, V=151936 fp32, rep 1.1, T=0",
                        "c1h": "c1 in bf16: B=1, V=151936 bf16 (c1's logits rounded), rep 1.1 over 64 ids, T 0.7, "
                               "top_k 50, top_p 0.9",
                        "c2": "c2: B=64, V=151936 bf16 N(0,3^2)+3 spikes, T~U[0.3,1.2], top_k in {0,20,50,100}, "
                              "top_p~U[0.8,1], presence 0.5, frequency 0.3 over 512 Zipf(1.1) ids/row",
                        "c2m": "c2 with min-p: c2's rows and penalties, top_k 0, T>=0.3, min_p in "
                               "{1e-3,0.02,0.05,0.1,0.2,0.3,1}, top_p in {1,0.9,0.5,0.95}, typical_p 0.6 on 1 row in 9",
                        "c2t": "c2 with typical-p: c2's rows and penalties, top_k 0, top_p 1, T in {0.3,0.6,1,1.5}, "
                               "typical_p in {0.01,...,0.99}, one row holding -inf",
                        "c2k": "c2 with large top-k: c2's rows and penalties, top_k in {257,...,5000}, top_p 1, "
                               "T>=0.3, typical_p 0.7 on 1 row in 11",
                        "c3": "c3: B=256, V=151936 fp32 Student-t(3)*2, top_p 0.95, T 1",
                        "c3f": "c3 flat: B=256, V=151936 fp32 N(0,0.1^2), top_p 0.95, T 1",
                        "c5": "c5: B=512, V=151936 fp16, half greedy, half T 0.9/k 40/p 0.92, rep 1.05 over "
                              "1024 ids/row, chosen + top-20 logprobs"}[args.config],
           "batch_rows": B, "vocab": w.V, "input_dtype": str(w.logits.dtype).replace("torch.", ""),
           "logits_buffers_rotated": nbuf, "hip_graph": use_graph, "algorithmic_bytes_per_call": abytes,
           "kernel": "gen_row_kernel" if args.generic else fast_path_kernel(w, io["flags"]) + " + gen_row_kernel (deferred-row filter)",
           "deferred_rows": int(deferred)}
    if args.allowed_frac is not None:
        cfg["legality_mask"] = f"random, {args.allowed_frac:.0%} of ids legal per row, packed bits"
    line = {
        "metric": METRIC if args.config == "c2" else f"sampled rows/sec ({args.config})",
        "value": round(rows_s, 1),
        "unit": "rows/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": Wm,
        "ms_per_step": round(ms_step, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": cfg,
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(gbs / PEAK_HBM_GBS, 4),
                     "traffic": None if args.generic else hbm_traffic(fast_path_kernel(w, io["flags"]).split(" ")[0], args.config)},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
