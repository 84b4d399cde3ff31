#!/usr/bin/env python3
"""Benchmark of the vocabulary-parallel cross entropy on one MI355X.

    python bench.py [--steps K] [--warmup W] [--workload c1..c5 [--two-pass]] [--gpus 1]
    python bench.py --gemm-core     (the fused path's GEMM core beside hipBLASLt)

Unfused workloads (c1-c3): a step is one forward + backward of the loss over
one batch of synthetic logits already resident in HBM, through the drop-in
``nmce.vocab_parallel_cross_entropy`` exactly as nano-megatron's GPT.forward
calls it (model.py:277-281): target validation, per-shard statistics, the
cross-shard combine, ``loss.mean()``, ``loss.backward()`` with the gradient
written in place into the (non-leaf) logits.

Fused workloads (c4, c5): a step is one forward + backward of
``nmce.lmhead_vocab_parallel_cross_entropy(hidden, weight, target, ...)``,
the LM-head projection (model.py:192) and the loss without stored logits:
target validation, the MFMA statistics GEMM, the combine, ``loss.mean()``
and ``loss.backward()`` producing the hidden and weight gradients.

Workloads:
  c2 (default)  TP=1, bf16 logits [8,2048,50304] ~ N(0,1), targets U[0,V)
  c3            one TP=2 rank's shard: bf16 [4,4096,64128] at vocab offset
                64128 ~ N(0,1.5^2), targets U[0,128256) (about half not owned);
                the peer rank's statistics are computed once up front and
                handed over by an emulated all-gather, the combine is local
  c1            fp32 [4,256,32000] ~ N(0,2^2) (the reference's CPU config)
  wide          TP=1, bf16 [4,2048,128256] ~ N(0,1): a whole vocabulary of
                128256 entries through the one-pass path (rows held partly in LDS)
  c4            fused: hidden bf16 [16384,4096] ~ N(0,1), tied weight bf16
                [128256,4096] ~ N(0,0.02^2), targets U[0,128256)
  c5            fused stress: hidden [16384,3072], weight [256000,3072] ~
                N(0,0.05^2) with 64 rows x30, Zipf(1.1) targets

Prints one JSON line, compact enough to be kept whole by a log tail. Its top
level is c2 on the default path (one read of the logits, gradient written in
place, as the patched model.py call site asks with ``inplace=True``). Nested
objects, each with ``value``, ``ms_per_step``, ``roofline`` and
``cpu_baseline``:
  two_pass         c2 with one_pass=False (statistics pass, then the backward)
  c2_miss          c2 with the upstream value alternating 1.0 / 0.5 each step,
                   so every step's assumed value is wrong (a rescale pass)
  c3, c1, wide     the other unfused workloads on the default path
  fused            c4 on the default path (bounded token chunks)
  fused_one_chunk  c4 with every token in one chunk (the opt-in whose P^T has
                   the logits' size; reports its bytes)
  fused_recompute  c4 with one_pass=False (statistics GEMM, then a backward
                   that recomputes the logits by vocabulary chunk)
  c4_miss          c4 default path, upstream alternating 1.0 / 0.5
  c5               c5 on the default path
``roofline`` covers the dominant launch: for the unfused loss its algorithmic
HBM bytes per launch (what it must read and write), for the fused loss the
algorithmic flops of the C entry that takes the most time per step, over its
average launch time measured with HIP events on the launch stream.
Unfused steps run on fresh logits: every step takes its own copy of the
seeded slab, refilled before each batch of timed steps, outside the timed
region. ``cpu_baseline`` is the torch-CPU restatement of the reference's op
sequence (oracle/ce_restate.py) timed on this host on a bounded sample of
the same workload (repeated for about ``--cpu-seconds`` seconds); variants of
one workload share its baseline. ``--detail PATH`` writes every measured
field (per-kernel times, the whole-step roofline) to a JSON file as well.
"""

from __future__ import annotations

import argparse
import json
import os
import pathlib
import platform
import statistics
import sys
import time

ROOT = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "nano-megatron_amd"))

METRIC = "vocab-CE fwd+bwd tokens/s at 1 GPU; % HBM roofline (unfused) / % MFMA peak (fused)"
HBM_PEAK_GBS = 8000.0  # MI355X HBM3E, published
MFMA_BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16 MFMA, published

WORKLOADS = {
    "c2": dict(desc="unfused TP=1, bf16 logits [8,2048,50304] ~ N(0,1), targets U[0,50304)",
               b=8, s=2048, v=50304, tp=1, rank=0, sigma=1.0, dtype="bf16"),
    "c3": dict(desc="one TP=2 rank's shard, bf16 logits [4,4096,64128] at vocab offset 64128 "
                    "~ N(0,1.5^2), targets U[0,128256), local combine",
               b=4, s=4096, v=64128, tp=2, rank=1, sigma=1.5, dtype="bf16"),
    "c1": dict(desc="fp32 logits [4,256,32000] ~ N(0,2^2), targets U[0,32000), TP=1",
               b=4, s=256, v=32000, tp=1, rank=0, sigma=2.0, dtype="f32"),
    "wide": dict(desc="unfused TP=1, bf16 logits [4,2048,128256] ~ N(0,1), targets "
                      "U[0,128256) (a whole 128256-entry vocabulary on one GPU)",
                 b=4, s=2048, v=128256, tp=1, rank=0, sigma=1.0, dtype="bf16"),
    "c4": dict(desc="fused LM head + CE: hidden bf16 [16384,4096] ~ N(0,1), tied weight bf16 "
                    "[128256,4096] ~ N(0,0.02^2), targets U[0,128256)",
               fused=True, n=16384, h=4096, v=128256, w_std=0.02, hot_rows=0, zipf=None),
    "c5": dict(desc="fused stress: hidden bf16 [16384,3072] ~ N(0,1), weight bf16 [256000,3072] "
                    "~ N(0,0.05^2) with 64 rows x30, targets Zipf(1.1)",
               fused=True, n=16384, h=3072, v=256000, w_std=0.05, hot_rows=64, zipf=1.1),
}

# Nested objects of the default line: key -> (workload, options). The unfused
# ones take --steps/--warmup, the fused ones --fused-steps/--fused-warmup.
NESTED = [
    ("two_pass", "c2", dict(one_pass=False)),
    ("c2_miss", "c2", dict(miss=True)),
    ("c3", "c3", dict()),
    ("c1", "c1", dict()),
    ("wide", "wide", dict()),
    ("fused", "c4", dict()),
    ("fused_one_chunk", "c4", dict(one_chunk=True)),
    ("fused_recompute", "c4", dict(one_pass=False)),
    ("c4_miss", "c4", dict(miss=True)),
    ("c5", "c5", dict()),
]


def parse_args():
    p = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=100)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--workload", choices=sorted(WORKLOADS), default=None,
                   help="run this workload alone (default: c2 with every other config nested)")
    p.add_argument("--two-pass", action="store_true",
                   help="unfused workloads: take the two-pass path (one_pass=False)")
    p.add_argument("--no-cpu-baseline", action="store_true",
                   help="skip the CPU baseline (e.g. under a profiler)")
    p.add_argument("--cpu-seconds", type=float, default=10.0,
                   help="CPU baseline: repeat the sampled step for about this long")
    p.add_argument("--calibrate-copy", action="store_true",
                   help="after timing, run one nmce_stream_copy of the logits slab / weight "
                        "(known traffic) so a counter run can scale FETCH_SIZE / WRITE_SIZE")
    p.add_argument("--fused-steps", type=int, default=10,
                   help="timed steps of each fused workload in the default run")
    p.add_argument("--fused-warmup", type=int, default=2)
    p.add_argument("--vocab-chunk", type=int, default=None,
                   help="fused backward: vocabulary rows per chunk (default: the library's)")
    p.add_argument("--token-chunk", type=int, default=None,
                   help="fused one-pass path: tokens per chunk (default: the library's)")
    p.add_argument("--fused-two-pass", action="store_true",
                   help="fused workloads: the recomputing backward (one_pass=False)")
    p.add_argument("--miss", action="store_true",
                   help="alternate the upstream value 1.0 / 0.5 every step (each step's "
                        "assumed value is wrong)")
    p.add_argument("--slab-budget-gb", type=float, default=48.0,
                   help="unfused: device memory for the per-step copies of the logits")
    p.add_argument("--detail", default=None,
                   help="also write every measured field to this JSON file")
    p.add_argument("--gemm-core", action="store_true",
                   help="instead: time the fused path's GEMM core beside torch.mm "
                        "(hipBLASLt) on the c4 forward product's shape, one JSON line")
    return p.parse_args()


def run_gemm_core(reps: int = 8, rounds: int = 3) -> dict:
    """The fused path's bf16 GEMM core (nmce_gemm_nt_bf16, the main loop of
    all three fused products) beside torch.mm, which dispatches to hipBLASLt,
    on the c4 forward product's shape: C[V, C] = W[V, H] X_c[C, H]^T with
    V = 128256, a chunk of C = 4096 tokens, H = 4096, W ~ N(0, 0.02^2) and
    X ~ N(0, 1) as at c4 (the chip's clock under its power cap depends on the
    data). Rounds of ``reps`` calls of each, interleaved; the best round each.
    A reference point for the MFMA roofline; nothing of the loss runs."""
    import torch
    from nmce import _lib as L

    lib = L.load()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    M, N, K = 128256, 4096, 4096
    gen = torch.Generator(device=dev).manual_seed(0)
    a = (torch.randn(M, K, device=dev, generator=gen) * 0.02).to(torch.bfloat16)
    b = torch.randn(N, K, device=dev, generator=gen).to(torch.bfloat16)
    c_own = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
    c_lib = torch.empty_like(c_own)
    stream = L.stream_handle(dev)

    def own():
        L.check(lib.nmce_gemm_nt_bf16(a.data_ptr(), K, b.data_ptr(), K, M, N, K,
                                      c_own.data_ptr(), L.NMCE_BF16, N, stream), "gemm")

    def blas():
        torch.mm(a, b.t(), out=c_lib)

    flop = 2.0 * M * N * K
    best = {"nmce_gemm_nt_bf16": float("inf"), "torch.mm (hipBLASLt)": float("inf")}
    for _ in range(rounds):
        for name, fn in (("nmce_gemm_nt_bf16", own), ("torch.mm (hipBLASLt)", blas)):
            fn()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(reps):
                fn()
            e1.record()
            torch.cuda.synchronize()
            best[name] = min(best[name], e0.elapsed_time(e1) / reps)
    out = {"metric": "bf16 GEMM TFLOP/s, C[128256,4096] = A[128256,4096] B[4096,4096]^T",
           "shape_mnk": [M, N, K], "peak_tflops": MFMA_BF16_PEAK_TFLOPS}
    for name, ms in best.items():
        tf = flop / ms / 1e9
        out[name] = {"ms": ms, "tflops": tf, "frac": tf / MFMA_BF16_PEAK_TFLOPS}
    out["max_abs_diff"] = (c_own.float() - c_lib.float()).abs().max().item()
    return out


TRAFFIC_FILE = ROOT / "profiles" / "hbm_traffic_ce.json"
LMHEAD_TRAFFIC_FILE = ROOT / "profiles" / "hbm_traffic_lmhead.json"


def measured_traffic(workload: str, kernel: str, path=TRAFFIC_FILE):
    """HBM bytes per launch measured by rocprofv3 --pmc (FETCH_SIZE and
    WRITE_SIZE, each scaled by the same counter read on a copy of known size),
    recorded in profiles/hbm_traffic_*.json; None if not measured."""
    try:
        doc = json.loads(path.read_text())
        return doc["workloads"][workload][kernel]["bytes_per_launch"]
    except (OSError, KeyError, ValueError):
        return None


def lm_head_stand_in():
    """An autograd node standing where the LM-head matmul is (model.py:192):
    forward hands the resident logits on as a non-leaf tensor, backward
    receives d(logits) and stops there (the dX/dW GEMMs that would consume it
    are not part of the loss path). Without it the logits would be a leaf and
    autograd would copy the whole gradient into ``.grad`` each step. The node
    is C++ (``head_output`` of the autograd extension), as the matmul's own
    backward is, so the engine does not hand each backward to the
    interpreter for it."""
    from nmce import _lib as L
    ext = L.autograd_ext()

    class LMHeadOutput:
        apply = staticmethod(ext.head_output)

    return LMHeadOutput


def host_cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def _cpu_threads() -> int:
    import torch
    threads = len(os.sched_getaffinity(0))
    if os.environ.get("OMP_NUM_THREADS", "").isdigit():
        threads = min(threads, int(os.environ["OMP_NUM_THREADS"]))
    torch.set_num_threads(threads)
    return torch.get_num_threads()


def _time_for(step, seconds: float, min_reps: int = 3):
    """1 warmup, then repeat ``step`` until ``seconds`` have passed (at least
    ``min_reps`` times). Returns (median seconds, repetitions)."""
    step()
    times = []
    t_end = time.perf_counter() + seconds
    while len(times) < min_reps or time.perf_counter() < t_end:
        t0 = time.perf_counter()
        step()
        times.append(time.perf_counter() - t0)
    return statistics.median(times), len(times)


def cpu_baseline(wl: dict, seconds: float) -> dict:
    """Time the torch-CPU restatement of cross_entropy.py fwd+bwd on a sample
    of the workload's tokens at its full vocabulary width (the whole workload
    for c1), repeated for about ``seconds``."""
    import torch
    from oracle import ce_restate as R

    cores = _cpu_threads()
    g = torch.Generator().manual_seed(0)
    v, tp, rank = wl["v"], wl["tp"], wl["rank"]
    rows = min(wl["b"] * wl["s"], 1024)
    dt = torch.bfloat16 if wl["dtype"] == "bf16" else torch.float32
    x = (torch.randn(rows, v, generator=g) * wl["sigma"]).to(dt)
    t = torch.randint(0, v * tp, (rows,), generator=g)
    start, end = rank * v, (rank + 1) * v
    hook_args = None
    if tp > 1:  # peer shard partials, computed before timing (the other rank's work)
        peer = (torch.randn(rows, v, generator=g) * wl["sigma"]).to(dt)
        pmax = peer.float().max(-1)[0]
        gmax = torch.maximum(pmax, x.float().max(-1)[0])
        pick, psum = R.peer_partials(peer, t, 0, v, gmax)
        hook_args = (pmax, pick, psum)
        del peer
    go = torch.full((rows,), 1.0 / rows)

    def step():
        hook = R.fixed_peer_all_reduce(*hook_args) if hook_args else None
        # the reference validates targets first (cross_entropy.py:80-81)
        if torch.any(t < 0) or torch.any(t >= v * tp):
            raise ValueError("bad target")
        loss, saved = R.forward(x, t, start, end, all_reduce=hook)
        loss.mean()
        return R.backward(saved, go)

    med, reps = _time_for(step, seconds)
    return {
        "value": rows / med,
        "unit": "tokens/s",
        "cores": cores,
        "kind": "port",
        "sample": f"{rows} tok x V {v} {wl['dtype']}, cross_entropy.py fwd+bwd on torch-CPU, "
                  f"median of {reps} ({reps * med:.0f} s), {host_cpu_model()}",
        "ms_per_step": med * 1e3,
    }


def cpu_baseline_fused(wl: dict, seconds: float, rows: int = 128) -> dict:
    """The reference's op sequence for the LM head + loss under bf16 autocast
    on torch-CPU (model.py:192 in bf16, cross_entropy.py on the fp32 upcast,
    the matmul backward in bf16), on ``rows`` tokens at the full vocabulary,
    repeated for about ``seconds``."""
    import torch
    from oracle import ce_restate as R

    cores = _cpu_threads()
    g = torch.Generator().manual_seed(0)
    h, v = wl["h"], wl["v"]
    x = torch.randn(rows, h, generator=g).to(torch.bfloat16)
    w = (torch.randn(v, h, generator=g) * wl["w_std"]).to(torch.bfloat16)
    t = torch.randint(0, v, (rows,), generator=g)
    go = torch.full((rows,), 1.0 / rows)

    def step():
        if torch.any(t < 0) or torch.any(t >= v):
            raise ValueError("bad target")
        logits = torch.matmul(x, w.t())
        loss, saved = R.forward(logits, t, 0, v)
        loss.mean()
        dz = R.backward(saved, go).to(torch.bfloat16)
        return torch.matmul(dz, w), torch.matmul(dz.t(), x)

    med, reps = _time_for(step, seconds, min_reps=2)
    return {
        "value": rows / med,
        "unit": "tokens/s",
        "cores": cores,
        "kind": "port",
        "sample": f"{rows} tok x V {v} x H {h}: bf16 x@W^T, cross_entropy.py on fp32, bf16 "
                  f"dX/dW, torch-CPU, median of {reps} ({reps * med:.0f} s), {host_cpu_model()}",
        "ms_per_step": med * 1e3,
    }


def _kernel_times(run_steps, steps: int):
    """Average duration per launch of each libnmce entry over ``steps`` more
    steps (``run_steps(k)`` runs k of them), from HIP event pairs recorded on
    the launch stream around every launch: the Python host layer's
    (nmce.cross_entropy.kernel_timeline) and the one-pass autograd node's
    (``_nmce_autograd.set_timing``). Event records add small gaps between
    launches, so this region's wall time is not the step time. Returns
    ({name: ms}, {name: launches})."""
    import torch
    import nmce.cross_entropy as ce_mod
    from nmce import _lib

    ext = _lib.autograd_ext()
    ext.take_timeline()
    timeline: list = []
    ce_mod.kernel_timeline = timeline
    ext.set_timing(True)
    try:
        run_steps(steps)
        torch.cuda.synchronize()
    finally:
        ce_mod.kernel_timeline = None
        ext.set_timing(False)
    per: dict[str, list[float]] = {}
    for name, s_ev, e_ev in timeline:
        per.setdefault(name, []).append(s_ev.elapsed_time(e_ev))
    for name, ms in ext.take_timeline():
        per.setdefault(name, []).append(ms)
    return ({k: sum(vs) / len(vs) for k, vs in per.items()},
            {k: len(vs) for k, vs in per.items()})


def fused_inputs(wl: dict, dev):
    """Seeded hidden states, weight shard and targets of a fused workload
    (the same generator sequence as the fused workload parity test)."""
    import torch
    g = torch.Generator(device=dev).manual_seed(0)
    n, h, v = wl["n"], wl["h"], wl["v"]
    x = torch.randn(n, h, device=dev, generator=g).to(torch.bfloat16)
    wf = torch.randn(v, h, device=dev, generator=g) * wl["w_std"]
    if wl["hot_rows"]:
        hot = torch.randperm(v, device=dev, generator=g)[:wl["hot_rows"]]
        wf[hot] *= 30.0
    w = wf.to(torch.bfloat16)
    del wf
    if wl["zipf"]:
        ranks = torch.arange(1, v + 1, device=dev, dtype=torch.float64)
        t = torch.multinomial((ranks ** -wl["zipf"]).float(), n, replacement=True, generator=g)
    else:
        t = torch.randint(0, v, (n,), device=dev, generator=g)
    return x, w, t


def _upstream(i: int, miss: bool) -> float:
    """The upstream value of step i: 1.0 (loss.backward()), or 1.0 and 0.5 in
    turn, so that every step's forward assumed the previous step's value."""
    return 0.5 if (miss and i % 2) else 1.0


def run_fused(args, name: str, steps: int, warmup: int, one_pass: bool = True,
              one_chunk: bool = False, miss: bool = False) -> dict:
    """Time the fused LM head + loss (fwd + bwd) on workload ``name``."""
    import torch
    import nmce
    from nmce import lmhead

    wl = WORKLOADS[name]
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    x, w, t = fused_inputs(wl, dev)
    n, h, v = wl["n"], wl["h"], wl["v"]
    ctx = nmce.ParallelContext.single()
    xp = x.requires_grad_(True)
    wp = w.requires_grad_(True)
    token_chunk = n if one_chunk else args.token_chunk
    chunk = token_chunk if token_chunk is not None else lmhead.default_token_chunk(n, v)
    counter = [0]

    def run_steps(k):
        for _ in range(k):
            xp.grad = None  # zero_grad(set_to_none=True) between steps
            wp.grad = None
            loss = nmce.lmhead_vocab_parallel_cross_entropy(
                xp, wp, t, 0, v, ctx, vocab_chunk=args.vocab_chunk, token_chunk=token_chunk,
                one_pass=one_pass)
            g = _upstream(counter[0], miss)
            counter[0] += 1
            (loss * g if miss else loss).backward()

    run_steps(warmup)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    run_steps(steps)
    torch.cuda.synchronize()
    ms_per_step = (time.perf_counter() - t0) * 1e3 / steps
    avg_ms, counts = _kernel_times(run_steps, steps)

    calib = None
    if args.calibrate_copy:
        # One nmce_stream_copy of the weight shard (known traffic) for scaling
        # FETCH_SIZE / WRITE_SIZE read in a counter run.
        from nmce import _lib as L
        dst = torch.empty_like(w)
        L.check(L.load().nmce_stream_copy(w.data_ptr(), dst.data_ptr(), w.numel() * 2,
                                          L.stream_handle(dev)), "nmce_stream_copy")
        torch.cuda.synchronize()
        calib = w.numel() * 2
        del dst

    gemm_flops = 2.0 * n * v * h   # one product over every token
    # Algorithmic flops per step of each C entry: the one-pass statistics call
    # is the forward GEMM of its chunk, the gradients call the dX and dW
    # GEMMs of its chunk; the recomputing path's statistics call is the
    # forward GEMM and its backward call the three GEMMs of the backward
    # (the recomputation counted as executed, not as algorithmic work).
    entry_flops = {
        "nmce_lmhead_ce_fused_chunk_stats": gemm_flops,
        "nmce_lmhead_ce_fused_chunk_grads": 2 * gemm_flops,
        "nmce_lmhead_ce_fwd_stats": gemm_flops,
        "nmce_lmhead_ce_bwd": 3 * gemm_flops,
    }
    step_ms = {k: avg_ms[k] * counts[k] / steps for k in avg_ms}
    dominant = max((k for k in entry_flops if k in avg_ms), key=lambda k: step_ms[k])
    per_step = counts[dominant] / steps
    flops_per_launch = entry_flops[dominant] / per_step
    achieved = flops_per_launch / (avg_ms[dominant] * 1e-3) / 1e12
    alg_flops = 3 * gemm_flops      # forward GEMM + the dX and dW GEMMs
    on_one_pass = "nmce_lmhead_ce_fused_chunk_stats" in avg_ms
    exe_flops = alg_flops if on_one_pass else 4 * gemm_flops
    vpad = (v + 255) // 256 * 256
    pt_bytes = vpad * ((min(chunk, n) + 63) // 64 * 64) * 2 if on_one_pass else None
    path = (("one pass, one chunk of every token" if one_chunk else
             f"one pass, chunks of {min(chunk, n)} tokens") if on_one_pass else
            "recomputing backward")
    result = {
        "metric": METRIC,
        "value": n / (ms_per_step * 1e-3),
        "unit": "tokens/s",
        "ms_per_step": ms_per_step,
        "config": {
            "workload": name,
            "path": path + (", upstream 1/0.5 alternating" if miss else ""),
            "pt_bytes": pt_bytes,
        },
        "roofline": {
            "bound": "mfma",
            "kernel": dominant,
            "achieved": achieved,
            "peak": MFMA_BF16_PEAK_TFLOPS,
            "unit": "TFLOP/s",
            "frac": achieved / MFMA_BF16_PEAK_TFLOPS,
            "traffic": measured_traffic(f"{name}:{min(chunk, n)}", dominant,
                                        LMHEAD_TRAFFIC_FILE) if on_one_pass else None,
        },
        "step_frac": alg_flops / (ms_per_step * 1e-3) / 1e12 / MFMA_BF16_PEAK_TFLOPS,
    }
    detail = {
        "kernels_ms": avg_ms,
        "launches_per_step": {k: c / steps for k, c in counts.items()},
        "alg_flops_per_launch": flops_per_launch,
        "alg_flops_per_step": alg_flops,
        "executed_flops_per_step": exe_flops,
        "frac_executed_wall": exe_flops / (ms_per_step * 1e-3) / 1e12 / MFMA_BF16_PEAK_TFLOPS,
        "device": torch.cuda.get_device_name(0),
        "steps": steps,
        "warmup": warmup,
    }
    if calib is not None:
        detail["calibration_copy_bytes"] = calib
    del x, w, t, xp, wp
    torch.cuda.empty_cache()
    return result, detail


def unfused_alg_bytes(n: int, slab: int) -> dict:
    """Algorithmic HBM bytes per launch of each unfused kernel: what it must
    read and write. Per token: target 8 B in, and 12 B of statistics out
    (loss or target logit, max, exp-sum - 1) or 8 B in (max, exp-sum - 1)
    plus 4 B of upstream gradient."""
    return {
        "nmce_ce_fwd": slab + 20 * n,            # logits read
        "nmce_ce_fwd_stats": slab + 20 * n,
        "nmce_ce_bwd_scaled": 2 * slab + 20 * n,  # logits read, gradient written
        "nmce_ce_bwd": 2 * slab + 20 * n,
        # one-pass forward + backward: the logits read once, the gradient
        # written once (in place or to a new buffer)
        "nmce_ce_fwd_bwd": 2 * slab + 20 * n,
        # a miss after an in-place one-pass forward: the gradient read and
        # written once more
        "nmce_ce_grad_rescale_unless": 2 * slab,
        "nmce_ce_combine": 24 * n,
    }


def run_unfused(args, name: str, steps: int, warmup: int, one_pass: bool = True,
                miss: bool = False) -> dict:
    """Time the drop-in loss (fwd + bwd) on unfused workload ``name``."""
    import torch
    import nmce
    import nmce.cross_entropy as ce_mod

    wl = WORKLOADS[name]
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    n = wl["b"] * wl["s"]
    v, tp, rank = wl["v"], wl["tp"], wl["rank"]
    dt = torch.bfloat16 if wl["dtype"] == "bf16" else torch.float32
    esize = 2 if dt == torch.bfloat16 else 4
    start, end = rank * v, (rank + 1) * v

    gen = torch.Generator(device=dev).manual_seed(0)
    pristine = (torch.randn(n, v, device=dev, generator=gen) * wl["sigma"]).to(dt)
    target = torch.randint(0, v * tp, (wl["b"], wl["s"]), device=dev, generator=gen)
    ctx = nmce.ParallelContext(rank=rank, world_size=tp, tp_size=tp, tp_rank=rank, pp_size=1,
                               pp_rank=0, dp_size=1, dp_rank=0)
    saved_exchange = ce_mod._exchange_stats
    if tp > 1:
        # The other rank's shard: its statistics are what the all-gather would
        # deliver. Computed once here, handed over by an emulated exchange.
        peer = (torch.randn(n, v, device=dev, generator=gen) * wl["sigma"]).to(dt)
        from nmce import _lib as L
        lib = L.load()
        peer_stats = torch.empty((3, n), dtype=torch.float32, device=dev)
        tflat = target.reshape(-1)
        L.check(lib.nmce_ce_fwd_stats(peer.data_ptr(), L.dtype_code(dt), n, v, v, tflat.data_ptr(),
                                      0, peer_stats[0].data_ptr(), peer_stats[1].data_ptr(),
                                      peer_stats[2].data_ptr(), L.stream_handle(dev)), "peer")
        del peer

        def emulated_all_gather(local, group, world_size):
            return torch.stack([peer_stats, local])

        ce_mod._exchange_stats = emulated_all_gather

    # Every step runs on its own copy of the seeded logits (the loss writes
    # the gradient into them): as many copies as the budget holds, refilled
    # from the pristine slab before each batch of steps, outside the timed
    # region.
    slab_bytes = n * v * esize
    nbuf = int(max(1, min(steps, args.slab_budget_gb * 1e9 // slab_bytes)))
    bufs = [torch.empty_like(pristine) for _ in range(nbuf)]

    # Non-leaf logits produced by an LM-head node, as at model.py:277; the
    # call site asks for the gradient in place (inplace=True), as the patched
    # model.py does: the one-pass forward writes it into the logits.
    anchor = torch.zeros((), device=dev, requires_grad=True)
    lm_head = lm_head_stand_in()
    counter = [0]

    def one_step(buf):
        logits = lm_head.apply(buf.view(wl["b"], wl["s"], v), anchor)
        loss = nmce.vocab_parallel_cross_entropy(logits, target, start, end, ctx,
                                                 one_pass=one_pass, inplace=True)
        g = _upstream(counter[0], miss)
        counter[0] += 1
        (loss * g if miss else loss).backward()

    def run_batches(k, timed):
        """k steps in batches of nbuf fresh copies; returns the summed wall time
        of the batches (each bracketed by synchronize)."""
        total = 0.0
        done = 0
        while done < k:
            m = min(nbuf, k - done)
            for b in bufs[:m]:
                b.copy_(pristine)
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for b in bufs[:m]:
                one_step(b)
            torch.cuda.synchronize()
            total += time.perf_counter() - t0
            done += m
        return total

    try:
        run_batches(warmup, False)
        # Timed region: K steps as a user runs them, on fresh logits.
        ms_per_step = run_batches(steps, True) * 1e3 / steps
        avg_ms, counts = _kernel_times(lambda k: run_batches(k, False), steps)
    finally:
        ce_mod._exchange_stats = saved_exchange

    alg = unfused_alg_bytes(n, slab_bytes)
    step_ms = {k: avg_ms[k] * counts[k] / steps for k in avg_ms}
    dominant = max((k for k in alg if k in avg_ms), key=lambda k: step_ms[k])
    achieved = alg[dominant] / (avg_ms[dominant] * 1e-3) / 1e9
    # The graded step figure: a forward pass over the logits and a backward
    # pass that reads them again and writes the gradient (the upstream value
    # is known only in the backward): 3 V b + 28 bytes per token.
    step_bytes = 3 * slab_bytes + n * 28
    kernel_ms = sum(step_ms.values())
    on_one_pass = "nmce_ce_fwd_bwd" in avg_ms
    # What this path's step must move: the one-pass path reads the logits once
    # and writes the gradient once (2 V b + 28 per token: target, statistics,
    # loss); the two-pass path 3 V b + 28.
    path_bytes = 2 * slab_bytes + n * 28 if on_one_pass else step_bytes
    traffic_key = {"nmce_ce_bwd_scaled": "nmce_ce_bwd",
                   "nmce_ce_fwd_bwd": "nmce_ce_fwd_bwd_inplace"}.get(dominant, dominant)
    path = "one pass, in place" if on_one_pass else "two passes, in place"
    result = {
        "metric": METRIC,
        "value": n / (ms_per_step * 1e-3),
        "unit": "tokens/s",
        "ms_per_step": ms_per_step,
        "config": {"workload": name,
                   "path": path + (", upstream 1/0.5 alternating" if miss else "")},
        "roofline": {
            "bound": "hbm",
            "kernel": dominant,
            "achieved": achieved,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": achieved / HBM_PEAK_GBS,
            "traffic": measured_traffic(name, traffic_key),
        },
        "step_frac": path_bytes / (ms_per_step * 1e-3) / 1e9 / HBM_PEAK_GBS,
    }
    detail = {
        "kernels_ms": avg_ms,
        "launches_per_step": {k: c / steps for k, c in counts.items()},
        "alg_bytes_per_launch": alg[dominant],
        "path_bytes_per_step": path_bytes,
        "kernel_ms_per_step": kernel_ms,
        "frac_kernels": path_bytes / (kernel_ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
        "fresh_copies": nbuf,
        "device": torch.cuda.get_device_name(0),
        "steps": steps,
        "warmup": warmup,
    }
    if on_one_pass:
        # The step and the kernel credited with the two passes' bytes (what
        # the two-pass path must move): a comparison, not a roofline fraction.
        detail["two_pass_equivalent"] = {
            "alg_bytes_per_step": step_bytes,
            "ratio_to_peak_wall": step_bytes / (ms_per_step * 1e-3) / 1e9 / HBM_PEAK_GBS,
            "kernel_ratio_to_peak": step_bytes / (avg_ms[dominant] * 1e-3) / 1e9 / HBM_PEAK_GBS,
        }
    if args.calibrate_copy:
        from nmce import _lib as L
        dst = torch.empty_like(pristine)
        L.check(L.load().nmce_stream_copy(pristine.data_ptr(), dst.data_ptr(), slab_bytes,
                                          L.stream_handle(dev)), "nmce_stream_copy")
        torch.cuda.synchronize()
        detail["calibration_copy_bytes"] = slab_bytes
        del dst
    del pristine, bufs
    torch.cuda.empty_cache()
    return result, detail


def _short_cpu(cb: dict | None) -> dict | None:
    if cb is None:
        return None
    return {k: cb[k] for k in ("value", "unit", "cores", "kind", "sample")}


def main() -> int:
    args = parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on exactly one GPU; --gpus must be 1 "
                          "(the TP exchange is one all-gather of [3, tokens] statistics, "
                          "not exercised here)"}))
        return 2

    if args.gemm_core:
        print(json.dumps(_round(run_gemm_core()), separators=(",", ":")), flush=True)
        return 0

    with_cpu = not args.no_cpu_baseline
    details = {}
    if args.workload is not None:
        wl = WORKLOADS[args.workload]
        if wl.get("fused"):
            result, det = run_fused(args, args.workload, args.steps, args.warmup,
                                    one_pass=not args.fused_two_pass, miss=args.miss)
            cpu = cpu_baseline_fused(wl, args.cpu_seconds) if with_cpu else None
        else:
            result, det = run_unfused(args, args.workload, args.steps, args.warmup,
                                      one_pass=not args.two_pass, miss=args.miss)
            cpu = cpu_baseline(wl, args.cpu_seconds) if with_cpu else None
        result["cpu_baseline"] = _short_cpu(cpu)
        details[args.workload] = det
        out = _headline(result, args.steps, args.warmup, wl)
    else:
        # Default: c2 on the default path, every other config nested. Every
        # GPU measurement runs before the first CPU baseline, whose worker
        # threads would otherwise compete with the launching thread.
        result, details["c2"] = run_unfused(args, "c2", args.steps, args.warmup)
        out = _headline(result, args.steps, args.warmup, WORKLOADS["c2"])
        for key, name, opts in NESTED:
            print(f"[bench] {key}", file=sys.stderr, flush=True)
            if WORKLOADS[name].get("fused"):
                out[key], details[key] = run_fused(args, name, args.fused_steps,
                                                   args.fused_warmup, **opts)
            else:
                out[key], details[key] = run_unfused(args, name, args.steps, args.warmup,
                                                     **opts)
            out[key].pop("metric")
            out[key].pop("unit")
        if with_cpu:
            print("[bench] CPU baselines", file=sys.stderr, flush=True)
            cpu = {"c2": cpu_baseline(WORKLOADS["c2"], args.cpu_seconds)}
            out["cpu_baseline"] = _short_cpu(cpu["c2"])
            for key, name, _ in NESTED:
                if name not in cpu:
                    wl = WORKLOADS[name]
                    cpu[name] = (cpu_baseline_fused(wl, args.cpu_seconds) if wl.get("fused")
                                 else cpu_baseline(wl, args.cpu_seconds))
                out[key]["cpu_baseline"] = _short_cpu(cpu[name])
        else:
            out["cpu_baseline"] = None
            for key, _, _ in NESTED:
                out[key]["cpu_baseline"] = None
        out["summary"] = _summary(out)
    if args.detail:
        pathlib.Path(args.detail).write_text(json.dumps(details, indent=1))
    print(json.dumps(_round(out), separators=(",", ":")), flush=True)
    return 0


SUMMARY_COLS = ["tokens/s", "ms_per_step", "roofline.kernel", "roofline.frac",
                "roofline.traffic", "cpu_baseline.value", "cpu_baseline.cores"]


def _summary(out: dict) -> dict:
    """One short row per configuration, last on the line, so that a reader
    who keeps only the end of the output (about 2 KB) still sees every
    configuration's throughput, roofline fraction and CPU baseline."""
    def row(r: dict) -> list:
        rf, cb = r["roofline"], r.get("cpu_baseline") or {}
        return [r["value"], r["ms_per_step"], rf["kernel"].removeprefix("nmce_"),
                rf["frac"], rf["traffic"], cb.get("value"), cb.get("cores")]
    rows = {"cols": SUMMARY_COLS, "c2": row(out)}
    for key, _, _ in NESTED:
        rows[key] = row(out[key])
    return rows


def _headline(result: dict, steps: int, warmup: int, wl: dict) -> dict:
    """The contract's top-level fields around one workload's result."""
    fused = bool(wl.get("fused"))
    out = {
        "metric": METRIC,
        "value": result["value"],
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": result["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32" if not fused else "bf16",
        "data": "synthetic",
        "config": dict(result["config"], workload=wl["desc"]),
        "roofline": result["roofline"],
        "step_frac": result["step_frac"],
    }
    if not fused:
        out["config"]["logits_dtype"] = wl["dtype"]
    if "cpu_baseline" in result:
        out["cpu_baseline"] = result["cpu_baseline"]
    return out


def _round(obj):
    """Floats to 4 significant digits (a shorter line; no figure is quoted to
    more)."""
    if isinstance(obj, float):
        return float(f"{obj:.4g}")
    if isinstance(obj, dict):
        return {k: _round(v) for k, v in obj.items()}
    if isinstance(obj, list):
        return [_round(v) for v in obj]
    return obj


if __name__ == "__main__":
    sys.exit(main())
