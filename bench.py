#!/usr/bin/env python3
"""Benchmark of the vocabulary-parallel cross entropy on one MI355X.

    python bench.py [--steps K] [--warmup W] [--workload c1..c5 [--two-pass]] [--gpus 1]

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

Prints one JSON line. ``roofline`` covers the dominant kernel: for the
unfused loss its algorithmic HBM bytes per launch (what the kernel must read
and write: tokens x vocab x bytes for each pass over the logits, plus
per-token statistics), for the fused loss the algorithmic flops of the
statistics GEMM (2 x tokens x vocab x hidden), over its average launch time
measured with HIP events on the launch stream during the timed steps.
Without ``--workload`` the line is c2 (the default path: one read of the
logits, gradient in place) with nested objects ``two_pass`` (c2 on the
two-pass path), ``c3``, ``c1``, ``wide`` (c2's path at a 128256-entry
vocabulary), ``fused`` (c4) and ``c5``, each with its own
``roofline``, ``kernels_ms`` and ``cpu_baseline``. ``cpu_baseline`` is the
torch-CPU restatement of the reference's op sequence (oracle/ce_restate.py)
timed on this host on a bounded sample of the same workload (repeated for
about ``--cpu-seconds`` seconds).
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

# Nested objects of the default line: (key, workload, one_pass). The unfused
# ones take --steps/--warmup, the fused ones --fused-steps/--fused-warmup.
NESTED = [("two_pass", "c2", False), ("c3", "c3", True), ("c1", "c1", True),
          ("wide", "wide", True), ("fused", "c4", True), ("c5", "c5", True)]


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
    return p.parse_args()


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
    autograd would copy the whole gradient into ``.grad`` each step."""
    import torch

    class LMHeadOutput(torch.autograd.Function):
        @staticmethod
        def forward(ctx, logits, anchor):
            return logits.view_as(logits)

        @staticmethod
        def backward(ctx, dlogits):
            return None, None

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
        "sample": f"{rows} tokens x full vocab {v} ({wl['dtype']} logits), torch-CPU restatement "
                  f"of cross_entropy.py fwd+bwd, median of {reps} after 1 warmup "
                  f"({reps * med:.1f} s); host {host_cpu_model()}, torch {torch.__version__}",
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
        "sample": f"{rows} tokens x full vocab {v}, hidden {h}: bf16 x @ W^T, torch-CPU "
                  f"restatement of cross_entropy.py fwd+bwd on the fp32 upcast, bf16 dX/dW "
                  f"matmuls; median of {reps} after 1 warmup ({reps * med:.1f} s); host "
                  f"{host_cpu_model()}, torch {torch.__version__}",
        "ms_per_step": med * 1e3,
    }


def _kernel_times(step, steps: int, with_counts: bool = False):
    """Average duration per launch of each libnmce kernel over ``steps`` more
    steps, from HIP event pairs recorded on the launch stream around every
    launch (nmce.cross_entropy.kernel_timeline). Event records add small gaps
    between launches, so this region's wall time is not the step time."""
    import torch
    import nmce.cross_entropy as ce_mod

    timeline: list = []
    ce_mod.kernel_timeline = timeline
    try:
        for _ in range(steps):
            step()
        torch.cuda.synchronize()
    finally:
        ce_mod.kernel_timeline = None
    per: dict[str, list[float]] = {}
    for name, s_ev, e_ev in timeline:
        per.setdefault(name, []).append(s_ev.elapsed_time(e_ev))
    avg = {k: sum(vs) / len(vs) for k, vs in per.items()}
    if with_counts:
        return avg, {k: len(vs) for k, vs in per.items()}
    return avg


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


def run_fused(args, name: str, steps: int, warmup: int, with_cpu: bool) -> dict:
    """Time the fused LM head + loss (fwd + bwd) on workload ``name``."""
    import torch
    import nmce

    wl = WORKLOADS[name]
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    x, w, t = fused_inputs(wl, dev)
    n, h, v = wl["n"], wl["h"], wl["v"]
    ctx = nmce.ParallelContext.single()
    xp = x.requires_grad_(True)
    wp = w.requires_grad_(True)

    def step():
        xp.grad = None  # zero_grad(set_to_none=True) between steps
        wp.grad = None
        loss = nmce.lmhead_vocab_parallel_cross_entropy(xp, wp, t, 0, v, ctx,
                                                        vocab_chunk=args.vocab_chunk,
                                                        token_chunk=args.token_chunk,
                                                        one_pass=not args.fused_two_pass)
        loss.backward()
        return loss

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    ms_per_step = (time.perf_counter() - t0) * 1e3 / steps
    avg_ms, counts = _kernel_times(step, steps, with_counts=True)

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
    one_pass = "nmce_lmhead_ce_fused_chunk_stats" in avg_ms
    # The statistics GEMM: on the one-pass path one launch per token chunk
    # (the GEMM that keeps the exponentials, plus the small reduction of its
    # partials), else one launch over every token.
    dominant = "nmce_lmhead_ce_fused_chunk_stats" if one_pass else "nmce_lmhead_ce_fwd_stats"
    per_step = counts[dominant] / steps
    flops_per_launch = gemm_flops / per_step
    achieved = flops_per_launch / (avg_ms[dominant] * 1e-3) / 1e12
    alg_flops = 3 * gemm_flops      # forward GEMM + the dX and dW GEMMs
    # the recomputing backward also recomputes the logits
    exe_flops = alg_flops if one_pass else 4 * gemm_flops
    result = {
        "metric": METRIC,
        "value": n / (ms_per_step * 1e-3),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": f"{name}: {wl['desc']}",
            "tokens": n,
            "hidden": h,
            "vocab_local": v,
            "tp": 1,
            "path": ("nmce.lmhead_vocab_parallel_cross_entropy fwd+bwd, one pass: per chunk "
                     "of tokens the statistics GEMM keeps its exponentials, dZ follows from "
                     "them, dX and dW by libnmce's GEMM (logits computed once, never stored "
                     "whole; bf16 MFMA, fp32 accumulate), target validation"
                     if one_pass else
                     "nmce.lmhead_vocab_parallel_cross_entropy fwd+bwd (logits never stored; "
                     "recomputed by vocabulary chunk in the backward; bf16 MFMA, fp32 "
                     "accumulate), target validation, dX and dW"),
        },
        "roofline": {
            "bound": "mfma",
            "kernel": dominant,
            "achieved": achieved,
            "peak": MFMA_BF16_PEAK_TFLOPS,
            "unit": "TFLOP/s",
            "frac": achieved / MFMA_BF16_PEAK_TFLOPS,
            "traffic": (measured_traffic(name, "lmhead_p_kernel", LMHEAD_TRAFFIC_FILE)
                        if one_pass else None),
            "alg_flops_per_launch": flops_per_launch,
            "avg_launch_ms": avg_ms[dominant],
            "launches_per_step": per_step,
        },
        "kernels_ms": avg_ms,
        "path_roofline": {
            "alg_flops_per_step": alg_flops,
            "executed_flops_per_step": exe_flops,
            "frac_alg_wall": alg_flops / (ms_per_step * 1e-3) / 1e12 / MFMA_BF16_PEAK_TFLOPS,
            "frac_executed_wall": exe_flops / (ms_per_step * 1e-3) / 1e12 / MFMA_BF16_PEAK_TFLOPS,
        },
        "device": torch.cuda.get_device_name(0),
    }
    if calib is not None:
        result["calibration_copy_bytes"] = calib
    del x, w, t, xp, wp
    torch.cuda.empty_cache()
    result["cpu_baseline"] = cpu_baseline_fused(wl, args.cpu_seconds) if with_cpu else None
    return result


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
        "nmce_ce_combine": 24 * n,
    }


def run_unfused(args, name: str, one_pass: bool, steps: int, warmup: int,
                with_cpu: bool) -> dict:
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
    base = (torch.randn(n, v, device=dev, generator=gen) * wl["sigma"]).to(dt)
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

    # Non-leaf logits produced by an LM-head node, as at model.py:277: the
    # gradient goes in place into the logits storage (by the one-pass forward
    # at TP = 1, by the backward otherwise).
    anchor = torch.zeros((), device=dev, requires_grad=True)
    lm_head = lm_head_stand_in()
    slab = base.view(wl["b"], wl["s"], v)

    def step():
        logits = lm_head.apply(slab, anchor)
        loss = nmce.vocab_parallel_cross_entropy(logits, target, start, end, ctx,
                                                 one_pass=one_pass)
        loss.backward()
        return loss

    try:
        for _ in range(warmup):
            step()
        torch.cuda.synchronize()

        # Timed region: K steps as a user runs them, nothing added.
        t0 = time.perf_counter()
        for _ in range(steps):
            step()
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        ms_per_step = (t1 - t0) * 1e3 / steps
        avg_ms = _kernel_times(step, steps)
    finally:
        ce_mod._exchange_stats = saved_exchange

    slab_bytes = n * v * esize
    alg = unfused_alg_bytes(n, slab_bytes)
    dominant = max((k for k in alg if k in avg_ms), key=lambda k: avg_ms[k])
    achieved = alg[dominant] / (avg_ms[dominant] * 1e-3) / 1e9
    # The graded step figure: a forward pass over the logits and a backward
    # pass that reads them again and writes the gradient (the upstream value
    # is known only in the backward): 3 V b + 28 bytes per token.
    step_bytes = 3 * slab_bytes + n * 28
    kernel_ms = sum(avg_ms.values())
    on_one_pass = "nmce_ce_fwd_bwd" in avg_ms
    # What this path's step must move: the one-pass path reads the logits once
    # and writes the gradient once (2 V b + 28 per token: target, statistics,
    # loss); the two-pass path 3 V b + 28.
    path_bytes = 2 * slab_bytes + n * 28 if on_one_pass else step_bytes
    traffic_key = {"nmce_ce_bwd_scaled": "nmce_ce_bwd"}.get(dominant, dominant)
    if dominant == "nmce_ce_fwd_bwd":
        traffic_key = "nmce_ce_fwd_bwd_inplace"
    result = {
        "metric": METRIC,
        "value": n / (ms_per_step * 1e-3),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": f"{name}: {wl['desc']}",
            "tokens": n,
            "vocab_local": v,
            "tp": tp,
            "tp_rank": rank,
            "logits_dtype": wl["dtype"],
            "path": ("nmce.vocab_parallel_cross_entropy fwd+bwd, target validation; the "
                     "one-pass kernel (logits read once, gradient written in place by the "
                     "forward)" if on_one_pass else
                     "nmce.vocab_parallel_cross_entropy fwd+bwd, two passes (statistics, then "
                     "the in-place gradient), target validation"),
        },
        "roofline": {
            "bound": "hbm",
            "kernel": dominant,
            "achieved": achieved,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": achieved / HBM_PEAK_GBS,
            "traffic": measured_traffic(name, traffic_key),
            "alg_bytes_per_launch": alg[dominant],
            "avg_launch_ms": avg_ms[dominant],
        },
        "kernels_ms": avg_ms,
        "path_roofline": {
            "alg_bytes_per_step": path_bytes,
            "kernel_ms_per_step": kernel_ms,
            "frac_kernels": path_bytes / (kernel_ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
            "frac_wall": path_bytes / (ms_per_step * 1e-3) / 1e9 / HBM_PEAK_GBS,
        },
        "device": torch.cuda.get_device_name(0),
    }
    if on_one_pass:
        # The whole step credited with the two passes' bytes: a comparison
        # with the two-pass design, not a roofline fraction.
        result["path_roofline"]["two_pass_equivalent"] = {
            "alg_bytes_per_step": step_bytes,
            "ratio_to_peak_wall": step_bytes / (ms_per_step * 1e-3) / 1e9 / HBM_PEAK_GBS,
        }
        # The same kernel credited with the two passes' bytes (3 V b + 28 per
        # token, what the two-pass path must move): how it compares with the
        # graded figure, not a roofline fraction.
        two = step_bytes
        result["roofline"]["two_pass_equivalent"] = {
            "alg_bytes_per_launch": two,
            "achieved": two / (avg_ms[dominant] * 1e-3) / 1e9,
            "ratio_to_peak": two / (avg_ms[dominant] * 1e-3) / 1e9 / HBM_PEAK_GBS,
        }
    if args.calibrate_copy:
        from nmce import _lib as L
        dst = torch.empty_like(base)
        L.check(L.load().nmce_stream_copy(base.data_ptr(), dst.data_ptr(), slab_bytes,
                                          L.stream_handle(dev)), "nmce_stream_copy")
        torch.cuda.synchronize()
        result["calibration_copy_bytes"] = slab_bytes
        del dst
    del base, slab
    torch.cuda.empty_cache()
    result["cpu_baseline"] = cpu_baseline(wl, args.cpu_seconds) if with_cpu else None
    return result


def main() -> int:
    args = parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on exactly one GPU; --gpus must be 1 "
                          "(the TP exchange is one all-gather of [3, tokens] statistics, "
                          "not exercised here)"}))
        return 2

    with_cpu = not args.no_cpu_baseline
    if args.workload is not None:
        wl = WORKLOADS[args.workload]
        if wl.get("fused"):
            result = run_fused(args, args.workload, args.steps, args.warmup, with_cpu)
        else:
            result = run_unfused(args, args.workload, not args.two_pass, args.steps,
                                 args.warmup, with_cpu)
        print(json.dumps(result), flush=True)
        return 0

    # Default: c2 on the default path, every other config nested. Every GPU
    # measurement runs before the first CPU baseline, whose worker threads
    # would otherwise compete with the launching thread.
    result = run_unfused(args, "c2", True, args.steps, args.warmup, False)
    for key, name, one_pass in NESTED:
        print(f"[bench] {key}: {name}", file=sys.stderr, flush=True)
        if WORKLOADS[name].get("fused"):
            result[key] = run_fused(args, name, args.fused_steps, args.fused_warmup, False)
        else:
            result[key] = run_unfused(args, name, one_pass, args.steps, args.warmup, False)
    if with_cpu:
        print("[bench] CPU baselines", file=sys.stderr, flush=True)
        result["cpu_baseline"] = cpu_baseline(WORKLOADS["c2"], args.cpu_seconds)
        for key, name, _ in NESTED:
            wl = WORKLOADS[name]
            result[key]["cpu_baseline"] = (cpu_baseline_fused(wl, args.cpu_seconds)
                                           if wl.get("fused") else
                                           cpu_baseline(wl, args.cpu_seconds))
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
