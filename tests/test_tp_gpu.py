"""Tensor parallelism end to end on one GPU: two or four ranks (the reference's
own TP checks use tp 2 and 4, check_tp_math.py:94-134) share cuda:0 and talk
over gloo (host copies), so every TP > 1 code path of the drop-ins runs on the
HIP kernels.

* unfused (cross_entropy.py:16-85 at world_size tp): each rank holds a
  ``[B, S, V/tp]`` shard of bf16 logits; the packed statistics are all-gathered
  once and combined on each rank;
* fused, TP without sequence parallelism (model.py:188-192 with ``f`` of
  mappings.py:83-94): every rank sees the full hidden state and its own
  vocabulary shard of the weight; the input gradient is all-reduced;
* fused, sequence parallel (mappings.py:109-120): every rank holds
  ``[B, S/tp, H]``; the tokens are gathered rank-major, the labels permuted to
  match, and the input gradient reduce-scattered back to the shards.

Every rank must return the same loss, equal to the fp64 closed form over the
full vocabulary (oracle ``closed_form`` / ``lmhead_closed_form``) within 1e-5
relative. The unfused logit gradient of each shard is the matching column
slice of the full-vocabulary gradient, within one bf16 rounding. The fused
gradients are held to a norm-relative error of 6e-3 against the exact fp64
products (each rank's bf16 partial input gradient is rounded once more by the
bf16 all-reduce / reduce-scatter).
"""

from __future__ import annotations

import os
import socket
import types

import numpy as np
import pytest
import torch
import torch.distributed as dist
import torch.multiprocessing as mp

from oracle import ce_oracle

pytestmark = pytest.mark.gpu

B, S, H, V = 2, 96, 128, 4 * 320


def _free_port() -> int:
    with socket.socket() as s:
        s.bind(("127.0.0.1", 0))
        return s.getsockname()[1]


def _inputs():
    g = torch.Generator().manual_seed(77)
    logits = (torch.randn(B, S, V, generator=g) * 2.0).to(torch.bfloat16)
    hidden = torch.randn(B, S, H, generator=g).to(torch.bfloat16)
    weight = (torch.randn(V, H, generator=g) * 0.3).to(torch.bfloat16)
    labels = torch.randint(0, V, (B, S), generator=g)
    return logits, hidden, weight, labels


def _worker(rank: int, world: int, port: int, out_dir: str) -> None:
    os.environ["MASTER_ADDR"] = "127.0.0.1"
    os.environ["MASTER_PORT"] = str(port)
    dist.init_process_group("gloo", rank=rank, world_size=world)
    try:
        torch.cuda.set_device(0)
        import nmce
        dev = torch.device("cuda:0")
        ctx = nmce.ParallelContext(rank=rank, world_size=world, tp_size=world, tp_rank=rank,
                                   pp_size=1, pp_rank=0, dp_size=1, dp_rank=0)
        logits, hidden, weight, labels = _inputs()
        per = V // world
        lo, hi = rank * per, (rank + 1) * per
        t = labels.to(dev)
        res = {}
        print(f"[rank {rank}] unfused", flush=True)
        x = logits[..., lo:hi].contiguous().to(dev).requires_grad_(True)
        loss = nmce.vocab_parallel_cross_entropy(x, t, lo, hi, ctx)
        loss.backward()
        res["u_loss"] = loss.item()
        res["u_grad"] = x.grad.float().cpu().numpy()

        cfg = types.SimpleNamespace(vocab_size=V, n_embd=H, sequence_parallel=False)
        for sp in (False, True):
            tag = "sp" if sp else "tp"
            print(f"[rank {rank}] fused {tag}", flush=True)
            head = nmce.FusedParallelLMHead(cfg, ctx)
            head.weight = torch.nn.Parameter(weight[lo:hi].to(dev))
            head.sequence_parallel = sp
            if sp:
                s2 = S // world
                xh = hidden[:, rank * s2:(rank + 1) * s2].contiguous().to(dev)
            else:
                xh = hidden.to(dev)
            xh.requires_grad_(True)
            loss = head(xh, t)
            loss.backward()
            res[f"{tag}_loss"] = loss.item()
            res[f"{tag}_dx"] = xh.grad.float().cpu().numpy()
            res[f"{tag}_dw"] = head.weight.grad.float().cpu().numpy()
        torch.cuda.synchronize()
        np.savez(os.path.join(out_dir, f"rank{rank}.npz"), **res)
        print(f"[rank {rank}] done", flush=True)
    finally:
        dist.destroy_process_group()


@pytest.fixture(scope="module", params=[2, 4], ids=["tp2", "tp4"])
def ranks(request, tmp_path_factory):
    assert torch.cuda.is_available(), "GPU tests need a ROCm device"
    world = request.param
    out = tmp_path_factory.mktemp(f"tp_gpu{world}")
    print(f"[tp_gpu] spawning {world} ranks on cuda:0", flush=True)
    mp.start_processes(_worker, args=(world, _free_port(), str(out)), nprocs=world, join=True,
                       start_method="spawn")
    return [dict(np.load(out / f"rank{r}.npz")) for r in range(world)]


def _nrel(got, want):
    return np.linalg.norm(got - want) / np.linalg.norm(want)


def test_unfused_tp_ranks(ranks):
    logits, _, _, labels = _inputs()
    n = B * S
    x = logits.reshape(n, V).double().numpy()
    loss, grad = ce_oracle.closed_form(x, labels.reshape(-1).numpy(), 1.0 / n)
    world = len(ranks)
    per = V // world
    for r in range(world):
        assert abs(ranks[r]["u_loss"] - loss.mean()) <= 1e-5 * loss.mean()
        got = ranks[r]["u_grad"].reshape(n, per).astype(np.float64)
        want = grad[:, r * per:(r + 1) * per]
        # one bf16 rounding of the fp32 gradient, plus a floor for tiny entries
        assert np.all(np.abs(got - want) <= 2.0 ** -8 * np.abs(want) + 1e-9)


@pytest.mark.parametrize("tag", ["tp", "sp"])
def test_fused_tp_ranks(ranks, tag):
    _, hidden, weight, labels = _inputs()
    n = B * S
    X = hidden.reshape(n, H).double().numpy()
    W = weight.double().numpy()
    loss, _, dx, dw = ce_oracle.lmhead_closed_form(X, W, labels.reshape(-1).numpy(),
                                                   np.full(n, 1.0 / n))
    dx = dx.reshape(B, S, H)
    world = len(ranks)
    per = V // world
    s2 = S // world
    for r in range(world):
        assert abs(ranks[r][f"{tag}_loss"] - loss.mean()) <= 1e-5 * loss.mean()
        want_dx = dx if tag == "tp" else dx[:, r * s2:(r + 1) * s2]
        assert _nrel(ranks[r][f"{tag}_dx"], want_dx) <= 6e-3
        assert _nrel(ranks[r][f"{tag}_dw"], dw[r * per:(r + 1) * per]) <= 6e-3
