"""The LM head's input-side collectives on the CPU (gloo, two ranks on 127.0.0.1).

``f`` (mappings.py:83-94) is the identity forward and all-reduces the gradient;
the sequence gather (mappings.py:109-120) concatenates the ranks' ``[B, S/tp,
H]`` shards along the sequence and SUM-reduce-scatters the gradient. The
rank-major gather must hold the same tokens as the natural-order one, in the
order ``targets_rank_major`` gives the labels, and its backward must hand each
rank the sum over ranks of the gradient of its own tokens. Every expected value
here is built from the definitions on one process, in float64.
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

WORLD = 2
B, S, H = 2, 6, 3


def _free_port() -> int:
    with socket.socket() as s:
        s.bind(("127.0.0.1", 0))
        return s.getsockname()[1]


def _full_input():
    return torch.arange(B * S * H, dtype=torch.float64).view(B, S, H) / 7.0


def _weights(rank):
    """Per-rank upstream gradient pattern: the loss is sum(out * C_rank)."""
    g = torch.Generator().manual_seed(100 + rank)
    return torch.randn(B * S * H, generator=g, dtype=torch.float64)


def _worker(rank: int, port: int, out_dir: str) -> None:
    os.environ["MASTER_ADDR"] = "127.0.0.1"
    os.environ["MASTER_PORT"] = str(port)
    dist.init_process_group("gloo", rank=rank, world_size=WORLD)
    try:
        import nmce
        ctx = types.SimpleNamespace(tp_size=WORLD, tp_rank=rank, tp_group=None)
        full = _full_input()
        sl = S // WORLD
        res = {}

        # f: identity forward, all-reduced gradient
        x = full.clone().requires_grad_(True)
        y = nmce.copy_to_tensor_parallel_region(x, ctx)
        (y * _weights(rank).view(B, S, H)).sum().backward()
        res["f_out"] = y.detach().numpy()
        res["f_grad"] = x.grad.numpy()

        # natural-order sequence gather
        xs = full[:, rank * sl:(rank + 1) * sl].clone().requires_grad_(True)
        y = nmce.gather_from_sequence_parallel_region(xs, ctx)
        (y * _weights(rank).view(B, S, H)).sum().backward()
        res["sp_out"] = y.detach().numpy()
        res["sp_grad"] = xs.grad.numpy()

        # rank-major gather and the matching label order
        xs = full[:, rank * sl:(rank + 1) * sl].clone().requires_grad_(True)
        rows = nmce.gather_tokens_rank_major(xs, ctx)
        (rows * _weights(rank).view(B * S, H)).sum().backward()
        res["rm_out"] = rows.detach().numpy()
        res["rm_grad"] = xs.grad.numpy()
        tok = torch.arange(B * S).view(B, S)
        res["rm_tok"] = nmce.targets_rank_major(tok, WORLD).numpy()
        np.savez(os.path.join(out_dir, f"rank{rank}.npz"), **res)
    finally:
        dist.destroy_process_group()


@pytest.fixture(scope="module")
def ranks(tmp_path_factory):
    out = tmp_path_factory.mktemp("mappings")
    mp.start_processes(_worker, args=(_free_port(), str(out)), nprocs=WORLD, join=True,
                       start_method="spawn")
    return [dict(np.load(out / f"rank{r}.npz")) for r in range(WORLD)]


def test_copy_to_tensor_parallel_region(ranks):
    full = _full_input().numpy()
    csum = sum(_weights(r).view(B, S, H).numpy() for r in range(WORLD))
    for r in range(WORLD):
        np.testing.assert_array_equal(ranks[r]["f_out"], full)
        np.testing.assert_allclose(ranks[r]["f_grad"], csum, rtol=1e-15, atol=1e-15)


def test_sequence_gather_natural_order(ranks):
    full = _full_input().numpy()
    csum = sum(_weights(r).view(B, S, H).numpy() for r in range(WORLD))
    sl = S // WORLD
    for r in range(WORLD):
        np.testing.assert_array_equal(ranks[r]["sp_out"], full)
        np.testing.assert_allclose(ranks[r]["sp_grad"], csum[:, r * sl:(r + 1) * sl],
                                   rtol=1e-15, atol=1e-15)


def test_rank_major_gather_matches_labels_and_reduce_scatters(ranks):
    full = _full_input().numpy().reshape(B * S, H)
    sl = S // WORLD
    # row (q, b, j) of the gather is token (b, q*sl + j)
    order = np.array([b * S + q * sl + j for q in range(WORLD) for b in range(B)
                      for j in range(sl)])
    csum = sum(_weights(r).view(B * S, H).numpy() for r in range(WORLD))
    for r in range(WORLD):
        np.testing.assert_array_equal(ranks[r]["rm_tok"], order)
        np.testing.assert_array_equal(ranks[r]["rm_out"], full[order])
        want = csum[r * B * sl:(r + 1) * B * sl].reshape(B, sl, H)
        np.testing.assert_allclose(ranks[r]["rm_grad"], want, rtol=1e-15, atol=1e-15)


def test_single_rank_mappings_are_identity():
    import nmce
    ctx = nmce.ParallelContext.single()
    x = torch.randn(2, 4, 3, requires_grad=True)
    for fn in (nmce.copy_to_tensor_parallel_region, nmce.gather_from_sequence_parallel_region):
        y = fn(x, ctx)
        assert torch.equal(y, x)
    rows = nmce.gather_tokens_rank_major(x, ctx)
    assert torch.equal(rows, x.reshape(8, 3))
    rows.sum().backward()
    assert torch.equal(x.grad, torch.ones_like(x))
    assert torch.equal(nmce.targets_rank_major(torch.arange(8).view(2, 4), 1), torch.arange(8))


def test_targets_rank_major_rejects_ragged_sequence():
    import nmce
    with pytest.raises(ValueError, match="not divisible"):
        nmce.targets_rank_major(torch.zeros(2, 5, dtype=torch.int64), 2)
