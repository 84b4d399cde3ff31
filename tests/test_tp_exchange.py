"""The TP > 1 statistics exchange on the CPU (gloo, two ranks on 127.0.0.1).

The reference combines the shards' (max, target pick, exp-sum) with three
dependent all-reduces (cross_entropy.py:22-23, :37-38, :42-43); the drop-in
all-gathers the packed ``[3, rows]`` statistics (max, exp-sum, target
logit) once and combines locally.
This checks the gather's layout and rank order, and that the oracle's combine
of the gathered stack equals the full-vocabulary closed form.
"""

from __future__ import annotations

import os
import socket

import numpy as np
import torch
import torch.distributed as dist
import torch.multiprocessing as mp

WORLD = 2
ROWS, SHARD = 6, 16


def _free_port() -> int:
    with socket.socket() as s:
        s.bind(("127.0.0.1", 0))
        return s.getsockname()[1]


def _worker(rank: int, port: int, out_dir: str) -> None:
    os.environ["MASTER_ADDR"] = "127.0.0.1"
    os.environ["MASTER_PORT"] = str(port)
    dist.init_process_group("gloo", rank=rank, world_size=WORLD)
    try:
        from nmce.cross_entropy import _exchange_stats
        from oracle import ce_oracle
        g = torch.Generator().manual_seed(7)
        x = torch.randn(ROWS, WORLD * SHARD, generator=g, dtype=torch.float64) * 3.0
        t = torch.randint(0, WORLD * SHARD, (ROWS,), generator=g)
        lo = rank * SHARD
        local = torch.from_numpy(np.stack(ce_oracle.shard_stats(
            x[:, lo:lo + SHARD].numpy(), t.numpy(), lo))).float()
        gathered = _exchange_stats(local, None, WORLD)
        np.save(os.path.join(out_dir, f"rank{rank}.npy"), gathered.numpy())
    finally:
        dist.destroy_process_group()


def test_exchange_gathers_shards_in_rank_order(tmp_path):
    port = _free_port()
    mp.start_processes(_worker, args=(port, str(tmp_path)), nprocs=WORLD, join=True,
                       start_method="spawn")
    from oracle import ce_oracle
    g = torch.Generator().manual_seed(7)
    x = torch.randn(ROWS, WORLD * SHARD, generator=g, dtype=torch.float64) * 3.0
    t = torch.randint(0, WORLD * SHARD, (ROWS,), generator=g)
    want = []
    for r in range(WORLD):
        lo = r * SHARD
        want.append(np.stack(ce_oracle.shard_stats(x[:, lo:lo + SHARD].numpy(), t.numpy(),
                                                   lo)).astype(np.float32))
    want = np.stack(want)
    for r in range(WORLD):
        got = np.load(tmp_path / f"rank{r}.npy")
        assert got.shape == (WORLD, 3, ROWS)
        np.testing.assert_array_equal(got, want)
    # the gathered stack combines to the full-vocabulary loss
    stack = want.astype(np.float64)
    _, _, loss = ce_oracle.combine([tuple(stack[r]) for r in range(WORLD)])
    full, _ = ce_oracle.closed_form(x.numpy(), t.numpy())
    np.testing.assert_allclose(loss, full, rtol=1e-5)
