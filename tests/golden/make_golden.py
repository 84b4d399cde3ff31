"""Write the golden vectors under tests/golden/.

Expected values come from ``torch.nn.functional.cross_entropy`` evaluated in
fp64 on the CPU -- the same library routine nano-megatron's own checks treat
as truth (tests/check_tp_math.py:107 and :146-156) -- and never from this
repository's oracle, so the fixtures pin the oracle rather than echo it.

    python tests/golden/make_golden.py

Fixtures:
  tp_math_2x5x16.npz      the reference check's inputs (torch.manual_seed(0),
                          randn(2,5,16), randint(0,16,(2,5))): per-token loss,
                          mean loss, gradient of the mean.
  shard_pair_f32.npz      [16, 1024] fp32 logits ~ N(0, 1.5^2) split as two
  shard_pair_bf16.npz     TP=2 shards of 512; targets include 0, 511, 512, 1023;
                          per-token loss and the full gradient (of the sum).
  edge_rows.npz           hand-built rows: constant, one dominant logit,
                          logits at +-60, a -inf entry, target at column 0 and
                          at the last column (V = 64).
  c1_digest.json          c1 = fp32 [4,256,32000] ~ N(0, 2^2), targets
                          U[0, 32000), torch.Generator seed 0: sha256 of the
                          inputs, all 1024 per-token losses, the mean, and
                          4096 seeded entries of the gradient of the mean.
"""

from __future__ import annotations

import hashlib
import json
import pathlib

import numpy as np
import torch
import torch.nn.functional as F

OUT = pathlib.Path(__file__).resolve().parent


def ce_fp64(logits: torch.Tensor, target: torch.Tensor, reduction: str):
    x = logits.detach().double().reshape(-1, logits.shape[-1]).requires_grad_(True)
    loss = F.cross_entropy(x, target.reshape(-1), reduction=reduction)
    return x, loss


def tp_math_fixture() -> None:
    torch.manual_seed(0)
    logits = torch.randn(2, 5, 16)
    labels = torch.randint(0, 16, (2, 5))
    _, per_token = ce_fp64(logits, labels, "none")
    x, mean = ce_fp64(logits, labels, "mean")
    mean.backward()
    np.savez(OUT / "tp_math_2x5x16.npz", logits=logits.numpy(), target=labels.numpy(),
             loss=per_token.detach().numpy(), mean=mean.detach().numpy(),
             grad_mean=x.grad.numpy())


def shard_pair_fixture(dtype: torch.dtype, name: str) -> None:
    g = torch.Generator().manual_seed(1234)
    n, vfull = 16, 1024
    logits = (torch.randn(n, vfull, generator=g) * 1.5).to(dtype).float()
    target = torch.randint(0, vfull, (n,), generator=g)
    target[:4] = torch.tensor([0, 511, 512, 1023])
    _, per_token = ce_fp64(logits, target, "none")
    x, total = ce_fp64(logits, target, "sum")
    total.backward()
    np.savez(OUT / name, logits=logits.numpy(), target=target.numpy(), tp=2,
             loss=per_token.detach().numpy(), grad_sum=x.grad.numpy().astype(np.float32))


def edge_rows_fixture() -> None:
    v = 64
    g = torch.Generator().manual_seed(7)
    rows = [
        torch.zeros(v),                                  # constant: loss = log V
        torch.full((v,), 3.25),                          # constant, shifted
        torch.cat([torch.tensor([30.0]), torch.zeros(v - 1)]),  # dominant at the target
        torch.randn(v, generator=g) * 60.0,              # large magnitudes
        torch.randn(v, generator=g).index_fill(0, torch.tensor([5]), float("-inf")),
        torch.randn(v, generator=g) - 100.0,             # all far below zero
        torch.randn(v, generator=g),                     # target at last column
        torch.randn(v, generator=g),                     # target at column 0
    ]
    logits = torch.stack(rows)
    target = torch.tensor([3, 10, 0, 17, 9, 40, v - 1, 0])
    _, per_token = ce_fp64(logits, target, "none")
    x, total = ce_fp64(logits, target, "sum")
    total.backward()
    np.savez(OUT / "edge_rows.npz", logits=logits.numpy(), target=target.numpy(),
             loss=per_token.detach().numpy(), grad_sum=x.grad.numpy())


def c1_inputs():
    """c1 inputs, regenerated identically by the tests from the same seed."""
    g = torch.Generator().manual_seed(0)
    logits = torch.randn(4, 256, 32000, generator=g) * 2.0
    target = torch.randint(0, 32000, (4, 256), generator=g)
    return logits, target


def sha256_of(*tensors: torch.Tensor) -> str:
    h = hashlib.sha256()
    for t in tensors:
        h.update(t.contiguous().numpy().tobytes())
    return h.hexdigest()


def c1_fixture() -> None:
    logits, target = c1_inputs()
    _, per_token = ce_fp64(logits, target, "none")
    x, mean = ce_fp64(logits, target, "mean")
    mean.backward()
    sel = torch.Generator().manual_seed(99)
    rows = torch.randint(0, 1024, (4096,), generator=sel)
    cols = torch.randint(0, 32000, (4096,), generator=sel)
    cols[:1024] = target.reshape(-1)[rows[:1024]]  # include target columns
    doc = {
        "shape": [4, 256, 32000],
        "sha256_inputs": sha256_of(logits, target),
        "loss": per_token.detach().tolist(),
        "mean": float(mean.detach()),
        "grad_rows": rows.tolist(),
        "grad_cols": cols.tolist(),
        "grad_vals": x.grad[rows, cols].tolist(),
    }
    (OUT / "c1_digest.json").write_text(json.dumps(doc))


if __name__ == "__main__":
    torch.set_num_threads(8)
    tp_math_fixture()
    shard_pair_fixture(torch.float32, "shard_pair_f32.npz")
    shard_pair_fixture(torch.bfloat16, "shard_pair_bf16.npz")
    edge_rows_fixture()
    c1_fixture()
    for p in sorted(OUT.iterdir()):
        print(p.name, p.stat().st_size)
