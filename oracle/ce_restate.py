"""torch-CPU restatement of the reference's op sequence, in fp32.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``). This is the timed CPU
baseline of ``bench.py`` (``cpu_baseline.kind = "port"``): the same ATen op
chain nano_megatron/cross_entropy.py runs, step for step, on the host cores.

Forward (cross_entropy.py:68-85 then :17-50):
  upcast (.float(), :83) -> row max (:21) -> [all-reduce MAX (:23)] ->
  shift (:24) -> target mask and local index (:28-30) -> gather and zero the
  masked picks (:32-36) -> [all-reduce SUM (:38)] -> exp (:40) -> row sum
  (:41) -> [all-reduce SUM (:43)] -> loss = log(sum) - pick (:45) -> softmax
  in place (:48).
Backward (:53-65): onehot subtract on owned rows (:59-62), scale by
grad_output (:64), cast back to the logits dtype (autograd of :83).

The all-reduces are a hook: identity at TP=1; for one rank of a TP group the
caller supplies the peers' partial values (the emulated collective).

Pinned by tests/test_oracle.py against ``ce_oracle.closed_form`` (fp64) and
the fp64 ``F.cross_entropy`` golden vectors, at fp32 tolerance.
"""

from __future__ import annotations

from typing import Callable, Optional

import torch

AllReduce = Callable[[torch.Tensor, str], None]  # (tensor, "max" | "sum"), in place


def forward(logits: torch.Tensor, target: torch.Tensor, vocab_start: int, vocab_end: int,
            all_reduce: Optional[AllReduce] = None):
    """Returns ``(per-token loss, saved)``; ``saved`` feeds ``backward``."""
    x = logits.float()
    m = x.max(dim=-1)[0]
    if all_reduce is not None:
        all_reduce(m, "max")
    x = x - m.unsqueeze(-1)
    mask = (target < vocab_start) | (target >= vocab_end)
    local = (target - vocab_start).clone()
    local[mask] = 0
    flat = x.view(-1, x.size(-1))
    rows = torch.arange(flat.size(0))
    pick = flat[rows, local.view(-1)].view_as(target).clone()
    pick[mask] = 0.0
    if all_reduce is not None:
        all_reduce(pick, "sum")
    e = x.exp()
    s = e.sum(dim=-1)
    if all_reduce is not None:
        all_reduce(s, "sum")
    loss = s.log() - pick
    e.div_(s.unsqueeze(-1))
    return loss, (e, mask, local, logits.dtype)


def backward(saved, grad_output: torch.Tensor) -> torch.Tensor:
    """Gradient w.r.t. the logits, in the logits dtype."""
    e, mask, local, dtype = saved
    flat = e.view(-1, e.size(-1))
    rows = torch.arange(flat.size(0))
    keep = (~mask).view(-1).to(flat.dtype)
    flat[rows, local.view(-1)] -= keep
    e.mul_(grad_output.unsqueeze(-1))
    return e.to(dtype)


def peer_partials(peer_logits: torch.Tensor, target: torch.Tensor, vocab_start: int,
                  vocab_end: int, global_max: torch.Tensor):
    """What one peer rank contributes to the SUM all-reduces (:38, :43), given
    the already reduced global max: its masked shifted target pick and its
    exp-sum."""
    x = peer_logits.float() - global_max.unsqueeze(-1)
    mask = (target < vocab_start) | (target >= vocab_end)
    local = (target - vocab_start).clamp(0, x.size(-1) - 1)
    pick = x.gather(-1, local.unsqueeze(-1)).squeeze(-1)
    pick[mask] = 0.0
    return pick, x.exp().sum(dim=-1)


def fixed_peer_all_reduce(peer_max: torch.Tensor, peer_pick: torch.Tensor,
                          peer_sum: torch.Tensor) -> AllReduce:
    """An emulated TP all-reduce for one rank whose peers' partials are known
    in advance (max at :23, target pick at :38, exp-sum at :43, in that order)."""
    order = iter([("max", peer_max), ("sum", peer_pick), ("sum", peer_sum)])

    def reduce(t: torch.Tensor, op: str) -> None:
        expect, value = next(order)
        if op != expect:
            raise RuntimeError(f"all-reduce order: got {op}, expected {expect}")
        if op == "max":
            torch.maximum(t, value, out=t)
        else:
            t.add_(value)

    return reduce
