"""Topology fields the loss path reads, and the vocabulary shard rule.

The loss functions only read ``ctx.tp_size``, ``ctx.tp_rank`` and
``ctx.tp_group``, so nano-megatron's own ``ParallelContext``
(nano_megatron/parallel.py:11-42) can be passed unchanged. This module gives a
stand-alone equivalent with the same field names and ``single()``
constructor for callers that do not import nano-megatron.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Any


@dataclass(frozen=True)
class ParallelContext:
    """Topology state of one rank (fields as in nano_megatron/parallel.py:11-30)."""

    rank: int
    world_size: int
    tp_size: int
    tp_rank: int
    pp_size: int
    pp_rank: int
    dp_size: int
    dp_rank: int
    tp_group: Any = None
    pp_group: Any = None
    dp_group: Any = None
    tied_group: Any = None
    tp_ranks: tuple[int, ...] = (0,)
    pp_ranks: tuple[int, ...] = (0,)
    dp_ranks: tuple[int, ...] = (0,)

    @classmethod
    def single(cls) -> "ParallelContext":
        """One rank, TP=PP=DP=1, no process groups (parallel.py:31-42)."""
        return cls(rank=0, world_size=1, tp_size=1, tp_rank=0, pp_size=1, pp_rank=0,
                   dp_size=1, dp_rank=0)


def divide(numerator: int, denominator: int) -> int:
    """Exact division or ``ValueError`` (tp_layers.py:28-31)."""
    if numerator % denominator != 0:
        raise ValueError(f"{numerator} is not divisible by {denominator}")
    return numerator // denominator


def vocab_range(vocab_size: int, tp_size: int, tp_rank: int) -> tuple[int, int]:
    """Global id range ``[start, end)`` held by TP rank ``tp_rank``.

    Each rank holds ``vocab_size / tp_size`` consecutive ids
    (tp_layers.py:98-106, model.py:242-245).
    """
    per = divide(vocab_size, tp_size)
    return tp_rank * per, (tp_rank + 1) * per
