"""The collectives on the LM head's input side, as autograd Functions.

Before the projection ``x @ W.t()`` the reference maps the hidden state into
the tensor-parallel region (model.py:188-191):

* without sequence parallelism, ``f`` (mappings.py:83-94): identity forward,
  all-reduce of the input gradient across the TP group on the way back;
* with sequence parallelism, the sequence all-gather (mappings.py:109-120):
  ``[B, S/tp, H]`` shards gathered into ``[B, S, H]`` forward, and the input
  gradient SUM-reduce-scattered back to the shards.

The loss needs every token once but not in any particular order, so the fused
LM head takes the gathered tokens in rank-major order, ``[tp * B * S/tp, H]``:
that is the layout ``all_gather_into_tensor`` produces and
``reduce_scatter_tensor`` consumes, so neither direction transposes anything
(the reference goes sequence-first and back, two copies each way,
mappings.py:43-79). The targets are permuted to the same order, which is an
int64 copy of one value per token. The natural-order gather stays available
for callers that want the logits themselves.

A gloo group gets host copies of device tensors: gloo collectives are only
run on CPU tensors here.
"""

from __future__ import annotations

import torch
import torch.distributed as dist


def _use_host(t: torch.Tensor, group) -> bool:
    return t.device.type != "cpu" and dist.get_backend(group) == dist.Backend.GLOO


def _all_reduce(t: torch.Tensor, group, world_size: int) -> torch.Tensor:
    """Sum of ``t`` over the group (mappings.py:28-34)."""
    if world_size == 1:
        return t
    if _use_host(t, group):
        h = t.cpu()
        dist.all_reduce(h, group=group)
        return h.to(t.device)
    t = t.contiguous()
    dist.all_reduce(t, group=group)
    return t


def _all_gather_rows(t: torch.Tensor, group, world_size: int) -> torch.Tensor:
    """``[rows, ...]`` of every rank, concatenated in rank order along dim 0."""
    host = _use_host(t, group)
    src = (t.cpu() if host else t).contiguous()
    out = torch.empty((world_size * src.shape[0],) + tuple(src.shape[1:]), dtype=src.dtype,
                      device=src.device)
    dist.all_gather_into_tensor(out, src, group=group)
    return out.to(t.device) if host else out


def _reduce_scatter_rows(t: torch.Tensor, group, world_size: int) -> torch.Tensor:
    """SUM over ranks of ``[world * rows, ...]``; rank r keeps rows block r."""
    if t.shape[0] % world_size:
        raise ValueError(f"{t.shape[0]} rows do not split over {world_size} ranks")
    host = _use_host(t, group)
    src = (t.cpu() if host else t).contiguous()
    out = torch.empty((src.shape[0] // world_size,) + tuple(src.shape[1:]), dtype=src.dtype,
                      device=src.device)
    dist.reduce_scatter_tensor(out, src, op=dist.ReduceOp.SUM, group=group)
    return out.to(t.device) if host else out


def _check_sequence_tensor(t: torch.Tensor) -> None:
    if t.dim() < 2:
        raise ValueError(f"sequence-parallel tensor needs at least 2 dims, got {tuple(t.shape)}")


class _CopyToTensorParallelRegion(torch.autograd.Function):
    """``f``: identity forward, all-reduce backward (mappings.py:83-94)."""

    @staticmethod
    def forward(ctx, x, group, world_size):
        ctx.group, ctx.world_size = group, world_size
        return x.view_as(x)

    @staticmethod
    def backward(ctx, grad):
        return _all_reduce(grad, ctx.group, ctx.world_size), None, None


class _GatherFromSequenceParallelRegion(torch.autograd.Function):
    """``[B, S/tp, ...]`` -> ``[B, S, ...]`` in TP-rank order along dim 1;
    backward SUM-reduce-scatters dim 1 (mappings.py:109-120)."""

    @staticmethod
    def forward(ctx, x, group, world_size):
        _check_sequence_tensor(x)
        ctx.group, ctx.world_size = group, world_size
        if world_size == 1:
            return x.view_as(x)
        g = _all_gather_rows(x.transpose(0, 1), group, world_size)  # [S, B, ...]
        return g.transpose(0, 1).contiguous()

    @staticmethod
    def backward(ctx, grad):
        if ctx.world_size == 1:
            return grad, None, None
        if grad.shape[1] % ctx.world_size:
            raise ValueError(f"sequence length {grad.shape[1]} is not divisible by TP size "
                             f"{ctx.world_size}")
        r = _reduce_scatter_rows(grad.transpose(0, 1), ctx.group, ctx.world_size)
        return r.transpose(0, 1).contiguous(), None, None


class _GatherTokensRankMajor(torch.autograd.Function):
    """``[B, S/tp, H]`` shards -> ``[tp * B * S/tp, H]``, rank r's tokens in
    rows block r; backward SUM-reduce-scatters the rows back. The same
    collectives as the natural-order gather, without the transposes."""

    @staticmethod
    def forward(ctx, x, group, world_size):
        _check_sequence_tensor(x)
        ctx.group, ctx.world_size, ctx.shape = group, world_size, x.shape
        rows = x.reshape(-1, x.shape[-1])
        if world_size == 1:
            return rows.view_as(rows)
        return _all_gather_rows(rows, group, world_size)

    @staticmethod
    def backward(ctx, grad):
        if ctx.world_size == 1:
            return grad.reshape(ctx.shape), None, None
        return (_reduce_scatter_rows(grad, ctx.group, ctx.world_size).reshape(ctx.shape),
                None, None)


def copy_to_tensor_parallel_region(x: torch.Tensor, ctx) -> torch.Tensor:
    """``f`` of mappings.py:83-94 for the group in ``ctx``."""
    return _CopyToTensorParallelRegion.apply(x, ctx.tp_group, ctx.tp_size)


def gather_from_sequence_parallel_region(x: torch.Tensor, ctx) -> torch.Tensor:
    """The sequence all-gather of mappings.py:109-120, in the reference's order."""
    return _GatherFromSequenceParallelRegion.apply(x, ctx.tp_group, ctx.tp_size)


def gather_tokens_rank_major(x: torch.Tensor, ctx) -> torch.Tensor:
    """Every TP rank's ``[B, S/tp, H]`` shard as ``[tp * B * S/tp, H]`` rows,
    rank-major. Pair it with :func:`targets_rank_major` on the labels."""
    return _GatherTokensRankMajor.apply(x, ctx.tp_group, ctx.tp_size)


def targets_rank_major(labels: torch.Tensor, tp_size: int) -> torch.Tensor:
    """Full-sequence ``[B, S]`` labels reordered to the rows of
    :func:`gather_tokens_rank_major`: row ``(r, b, j)`` holds token
    ``(b, r * S/tp + j)``."""
    if labels.dim() != 2:
        raise ValueError(f"labels must be [batch, seq], got {tuple(labels.shape)}")
    b, s = labels.shape
    if s % tp_size:
        raise ValueError(f"sequence length {s} is not divisible by TP size {tp_size}")
    return labels.view(b, tp_size, s // tp_size).transpose(0, 1).reshape(-1)
