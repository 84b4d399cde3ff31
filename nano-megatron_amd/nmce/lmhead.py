"""Fused LM head + vocabulary-parallel cross entropy on gfx950 HIP kernels.

Drop-in for the tail of nano_megatron's ``GPT.forward`` (model.py:277-281):

    logits = self.lm_head(self.final_norm(h))          # x @ W.t(), model.py:192
    return vocab_parallel_cross_entropy(logits, labels, start, end, self.ctx)

becomes

    return lmhead_vocab_parallel_cross_entropy(x, W, labels, start, end, self.ctx)

with ``x`` the (already TP-mapped, model.py:188-191) hidden state and ``W`` the
LM head's vocabulary shard ``[V/tp, H]``. The loss and its gradients with
respect to ``x`` and ``W`` are those of the two-step reference, but the
``[tokens, V/tp]`` logits are never stored: the one-pass path holds the
bf16 exponentials of one chunk of tokens at a time (by default at most a
quarter of them and at most 2 GiB), the recomputing path two bf16 copies of
one vocabulary chunk's logit gradient.

When a gradient is wanted (grad mode on, ``x`` or ``W`` requiring grad) the
wrapper takes the one-pass path: the forward goes through the tokens in
chunks, keeps each chunk's exponentials, forms dZ once the chunk's row
statistics are combined, and computes dX and dW right away for the upstream
value that the last backward from the same call site received (1.0 at
first), as the reference's forward computes the softmax that its backward
returns (cross_entropy.py:48-49). The logits are computed once (6 N V H flops
in all). The backward hands the gradients out, rescaled when its upstream
value differs. Otherwise (no gradient wanted, ``one_pass=False``, or the
per-token Function) the forward keeps two floats per token and the backward
recomputes the logits one vocabulary chunk at a time.

Numerics: the reference runs the projection in bf16 under autocast
(model.py:255-257), so its logits are rounded to bf16 before the loss; here
they stay fp32 from the MFMA accumulators into the softmax. The logit
gradient is rounded to bf16 before the two backward products, as the
reference's autocast matmul backward consumes a bf16 gradient; on the
one-pass path it is formed from the kept exponentials, themselves bf16, so
it carries two roundings (each relative 2^-9) instead of one.

Both ``x`` and ``W`` must be bf16 on a ROCm device; there is no CPU path.
"""

from __future__ import annotations

import sys

import torch

from . import _lib
from .cross_entropy import (_check_hint, _check_target, _exchange_stats, _launch, _site_hint,
                            launch_target_check)
from .mappings import (
    copy_to_tensor_parallel_region,
    gather_from_sequence_parallel_region,
    gather_tokens_rank_major,
    targets_rank_major,
)
from .parallel import divide

# Default vocabulary rows per chunk of the recomputing backward: the chunk's
# logit gradient is held twice in bf16 (4 * tokens * chunk bytes), so no
# tensor the size of the full logits ever exists. A chunk covering the whole
# shard needs no fp32 accumulation of dX, at the price of a full-size dZ.
DEFAULT_VOCAB_CHUNK = 32768

# The one-pass path goes through the tokens in chunks. A chunk's
# exponentials, turned into its dZ^T in place, take 2 * V * chunk bytes
# (bf16), so the chunk bounds what the fused loss holds of the logits: by
# default at most a quarter of the tokens (rounded up to whole 256-token
# tiles; every token only when there are at most 256) and at most
# CHUNK_BUDGET_BYTES, so nothing the size of the [tokens, V] logits is
# allocated. dW is then accumulated in fp32 across the chunks by the GEMM
# epilogue (measured on one MI355X: [16384, 4096] x [128256, 4096] 3.4% slower
# in four chunks of 4096 tokens than in one chunk, [16384, 3072] x
# [256000, 3072] 1.6%).
CHUNK_BUDGET_BYTES = 2 << 30
CHUNK_FRACTION = 4


def default_token_chunk(n_tokens: int, vocab_local: int) -> int:
    """Tokens per one-pass chunk: a quarter of the tokens rounded up to a
    multiple of 256 (at least 256), and no more than fit
    ``CHUNK_BUDGET_BYTES`` of bf16 exponentials (at least 256)."""
    quarter = -(-n_tokens // CHUNK_FRACTION)
    chunk = max(256, -(-quarter // 256) * 256)
    fit = max(256, CHUNK_BUDGET_BYTES // (2 * max(1, vocab_local)) // 256 * 256)
    return min(chunk, fit, max(n_tokens, 1))

_ALIGN = 64  # hidden size granularity of the GEMM kernels


def _padded_hidden(t: torch.Tensor, hp: int) -> torch.Tensor:
    """``t`` [rows, H] as a contiguous [rows, hp] bf16 tensor (zero columns appended)."""
    rows, h = t.shape
    if h == hp and t.is_contiguous() and t.data_ptr() % 16 == 0:
        return t
    out = torch.zeros((rows, hp), dtype=t.dtype, device=t.device)
    out[:, :h] = t
    return out


def _workspace(nbytes: int, device: torch.device) -> torch.Tensor:
    return torch.empty(max(int(nbytes), 16), dtype=torch.uint8, device=device)


def _fused_layout(lib, n: int, hp: int, v: int, token_chunk: int) -> dict:
    import ctypes
    buf = (ctypes.c_int64 * _lib.NMCE_LMHEAD_FUSED_LAYOUT_FIELDS)()
    _lib.check(lib.nmce_lmhead_ce_fused_layout(n, hp, v, token_chunk, ctypes.addressof(buf)),
               "nmce_lmhead_ce_fused_layout")
    keys = ("total", "chunk", "n_chunks", "ldt", "vpad", "nb", "off_pt", "off_part", "off_acc",
            "off_dxp", "dx_splits", "off_xt")
    return dict(zip(keys, (int(b) for b in buf)))


def _check_fused_operands(hidden, weight, vocab_start, vocab_end):
    if not (hidden.is_cuda and weight.is_cuda):
        raise RuntimeError("nmce: hidden and weight must be on a ROCm device "
                           "(there is no CPU path)")
    if hidden.dtype != torch.bfloat16 or weight.dtype != torch.bfloat16:
        raise TypeError("nmce: the fused LM head computes in bf16; got hidden "
                        f"{hidden.dtype}, weight {weight.dtype}")
    if weight.dim() != 2 or hidden.shape[-1] != weight.shape[1]:
        raise ValueError(f"nmce: hidden {tuple(hidden.shape)} and weight "
                         f"{tuple(weight.shape)} do not share the hidden size")
    if weight.shape[0] != vocab_end - vocab_start:
        raise ValueError(f"nmce: weight holds {weight.shape[0]} vocabulary rows but the "
                         f"shard [{vocab_start}, {vocab_end}) has {vocab_end - vocab_start}")


class _LMHeadVocabParallelCrossEntropyMean(torch.autograd.Function):
    """Mean loss of ``hidden @ weight.t()`` over a vocabulary shard, one pass.

    ``forward(hidden, weight, target, vocab_start, vocab_end, group,
    world_size, hint, token_chunk)`` returns the 0-dim mean of the per-token
    loss (torch's mean, cross_entropy.py:85) and computes the gradients of
    ``hidden`` and ``weight`` for the upstream value ``usable(hint[0])`` of
    the mean, chunk by chunk over the tokens (nmce_lmhead_ce_fused_*). The
    backward hands them out when its upstream value is that one and rescales
    them otherwise (within two bf16 units in the last place; exactly for a
    power-of-two ratio), writing the value it received into ``hint``. A
    second backward through the same graph recomputes them (the vocabulary-
    chunked backward of ``_LMHeadVocabParallelCrossEntropy``).
    """

    @staticmethod
    def forward(ctx, hidden, weight, target, vocab_start, vocab_end, group, world_size, hint,
                token_chunk=None):
        _check_fused_operands(hidden, weight, vocab_start, vocab_end)
        _check_target(target, hidden.shape[:-1], hidden.device)
        lib = _lib.load()
        dev = hidden.device
        stream = _lib.stream_handle(dev)
        H = hidden.shape[-1]
        V = weight.shape[0]
        hp = (H + _ALIGN - 1) // _ALIGN * _ALIGN
        x = _padded_hidden(hidden.reshape(-1, H), hp)
        w = _padded_hidden(weight, hp)
        n = x.shape[0]
        tgt = target.reshape(-1)
        if not tgt.is_contiguous():
            tgt = tgt.contiguous()
        ctx.vocab_start = vocab_start
        ctx.hidden_shape = hidden.shape
        ctx.H = H
        ctx.hint = hint
        ctx.handed_out = False
        if n == 0:  # an empty batch: nothing to launch; torch's mean of nothing
            ctx.empty = True
            ctx.weight_shape = weight.shape
            return torch.empty(0, dtype=torch.float32, device=dev).mean()
        ctx.empty = False
        chunk = default_token_chunk(n, V) if token_chunk is None else int(token_chunk)
        L = _fused_layout(lib, n, hp, V, chunk)
        ws = _workspace(L["total"], dev)
        args = (x.data_ptr(), w.data_ptr(), _lib.NMCE_BF16, n, hp, V)
        assumed = torch.empty(1, dtype=torch.float32, device=dev)
        _launch("nmce_hint_assume", lib.nmce_hint_assume, hint.data_ptr(), assumed.data_ptr(),
                stream)
        local = torch.empty((3, n), dtype=torch.float32, device=dev)  # max, sum - 1, target z
        out = torch.empty((3, n), dtype=torch.float32, device=dev)    # loss, max, sum - 1
        dx = torch.empty((n, hp), dtype=torch.bfloat16, device=dev)
        dw = torch.empty((V, hp), dtype=torch.bfloat16, device=dev)
        step = L["chunk"]
        for c in range(L["n_chunks"]):
            t0 = c * step
            nc = min(step, n - t0)
            _launch("nmce_lmhead_ce_fused_chunk_stats", lib.nmce_lmhead_ce_fused_chunk_stats,
                    *args, tgt.data_ptr(), vocab_start, chunk, c, local[0].data_ptr(),
                    local[1].data_ptr(), local[2].data_ptr(), ws.data_ptr(), ws.numel(), stream)
            if world_size == 1:
                base, stride = local.data_ptr() + 4 * t0, 3 * n
            else:
                stats = _exchange_stats(local[:, t0:t0 + nc], group, world_size)
                base, stride = stats.data_ptr(), 3 * nc
            _launch("nmce_ce_combine", lib.nmce_ce_combine, base, base + 4 * (stride // 3),
                    base + 8 * (stride // 3), world_size, stride, nc,
                    out[0].data_ptr() + 4 * t0, out[1].data_ptr() + 4 * t0,
                    out[2].data_ptr() + 4 * t0, stream)
            _launch("nmce_lmhead_ce_fused_chunk_grads", lib.nmce_lmhead_ce_fused_chunk_grads,
                    *args, tgt.data_ptr(), vocab_start, chunk, c, out[1].data_ptr(),
                    out[2].data_ptr(), local[2].data_ptr(), assumed.data_ptr(), 0, float(n),
                    dx.data_ptr(), dw.data_ptr(), ws.data_ptr(), ws.numel(), stream)
        ctx.save_for_backward(x, w, tgt, out[1:], dx, dw, assumed)
        return out[0].mean()

    @staticmethod
    def backward(ctx, grad_output):
        if ctx.empty:
            dev = grad_output.device
            return (torch.zeros(ctx.hidden_shape, dtype=torch.bfloat16, device=dev),
                    torch.zeros(ctx.weight_shape, dtype=torch.bfloat16, device=dev),
                    None, None, None, None, None, None, None)
        x, w, tgt, row_stat, dx, dw, assumed = ctx.saved_tensors
        lib = _lib.load()
        go = grad_output.reshape(1)
        if go.dtype != torch.float32:
            go = go.float()
        n, hp = x.shape
        V = w.shape[0]
        if ctx.handed_out:
            # dx / dw belong to the first backward's consumers: recompute.
            g_tok = go / n  # the per-token value MeanBackward forms, broadcast
            dw = torch.empty((V, hp), dtype=torch.bfloat16, device=x.device)
            dx = _recompute_backward(lib, x, w, tgt, ctx.vocab_start, row_stat, g_tok, 0,
                                     DEFAULT_VOCAB_CHUNK, dw)
        else:
            stream = _lib.stream_handle(x.device)
            _launch("nmce_ce_grad_rescale_unless", lib.nmce_ce_grad_rescale_unless,
                    dx.data_ptr(), _lib.NMCE_BF16, n, hp, hp, go.data_ptr(), assumed.data_ptr(),
                    ctx.hint.data_ptr(), stream)
            _launch("nmce_ce_grad_rescale_unless", lib.nmce_ce_grad_rescale_unless,
                    dw.data_ptr(), _lib.NMCE_BF16, V, hp, hp, go.data_ptr(), assumed.data_ptr(),
                    None, stream)
            ctx.handed_out = True
        H = ctx.H
        if hp != H:
            dx = dx[:, :H]
            dw = dw[:, :H].contiguous()
        return (dx.reshape(ctx.hidden_shape), dw, None, None, None, None, None, None, None)


def _recompute_backward(lib, x, w, tgt, vocab_start, row_stat, go, gstride, vocab_chunk, dw):
    """dX (returned) and dW (into ``dw``) by recomputing the logits one
    vocabulary chunk at a time (nmce_lmhead_ce_bwd: the dZ kernel and the
    library's own MFMA GEMM for both products)."""
    n, hp = x.shape
    V = w.shape[0]
    dev = x.device
    dx = torch.empty((n, hp), dtype=torch.bfloat16, device=dev)
    ws = _workspace(lib.nmce_lmhead_ce_bwd_workspace_bytes(n, hp, V, vocab_chunk), dev)
    _launch("nmce_lmhead_ce_bwd", lib.nmce_lmhead_ce_bwd, x.data_ptr(), w.data_ptr(),
            _lib.NMCE_BF16, n, hp, V, tgt.data_ptr(), vocab_start,
            row_stat[0].data_ptr(), row_stat[1].data_ptr(), go.data_ptr(), gstride,
            dx.data_ptr(), dw.data_ptr(), vocab_chunk, ws.data_ptr(), ws.numel(),
            _lib.stream_handle(dev))
    return dx


class _LMHeadVocabParallelCrossEntropy(torch.autograd.Function):
    """Per-token loss of ``hidden @ weight.t()`` over a vocabulary shard.

    ``forward(hidden, weight, target, vocab_start, vocab_end, group, world_size,
    vocab_chunk=None)``: ``hidden`` is ``[..., H]`` bf16, ``weight`` is
    ``[vocab_end - vocab_start, H]`` bf16 and ``target`` has ``hidden``'s
    leading shape. Returns the fp32 per-token loss (cross_entropy.py:45).
    ``backward`` returns the bf16 gradients of ``hidden`` (this shard's
    contribution) and ``weight``.
    """

    @staticmethod
    def forward(ctx, hidden, weight, target, vocab_start, vocab_end, group, world_size,
                vocab_chunk=None):
        _check_fused_operands(hidden, weight, vocab_start, vocab_end)
        _check_target(target, hidden.shape[:-1], hidden.device)
        lib = _lib.load()
        dev = hidden.device
        stream = _lib.stream_handle(dev)
        H = hidden.shape[-1]
        V = weight.shape[0]
        hp = (H + _ALIGN - 1) // _ALIGN * _ALIGN
        x = _padded_hidden(hidden.reshape(-1, H), hp)
        w = _padded_hidden(weight, hp)
        n = x.shape[0]
        tgt = target.reshape(-1)
        if not tgt.is_contiguous():
            tgt = tgt.contiguous()

        ctx.vocab_start = vocab_start
        ctx.vocab_chunk = DEFAULT_VOCAB_CHUNK if vocab_chunk is None else int(vocab_chunk)
        ctx.hidden_shape = hidden.shape
        ctx.H = H
        if n == 0:  # an empty batch: nothing to launch
            ctx.empty = True
            ctx.weight_shape = weight.shape
            return torch.empty(target.shape, dtype=torch.float32, device=dev)
        ctx.empty = False
        out = torch.empty((3, n), dtype=torch.float32, device=dev)  # loss, max, sumexp - 1
        loss, row_stat = out[0], out[1:]
        local = torch.empty((3, n), dtype=torch.float32, device=dev)
        ws = _workspace(lib.nmce_lmhead_ce_fwd_workspace_bytes(n, hp, V), dev)
        _launch("nmce_lmhead_ce_fwd_stats", lib.nmce_lmhead_ce_fwd_stats, x.data_ptr(),
                w.data_ptr(), _lib.NMCE_BF16, n, hp, V, tgt.data_ptr(), vocab_start,
                local[0].data_ptr(), local[1].data_ptr(), local[2].data_ptr(), ws.data_ptr(),
                ws.numel(), stream)
        if world_size == 1:
            stats, stride = local, 3 * n
        else:
            stats, stride = _exchange_stats(local, group, world_size), 3 * n
        base = stats.data_ptr()
        _launch("nmce_ce_combine", lib.nmce_ce_combine, base, base + 4 * n, base + 8 * n,
                world_size, stride, n, loss.data_ptr(), row_stat[0].data_ptr(),
                row_stat[1].data_ptr(), stream)

        ctx.save_for_backward(x, w, tgt, row_stat)
        return loss.view(target.shape)

    @staticmethod
    def backward(ctx, grad_output):
        if ctx.empty:
            dev = grad_output.device
            return (torch.zeros(ctx.hidden_shape, dtype=torch.bfloat16, device=dev),
                    torch.zeros(ctx.weight_shape, dtype=torch.bfloat16, device=dev),
                    None, None, None, None, None, None)
        x, w, tgt, row_stat = ctx.saved_tensors
        lib = _lib.load()
        dev = x.device
        n, hp = x.shape
        V = w.shape[0]
        go = grad_output
        if go.dtype != torch.float32:
            go = go.float()
        if go.numel() > 0 and all(s == 0 for s in go.stride()):
            gstride = 0  # expanded scalar, e.g. from loss.mean()
        else:
            go = go.reshape(-1)
            if not go.is_contiguous():
                go = go.contiguous()
            gstride = 1
        dw = torch.empty((V, hp), dtype=torch.bfloat16, device=dev)
        dx = _recompute_backward(lib, x, w, tgt, ctx.vocab_start, row_stat, go, gstride,
                                 ctx.vocab_chunk, dw)
        H = ctx.H
        if hp != H:
            dx = dx[:, :H]
            dw = dw[:, :H].contiguous()
        return (dx.reshape(ctx.hidden_shape), dw, None, None, None, None, None, None)


def lmhead_vocab_parallel_cross_entropy(
    hidden: torch.Tensor,
    weight: torch.Tensor,
    target: torch.Tensor,
    vocab_start: int,
    vocab_end: int,
    ctx,
    *,
    vocab_chunk: int | None = None,
    token_chunk: int | None = None,
    validate: bool = True,
    one_pass: bool = True,
    upstream_hint: torch.Tensor | None = None,
) -> torch.Tensor:
    """Mean cross-entropy of ``hidden @ weight.t()`` against ``target``.

    Equals ``vocab_parallel_cross_entropy(hidden @ weight.t(), target,
    vocab_start, vocab_end, ctx)`` (cross_entropy.py:68-85 after
    model.py:192) without storing the logits. ``hidden`` is ``[b, s, H]`` (or
    ``[tokens, H]``), ``weight`` is ``[V/tp, H]``; returns a 0-dim fp32
    tensor. Same ``ValueError`` as the reference for an out-of-range target.

    When a gradient is wanted the forward is one pass (module docstring),
    going through ``token_chunk`` tokens at a time (default
    ``default_token_chunk``: a quarter of the tokens, within
    ``CHUNK_BUDGET_BYTES``; pass the token count to hold every token's
    exponentials at once) and assuming the upstream value held by
    ``upstream_hint`` (a one-element fp32 device tensor; default: one per
    call site). ``one_pass=False`` selects the forward that keeps only the
    row statistics, with a backward that recomputes the logits in chunks of
    ``vocab_chunk`` vocabulary rows.

    The product is computed in bf16. Inside a bf16 autocast region (as
    model.py:255-257 runs the LM head) an fp32 ``hidden`` or ``weight`` is cast
    to bf16 the way autocast casts a matmul's operands: through autograd, so an
    fp32 parameter receives the bf16 gradient cast back to fp32 and summed into
    its ``.grad`` with every other use of it (the tied embedding,
    model.py:235-236). Outside autocast, both must already be bf16.
    """
    if not (hidden.is_cuda and weight.is_cuda):
        raise RuntimeError("nmce: hidden and weight must be on a ROCm device "
                           "(there is no CPU path)")
    if hidden.dtype != torch.bfloat16 or weight.dtype != torch.bfloat16:
        dev_type = hidden.device.type
        if not (torch.is_autocast_enabled(dev_type)
                and torch.get_autocast_dtype(dev_type) == torch.bfloat16):
            raise TypeError("nmce: the fused LM head computes in bf16; got hidden "
                            f"{hidden.dtype}, weight {weight.dtype} outside a bf16 autocast "
                            "region")
        hidden = hidden.to(torch.bfloat16)
        weight = weight.to(torch.bfloat16)
    vocab_size = ctx.tp_size * (vocab_end - vocab_start)
    _check_target(target, hidden.shape[:-1], hidden.device)
    want_grad = torch.is_grad_enabled() and (hidden.requires_grad or weight.requires_grad)
    if one_pass and want_grad:
        if upstream_hint is None:
            caller = sys._getframe(1)
            hint = _site_hint(hidden.device, (caller.f_code.co_filename, caller.f_lineno))
        else:
            _check_hint(upstream_hint, hidden.device)
            hint = upstream_hint
    pending = launch_target_check(target, vocab_size) if validate else None
    try:
        if one_pass and want_grad:
            loss = _LMHeadVocabParallelCrossEntropyMean.apply(
                hidden, weight, target, vocab_start, vocab_end, ctx.tp_group, ctx.tp_size, hint,
                token_chunk)
        else:
            loss = _LMHeadVocabParallelCrossEntropy.apply(
                hidden, weight, target, vocab_start, vocab_end, ctx.tp_group, ctx.tp_size,
                vocab_chunk).mean()
    except BaseException:
        if pending is not None:
            pending.wait()  # the check kernel writes into the pending host buffer
        raise
    if pending is not None:
        pending.raise_if_bad()
    return loss


class FusedParallelLMHead(torch.nn.Module):
    """Vocabulary-sharded output projection with the loss fused in.

    Drop-in for nano_megatron's ``ParallelLMHead`` (model.py:169-192): the
    same constructor ``(config, ctx)`` (reads ``config.vocab_size``,
    ``config.n_embd`` and ``config.sequence_parallel``), the same ``weight``
    parameter ``[V/tp, n_embd]`` initialised N(0, 0.02^2) and marked
    ``tensor_parallel_sharded``, so ``lm_head.weight = embedding.weight`` ties
    it as model.py:235-236 does. ``forward(x)`` returns the logits exactly as
    the reference's forward does (a plain matmul; there is nothing to fuse).
    ``forward(x, labels)`` returns the mean cross entropy of those logits
    against the full-vocabulary ``labels`` ``[B, S]`` without storing them,
    i.e. what ``vocab_parallel_cross_entropy(self(x), labels, *range, ctx)``
    returns (model.py:277-281).

    The input mapping is the reference's (model.py:188-191): ``f`` (identity,
    all-reduced input gradient) at TP > 1, or the sequence all-gather under
    sequence parallelism, which the loss takes in rank-major token order (no
    transposes; the labels are permuted to match).
    """

    def __init__(self, config, ctx):
        super().__init__()
        self.ctx = ctx
        per_partition = divide(config.vocab_size, ctx.tp_size)
        self.weight = torch.nn.Parameter(torch.empty(per_partition, config.n_embd))
        self.weight.tensor_parallel_sharded = True
        self.sequence_parallel = bool(getattr(config, "sequence_parallel", False))
        self.vocab_chunk = None  # backward chunk; None = DEFAULT_VOCAB_CHUNK
        self.token_chunk = None  # one-pass chunk; None = default_token_chunk
        # The upstream value the one-pass forward assumes, per module and
        # device (created on first use on that device).
        self._hints: dict = {}
        torch.nn.init.normal_(self.weight, std=0.02)

    def vocab_range(self) -> tuple[int, int]:
        """This rank's global id range (model.py:242-245)."""
        per = self.weight.shape[0]
        return self.ctx.tp_rank * per, (self.ctx.tp_rank + 1) * per

    def forward(self, x: torch.Tensor, labels: torch.Tensor | None = None) -> torch.Tensor:
        if labels is None:
            if self.sequence_parallel:
                x = gather_from_sequence_parallel_region(x, self.ctx)
            else:
                x = copy_to_tensor_parallel_region(x, self.ctx)
            return x @ self.weight.t()
        start, end = self.vocab_range()
        if self.sequence_parallel:
            rows = gather_tokens_rank_major(x, self.ctx)
            target = targets_rank_major(labels, self.ctx.tp_size)
        else:
            rows = copy_to_tensor_parallel_region(x, self.ctx)
            target = labels
        dev = rows.device
        hint = self._hints.get(dev)
        if hint is None:
            hint = torch.ones(1, dtype=torch.float32, device=dev)
            self._hints[dev] = hint
        return lmhead_vocab_parallel_cross_entropy(rows, self.weight, target, start, end,
                                                   self.ctx, vocab_chunk=self.vocab_chunk,
                                                   token_chunk=self.token_chunk,
                                                   upstream_hint=hint)
