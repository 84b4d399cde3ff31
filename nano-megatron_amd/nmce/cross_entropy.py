"""Cross entropy over a vocabulary-sharded logit slab, on gfx950 HIP kernels.

Drop-in for nano_megatron/cross_entropy.py:16-85. Same names, same arguments,
same returned loss (per-token fp32 from the Function, its mean from the
wrapper), same ``ValueError`` for a target outside the vocabulary.

Differences from the reference, all deliberate:

* bf16 logits are consumed directly. The reference upcasts them with
  ``.float()`` (cross_entropy.py:83) and autograd casts the fp32 gradient
  back; here the math is fp32 in registers and the gradient is written once,
  in the logits dtype.
* Nothing of size ``[tokens, vocab]`` is kept between forward and backward:
  the reference saves the fp32 softmax (:48-49); this keeps two floats per
  token (row max, row exp-sum minus one) and recomputes the softmax in
  backward from the logits. The exp-sum leaves out the maximum's own term
  (exactly 1), so a confident token's loss log1p(sum - 1) and target gradient
  -(sum - 1)/sum * g keep their relative precision; the reference's log(sum)
  and softmax - 1 give the same values up to fp32 cancellation near 1.
* The wrapper at TP = 1, when a gradient is wanted (grad mode on and the
  logits require grad) and the rows fit (V a whole number of 16-byte
  vectors, at most 131072 bf16 / 65536 fp32 columns), reads the logits once:
  its forward also writes the gradient for the upstream value that the last
  backward from the same call site received (1.0, as for
  ``loss.backward()``, before the first) -- as the reference's forward
  computes the softmax its backward returns (:48-49). A loss scaled the same
  way every step keeps the forward's gradient from the second step on. The
  gradient goes into a new ``[tokens, vocab]`` buffer, or into the logits'
  own storage when the caller asks for that with ``inplace=True``. A
  backward whose upstream value differs rewrites a separate buffer from the
  logits (bit-identical to the two-pass path), and rescales an in-place one
  (within four fp32 or two bf16 units in the last place: the written
  gradient and the ratio are each rounded once; exact for a power-of-two
  ratio). ``one_pass=False`` turns it off. This path's autograd node is C++
  (``_nmce_autograd``, built beside ``libnmce.so``): a Python node's backward
  costs the engine a hand-over to the interpreter, tens of microseconds per
  call, which a small batch pays in full.
* The gradient is written **in place** into the logits storage with
  ``inplace=True`` (as at model.py:277-281, where the logits come straight
  from the LM-head matmul, which does not save them): by the forward on the
  one-pass path, by the backward on the two-pass path. With the default
  ``inplace=None`` the forward never writes into the logits: the one-pass
  path writes a new buffer, and the two-pass backward writes into non-leaf
  logits only once the backward runs (the forward has returned by then).
  ``inplace=False`` never writes into them; leaf tensors are never
  overwritten. The version counter of the logits is bumped after an
  in-place write, so any other autograd node that saved them fails loudly
  instead of reading gradients. A target outside the vocabulary leaves the
  logits untouched on every path: the one-pass kernel reads a flag that the
  target check sets on the same stream before it writes anything.
* With ``tp_size > 1`` the three dependent all-reduces (:23, :38, :43) become
  one all-gather of packed ``[3, tokens]`` statistics followed by a local
  combine.
* The wrapper's ``loss.mean()`` (:85) is taken inside its own Function, whose
  backward hands the loss kernel the mean's scalar gradient and the token
  count: the kernel divides in fp32 exactly as ``MeanBackward`` would, so the
  gradient is bit-identical and the expand/divide pass is gone.

There is no CPU path: the tensors must be on a ROCm device and ``libnmce.so``
must be built; anything else raises.
"""

from __future__ import annotations

import sys
import threading

import torch
import torch.distributed as dist

from . import _lib

# Optional launch timeline. When set to a list, every kernel launch of this
# module appends (name, start_event, end_event), both recorded on the launch
# stream, so a caller can time each kernel inside a running workload.
kernel_timeline: list | None = None

# Per (device, call site): one float, the upstream value of the mean that the
# last one-pass backward of a loss computed at that site received (the 1.0 of
# ``loss.backward()`` until one has run). The one-pass forward computes the
# gradient for it, so a training loop that scales its loss the same way every
# step (e.g. by 1/num_microbatches, pipeline.py:127) keeps the forward's
# gradient from its second step on, and two losses scaled differently at two
# sites do not spoil each other's guess. The backward writes it in stream
# order; no host synchronisation is involved.
_upstream_hints: dict[tuple, torch.Tensor] = {}


def _site_hint(dev: torch.device, site: tuple) -> torch.Tensor:
    idx = dev.index if dev.index is not None else torch.cuda.current_device()
    key = (idx,) + site
    t = _upstream_hints.get(key)
    if t is None:
        t = torch.ones(1, dtype=torch.float32, device=dev)
        _upstream_hints[key] = t
    return t


def _check_hint(hint: torch.Tensor, dev: torch.device) -> None:
    if hint.device != dev or hint.dtype != torch.float32 or hint.numel() != 1:
        raise ValueError("nmce: upstream_hint must be a one-element float32 tensor on the "
                         "logits' device")


def _launch(name: str, fn, *args) -> None:
    timeline = kernel_timeline
    if timeline is None:
        _lib.check(fn(*args), name)
        return
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    status = fn(*args)
    end.record()
    timeline.append((name, start, end))
    _lib.check(status, name)


def _as_rows(logits: torch.Tensor) -> torch.Tensor | None:
    """``[..., V]`` -> ``[rows, V]`` view sharing storage, or None if not viewable."""
    if logits.dim() == 0 or logits.stride(-1) != 1:
        return None
    try:
        return logits.view(-1, logits.shape[-1])
    except RuntimeError:
        return None


def _check_target(target: torch.Tensor, lead_shape, device: torch.device) -> None:
    """``target`` must be int64 on ``device`` with the token shape ``lead_shape``."""
    if target.device != device:
        raise RuntimeError(f"nmce: target on {target.device}, inputs on {device}")
    if target.dtype != torch.int64:
        raise TypeError(f"nmce: target must be int64, got {target.dtype}")
    if tuple(target.shape) != tuple(lead_shape):
        raise ValueError(
            f"nmce: target shape {tuple(target.shape)} does not match the token shape "
            f"{tuple(lead_shape)} of the inputs")


def _check_inputs(logits: torch.Tensor, target: torch.Tensor, vocab_start: int,
                  vocab_end: int) -> None:
    if not logits.is_cuda:
        raise RuntimeError("nmce: logits must be on a ROCm device (there is no CPU path)")
    _check_target(target, logits.shape[:-1], logits.device)
    _lib.dtype_code(logits.dtype)
    if vocab_end - vocab_start != logits.shape[-1]:
        raise ValueError(
            f"nmce: logits hold {logits.shape[-1]} vocabulary entries but the shard "
            f"[{vocab_start}, {vocab_end}) has {vocab_end - vocab_start}")


# Event queries (about a microsecond each) before the target check falls back
# to a blocking wait.
_CHECK_POLLS = 200


# Pinned count buffers and their events, per device, reused once a check is
# over (allocating them cost a few microseconds per call, which a small batch
# pays every step).
_check_free: dict[int, list] = {}
_check_lock = threading.Lock()


def _check_slot(dev_index: int, slots: int):
    with _check_lock:
        free = _check_free.setdefault(dev_index, [])
        for i, (host, event) in enumerate(free):
            if host.numel() >= slots:
                return free.pop(i)
    cap = 1 << max(slots - 1, 0).bit_length()
    return torch.empty(cap, dtype=torch.int32, pin_memory=True), torch.cuda.Event()


class _PendingCheck:
    """Bad-target counts on their way to pinned host memory.

    The check kernel writes the counts straight into ``host`` (pinned memory
    is mapped into the device's address space at its host address), so the
    buffer must not be reused until ``event`` has completed: every caller ends
    with ``raise_if_bad()`` or, when it leaves early on an exception,
    ``wait()``, which return the buffer and the event to the per-device pool.
    """

    def __init__(self, dev_index: int, host: torch.Tensor, event: torch.cuda.Event, slots: int):
        self.dev_index = dev_index
        self.host = host
        self.event = event
        self.slots = slots
        self.bad = None

    def wait(self) -> None:
        if self.bad is not None:
            return
        # The counts usually reach the host within microseconds of the call:
        # poll first, so that a blocking wait's wake-up latency (tens of
        # microseconds, per step of a small batch) is paid only by long waits.
        event = self.event
        for _ in range(_CHECK_POLLS):
            if event.query():
                break
        else:
            event.synchronize()
        self.bad = bool(self.host.numpy()[:self.slots].any())
        with _check_lock:
            _check_free.setdefault(self.dev_index, []).append((self.host, self.event))

    def raise_if_bad(self) -> None:
        self.wait()
        if self.bad:
            raise ValueError("target token id is outside the model vocabulary")


_side_streams: dict[int, torch.cuda.Stream] = {}


def _side_stream(device: torch.device) -> torch.cuda.Stream:
    """A per-device stream (default priority) for the target check."""
    idx = device.index if device.index is not None else torch.cuda.current_device()
    stream = _side_streams.get(idx)
    if stream is None:
        stream = torch.cuda.Stream(device=idx)
        _side_streams[idx] = stream
    return stream


def launch_target_check(target: torch.Tensor, vocab_size: int) -> _PendingCheck | None:
    """Start the target check of cross_entropy.py:79-81 without blocking.

    One kernel counts targets outside ``[0, vocab_size)`` straight into pinned
    host memory, on a side stream ordered after the work already queued on the
    current stream; ``raise_if_bad()`` on the result waits for that kernel
    alone. The loss kernels go on the current stream meanwhile, so the check
    adds nothing to the loss stream's timeline. (The one-pass path runs its
    check on the loss stream, with a device word its kernel reads, inside the
    C++ call: ``_nmce_autograd.one_pass_mean_checked``.)
    """
    lib = _lib.load()
    t = target.reshape(-1)
    if not t.is_contiguous():
        t = t.contiguous()
    n = t.numel()
    if n == 0:
        return None
    slots = lib.nmce_validate_slots(n)
    dev_index = t.device.index if t.device.index is not None else torch.cuda.current_device()
    host, event = _check_slot(dev_index, slots)
    main = torch.cuda.current_stream(t.device)
    side = _side_stream(t.device)
    side.wait_stream(main)  # the targets are complete in the current stream's order
    with torch.cuda.stream(side):
        _launch("nmce_validate_targets", lib.nmce_validate_targets, t.data_ptr(), n,
                vocab_size, host.data_ptr(), side.cuda_stream)
        event.record(side)
    t.record_stream(side)  # keep the targets' memory until the side stream is done
    return _PendingCheck(dev_index, host, event, slots)


def validate_targets(target: torch.Tensor, vocab_size: int) -> None:
    """Raise ``ValueError`` if any target is outside ``[0, vocab_size)``.

    Same check and message as cross_entropy.py:79-81, as one kernel and one
    small device-to-host read (the reference runs two ``torch.any``
    reductions, each a host sync).
    """
    pending = launch_target_check(target, vocab_size)
    if pending is not None:
        pending.raise_if_bad()


def _exchange_stats(local: torch.Tensor, group, world_size: int) -> torch.Tensor:
    """All-gather the packed ``[3, rows]`` statistics of every TP rank.

    One collective of 12 bytes per token instead of the reference's three
    dependent all-reduces (cross_entropy.py:23, :38, :43). Returns
    ``[world_size, 3, rows]`` in rank order on ``local``'s device. A gloo group
    gets host copies (gloo collectives are only used on CPU tensors here).
    """
    host = dist.get_backend(group) == dist.Backend.GLOO and local.device.type != "cpu"
    src = (local.cpu() if host else local).contiguous()
    # the concatenated output form ([world * 3, rows]) is the one every
    # backend accepts; the stacked view is the same memory
    gathered = torch.empty((world_size * src.shape[0],) + tuple(src.shape[1:]),
                           dtype=src.dtype, device=src.device)
    dist.all_gather_into_tensor(gathered, src, group=group)
    gathered = gathered.view((world_size,) + tuple(src.shape))
    return gathered.to(local.device) if host else gathered


def _resolve_inplace(logits: torch.Tensor, inplace, in_forward: bool = False) -> bool:
    """Whether the gradient goes into the logits' storage. ``inplace=None``:
    for a gradient written by the backward (two-pass path), in place iff the
    logits are a non-leaf tensor; for one written by the forward (one-pass
    path), never, so the logits read the same after the call returns.
    ``inplace=True`` asks for it either way; a leaf that requires grad is
    never overwritten."""
    if inplace is None:
        return (not in_forward) and logits.grad_fn is not None
    if inplace and logits.grad_fn is None and logits.requires_grad:
        raise ValueError("nmce: refusing to write the gradient into a leaf tensor; "
                         "pass inplace=False or None")
    return bool(inplace)


def _ce_forward(ctx, logits, target, vocab_start, vocab_end, group, world_size, inplace):
    """Forward of one shard (cross_entropy.py:17-50): returns the flat per-token
    fp32 loss and leaves on ``ctx`` what the backward needs."""
    _check_inputs(logits, target, vocab_start, vocab_end)
    lib = _lib.load()
    dev = logits.device
    stream = _lib.stream_handle(dev)
    V = logits.shape[-1]

    rows = _as_rows(logits)
    inplace = _resolve_inplace(logits, inplace)
    if rows is None:  # not viewable as [rows, V]: work on a contiguous copy
        rows = logits.contiguous().view(-1, V)
        inplace = False
    n = rows.shape[0]
    ld = rows.stride(0) if n > 1 else V
    tgt = target.reshape(-1)
    if not tgt.is_contiguous():
        tgt = tgt.contiguous()

    dcode = _lib.dtype_code(rows.dtype)
    # out[0] = per-token loss, out[1] = global row max, out[2] = global exp-sum - 1
    out = torch.empty((3, n), dtype=torch.float32, device=dev)
    loss, row_stat = out[0], out[1:]
    if world_size == 1:
        # One shard holds the whole vocabulary: statistics and loss in one pass.
        _launch("nmce_ce_fwd", lib.nmce_ce_fwd, rows.data_ptr(), dcode, n, V, ld,
                tgt.data_ptr(), loss.data_ptr(), row_stat[0].data_ptr(),
                row_stat[1].data_ptr(), stream)
    else:
        local = torch.empty((3, n), dtype=torch.float32, device=dev)
        _launch("nmce_ce_fwd_stats", lib.nmce_ce_fwd_stats, rows.data_ptr(), dcode, n, V, ld,
                tgt.data_ptr(), vocab_start, local[0].data_ptr(), local[1].data_ptr(),
                local[2].data_ptr(), stream)
        stats = _exchange_stats(local, group, world_size)
        _launch("nmce_ce_combine", lib.nmce_ce_combine, stats.data_ptr(),
                stats.data_ptr() + 4 * n, stats.data_ptr() + 8 * n, world_size, 3 * n, n,
                loss.data_ptr(), row_stat[0].data_ptr(), row_stat[1].data_ptr(), stream)

    ctx.inplace = bool(inplace)
    ctx.vocab_start = vocab_start
    ctx.logits_shape = logits.shape
    ctx.ld = ld
    # `rows` aliases `logits` unless a contiguous copy was made above.
    ctx.save_for_backward(rows, tgt, row_stat, logits if ctx.inplace else None)
    return loss


def _one_pass_rows(logits: torch.Tensor, world_size: int) -> torch.Tensor | None:
    """``[rows, V]`` view of ``logits`` when the one-pass kernel takes them:
    TP = 1, V a whole number of 16-byte vectors within the kernel's limit,
    rows 16-byte aligned. Otherwise None."""
    if world_size != 1 or logits.dtype not in (torch.float32, torch.bfloat16):
        return None
    rows = _as_rows(logits)
    if rows is None or rows.shape[0] == 0:
        return None
    es = rows.element_size()
    V = rows.shape[1]
    ld = rows.stride(0) if rows.shape[0] > 1 else V
    if (V * es) % 16 or (ld * es) % 16 or rows.data_ptr() % 16:
        return None
    code = _lib.dtype_code(rows.dtype)
    limit = _one_pass_limit.get(code)
    if limit is None:
        limit = _one_pass_limit[code] = int(_lib.load().nmce_ce_fwd_bwd_max_vocab(code))
    if V > limit:
        return None
    return rows


# The one-pass kernel's widest row per dtype code (a property of the library).
_one_pass_limit: dict[int, int] = {}


def _grad_operand(grad_output):
    """(fp32 tensor, row stride) for the kernels; stride 0 for an expanded
    scalar such as the gradient torch's MeanBackward passes."""
    go = grad_output
    if go.dtype != torch.float32:
        go = go.float()
    if go.numel() > 0 and all(s == 0 for s in go.stride()):
        return go, 0
    go = go.reshape(-1)
    if not go.is_contiguous():
        go = go.contiguous()
    return go, 1


def _ce_backward(ctx, go, gstride, gdiv):
    """Backward of one shard (cross_entropy.py:53-65) with the per-token
    gradient ``go[r * gstride] / gdiv``; returns the logits gradient."""
    rows, tgt, row_stat, original = ctx.saved_tensors
    lib = _lib.load()
    n, V = rows.shape
    if ctx.inplace:
        out = rows
        ld_out = ctx.ld
    else:
        out = torch.empty((n, V), dtype=rows.dtype, device=rows.device)
        ld_out = V
    _launch("nmce_ce_bwd_scaled", lib.nmce_ce_bwd_scaled,
            rows.data_ptr(), out.data_ptr(), _lib.dtype_code(rows.dtype), n, V, ctx.ld, ld_out,
            tgt.data_ptr(), ctx.vocab_start, row_stat[0].data_ptr(), row_stat[1].data_ptr(),
            go.data_ptr(), gstride, gdiv, _lib.stream_handle(rows.device))
    if ctx.inplace:
        # The logits now hold the gradient: make later readers that saved
        # them fail their version check.
        torch.autograd.graph.increment_version(original)
        grad = original.detach()
    else:
        grad = out.view(ctx.logits_shape)
    return grad


class _VocabParallelCrossEntropy(torch.autograd.Function):
    """Per-token loss over a vocabulary shard (cross_entropy.py:16-65).

    ``forward(logits, target, vocab_start, vocab_end, group, world_size,
    inplace=None)`` returns the per-token fp32 loss with ``target``'s shape;
    ``backward`` returns the logits gradient in the logits dtype.
    """

    @staticmethod
    def forward(ctx, logits, target, vocab_start, vocab_end, group, world_size, inplace=None):
        loss = _ce_forward(ctx, logits, target, vocab_start, vocab_end, group, world_size,
                           inplace)
        return loss.view(target.shape)

    @staticmethod
    def backward(ctx, grad_output):
        go, gstride = _grad_operand(grad_output)
        return _ce_backward(ctx, go, gstride, 1.0), None, None, None, None, None, None


class _VocabParallelCrossEntropyMean(torch.autograd.Function):
    """``_VocabParallelCrossEntropy`` followed by ``.mean()`` (cross_entropy.py:85)
    as one node, on the two-pass path: the forward returns the 0-dim mean
    (torch's, on the same per-token values), and the backward hands the scalar
    gradient of the mean straight to the kernel, which divides it by the token
    count per row. That is the same fp32 quotient torch's MeanBackward would
    expand, so the gradient is bit-identical, without MeanBackward's two
    kernels. (The one-pass path's node is ``_nmce_autograd.one_pass_mean``.)
    """

    @staticmethod
    def forward(ctx, logits, target, vocab_start, vocab_end, group, world_size, inplace=None):
        loss = _ce_forward(ctx, logits, target, vocab_start, vocab_end, group, world_size,
                           inplace)
        ctx.n_tokens = loss.numel()
        return loss.mean()

    @staticmethod
    def backward(ctx, grad_output):
        go = grad_output.reshape(1)
        if go.dtype != torch.float32:
            go = go.float()
        gdiv = float(max(ctx.n_tokens, 1))
        return _ce_backward(ctx, go, 0, gdiv), None, None, None, None, None, None


def _one_pass_apply(logits, target, hint, vocab_size, inplace, vocab_start):
    """The one-pass loss at TP = 1 (cross_entropy.py:16-65 and the mean of :85)
    as a C++ autograd node over nmce_ce_fwd_bwd: one read of the logits writes
    the per-token loss, the row statistics and the gradient of the mean for
    the upstream value ``hint`` holds, into the logits' storage when
    ``inplace`` or into a new buffer. Its backward keeps that gradient when its
    upstream value is the assumed one; otherwise it rewrites a separate buffer
    from the logits (bit-identical to the two-pass path) or rescales an
    in-place one, writing the value it received into ``hint``. The buffer is
    handed out once: a second backward through the same graph gets a new
    buffer from the logits, or raises when they hold the gradient. ``target``
    is flat and contiguous. With ``vocab_size`` the target check of
    cross_entropy.py:79-81 runs first on the same stream and leaves a device
    word the kernel reads: on a target outside ``[0, vocab_size)`` the kernel
    writes nothing and the reference's ``ValueError`` is raised once the
    check's count is in; ``None`` skips the check. Returns the 0-dim mean
    loss. Only the wrapper calls it, after checking the inputs."""
    ext = _lib.autograd_ext()
    if vocab_size is None:
        return ext.one_pass_mean(logits, target, hint, None, inplace, vocab_start)
    return ext.one_pass_mean_checked(logits, target, hint, vocab_size, inplace, vocab_start)


def vocab_parallel_cross_entropy(
    logits: torch.Tensor,
    target: torch.Tensor,
    vocab_start: int,
    vocab_end: int,
    ctx,
    *,
    inplace: bool | None = None,
    validate: bool = True,
    one_pass: bool = True,
    upstream_hint: torch.Tensor | None = None,
) -> torch.Tensor:
    """Mean cross-entropy loss from vocab-sharded ``logits`` (cross_entropy.py:68-85).

    ``logits`` is ``[b, s, V/tp]`` (fp32 or bf16); ``target`` is ``[b, s]`` of
    global token ids; ``ctx`` provides ``tp_size`` and ``tp_group``. Returns a
    0-dim fp32 tensor. ``validate=False`` skips the host-synchronising target
    check (the kernels never read out of bounds either way).

    ``inplace=True`` writes the gradient into the logits' storage (the call
    site at model.py:277-281 can: the LM head's output is read by nothing
    else); ``None`` (default) does so only from the two-pass backward, for
    non-leaf logits; ``False`` never does.

    At TP = 1, when a gradient is wanted (grad mode on, logits requiring grad)
    and the rows fit the one-pass kernel (V a whole number of 16-byte vectors,
    at most 131072 bf16 or 65536 fp32 columns, rows 16-byte aligned), the
    forward reads the logits once and also writes their gradient, for the
    upstream value the previous backward of this call site received (1.0 at
    first): in place with ``inplace=True`` (the logits hold the gradient once
    the forward returns), else into a new buffer. The backward redoes it only
    when its upstream value differs: bit-identical to the two-pass path, which
    ``one_pass=False`` selects, for a new buffer; rescaled, within four fp32
    or two bf16 units in the last place, in place. ``upstream_hint`` (a
    one-element fp32 device tensor) replaces the call site's value: the
    forward assumes what it holds and the backward stores what it receives
    there.

    A target outside the vocabulary raises the reference's ``ValueError``
    before this returns, and the logits are left as they were: on the
    one-pass path the check runs on the loss stream and the kernel writes
    nothing when it failed; the two-pass path writes only in its backward.
    On the one-pass path the check, the kernel and the wait for the check's
    count are one call into the C++ module (``_one_pass_apply``).
    """
    _check_inputs(logits, target, vocab_start, vocab_end)
    vocab_size = ctx.tp_size * (vocab_end - vocab_start)
    hint = None
    if (one_pass and torch.is_grad_enabled() and logits.requires_grad
            and _one_pass_rows(logits, ctx.tp_size) is not None):
        if upstream_hint is None:
            caller = sys._getframe(1)
            hint = _site_hint(logits.device, (caller.f_code.co_filename, caller.f_lineno))
        else:
            _check_hint(upstream_hint, logits.device)
            hint = upstream_hint
    if hint is not None:
        tgt = target.reshape(-1)
        if not tgt.is_contiguous():
            tgt = tgt.contiguous()
        return _one_pass_apply(logits, tgt, hint, vocab_size if validate else None,
                               _resolve_inplace(logits, inplace, in_forward=True), vocab_start)
    pending = launch_target_check(target, vocab_size) if validate else None
    # The loss kernels are enqueued before the host waits for the check, so
    # the GPU is busy while the host reads the counts. They never read out of
    # bounds on a bad target; their result is discarded when the check fails.
    try:
        loss = _VocabParallelCrossEntropyMean.apply(
            logits, target, vocab_start, vocab_end, ctx.tp_group, ctx.tp_size, inplace)
    except BaseException:
        if pending is not None:
            pending.wait()
        raise
    if pending is not None:
        pending.raise_if_bad()
    return loss
