"""numpy fp64 oracle of the vocabulary-parallel cross entropy.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Follows nano_megatron/cross_entropy.py:

* ``shard_stats``  -- one rank's forward reductions (:21 max, :28-36 masked
  target pick, :40-41 exp-sum), before any all-reduce.
* ``combine``      -- what the three all-reduces and :45 produce from the
  per-rank values (MAX of maxima, SUM of target picks, SUM of rescaled
  exp-sums; ``loss = log(sum) - (x_t - max)``).
* ``shard_grad``   -- backward (:53-65): softmax minus the one-hot on the
  owning rank, times grad_output.
* ``closed_form``  -- full-vocabulary ``logsumexp(x) - x[t]`` and
  ``(softmax(x) - onehot(t)) * g``.

Pinned by (tests/test_oracle.py):
* golden vectors from ``torch.nn.functional.cross_entropy`` in fp64
  (tests/golden/make_golden.py), including the reference's own check shape
  [2,5,16] seed 0 with tp in {2,4} (tests/check_tp_math.py:94-158);
* brute force: sharded stats + combine == closed form on the concatenated
  full-vocabulary slab; shard grads == column slices of the full grad;
* invariants: shift invariance, full-vocab grad rows sum to 0, loss >= 0,
  constant rows give log V, V = 1 gives 0;
* planted mistakes (dropped max shift, missing mask, off-by-one offset, wrong
  sign) fail at least one of the above.

The fused LM head + loss (nano_megatron/model.py:192 feeding
cross_entropy.py:16-85):

* ``lmhead_closed_form`` -- logits ``z = hidden @ weight^T`` in fp64, then
  ``closed_form`` on them; gradients ``dhidden = dZ @ weight`` and
  ``dweight = dZ^T @ hidden`` (the matmul backward of model.py:192).
* ``lmhead_sharded``     -- the same over a vocabulary-sharded weight: per-rank
  logits, ``shard_stats`` / ``combine`` / ``shard_grad`` on them, each rank's
  weight rows and its partial hidden gradient (summed by the caller, as the
  TP all-reduce of mappings.py:83-94 does).

Pinned by (tests/test_oracle.py): fp64 autograd through
``F.cross_entropy(hidden @ weight.T)`` (loss, both gradients), the sharded
form summing to the full one, and planted mistakes (weight transposed into
the hidden gradient, the onehot dropped from the weight gradient) failing.
"""

from __future__ import annotations

import numpy as np


def closed_form(x: np.ndarray, target: np.ndarray, grad_output=None):
    """Full-vocabulary loss and gradient in fp64.

    ``x``: [N, V] logits (any float dtype; upcast to fp64), ``target``: [N] ids.
    Returns ``(loss[N], grad[N, V])`` with ``grad = (softmax - onehot) * g``;
    ``grad_output`` is a scalar or [N] (default 1).
    """
    x = np.asarray(x, dtype=np.float64)
    t = np.asarray(target, dtype=np.int64)
    n = x.shape[0]
    m = x.max(axis=1)
    e = np.exp(x - m[:, None])
    s = e.sum(axis=1)
    lse = m + np.log(s)
    loss = lse - x[np.arange(n), t]
    g = np.ones(n) if grad_output is None else np.broadcast_to(
        np.asarray(grad_output, dtype=np.float64), (n,))
    grad = e / s[:, None]
    grad[np.arange(n), t] -= 1.0
    grad *= g[:, None]
    return loss, grad


def shard_stats(x_shard: np.ndarray, target: np.ndarray, vocab_start: int):
    """One rank's local reductions (cross_entropy.py:21, :28-36, :40-41), fp64.

    Returns ``(m, s, t)``: row max, ``sum exp(x - m)`` and the raw target
    logit if this shard owns it (else 0.0).
    """
    x = np.asarray(x_shard, dtype=np.float64)
    n, v = x.shape
    tgt = np.asarray(target, dtype=np.int64)
    m = x.max(axis=1)
    s = np.exp(x - m[:, None]).sum(axis=1)
    local = tgt - vocab_start
    owned = (local >= 0) & (local < v)
    t = np.where(owned, x[np.arange(n), np.clip(local, 0, v - 1)], 0.0)
    return m, s, t


def combine(stats):
    """Merge per-shard ``(m, s, t)`` triples; returns ``(M, S, loss)``.

    M = max_k m_k; S = sum_k s_k exp(m_k - M); loss = log S - (sum_k t_k - M)
    (the all-reduces of cross_entropy.py:23, :38, :43 and the loss of :45).
    """
    ms = np.stack([st[0] for st in stats])
    M = ms.max(axis=0)
    S = sum(st[1] * np.exp(st[0] - M) for st in stats)
    xt = sum(st[2] for st in stats)
    return M, S, np.log(S) - (xt - M)


def shard_grad(x_shard: np.ndarray, target: np.ndarray, vocab_start: int, M, S,
               grad_output=None):
    """Backward on one shard (cross_entropy.py:53-65) in fp64."""
    x = np.asarray(x_shard, dtype=np.float64)
    n, v = x.shape
    g = np.ones(n) if grad_output is None else np.broadcast_to(
        np.asarray(grad_output, dtype=np.float64), (n,))
    grad = np.exp(x - M[:, None]) / S[:, None]
    local = np.asarray(target, dtype=np.int64) - vocab_start
    owned = (local >= 0) & (local < v)
    rows = np.nonzero(owned)[0]
    grad[rows, local[rows]] -= 1.0
    return grad * g[:, None]


def sharded(x_full: np.ndarray, target: np.ndarray, tp: int, grad_output=None):
    """Brute-force TP emulation: slice the full slab into ``tp`` shards, run
    ``shard_stats`` on each, ``combine``, then ``shard_grad`` per shard.

    Returns ``(loss, [grad_shard_0, ...], M, S)``.
    """
    n, vfull = x_full.shape
    if vfull % tp:
        raise ValueError(f"{vfull} is not divisible by {tp}")
    per = vfull // tp
    shards = [x_full[:, r * per:(r + 1) * per] for r in range(tp)]
    stats = [shard_stats(sh, target, r * per) for r, sh in enumerate(shards)]
    M, S, loss = combine(stats)
    grads = [shard_grad(sh, target, r * per, M, S, grad_output) for r, sh in enumerate(shards)]
    return loss, grads, M, S


def bf16_round(x: np.ndarray) -> np.ndarray:
    """Round fp32/fp64 values to bf16 (nearest even), returned as fp32."""
    f = np.asarray(x, dtype=np.float32)
    u = f.view(np.uint32).astype(np.uint64)
    nan = np.isnan(f)
    rounded = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    out = rounded.astype(np.uint32).view(np.float32)
    return np.where(nan, np.float32(np.nan), out)


def lmhead_closed_form(hidden: np.ndarray, weight: np.ndarray, target: np.ndarray,
                       grad_output=None):
    """Loss and gradients of ``closed_form(hidden @ weight^T)`` in fp64.

    ``hidden`` [N, H], ``weight`` [V, H] (model.py:192: ``x @ self.weight.t()``),
    ``target`` [N]. Returns ``(loss[N], dz[N, V], dhidden[N, H], dweight[V, H])``
    where ``dz`` is the logit gradient of cross_entropy.py:53-65.
    """
    X = np.asarray(hidden, dtype=np.float64)
    W = np.asarray(weight, dtype=np.float64)
    z = X @ W.T
    loss, dz = closed_form(z, target, grad_output)
    return loss, dz, dz @ W, dz.T @ X


def lmhead_sharded(hidden: np.ndarray, weight: np.ndarray, target: np.ndarray, tp: int,
                   grad_output=None):
    """The fused loss over ``tp`` vocabulary shards of ``weight`` (rows
    ``[r*V/tp, (r+1)*V/tp)`` on rank r, tp_layers.py:98-110), combined the way
    cross_entropy.py:22-45 does. Returns ``(loss[N], dhidden_parts[tp][N, H],
    dweight[V, H])``; the ranks' hidden gradients are partial sums (the TP
    all-reduce of the LM head's input mapping adds them)."""
    X = np.asarray(hidden, dtype=np.float64)
    W = np.asarray(weight, dtype=np.float64)
    v = W.shape[0]
    assert v % tp == 0
    per = v // tp
    n = X.shape[0]
    g = np.full(n, 1.0) if grad_output is None else np.broadcast_to(
        np.asarray(grad_output, dtype=np.float64), (n,))
    zs = [X @ W[r * per:(r + 1) * per].T for r in range(tp)]
    stats = [shard_stats(zs[r], target, r * per) for r in range(tp)]
    M, S, loss = combine(stats)
    parts, dws = [], []
    for r in range(tp):
        dz = shard_grad(zs[r], target, r * per, M, S, g)
        parts.append(dz @ W[r * per:(r + 1) * per])
        dws.append(dz.T @ X)
    return loss, parts, np.concatenate(dws, axis=0)

