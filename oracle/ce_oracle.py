"""numpy fp64 oracle of the vocabulary-parallel cross entropy.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

Follows nano_megatron/cross_entropy.py:

* ``shard_stats``  -- one rank's forward reductions (:21 max, :28-36 masked
  target pick, :40-41 exp-sum), before any all-reduce.
* ``combine``      -- what the three all-reduces and :45 produce from the
  per-rank values (MAX of maxima, SUM of target picks, SUM of rescaled
  exp-sums; ``loss = log(sum) - (x_t - max)``). Exp-sums are carried minus
  the maximum's own 1 and the loss is ``log1p(sum - 1)``, so a confident
  token's loss and target gradient keep their relative precision.
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
* -inf logits, with a shard that is -inf across a whole row, against fp64
  autograd through ``F.cross_entropy``;
* confident tokens (margins 20 to 80, a tie at the maximum) against 60-digit
  decimal arithmetic, 1e-12 relative on every loss and gradient entry;
* planted mistakes (dropped max shift, missing mask, off-by-one offset, wrong
  sign, an all -inf shard's sum left unguarded, log(sum) and softmax - 1 by
  subtraction) fail at least one of the above.

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


def _sum_without(e: np.ndarray, cols: np.ndarray) -> np.ndarray:
    """Row sums of ``e`` with the term at ``cols[r]`` left out of row r."""
    em = e.copy()
    em[np.arange(e.shape[0]), cols] = 0.0
    return em.sum(axis=1)


def closed_form(x: np.ndarray, target: np.ndarray, grad_output=None):
    """Full-vocabulary loss and gradient in fp64.

    ``x``: [N, V] logits (any float dtype; upcast to fp64), ``target``: [N] ids.
    Returns ``(loss[N], grad[N, V])`` with ``grad = (softmax - onehot) * g``;
    ``grad_output`` is a scalar or [N] (default 1).

    The two differences from 1 are formed as sums of the remaining terms, not
    by subtraction: ``log(s) = log1p(s - 1)`` with ``s - 1`` the sum without
    the maximum's own term (exactly 1), and ``softmax_t - 1 = -(s - e_t) / s``
    with ``s - e_t`` the sum without the target's term. For a confident token
    every other term lies below fp64's resolution near 1, where ``log(s)`` and
    ``e_t / s - 1`` would round to 0; these forms keep the relative precision.
    """
    x = np.asarray(x, dtype=np.float64)
    t = np.asarray(target, dtype=np.int64)
    n = x.shape[0]
    rows = np.arange(n)
    m = x.max(axis=1)
    e = np.exp(x - m[:, None])
    s = e.sum(axis=1)
    s_m1 = _sum_without(e, x.argmax(axis=1))
    loss = np.log1p(s_m1) - (x[rows, t] - m)
    g = np.ones(n) if grad_output is None else np.broadcast_to(
        np.asarray(grad_output, dtype=np.float64), (n,))
    grad = e / s[:, None]
    grad[rows, t] = -_sum_without(e, t) / s
    grad *= g[:, None]
    return loss, grad


def shard_stats(x_shard: np.ndarray, target: np.ndarray, vocab_start: int):
    """One rank's local reductions (cross_entropy.py:21, :28-36, :40-41), fp64.

    Returns ``(m, s1, t)``: row max, ``sum exp(x - m) - 1`` (the sum without
    the maximum's own term) and the raw target logit if this shard owns it
    (else 0.0). A row that is -inf across the whole shard has ``s1 = -1`` (an
    empty sum): in the reference every shard subtracts the all-reduced, finite
    maximum first, so such a shard's terms are exp(-inf) = 0.
    """
    x = np.asarray(x_shard, dtype=np.float64)
    n, v = x.shape
    tgt = np.asarray(target, dtype=np.int64)
    m = x.max(axis=1)
    empty = np.isneginf(m)
    e = np.exp(x - np.where(empty, 0.0, m)[:, None])
    s1 = np.where(empty, -1.0, _sum_without(e, x.argmax(axis=1)))
    local = tgt - vocab_start
    owned = (local >= 0) & (local < v)
    t = np.where(owned, x[np.arange(n), np.clip(local, 0, v - 1)], 0.0)
    return m, s1, t


def combine(stats):
    """Merge per-shard ``(m, s1, t)`` triples; returns ``(M, S1, loss)``.

    M = max_k m_k; S1 = sum_k (1 + s1_k) exp(m_k - M) - 1, formed without the
    subtraction (each shard at the maximum adds s1_k + 1, one such 1 is left
    out); loss = log1p(S1) - (sum_k t_k - M). These are the all-reduces of
    cross_entropy.py:23, :38, :43 and the loss of :45 (log(sum) = log1p(S1)).
    """
    ms = np.stack([st[0] for st in stats])
    M = ms.max(axis=0)
    with np.errstate(invalid="ignore"):
        terms = [np.where(st[0] == M, st[1], (1.0 + st[1]) * np.exp(st[0] - M))
                 for st in stats]
    n_top = sum((st[0] == M).astype(np.float64) for st in stats)
    S1 = sum(terms) + (n_top - 1.0)
    xt = sum(st[2] for st in stats)
    return M, S1, np.log1p(S1) - (xt - M)


def shard_grad(x_shard: np.ndarray, target: np.ndarray, vocab_start: int, M, S1,
               grad_output=None):
    """Backward on one shard (cross_entropy.py:53-65) in fp64, from the combined
    ``(M, S1)``. The owned target column's ``softmax - 1`` is formed as
    ``(expm1(x_t - M) - S1) / (1 + S1)``: the same value, without the
    subtraction from 1."""
    x = np.asarray(x_shard, dtype=np.float64)
    n, v = x.shape
    g = np.ones(n) if grad_output is None else np.broadcast_to(
        np.asarray(grad_output, dtype=np.float64), (n,))
    S = 1.0 + S1
    grad = np.exp(x - M[:, None]) / S[:, None]
    local = np.asarray(target, dtype=np.int64) - vocab_start
    owned = (local >= 0) & (local < v)
    rows = np.nonzero(owned)[0]
    d = x[rows, local[rows]] - M[rows]
    grad[rows, local[rows]] = (np.expm1(d) - S1[rows]) / S[rows]
    return grad * g[:, None]


def sharded(x_full: np.ndarray, target: np.ndarray, tp: int, grad_output=None):
    """Brute-force TP emulation: slice the full slab into ``tp`` shards, run
    ``shard_stats`` on each, ``combine``, then ``shard_grad`` per shard.

    Returns ``(loss, [grad_shard_0, ...], M, S1)``.
    """
    n, vfull = x_full.shape
    if vfull % tp:
        raise ValueError(f"{vfull} is not divisible by {tp}")
    per = vfull // tp
    shards = [x_full[:, r * per:(r + 1) * per] for r in range(tp)]
    stats = [shard_stats(sh, target, r * per) for r, sh in enumerate(shards)]
    M, S1, loss = combine(stats)
    grads = [shard_grad(sh, target, r * per, M, S1, grad_output) for r, sh in enumerate(shards)]
    return loss, grads, M, S1


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
    M, S1, loss = combine(stats)
    parts, dws = [], []
    for r in range(tp):
        dz = shard_grad(zs[r], target, r * per, M, S1, g)
        parts.append(dz @ W[r * per:(r + 1) * per])
        dws.append(dz.T @ X)
    return loss, parts, np.concatenate(dws, axis=0)

