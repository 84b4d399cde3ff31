"""Pins the CPU oracle (oracle/) before anything is compared against it.

Checks, each chosen so a plausible mistake fails at least one of them:
* golden vectors from fp64 ``F.cross_entropy`` (tests/golden/make_golden.py),
  including the reference's own check shape [2,5,16] seed 0 at tp in {2,4}
  (nano-megatron tests/check_tp_math.py:94-158) and the c1 workload;
* brute force: per-shard stats + combine on the concatenated slab equal the
  full-vocabulary closed form; shard gradients are column slices of the full
  gradient;
* invariants: shift invariance, full-vocab gradient rows sum to 0, loss >= 0,
  constant rows give log V, V = 1 gives loss 0 and gradient 0;
* -inf logits, including a shard that is -inf across a whole row, against
  fp64 autograd through ``F.cross_entropy``;
* confident tokens (target margins 20 to 80, a tie at the maximum) against
  60-digit decimal arithmetic, to 1e-12 relative on every entry -- which the
  subtraction forms log(sum) and softmax - 1 fail;
* planted mistakes: mutated copies of the oracle (missing target mask,
  off-by-one shard offset, combine without rescale, onehot with the wrong
  sign, a dropped max shift) must fail these checks.
* the fused LM head + loss (``lmhead_closed_form``, ``lmhead_sharded``):
  fp64 autograd through ``F.cross_entropy(hidden @ weight.T)`` with per-token
  weights, the sharded form (tp 2, 4, 5) summing to it, and planted mistakes
  (onehot missing from either gradient, shard offsets dropped) failing.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from _util import assert_close_rel, c1_inputs, load_json, load_npz, sha256_of
from oracle import ce_oracle as O
from oracle import ce_restate as R

# ---------------------------------------------------------------- check bodies


def check_tp_math(sharded=O.sharded, closed=O.closed_form):
    gold = load_npz("tp_math_2x5x16.npz")
    x = gold["logits"].reshape(10, 16)
    t = gold["target"].ravel()
    loss, grad = closed(x, t, 1.0 / 10)
    assert_close_rel(loss, gold["loss"], 1e-12, what="closed-form loss")
    assert_close_rel(loss.mean(), gold["mean"], 1e-12, what="closed-form mean")
    assert_close_rel(grad, gold["grad_mean"], 1e-12, 1e-15, what="closed-form grad")
    for tp in (2, 4):
        l, grads, _, _ = sharded(x, t, tp, 1.0 / 10)
        assert_close_rel(l, gold["loss"], 1e-12, what=f"tp={tp} loss")
        assert_close_rel(np.concatenate(grads, 1), gold["grad_mean"], 1e-12, 1e-15,
                         what=f"tp={tp} grad")


def check_shard_pairs(sharded=O.sharded):
    for name in ("shard_pair_f32.npz", "shard_pair_bf16.npz"):
        gold = load_npz(name)
        l, grads, _, _ = sharded(gold["logits"], gold["target"], int(gold["tp"]))
        assert_close_rel(l, gold["loss"], 1e-12, what=f"{name} loss")
        assert_close_rel(np.concatenate(grads, 1), gold["grad_sum"], 1e-6, 1e-12,
                         what=f"{name} grad")


def check_edge_rows(closed=O.closed_form):
    """The fixture comes from torch's fp64 cross_entropy, which forms
    log_softmax = x - (m + log s): each of its roundings costs up to 2^-53 |m|
    absolute, which on the dominant-logit row (margin 30, loss 5.9e-12) is
    1e-4 of the value. So each row's loss and gradient are compared within
    1e-12 relative plus 2^-50 (1 + |m|) absolute; the confident-row check
    against decimal arithmetic pins those entries to 1e-12 relative."""
    gold = load_npz("edge_rows.npz")
    x = gold["logits"].astype(np.float64)
    l, g = closed(x, gold["target"])
    floor = 2.0 ** -50 * (1.0 + np.abs(x.max(axis=1)))
    assert_close_rel(l, gold["loss"], 1e-12, floor, what="edge loss")
    assert_close_rel(g, gold["grad_sum"], 1e-12, floor[:, None], what="edge grad")


def check_brute_force(sharded=O.sharded, closed=O.closed_form):
    rng = np.random.default_rng(1)
    for tp, (n, v) in ((2, (7, 64)), (4, (5, 128)), (3, (6, 99))):
        x = rng.normal(0, 3, (n, v))
        t = rng.integers(0, v, n)
        t[0], t[-1] = 0, v - 1
        fl, fg = closed(x, t)
        sl, sg, _, _ = sharded(x, t, tp)
        assert_close_rel(sl, fl, 1e-12, 1e-14, what=f"tp={tp} sharded vs closed loss")
        assert_close_rel(np.concatenate(sg, 1), fg, 1e-12, 1e-15, what=f"tp={tp} grad")


def check_neg_inf_shards(sharded=O.sharded, closed=O.closed_form):
    """-inf logits (masked vocabulary entries), including rows where one whole
    shard is -inf: the reference subtracts the all-reduced finite maximum on
    every shard, so such a shard adds exactly 0 to the sum. Against fp64
    autograd through F.cross_entropy and the closed form."""
    rng = np.random.default_rng(5)
    n, v, tp = 9, 12, 3
    x = rng.normal(0, 4, (n, v))
    t = rng.integers(4, v, n)               # targets never in shard 0
    x[rng.random((n, v)) < 0.3] = -np.inf
    x[np.arange(n), t] = rng.normal(0, 4, n)  # targets stay finite
    x[:4, :4] = -np.inf                     # rows 0-3: shard 0 entirely -inf
    xt = torch.from_numpy(x).requires_grad_(True)
    ref = torch.nn.functional.cross_entropy(xt, torch.from_numpy(t), reduction="none")
    ref.sum().backward()
    fl, fg = closed(x, t)
    assert_close_rel(fl, ref.detach().numpy(), 1e-12, 1e-14, what="-inf closed loss")
    assert_close_rel(fg, xt.grad.numpy(), 1e-12, 1e-15, what="-inf closed grad")
    sl, sg, _, _ = sharded(x, t, tp)
    assert_close_rel(sl, fl, 1e-12, 1e-14, what="-inf sharded loss")
    assert_close_rel(np.concatenate(sg, 1), fg, 1e-12, 1e-15, what="-inf sharded grad")


def _decimal_reference(x: np.ndarray, t: np.ndarray):
    """Loss and gradient (g = 1) of each row in 60-digit decimal arithmetic,
    straight from the definitions: loss = ln(sum_j e^(x_j)) - x_t,
    grad_j = e^(x_j) / sum - [j == t]. The fp64 inputs convert exactly."""
    from decimal import Decimal, localcontext
    loss = np.empty(x.shape[0])
    grad = np.empty(x.shape)
    with localcontext() as ctx:
        ctx.prec = 60
        for r in range(x.shape[0]):
            ex = [Decimal(float(v)).exp() for v in x[r]]
            s = sum(ex)
            loss[r] = float(s.ln() - Decimal(float(x[r, t[r]])))
            for j in range(x.shape[1]):
                grad[r, j] = float(ex[j] / s - (1 if j == t[r] else 0))
    return loss, grad


def check_confident_rows(sharded=O.sharded, closed=O.closed_form):
    """Tokens whose target leads by 20 to 80: every other softmax term is below
    fp64's resolution near 1 for the larger margins, so loss = log(sum) and
    softmax_t - 1 are differences that fp64 rounds to 0. Each value must hold
    its relative precision against decimal arithmetic: 1e-12 relative on every
    loss and gradient entry (the non-target entries and the target entry
    alike), for the closed form and the tp = 2 and 3 sharded forms."""
    rng = np.random.default_rng(11)
    n, v = 6, 12
    x = rng.normal(0, 2, (n, v))
    t = np.array([0, 3, 5, 7, 11, 4])
    x[np.arange(n), t] += np.array([20.0, 30.0, 40.0, 45.0, 60.0, 80.0])
    x[5, 9] = x[5, 4]                      # a tie at the maximum with the target
    dl, dg = _decimal_reference(x, t)
    fl, fg = closed(x, t)
    assert_close_rel(fl, dl, 1e-12, what="confident closed loss")
    assert_close_rel(fg, dg, 1e-12, what="confident closed grad")
    for tp in (2, 3):
        sl, sg, _, _ = sharded(x, t, tp)
        assert_close_rel(sl, dl, 1e-12, what=f"confident tp={tp} loss")
        assert_close_rel(np.concatenate(sg, 1), dg, 1e-12, what=f"confident tp={tp} grad")


# ------------------------------------------------------------------- the tests


def test_oracle_tp_math_golden():
    check_tp_math()


def test_oracle_shard_pair_golden():
    check_shard_pairs()


def test_oracle_edge_rows_golden():
    check_edge_rows()


def test_oracle_brute_force_sharding():
    check_brute_force()


def test_oracle_neg_inf_shards():
    check_neg_inf_shards()


def test_oracle_confident_rows():
    check_confident_rows()


def test_oracle_c1_golden():
    """The c1 workload (fp32 [4,256,32000] ~ N(0,2^2), seed 0) in full."""
    gold = load_json("c1_digest.json")
    x, t = c1_inputs()
    assert sha256_of(x, t) == gold["sha256_inputs"]
    loss, grad = O.closed_form(x.reshape(1024, 32000).numpy(), t.reshape(-1).numpy(), 1 / 1024)
    assert_close_rel(loss, gold["loss"], 1e-12, what="c1 loss")
    assert_close_rel(loss.mean(), gold["mean"], 1e-12, what="c1 mean")
    got = grad[np.array(gold["grad_rows"]), np.array(gold["grad_cols"])]
    assert_close_rel(got, gold["grad_vals"], 1e-10, 1e-18, what="c1 grad")


def test_oracle_invariants():
    rng = np.random.default_rng(2)
    x = rng.normal(0, 2, (6, 50))
    t = rng.integers(0, 50, 6)
    l, g = O.closed_form(x, t)
    assert (l >= 0).all()
    assert np.allclose(g.sum(1), 0.0, atol=1e-14)
    l2, g2 = O.closed_form(x + rng.normal(0, 10, (6, 1)), t)  # per-row shift
    assert np.allclose(l, l2, rtol=1e-12, atol=1e-12) and np.allclose(g, g2, atol=1e-14)
    lc, _ = O.closed_form(np.full((3, 77), 1.5), np.array([0, 5, 76]))
    assert np.allclose(lc, np.log(77), rtol=1e-14)
    l1, g1 = O.closed_form(np.array([[4.0], [-2.0]]), np.array([0, 0]))
    assert np.all(l1 == 0) and np.all(g1 == 0)
    ld, _ = O.closed_form(np.array([[50.0] + [0.0] * 9]), np.array([0]))
    assert ld[0] < 1e-20


def test_restatement_matches_golden():
    """The torch-CPU op-sequence restatement (the timed CPU baseline) agrees
    with F.cross_entropy fp64 at fp32 accuracy, at TP=1 and as rank 1 of a
    TP=2 pair whose peer partials are fed through the emulated all-reduce."""
    gold = load_npz("tp_math_2x5x16.npz")
    x = torch.from_numpy(gold["logits"])
    t = torch.from_numpy(gold["target"])
    loss, saved = R.forward(x, t, 0, 16)
    assert loss.dtype == torch.float32
    assert_close_rel(loss.numpy().ravel(), gold["loss"], 1e-6, what="restated loss")
    g = R.backward(saved, torch.full((2, 5), 0.1))
    assert_close_rel(g.numpy().reshape(10, 16), gold["grad_mean"], 1e-5, 1e-9,
                     what="restated grad")

    gold = load_npz("shard_pair_bf16.npz")
    full = torch.from_numpy(gold["logits"]).to(torch.bfloat16)
    t = torch.from_numpy(gold["target"])
    mine, peer = full[:, 512:], full[:, :512]
    gmax = torch.maximum(mine.float().max(-1)[0], peer.float().max(-1)[0])
    pick, psum = R.peer_partials(peer, t, 0, 512, gmax)
    hook = R.fixed_peer_all_reduce(peer.float().max(-1)[0], pick, psum)
    loss, saved = R.forward(mine, t, 512, 1024, all_reduce=hook)
    assert_close_rel(loss.numpy(), gold["loss"], 1e-6, what="rank-1 loss")
    g = R.backward(saved, torch.ones(16))
    assert g.dtype == torch.bfloat16
    assert_close_rel(g.float().numpy(), gold["grad_sum"][:, 512:], 2 ** -8, 1e-30,
                     what="rank-1 bf16 grad")


# ------------------------------------------------------------ planted mistakes


def _mut_stats_no_mask(x_shard, target, vocab_start):
    m, s1, _ = O.shard_stats(x_shard, target, vocab_start)
    x = np.asarray(x_shard, dtype=np.float64)
    local = np.clip(np.asarray(target) - vocab_start, 0, x.shape[1] - 1)
    return m, s1, x[np.arange(x.shape[0]), local]  # forgets to zero unowned picks


def _mut_stats_unguarded(x_shard, target, vocab_start):
    x = np.asarray(x_shard, dtype=np.float64)
    n, v = x.shape
    m = x.max(1)
    with np.errstate(invalid="ignore"):
        s1 = np.exp(x - m[:, None]).sum(1) - 1.0  # an all -inf row gives nan
    local = np.asarray(target) - vocab_start
    owned = (local >= 0) & (local < v)
    return m, s1, np.where(owned, x[np.arange(n), np.clip(local, 0, v - 1)], 0.0)


def _mut_stats_offset(x_shard, target, vocab_start):
    return O.shard_stats(x_shard, target, vocab_start + 1)


def _mut_combine_no_rescale(stats):
    M = np.stack([st[0] for st in stats]).max(0)
    S1 = sum(1.0 + st[1] for st in stats) - 1.0  # shard sums added unscaled
    xt = sum(st[2] for st in stats)
    return M, S1, np.log1p(S1) - (xt - M)


def _sharded_with(stats_fn=O.shard_stats, combine_fn=O.combine, grad_fn=O.shard_grad):
    def run(x_full, target, tp, grad_output=None):
        n, vfull = x_full.shape
        per = vfull // tp
        shards = [x_full[:, r * per:(r + 1) * per] for r in range(tp)]
        stats = [stats_fn(sh, target, r * per) for r, sh in enumerate(shards)]
        M, S1, loss = combine_fn(stats)
        grads = [grad_fn(sh, target, r * per, M, S1, grad_output) for r, sh in enumerate(shards)]
        return loss, grads, M, S1
    return run


def _mut_grad_sign(x_shard, target, vocab_start, M, S1, grad_output=None):
    g = O.shard_grad(x_shard, target, vocab_start, M, S1, None)
    local = np.asarray(target) - vocab_start
    owned = (local >= 0) & (local < g.shape[1])
    rows = np.nonzero(owned)[0]
    g[rows, local[rows]] += 2.0  # onehot added instead of subtracted
    go = 1.0 if grad_output is None else np.asarray(grad_output)
    return g * (go if np.ndim(go) == 0 else go[:, None])


def _mut_closed_no_shift(x, target, grad_output=None):
    x = np.asarray(x, dtype=np.float32)  # fp32 with no max shift overflows
    e = np.exp(x)
    s = e.sum(1, dtype=np.float32)
    loss = np.log(s) - x[np.arange(x.shape[0]), target]
    g = e / s[:, None]
    g[np.arange(x.shape[0]), target] -= 1
    go = 1.0 if grad_output is None else grad_output
    return loss.astype(np.float64), g.astype(np.float64) * go


def _mut_closed_subtracting(x, target, grad_output=None):
    x = np.asarray(x, dtype=np.float64)
    rows = np.arange(x.shape[0])
    m = x.max(1)
    e = np.exp(x - m[:, None])
    s = e.sum(1)
    loss = np.log(s) - (x[rows, target] - m)   # log of a sum that rounded to 1
    g = e / s[:, None]
    g[rows, target] -= 1.0                     # softmax - 1 by subtraction
    go = 1.0 if grad_output is None else grad_output
    return loss, g * go


def _mut_grad_subtracting(x_shard, target, vocab_start, M, S1, grad_output=None):
    x = np.asarray(x_shard, dtype=np.float64)
    g = np.exp(x - M[:, None]) / (1.0 + S1)[:, None]
    local = np.asarray(target) - vocab_start
    owned = (local >= 0) & (local < x.shape[1])
    rows = np.nonzero(owned)[0]
    g[rows, local[rows]] -= 1.0
    go = 1.0 if grad_output is None else np.asarray(grad_output)
    return g * (go if np.ndim(go) == 0 else go[:, None])


def test_planted_subtractions_are_caught():
    with pytest.raises(AssertionError):
        check_confident_rows(closed=_mut_closed_subtracting)
    with pytest.raises(AssertionError):
        check_confident_rows(sharded=_sharded_with(grad_fn=_mut_grad_subtracting))


@pytest.mark.parametrize("mutant,check", [
    (_sharded_with(stats_fn=_mut_stats_no_mask), check_tp_math),
    (_sharded_with(stats_fn=_mut_stats_offset), check_shard_pairs),
    (_sharded_with(combine_fn=_mut_combine_no_rescale), check_brute_force),
    (_sharded_with(grad_fn=_mut_grad_sign), check_shard_pairs),
    (_sharded_with(stats_fn=_mut_stats_unguarded), check_neg_inf_shards),
])
def test_planted_mistakes_in_sharding_are_caught(mutant, check):
    with pytest.raises(AssertionError):
        check(sharded=mutant)


def test_planted_dropped_shift_is_caught():
    with np.errstate(over="ignore", invalid="ignore"):
        with pytest.raises(AssertionError):
            check_edge_rows(closed=_mut_closed_no_shift)


# ------------------------------------------------ fused LM head + loss oracle

def _torch_lmhead(X, W, t, g):
    """fp64 autograd of F.cross_entropy(X @ W^T) with per-token weights g."""
    Xt = torch.tensor(X, dtype=torch.float64, requires_grad=True)
    Wt = torch.tensor(W, dtype=torch.float64, requires_grad=True)
    z = Xt @ Wt.T
    per = torch.nn.functional.cross_entropy(z, torch.tensor(t), reduction="none")
    (per * torch.tensor(g)).sum().backward()
    return per.detach().numpy(), Xt.grad.numpy(), Wt.grad.numpy()


def check_lmhead(closed=O.lmhead_closed_form, sharded=O.lmhead_sharded):
    rng = np.random.default_rng(7)
    n, h, v = 24, 12, 40
    X = rng.standard_normal((n, h))
    W = rng.standard_normal((v, h)) * 0.7
    t = rng.integers(0, v, n)
    g = rng.uniform(0.1, 2.0, n)
    tl, tdx, tdw = _torch_lmhead(X, W, t, g)
    loss, dz, dx, dw = closed(X, W, t, g)
    assert_close_rel(loss, tl, 1e-12, 1e-14, what="lmhead loss")
    assert_close_rel(dx, tdx, 1e-10, 1e-14, what="lmhead dhidden")
    assert_close_rel(dw, tdw, 1e-10, 1e-14, what="lmhead dweight")
    for tp in (2, 4, 5):
        sl, parts, sdw = sharded(X, W, t, tp, g)
        assert_close_rel(sl, tl, 1e-12, 1e-14, what=f"lmhead tp={tp} loss")
        assert_close_rel(sum(parts), tdx, 1e-10, 1e-14, what=f"lmhead tp={tp} dhidden")
        assert_close_rel(sdw, tdw, 1e-10, 1e-14, what=f"lmhead tp={tp} dweight")


def test_oracle_lmhead_against_autograd():
    check_lmhead()


def _lmhead_hidden_grad_without_onehot(hidden, weight, target, grad_output=None):
    loss, dz, dx, dw = O.lmhead_closed_form(hidden, weight, target, grad_output)
    W = np.asarray(weight, dtype=np.float64)
    n = dz.shape[0]
    g = np.ones(n) if grad_output is None else np.broadcast_to(grad_output, (n,))
    # mistake: dhidden from the softmax alone (the target row of W not subtracted)
    return loss, dz, dx + g[:, None] * W[target], dw


def _lmhead_weight_grad_without_onehot(hidden, weight, target, grad_output=None):
    loss, dz, dx, dw = O.lmhead_closed_form(hidden, weight, target, grad_output)
    X = np.asarray(hidden, dtype=np.float64)
    p = dz.copy()
    n = p.shape[0]
    g = np.ones(n) if grad_output is None else np.broadcast_to(grad_output, (n,))
    p[np.arange(n), target] += g  # mistake: the onehot is not subtracted in dW
    return loss, dz, dx, p.T @ X


def _lmhead_shard_offset_dropped(hidden, weight, target, tp, grad_output=None):
    X = np.asarray(hidden, dtype=np.float64)
    W = np.asarray(weight, dtype=np.float64)
    per = W.shape[0] // tp
    zs = [X @ W[r * per:(r + 1) * per].T for r in range(tp)]
    stats = [O.shard_stats(zs[r], target, 0) for r in range(tp)]  # mistake: offset 0
    M, S, loss = O.combine(stats)
    parts = [O.shard_grad(zs[r], target, 0, M, S, grad_output) @ W[r * per:(r + 1) * per]
             for r in range(tp)]
    dws = [O.shard_grad(zs[r], target, 0, M, S, grad_output).T @ X for r in range(tp)]
    return loss, parts, np.concatenate(dws)


@pytest.mark.parametrize("closed,sharded", [
    (_lmhead_hidden_grad_without_onehot, O.lmhead_sharded),
    (_lmhead_weight_grad_without_onehot, O.lmhead_sharded),
    (O.lmhead_closed_form, _lmhead_shard_offset_dropped),
])
def test_planted_lmhead_mistakes_are_caught(closed, sharded):
    with pytest.raises(AssertionError):
        check_lmhead(closed, sharded)

