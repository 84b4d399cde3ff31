"""GPU parity of the unfused vocabulary-parallel cross entropy (libnmce HIP kernels).

Every test runs the HIP path through the C ABI (directly, or through the
drop-in ``nmce.vocab_parallel_cross_entropy``) and compares it with the fp64
oracle (oracle/ce_oracle.py), the fp64 ``F.cross_entropy`` golden vectors
(tests/golden/), or, at full workload size, a chunked fp64 PyTorch reference
of the same op plus size-independent properties.

Tolerances (stated per test):
* fp32 logits: per-token loss and gradient within 1e-5 relative (plus an
  absolute floor far below the values compared);
* bf16 logits: the reference computes in fp32 on the bf16 values, so the loss
  is held to fp32 accuracy (1e-5 relative, well inside the 2e-2 per-token and
  1e-3 mean bound); bf16 gradients within one bf16 ulp of the rounded exact
  gradient.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from _util import (assert_bf16_close, assert_close_rel, c1_inputs, load_json, load_npz,
                   sha256_of)
from oracle import ce_oracle

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


@pytest.fixture(scope="module", autouse=True)
def _lib():
    assert torch.cuda.is_available(), "GPU tests need a ROCm device"
    from nmce import _lib as L
    lib = L.load()
    print(f"[gpu] libnmce version {lib.nmce_version():#x} on {torch.cuda.get_device_name(0)}",
          flush=True)
    return lib


def nm():
    import nmce
    return nmce


def run_shards(shards: list[torch.Tensor], target: torch.Tensor, grad_output=None,
               grad_dtype_out=None):
    """Run stats on every shard, combine locally, then bwd on every shard,
    all through the C ABI. Returns (loss, g_max, g_sum, [grad per shard])."""
    from nmce import _lib as L
    lib = L.load()
    tp = len(shards)
    n, v = shards[0].shape
    stream = L.stream_handle(torch.device(DEV))
    stats = torch.empty((tp, 3, n), dtype=torch.float32, device=DEV)
    for r, sh in enumerate(shards):
        assert sh.shape == (n, v) and sh.stride(1) == 1
        L.check(lib.nmce_ce_fwd_stats(sh.data_ptr(), L.dtype_code(sh.dtype), n, v, sh.stride(0),
                                      target.data_ptr(), r * v, stats[r, 0].data_ptr(),
                                      stats[r, 1].data_ptr(), stats[r, 2].data_ptr(), stream),
                "stats")
    loss = torch.empty(n, dtype=torch.float32, device=DEV)
    gm = torch.empty(n, dtype=torch.float32, device=DEV)
    gs = torch.empty(n, dtype=torch.float32, device=DEV)
    base = stats.data_ptr()
    L.check(lib.nmce_ce_combine(base, base + 4 * n, base + 8 * n, tp, 3 * n, n,
                                loss.data_ptr(), gm.data_ptr(), gs.data_ptr(), stream), "combine")
    if grad_output is None:
        go = torch.ones(1, dtype=torch.float32, device=DEV)
        gstride = 0
    else:
        go = grad_output.to(DEV, torch.float32).contiguous()
        gstride = 1
    grads = []
    for r, sh in enumerate(shards):
        out = torch.empty((n, v), dtype=sh.dtype, device=DEV)
        L.check(lib.nmce_ce_bwd(sh.data_ptr(), out.data_ptr(), L.dtype_code(sh.dtype), n, v,
                                sh.stride(0), v, target.data_ptr(), r * v, gm.data_ptr(),
                                gs.data_ptr(), go.data_ptr(), gstride, stream), "bwd")
        grads.append(out)
    torch.cuda.synchronize()
    return loss, gm, gs, grads


# --------------------------------------------------------------------------
# golden vectors


def test_tp_math_fixture_tp1_grad_and_sharded_loss():
    """The reference's own check shape (check_tp_math.py:94-158): [2,5,16],
    seed 0; tp=1 through the drop-in, tp in {2,4} through per-shard stats and
    the local combine."""
    gold = load_npz("tp_math_2x5x16.npz")
    logits = torch.from_numpy(gold["logits"]).to(DEV).requires_grad_(True)
    target = torch.from_numpy(gold["target"]).to(DEV)
    loss = nm().vocab_parallel_cross_entropy(logits, target, 0, 16, nm().ParallelContext.single())
    loss.backward()
    assert loss.dtype == torch.float32 and loss.dim() == 0
    assert_close_rel(loss.item(), gold["mean"], 1e-5, what="mean loss")
    assert_close_rel(logits.grad.cpu().numpy().reshape(10, 16), gold["grad_mean"], 1e-5, 1e-9,
                     what="grad")
    x = torch.from_numpy(gold["logits"]).reshape(10, 16).to(DEV)
    t = target.reshape(-1)
    for tp in (2, 4):
        per = 16 // tp
        shards = [x[:, r * per:(r + 1) * per] for r in range(tp)]
        l, _, _, grads = run_shards(shards, t)
        assert_close_rel(l.cpu().numpy(), gold["loss"], 1e-5, what=f"tp={tp} loss")
        g = torch.cat(grads, 1).cpu().numpy() / 10.0
        assert_close_rel(g, gold["grad_mean"], 1e-5, 1e-9, what=f"tp={tp} grad")


@pytest.mark.parametrize("name", ["shard_pair_f32.npz", "shard_pair_bf16.npz"])
def test_shard_pair_fixture(name):
    """Two TP=2 shards of a [16,1024] slab (targets at 0, 511, 512, 1023),
    combined locally, against F.cross_entropy in fp64."""
    gold = load_npz(name)
    dtype = torch.bfloat16 if "bf16" in name else torch.float32
    x = torch.from_numpy(gold["logits"]).to(DEV).to(dtype)
    t = torch.from_numpy(gold["target"]).to(DEV)
    shards = [x[:, :512], x[:, 512:]]
    loss, _, _, grads = run_shards(shards, t)
    assert_close_rel(loss.cpu().numpy(), gold["loss"], 1e-5, what="loss")
    g = torch.cat(grads, 1).float().cpu().numpy()
    if dtype == torch.float32:
        assert_close_rel(g, gold["grad_sum"], 1e-5, 1e-12, what="grad")
    else:
        assert_bf16_close(g, gold["grad_sum"], what="bf16 grad", atol=1e-30)


# fp32's smallest normal: softmax terms below it (exp(-120) on a +-60 row)
# come out of the exponential as 0. That is the only absolute slack the fp32
# checks allow: 2^-126 per entry, and per term of a sum (V * 2^-126 on a
# loss whose sum - 1 is itself near that range).
FP32_TINY = 2.0 ** -126


def test_edge_rows_fixture():
    """Constant rows, a dominant logit, +-60 logits, a -inf entry, targets at
    the first and last column. Against the fixture (torch's fp64
    cross_entropy, whose own rounding is ~1e-15 absolute) with that floor, and
    against the oracle on the same values to 1e-5 relative alone: the dominant
    logit's loss (5.9e-12) and target gradient keep their relative precision."""
    gold = load_npz("edge_rows.npz")
    x = torch.from_numpy(gold["logits"]).to(DEV)
    t = torch.from_numpy(gold["target"]).to(DEV)
    loss, _, _, grads = run_shards([x], t)
    got_l, got_g = loss.cpu().numpy(), grads[0].cpu().numpy()
    assert_close_rel(got_l, gold["loss"], 1e-5, 1e-14, what="loss vs fixture")
    assert_close_rel(got_g, gold["grad_sum"], 1e-5, 1e-14, what="grad vs fixture")
    ol, og = ce_oracle.closed_form(gold["logits"], gold["target"])
    assert_close_rel(got_l, ol, 1e-5, FP32_TINY, what="loss vs oracle")
    assert_close_rel(got_g, og, 1e-5, FP32_TINY, what="grad vs oracle")


@pytest.mark.parametrize("tp", [1, 2, 3])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_confident_tokens(dtype, tp):
    """Tokens whose target leads the row by 5 to 80 (rows of width 3 * 16768,
    logits ~ N(0, 2^2)), with a tie at the maximum on one row and the target
    below the maximum on another. fp32 rows: loss and every gradient entry
    within 1e-5 relative of the oracle -- for the larger margins the loss and
    the target's gradient are below 1e-10 and exist only through the
    (max, sum - 1) statistics -- plus V * 2^-126 times |g| for the terms under
    fp32's normal range (at margin 80 the loss is 7e-34, and those terms
    matter). bf16 rows: the bf16 gradient within one ulp, the loss and the
    target column within the derived bound on their sum - 1."""
    from test_sweep_gpu import bf16_fold_bound, bf16_fold_floor
    n, v = 12, 3 * 16768
    per = v // tp
    g = torch.Generator().manual_seed(123)
    x = torch.randn(n, v, generator=g) * 2.0
    t = torch.randint(0, v, (n,), generator=g)
    margins = torch.tensor([5.0, 10, 15, 20, 25, 30, 40, 50, 60, 80, 0, -3])
    x[torch.arange(n), t] = x.max(1).values + margins
    x[10, (t[10] + 7) % v] = x[10, t[10]]            # tie with the target
    x = x.to(dtype)
    xd = x.to(DEV)
    shards = [xd[:, r * per:(r + 1) * per] for r in range(tp)]
    go = torch.rand(n, generator=g) + 0.5
    loss, _, _, grads = run_shards(shards, t.to(DEV), grad_output=go)
    ol, og, _, _ = ce_oracle.sharded(x.double().numpy(), t.numpy(), tp, go.double().numpy())
    got_l = loss.cpu().numpy()
    if dtype == torch.float32:
        flush = v * FP32_TINY
        assert_close_rel(got_l, ol, 1e-5, flush, what="confident loss")
        for r in range(tp):
            assert_close_rel(grads[r].cpu().numpy(), og[r], 1e-5, flush * float(go.max()),
                             what=f"confident grad shard {r}")
    else:
        assert_close_rel(got_l, ol, 1e-5, bf16_fold_bound(per), what="confident bf16 loss")
        floor = bf16_fold_floor(n, v, tp, t.numpy(), go.double().numpy())
        for r in range(tp):
            assert_bf16_close(grads[r].double().cpu().numpy(), og[r],
                              what=f"confident bf16 grad shard {r}",
                              atol=FP32_TINY * float(go.max()) + floor[:, r * per:(r + 1) * per])


def test_c1_golden_through_dropin():
    """c1: fp32 [4,256,32000] ~ N(0,2^2), seed 0 -- the CPU reference config --
    on the GPU through the drop-in, against F.cross_entropy fp64 vectors."""
    gold = load_json("c1_digest.json")
    logits_cpu, target_cpu = c1_inputs()
    assert sha256_of(logits_cpu, target_cpu) == gold["sha256_inputs"], "c1 input generator drifted"
    logits = logits_cpu.to(DEV).requires_grad_(True)
    target = target_cpu.to(DEV)
    import nmce
    per_token = nmce._VocabParallelCrossEntropy.apply(logits, target, 0, 32000, None, 1)
    assert_close_rel(per_token.detach().cpu().numpy().ravel(), gold["loss"], 1e-5,
                     what="c1 per-token loss")
    mean = per_token.mean()
    assert_close_rel(mean.item(), gold["mean"], 1e-6, what="c1 mean")
    mean.backward()
    g = logits.grad.reshape(1024, 32000)
    rows = torch.tensor(gold["grad_rows"], device=DEV)
    cols = torch.tensor(gold["grad_cols"], device=DEV)
    # grads are O(1/1024 * p); atol 1e-13 is far below every sampled value
    assert_close_rel(g[rows, cols].cpu().numpy(), gold["grad_vals"], 1e-5, 1e-13, what="c1 grad")
    # logits were a leaf: never overwritten
    assert torch.equal(logits.detach().cpu(), logits_cpu)


# --------------------------------------------------------------------------
# oracle on seeded inputs: shapes, alignment, strides, grad_output


def _oracle_check(x: torch.Tensor, t: torch.Tensor, tp: int, go=None, what=""):
    """HIP over tp shards vs ce_oracle.sharded on the same values."""
    n, vfull = x.shape
    per = vfull // tp
    shards = [x[:, r * per:(r + 1) * per] for r in range(tp)]
    loss, gm, gs, grads = run_shards(shards, t, grad_output=go)
    xv = x.float().cpu().numpy()
    tv = t.cpu().numpy()
    gov = None if go is None else go.cpu().numpy()
    ol, og, oM, oS1 = ce_oracle.sharded(xv, tv, tp, gov)
    # fp32 rows keep their sum - 1 to relative precision, so the loss is held
    # to 1e-5 relative alone; bf16 rows carry up to ~1e-6 absolute in it
    loss_atol = 1e-30 if x.dtype == torch.float32 else 1e-6
    assert_close_rel(loss.cpu().numpy(), ol, 1e-5, loss_atol, what=f"{what} loss")
    assert_close_rel(gm.cpu().numpy(), oM, 0, 0, what=f"{what} row max")
    # the exp-sum is carried minus one: relative to itself for fp32 rows,
    # relative to the whole sum for bf16 rows (their lanes round with the 1 in)
    if x.dtype == torch.float32:
        assert_close_rel(gs.cpu().numpy(), oS1, 1e-5, what=f"{what} row sumexp - 1")
    else:
        assert_close_rel(gs.cpu().numpy(), oS1, 0.0, 1e-5 * (1.0 + oS1),
                         what=f"{what} row sumexp - 1")
    for r in range(tp):
        got = grads[r].float().cpu().numpy()
        if x.dtype == torch.float32:
            assert_close_rel(got, og[r], 1e-5, 1e-12, what=f"{what} grad shard {r}")
        else:
            assert_bf16_close(got, og[r], what=f"{what} bf16 grad shard {r}", atol=1e-30)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("n,vfull,tp", [(3, 1, 1), (5, 7, 1), (4, 1001, 1), (64, 4096, 2),
                                        (33, 2 * 3001, 2), (8, 4 * 8192, 4), (2, 50304, 1)])
def test_oracle_shapes(dtype, n, vfull, tp):
    """Ragged widths (V=1, 7, 1001, 3001: heads and tails off the 16-byte
    grid), several shards, targets drawn over the full vocabulary."""
    g = torch.Generator().manual_seed(n * 131 + vfull + tp)
    x = (torch.randn(n, vfull, generator=g) * 1.5).to(dtype)
    t = torch.randint(0, vfull, (n,), generator=g)
    _oracle_check(x.to(DEV), t.to(DEV), tp, what=f"{dtype} n={n} V={vfull} tp={tp}")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_unaligned_and_strided_rows(dtype):
    """Rows that start off a 16-byte boundary and a leading dimension larger
    than the shard width (a column slice of a wider buffer)."""
    g = torch.Generator().manual_seed(5)
    big = (torch.randn(37, 2053, generator=g) * 2.0).to(dtype).to(DEV)
    for c0, width in ((1, 2000), (3, 2048), (0, 2053), (5, 17)):
        x = big[:, c0:c0 + width]
        t = torch.randint(0, width, (37,), generator=g).to(DEV)
        _oracle_check(x, t, 1, what=f"{dtype} slice [{c0}:{c0 + width}]")


def test_grad_output_vector_and_signs():
    """Per-token grad_output (mixed sign, zero) instead of the uniform mean."""
    g = torch.Generator().manual_seed(11)
    x = torch.randn(16, 3000, generator=g).to(DEV)
    t = torch.randint(0, 3000, (16,), generator=g).to(DEV)
    go = torch.randn(16, generator=g)
    go[3] = 0.0
    _oracle_check(x, t, 1, go=go, what="fp32 grad_output vector")
    _oracle_check(x, t, 2, go=go, what="fp32 grad_output vector tp=2")


def test_nan_propagates():
    """NaN logits give NaN loss for that row only (the reference has no checks)."""
    x = torch.randn(4, 512, device=DEV)
    x[2, 100] = float("nan")
    t = torch.tensor([0, 1, 2, 3], device=DEV)
    loss, _, _, _ = run_shards([x], t)
    ln = loss.cpu()
    assert torch.isnan(ln[2]) and torch.isfinite(ln[[0, 1, 3]]).all()


def test_misaligned_grad_buffer_uses_scalar_path():
    """grad buffer whose rows sit at a different 16-byte phase than the logits."""
    from nmce import _lib as L
    lib = L.load()
    n, v = 9, 1003
    x = torch.randn(n, v, device=DEV)
    t = torch.randint(0, v, (n,), device=DEV)
    _, gm, gs, grads = run_shards([x], t)
    buf = torch.zeros(n * v + 1, device=DEV)
    out = buf[1:].view(n, v)
    one = torch.ones(1, device=DEV)
    L.check(lib.nmce_ce_bwd(x.data_ptr(), out.data_ptr(), 0, n, v, v, v, t.data_ptr(), 0,
                            gm.data_ptr(), gs.data_ptr(), one.data_ptr(), 0,
                            L.stream_handle(torch.device(DEV))), "bwd")
    torch.cuda.synchronize()
    assert torch.equal(out, grads[0])


# --------------------------------------------------------------------------
# drop-in semantics


def test_inplace_on_nonleaf_logits_with_lm_head():
    """Behind an LM-head matmul (model.py:185-192,277-281) the gradient is
    written into the logits storage and dH, dW match an fp64 reference."""
    import nmce
    g = torch.Generator().manual_seed(3)
    h = torch.randn(2, 64, 96, generator=g).to(DEV).requires_grad_(True)
    w = (torch.randn(1000, 96, generator=g) * 0.05).to(DEV).requires_grad_(True)
    t = torch.randint(0, 1000, (2, 64), generator=g).to(DEV)
    logits = h @ w.t()
    storage = logits.data_ptr()
    loss = nmce.vocab_parallel_cross_entropy(logits, t, 0, 1000, nmce.ParallelContext.single(),
                                             inplace=True)
    loss.backward()
    assert logits.data_ptr() == storage
    h64 = h.detach().double().requires_grad_(True)
    w64 = w.detach().double().requires_grad_(True)
    ref = F.cross_entropy((h64 @ w64.t()).reshape(-1, 1000), t.reshape(-1))
    ref.backward()
    assert_close_rel(loss.item(), ref.item(), 1e-5, what="loss")
    assert_close_rel(h.grad.cpu().numpy(), h64.grad.cpu().numpy(), 1e-4, 1e-7, what="dH")
    assert_close_rel(w.grad.cpu().numpy(), w64.grad.cpu().numpy(), 1e-4, 1e-7, what="dW")
    # the logits storage now holds d loss / d logits: rows sum to zero
    assert torch.allclose(logits.detach().double().sum(-1), torch.zeros(2, 64, device=DEV,
                          dtype=torch.float64), atol=1e-6)


def test_out_of_place_keeps_logits():
    import nmce
    x = torch.randn(8, 300, device=DEV)
    t = torch.randint(0, 300, (8,), device=DEV)
    base = x.clone().requires_grad_(True)
    logits = base * 1.0  # non-leaf
    before = logits.detach().clone()
    nmce.vocab_parallel_cross_entropy(logits, t, 0, 300, nmce.ParallelContext.single(),
                                      inplace=False).backward()
    assert torch.equal(logits.detach(), before)
    ref = F.cross_entropy(x.double(), t)
    xr = x.double().requires_grad_(True)
    F.cross_entropy(xr, t).backward()
    assert_close_rel(base.grad.cpu().numpy(), xr.grad.cpu().numpy(), 1e-5, 1e-12, what="grad")
    assert ref.isfinite()


def test_inplace_bumps_version_counter():
    """An op that saved the logits sees the in-place write as an error."""
    import nmce
    x = torch.randn(4, 64, device=DEV, requires_grad=True)
    logits = x * 2.0
    side = (logits * logits).sum()  # saves `logits`
    loss = nmce.vocab_parallel_cross_entropy(logits, torch.zeros(4, dtype=torch.long, device=DEV),
                                             0, 64, nmce.ParallelContext.single(), inplace=True)
    with pytest.raises(RuntimeError, match="modified by an inplace operation"):
        (loss + side).backward()


def test_out_of_vocabulary_target_raises():
    import nmce
    x = torch.randn(2, 3, 16, device=DEV)
    for bad in (16, -1, 10 ** 9):
        t = torch.zeros(2, 3, dtype=torch.long, device=DEV)
        t[1, 2] = bad
        with pytest.raises(ValueError, match="target token id is outside the model vocabulary"):
            nmce.vocab_parallel_cross_entropy(x, t, 0, 16, nmce.ParallelContext.single())
    # vocab_size = tp * shard width: ids in another rank's shard are valid
    ctx = nmce.ParallelContext(rank=1, world_size=2, tp_size=2, tp_rank=1, pp_size=1, pp_rank=0,
                               dp_size=1, dp_rank=0)
    t = torch.full((2, 3), 20, dtype=torch.long, device=DEV)
    nmce.validate_targets(t, ctx.tp_size * 16)


def test_target_check_waits_when_the_loss_raises(monkeypatch):
    """The check kernel writes its counts straight into a pinned host buffer,
    so a loss call that leaves on an exception must still wait for it before
    the buffer can go back to the allocator; both wrappers do for the checks
    they launch from Python (the two-pass and the fused path). The one-pass
    path's check runs inside its C++ call, whose guard waits on every way out
    (test_bad_target_leaves_in_place_logits_intact reuses its slots)."""
    import nmce
    from nmce import cross_entropy as ce
    from nmce import lmhead as lm
    waited = []
    real_wait = ce._PendingCheck.wait

    def wait(self):
        waited.append(self)
        real_wait(self)

    monkeypatch.setattr(ce._PendingCheck, "wait", wait)

    def boom(*args, **kwargs):
        raise RuntimeError("planted")

    ctx = nmce.ParallelContext.single()
    t = torch.zeros(2, 3, dtype=torch.long, device=DEV)
    for one_pass in (True, False):
        x = torch.randn(2, 3, 16, device=DEV, requires_grad=True)
        monkeypatch.setattr(ce._VocabParallelCrossEntropyMean, "apply", boom)
        monkeypatch.setattr(ce, "_one_pass_apply", boom)
        with pytest.raises(RuntimeError, match="planted"):
            nmce.vocab_parallel_cross_entropy(x * 1.0, t, 0, 16, ctx, one_pass=one_pass)
        monkeypatch.undo()
        monkeypatch.setattr(ce._PendingCheck, "wait", wait)
    h = torch.randn(6, 64, device=DEV).to(torch.bfloat16).requires_grad_(True)
    w = torch.randn(16, 64, device=DEV).to(torch.bfloat16).requires_grad_(True)
    monkeypatch.setattr(lm._LMHeadVocabParallelCrossEntropyMean, "apply", boom)
    with pytest.raises(RuntimeError, match="planted"):
        nmce.lmhead_vocab_parallel_cross_entropy(h, w, t.reshape(-1), 0, 16, ctx)
    assert len(waited) == 2
    assert all(p.event.query() for p in waited)
    # and the normal path still raises on a bad target after the direct write
    monkeypatch.undo()
    bad = t.clone()
    bad[0, 1] = 16
    with pytest.raises(ValueError, match="target token id is outside the model vocabulary"):
        nmce.vocab_parallel_cross_entropy(torch.randn(2, 3, 16, device=DEV), bad, 0, 16, ctx)


def test_bf16_dropin_returns_bf16_grad_and_fp32_loss():
    """bf16 logits -> fp32 loss (test_recompute.py:72-75), bf16 grad."""
    import nmce
    x = torch.randn(2, 8, 256, device=DEV).to(torch.bfloat16).requires_grad_(True)
    t = torch.randint(0, 256, (2, 8), device=DEV)
    loss = nmce.vocab_parallel_cross_entropy(x, t, 0, 256, nmce.ParallelContext.single())
    assert loss.dtype == torch.float32
    loss.backward()
    assert x.grad.dtype == torch.bfloat16
    _, og = ce_oracle.closed_form(x.detach().float().cpu().numpy().reshape(16, 256),
                                  t.cpu().numpy().ravel(), 1.0 / 16)
    assert_bf16_close(x.grad.float().cpu().numpy().reshape(16, 256), og, what="bf16 grad",
                      atol=1e-30)


# --------------------------------------------------------------------------
# full workload sizes


def _torch_ref_rows(x: torch.Tensor, t: torch.Tensor, chunk: int = 1024):
    """fp64 per-token loss (logsumexp - x_t) computed on the GPU chunk by chunk."""
    out = []
    for a in range(0, x.shape[0], chunk):
        xc = x[a:a + chunk].double()
        out.append(torch.logsumexp(xc, -1) - xc.gather(1, t[a:a + chunk, None]).squeeze(1))
    return torch.cat(out)


def test_c2_full_size_bf16():
    """c2: bf16 [8,2048,50304] ~ N(0,1), TP=1, in-place bf16 grad. Loss vs a
    chunked fp64 reference, grads vs the fp64 softmax on sampled rows,
    size-independent properties on every row, and the CPU oracle on 32 rows."""
    import nmce
    print("[gpu] c2 bf16 [8,2048,50304]", flush=True)
    gen = torch.Generator(device=DEV).manual_seed(0)
    N, V = 8 * 2048, 50304
    x = torch.randn(N, V, device=DEV, generator=gen).to(torch.bfloat16)
    t = torch.randint(0, V, (N,), device=DEV, generator=gen)
    ref_loss = _torch_ref_rows(x, t)
    xs = x[::512].clone()  # 32 rows kept for the gradient checks
    ts = t[::512].clone()
    leaf = torch.zeros((), device=DEV, requires_grad=True)
    logits = (x + leaf).view(8, 2048, V)  # non-leaf on the same storage kind
    per_token = nmce._VocabParallelCrossEntropy.apply(logits, t.view(8, 2048), 0, V, None, 1)
    assert_close_rel(per_token.detach().reshape(-1).cpu().numpy(), ref_loss.cpu().numpy(), 1e-5,
                     what="c2 loss")
    mean = per_token.mean()
    assert abs(mean.item() - ref_loss.mean().item()) <= 1e-6 * abs(ref_loss.mean().item())
    del x
    mean.backward()
    grad = logits.detach().view(N, V)  # in place: logits now hold the gradient
    # every row of the full-vocab gradient sums to 0 (softmax sums to 1)
    rs = grad.float().sum(-1) * N
    assert rs.abs().max().item() < 2e-2, rs.abs().max().item()
    _, og = ce_oracle.closed_form(xs.float().cpu().numpy(), ts.cpu().numpy(), 1.0 / N)
    assert_bf16_close(grad[::512].float().cpu().numpy(), og, what="c2 grad rows", atol=1e-30)


def test_c3_shard_pair_local_combine():
    """c3: one TP=2 rank's shard bf16 [4,4096,64128] at offset 64128, N(0,1.5^2),
    targets over [0,128256) (about half masked); rank 0's shard generated from
    the same stream and combined locally."""
    print("[gpu] c3 bf16 2 x [16384,64128]", flush=True)
    gen = torch.Generator(device=DEV).manual_seed(0)
    N, V = 4 * 4096, 64128
    full = (torch.randn(N, 2 * V, device=DEV, generator=gen) * 1.5).to(torch.bfloat16)
    t = torch.randint(0, 2 * V, (N,), device=DEV, generator=gen)
    owned = ((t >= V).float().mean().item())
    assert 0.45 < owned < 0.55
    ref_loss = _torch_ref_rows(full, t)
    shards = [full[:, :V].contiguous(), full[:, V:].contiguous()]
    xs = full[::1024].float().cpu().numpy()
    ts = t[::1024].cpu().numpy()
    del full
    loss, _, _, grads = run_shards(shards, t, grad_output=torch.full((N,), 1.0 / N))
    assert_close_rel(loss.cpu().numpy(), ref_loss.cpu().numpy(), 1e-5, what="c3 loss")
    _, og = ce_oracle.closed_form(xs, ts, 1.0 / N)
    got = torch.cat([grads[0][::1024], grads[1][::1024]], 1).float().cpu().numpy()
    assert_bf16_close(got, og, what="c3 grads", atol=1e-30)


# --------------------------------------------------------------------------
# kernel-path equivalences


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_fused_single_shard_forward_equals_stats_plus_combine(dtype):
    """nmce_ce_fwd (TP=1, combine folded in) is bit-identical to
    nmce_ce_fwd_stats + nmce_ce_combine(tp=1)."""
    from nmce import _lib as L
    lib = L.load()
    g = torch.Generator().manual_seed(21)
    n, v = 300, 5003
    x = (torch.randn(n, v, generator=g) * 3.0).to(dtype).to(DEV)
    t = torch.randint(0, v, (n,), generator=g).to(DEV)
    loss, gm, gs, _ = run_shards([x], t)
    out = torch.empty((3, n), device=DEV)
    L.check(lib.nmce_ce_fwd(x.data_ptr(), L.dtype_code(dtype), n, v, v, t.data_ptr(),
                            out[0].data_ptr(), out[1].data_ptr(), out[2].data_ptr(),
                            L.stream_handle(torch.device(DEV))), "fwd")
    torch.cuda.synchronize()
    assert torch.equal(out[0], loss) and torch.equal(out[1], gm) and torch.equal(out[2], gs)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_flat_and_row_backward_agree(dtype):
    """The flat backward (aligned rows, width a multiple of 16 bytes) and the
    row-per-workgroup backward (rows off the 16-byte grid) write identical
    gradients for identical values."""
    from nmce import _lib as L
    lib = L.load()
    g = torch.Generator().manual_seed(22)
    n, v = 129, 4096
    vals = (torch.randn(n, v, generator=g) * 2.0).to(dtype)
    t = torch.randint(0, v, (n,), generator=g).to(DEV)
    aligned = vals.to(DEV)
    big = torch.zeros(n, v + 1, dtype=dtype, device=DEV)
    big[:, 1:] = aligned
    shifted = big[:, 1:]  # same values, rows one element off the grid
    stream = L.stream_handle(torch.device(DEV))
    _, gm, gs, _ = run_shards([aligned], t)
    go = torch.full((1,), 0.37, device=DEV)
    outs = []
    for x in (aligned, shifted):
        o = torch.empty_like(x) if x is aligned else big.clone()[:, 1:]
        L.check(lib.nmce_ce_bwd(x.data_ptr(), o.data_ptr(), L.dtype_code(dtype), n, v,
                                x.stride(0), o.stride(0), t.data_ptr(), 0, gm.data_ptr(),
                                gs.data_ptr(), go.data_ptr(), 0, stream), "bwd")
        outs.append(o)
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1])


def test_validation_overlaps_and_still_raises_before_returning():
    """A bad target raises from the call even though the loss kernels were
    enqueued before the check completed; a good batch right after is fine."""
    import nmce
    x = torch.randn(4, 2048, 1000, device=DEV).to(torch.bfloat16)
    t = torch.randint(0, 1000, (4, 2048), device=DEV)
    t[3, 2047] = 1000
    with pytest.raises(ValueError, match="outside the model vocabulary"):
        nmce.vocab_parallel_cross_entropy(x, t, 0, 1000, nmce.ParallelContext.single())
    t[3, 2047] = 999
    loss = nmce.vocab_parallel_cross_entropy(x, t, 0, 1000, nmce.ParallelContext.single())
    ref = _torch_ref_rows(x.view(-1, 1000), t.view(-1)).mean()
    assert abs(loss.item() - ref.item()) <= 1e-5 * abs(ref.item())


def test_stream_copy_calibration_kernel():
    """nmce_stream_copy copies exactly (it calibrates the byte counters)."""
    from nmce import _lib as L
    lib = L.load()
    src = torch.randint(-2**31, 2**31 - 1, (4 * 1000 + 4,), dtype=torch.int32, device=DEV)
    dst = torch.zeros_like(src)
    L.check(lib.nmce_stream_copy(src.data_ptr(), dst.data_ptr(), src.numel() * 4,
                                 L.stream_handle(torch.device(DEV))), "copy")
    torch.cuda.synchronize()
    assert torch.equal(src, dst)
    assert lib.nmce_stream_copy(src.data_ptr(), dst.data_ptr(), 12, None) == -2


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("inplace", [False, True])
def test_wrapper_mean_backward_is_bit_identical(dtype, inplace):
    """The wrapper folds loss.mean() (cross_entropy.py:85) into the kernel: its
    gradient must equal, bit for bit, the per-token Function followed by
    torch's .mean() and MeanBackward, and its loss must be torch's mean."""
    import nmce
    print(f"[gpu] wrapper mean {dtype} inplace={inplace}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(5)
    b, s, v = 3, 37, 1000
    base = (torch.randn(b, s, v, device=DEV, generator=g) * 3.0).to(dtype)
    t = torch.randint(0, v, (b, s), device=DEV, generator=g)
    ctx = nmce.ParallelContext.single()
    results = []
    for fused_mean in (True, False):
        leaf = base.detach().clone().requires_grad_(True)
        logits = leaf * 1.0 if inplace else leaf
        if fused_mean:
            loss = nmce.vocab_parallel_cross_entropy(logits, t, 0, v, ctx, inplace=inplace)
        else:
            loss = nmce._VocabParallelCrossEntropy.apply(logits, t, 0, v, None, 1,
                                                         inplace).mean()
        (loss * 0.37).backward()
        results.append((loss.detach().clone(), leaf.grad.detach().clone()))
    (l1, g1), (l2, g2) = results
    assert torch.equal(l1, l2), (l1.item(), l2.item())
    assert torch.equal(g1.view(torch.int16) if dtype == torch.bfloat16 else g1,
                       g2.view(torch.int16) if dtype == torch.bfloat16 else g2)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_empty_batch(dtype):
    """Zero tokens, handled as the reference's torch ops handle them: the
    per-token loss is an empty [0, s] tensor, the mean is torch's mean of
    nothing (NaN), and the backward returns an empty gradient of the logits'
    shape and dtype."""
    import nmce
    ctx = nmce.ParallelContext.single()
    x = torch.zeros(0, 16, 1000, dtype=dtype, device=DEV, requires_grad=True)
    t = torch.zeros(0, 16, dtype=torch.int64, device=DEV)
    per_token = nmce._VocabParallelCrossEntropy.apply(x, t, 0, 1000, None, 1)
    assert per_token.shape == (0, 16) and per_token.dtype == torch.float32
    per_token.sum().backward()
    assert x.grad.shape == x.shape and x.grad.dtype == dtype
    x.grad = None
    loss = nmce.vocab_parallel_cross_entropy(x, t, 0, 1000, ctx)
    want = torch.zeros(0, device=DEV).mean()  # torch's mean of an empty tensor
    assert loss.dim() == 0 and torch.isnan(loss) and torch.isnan(want)
    loss.backward()
    assert x.grad.shape == x.shape


def test_slab_at_the_flat_kernel_limit():
    """Maximum sizes: a bf16 slab of 2^21 rows x 8192 (32 GiB, 2^34 elements)
    with its gradient out of place (another 32 GiB). Every row offset past
    2^31 elements is exercised, and the backward's two paths meet at their
    boundary: 2^21 - 1 rows hold 2^31 - 1024 vectors and take the flat kernel
    (it numbers vectors in 32 bits); all 2^21 rows hold 2^31 and take the
    row kernel. On the shared rows the two gradients must be identical, and
    sampled rows -- the first, the last, and those on either side of the
    2^31-element and 2^31-vector offsets -- must match the oracle."""
    from nmce import _lib as L
    lib = L.load()
    free, _ = torch.cuda.mem_get_info()
    if free < 70 * 2 ** 30:
        pytest.skip(f"needs 70 GiB of free device memory, {free / 2 ** 30:.0f} GiB free")
    n, v = 2 ** 21, 8192
    g = torch.Generator(device=DEV).manual_seed(17)
    x = torch.empty((n, v), dtype=torch.bfloat16, device=DEV)
    for a in range(0, n, 2 ** 15):
        x[a:a + 2 ** 15] = torch.randn((2 ** 15, v), generator=g, device=DEV) * 1.5
    t = torch.randint(0, v, (n,), generator=g, device=DEV)
    stream = L.stream_handle(torch.device(DEV))
    code = L.dtype_code(torch.bfloat16)
    out = torch.empty((3, n), dtype=torch.float32, device=DEV)
    L.check(lib.nmce_ce_fwd(x.data_ptr(), code, n, v, v, t.data_ptr(), out[0].data_ptr(),
                            out[1].data_ptr(), out[2].data_ptr(), stream), "fwd")
    one = torch.ones(1, dtype=torch.float32, device=DEV)
    grad = torch.empty_like(x)
    # rows [0, n-1): the flat kernel
    L.check(lib.nmce_ce_bwd(x.data_ptr(), grad.data_ptr(), code, n - 1, v, v, v, t.data_ptr(), 0,
                            out[1].data_ptr(), out[2].data_ptr(), one.data_ptr(), 0, stream),
            "bwd flat")
    torch.cuda.synchronize()
    rows = torch.tensor([0, 1, 2 ** 18 - 1, 2 ** 18, 2 ** 20 + 12345, n - 2], device=DEV)
    flat_rows = grad[rows].clone()
    # all n rows: the row kernel
    L.check(lib.nmce_ce_bwd(x.data_ptr(), grad.data_ptr(), code, n, v, v, v, t.data_ptr(), 0,
                            out[1].data_ptr(), out[2].data_ptr(), one.data_ptr(), 0, stream),
            "bwd rows")
    torch.cuda.synchronize()
    assert torch.equal(flat_rows, grad[rows]), "flat and row kernels differ"
    rows = torch.cat([rows, torch.tensor([n - 1], device=DEV)])
    xs, ts = x[rows].float().cpu().numpy(), t[rows].cpu().numpy()
    ol, og = ce_oracle.closed_form(xs, ts)
    assert_close_rel(out[0][rows].cpu().numpy(), ol, 1e-5, 1e-6, what="loss")
    assert_bf16_close(grad[rows].double().cpu().numpy(), og, what="grad", atol=1e-30)
    del x, grad
    torch.cuda.empty_cache()


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("shape", [(3, 37, 1000), (2, 512, 32000), (1, 64, 50304), (4, 8, 8)])
def test_one_pass_is_bit_identical(dtype, shape):
    """The wrapper's one-pass path (TP = 1) against its two-pass path on the same
    values: the loss, and the gradient for the upstream value the forward
    assumed (``loss.backward()``, the buffer kept as written) and for others
    (0.5, 0.37 and 3.0: rewritten from the logits), all bit for bit. Widths of
    1 to 8 vectors per lane and a vocabulary of one vector per row; the logits
    are left as they were."""
    import nmce
    b, s, v = shape
    if v > nmce._lib.load().nmce_ce_fwd_bwd_max_vocab(nmce._lib.dtype_code(dtype)):
        pytest.skip("wider than the one-pass kernel")
    print(f"[gpu] one-pass {dtype} {shape}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(11)
    base = (torch.randn(b, s, v, device=DEV, generator=g) * 3.0).to(dtype)
    t = torch.randint(0, v, (b, s), device=DEV, generator=g)
    ctx = nmce.ParallelContext.single()
    for upstream in (1.0, 0.5, 0.37, 3.0):
        out = []
        for one_pass in (True, False):
            leaf = base.detach().clone().requires_grad_(True)
            logits = leaf * 1.0
            before = logits.detach().clone()
            loss = nmce.vocab_parallel_cross_entropy(logits, t, 0, v, ctx, inplace=False,
                                                     one_pass=one_pass)
            (loss * upstream).backward()
            assert torch.equal(logits.detach(), before), "the logits were modified"
            out.append((loss.detach(), leaf.grad.detach()))
        (l1, g1), (l2, g2) = out
        assert torch.equal(l1, l2), (upstream, l1.item(), l2.item())
        if dtype == torch.bfloat16:
            g1, g2 = g1.view(torch.int16), g2.view(torch.int16)
        assert torch.equal(g1, g2), f"gradient differs at upstream {upstream}"


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_one_pass_slot_boundaries(dtype):
    """The one-pass kernel (a 1024-lane workgroup per row, vector slot k of lane
    t at vector t + 1024 k) at widths on and next to every slot boundary it
    handles in registers: one vector, a slot short of, at and past a full
    slot, the 4- and 8-slot instantiations' edges, and seeded widths between.
    Odd row counts, 37 and 513 rows. Loss and gradient bit-identical to the
    two-pass path at upstream values 1.0 (the gradient the forward wrote) and
    0.5 (rescaled), the logits left as they were."""
    import nmce
    epv = 16 // torch.tensor([], dtype=dtype).element_size()
    slot = 1024 * epv
    widths = [epv, slot - epv, slot, slot + epv, 2 * slot + 7 * epv, 4 * slot - epv, 4 * slot,
              4 * slot + epv, 8 * slot - epv, 8 * slot]
    rng = np.random.default_rng(29)
    widths += [int(w) * epv for w in rng.integers(1, 8 * 1024, size=4)]
    ctx = nmce.ParallelContext.single()
    for v in widths:
        for n in (37, 513):
            print(f"[gpu] one-pass slots {dtype} n={n} v={v}", flush=True)
            g = torch.Generator(device=DEV).manual_seed(v + n)
            base = (torch.randn(n, v, device=DEV, generator=g) * 2.5).to(dtype)
            t = torch.randint(0, v, (n,), device=DEV, generator=g)
            for upstream in (1.0, 0.5):
                out = []
                for one_pass in (True, False):
                    leaf = base.detach().clone().requires_grad_(True)
                    logits = leaf * 1.0
                    before = logits.detach().clone()
                    loss = nmce.vocab_parallel_cross_entropy(logits, t, 0, v, ctx, inplace=False,
                                                             one_pass=one_pass)
                    (loss * upstream).backward()
                    assert torch.equal(logits.detach(), before), "the logits were modified"
                    out.append((loss.detach(), leaf.grad.detach()))
                (l1, g1), (l2, g2) = out
                assert torch.equal(l1, l2), (v, n, upstream, l1.item(), l2.item())
                if dtype == torch.bfloat16:
                    g1, g2 = g1.view(torch.int16), g2.view(torch.int16)
                assert torch.equal(g1, g2), f"gradient differs at v={v} n={n} upstream {upstream}"


def test_one_pass_falls_back():
    """Rows the one-pass kernel does not take run the two-pass path with the
    same results: a width that is not a whole number of vectors, a width past
    the kernel's limit, a row stride off the 16-byte grid."""
    import nmce
    ctx = nmce.ParallelContext.single()
    g = torch.Generator(device=DEV).manual_seed(12)
    cases = [torch.randn(4, 1001, device=DEV, generator=g),
             torch.randn(2, 70000, device=DEV, generator=g).to(torch.bfloat16),
             torch.randn(4, 1030, device=DEV, generator=g)[:, :1024]]
    for x in cases:
        t = torch.randint(0, x.shape[1], (x.shape[0],), device=DEV, generator=g)
        grads = []
        for one_pass in (True, False):
            leaf = x.detach().clone().requires_grad_(True)
            nmce.vocab_parallel_cross_entropy(leaf * 1.0, t, 0, x.shape[1], ctx, inplace=False,
                                              one_pass=one_pass).backward()
            grads.append(leaf.grad)
        assert torch.equal(grads[0], grads[1])


class _HitRecorder:
    """Records (assumed, received) upstream values of every one-pass loss's
    backward: the value its forward assumed (saved by the autograd node) and
    the gradient that reaches the loss (a hook, which runs before the node's
    backward). The forward's gradient stands when they are equal."""

    def __init__(self, monkeypatch):
        from nmce import _lib
        from nmce import cross_entropy as ce
        self.calls = []
        original = ce._one_pass_apply
        ext = _lib.autograd_ext()

        def wrapped(*args):
            loss = original(*args)
            loss.register_hook(
                lambda g: self.calls.append((ext.assumed_of(loss).item(), g.item())))
            return loss

        monkeypatch.setattr(ce, "_one_pass_apply", wrapped)


def test_one_pass_follows_the_upstream_value(monkeypatch):
    """The one-pass forward computes the gradient for the upstream value the
    last backward received: a loss scaled by 0.25 every step has its first
    backward rewrite the gradient and record 0.25, after which the forward's
    gradient stands. Both steps are bit-identical to the two-pass path."""
    import nmce
    rec = _HitRecorder(monkeypatch)
    ctx = nmce.ParallelContext.single()
    g = torch.Generator(device=DEV).manual_seed(13)
    x = torch.randn(64, 4096, device=DEV, generator=g).to(torch.bfloat16)
    t = torch.randint(0, 4096, (64,), device=DEV, generator=g)
    hint = torch.ones(1, dtype=torch.float32, device=DEV)
    for step in range(2):
        grads = []
        for one_pass in (True, False):
            leaf = x.clone().requires_grad_(True)
            loss = nmce.vocab_parallel_cross_entropy(leaf * 1.0, t, 0, 4096, ctx, inplace=False,
                                                     one_pass=one_pass, upstream_hint=hint)
            (loss * 0.25).backward()
            grads.append(leaf.grad.view(torch.int16))
        assert torch.equal(grads[0], grads[1]), f"step {step}"
        assert hint.item() == 0.25
    assert rec.calls == [(1.0, 0.25), (0.25, 0.25)]


def _two_sites(nmce, ctx, a, b, t, v):
    """Two losses computed at two call sites (two source lines)."""
    la = nmce.vocab_parallel_cross_entropy(a, t, 0, v, ctx, inplace=False)
    lb = nmce.vocab_parallel_cross_entropy(b, t, 0, v, ctx, inplace=False)
    return la, lb


def test_one_pass_hints_are_per_call_site(monkeypatch):
    """Two losses scaled by 1.0 and 0.1, computed at two call sites and
    differentiated together every step, each keep their own upstream value:
    from the second step on both forwards' gradients stand. Gradients match
    the two-pass path bit for bit on every step."""
    import nmce
    rec = _HitRecorder(monkeypatch)
    ctx = nmce.ParallelContext.single()
    g = torch.Generator(device=DEV).manual_seed(21)
    v = 2048
    x = torch.randn(2, 128, v, device=DEV, generator=g).to(torch.bfloat16)
    t = torch.randint(0, v, (128,), device=DEV, generator=g)
    for step in range(3):
        a = x[0].clone().requires_grad_(True)
        b = x[1].clone().requires_grad_(True)
        la, lb = _two_sites(nmce, ctx, a * 1.0, b * 1.0, t, v)
        (la * 1.0 + lb * 0.1).backward()
        for leaf, scale in ((a, 1.0), (b, 0.1)):
            ref = leaf.detach().clone().requires_grad_(True)
            (nmce.vocab_parallel_cross_entropy(ref * 1.0, t, 0, v, ctx, one_pass=False)
             * scale).backward()
            assert torch.equal(leaf.grad.view(torch.int16), ref.grad.view(torch.int16)), step
    got = sorted(rec.calls[2:])  # steps 2 and 3: both sites hit
    assert len(rec.calls) == 6
    assert all(a == b for a, b in rec.calls[2:]), rec.calls
    assert sorted(set(c[1] for c in got)) == sorted({1.0, np.float32(0.1).item()})


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("shape", [(3, 37, 1000), (2, 512, 32000), (1, 600, 50304), (4, 8, 8)])
def test_one_pass_in_place(dtype, shape):
    """Non-leaf logits at TP = 1 with inplace=True: the one-pass forward writes
    the gradient into the logits' own storage. Upstream 1.0 (the forward's value)
    and 0.5 (a power-of-two rescale) are bit-identical to the two-pass path
    (which writes in place too, in its backward); 0.37 and 3.0 are rescaled
    and within four fp32 / two bf16 units in the last place (the written
    gradient and the ratio are each rounded once)."""
    import nmce
    b, s, v = shape
    if v > nmce._lib.load().nmce_ce_fwd_bwd_max_vocab(nmce._lib.dtype_code(dtype)):
        pytest.skip("wider than the one-pass kernel")
    print(f"[gpu] one-pass in place {dtype} {shape}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(15)
    base = (torch.randn(b, s, v, device=DEV, generator=g) * 3.0).to(dtype)
    t = torch.randint(0, v, (b, s), device=DEV, generator=g)
    ctx = nmce.ParallelContext.single()
    # two bf16 ulps (2^-7 relative at the bottom of a binade) / four fp32 ulps
    ulp = 2.0 ** -6 if dtype == torch.bfloat16 else 2.0 ** -21
    for upstream in (1.0, 0.5, 0.37, 3.0):
        out = []
        for one_pass in (True, False):
            hint = torch.ones(1, dtype=torch.float32, device=DEV)
            anchor = torch.zeros((), device=DEV, requires_grad=True)
            logits = base.clone() + anchor.to(dtype)  # non-leaf, own storage
            storage = logits.data_ptr()
            loss = nmce.vocab_parallel_cross_entropy(logits, t, 0, v, ctx, one_pass=one_pass,
                                                     upstream_hint=hint, inplace=True)
            grads = []
            logits.register_hook(lambda gr: grads.append(gr))
            (loss * upstream).backward()
            assert grads[0].data_ptr() == storage, "the gradient is not in the logits' storage"
            out.append((loss.detach(), grads[0].detach().clone()))
        (l1, g1), (l2, g2) = out
        assert torch.equal(l1, l2), (upstream, l1.item(), l2.item())
        if upstream in (1.0, 0.5):
            a, c = (g1.view(torch.int16), g2.view(torch.int16)) if dtype == torch.bfloat16 \
                else (g1, g2)
            assert torch.equal(a, c), f"gradient differs at upstream {upstream}"
        else:
            err = (g1.double() - g2.double()).abs()
            bound = ulp * g2.double().abs() + 1e-38
            assert bool((err <= bound).all()), f"upstream {upstream}: {err.max().item():.3e}"


def test_one_pass_writes_nothing_without_grad():
    """No gradient wanted, no gradient written: under torch.no_grad(), and for
    logits that do not require grad, the forward allocates no [N, V] buffer
    and leaves non-leaf logits as they were; the loss is the two-pass one."""
    import nmce
    ctx = nmce.ParallelContext.single()
    g = torch.Generator(device=DEV).manual_seed(16)
    n, v = 4096, 32768
    x = torch.randn(n, v, device=DEV, generator=g).to(torch.bfloat16)
    t = torch.randint(0, v, (n,), device=DEV, generator=g)
    slab = n * v * 2
    anchor = torch.zeros((), device=DEV, requires_grad=True)
    logits = x + anchor.to(torch.bfloat16)  # non-leaf: would be written in place
    ref = nmce.vocab_parallel_cross_entropy(x.clone().requires_grad_(True), t, 0, v, ctx,
                                            one_pass=False).item()
    for mode in ("no_grad", "no_requires_grad"):
        snapshot = logits if mode == "no_grad" else x.clone()
        torch.cuda.synchronize()
        torch.cuda.reset_peak_memory_stats()
        before = torch.cuda.memory_allocated()
        if mode == "no_grad":
            with torch.no_grad():
                loss = nmce.vocab_parallel_cross_entropy(snapshot, t, 0, v, ctx)
        else:
            loss = nmce.vocab_parallel_cross_entropy(snapshot, t, 0, v, ctx)
        torch.cuda.synchronize()
        peak = torch.cuda.max_memory_allocated() - before
        assert peak < slab // 8, f"{mode}: {peak} bytes allocated"
        assert loss.item() == ref, mode
        assert torch.equal(snapshot.view(torch.int16), x.view(torch.int16)), mode


def test_one_pass_retain_graph():
    """A second backward through the same graph: a separate one-pass buffer is
    handed out once, so the leaf's .grad accumulates the first gradient plus
    one written anew for the second upstream value (bit-identical to the
    two-pass path); the in-place form has no logits left and raises."""
    import nmce
    ctx = nmce.ParallelContext.single()
    g = torch.Generator(device=DEV).manual_seed(17)
    n, v = 256, 8192
    x = torch.randn(n, v, device=DEV, generator=g).to(torch.bfloat16)
    t = torch.randint(0, v, (n,), device=DEV, generator=g)
    grads = []
    for one_pass in (True, False):
        leaf = x.clone().requires_grad_(True)
        loss = nmce.vocab_parallel_cross_entropy(leaf, t, 0, v, ctx, one_pass=one_pass)
        loss.backward(retain_graph=True)
        first = leaf.grad.clone()
        (loss * 0.5).backward()
        grads.append((first, leaf.grad))
    assert torch.equal(grads[0][0].view(torch.int16), grads[1][0].view(torch.int16))
    assert torch.equal(grads[0][1].view(torch.int16), grads[1][1].view(torch.int16))
    anchor = torch.zeros((), device=DEV, requires_grad=True)
    loss = nmce.vocab_parallel_cross_entropy(x.clone() + anchor.to(torch.bfloat16), t, 0, v, ctx,
                                             inplace=True)
    loss.backward(retain_graph=True)
    with pytest.raises(RuntimeError, match="second backward"):
        loss.backward()


def test_one_pass_default_leaves_logits_readable():
    """With the default inplace=None the one-pass forward writes its gradient
    into a separate buffer: non-leaf logits read the same after the forward
    (an accuracy metric or a log line computed from them is not corrupted)
    and after the backward, and the gradient equals the in-place one."""
    import nmce
    ctx = nmce.ParallelContext.single()
    g = torch.Generator(device=DEV).manual_seed(18)
    n, v = 512, 50304
    x = torch.randn(n, v, device=DEV, generator=g).to(torch.bfloat16)
    t = torch.randint(0, v, (n,), device=DEV, generator=g)
    grads = []
    for inplace in (None, True):
        hint = torch.ones(1, dtype=torch.float32, device=DEV)
        anchor = torch.zeros((), device=DEV, requires_grad=True)
        logits = x.clone() + anchor.to(torch.bfloat16)  # non-leaf, own storage
        got = []
        logits.register_hook(lambda gr: got.append(gr))
        loss = nmce.vocab_parallel_cross_entropy(logits, t, 0, v, ctx, inplace=inplace,
                                                 upstream_hint=hint)
        torch.cuda.synchronize()
        if inplace is None:
            assert torch.equal(logits.detach().view(torch.int16), x.view(torch.int16))
            assert torch.equal(logits.detach().argmax(-1), x.argmax(-1))
        loss.backward()
        if inplace is None:
            assert torch.equal(logits.detach().view(torch.int16), x.view(torch.int16))
            assert got[0].data_ptr() != logits.data_ptr()
        else:
            assert got[0].data_ptr() == logits.data_ptr()
        grads.append(got[0].detach().clone())
    assert torch.equal(grads[0].view(torch.int16), grads[1].view(torch.int16))


def test_one_pass_on_a_side_stream():
    """The validated one-pass path on a stream other than the default one: the
    target check, its device word (one per device and stream) and the kernel
    run on the caller's current stream, so the loss and the in-place gradient
    are bit for bit those of the default stream; a bad target raises there
    and leaves the logits intact, and the default stream's next call is
    unaffected."""
    import nmce
    ctx = nmce.ParallelContext.single()
    g = torch.Generator(device=DEV).manual_seed(23)
    n, v = 512, 32000
    x = torch.randn(n, v, device=DEV, generator=g).to(torch.bfloat16)
    t = torch.randint(0, v, (n,), device=DEV, generator=g)
    hint = torch.ones(1, dtype=torch.float32, device=DEV)

    def run(targets):
        anchor = torch.zeros((), device=DEV, requires_grad=True)
        logits = x.clone() + anchor.to(torch.bfloat16)
        got = []
        logits.register_hook(lambda gr: got.append(gr))
        loss = nmce.vocab_parallel_cross_entropy(logits, targets, 0, v, ctx, inplace=True,
                                                 upstream_hint=hint)
        loss.backward()
        return loss.detach(), got[0]

    ref_loss, ref_grad = run(t)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        loss, grad = run(t)
        bad = t.clone()
        bad[n // 3] = v
        anchor = torch.zeros((), device=DEV, requires_grad=True)
        logits = x.clone() + anchor.to(torch.bfloat16)
        with pytest.raises(ValueError, match="target token id is outside the model vocabulary"):
            nmce.vocab_parallel_cross_entropy(logits, bad, 0, v, ctx, inplace=True,
                                              upstream_hint=hint)
        intact = torch.equal(logits.detach().view(torch.int16), x.view(torch.int16))
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    assert intact
    assert torch.equal(loss, ref_loss)
    assert torch.equal(grad.view(torch.int16), ref_grad.view(torch.int16))
    again_loss, again_grad = run(t)
    assert torch.equal(again_loss, ref_loss)
    assert torch.equal(again_grad.view(torch.int16), ref_grad.view(torch.int16))


@pytest.mark.parametrize("v", [50304, 128256])
def test_bad_target_leaves_in_place_logits_intact(v):
    """A target outside the vocabulary on the in-place one-pass path (the
    regular and the wide-row kernel): the wrapper raises the reference's
    ValueError and the logits are bit for bit what they were (the kernel reads
    the check's device flag and writes nothing), as the reference raises before
    touching anything (cross_entropy.py:79-81). The next call with good targets
    works as usual."""
    import nmce
    ctx = nmce.ParallelContext.single()
    g = torch.Generator(device=DEV).manual_seed(19)
    n = 300
    x = torch.randn(n, v, device=DEV, generator=g).to(torch.bfloat16)
    for bad in (v, -1, 10 ** 12):
        print(f"[gpu] bad target {bad} v={v} in place", flush=True)
        t = torch.randint(0, v, (n,), device=DEV, generator=g)
        t[n // 2] = bad
        anchor = torch.zeros((), device=DEV, requires_grad=True)
        logits = x.clone() + anchor.to(torch.bfloat16)
        with pytest.raises(ValueError, match="target token id is outside the model vocabulary"):
            nmce.vocab_parallel_cross_entropy(logits, t, 0, v, ctx, inplace=True)
        torch.cuda.synchronize()
        assert torch.equal(logits.detach().view(torch.int16), x.view(torch.int16)), bad
    t = torch.randint(0, v, (n,), device=DEV, generator=g)
    hint = torch.ones(1, dtype=torch.float32, device=DEV)
    leaf = x.clone().requires_grad_(True)
    ref = nmce.vocab_parallel_cross_entropy(leaf, t, 0, v, ctx, one_pass=False)
    ref.backward()
    anchor = torch.zeros((), device=DEV, requires_grad=True)
    logits = x.clone() + anchor.to(torch.bfloat16)
    got = []
    logits.register_hook(lambda gr: got.append(gr))
    loss = nmce.vocab_parallel_cross_entropy(logits, t, 0, v, ctx, inplace=True,
                                             upstream_hint=hint)
    loss.backward()
    assert loss.item() == ref.item()
    assert torch.equal(got[0].view(torch.int16), leaf.grad.view(torch.int16))


@pytest.mark.parametrize("dtype,v", [(torch.bfloat16, 65544), (torch.bfloat16, 128256),
                                     (torch.bfloat16, 131072), (torch.float32, 32776),
                                     (torch.float32, 50304), (torch.float32, 65536)])
def test_one_pass_wide_rows(dtype, v):
    """Rows past 8 vectors per lane take the one-pass kernel that keeps part of
    the row in LDS (up to 131072 bf16 / 65536 fp32 columns): 600 rows (more
    than its one workgroup per compute unit, so rows are walked with the next
    row's loads in flight), in place and into a separate buffer, at upstream
    1.0 and 0.5, bit for bit against the two-pass path; the loss against an
    fp64 reference and sampled gradient rows against the oracle."""
    import nmce
    assert v <= nmce._lib.load().nmce_ce_fwd_bwd_max_vocab(nmce._lib.dtype_code(dtype))
    print(f"[gpu] one-pass wide {dtype} V={v}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(18)
    n = 600
    x = (torch.randn(n, v, device=DEV, generator=g) * 2.0).to(dtype)
    t = torch.randint(0, v, (n,), device=DEV, generator=g)
    ctx = nmce.ParallelContext.single()
    ref_loss = _torch_ref_rows(x, t)
    for upstream in (1.0, 0.5):
        leaf = x.clone().requires_grad_(True)
        loss2 = nmce.vocab_parallel_cross_entropy(leaf, t, 0, v, ctx, one_pass=False)
        (loss2 * upstream).backward()
        ref_grad = leaf.grad
        for inplace in (False, True):
            hint = torch.ones(1, dtype=torch.float32, device=DEV)
            anchor = torch.zeros((), device=DEV, requires_grad=True)
            logits = x.clone() + anchor.to(dtype)
            got = []
            logits.register_hook(lambda gr: got.append(gr))
            loss = nmce.vocab_parallel_cross_entropy(logits, t, 0, v, ctx, inplace=inplace,
                                                     upstream_hint=hint)
            (loss * upstream).backward()
            assert loss.item() == loss2.item(), (upstream, inplace)
            a, b = got[0], ref_grad
            if dtype == torch.bfloat16:
                a, b = a.view(torch.int16), b.view(torch.int16)
            assert torch.equal(a, b), (upstream, inplace)
    assert abs(loss2.item() - ref_loss.mean().item()) <= 1e-5 * abs(ref_loss.mean().item())
    pick = torch.arange(0, n, 97, device=DEV)
    _, og = ce_oracle.closed_form(x[pick].float().cpu().numpy(), t[pick].cpu().numpy(),
                                  1.0 / n)
    leaf = x.clone().requires_grad_(True)
    nmce.vocab_parallel_cross_entropy(leaf, t, 0, v, ctx).backward()
    got = leaf.grad[pick].double().cpu().numpy()
    if dtype == torch.bfloat16:
        assert_bf16_close(got, og, what="wide grad rows", atol=1e-30)
    else:
        assert_close_rel(got, og, 1e-5, 1e-30, what="wide grad rows")


@pytest.mark.parametrize("dtype,v", [(torch.bfloat16, 131080), (torch.float32, 65540)])
def test_past_the_one_pass_width(dtype, v):
    """One vector past the one-pass kernel's widest row the wrapper takes the
    two-pass path (a Python autograd node, not the C++ one-pass node) and
    still gives the reference's loss and gradient: the loss against an fp64
    reference, sampled gradient rows against the oracle."""
    import nmce
    assert v > nmce._lib.load().nmce_ce_fwd_bwd_max_vocab(nmce._lib.dtype_code(dtype))
    print(f"[gpu] past the one-pass width {dtype} V={v}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(23)
    n = 300
    x = (torch.randn(n, v, device=DEV, generator=g) * 2.0).to(dtype)
    t = torch.randint(0, v, (n,), device=DEV, generator=g)
    ctx = nmce.ParallelContext.single()
    leaf = x.clone().requires_grad_(True)
    loss = nmce.vocab_parallel_cross_entropy(leaf, t, 0, v, ctx)
    assert "CppNode" not in loss.grad_fn.name(), loss.grad_fn.name()
    loss.backward()
    ref_loss = _torch_ref_rows(x, t)
    assert abs(loss.item() - ref_loss.mean().item()) <= 1e-5 * abs(ref_loss.mean().item())
    pick = torch.arange(0, n, 37, device=DEV)
    _, og = ce_oracle.closed_form(x[pick].float().cpu().numpy(), t[pick].cpu().numpy(),
                                  1.0 / n)
    got = leaf.grad[pick].double().cpu().numpy()
    if dtype == torch.bfloat16:
        assert_bf16_close(got, og, what="grad rows past the one-pass width", atol=1e-30)
    else:
        assert_close_rel(got, og, 1e-5, 1e-30, what="grad rows past the one-pass width")
    # one vector narrower takes the one-pass node
    w = v - (8 if dtype == torch.bfloat16 else 4)
    leaf2 = x[:, :w].contiguous().requires_grad_(True)
    t2 = torch.remainder(t, w)
    loss2 = nmce.vocab_parallel_cross_entropy(leaf2, t2, 0, w, ctx)
    assert "CppNode" in loss2.grad_fn.name(), loss2.grad_fn.name()


def test_one_pass_wide_extreme_rows():
    """The wide one-pass kernel against the two-pass path, bit for bit, on
    edge rows at V = 128256: -inf entries (30% of each row, never the
    target), maxima tied across half a row, targets leading by 40 and 80,
    logits of scale 60."""
    import nmce
    ctx = nmce.ParallelContext.single()
    g = torch.Generator().manual_seed(19)
    n, v = 320, 128256
    x = torch.randn(n, v, generator=g) * 2.0
    t = torch.randint(0, v, (n,), generator=g)
    mask = torch.rand(n, v, generator=g) < 0.3
    mask[torch.arange(n), t] = False
    x[:64][mask[:64]] = float("-inf")
    x[64:128, : v // 2] = x[64:128].max()
    x[128:160][torch.arange(32), t[128:160]] += 40.0
    x[160:192][torch.arange(32), t[160:192]] += 80.0
    x[192:] *= 30.0
    x, t = x.to(torch.bfloat16).to(DEV), t.to(DEV)
    out = []
    for one_pass in (True, False):
        leaf = x.clone().requires_grad_(True)
        loss = nmce.vocab_parallel_cross_entropy(leaf * 1.0, t, 0, v, ctx, inplace=False,
                                                 one_pass=one_pass)
        (loss * 0.7).backward()
        out.append((loss.detach(), leaf.grad.view(torch.int16)))
    assert torch.equal(out[0][0], out[1][0]) or (out[0][0].isnan() and out[1][0].isnan())
    assert torch.equal(out[0][1], out[1][1])


def test_c2_full_size_one_pass():
    """c2 through the wrapper's default path, the configuration the benchmark
    times: bf16 [8,2048,50304] ~ N(0,1) at TP = 1 runs ce_fwdbwd_kernel<bf16, 8>
    over 16384 rows on a grid of two workgroups per compute unit, each walking
    rows with the next row's loads in flight. In place (non-leaf logits) and
    into a separate buffer, at upstream 1.0 and 0.5, against the two-pass path
    bit for bit on the whole slab; the loss against a chunked fp64 reference;
    sampled gradient rows against the oracle."""
    import nmce
    print("[gpu] c2 one-pass bf16 [8,2048,50304]", flush=True)
    gen = torch.Generator(device=DEV).manual_seed(0)
    N, V = 8 * 2048, 50304
    x = torch.randn(N, V, device=DEV, generator=gen).to(torch.bfloat16)
    t = torch.randint(0, V, (N,), device=DEV, generator=gen)
    ref_loss = _torch_ref_rows(x, t)
    ctx = nmce.ParallelContext.single()
    tv = t.view(8, 2048)
    pick = torch.arange(0, N, 509, device=DEV)
    xs, ts = x[pick].float().cpu().numpy(), t[pick].cpu().numpy()
    for upstream in (1.0, 0.5):
        # the two-pass reference, into a separate buffer
        leaf = x.view(8, 2048, V).clone().requires_grad_(True)
        loss2 = nmce.vocab_parallel_cross_entropy(leaf, tv, 0, V, ctx, one_pass=False)
        (loss2 * upstream).backward()
        ref_grad = leaf.grad.view(N, V)
        del leaf
        for inplace in (False, True):
            hint = torch.ones(1, dtype=torch.float32, device=DEV)
            anchor = torch.zeros((), device=DEV, requires_grad=True)
            logits = x.view(8, 2048, V).clone() + anchor.to(torch.bfloat16)
            got = []
            logits.register_hook(lambda gr: got.append(gr))
            loss = nmce.vocab_parallel_cross_entropy(logits, tv, 0, V, ctx, inplace=inplace,
                                                     upstream_hint=hint)
            (loss * upstream).backward()
            assert loss.item() == loss2.item()
            grad = got[0].view(N, V)
            assert (grad.data_ptr() == logits.data_ptr()) == inplace
            assert torch.equal(grad.view(torch.int16), ref_grad.view(torch.int16)), \
                (upstream, inplace)
            del logits, got, grad
        if upstream == 1.0:
            per_token = nmce._VocabParallelCrossEntropy.apply(x.view(8, 2048, V), tv, 0, V,
                                                              None, 1, False)
            assert_close_rel(per_token.reshape(-1).cpu().numpy(), ref_loss.cpu().numpy(), 1e-5,
                             what="c2 loss")
            assert abs(loss2.item() - ref_loss.mean().item()) <= 1e-6 * abs(
                ref_loss.mean().item())
            rs = ref_grad.float().sum(-1) * N
            assert rs.abs().max().item() < 2e-2, rs.abs().max().item()
            _, og = ce_oracle.closed_form(xs, ts, 1.0 / N)
            assert_bf16_close(ref_grad[pick].float().cpu().numpy(), og, what="c2 grad rows",
                              atol=1e-30)
        del ref_grad
    torch.cuda.empty_cache()


def test_wide_full_size_one_pass():
    """The wide-row workload the benchmark times, bf16 [4,2048,128256] ~ N(0,1)
    at TP = 1: the one-pass kernel that keeps part of each row in LDS walks
    8192 rows, 32 per workgroup on 256 compute units, with the next row's loads
    in flight. In place and into a separate buffer, at upstream 1.0 and 0.5,
    bit for bit against the two-pass path on the whole slab; the loss against a
    chunked fp64 reference; sampled gradient rows against the oracle."""
    import nmce
    print("[gpu] wide one-pass bf16 [4,2048,128256]", flush=True)
    gen = torch.Generator(device=DEV).manual_seed(3)
    N, V = 4 * 2048, 128256
    x = torch.randn(N, V, device=DEV, generator=gen).to(torch.bfloat16)
    t = torch.randint(0, V, (N,), device=DEV, generator=gen)
    ctx = nmce.ParallelContext.single()
    tv = t.view(4, 2048)
    for upstream in (1.0, 0.5):
        leaf = x.view(4, 2048, V).clone().requires_grad_(True)
        loss2 = nmce.vocab_parallel_cross_entropy(leaf, tv, 0, V, ctx, one_pass=False)
        (loss2 * upstream).backward()
        ref_grad = leaf.grad.view(N, V)
        del leaf
        for inplace in (False, True):
            hint = torch.ones(1, dtype=torch.float32, device=DEV)
            anchor = torch.zeros((), device=DEV, requires_grad=True)
            logits = x.view(4, 2048, V).clone() + anchor.to(torch.bfloat16)
            got = []
            logits.register_hook(lambda gr: got.append(gr))
            loss = nmce.vocab_parallel_cross_entropy(logits, tv, 0, V, ctx, inplace=inplace,
                                                     upstream_hint=hint)
            (loss * upstream).backward()
            assert loss.item() == loss2.item()
            grad = got[0].view(N, V)
            assert (grad.data_ptr() == logits.data_ptr()) == inplace
            assert torch.equal(grad.view(torch.int16), ref_grad.view(torch.int16)), \
                (upstream, inplace)
            del logits, got, grad
        if upstream == 1.0:
            ref_loss = _torch_ref_rows(x, t)
            assert abs(loss2.item() - ref_loss.mean().item()) <= 1e-6 * abs(
                ref_loss.mean().item())
            pick = torch.arange(0, N, 1021, device=DEV)
            _, og = ce_oracle.closed_form(x[pick].float().cpu().numpy(), t[pick].cpu().numpy(),
                                          1.0 / N)
            assert_bf16_close(ref_grad[pick].float().cpu().numpy(), og, what="wide grad rows",
                              atol=1e-30)
        del ref_grad
    torch.cuda.empty_cache()


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_one_pass_extreme_rows(dtype):
    """The one-pass path against the two-pass path, bit for bit, on rows at the
    edges: -inf entries (30% of each row, never the target), maxima tied
    across half a row, targets leading by 40 and 80, logits of scale 60."""
    import nmce
    ctx = nmce.ParallelContext.single()
    g = torch.Generator().manual_seed(14)
    n, v = 256, 4096
    x = torch.randn(n, v, generator=g) * 2.0
    t = torch.randint(0, v, (n,), generator=g)
    mask = torch.rand(n, v, generator=g) < 0.3
    mask[torch.arange(n), t] = False
    x[:64][mask[:64]] = float("-inf")
    x[64:128, : v // 2] = x[64:128].max()
    x[128:160][torch.arange(32), t[128:160]] += 40.0
    x[160:192][torch.arange(32), t[160:192]] += 80.0
    x[192:] *= 30.0
    x, t = x.to(dtype).to(DEV), t.to(DEV)
    for upstream in (1.0, 0.7):
        out = []
        for one_pass in (True, False):
            leaf = x.clone().requires_grad_(True)
            loss = nmce.vocab_parallel_cross_entropy(leaf * 1.0, t, 0, v, ctx, inplace=False,
                                                     one_pass=one_pass)
            (loss * upstream).backward()
            out.append((loss.detach(), leaf.grad))
        assert torch.equal(out[0][0], out[1][0]) or (out[0][0].isnan() and out[1][0].isnan())
        a, b = out[0][1], out[1][1]
        if dtype == torch.bfloat16:
            a, b = a.view(torch.int16), b.view(torch.int16)
        assert torch.equal(a, b), f"gradient differs at upstream {upstream}"
