"""Seeded sweeps of both loss paths through the C ABI.

Fused LM head + loss, over shapes, shard splits and backward chunks:

Each case draws tokens n, hidden size h (a multiple of 64, the C ABI's
granularity), a shard width and a TP degree (the vocabulary is tp shards of
that width, combined locally as the TP exchange would), a backward chunk and
either the mean's scalar gradient or a per-token one with mixed signs. The
combined loss must equal the fp64 closed form over the full vocabulary within
1e-5 relative; dW (the shards' rows stacked) and dH (the shards' partial sums
added) are checked as in test_lmhead_gpu.py: norm-relative 4e-3 against the
exact fp64 product, element-wise within one bf16 rounding plus a one-ulp dZ
flip per term of the product taken with dZ rounded to bf16.

Unfused loss, over dtypes, ragged shard widths, padded and misaligned row
strides, TP splits and gradient forms (tolerances in its docstring).

Extreme inputs, both paths: logit scales up to 60, -inf entries and whole -inf
shards, ties at the maximum, confident tokens, vocabularies of one or two rows
per shard (tolerances in the docstrings).
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import ce_oracle
from test_lmhead_gpu import DEV, GradRef, check_grad

pytestmark = pytest.mark.gpu


def bf16_fold_bound(v_shard: int) -> float:
    """Absolute bound on the error of a bf16 row's sum - 1 (and so on a
    confident token's loss), as derived in ``bf16_fold_floor``."""
    nvec = -(-v_shard // 8)
    folds = -(-nvec // 2048) + 2
    return (4 + folds) * 2.0 ** -24


def bf16_fold_floor(n: int, v: int, tp: int, t: np.ndarray, g) -> np.ndarray:
    """[n, v] absolute floor on the target column of a bf16 row's gradient.

    A bf16 row's statistics pass sums exp(x - max) per lane in fp32 with the
    maximum's 1 inside the running sum (fp32 rows keep it apart). For a
    confident token that sum lies in [1, 2), where each rounding costs at most
    2^-24: the chunk holding the maximum rounds at most 4 times in its 16-term
    tree, and every fold from there on once more. A lane of the 1024-lane
    workgroup folds at most ceil(nvec / 2048) 16-term chunks of the shard's
    nvec = ceil(v_shard / 8) vectors, one 8-term chunk and one head/tail term.
    The merges across lanes, waves and shards add the other terms without
    that rounding, so sum - 1 is off by at most (4 + folds) * 2^-24, and the
    target's gradient -(sum - 1) / sum * g by that times |g|."""
    gv = np.broadcast_to(np.abs(np.asarray(g, dtype=np.float64)), (n,))
    f = np.zeros((n, v))
    f[np.arange(n), np.asarray(t)] = bf16_fold_bound(v // tp) * gv
    return f


def _cases(count=24, seed=2024):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(count):
        tp = int(rng.choice([1, 1, 2, 3]))
        per = int(rng.choice([1, 7, 100, 128, 255, 256, 300, 777, 1024, 1500]))
        n = int(rng.choice([1, 3, 63, 64, 65, 200, 256, 300, 511]))
        h = int(rng.choice([64, 128, 192, 320]))
        chunk = int(rng.choice([0, 256, 512]))
        per_token = bool(rng.integers(0, 2))
        out.append((i, n, h, per, tp, chunk, per_token))
    return out


def _run_shards(x, w, t, tp, chunk, go):
    """Forward stats per shard, local combine, backward per shard."""
    from nmce import _lib as L
    lib = L.load()
    n, h = x.shape
    v = w.shape[0]
    per = v // tp
    stream = L.stream_handle(torch.device(DEV))
    xd, td = x.to(DEV), t.to(DEV)
    stats = torch.empty((tp, 3, n), dtype=torch.float32, device=DEV)
    for r in range(tp):
        wd = w[r * per:(r + 1) * per].contiguous().to(DEV)
        ws = torch.empty(max(lib.nmce_lmhead_ce_fwd_workspace_bytes(n, h, per), 16),
                         dtype=torch.uint8, device=DEV)
        L.check(lib.nmce_lmhead_ce_fwd_stats(xd.data_ptr(), wd.data_ptr(), L.NMCE_BF16, n, h,
                                             per, td.data_ptr(), r * per,
                                             stats[r, 0].data_ptr(), stats[r, 1].data_ptr(),
                                             stats[r, 2].data_ptr(), ws.data_ptr(), ws.numel(),
                                             stream), "fwd_stats")
    out = torch.empty((3, n), dtype=torch.float32, device=DEV)
    b = stats.data_ptr()
    L.check(lib.nmce_ce_combine(b, b + 4 * n, b + 8 * n, tp, 3 * n, n, out[0].data_ptr(),
                                out[1].data_ptr(), out[2].data_ptr(), stream), "combine")
    if go is None:
        god, gs = torch.full((1,), 1.0 / n, dtype=torch.float32, device=DEV), 0
    else:
        god, gs = torch.as_tensor(go, dtype=torch.float32).to(DEV), 1
    dxs, dws = [], []
    for r in range(tp):
        wd = w[r * per:(r + 1) * per].contiguous().to(DEV)
        dx = torch.empty((n, h), dtype=torch.bfloat16, device=DEV)
        dw = torch.empty((per, h), dtype=torch.bfloat16, device=DEV)
        ws = torch.empty(lib.nmce_lmhead_ce_bwd_workspace_bytes(n, h, per, chunk),
                         dtype=torch.uint8, device=DEV)
        L.check(lib.nmce_lmhead_ce_bwd(xd.data_ptr(), wd.data_ptr(), L.NMCE_BF16, n, h, per,
                                       td.data_ptr(), r * per, out[1].data_ptr(),
                                       out[2].data_ptr(), god.data_ptr(), gs, dx.data_ptr(),
                                       dw.data_ptr(), chunk, ws.data_ptr(), ws.numel(), stream),
                "bwd")
        dxs.append(dx.double().cpu().numpy())
        dws.append(dw.double().cpu().numpy())
    torch.cuda.synchronize()
    return out[0].cpu().numpy(), sum(dxs), np.concatenate(dws)


@pytest.mark.parametrize("case", _cases(), ids=lambda c: f"case{c[0]}")
def test_fused_sweep(case):
    i, n, h, per, tp, chunk, per_token = case
    v = per * tp
    print(f"[sweep] case {i}: n={n} h={h} shard={per} tp={tp} chunk={chunk} "
          f"per_token={per_token}", flush=True)
    g = torch.Generator().manual_seed(1000 + i)
    x = torch.randn(n, h, generator=g).to(torch.bfloat16)
    w = (torch.randn(v, h, generator=g) * 0.4).to(torch.bfloat16)
    # targets over the whole vocabulary, plus every shard's edges when they fit
    t = torch.randint(0, v, (n,), generator=g)
    edges = [e for r in range(tp) for e in (r * per, r * per + per - 1)]
    for k, e in enumerate(edges[:n]):
        t[k] = e
    go = None
    if per_token:
        go = (torch.rand(n, generator=g) * 2.0 - 0.5).numpy()
    loss, dx, dw = _run_shards(x, w, t, tp, chunk, go)
    X, W = x.double().numpy(), w.double().numpy()
    gv = np.full(n, 1.0 / n) if go is None else go.astype(np.float64)
    rl, dz, _, _ = ce_oracle.lmhead_closed_form(X, W, t.numpy(), gv)
    np.testing.assert_allclose(loss, rl, rtol=1e-5, atol=1e-6)
    check_grad(dx, GradRef(dz, W), f"case {i} dH")
    check_grad(dw, GradRef(dz.T.copy(), X), f"case {i} dW")


def _unfused_cases(count=24, seed=77):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(count):
        dtype = [torch.float32, torch.bfloat16][int(rng.integers(0, 2))]
        n = int(rng.choice([1, 2, 17, 64, 100, 1000]))
        per = int(rng.choice([1, 2, 7, 8, 9, 15, 16, 17, 100, 1023, 1024, 1025, 4097]))
        tp = int(rng.choice([1, 2, 3]))
        pad = int(rng.choice([0, 1, 8, 13]))
        offset = int(rng.choice([0, 1, 3]))
        per_token = bool(rng.integers(0, 2))
        out.append((i, dtype, n, per, tp, pad, offset, per_token))
    return out


@pytest.mark.parametrize("case", _unfused_cases(), ids=lambda c: f"case{c[0]}")
def test_unfused_sweep(case):
    """The unfused kernels through the C ABI on shards that are column slices of
    one padded, possibly misaligned slab: row stride V_full + pad, the slab
    starting ``offset`` elements into its allocation (so rows may sit off the
    16-byte grid and take the element-wise paths), tp shards combined locally,
    the mean's scalar gradient or a per-token one. Loss within 1e-5 relative of
    the oracle's sharded fp64 form (bf16 rows: plus ``bf16_fold_bound``); fp32
    gradients within 1e-5 relative, bf16 gradients within one bf16 ulp, plus
    on the target column of a bf16 row the bound of ``bf16_fold_floor``."""
    from _util import assert_bf16_close, assert_close_rel
    from nmce import _lib as L
    i, dtype, n, per, tp, pad, offset, per_token = case
    print(f"[sweep] unfused case {i}: {dtype} n={n} shard={per} tp={tp} pad={pad} "
          f"offset={offset} per_token={per_token}", flush=True)
    lib = L.load()
    v = per * tp
    ld = v + pad
    g = torch.Generator().manual_seed(5000 + i)
    x = (torch.randn(n, v, generator=g) * 2.0).to(dtype)
    t = torch.randint(0, v, (n,), generator=g)
    edges = [e for r in range(tp) for e in (r * per, r * per + per - 1)]
    for k, e in enumerate(edges[:n]):
        t[k] = e
    go = (torch.rand(n, generator=g) * 2.0 - 0.5) if per_token else None
    store = torch.zeros(offset + n * ld, dtype=dtype, device=DEV)
    slab = store[offset:].view(n, ld)
    slab[:, :v] = x.to(DEV)
    td = t.to(DEV)
    stream = L.stream_handle(torch.device(DEV))
    code = L.dtype_code(dtype)
    stats = torch.empty((tp, 3, n), dtype=torch.float32, device=DEV)
    for r in range(tp):
        sh = slab[:, r * per:(r + 1) * per]
        L.check(lib.nmce_ce_fwd_stats(sh.data_ptr(), code, n, per, ld, td.data_ptr(), r * per,
                                      stats[r, 0].data_ptr(), stats[r, 1].data_ptr(),
                                      stats[r, 2].data_ptr(), stream), "stats")
    out = torch.empty((3, n), dtype=torch.float32, device=DEV)
    b = stats.data_ptr()
    L.check(lib.nmce_ce_combine(b, b + 4 * n, b + 8 * n, tp, 3 * n, n, out[0].data_ptr(),
                                out[1].data_ptr(), out[2].data_ptr(), stream), "combine")
    if go is None:
        god, gs = torch.full((1,), 1.0 / n, dtype=torch.float32, device=DEV), 0
    else:
        god, gs = go.to(DEV), 1
    grads = []
    for r in range(tp):
        sh = slab[:, r * per:(r + 1) * per]
        gr = torch.empty((n, per), dtype=dtype, device=DEV)
        L.check(lib.nmce_ce_bwd(sh.data_ptr(), gr.data_ptr(), code, n, per, ld, per,
                                td.data_ptr(), r * per, out[1].data_ptr(), out[2].data_ptr(),
                                god.data_ptr(), gs, stream), "bwd")
        grads.append(gr)
    torch.cuda.synchronize()
    gov = np.full(n, 1.0 / n) if go is None else go.double().numpy()
    ol, og, _, _ = ce_oracle.sharded(x.double().numpy(), t.numpy(), tp, gov)
    # fp32 rows: relative only; bf16 rows: plus the bound on their sum - 1
    loss_atol = 1e-30 if dtype == torch.float32 else bf16_fold_bound(per)
    assert_close_rel(out[0].cpu().numpy(), ol, 1e-5, loss_atol, what=f"case {i} loss")
    floor = bf16_fold_floor(n, v, tp, t.numpy(), gov)
    for r in range(tp):
        got = grads[r].double().cpu().numpy()
        if dtype == torch.float32:
            assert_close_rel(got, og[r], 1e-5, 1e-12, what=f"case {i} grad shard {r}")
        else:
            fl = floor[:, r * per:(r + 1) * per]
            assert_bf16_close(got, og[r], what=f"case {i} bf16 grad shard {r}", atol=1e-30 + fl)


def _extreme_cases(count=40, seed=4242):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(count):
        out.append(dict(
            i=i,
            dtype=[torch.float32, torch.bfloat16][int(rng.integers(0, 2))],
            n=int(rng.choice([1, 7, 64, 333])),
            per=int(rng.choice([1, 3, 16, 100, 1025, 5000])),
            tp=int(rng.choice([1, 2, 3])),
            scale=float(rng.choice([0.01, 1.0, 5.0, 20.0, 60.0])),
            kind=int(rng.integers(0, 4)),
            per_token=bool(rng.integers(0, 2))))
    return out


@pytest.mark.parametrize("case", _extreme_cases(), ids=lambda c: f"case{c['i']}")
def test_unfused_extreme_inputs(case):
    """The unfused kernels through the C ABI on inputs at the edges of fp32:
    logit scales 0.01 to 60; -inf entries (30% of a row, never the target),
    which at small shard widths leave whole shards -inf on some rows; maxima
    tied across half the row; and confident rows whose target leads by 40.
    Against the oracle's sharded fp64 form: fp32 loss and gradients within
    1e-5 relative (plus 2^-126 per entry and per summed term, for softmax terms
    below fp32's normal range), bf16 as in ``test_unfused_sweep``."""
    from _util import assert_bf16_close, assert_close_rel
    from nmce import _lib as L
    c = case
    n, per, tp, dtype = c["n"], c["per"], c["tp"], c["dtype"]
    v = per * tp
    print(f"[extreme] case {c['i']}: {c}", flush=True)
    lib = L.load()
    g = torch.Generator().manual_seed(20000 + c["i"])
    x = torch.randn(n, v, generator=g) * c["scale"]
    t = torch.randint(0, v, (n,), generator=g)
    if c["kind"] == 1 and v > 1:
        mask = torch.rand(n, v, generator=g) < 0.3
        mask[torch.arange(n), t] = False
        x[mask] = float("-inf")
    elif c["kind"] == 2:
        x[:, : max(1, v // 2)] = x.max()
    elif c["kind"] == 3:
        x[torch.arange(n), t] += 40.0
    x = x.to(dtype)
    go = (torch.rand(n, generator=g) * 2.0 - 0.5) if c["per_token"] else None
    xd, td = x.to(DEV), t.to(DEV)
    stream = L.stream_handle(torch.device(DEV))
    code = L.dtype_code(dtype)
    stats = torch.empty((tp, 3, n), dtype=torch.float32, device=DEV)
    for r in range(tp):
        sh = xd[:, r * per:(r + 1) * per]
        L.check(lib.nmce_ce_fwd_stats(sh.data_ptr(), code, n, per, v, td.data_ptr(), r * per,
                                      stats[r, 0].data_ptr(), stats[r, 1].data_ptr(),
                                      stats[r, 2].data_ptr(), stream), "stats")
    out = torch.empty((3, n), dtype=torch.float32, device=DEV)
    b = stats.data_ptr()
    L.check(lib.nmce_ce_combine(b, b + 4 * n, b + 8 * n, tp, 3 * n, n, out[0].data_ptr(),
                                out[1].data_ptr(), out[2].data_ptr(), stream), "combine")
    if go is None:
        god, gs = torch.full((1,), 1.0 / n, dtype=torch.float32, device=DEV), 0
    else:
        god, gs = go.to(DEV), 1
    grads = []
    for r in range(tp):
        sh = xd[:, r * per:(r + 1) * per]
        gr = torch.empty((n, per), dtype=dtype, device=DEV)
        L.check(lib.nmce_ce_bwd(sh.data_ptr(), gr.data_ptr(), code, n, per, v, per, td.data_ptr(),
                                r * per, out[1].data_ptr(), out[2].data_ptr(), god.data_ptr(), gs,
                                stream), "bwd")
        grads.append(gr)
    torch.cuda.synchronize()
    gov = np.full(n, 1.0 / n) if go is None else go.double().numpy()
    ol, og, _, _ = ce_oracle.sharded(x.double().numpy(), t.numpy(), tp, gov)
    tiny = 2.0 ** -126
    gmax = float(np.abs(gov).max())
    if dtype == torch.float32:
        assert_close_rel(out[0].cpu().numpy(), ol, 1e-5, v * tiny, what="loss")
        for r in range(tp):
            assert_close_rel(grads[r].double().cpu().numpy(), og[r], 1e-5, v * tiny * gmax,
                             what=f"grad shard {r}")
    else:
        assert_close_rel(out[0].cpu().numpy(), ol, 1e-5, bf16_fold_bound(per), what="loss")
        floor = bf16_fold_floor(n, v, tp, t.numpy(), gov)
        for r in range(tp):
            assert_bf16_close(grads[r].double().cpu().numpy(), og[r], what=f"bf16 grad shard {r}",
                              atol=tiny * gmax + floor[:, r * per:(r + 1) * per])


def _extreme_fused_cases(count=24, seed=4343):
    rng = np.random.default_rng(seed)
    return [dict(i=i, n=int(rng.choice([1, 64, 300])), h=int(rng.choice([64, 128, 256])),
                 per=int(rng.choice([1, 2, 100, 300, 1024])), tp=int(rng.choice([1, 2])),
                 wscale=float(rng.choice([0.02, 0.3, 1.0, 3.0])),
                 chunk=int(rng.choice([0, 256])), per_token=bool(rng.integers(0, 2)))
            for i in range(count)]


@pytest.mark.parametrize("case", _extreme_fused_cases(), ids=lambda c: f"case{c['i']}")
def test_fused_extreme_inputs(case):
    """The fused path on logit scales up to ~50 (weights x 3 over H = 256),
    vocabularies of 1 or 2 rows per shard and single tokens: the loss within
    1e-5 relative of the fp64 closed form plus four fp32 ulps of the largest
    |z| (the logits are fp32 sums of bf16 products), and both gradients as in
    ``test_fused_sweep``, whose bounds carry the underflow and rounding-noise
    terms these inputs reach."""
    c = case
    n, h, per, tp = c["n"], c["h"], c["per"], c["tp"]
    v = per * tp
    print(f"[extreme] fused case {c['i']}: {c}", flush=True)
    g = torch.Generator().manual_seed(30000 + c["i"])
    x = torch.randn(n, h, generator=g).to(torch.bfloat16)
    w = (torch.randn(v, h, generator=g) * c["wscale"]).to(torch.bfloat16)
    t = torch.randint(0, v, (n,), generator=g)
    go = (torch.rand(n, generator=g) * 2.0 - 0.5).numpy() if c["per_token"] else None
    loss, dx, dw = _run_shards(x, w, t, tp, c["chunk"], go)
    X, W = x.double().numpy(), w.double().numpy()
    gv = np.full(n, 1.0 / n) if go is None else go.astype(np.float64)
    rl, dz, _, _ = ce_oracle.lmhead_closed_form(X, W, t.numpy(), gv)
    zmax = float(np.abs(X @ W.T).max())
    np.testing.assert_allclose(loss, rl, rtol=1e-5, atol=max(1e-6, 4 * 2.0 ** -24 * zmax))
    check_grad(dx, GradRef(dz, W), f"case {c['i']} dH")
    check_grad(dw, GradRef(dz.T.copy(), X), f"case {c['i']} dW")


def _one_pass_cases(count=32, seed=99):
    rng = np.random.default_rng(seed)
    out = []
    for i in range(count):
        dtype = [torch.float32, torch.bfloat16][int(rng.integers(0, 2))]
        epv = 4 if dtype == torch.float32 else 8
        limit = 16 * 1024 * epv  # the kernel's widest row (16 vectors per lane)
        # vectors per row across the kernels' ranges: up to 4 and 8 per lane
        # (registers), 9 to 16 per lane (registers and LDS), and their edges
        nvec = int(rng.choice([1, 3, 64, 1023, 1024, 1025, 4096, 4097, 8191, 8192, 8193,
                               9000, 12345, 16383, 16384]))
        v = min(nvec * epv, limit)
        n = int(rng.choice([1, 2, 7, 300, 1000, 2500]))
        pad_vecs = int(rng.choice([0, 0, 1, 5]))
        inplace = bool(rng.integers(0, 2))
        hint = float(rng.choice([1.0, 0.5, -2.0, 0.0, 3.0e-39, float("inf"), float("nan"), 7.0]))
        out.append((i, dtype, n, v, pad_vecs * epv, inplace, hint))
    return out


@pytest.mark.parametrize("case", _one_pass_cases(), ids=lambda c: f"case{c[0]}")
def test_one_pass_sweep(case):
    """nmce_ce_fwd_bwd through the C ABI on widths across its kernels (up to 4,
    8 and 16 vectors per lane, the last with part of the row in LDS), padded
    row strides, in place or into a separate buffer, and hint values that are
    used as they are or replaced by 1 (zero, subnormal, infinite, NaN). Loss
    and statistics equal nmce_ce_fwd's bit for bit, the gradient equals
    nmce_ce_bwd_scaled's for the value the kernel reports it assumed, and an
    in-place call leaves nothing of the logits but the gradient."""
    from nmce import _lib as L
    i, dtype, n, v, pad, inplace, hint = case
    print(f"[sweep] one-pass case {i}: {dtype} n={n} v={v} pad={pad} inplace={inplace} "
          f"hint={hint}", flush=True)
    lib = L.load()
    assert v <= lib.nmce_ce_fwd_bwd_max_vocab(L.dtype_code(dtype))
    ld = v + pad
    g = torch.Generator(device=DEV).manual_seed(40000 + i)
    slab = torch.zeros((n, ld), dtype=dtype, device=DEV)
    slab[:, :v] = (torch.randn(n, v, device=DEV, generator=g) * 2.5).to(dtype)
    t = torch.randint(0, v, (n,), device=DEV, generator=g)
    t[0] = v - 1
    if n > 1:
        t[1] = 0
    code = L.dtype_code(dtype)
    stream = L.stream_handle(torch.device(DEV))
    # two-pass reference: statistics and loss, then the gradient for a value
    ref = torch.empty((3, n), dtype=torch.float32, device=DEV)
    L.check(lib.nmce_ce_fwd(slab.data_ptr(), code, n, v, ld, t.data_ptr(), ref[0].data_ptr(),
                            ref[1].data_ptr(), ref[2].data_ptr(), stream), "fwd")
    expect = torch.full((1,), hint, dtype=torch.float32, device=DEV)
    assumed = torch.empty(1, dtype=torch.float32, device=DEV)
    out = torch.empty((3, n), dtype=torch.float32, device=DEV)
    work = slab.clone()
    grad = work if inplace else torch.empty((n, v), dtype=dtype, device=DEV)
    ldg = ld if inplace else v
    L.check(lib.nmce_ce_fwd_bwd(work.data_ptr(), grad.data_ptr(), code, n, v, ld, ldg,
                                t.data_ptr(), out[0].data_ptr(), out[1].data_ptr(),
                                out[2].data_ptr(), expect.data_ptr(), assumed.data_ptr(),
                                None, float(n), stream), "fwd_bwd")
    torch.cuda.synchronize()
    a = assumed.item()
    usable = math.isfinite(hint) and abs(hint) >= 1.17549435e-38
    assert a == (hint if usable else 1.0), (hint, a)
    bits = torch.int16 if dtype == torch.bfloat16 else torch.int32
    assert torch.equal(out.view(torch.int32), ref.view(torch.int32)), f"case {i} statistics"
    want = torch.empty((n, v), dtype=dtype, device=DEV)
    L.check(lib.nmce_ce_bwd_scaled(slab.data_ptr(), want.data_ptr(), code, n, v, ld, v,
                                   t.data_ptr(), 0, ref[1].data_ptr(), ref[2].data_ptr(),
                                   assumed.data_ptr(), 0, float(n), stream), "bwd")
    torch.cuda.synchronize()
    got = grad[:, :v] if inplace else grad
    assert torch.equal(got.view(bits), want.view(bits)), f"case {i} gradient"
    if inplace and pad:
        assert torch.equal(work[:, v:], slab[:, v:]), f"case {i} padding touched"
