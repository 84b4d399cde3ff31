"""GPU parity of the fused LM head + cross entropy (libnmce HIP kernels).

The fused path computes the loss of ``hidden @ weight.t()`` (model.py:192
followed by cross_entropy.py:16-85) without storing the logits. Checks:

* the GEMM core (``nmce_gemm_nt_bf16``) against an fp64 product of the same
  bf16 values: fp32 output within 1e-5 of the largest |entry| of that row's
  dot-product scale, bf16 output within one bf16 ulp plus that floor;
* per-token loss against the fp64 closed form ``logsumexp(z) - z_t`` on the
  same bf16 inputs (small shapes: every token; workload shapes: seeded token
  subsets): within 1e-5 relative (the logits are exact bf16 products summed
  in fp32, so the loss keeps fp32 accuracy);
* the hidden / weight gradients against the fp64 closed form
  ``dZ = (softmax - onehot) * g``, ``dH = dZ W``, ``dW = dZ^T H``. The kernels
  round dZ to bf16 before the two products (as the reference's autocast
  backward does) and write bf16 results, so each gradient is held to a
  norm-relative error of 4e-3 against the exact product (bf16 rounding alone
  gives about 1.5e-3), and every element to the same product taken with dZ
  rounded to bf16: within one bf16 rounding of the result (2^-8 relative) plus
  2^-7 * sum |dZ||W| (the kernels' fp32 dZ and the fp64 dZ can round to
  neighbouring bf16 values at ties: one ulp, at most 2^-7 relative, per term),
  plus 2^-120 * sum |W| for dZ terms below fp32's normal range, which the
  exponential returns as 0, and 2^-126 for outputs below it; the norm bound
  adds 2^-8 * ||sqrt(dZ^2 W^2)||, the size of dZ's rounding noise, which a
  cancelling product (one token over a small vocabulary) does not average
  away;
* shard masking / offsets through a locally combined two-shard split, the
  chunked backward against the one-chunk backward, ragged sizes, and the
  drop-in wrapper against the unfused loss on the stored logits.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import ce_oracle

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


@pytest.fixture(scope="module", autouse=True)
def _lib():
    assert torch.cuda.is_available(), "GPU tests need a ROCm device"
    from nmce import _lib as L
    lib = L.load()
    print(f"[gpu] libnmce {lib.nmce_version():#x} on {torch.cuda.get_device_name(0)}",
          flush=True)
    return lib


def _gen(seed):
    return torch.Generator().manual_seed(seed)


def make_inputs(n, h, v, seed=0, x_std=1.0, w_std=0.02, v_total=None):
    g = _gen(seed)
    x = (torch.randn(n, h, generator=g) * x_std).to(torch.bfloat16)
    w = (torch.randn(v, h, generator=g) * w_std).to(torch.bfloat16)
    t = torch.randint(0, v_total or v, (n,), generator=g)
    return x, w, t


def _bf16_round(a: np.ndarray) -> np.ndarray:
    return torch.from_numpy(np.ascontiguousarray(a)).float().to(torch.bfloat16).double().numpy()


# Values below fp32's (and bf16's) normal range, 2^-126: dZ entries there (a
# softmax term under 2^-126, e.g. a logit margin past 87) come out of the
# exponential as 0, which through a product costs at most 2^-126 |g| per term
# (2^-120 sum_k |b_k| with |g| <= 2^6); and an output element there is flushed
# or held as a subnormal, off by up to 2^-126. Far below any value compared.
UNDERFLOW = 2.0 ** -120
FP32_TINY = 2.0 ** -126


class GradRef:
    """Exact fp64 gradient ``a @ b`` plus the same product with ``a`` (dZ)
    rounded to bf16, the l1 product |a| @ |b| that bounds rounding flips, the
    root-sum-square product sqrt(|a|^2 @ |b|^2) that sizes the random part of
    dZ's rounding, and the underflow allowance per output element."""

    def __init__(self, a: np.ndarray, b: np.ndarray):
        self.exact = a @ b
        ab = _bf16_round(a)
        self.rounded = ab @ b
        self.l1 = np.abs(ab) @ np.abs(b)
        self.rss = np.sqrt((ab * ab) @ (b * b))
        self.tiny = UNDERFLOW * np.abs(b).sum(axis=0)[None, :] + FP32_TINY


def fp64_reference(x, w, t, g=None):
    """The oracle's fp64 loss and gradients of the fused path on the bf16 values
    (oracle/ce_oracle.py ``lmhead_closed_form``). Returns (loss, dz, GradRef
    for dH, GradRef for dW); ``g`` defaults to the mean's 1/N."""
    X = x.double().numpy()
    W = w.double().numpy()
    n = X.shape[0]
    g = np.full(n, 1.0 / n) if g is None else np.asarray(g, dtype=np.float64)
    loss, dz, _, _ = ce_oracle.lmhead_closed_form(X, W, t.numpy(), g)
    return loss, dz, GradRef(dz, W), GradRef(dz.T.copy(), X)


def check_grad(got, ref: GradRef, what, norm_tol=4e-3):
    got = np.asarray(got, dtype=np.float64)
    norm = max(np.linalg.norm(ref.exact), 1e-300)
    nrel = np.linalg.norm(got - ref.exact) / norm
    tiny = np.broadcast_to(ref.tiny, ref.exact.shape)
    # Rounding dZ to bf16 moves each term of a product by up to 2^-9 of it,
    # with signs that vary: a bias-free error of size ~2^-9 * rss per element.
    # On large products rss is far below the result and norm_tol governs; a
    # product that cancels (one token's dH over a small vocabulary) keeps the
    # noise of its terms, and 2^-8 * rss covers it.
    allowed = norm_tol + (2.0 ** -8 * np.linalg.norm(ref.rss) + np.linalg.norm(tiny)) / norm
    assert nrel <= allowed, f"{what}: norm-relative error {nrel:.3e} > {allowed:.3e}"
    # output rounding (half a bf16 ulp, <= 2^-8 relative) plus one bf16 ulp
    # (<= 2^-7 relative) on any dZ term whose rounding flipped at a tie, plus
    # the underflow allowance
    bound = 2.0 ** -8 * np.abs(ref.rounded) + 2.0 ** -7 * ref.l1 + tiny
    bad = np.abs(got - ref.rounded) > bound
    assert not bad.any(), (f"{what}: {int(bad.sum())} elements off; first at "
                           f"{np.argwhere(bad)[0]}: {got[bad][0]} vs {ref.rounded[bad][0]}")
    return nrel


def run_fused(x, w, t, vstart=0, vchunk=None, g=None, tp_stats=None):
    """Forward stats + combine + backward through the C ABI. Returns
    (loss, dx, dw) as numpy; ``tp_stats`` returns the raw shard stats instead."""
    from nmce import _lib as L
    lib = L.load()
    n, h = x.shape
    v = w.shape[0]
    xd, wd = x.to(DEV), w.to(DEV)
    td = t.to(DEV)
    stream = L.stream_handle(torch.device(DEV))
    stats = torch.empty((3, n), dtype=torch.float32, device=DEV)
    ws = torch.empty(max(lib.nmce_lmhead_ce_fwd_workspace_bytes(n, h, v), 16), dtype=torch.uint8,
                     device=DEV)
    L.check(lib.nmce_lmhead_ce_fwd_stats(xd.data_ptr(), wd.data_ptr(), L.NMCE_BF16, n, h, v,
                                         td.data_ptr(), vstart, stats[0].data_ptr(),
                                         stats[1].data_ptr(), stats[2].data_ptr(), ws.data_ptr(),
                                         ws.numel(), stream), "fwd_stats")
    if tp_stats is not None:
        return stats
    out = torch.empty((3, n), dtype=torch.float32, device=DEV)
    b = stats.data_ptr()
    L.check(lib.nmce_ce_combine(b, b + 4 * n, b + 8 * n, 1, 3 * n, n, out[0].data_ptr(),
                                out[1].data_ptr(), out[2].data_ptr(), stream), "combine")
    if g is None:
        go = torch.full((1,), 1.0 / n, dtype=torch.float32, device=DEV)
        gs = 0
    else:
        go = torch.as_tensor(g, dtype=torch.float32).to(DEV)
        gs = 1
    dx = torch.empty((n, h), dtype=torch.bfloat16, device=DEV)
    dw = torch.empty((v, h), dtype=torch.bfloat16, device=DEV)
    chunk = 0 if vchunk is None else vchunk
    ws2 = torch.empty(lib.nmce_lmhead_ce_bwd_workspace_bytes(n, h, v, chunk), dtype=torch.uint8,
                      device=DEV)
    L.check(lib.nmce_lmhead_ce_bwd(xd.data_ptr(), wd.data_ptr(), L.NMCE_BF16, n, h, v,
                                   td.data_ptr(), vstart, out[1].data_ptr(), out[2].data_ptr(),
                                   go.data_ptr(), gs, dx.data_ptr(), dw.data_ptr(), chunk,
                                   ws2.data_ptr(), ws2.numel(), stream), "bwd")
    torch.cuda.synchronize()
    return (out[0].cpu().numpy(), dx.float().cpu().numpy(), dw.float().cpu().numpy())


# ---------------------------------------------------------------------------
# GEMM core
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("m,n,k", [(256, 256, 64), (512, 768, 256), (300, 520, 128),
                                   (1000, 777, 320), (1, 3, 64), (2048, 1024, 4096)])
@pytest.mark.parametrize("out", ["f32", "bf16"])
def test_gemm_nt(m, n, k, out):
    from nmce import _lib as L
    lib = L.load()
    print(f"[gemm] m={m} n={n} k={k} out={out}", flush=True)
    g = _gen(m * 7 + n * 3 + k)
    a = torch.randn(m, k, generator=g).to(torch.bfloat16)
    b = torch.randn(n, k, generator=g).to(torch.bfloat16)
    ad, bd = a.to(DEV), b.to(DEV)
    dt = torch.float32 if out == "f32" else torch.bfloat16
    c = torch.full((m, n), float("nan"), dtype=dt, device=DEV)
    L.check(lib.nmce_gemm_nt_bf16(ad.data_ptr(), k, bd.data_ptr(), k, m, n, k, c.data_ptr(),
                                  L.NMCE_F32 if out == "f32" else L.NMCE_BF16, n,
                                  L.stream_handle(torch.device(DEV))), "gemm")
    torch.cuda.synchronize()
    ref = a.double().numpy() @ b.double().numpy().T
    got = c.float().cpu().numpy().astype(np.float64)
    scale = np.sqrt(k) * 4.0  # |a||b| scale of one dot product of N(0,1) values
    err = np.abs(got - ref)
    bound = 1e-5 * scale + (2.0 ** -8 * np.abs(ref) if out == "bf16" else 0.0)
    assert np.isfinite(got).all()
    assert (err <= bound).all(), f"max err {err.max():.3e} (bound {np.min(bound):.3e})"


@pytest.mark.parametrize("m,n,k", [(256, 256, 64), (300, 520, 128), (1000, 777, 320),
                                   (1, 3, 64), (999, 1001, 1024)])
@pytest.mark.parametrize("a_mn", [1, 0])
def test_gemm_mn_is_the_nt_product_of_the_transposes(m, n, k, a_mn):
    """The MN-contiguous operand path (ds_read_b64_tr_b16 fragments, used by
    the fused dX product on dZ^T and W as they lie) gives the same
    bits as the K-contiguous one on the transposed operands: every lane's
    fragment holds the same 8 values in the same k order. Columns past m and
    n (up to the 8-element padding) hold NaN, which the product must not
    read into any written output."""
    from nmce import _lib as L
    lib = L.load()
    print(f"[gemm mn] m={m} n={n} k={k} a_mn={a_mn}", flush=True)
    g = _gen(m * 5 + n * 11 + k + a_mn)
    a = torch.randn(m, k, generator=g).to(torch.bfloat16).to(DEV)
    b = torch.randn(n, k, generator=g).to(torch.bfloat16).to(DEV)
    lda = (m + 7) // 8 * 8 + 8 if a_mn else k
    ldb = (n + 7) // 8 * 8
    if a_mn:
        a_s = torch.full((k, lda), float("nan"), dtype=torch.bfloat16, device=DEV)
        a_s[:, :m] = a.t()
    else:
        a_s = a
    b_s = torch.full((k, ldb), float("nan"), dtype=torch.bfloat16, device=DEV)
    b_s[:, :n] = b.t()
    stream = L.stream_handle(torch.device(DEV))
    c_mn = torch.full((m, n + 5), float("nan"), dtype=torch.bfloat16, device=DEV)
    c_nt = torch.full((m, n), float("nan"), dtype=torch.bfloat16, device=DEV)
    L.check(lib.nmce_gemm_mn_bf16(a_mn, a_s.data_ptr(), lda, b_s.data_ptr(), ldb, m, n, k,
                                  c_mn.data_ptr(), n + 5, stream), "gemm mn")
    L.check(lib.nmce_gemm_nt_bf16(a.data_ptr(), k, b.data_ptr(), k, m, n, k, c_nt.data_ptr(),
                                  L.NMCE_BF16, n, stream), "gemm nt")
    torch.cuda.synchronize()
    assert torch.equal(c_mn[:, :n].view(torch.int16), c_nt.view(torch.int16))
    assert torch.isnan(c_mn[:, n:].float()).all(), "wrote past n"


def test_gemm_rejects_bad_k():
    from nmce import _lib as L
    lib = L.load()
    a = torch.zeros(64, 100, dtype=torch.bfloat16, device=DEV)
    st = lib.nmce_gemm_nt_bf16(a.data_ptr(), 100, a.data_ptr(), 100, 64, 64, 100, a.data_ptr(),
                               L.NMCE_F32, 64, None)
    assert st == -2


# ---------------------------------------------------------------------------
# Fused loss: small shapes against the fp64 closed form
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("n,h,v", [(256, 64, 256), (300, 128, 1000), (77, 192, 513),
                                   (512, 256, 2048), (1, 64, 5)])
def test_fused_small(n, h, v):
    print(f"[fused] n={n} h={h} v={v}", flush=True)
    x, w, t = make_inputs(n, h, v, seed=n + v, x_std=1.0, w_std=0.5)
    loss, dx, dw = run_fused(x, w, t)
    rl, _, rdx, rdw = fp64_reference(x, w, t)
    np.testing.assert_allclose(loss, rl, rtol=1e-5, atol=1e-6)
    check_grad(dx, rdx, "dH")
    check_grad(dw, rdw, "dW")


def test_fused_per_token_grad_output():
    n, h, v = 300, 128, 1000
    x, w, t = make_inputs(n, h, v, seed=3, w_std=0.5)
    g = np.random.default_rng(3).uniform(0.1, 2.0, n).astype(np.float32)
    loss, dx, dw = run_fused(x, w, t, g=g)
    rl, _, rdx, rdw = fp64_reference(x, w, t, g=g.astype(np.float64))
    np.testing.assert_allclose(loss, rl, rtol=1e-5, atol=1e-6)
    check_grad(dx, rdx, "dH")
    check_grad(dw, rdw, "dW")


@pytest.mark.parametrize("chunk", [256, 512, 768])
def test_fused_chunked_backward_matches(chunk):
    n, h, v = 384, 128, 2000
    x, w, t = make_inputs(n, h, v, seed=11, w_std=0.5)
    _, dx1, dw1 = run_fused(x, w, t, vchunk=None)
    _, dx2, dw2 = run_fused(x, w, t, vchunk=chunk)
    # dW rows are computed identically per chunk; dH sums chunk partials in fp32.
    np.testing.assert_array_equal(dw1, dw2)
    rl, _, rdx, _ = fp64_reference(x, w, t)
    check_grad(dx2, rdx, f"dH chunk {chunk}")
    check_grad(dx1, rdx, "dH one chunk")


def test_bwd_dz_buffers():
    """The recomputed logit gradient itself, read back from the workspace after
    ``nmce_lmhead_ce_bwd_dz`` for both chunks of a ragged shard (300 tokens,
    1000 rows, chunk 512): dZ [N, chunk] against the oracle's fp64 dZ within
    one bf16 rounding (2^-8 relative, 2^-7 where the fp32 and fp64 values
    round to neighbours at a tie), dZ^T bit-for-bit its transpose, and the
    padding (rows past the shard, tokens past N) exactly zero."""
    import ctypes
    from nmce import _lib as L
    lib = L.load()
    n, h, v, chunk = 300, 128, 1000, 512
    x, w, t = make_inputs(n, h, v, seed=31, x_std=1.0, w_std=0.3)
    g = torch.rand(n, generator=_gen(32)) + 0.5
    print(f"[dz buffers] n={n} h={h} v={v} chunk={chunk}", flush=True)
    _, ref, _, _ = fp64_reference(x, w, t, g.double().numpy())
    xd, wd, td = x.to(DEV), w.to(DEV), t.to(DEV)
    stream = L.stream_handle(torch.device(DEV))
    stats = torch.empty((3, n), dtype=torch.float32, device=DEV)
    fws = torch.empty(lib.nmce_lmhead_ce_fwd_workspace_bytes(n, h, v), dtype=torch.uint8,
                      device=DEV)
    L.check(lib.nmce_lmhead_ce_fwd_stats(xd.data_ptr(), wd.data_ptr(), L.NMCE_BF16, n, h, v,
                                         td.data_ptr(), 0, stats[0].data_ptr(),
                                         stats[1].data_ptr(), stats[2].data_ptr(),
                                         fws.data_ptr(), fws.numel(), stream), "fwd_stats")
    out = torch.empty((3, n), dtype=torch.float32, device=DEV)
    b = stats.data_ptr()
    L.check(lib.nmce_ce_combine(b, b + 4 * n, b + 8 * n, 1, 3 * n, n, out[0].data_ptr(),
                                out[1].data_ptr(), out[2].data_ptr(), stream), "combine")
    go = g.float().to(DEV)
    buf = (ctypes.c_int64 * L.NMCE_LMHEAD_LAYOUT_FIELDS)()
    L.check(lib.nmce_lmhead_ce_bwd_layout(n, h, v, chunk, ctypes.addressof(buf)), "layout")
    lay = dict(zip(("total", "ldt", "vpad", "chunk", "n_chunks", "off_xt", "off_wt", "off_dzt",
                    "off_dz", "off_acc"), (int(b) for b in buf)))
    ldt = lay["ldt"]

    def bf16_view(offset, rows, cols):
        return ws[offset:offset + rows * cols * 2].view(torch.bfloat16).view(rows, cols)

    assert lay["n_chunks"] == 2 and ldt == 320
    ws = torch.zeros(lay["total"], dtype=torch.uint8, device=DEV)
    L.check(lib.nmce_lmhead_ce_bwd_prepare(xd.data_ptr(), wd.data_ptr(), L.NMCE_BF16, n, h, v,
                                           chunk, ws.data_ptr(), ws.numel(), stream), "prepare")
    for c in range(2):
        # poison both gradient buffers so that every checked byte is shown written
        ws[lay["off_dzt"]:lay["off_dzt"] + chunk * ldt * 2].fill_(0x7f)
        ws[lay["off_dz"]:lay["off_dz"] + n * chunk * 2].fill_(0x7f)
        L.check(lib.nmce_lmhead_ce_bwd_dz(xd.data_ptr(), wd.data_ptr(), L.NMCE_BF16, n, h, v,
                                          td.data_ptr(), 0, out[1].data_ptr(),
                                          out[2].data_ptr(), go.data_ptr(), 1, chunk, c,
                                          ws.data_ptr(), ws.numel(), stream), "bwd_dz")
        torch.cuda.synchronize()
        v0 = c * chunk
        mvalid = min(chunk, v - v0)
        mpad = (mvalid + 255) // 256 * 256
        dz = bf16_view(lay["off_dz"], n, chunk)
        dzt = bf16_view(lay["off_dzt"], chunk, ldt)
        got = dz[:, :mvalid].double().cpu().numpy()
        want = ref[:, v0:v0 + mvalid]
        bound = 2.0 ** -7 * np.abs(want) + 1e-30
        bad = np.abs(got - want) > bound
        assert not bad.any(), (f"chunk {c}: {int(bad.sum())} dZ entries off; first at "
                               f"{np.argwhere(bad)[0]}: {got[bad][0]} vs {want[bad][0]}")
        assert np.abs(got - want).max() <= 2.0 ** -8 * np.abs(want).max()
        raw = dz.view(torch.int16)
        rawt = dzt.view(torch.int16)
        assert torch.equal(rawt[:mvalid, :n], raw[:, :mvalid].t()), f"chunk {c}: dZ^T != dZ^T"
        assert not raw[:, mvalid:mpad].any(), f"chunk {c}: vocabulary padding of dZ"
        assert not rawt[mvalid:mpad, :].any(), f"chunk {c}: vocabulary padding of dZ^T"
        assert not rawt[:, n:ldt].any(), f"chunk {c}: token padding of dZ^T"


@pytest.mark.parametrize("v,chunk", [(1024, 0), (1000, 192)])
def test_fused_two_shards_combined(v, chunk):
    """TP=2 split of the vocabulary, shards combined locally: same loss and the
    same gradients (dW rows per shard, dH summed) as the full vocabulary. The
    second case has ragged 500-row shards recomputed in chunks (the 192 rows
    asked for round up to one 256-row tile), so each shard's second chunk is
    ragged and shard 1's chunks start at global ids that are not multiples of
    128."""
    from nmce import _lib as L
    lib = L.load()
    n, h = 300, 128
    x, w, t = make_inputs(n, h, v, seed=5, w_std=0.5)
    half = v // 2
    stats = [run_fused(x, w[r * half:(r + 1) * half], t, vstart=r * half, tp_stats=True)
             for r in range(2)]
    stack = torch.stack(stats)  # [2, 3, n]
    out = torch.empty((3, n), dtype=torch.float32, device=DEV)
    b = stack.data_ptr()
    L.check(lib.nmce_ce_combine(b, b + 4 * n, b + 8 * n, 2, 3 * n, n, out[0].data_ptr(),
                                out[1].data_ptr(), out[2].data_ptr(),
                                L.stream_handle(torch.device(DEV))), "combine")
    rl, _, rdx, rdw = fp64_reference(x, w, t)
    np.testing.assert_allclose(out[0].cpu().numpy(), rl, rtol=1e-5, atol=1e-6)
    # each shard owns about half the targets
    own0 = (t < half).float().mean().item()
    assert 0.3 < own0 < 0.7
    dxs, dws = [], []
    for r in range(2):
        xd, wd = x.to(DEV), w[r * half:(r + 1) * half].contiguous().to(DEV)
        dx = torch.empty((n, h), dtype=torch.bfloat16, device=DEV)
        dw = torch.empty((half, h), dtype=torch.bfloat16, device=DEV)
        go = torch.full((1,), 1.0 / n, dtype=torch.float32, device=DEV)
        td = t.to(DEV)
        ws = torch.empty(lib.nmce_lmhead_ce_bwd_workspace_bytes(n, h, half, chunk),
                         dtype=torch.uint8, device=DEV)
        L.check(lib.nmce_lmhead_ce_bwd(xd.data_ptr(), wd.data_ptr(), L.NMCE_BF16, n, h, half,
                                       td.data_ptr(), r * half, out[1].data_ptr(),
                                       out[2].data_ptr(), go.data_ptr(), 0, dx.data_ptr(),
                                       dw.data_ptr(), chunk, ws.data_ptr(), ws.numel(),
                                       L.stream_handle(torch.device(DEV))), "bwd")
        dxs.append(dx.float().cpu().numpy())
        dws.append(dw.float().cpu().numpy())
    check_grad(np.concatenate(dws), rdw, "dW (two shards)")
    check_grad(dxs[0] + dxs[1], rdx, "dH (sum of shards)")


@pytest.mark.parametrize("chunk", [256, 768, None])
def test_dropin_recomputing_backward(chunk):
    """The drop-in's recomputing backward (one_pass=False: libnmce's dZ kernel
    and its own GEMM for both products, dX accumulated in fp32 over the
    vocabulary chunks) against the fp64 closed form."""
    import nmce
    n, h, v = 320, 128, 1900
    x, w, t = make_inputs(n, h, v, seed=17, w_std=0.5)
    xd = x.to(DEV).requires_grad_(True)
    wd = w.to(DEV).requires_grad_(True)
    loss = nmce.lmhead_vocab_parallel_cross_entropy(xd, wd, t.to(DEV), 0, v,
                                                    nmce.ParallelContext.single(),
                                                    vocab_chunk=chunk, one_pass=False)
    loss.backward()
    rl, _, rdx, rdw = fp64_reference(x, w, t)
    assert abs(loss.item() - rl.mean()) <= 1e-5 * abs(rl.mean())
    check_grad(xd.grad.float().cpu().numpy(), rdx, f"dH (chunk {chunk})")
    check_grad(wd.grad.float().cpu().numpy(), rdw, f"dW (chunk {chunk})")


@pytest.mark.parametrize("v", [1024, 640, 600])
def test_fused_boundary_targets_two_shards(v):
    """Targets at the first and last vocabulary row of each shard and on both
    sides of the shard boundary, TP=2 combined locally, against the oracle's
    sharded form (cross_entropy.py:28-36 masking, tp_layers.py:98-110 offsets).
    Shards of 320 and 300 rows end inside a 128-row partial block: the block's
    padding rows cover the next shard's first ids, which must pick nothing."""
    from nmce import _lib as L
    lib = L.load()
    n, h = 64, 128
    half = v // 2
    x, w, _ = make_inputs(n, h, v, seed=41, w_std=0.5)
    edges = [0, half - 1, half, v - 1, 1, half + 1, half - 2, v - 2, half + 40, half + 63]
    t = torch.tensor([edges[i % len(edges)] for i in range(n)], dtype=torch.int64)
    stats = torch.stack([run_fused(x, w[r * half:(r + 1) * half].contiguous(), t, vstart=r * half,
                                   tp_stats=True) for r in range(2)])
    out = torch.empty((3, n), dtype=torch.float32, device=DEV)
    b = stats.data_ptr()
    L.check(lib.nmce_ce_combine(b, b + 4 * n, b + 8 * n, 2, 3 * n, n, out[0].data_ptr(),
                                out[1].data_ptr(), out[2].data_ptr(),
                                L.stream_handle(torch.device(DEV))), "combine")
    rl, parts, rdw = ce_oracle.lmhead_sharded(x.double().numpy(), w.double().numpy(), t.numpy(),
                                              2, 1.0 / n)
    np.testing.assert_allclose(out[0].cpu().numpy(), rl, rtol=1e-5, atol=1e-6)
    # each shard's picked target logit is exactly the owned raw logit or 0
    z = x.double().numpy() @ w.double().numpy().T
    for r in range(2):
        own = (t.numpy() >= r * half) & (t.numpy() < (r + 1) * half)
        pick = stats[r, 2].cpu().numpy()
        assert np.all(pick[~own] == 0.0)
        np.testing.assert_allclose(pick[own], z[np.arange(n)[own], t.numpy()[own]], rtol=1e-5,
                                   atol=1e-5)


def test_fused_nan_propagates():
    """A NaN hidden state gives that token a NaN loss (the reference has no
    checks, so NaN propagates); the other tokens are unaffected."""
    n, h, v = 64, 64, 300
    x, w, t = make_inputs(n, h, v, seed=43, w_std=0.5)
    x[7, 3] = float("nan")
    loss, _, _ = run_fused(x, w, t)
    assert np.isnan(loss[7])
    mask = np.ones(n, dtype=bool)
    mask[7] = False
    rl, _, _, _ = fp64_reference(x[mask], w, t[mask])
    np.testing.assert_allclose(loss[mask], rl, rtol=1e-5, atol=1e-6)


def test_fused_zero_grad_output_rows():
    """Per-token grad_output with zeros: those tokens contribute nothing to dW
    and get a zero dH row."""
    n, h, v = 128, 64, 500
    x, w, t = make_inputs(n, h, v, seed=47, w_std=0.5)
    g = np.where(np.arange(n) % 3 == 0, 0.0, 1.0 / n).astype(np.float32)
    loss, dx, dw = run_fused(x, w, t, g=g)
    assert np.all(dx[g == 0.0] == 0.0)
    rl, _, rdx, rdw = fp64_reference(x, w, t, g=g.astype(np.float64))
    check_grad(dx, rdx, "dH")
    check_grad(dw, rdw, "dW")


def test_fused_ragged_hidden_is_padded():
    """H = 100 is not a multiple of 64: the wrapper pads with zero columns."""
    import nmce
    n, h, v = 128, 100, 700
    x, w, t = make_inputs(n, h, v, seed=9, w_std=0.5)
    xd = x.to(DEV).requires_grad_(True)
    wd = w.to(DEV).requires_grad_(True)
    loss = nmce.lmhead_vocab_parallel_cross_entropy(xd, wd, t.to(DEV), 0, v,
                                                    nmce.ParallelContext.single())
    loss.backward()
    rl, _, rdx, rdw = fp64_reference(x, w, t)
    assert abs(loss.item() - rl.mean()) <= 1e-5 * abs(rl.mean())
    assert xd.grad.shape == (n, h) and wd.grad.shape == (v, h)
    check_grad(xd.grad.float().cpu().numpy(), rdx, "dH")
    check_grad(wd.grad.float().cpu().numpy(), rdw, "dW")


def test_dropin_matches_unfused_on_stored_logits():
    """lmhead_vocab_parallel_cross_entropy(x, W, t) == vocab_parallel_cross_entropy(x W^T, t)."""
    import nmce
    b, s, h, v = 2, 160, 256, 3000
    x, w, t = make_inputs(b * s, h, v, seed=21, w_std=0.3)
    ctx = nmce.ParallelContext.single()
    xd = x.view(b, s, h).to(DEV).requires_grad_(True)
    wd = w.to(DEV).requires_grad_(True)
    td = t.view(b, s).to(DEV)
    loss_f = nmce.lmhead_vocab_parallel_cross_entropy(xd, wd, td, 0, v, ctx)
    loss_f.backward()
    xu = x.view(b, s, h).to(DEV).float()
    wu = w.to(DEV).float()
    logits = torch.matmul(xu, wu.t().contiguous()).requires_grad_(True)
    loss_u = nmce.vocab_parallel_cross_entropy(logits, td, 0, v, ctx, inplace=False)
    loss_u.backward()
    assert loss_f.dtype == torch.float32 and loss_f.dim() == 0
    assert abs(loss_f.item() - loss_u.item()) <= 1e-5 * abs(loss_u.item())
    # the unfused path's fp32 logit gradient, through the same two products
    dz = logits.grad.reshape(b * s, v).double().cpu().numpy()
    check_grad(xd.grad.float().cpu().numpy().reshape(b * s, h),
               GradRef(dz, w.double().numpy()), "dH vs unfused")
    check_grad(wd.grad.float().cpu().numpy(), GradRef(dz.T.copy(), x.double().numpy()),
               "dW vs unfused")


def test_tied_embedding_and_head_gradients_sum():
    """model.py:235-236 ties the LM head to the embedding: one parameter used by
    the lookup and by the fused head, so its gradient is the head's dW plus the
    embedding's scatter of dX. Checked against the oracle in fp64."""
    import nmce
    n, h, v = 256, 128, 1000
    g = _gen(31)
    w0 = (torch.randn(v, h, generator=g) * 0.5).to(torch.bfloat16)
    ids = torch.randint(0, v, (n,), generator=g)
    t = torch.randint(0, v, (n,), generator=g)
    wd = w0.to(DEV).requires_grad_(True)
    x = torch.nn.functional.embedding(ids.to(DEV), wd) * 2.0   # exact in bf16
    loss = nmce.lmhead_vocab_parallel_cross_entropy(x, wd, t.to(DEV), 0, v,
                                                    nmce.ParallelContext.single())
    loss.backward()
    X = 2.0 * w0.double().numpy()[ids.numpy()]
    W = w0.double().numpy()
    rl, dz, dx, dw = ce_oracle.lmhead_closed_form(X, W, t.numpy(), np.full(n, 1.0 / n))
    ref = dw.copy()
    np.add.at(ref, ids.numpy(), 2.0 * dx)
    got = wd.grad.double().cpu().numpy()
    assert abs(loss.item() - rl.mean()) <= 1e-5 * abs(rl.mean())
    nrel = np.linalg.norm(got - ref) / np.linalg.norm(ref)
    assert nrel <= 8e-3, f"tied weight gradient norm-relative error {nrel:.3e}"


def test_fused_head_module_fp32_tied_weight_under_autocast():
    """GPT.forward's tail with the fused head (model.py:235-236, 255-281): an
    fp32 parameter shared by the embedding lookup and FusedParallelLMHead, run
    under bf16 autocast. The head consumes the parameter rounded to bf16 (as
    autocast's matmul does), and the parameter's fp32 .grad is the head's dW
    plus the lookup's scatter of dX, against the oracle in fp64. The logits
    path is autocast's own product, and outside autocast the fp32 weight is
    refused."""
    import types
    import nmce
    b, s, h, v = 2, 128, 128, 1000
    cfg = types.SimpleNamespace(vocab_size=v, n_embd=h, sequence_parallel=False)
    torch.manual_seed(41)
    head = nmce.FusedParallelLMHead(cfg, nmce.ParallelContext.single())
    with torch.no_grad():
        head.weight.mul_(25.0)  # std 0.5: a loss well away from log V
    head = head.to(DEV)
    W = head.weight
    g = _gen(41)
    ids = torch.randint(0, v, (b, s), generator=g)
    t = torch.randint(0, v, (b, s), generator=g)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        x = torch.nn.functional.embedding(ids.to(DEV), W).to(torch.bfloat16) * 2.0
        loss = head(x, t.to(DEV))
        logits = head(x)
        want_logits = x @ W.t()
    loss.backward()
    assert W.grad.dtype == torch.float32 and logits.dtype == torch.bfloat16
    assert torch.equal(logits, want_logits)
    n = b * s
    Wb = W.detach().to(torch.bfloat16).double().cpu().numpy()
    X = 2.0 * Wb[ids.reshape(-1).numpy()]
    rl, _, dx, dw = ce_oracle.lmhead_closed_form(X, Wb, t.reshape(-1).numpy(),
                                                 np.full(n, 1.0 / n))
    ref = dw.copy()
    np.add.at(ref, ids.reshape(-1).numpy(), 2.0 * dx)
    assert abs(loss.item() - rl.mean()) <= 1e-5 * abs(rl.mean())
    got = W.grad.double().cpu().numpy()
    nrel = np.linalg.norm(got - ref) / np.linalg.norm(ref)
    assert nrel <= 8e-3, f"tied fp32 weight gradient norm-relative error {nrel:.3e}"
    with pytest.raises(TypeError, match="bf16"):
        head(x.detach(), t.to(DEV))
    # sequence parallelism at TP = 1: the rank-major token order is the natural
    # one, so the loss is the same
    head.sequence_parallel = True
    with torch.autocast("cuda", dtype=torch.bfloat16):
        loss_sp = head(x.detach(), t.to(DEV))
    assert loss_sp.item() == loss.item()


def test_dropin_rejects_bad_target():
    import nmce
    x, w, t = make_inputs(64, 64, 100, seed=1)
    t[5] = 100
    with pytest.raises(ValueError, match="outside the model vocabulary"):
        nmce.lmhead_vocab_parallel_cross_entropy(x.to(DEV), w.to(DEV), t.to(DEV), 0, 100,
                                                 nmce.ParallelContext.single())


# ---------------------------------------------------------------------------
# Workload shapes: token / vocabulary subsets against fp32-on-GPU references
# ---------------------------------------------------------------------------

def _subset_reference(xd, wd, td, rows, g):
    """Loss and a dH GradRef for token subset ``rows`` (fp64, full vocabulary)."""
    zs = (xd[rows].double() @ wd.double().t())
    lse = torch.logsumexp(zs, dim=1)
    loss = lse - zs[torch.arange(len(rows), device=DEV), td[rows]]
    p = torch.exp(zs - lse[:, None])
    p[torch.arange(len(rows), device=DEV), td[rows]] -= 1.0
    return loss.cpu().numpy(), _grad_ref_gpu(p * g, wd.double())


def _grad_ref_gpu(a: torch.Tensor, b: torch.Tensor) -> GradRef:
    ref = GradRef.__new__(GradRef)
    ref.exact = (a @ b).cpu().numpy()
    ab = a.float().to(torch.bfloat16).double()
    ref.rounded = (ab @ b).cpu().numpy()
    ref.l1 = (ab.abs() @ b.abs()).cpu().numpy()
    ref.rss = ((ab * ab) @ (b * b)).sqrt().cpu().numpy()
    ref.tiny = (UNDERFLOW * b.abs().sum(dim=0)).cpu().numpy()[None, :] + FP32_TINY
    return ref


def _dw_subset_reference(xd, wd, td, vrows, lse_all, g):
    """dW GradRef for rows ``vrows`` in fp64, given every token's fp64 logsumexp."""
    zc = xd.double() @ wd[vrows].double().t()                       # [N, |vrows|]
    p = torch.exp(zc - lse_all[:, None])
    onehot = (td[:, None] == vrows[None, :]).double()
    return _grad_ref_gpu(((p - onehot) * g).t().contiguous(), xd.double())


def _lse_all(xd, wd, chunk=1024):
    out = []
    wt = wd.double().t().contiguous()
    for i in range(0, xd.shape[0], chunk):
        out.append(torch.logsumexp(xd[i:i + chunk].double() @ wt, dim=1))
    return torch.cat(out)


@pytest.mark.parametrize("route", ["one_pass", "one_pass_one_chunk", "recompute"])
@pytest.mark.parametrize("cfg", ["c4", "c5"])
def test_fused_workload(cfg, route):
    """c4: hidden [16384, 4096] ~ N(0,1), W [128256, 4096] ~ N(0, 0.02^2), uniform
    targets. c5: hidden [16384, 3072], W [256000, 3072] ~ N(0, 0.05^2) with 64
    rows x30, Zipf(1.1) targets (logits far beyond +-60). Every route: the
    drop-in's default one-pass path (bounded token chunks, dW accumulated in
    fp32 across them; the mean loss equal to the per-token Function's, bit for
    bit), the same as one chunk of all 16384 tokens (the opt-in that holds the
    exponentials of every token), and the recomputing backward (dX accumulated
    in fp32 over the 32768-row vocabulary chunks, 4 at c4, 8 at c5)."""
    import nmce
    g = torch.Generator(device=DEV).manual_seed(0)
    if cfg == "c4":
        n, h, v = 16384, 4096, 128256
        x = torch.randn(n, h, device=DEV, generator=g).to(torch.bfloat16)
        w = (torch.randn(v, h, device=DEV, generator=g) * 0.02).to(torch.bfloat16)
        t = torch.randint(0, v, (n,), device=DEV, generator=g)
    else:
        n, h, v = 16384, 3072, 256000
        x = torch.randn(n, h, device=DEV, generator=g).to(torch.bfloat16)
        wf = torch.randn(v, h, device=DEV, generator=g) * 0.05
        hot = torch.randperm(v, device=DEV, generator=g)[:64]
        wf[hot] *= 30.0
        w = wf.to(torch.bfloat16)
        del wf
        ranks = torch.arange(1, v + 1, device=DEV, dtype=torch.float64)
        t = torch.multinomial((ranks ** -1.1).float(), n, replacement=True, generator=g)
    print(f"[fused-workload] {cfg} n={n} h={h} v={v} backward {route}", flush=True)
    ctx = nmce.ParallelContext.single()
    xd = x.clone().requires_grad_(True)
    wd = w.clone().requires_grad_(True)
    if route.startswith("one_pass"):
        hint = torch.ones(1, dtype=torch.float32, device=DEV)
        chunk = n if route == "one_pass_one_chunk" else None
        loss = nmce.lmhead_vocab_parallel_cross_entropy(xd, wd, t, 0, v, ctx,
                                                        token_chunk=chunk, upstream_hint=hint)
        loss.backward()
        with torch.no_grad():
            per_tok = nmce._LMHeadVocabParallelCrossEntropy.apply(x, w, t, 0, v, None, 1, None)
        assert loss.item() == per_tok.mean().item()
    else:
        per_tok = nmce._LMHeadVocabParallelCrossEntropy.apply(xd, wd, t, 0, v, None, 1, None)
        loss = per_tok.mean()
        loss.backward()
    torch.cuda.synchronize()
    gval = 1.0 / n
    rows = torch.randperm(n, device=DEV, generator=g)[:256]
    rl, rdx = _subset_reference(x, w, t, rows, gval)
    got = per_tok[rows].detach().cpu().numpy()
    np.testing.assert_allclose(got, rl, rtol=1e-5, atol=1e-5)
    check_grad(xd.grad[rows].float().cpu().numpy(), rdx, f"{cfg} dH rows")
    lse = _lse_all(x, w)
    # the weight rows of the most frequent targets plus a random sample
    vrows = torch.cat([torch.bincount(t, minlength=v).topk(8).indices,
                       torch.randperm(v, device=DEV, generator=g)[:56]])
    if cfg == "c5":
        vrows = torch.cat([vrows, hot[:8]])
    rdw = _dw_subset_reference(x, w, t, vrows, lse, gval)
    check_grad(wd.grad[vrows].float().cpu().numpy(), rdw, f"{cfg} dW rows")
    # mean loss within 1e-3 relative of the fp64 mean over all tokens
    zt = (x.double() * w[t].double()).sum(dim=1)
    ref_mean = (lse - zt).mean().item()
    assert abs(loss.item() - ref_mean) <= 1e-5 * abs(ref_mean)
    if cfg == "c5":
        zmax = 0.0
        for i in range(0, n, 2048):
            zmax = max(zmax, (x[i:i + 2048].float() @ w[hot].float().t()).abs().max().item())
        print(f"[fused-workload] c5 max |logit| on the scaled rows: {zmax:.1f}", flush=True)
        assert zmax > 60.0


# ---------------------------------------------------------------------------
# The one-pass path (the drop-in's default when a gradient is wanted)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("n,h,v,chunk", [(300, 128, 777, None), (1000, 192, 1900, 256),
                                         (513, 100, 3001, 256), (64, 64, 1, None),
                                         (700, 64, 129, 512), (2048, 256, 20000, 768),
                                         (1100, 320, 7800, 256)])
def test_one_pass_fused_against_oracle(n, h, v, chunk):
    """The drop-in's one-pass forward (dX and dW formed chunk by chunk over the
    tokens, for the assumed upstream 1.0) against the fp64 closed form: one
    chunk, several with a short last one, a hidden size padded to 64, a
    vocabulary of one row and one that ends a row into a 128-row block. The
    last two split a chunk's dX product over K (its tiles are too few for the
    device): 8 equal ranges at V = 20000, and 3 at V = 7800 with a shorter last
    range and a hidden size of 320 (a 64-column edge tile)."""
    import nmce
    print(f"[gpu] one-pass fused n={n} h={h} v={v} chunk={chunk}", flush=True)
    x, w, t = make_inputs(n, h, v, seed=n + v, w_std=0.5)
    xd = x.to(DEV).requires_grad_(True)
    wd = w.to(DEV).requires_grad_(True)
    hint = torch.ones(1, dtype=torch.float32, device=DEV)
    loss = nmce.lmhead_vocab_parallel_cross_entropy(xd, wd, t.to(DEV), 0, v,
                                                    nmce.ParallelContext.single(),
                                                    token_chunk=chunk, upstream_hint=hint)
    loss.backward()
    rl, _, rdx, rdw = fp64_reference(x, w, t)
    assert abs(loss.item() - rl.mean()) <= 1e-5 * abs(rl.mean()) + 1e-30
    check_grad(xd.grad.float().cpu().numpy(), rdx, "dH")
    check_grad(wd.grad.float().cpu().numpy(), rdw, "dW")


@pytest.mark.parametrize("n,chunk", [(2048, 2048), (2000, 512)])
def test_fused_dw_product_is_bit_identical(n, chunk):
    """The one-pass path's dW product of each token chunk (V = 33000, 129
    tile rows with a ragged last one, x H = 1024) equals the GEMM core's own
    products on the same dZ^T, as the chunks leave it in the workspace: with
    one chunk (bf16 out) nmce_gemm_mn_bf16's product; with four chunks, the
    last one short (fp32 accumulation, rounded to bf16 by the last), the
    core's fp32 products of the chunks (nmce_gemm_nt_bf16 on X_c^T, zero past
    the chunk's tokens) summed in chunk order and rounded once. Compared as
    values (the two may differ in the sign of a zero only). The fp32
    read-add-store epilogue checked here is where a VALU write of a 16-byte
    store's data registers right after the store corrupts the first dword of
    some lanes, when the compiler omits the wait state (buffer_store_b128)."""
    from nmce import _lib as L
    from nmce import lmhead
    lib = L.load()
    h, v = 1024, 33000
    print(f"[gpu] chunked dW product n={n} chunk={chunk} v={v} h={h}", flush=True)
    x, w, t = make_inputs(n, h, v, seed=71, w_std=0.5)
    xd, wd, td = x.to(DEV), w.to(DEV), t.to(DEV)
    stream = L.stream_handle(torch.device(DEV))
    lay = lmhead._fused_layout(lib, n, h, v, chunk)
    ws = torch.zeros(lay["total"], dtype=torch.uint8, device=DEV)
    args = (xd.data_ptr(), wd.data_ptr(), L.NMCE_BF16, n, h, v)
    local = torch.empty((3, n), dtype=torch.float32, device=DEV)
    out = torch.empty((3, n), dtype=torch.float32, device=DEV)
    go = torch.ones(1, dtype=torch.float32, device=DEV)
    dx = torch.empty((n, h), dtype=torch.bfloat16, device=DEV)
    dw = torch.empty((v, h), dtype=torch.bfloat16, device=DEV)
    ldt, vpad, step = lay["ldt"], lay["vpad"], lay["chunk"]
    pt = lay["off_pt"]
    dzt = ws[pt:pt + vpad * ldt * 2].view(torch.bfloat16).view(vpad, ldt)  # dZ_c^T after grads
    acc = ref = None
    for c in range(lay["n_chunks"]):
        t0 = c * step
        nc = min(step, n - t0)
        L.check(lib.nmce_lmhead_ce_fused_chunk_stats(
            *args, td.data_ptr(), 0, chunk, c, local[0].data_ptr(), local[1].data_ptr(),
            local[2].data_ptr(), ws.data_ptr(), ws.numel(), stream), "chunk stats")
        base = local.data_ptr() + 4 * t0
        L.check(lib.nmce_ce_combine(base, base + 4 * n, base + 8 * n, 1, 3 * n, nc,
                                    out[0].data_ptr() + 4 * t0, out[1].data_ptr() + 4 * t0,
                                    out[2].data_ptr() + 4 * t0, stream), "combine")
        L.check(lib.nmce_lmhead_ce_fused_chunk_grads(
            *args, td.data_ptr(), 0, chunk, c, out[1].data_ptr(), out[2].data_ptr(),
            local[2].data_ptr(), go.data_ptr(), 0, float(n), dx.data_ptr(), dw.data_ptr(),
            ws.data_ptr(), ws.numel(), stream), "chunk grads")
        if lay["n_chunks"] == 1:
            assert ldt == n
            ref = torch.empty((v, h), dtype=torch.bfloat16, device=DEV)
            L.check(lib.nmce_gemm_mn_bf16(0, dzt.data_ptr(), ldt, xd.data_ptr(), h, v, h, ldt,
                                          ref.data_ptr(), h, stream), "gemm_mn")
        else:
            xt = torch.zeros((h, ldt), dtype=torch.bfloat16, device=DEV)
            xt[:, :nc] = xd[t0:t0 + nc].t()
            part = torch.empty((v, h), dtype=torch.float32, device=DEV)
            L.check(lib.nmce_gemm_nt_bf16(dzt.data_ptr(), ldt, xt.data_ptr(), ldt, v, h, ldt,
                                          part.data_ptr(), L.NMCE_F32, h, stream), "gemm_nt")
            acc = part if acc is None else acc + part
    torch.cuda.synchronize()
    if ref is None:
        ref = acc.to(torch.bfloat16)
    same = dw.float() == ref.float()
    assert same.all(), (f"{int((~same).sum())} of {same.numel()} dW elements differ; first at "
                        f"{torch.nonzero(~same)[0].tolist()}")
    assert dw.float().abs().sum().item() > 0


def test_one_pass_fused_follows_the_upstream_value():
    """A loss scaled by 0.25 each step: the first backward rescales the forward's
    gradients (a power-of-two ratio, so exactly) and records 0.25, after which
    the forward's gradients stand; 0.37 rescales by a ratio that rounds. Every
    step against the fp64 closed form for its upstream value."""
    import nmce
    n, h, v = 512, 128, 1500
    x, w, t = make_inputs(n, h, v, seed=61, w_std=0.5)
    hint = torch.ones(1, dtype=torch.float32, device=DEV)
    grads = []
    for scale in (0.25, 0.25, 0.37):
        xd = x.to(DEV).requires_grad_(True)
        wd = w.to(DEV).requires_grad_(True)
        loss = nmce.lmhead_vocab_parallel_cross_entropy(xd, wd, t.to(DEV), 0, v,
                                                        nmce.ParallelContext.single(),
                                                        token_chunk=256, upstream_hint=hint)
        (loss * scale).backward()
        assert hint.item() == np.float32(scale)
        rl, _, rdx, rdw = fp64_reference(x, w, t, g=np.full(n, scale / n))
        check_grad(xd.grad.float().cpu().numpy(), rdx, f"dH at {scale}")
        check_grad(wd.grad.float().cpu().numpy(), rdw, f"dW at {scale}")
        grads.append((xd.grad.clone(), wd.grad.clone()))
    # the hit (second step) and the exact power-of-two rescale agree bit for bit
    assert torch.equal(grads[0][0].view(torch.int16), grads[1][0].view(torch.int16))
    assert torch.equal(grads[0][1].view(torch.int16), grads[1][1].view(torch.int16))


def test_one_pass_fused_retain_graph_and_no_grad():
    """A second backward through the same graph recomputes the gradients (the
    first ones were handed out), so the leaves accumulate both; a forward
    under no_grad computes no gradient and returns the same loss."""
    import nmce
    n, h, v = 384, 128, 1200
    x, w, t = make_inputs(n, h, v, seed=67, w_std=0.5)
    ctx = nmce.ParallelContext.single()
    xd = x.to(DEV).requires_grad_(True)
    wd = w.to(DEV).requires_grad_(True)
    loss = nmce.lmhead_vocab_parallel_cross_entropy(xd, wd, t.to(DEV), 0, v, ctx,
                                                    token_chunk=256)
    loss.backward(retain_graph=True)
    (loss * 0.5).backward()
    rl, _, rdx, rdw = fp64_reference(x, w, t, g=np.full(n, 1.5 / n))
    check_grad(xd.grad.float().cpu().numpy(), rdx, "dH, two backwards")
    check_grad(wd.grad.float().cpu().numpy(), rdw, "dW, two backwards")
    with torch.no_grad():
        torch.cuda.synchronize()
        before = torch.cuda.memory_allocated()
        torch.cuda.reset_peak_memory_stats()
        nograd = nmce.lmhead_vocab_parallel_cross_entropy(xd, wd, t.to(DEV), 0, v, ctx)
        torch.cuda.synchronize()
        peak = torch.cuda.max_memory_allocated() - before
    assert nograd.item() == loss.item()
    assert peak < n * v * 2, f"a no-grad forward allocated {peak} bytes"


def test_fused_empty_batch():
    """Zero tokens through the fused head, nothing launched: an empty
    per-token loss, the mean is NaN (torch's mean of nothing), the hidden
    gradient is empty and the weight gradient is zero (a sum over no tokens),
    as x @ W.t() followed by the reference's loss gives."""
    import nmce
    ctx = nmce.ParallelContext.single()
    h = torch.zeros(0, 128, dtype=torch.bfloat16, device=DEV, requires_grad=True)
    w = (torch.randn(500, 128, generator=_gen(5)) * 0.02).to(torch.bfloat16).to(DEV)
    w.requires_grad_(True)
    t = torch.zeros(0, dtype=torch.int64, device=DEV)
    per = nmce._LMHeadVocabParallelCrossEntropy.apply(h, w, t, 0, 500, None, 1)
    assert per.shape == (0,)
    per.sum().backward()
    assert h.grad.shape == h.shape and not w.grad.any()
    h.grad = w.grad = None
    loss = nmce.lmhead_vocab_parallel_cross_entropy(h, w, t, 0, 500, ctx)
    assert loss.dim() == 0 and torch.isnan(loss)
    loss.backward()
    assert h.grad.shape == h.shape
    assert w.grad.shape == w.shape and not w.grad.any()
