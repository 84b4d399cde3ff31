"""The allocation-free fused forward statistics (nmce_lmhead_ce_fwd_stats_noalloc)
against the workspace entry point it mirrors (nmce_lmhead_ce_fwd_stats), through
the C ABI, bit for bit: two calls in a row on one GPU, the second smaller (the
fixed scratch keeps the first call's contents), the first large enough to take
three launches. A size past the scratch is refused before anything runs."""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _stats(lib, L, x, w, t, vstart, noalloc):
    n, h = x.shape
    v = w.shape[0]
    out = torch.full((3, n), float("nan"), dtype=torch.float32, device=DEV)
    stream = L.stream_handle(torch.device(DEV))
    if noalloc:
        st = lib.nmce_lmhead_ce_fwd_stats_noalloc(
            x.data_ptr(), w.data_ptr(), L.NMCE_BF16, n, h, v, t.data_ptr(), vstart,
            out[0].data_ptr(), out[1].data_ptr(), out[2].data_ptr(), stream)
    else:
        ws = torch.empty(lib.nmce_lmhead_ce_fwd_workspace_bytes(n, h, v), dtype=torch.uint8,
                         device=DEV)
        st = lib.nmce_lmhead_ce_fwd_stats(
            x.data_ptr(), w.data_ptr(), L.NMCE_BF16, n, h, v, t.data_ptr(), vstart,
            out[0].data_ptr(), out[1].data_ptr(), out[2].data_ptr(), ws.data_ptr(), ws.numel(),
            stream)
    L.check(st, "noalloc" if noalloc else "workspace")
    torch.cuda.synchronize()
    return out


def test_noalloc_matches_the_workspace_entry_point():
    from nmce import _lib as L
    lib = L.load()
    g = torch.Generator(device=DEV).manual_seed(31)
    # (tokens, hidden, shard rows, shard start): 12000 tokens over a 128256-row
    # shard take three launches (5376 tokens each fit the 64 MiB scratch);
    # the second call is smaller, and half its targets lie outside its shard.
    for n, h, v, vstart in ((12000, 256, 128256, 0), (700, 128, 50000, 50000)):
        print(f"[gpu] noalloc n={n} h={h} v={v} vstart={vstart}", flush=True)
        x = torch.randn(n, h, device=DEV, generator=g).to(torch.bfloat16)
        w = (torch.randn(v, h, device=DEV, generator=g) * 0.3).to(torch.bfloat16)
        t = torch.randint(0, vstart + 2 * v if vstart else v, (n,), device=DEV, generator=g)
        got = _stats(lib, L, x, w, t, vstart, noalloc=True)
        ref = _stats(lib, L, x, w, t, vstart, noalloc=False)
        assert not torch.isnan(ref).any()
        assert torch.equal(got, ref), (n, v, (got - ref).abs().max().item())


def test_noalloc_refuses_a_vocabulary_past_its_scratch():
    from nmce import _lib as L
    lib = L.load()
    x = torch.zeros(1, 64, dtype=torch.bfloat16, device=DEV)
    w = torch.zeros(1, 64, dtype=torch.bfloat16, device=DEV)
    t = torch.zeros(1, dtype=torch.int64, device=DEV)
    out = torch.zeros(3, 1, dtype=torch.float32, device=DEV)
    # 3 * ceil(V / 128) floats per token must fit 64 MiB: V = 715,827,840 is
    # the largest; one more row is refused before any launch.
    st = lib.nmce_lmhead_ce_fwd_stats_noalloc(
        x.data_ptr(), w.data_ptr(), L.NMCE_BF16, 1, 64, 715_827_841, t.data_ptr(), 0,
        out[0].data_ptr(), out[1].data_ptr(), out[2].data_ptr(),
        L.stream_handle(torch.device(DEV)))
    assert st == -7
    assert b"scratch" in lib.nmce_status_string(st)
    torch.cuda.synchronize()
    assert not out.any()
