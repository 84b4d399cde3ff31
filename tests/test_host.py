"""Host-side checks that need no GPU: the C ABI loads and exports what
include/nmce.h declares, argument errors are reported before any launch, and
the Python drop-in refuses what it cannot run (there is no CPU path)."""

from __future__ import annotations

import ast
import pathlib

import pytest
import torch

from _util import header_functions

ROOT = pathlib.Path(__file__).resolve().parent.parent
PKG = ROOT / "nano-megatron_amd" / "nmce"


@pytest.fixture(scope="module")
def lib():
    from nmce import _lib as L
    return L.load()


def test_library_exports_every_declared_symbol(lib):
    from nmce import _lib as L
    names = header_functions()
    assert "nmce_ce_fwd_stats" in names and "nmce_ce_bwd" in names
    for name in names:
        assert hasattr(lib, name), f"{name} declared in include/nmce.h but not exported"
        assert name in L.SIGNATURES, f"{name} has no ctypes signature"
    assert set(L.SIGNATURES) == set(names), "ctypes signatures and header disagree"


def test_autograd_extension_loads(lib):
    """The one-pass loss's C++ autograd node is built next to libnmce.so, links
    against it, and imports without a GPU; its timeline starts empty."""
    from nmce import _lib as L
    ext = L.autograd_ext()
    assert pathlib.Path(ext.__file__).parent == L.LIB_PATH.parent
    for name in ("one_pass_mean", "one_pass_mean_checked", "assumed_of", "set_timing",
                 "take_timeline", "head_output"):
        assert hasattr(ext, name), name
    assert ext.take_timeline() == []


def test_head_output_node():
    """The measurements' stand-in for the LM-head node: the logits come back as
    a non-leaf alias (same storage) with a C++ grad_fn, and its backward hands
    no gradient to the anchor. Pure autograd: it runs on CPU tensors."""
    from nmce import _lib as L
    ext = L.autograd_ext()
    x = torch.randn(4, 6)
    anchor = torch.zeros((), requires_grad=True)
    y = ext.head_output(x, anchor)
    assert y.requires_grad and not y.is_leaf and y.data_ptr() == x.data_ptr()
    assert y.grad_fn is not None and "CppNode" in y.grad_fn.name()
    (y * 2.0).sum().backward()
    assert anchor.grad is None


def test_status_strings(lib):
    assert lib.nmce_status_string(0) == b"ok"
    for code in range(-6, 0):
        assert lib.nmce_status_string(code) not in (b"", b"unknown status")
    assert lib.nmce_status_string(-99) == b"unknown status"
    assert lib.nmce_version() >> 16 >= 1


def test_argument_errors_before_launch(lib):
    """Every one of these returns before touching the device."""
    p = 4096  # a fake, aligned device address; never dereferenced
    assert lib.nmce_ce_fwd_stats(p, 7, 4, 8, 8, p, 0, p, p, p, None) == -1
    assert lib.nmce_ce_fwd_stats(p, 1, 4, 0, 8, p, 0, p, p, p, None) == -2
    assert lib.nmce_ce_fwd_stats(p, 1, 4, 8, 4, p, 0, p, p, p, None) == -2
    assert lib.nmce_ce_fwd_stats(p, 1, -1, 8, 8, p, 0, p, p, p, None) == -2
    assert lib.nmce_ce_fwd_stats(p, 1, 0, 8, 8, None, 0, None, None, None, None) == 0
    assert lib.nmce_ce_fwd_stats(p, 1, 4, 8, 8, None, 0, p, p, p, None) == -4
    assert lib.nmce_ce_fwd_stats(p + 1, 1, 4, 8, 8, p, 0, p, p, p, None) == -3
    assert lib.nmce_ce_fwd(p, 3, 4, 8, 8, p, p, p, p, None) == -1
    assert lib.nmce_ce_fwd(p, 0, 4, 8, 7, p, p, p, p, None) == -2
    assert lib.nmce_ce_fwd(p, 0, 4, 8, 8, p, None, p, p, None) == -4
    assert lib.nmce_ce_fwd(p + 2, 0, 4, 8, 8, p, p, p, p, None) == -3
    assert lib.nmce_ce_fwd(p, 0, 0, 8, 8, None, None, None, None, None) == 0
    assert lib.nmce_ce_combine(p, p, p, 0, 4, 4, p, p, p, None) == -5
    assert lib.nmce_ce_combine(p, p, p, 2, 3, 4, p, p, p, None) == -2
    assert lib.nmce_ce_combine(None, p, p, 1, 4, 4, p, p, p, None) == -4
    assert lib.nmce_ce_bwd(p, p, 1, 4, 8, 8, 16, p, 0, p, p, p, 0, None) == -2  # in place, ld differs
    assert lib.nmce_ce_bwd(p, p, 1, 4, 8, 8, 8, p, 0, p, p, p, -1, None) == -2
    assert lib.nmce_ce_bwd(p, p, 2, 4, 8, 8, 8, p, 0, p, p, p, 0, None) == -1
    assert lib.nmce_ce_bwd(p, p + 1, 1, 4, 8, 8, 8, p, 0, p, p, p, 0, None) == -3
    assert lib.nmce_ce_bwd_scaled(p, p, 1, 4, 8, 8, 8, p, 0, p, p, p, 0, 0.0, None) == -2
    assert lib.nmce_ce_bwd_scaled(p, p, 1, 4, 8, 8, 8, p, 0, p, p, p, 0, -1.0, None) == -2
    assert lib.nmce_ce_bwd_scaled(p, p, 1, 0, 8, 8, 8, None, 0, None, None, None, 0, 2.0, None) == 0
    assert lib.nmce_validate_targets(p, 4, 0, p, None) == -2
    assert lib.nmce_validate_targets(None, 4, 10, p, None) == -4


def test_lmhead_argument_errors_before_launch(lib):
    """The fused entry points report bad arguments before touching the device."""
    import ctypes
    p = 4096  # a fake, aligned device address; never dereferenced
    ws = 1 << 40
    fwd = lib.nmce_lmhead_ce_fwd_stats
    assert fwd(p, p, 0, 16, 64, 100, p, 0, p, p, p, p, ws, None) == -1      # fp32 not supported
    assert fwd(p, p, 1, 16, 100, 100, p, 0, p, p, p, p, ws, None) == -2    # H not a multiple of 64
    assert fwd(p, p, 1, 16, 64, 0, p, 0, p, p, p, p, ws, None) == -2       # empty shard
    assert fwd(p, p, 1, 0, 64, 100, None, 0, None, None, None, None, 0, None) == 0
    assert fwd(p + 2, p, 1, 16, 64, 100, p, 0, p, p, p, p, ws, None) == -3
    assert fwd(p, p, 1, 16, 64, 100, None, 0, p, p, p, p, ws, None) == -4
    assert fwd(p, p, 1, 16, 64, 100, p, 0, p, p, p, p, 16, None) == -6     # workspace too small
    bwd = lib.nmce_lmhead_ce_bwd_dz
    assert bwd(p, p, 1, 16, 64, 100, p, 0, p, p, p, 0, 0, 1, p, ws, None) == -2  # chunk 1 of 1
    assert bwd(p, p, 1, 16, 64, 100, None, 0, p, p, p, 0, 0, 0, p, ws, None) == -4
    assert bwd(p, p, 1, 16, 64, 100, p, 0, p, p, p, -1, 0, 0, p, ws, None) == -2
    assert lib.nmce_lmhead_ce_bwd_prepare(p, p, 1, 16, 64, 100, 0, p, 8, None) == -6
    assert lib.nmce_lmhead_ce_bwd_layout(16, 64, 100, 0, None) == -4
    assert lib.nmce_gemm_nt_bf16(p, 64, p, 64, 16, 16, 100, p, 0, 16, None) == -2
    assert lib.nmce_gemm_nt_bf16(p, 64, p, 64, 16, 16, 64, p, 7, 16, None) == -1
    assert lib.nmce_gemm_nt_bf16(p, 60, p, 64, 16, 16, 64, p, 0, 16, None) == -3
    stats = lib.nmce_lmhead_ce_fused_chunk_stats
    assert stats(p, p, 0, 16, 64, 100, p, 0, 0, 0, p, p, p, p, ws, None) == -1   # fp32
    assert stats(p, p, 1, 16, 100, 100, p, 0, 0, 0, p, p, p, p, ws, None) == -2  # H % 64
    assert stats(p, p, 1, 16, 64, 100, p, 0, 0, 1, p, p, p, p, ws, None) == -2   # chunk 1 of 1
    assert stats(p, p, 1, 16, 64, 100, None, 0, 0, 0, p, p, p, p, ws, None) == -4
    assert stats(p, p, 1, 16, 64, 100, p, 0, 0, 0, p, p, p, p, 16, None) == -6   # workspace
    # The rescale's grid holds at most 65535 blocks of 128 vocabulary rows,
    # and the vocabulary is padded to 256: 8388352 rows fit, one more does not.
    assert stats(p, p, 1, 16, 64, 8388352, p, 0, 0, 0, p, p, p, p, 16, None) == -6
    assert stats(p, p, 1, 16, 64, 8388353, p, 0, 0, 0, p, p, p, p, ws, None) == -2
    grads = lib.nmce_lmhead_ce_fused_chunk_grads
    assert grads(p, p, 1, 16, 64, 100, p, 0, 0, 0, p, p, p, p, 0, 0.0, p, p, p, ws,
                 None) == -2  # gout_div must be positive
    assert grads(p, p, 1, 16, 64, 100, p, 0, 0, 0, p, p, p, p, 0, 16.0, p, None, p, ws,
                 None) == -4
    assert grads(p, p, 1, 16, 64, 8388353, p, 0, 0, 0, p, p, p, p, 0, 16.0, p, p, p, ws,
                 None) == -2
    mn = lib.nmce_gemm_mn_bf16
    assert mn(1, p, 16, p, 16, 16, 16, 100, p, 16, None) == -2  # k not a multiple of 64
    assert mn(1, p, 8, p, 16, 16, 16, 64, p, 16, None) == -3    # lda below m rounded to 8
    assert mn(0, p, 32, p, 16, 16, 16, 64, p, 16, None) == -3   # K-contiguous a: lda < k
    assert mn(1, p, 16, p, 8, 16, 16, 64, p, 16, None) == -3    # ldb below n rounded to 8
    assert mn(1, p, 16, p, 16, 16, 16, 64, None, 16, None) == -4


def test_lmhead_workspace_layout(lib):
    """The backward workspace layout at the c4 shape: padding, chunking and
    256-byte aligned, non-overlapping regions."""
    import ctypes
    n, h, v, chunk = 16384, 4096, 128256, 32768
    buf = (ctypes.c_int64 * 10)()
    assert lib.nmce_lmhead_ce_bwd_layout(n, h, v, chunk, ctypes.addressof(buf)) == 0
    total, ldt, vpad, ch, nch, o_xt, o_wt, o_dzt, o_dz, o_acc = list(buf)
    assert (ldt, vpad, ch, nch) == (16384, 128256, 32768, 4)
    regions = [(o_xt, h * ldt * 2), (o_wt, h * vpad * 2), (o_dzt, ch * ldt * 2),
               (o_dz, n * ch * 2), (o_acc, n * h * 4)]
    for (a, sa), (b, _) in zip(regions, regions[1:]):
        assert a % 256 == 0 and a + sa <= b
    assert o_acc + n * h * 4 <= total
    assert total == lib.nmce_lmhead_ce_bwd_workspace_bytes(n, h, v, chunk)
    # ragged sizes round up: tokens to 64, vocabulary rows to 256
    assert lib.nmce_lmhead_ce_bwd_layout(77, 192, 513, 0, ctypes.addressof(buf)) == 0
    assert (buf[1], buf[2], buf[3], buf[4]) == (128, 768, 768, 1)
    assert lib.nmce_lmhead_ce_fwd_workspace_bytes(n, h, v) >= 3 * ((v + 127) // 128) * n * 4


def test_default_chunk_never_holds_full_logits(lib):
    """The drop-in's default one-pass path at the fused workloads (c4: 16384
    tokens x 128256 rows, H 4096; c5: 16384 x 256000, H 3072) allocates no
    buffer of the [tokens, V] logits' size: the workspace's one chunk-sized
    buffer, P^T, holds a quarter of the tokens (4096), its largest buffer is
    the fp32 dW accumulator [V, H] (a size set by H, not by the tokens), and
    the whole workspace stays under the bf16 logits' size. The recomputing backward's default vocabulary chunk
    keeps each of its two gradient buffers under a third of the logits."""
    import ctypes
    from nmce import _lib as L
    from nmce import lmhead
    buf = (ctypes.c_int64 * L.NMCE_LMHEAD_FUSED_LAYOUT_FIELDS)()
    for n, h, v in ((16384, 4096, 128256), (16384, 3072, 256000)):
        logits_bytes = n * v * 2  # the bf16 logits
        chunk = lmhead.default_token_chunk(n, v)
        assert chunk == 4096
        assert lib.nmce_lmhead_ce_fused_layout(n, h, v, chunk, ctypes.addressof(buf)) == 0
        total, got_chunk, n_chunks = buf[0], buf[1], buf[2]
        off_pt, off_part, off_acc, off_dxp = buf[6], buf[7], buf[8], buf[9]
        assert (got_chunk, n_chunks) == (4096, 4)
        pt_bytes = off_part - off_pt
        assert pt_bytes == ((v + 255) // 256 * 256) * 4096 * 2
        assert 4 * pt_bytes <= logits_bytes + 4 * 256 * 4096 * 2
        off_xt = buf[11]
        regions = [off_part - off_pt, off_acc - off_part, off_dxp - off_acc,
                   off_xt - off_dxp, total - off_xt]
        assert max(regions) == off_dxp - off_acc and max(regions) <= logits_bytes / 2
        assert total - off_xt == h * 4096 * 2  # X_c^T, the dW product's second operand
        assert total < logits_bytes
        assert off_dxp - off_acc == (v * h * 4 + 255) // 256 * 256  # fp32 dW accumulator
    buf = (ctypes.c_int64 * 10)()
    for n, h, v in ((16384, 4096, 128256), (16384, 3072, 256000)):
        assert lib.nmce_lmhead_ce_bwd_layout(n, h, v, lmhead.DEFAULT_VOCAB_CHUNK,
                                             ctypes.addressof(buf)) == 0
        chunk, n_chunks = buf[3], buf[4]
        assert n_chunks >= 4 and 3 * chunk <= v
        assert lib.nmce_lmhead_ce_bwd_layout(n, h, v, 1 << 20, ctypes.addressof(buf)) == 0
        assert buf[4] == 1


def test_one_pass_token_chunk_budget(lib):
    """The one-pass path's default token chunk: a quarter of the tokens rounded
    up to 256 (at least 256; all of them up to 256), and no more than fit
    CHUNK_BUDGET_BYTES of exponentials (2 V bytes per token); the fused layout
    then holds one chunk (no fp32 dW accumulator) or several (with one). A
    chunk of every token is the explicit opt-in with P^T the logits' size."""
    import ctypes
    from nmce import _lib as L
    from nmce import lmhead
    budget = lmhead.CHUNK_BUDGET_BYTES
    chunk = lmhead.default_token_chunk
    assert chunk(16384, 128256) == 4096 and chunk(16384, 256000) == 4096
    assert chunk(1000, 5000) == 256 and chunk(256, 1000) == 256 and chunk(100, 1000) == 100
    for n, v in ((65536, 256000), (1 << 20, 128256), (40000, 1000000)):
        c = chunk(n, v)
        assert c < n and c % 256 == 0 and 4 * c <= n + 1024
        assert 2 * v * c <= budget
    assert chunk(100000, 1 << 40) == 256  # at least one tile column
    buf = (ctypes.c_int64 * L.NMCE_LMHEAD_FUSED_LAYOUT_FIELDS)()
    # fields: total, chunk, n_chunks, ldt, vpad, nb, off_pt, off_part, off_acc, off_dxp,
    # dx_splits, off_xt
    assert lib.nmce_lmhead_ce_fused_layout(16384, 4096, 128256, 16384,
                                           ctypes.addressof(buf)) == 0
    assert (buf[1], buf[2]) == (16384, 1) and buf[8] == buf[9] == buf[11]  # no accumulator
    # P^T [vpad, ldt] bf16 is the one buffer of the vocabulary's and the chunk's
    # size; the chunk's hidden rows transposed, X_c^T [h, ldt], the only copy
    assert buf[7] - buf[6] == 128256 * 16384 * 2
    assert buf[0] - buf[11] == 4096 * 16384 * 2
    n, v = 65536, 256000
    assert lib.nmce_lmhead_ce_fused_layout(n, 3072, v, chunk(n, v), ctypes.addressof(buf)) == 0
    assert buf[2] > 1 and buf[9] - buf[8] >= v * 3072 * 4  # fp32 dW accumulator
    regions = [buf[6], buf[7], buf[8], buf[9], buf[11], buf[0]]
    assert all(r % 256 == 0 for r in regions) and regions == sorted(regions)


def test_fused_dx_split_choice(lib):
    """A chunk's dX product (tokens x H tiles, K = the padded vocabulary) is
    split over K when its 256x256 tiles leave compute units idle; the fp32
    partials region holds every range. On a device with 256 compute units (the
    choice depends on the current device; this host has none, so the query's
    fallback of 256 applies): 4096 tokens x 4096 fill one round unsplit,
    4096 x 3072 (192 tiles) take 4 ranges of 64000, 2048 x 3072 take 8."""
    import ctypes
    from nmce import _lib as L
    buf = (ctypes.c_int64 * L.NMCE_LMHEAD_FUSED_LAYOUT_FIELDS)()
    for n, h, v, ch, splits in ((16384, 4096, 128256, 4096, 1), (16384, 3072, 256000, 4096, 4),
                                (16384, 3072, 256000, 2048, 8), (16384, 3072, 256000, 16384, 1),
                                (300, 128, 777, 256, 1)):
        assert lib.nmce_lmhead_ce_fused_layout(n, h, v, ch, ctypes.addressof(buf)) == 0
        assert buf[10] == splits, (n, h, v, ch, buf[10])
        want = (splits * ch * h * 4 + 255) // 256 * 256 if splits > 1 else 0
        assert buf[11] - buf[9] == want


def test_validate_slots(lib):
    assert lib.nmce_validate_slots(0) == 0
    assert lib.nmce_validate_slots(1) == 1
    assert lib.nmce_validate_slots(1024) == 1
    assert lib.nmce_validate_slots(1025) == 2
    assert lib.nmce_validate_slots(16384) == 16


def test_dropin_has_no_cpu_path():
    import nmce
    x = torch.randn(2, 3, 8)
    t = torch.zeros(2, 3, dtype=torch.long)
    with pytest.raises(RuntimeError, match="no CPU path"):
        nmce.vocab_parallel_cross_entropy(x, t, 0, 8, nmce.ParallelContext.single())
    with pytest.raises(RuntimeError, match="no CPU path"):
        nmce._VocabParallelCrossEntropy.apply(x, t, 0, 8, None, 1)


def test_fused_dropin_has_no_cpu_path():
    import nmce
    x = torch.randn(4, 64).to(torch.bfloat16)
    w = torch.randn(10, 64).to(torch.bfloat16)
    t = torch.zeros(4, dtype=torch.long)
    with pytest.raises(RuntimeError, match="no CPU path"):
        nmce._LMHeadVocabParallelCrossEntropy.apply(x, w, t, 0, 10, None, 1)


def test_fused_lm_head_module_mirrors_parallel_lm_head():
    """FusedParallelLMHead(config, ctx) has ParallelLMHead's weight layout,
    initialisation and attributes (model.py:169-192); its logits path is the
    reference's plain product; the fused loss has no CPU path."""
    import types
    import nmce
    cfg = types.SimpleNamespace(vocab_size=1000, n_embd=64, sequence_parallel=False)
    torch.manual_seed(0)
    head = nmce.FusedParallelLMHead(cfg, nmce.ParallelContext.single())
    assert head.weight.shape == (1000, 64) and head.weight.dtype == torch.float32
    assert head.weight.tensor_parallel_sharded is True
    assert abs(float(head.weight.std()) - 0.02) < 2e-3
    assert head.vocab_range() == (0, 1000)
    x = torch.randn(2, 3, 64)
    assert torch.equal(head(x), x @ head.weight.t())
    labels = torch.zeros(2, 3, dtype=torch.long)
    with pytest.raises(RuntimeError, match="no CPU path"):
        head(x, labels)
    tp2 = nmce.ParallelContext(rank=1, world_size=2, tp_size=2, tp_rank=1, pp_size=1,
                               pp_rank=0, dp_size=1, dp_rank=0)
    assert nmce.FusedParallelLMHead(cfg, tp2).vocab_range() == (500, 1000)
    with pytest.raises(ValueError, match="not divisible"):
        nmce.FusedParallelLMHead(types.SimpleNamespace(vocab_size=1001, n_embd=8), tp2)


def test_parallel_context_and_shard_rule():
    import nmce
    ctx = nmce.ParallelContext.single()
    assert (ctx.tp_size, ctx.tp_rank, ctx.tp_group, ctx.world_size) == (1, 0, None, 1)
    assert nmce.vocab_range(128256, 2, 1) == (64128, 128256)
    assert nmce.vocab_range(50304, 1, 0) == (0, 50304)
    assert nmce.divide(12, 4) == 3
    with pytest.raises(ValueError, match="not divisible"):
        nmce.vocab_range(10, 3, 0)


def test_product_never_imports_the_oracle():
    """The shipped package must not reach the CPU oracle in any form."""
    for path in PKG.glob("*.py"):
        tree = ast.parse(path.read_text())
        for node in ast.walk(tree):
            if isinstance(node, ast.Import):
                mods = [a.name for a in node.names]
            elif isinstance(node, ast.ImportFrom):
                mods = [node.module or ""]
            else:
                continue
            for m in mods:
                assert not m.split(".")[0] == "oracle", f"{path.name} imports {m}"


def test_one_pass_route_edges(lib):
    """Which rows the wrapper hands to the one-pass kernel: TP = 1, fp32 or
    bf16, a width of whole 16-byte vectors up to the kernel's limit (131072
    bf16, 65536 fp32 columns), 16-byte aligned rows. One vector past the
    limit, a ragged width, an unaligned row stride, TP > 1, fp16 and an empty
    batch take the two-pass path. Host-side only (CPU tensors)."""
    from nmce import cross_entropy as ce
    from nmce import _lib as L
    assert lib.nmce_ce_fwd_bwd_max_vocab(L.NMCE_BF16) == 131072
    assert lib.nmce_ce_fwd_bwd_max_vocab(L.NMCE_F32) == 65536
    take = ce._one_pass_rows
    assert take(torch.zeros(2, 131072, dtype=torch.bfloat16), 1) is not None
    assert take(torch.zeros(2, 131080, dtype=torch.bfloat16), 1) is None
    assert take(torch.zeros(2, 65536), 1) is not None
    assert take(torch.zeros(2, 65540), 1) is None
    assert take(torch.zeros(3, 4, 1000, dtype=torch.bfloat16), 1) is not None
    assert take(torch.zeros(2, 1001, dtype=torch.bfloat16), 1) is None  # not whole vectors
    assert take(torch.zeros(2, 1009, dtype=torch.bfloat16)[:, :1008], 1) is None  # row stride
    assert take(torch.zeros(2, 1000, dtype=torch.bfloat16), 2) is None  # TP > 1
    assert take(torch.zeros(2, 1000, dtype=torch.float16), 1) is None
    assert take(torch.zeros(0, 1000, dtype=torch.bfloat16), 1) is None


def test_wide_buffer_stores_go_through_the_helper():
    """Buffer stores wider than 8 bytes are issued only by buffer_store_b128,
    which keeps the scalar offset the constant 0: with a register scalar
    offset the compiler omits the wait state a VALU write of the store's data
    registers needs right after the store."""
    import re
    csrc = ROOT / "nano-megatron_amd" / "csrc"
    pattern = re.compile(r"__builtin_amdgcn_raw_buffer_store_b(96|128)\b")
    for path in sorted(csrc.glob("*.hip")) + sorted(csrc.glob("*.h")):
        for i, line in enumerate(path.read_text().splitlines(), 1):
            if pattern.search(line):
                assert path.name == "nmce_device.h", f"{path.name}:{i}: {line.strip()}"
    helper = (csrc / "nmce_device.h").read_text()
    assert "__builtin_amdgcn_raw_buffer_store_b128(v, r, voff, 0, kAux)" in helper


def test_bench_refuses_more_than_one_gpu():
    """bench.py runs on exactly one GPU: --gpus 2 exits with status 2 and says why."""
    import subprocess
    import sys
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2
    assert "exactly one GPU" in r.stdout


def test_bench_summary_fits_the_end_of_the_line():
    """The default line ends with one row per configuration; with realistic
    figures the rows stay inside the last 1.5 KB of the line, so a reader that
    keeps only the end of the output still sees every configuration."""
    import importlib.util
    import json
    spec = importlib.util.spec_from_file_location("bench_under_test", ROOT / "bench.py")
    bench = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(bench)

    def result(kernel, frac):
        return {"value": 12345678.9, "ms_per_step": 0.123456, "config": {"workload": "w"},
                "roofline": {"bound": "hbm", "kernel": kernel, "achieved": 6000.1,
                             "peak": 8000.0, "unit": "GB/s", "frac": frac,
                             "traffic": 34219982819},
                "step_frac": 0.7,
                "cpu_baseline": {"value": 1234567.8, "unit": "tokens/s", "cores": 16,
                                 "kind": "port", "sample": "s" * 80}}
    out = {"metric": bench.METRIC, **result("nmce_ce_fwd_bwd", 0.759)}
    for key, _, _ in bench.NESTED:
        out[key] = result("nmce_lmhead_ce_fused_chunk_grads", 0.4633)
    out["summary"] = bench._summary(out)
    line = json.dumps(bench._round(out), separators=(",", ":"))
    tail = line[line.index('"summary"'):]
    assert len(tail) < 1500, len(tail)
    back = json.loads(line)["summary"]
    assert list(back) == ["cols", "c2"] + [k for k, _, _ in bench.NESTED]
    for key in back:
        if key != "cols":
            row = dict(zip(back["cols"], back[key]))
            assert row["roofline.frac"] in (0.759, 0.4633)
            assert row["cpu_baseline.value"] == 1235000.0 and row["cpu_baseline.cores"] == 16
