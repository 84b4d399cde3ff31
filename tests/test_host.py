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
    assert lib.nmce_validate_targets(p, 4, 0, p, None) == -2
    assert lib.nmce_validate_targets(None, 4, 10, p, None) == -4


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
