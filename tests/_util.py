"""Shared helpers for the test-suite (not collected by pytest)."""

from __future__ import annotations

import ctypes
import hashlib
import json
import pathlib

import numpy as np
import torch

GOLDEN = pathlib.Path(__file__).resolve().parent / "golden"

ULP_BF16 = 2.0 ** -8  # spacing of bf16 values in [1, 2)


def load_npz(name: str) -> dict:
    with np.load(GOLDEN / name, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def load_json(name: str) -> dict:
    return json.loads((GOLDEN / name).read_text())


def sha256_of(*tensors: torch.Tensor) -> str:
    h = hashlib.sha256()
    for t in tensors:
        h.update(t.contiguous().cpu().numpy().tobytes())
    return h.hexdigest()


def c1_inputs():
    """c1 = fp32 [4,256,32000] ~ N(0, 2^2), targets U[0,32000), CPU generator seed 0."""
    g = torch.Generator().manual_seed(0)
    logits = torch.randn(4, 256, 32000, generator=g) * 2.0
    target = torch.randint(0, 32000, (4, 256), generator=g)
    return logits, target


def header_functions() -> list[str]:
    """Names of the functions declared in include/nmce.h."""
    import re
    text = (pathlib.Path(__file__).resolve().parent.parent / "include" / "nmce.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(nmce_\w+)\s*\(", text)))


def assert_close_rel(actual, expected, rtol, atol=0.0, what=""):
    a = np.asarray(actual, dtype=np.float64)
    e = np.asarray(expected, dtype=np.float64)
    err = np.abs(a - e)
    bound = atol + rtol * np.abs(e)
    bad = ~(err <= bound)
    if bad.any():
        i = np.flatnonzero(bad.ravel())[0]
        raise AssertionError(
            f"{what}: {int(bad.sum())} of {a.size} outside rtol={rtol} atol={atol}; first at flat "
            f"{i}: got {a.ravel()[i]!r} expected {e.ravel()[i]!r}; max abs err {err.max():.3e}")


def assert_bf16_close(actual_bf16: np.ndarray, expected: np.ndarray, what="", ulps=1.0,
                      atol=0.0):
    """bf16 values within ``ulps`` bf16 ulps (relative 2^-8) of ``expected``."""
    assert_close_rel(actual_bf16, expected, rtol=ulps * ULP_BF16, atol=atol, what=what)
