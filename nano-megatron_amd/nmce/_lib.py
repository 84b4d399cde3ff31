"""ctypes binding of ``libnmce.so`` (declared in ``include/nmce.h``).

The library is loaded after ``import torch`` so that its ``libamdhip64.so.7``
dependency resolves to the HIP runtime torch already mapped: both then share
one runtime, one device context and torch's streams.

There is no fallback: if the library is missing or a call fails, the caller
gets an exception.
"""

from __future__ import annotations

import ctypes
import pathlib
import threading

import torch  # noqa: F401  (must be imported before the HIP library is loaded)

LIB_PATH = pathlib.Path(__file__).resolve().parent / "libnmce.so"

NMCE_F32 = 0
NMCE_BF16 = 1
NMCE_VALIDATE_ROWS_PER_SLOT = 1024

_c_int = ctypes.c_int
_i64 = ctypes.c_int64
_p = ctypes.c_void_p

# name -> (restype, argtypes), mirroring include/nmce.h
SIGNATURES: dict[str, tuple] = {
    "nmce_status_string": (ctypes.c_char_p, [_c_int]),
    "nmce_version": (_c_int, []),
    "nmce_ce_fwd_stats": (_c_int, [_p, _c_int, _i64, _i64, _i64, _p, _i64, _p, _p, _p, _p]),
    "nmce_ce_fwd": (_c_int, [_p, _c_int, _i64, _i64, _i64, _p, _p, _p, _p, _p]),
    "nmce_ce_combine": (_c_int, [_p, _p, _p, _c_int, _i64, _i64, _p, _p, _p, _p]),
    "nmce_validate_slots": (_i64, [_i64]),
    "nmce_validate_targets": (_c_int, [_p, _i64, _i64, _p, _p]),
    "nmce_validate_targets_once": (_c_int, [_p, _i64, _i64, _p, _p, _p]),
    "nmce_stream_copy": (_c_int, [_p, _p, _i64, _p]),
    "nmce_ce_bwd": (_c_int, [_p, _p, _c_int, _i64, _i64, _i64, _i64, _p, _i64, _p, _p, _p, _i64, _p]),
    "nmce_ce_bwd_scaled": (_c_int, [_p, _p, _c_int, _i64, _i64, _i64, _i64, _p, _i64, _p, _p, _p, _i64,
                                    ctypes.c_float, _p]),
    "nmce_ce_bwd_scaled_unless": (_c_int, [_p, _p, _c_int, _i64, _i64, _i64, _i64, _p, _i64, _p,
                                           _p, _p, ctypes.c_float, _p, _p, _p]),
    "nmce_ce_fwd_bwd_max_vocab": (_i64, [_c_int]),
    "nmce_ce_fwd_bwd": (_c_int, [_p, _p, _c_int, _i64, _i64, _i64, _i64, _p, _p, _p, _p, _p, _p,
                                 _p, ctypes.c_float, _p]),
    "nmce_ce_grad_rescale_unless": (_c_int, [_p, _c_int, _i64, _i64, _i64, _p, _p, _p, _p]),
    "nmce_lmhead_ce_fwd_workspace_bytes": (_i64, [_i64, _i64, _i64]),
    "nmce_lmhead_ce_fwd_stats": (_c_int, [_p, _p, _c_int, _i64, _i64, _i64, _p, _i64, _p, _p, _p,
                                          _p, _i64, _p]),
    "nmce_lmhead_ce_fwd_stats_noalloc": (_c_int, [_p, _p, _c_int, _i64, _i64, _i64, _p, _i64, _p,
                                                  _p, _p, _p]),
    "nmce_lmhead_ce_bwd_workspace_bytes": (_i64, [_i64, _i64, _i64, _i64]),
    "nmce_lmhead_ce_bwd": (_c_int, [_p, _p, _c_int, _i64, _i64, _i64, _p, _i64, _p, _p, _p, _i64,
                                    _p, _p, _i64, _p, _i64, _p]),
    "nmce_lmhead_ce_fused_layout": (_c_int, [_i64, _i64, _i64, _i64, _p]),
    "nmce_hint_assume": (_c_int, [_p, _p, _p]),
    "nmce_lmhead_ce_fused_chunk_stats": (_c_int, [_p, _p, _c_int, _i64, _i64, _i64, _p, _i64,
                                                  _i64, _i64, _p, _p, _p, _p, _i64, _p]),
    "nmce_lmhead_ce_fused_chunk_grads": (_c_int, [_p, _p, _c_int, _i64, _i64, _i64, _p, _i64,
                                                  _i64, _i64, _p, _p, _p, _p, _i64,
                                                  ctypes.c_float, _p, _p, _p, _i64, _p]),
    "nmce_gemm_nt_bf16": (_c_int, [_p, _i64, _p, _i64, _i64, _i64, _i64, _p, _c_int, _i64, _p]),
    "nmce_gemm_mn_bf16": (_c_int, [_c_int, _p, _i64, _p, _i64, _i64, _i64, _i64, _p, _i64, _p]),
    "nmce_lmhead_ce_bwd_layout": (_c_int, [_i64, _i64, _i64, _i64, _p]),
    "nmce_lmhead_ce_bwd_prepare": (_c_int, [_p, _p, _c_int, _i64, _i64, _i64, _i64, _p, _i64, _p]),
    "nmce_lmhead_ce_bwd_dz": (_c_int, [_p, _p, _c_int, _i64, _i64, _i64, _p, _i64, _p, _p, _p,
                                       _i64, _i64, _i64, _p, _i64, _p]),
}

NMCE_LMHEAD_LAYOUT_FIELDS = 10
NMCE_LMHEAD_FUSED_LAYOUT_FIELDS = 12

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


class NmceError(RuntimeError):
    """A libnmce entry point returned a nonzero status."""


def load() -> ctypes.CDLL:
    """Load and type the library once per process."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise NmceError(
                    f"{LIB_PATH} is not built; run `python -m nmce._build` in "
                    "nano-megatron_amd/ (or __graft_entry__.build())"
                )
            lib = ctypes.CDLL(str(LIB_PATH))
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            _lib = lib
    return _lib


_ext = None


def autograd_ext():
    """The ``_nmce_autograd`` extension (the one-pass loss's autograd node,
    built beside ``libnmce.so`` and linked against it), imported once."""
    global _ext
    if _ext is None:
        load()  # libnmce.so first, from this package's directory
        try:
            from . import _nmce_autograd
        except ImportError as e:
            raise NmceError(
                f"the _nmce_autograd extension is not built next to {LIB_PATH} ({e}); run "
                "`python -m nmce._build` in nano-megatron_amd/ (or __graft_entry__.build())"
            ) from e
        _ext = _nmce_autograd
    return _ext


def check(status: int, what: str) -> None:
    if status != 0:
        msg = load().nmce_status_string(status).decode()
        raise NmceError(f"{what} failed with status {status}: {msg}")


def dtype_code(dtype: torch.dtype) -> int:
    if dtype == torch.float32:
        return NMCE_F32
    if dtype == torch.bfloat16:
        return NMCE_BF16
    raise TypeError(f"unsupported logits dtype {dtype}; expected float32 or bfloat16")


# torch's raw-stream query (what its compiled kernels' launchers call): a
# fraction of the cost of building a Stream object per launch, which matters
# for small batches, where a step is a few microseconds of GPU work.
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_handle(device: torch.device) -> int:
    """The raw hipStream_t of torch's current stream on ``device``."""
    if _raw_stream is not None:
        idx = device.index if device.index is not None else torch.cuda.current_device()
        return _raw_stream(idx)
    return torch.cuda.current_stream(device).cuda_stream

