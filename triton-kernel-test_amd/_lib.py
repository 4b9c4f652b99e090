"""ctypes binding of liblrq.so (the HIP kernels behind the C ABI in include/lrq.h).

There is no fallback: if the library is missing or fails to load, every entry point
raises.  Build it with ``python triton-kernel-test_amd/build.py`` (or
``__graft_entry__.build()``).
"""

from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, c_float, c_int32, c_int64, c_size_t, c_void_p
from pathlib import Path

LIB_PATH = Path(os.environ.get("LRQ_LIBRARY", Path(__file__).resolve().parent / "liblrq.so"))

LRQ_OK = 0
LRQ_ERR_NULL = -1
LRQ_ERR_SHAPE = -2
LRQ_ERR_UNSUPPORTED = -3
LRQ_ERR_ALIGN = -4
LRQ_ERR_WORKSPACE = -5
LRQ_FLAG_HADAMARD = 1
LRQ_GEMM_T_SCRATCH_BYTES = 16 * 1024 * 1024  # include/lrq.h


class LrqTensors(ctypes.Structure):
    """Mirror of ``lrq_tensors`` in include/lrq.h."""

    _fields_ = [
        ("rows", c_int64), ("hidden", c_int64),
        ("rank", c_int32), ("bits", c_int32), ("group", c_int32), ("flags", c_int32),
        ("L", c_void_p), ("ld_L", c_int64),
        ("V", c_void_p), ("Vt", c_void_p),
        ("codes", c_void_p), ("ld_codes", c_int64),
        ("qparams", c_void_p), ("ld_qp", c_int64),
        ("outlier_idx", c_void_p), ("n_outlier", c_int32),
        ("side", c_void_p), ("ld_side", c_int64),
    ]


_T = POINTER(LrqTensors)

# name -> (restype, argtypes); must cover every function declared in include/*.h (the drop-in
# ABI in lrq.h and the test hooks in lrq_test_hooks.h)
SIGNATURES = {
    "lrq_encode": (c_int32, [_T, c_void_p, c_int64, c_void_p]),
    "lrq_encode_twopass": (c_int32, [_T, c_void_p, c_int64, c_void_p]),
    "lrq_decode": (c_int32, [_T, c_void_p, c_int64, c_void_p]),
    "lrq_silu_bwd": (c_int32, [_T, c_void_p, c_int64, c_void_p, c_int64, c_void_p]),
    "lrq_gelu_bwd": (c_int32, [_T, c_void_p, c_int64, c_void_p, c_int64, c_void_p]),
    "lrq_mul": (c_int32, [_T, c_void_p, c_int64, c_void_p, c_int64, c_void_p]),
    "lrq_softmax_bwd": (c_int32, [_T, c_void_p, c_int64, c_void_p, c_int64, c_void_p]),
    "lrq_dequant_gemm": (c_int32, [_T, c_void_p, c_int32, c_void_p, c_int64, c_int32, c_void_p]),
    "lrq_dequant_gemm_t": (c_int32, [_T, c_void_p, c_int64, c_int32, c_void_p, c_int64, c_int32, c_void_p,
                                     c_int64, c_void_p]),
    "lrq_dequant_gemm_t_workspace": (c_int64, [_T, c_int32]),
    "lrq_lora_grads": (c_int32, [_T, c_void_p, c_int64, c_void_p, c_int64, c_int32, c_void_p, c_int64, c_int32,
                                 c_void_p, c_int64, c_int32, c_void_p, c_int64, c_void_p]),
    "lrq_lora_grads_workspace": (c_int64, [_T, c_int32]),
    "lrq_dequant_gemm_t_noalloc": (c_int32, [_T, c_void_p, c_int64, c_int32, c_void_p, c_int64, c_int32, c_void_p]),
    "lrq_colmax": (c_int32, [c_void_p, c_int64, c_int64, c_int64, c_void_p, c_void_p]),
    "lrq_topk": (c_int32, [c_void_p, c_int64, c_int32, c_void_p, c_void_p]),
    "lrq_transpose_bf16": (c_int32, [c_void_p, c_int64, c_int64, c_void_p, c_void_p]),
    "lrq_wht128": (c_int32, [c_void_p, c_int64, c_int64, c_int64, c_void_p, c_int64, c_void_p]),
    "lrq_legacy_encode": (c_int32, [c_void_p, c_void_p, c_int32, c_void_p, c_int64, c_int64, c_int64,
                                    c_int64, c_int64, c_void_p, c_int64, c_int32, c_float, c_void_p,
                                    c_void_p, c_void_p]),
    "lrq_legacy_decode": (c_int32, [c_void_p, c_void_p, c_int32, c_void_p, c_void_p, c_void_p, c_int64,
                                    c_int64, c_int64, c_int64, c_int32, c_void_p, c_void_p]),
    "lrq_legacy_fused": (c_int32, [c_void_p, c_void_p, c_int32, c_void_p, c_void_p, c_int64, c_int64,
                                   c_int64, c_int64, c_int32, c_int32, c_void_p, c_void_p, c_void_p]),
    "lrq_legacy_dequant_gemm": (c_int32, [c_void_p, c_void_p, c_int32, c_void_p, c_void_p, c_int64, c_int64,
                                          c_int64, c_int64, c_int32, c_void_p, c_int64, c_int32, c_void_p, c_int64,
                                          c_void_p]),
    "lrq_coo_compact": (c_int32, [c_void_p, c_int64, c_int64, c_int64, c_void_p, c_int64, c_void_p, c_int64,
                                  c_void_p, c_void_p, c_void_p, c_int64, c_void_p]),
    "lrq_coo_workspace": (c_int64, [c_int64, c_int64, c_int64]),
    "lrq_legacy_encode_coo": (c_int32, [c_void_p, c_void_p, c_int32, c_void_p, c_int64, c_int64, c_int64,
                                        c_int64, c_int64, c_void_p, c_int64, c_int32, c_float, c_void_p,
                                        c_void_p, c_void_p, c_int64, c_void_p, c_int64, c_void_p, c_void_p,
                                        c_void_p, c_int64, c_void_p]),
    "lrq_legacy_decode_coo": (c_int32, [c_void_p, c_void_p, c_int32, c_void_p, c_void_p, c_void_p, c_void_p,
                                        c_int64, c_void_p, c_int64, c_int64, c_int64, c_int64, c_int32, c_void_p,
                                        c_void_p]),
    "lrq_legacy_kth_residual": (c_int32, [c_void_p, c_void_p, c_int32, c_void_p, c_int64, c_int64, c_int64,
                                          c_int64, c_void_p, c_void_p, c_int64, c_void_p]),
    "lrq_lowrank_add": (c_int32, [c_void_p, c_void_p, c_int32, c_void_p, c_int64, c_int64, c_int64,
                                  c_void_p, c_void_p]),
    "lrq_dense_elementwise": (c_int32, [c_int32, c_void_p, c_void_p, c_void_p, c_int64, c_void_p]),
    "lrq_dense_softmax_bwd": (c_int32, [c_void_p, c_void_p, c_void_p, c_int64, c_int64, c_void_p]),
    "lrq_threshold_split": (c_int32, [c_void_p, c_int64, c_float, c_void_p, c_void_p, c_void_p]),
    "lrq_gather_rows_zero": (c_int32, [c_void_p, c_int64, c_int64, c_int64, c_void_p, c_int32, c_void_p,
                                       c_void_p]),
    "lrq_status_string": (ctypes.c_char_p, [c_int32]),
    "lrq_abi_version": (c_int32, []),
}

_lib = None
_missing: set[str] = set()


def load():
    """Load liblrq.so once and bind every known symbol; raise if the library is absent."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise RuntimeError(
            f"liblrq.so not found at {LIB_PATH}; build it with `python triton-kernel-test_amd/build.py` "
            "(there is no CPU fallback for this path)")
    lib = ctypes.CDLL(str(LIB_PATH))
    for name, (res, args) in SIGNATURES.items():
        try:
            fn = getattr(lib, name)
        except AttributeError:
            _missing.add(name)
            continue
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def missing_symbols() -> set[str]:
    load()
    return set(_missing)


def status_string(code: int) -> str:
    return load().lrq_status_string(int(code)).decode()


def check(code: int, what: str) -> None:
    """Map a non-zero status to an exception (ValueError for argument errors)."""
    if code == LRQ_OK:
        return
    msg = f"{what}: {status_string(code)} (status {code})"
    if code < 0:
        raise ValueError(msg)
    raise RuntimeError(msg)


def call_raw(name: str, *args) -> int:
    """Call an entry point and return its status without raising."""
    lib = load()
    if name in _missing:
        raise RuntimeError(f"{name} is not exported by {LIB_PATH}")
    return int(getattr(lib, name)(*args))


def call(name: str, *args) -> None:
    check(call_raw(name, *args), name)


__all__ = ["LrqTensors", "load", "call", "call_raw", "check", "status_string", "missing_symbols", "SIGNATURES",
           "LIB_PATH", "LRQ_FLAG_HADAMARD", "c_size_t"]
