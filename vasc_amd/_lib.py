"""ctypes binding of ``libvasc_hip.so`` (declared in ``include/vasc_hip.h``).

There is no CPU fallback: every operator of this package runs the HIP
kernels or raises. ``load()`` raises ``RuntimeError`` when the library has
not been built (``python -m vasc_amd.build``).
"""
from __future__ import annotations

import ctypes
import threading
from ctypes import c_float, c_int32, c_int64, c_size_t, c_void_p
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libvasc_hip.so"

VASC_OK = 0
MODE_TOPK = 0
MODE_VASC = 1
WS_ROW_TOTAL = 0
WS_ROW_PAIR_SUM = 1
WS_ROW_CAPACITY = 2
WS_ADMITTED_DEBT = 3

P = c_void_p
I64 = c_int64
I32 = c_int32

# name -> (restype, argtypes); mirrors include/vasc_hip.h and include/vasc_runner.h.
SIGNATURES: dict[str, tuple] = {
    "vasc_last_error": (ctypes.c_char_p, []),
    "vasc_abi_version": (c_int32, []),
    "vasc_pool_qk_max": (c_int32, [P, I64, I64, I64, P, I64, I64, I64, I64, I64, I64, I64, I64, I64, I64,
                                  P, P, P]),
    "vasc_pool_qkv": (c_int32, [P, I64, I64, I64, P, I64, I64, I64, P, I64, I64, I64,
                                I64, I64, I64, I64, I64, I64, I64, P, P, P, P, P]),
    "vasc_pooled_softmax": (c_int32, [P, P, I64, I64, I64, I64, I64, c_float, I32, P, P, P, P]),
    "vasc_pooled_softmax_workspace_size": (I64, [I64, I64, I64, I64]),
    "vasc_pair_innovation": (c_int32, [P, I64, I64, I64, I64, P, P]),
    "vasc_select_workspace_size": (c_size_t, [I64, I64, I64, I64]),
    "vasc_select_workspace_offset": (I64, [I64, I64, I64, I64, I32]),
    "vasc_select_blocks": (c_int32, [P, P, I64, I64, I64, I64, I32, I32, P, P, I32, I32, I32,
                                     P, P, P, P, P, P, P, P, P, P, I64, P, P, c_size_t, P]),
    "vasc_select_blocks_noalloc": (c_int32, [P, P, I64, I64, I64, I64, I32, I32, P, P, I32, I32, I32,
                                             P, P, P, P, P, P, P, P, P, P, I64, P, P]),
    "vasc_settle_terminal": (c_int32, [P, P, P, I64, P, P]),
    "vasc_cdf_counts": (c_int32, [P, I64, I64, I64, I64, P, I32, I32, P, P, P]),
    "vasc_priority_order": (c_int32, [P, P, P, I64, I32, I64, I64, I64, P, P]),
    "vasc_packed_v_elems": (c_int64, [I64, I64, I64, I64]),
    "vasc_pack_v": (c_int32, [P, I64, I64, I64, I64, I64, I64, I64, P, P]),
    "vasc_block_sparse_attn_fwd": (c_int32, [P, I64, I64, I64, P, I64, I64, I64, P, P, I64, I64, I64,
                                             I64, I64, I64, I64, I64, P, I64, P, I32, c_float, P]),
    "vasc_block_sparse_attn_pv_fwd": (c_int32, [P, I64, I64, I64, P, I64, I64, I64, P, P, I64, I64, I64,
                                                I64, I64, I64, I64, I64, P, I64, P, I32, c_float, P, P, P]),
    "vasc_dense_attn_fwd": (c_int32, [P, I64, I64, I64, P, I64, I64, I64, P, P, I64, I64, I64,
                                      I64, I64, I64, I64, I64, c_float, P]),
    "vasc_global_attn_fwd": (c_int32, [P, I64, I64, I64, P, I64, I64, I64, P, I64, I64, I64, P,
                                       P, I64, I64, I64, P, I64, I64, I64, I64, I64, I64, I64, I64, I64,
                                       P, I64, P, c_float, P]),
    "vasc_global_attn_tokens_fwd": (c_int32, [P, I64, I64, I64, P, I64, I64, I64, P, I64, I64, I64, P, P,
                                              I64, I64, I64, I64, I64, I64, I64, P, I64, P, c_float, P]),
    "vasc_pack_qkv": (c_int32, [P, I64, I64, I64, P, I64, I64, I64, P, I64, I64, I64,
                                I64, I64, I64, I64, I64, I64, P, P, c_float, I32, P, P, c_float, I32,
                                P, I64, I64, P, P, I64, P, P, P, P, P]),
    "vasc_pack_global": (c_int32, [P, I64, I64, I64, P, I64, I64, I64, P, I64, I64, I64,
                                   I64, I64, I64, I64, I64, I64, P, P, c_float, I32, P, P, c_float, I32,
                                   P, I64, I64, P, P, I64, P, P, P, P, P, P, P, P, P]),
    "vasc_restore_tokens": (c_int32, [P, I64, I64, I64, P, I64, I64, I64, I64, I64, I64, I64, I64, I64,
                                      P, P]),
    # include/vasc_runner.h
    "vasc_residual_norm": (c_int32, [P, I64, P, I64, P, P, P, c_float, P, I64, P, I64, I64, I64, P]),
}

_lock = threading.Lock()
_lib = None


def load() -> ctypes.CDLL:
    """Load and type the library once; raises if it is missing."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise RuntimeError(
                    f"{LIB_PATH} is not built; run `python -m vasc_amd.build` "
                    "(the HIP kernels have no CPU fallback)")
            lib = ctypes.CDLL(str(LIB_PATH))
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            _lib = lib
    return _lib


class VascError(RuntimeError):
    """A non-zero status from libvasc_hip.so."""


class VascArgumentError(VascError, ValueError):
    """Status VASC_ERR_ARGUMENT."""


def call(name: str, *args) -> None:
    """Call an int-status entry point and raise on failure."""
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc != VASC_OK:
        msg = lib.vasc_last_error().decode(errors="replace")
        if rc == 1:
            raise VascArgumentError(f"{name}: {msg}")
        raise VascError(f"{name} failed ({rc}): {msg}")


def fn(name: str):
    return getattr(load(), name)
