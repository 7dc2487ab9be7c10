"""ctypes binding of libinnerq_hip.so (the C ABI in include/innerq_abi.h).

Loading fails loudly when the library has not been built: there is no CPU
fallback anywhere in the product path.
"""
from __future__ import annotations

import ctypes
import os
import threading

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libinnerq_hip.so")

IQ_OK = 0
IQ_MODE_ASYM = 0
IQ_MODE_SYM = 1
IQ_MODE_HYBRID = 2
IQ_MODE_BF16 = 0x100  # OR-ed into a mode: bf16 activations
ABI_VERSION = 3
TOKEN_BLOCK = 64

STATUS = {
    0: "IQ_OK", -1: "IQ_ERR_NULL", -2: "IQ_ERR_BITS", -3: "IQ_ERR_GROUP", -4: "IQ_ERR_SHAPE",
    -5: "IQ_ERR_ALIGN", -6: "IQ_ERR_WORKSPACE", -7: "IQ_ERR_MODE", -8: "IQ_ERR_RANGE", -9: "IQ_ERR_HIP",
}


class IQError(RuntimeError):
    """A C-ABI entry point returned a negative status."""

    def __init__(self, fn: str, status: int):
        self.status = status
        super().__init__(f"{fn} failed: {STATUS.get(status, status)} ({strerror(status)})")


class iq_segment(ctypes.Structure):
    _fields_ = [
        ("dense", ctypes.c_void_p),
        ("s_b", ctypes.c_int64), ("s_h", ctypes.c_int64), ("s_t", ctypes.c_int64),
        ("n", ctypes.c_int),
        ("codes", ctypes.c_void_p),
        ("meta", ctypes.c_void_p),
        ("t_cap", ctypes.c_int64),
        ("t0", ctypes.c_int),
        ("bits", ctypes.c_int), ("group", ctypes.c_int), ("mode", ctypes.c_int),
    ]


P = ctypes.c_void_p
I = ctypes.c_int
L = ctypes.c_int64
F = ctypes.c_float
S = ctypes.c_size_t

class iq_window(ctypes.Structure):
    _fields_ = [
        ("buf", ctypes.c_void_p),
        ("s_b", ctypes.c_int64), ("s_h", ctypes.c_int64), ("s_t", ctypes.c_int64),
        ("cap", ctypes.c_int), ("start", ctypes.c_int), ("n", ctypes.c_int),
        ("x", ctypes.c_void_p),
        ("sx_b", ctypes.c_int64), ("sx_h", ctypes.c_int64), ("sx_t", ctypes.c_int64),
        ("m", ctypes.c_int), ("flush", ctypes.c_int),
        ("codes", ctypes.c_void_p), ("meta", ctypes.c_void_p),
        ("t_cap", ctypes.c_int64), ("t_off", ctypes.c_int64),
        ("bits", ctypes.c_int), ("group", ctypes.c_int), ("mode", ctypes.c_int), ("axis", ctypes.c_int),
        ("norm", ctypes.c_void_p),
        ("deq_rows", ctypes.c_int),
    ]


class iq_split_plan(ctypes.Structure):
    _fields_ = [("nsplit", ctypes.c_int), ("nsf", ctypes.c_int), ("grid", ctypes.c_int), ("nrep", ctypes.c_int),
                ("pair_e0", ctypes.c_int), ("bf16", ctypes.c_int), ("reserved", ctypes.c_int * 2)]


SIGNATURES = {
    "iq_abi_version": (I, []),
    "iq_strerror": (ctypes.c_char_p, [I]),
    "iq_k_store_bytes": (I, [L, L, L, L, I, I, I, ctypes.POINTER(L), ctypes.POINTER(L)]),
    "iq_v_store_bytes": (I, [L, L, L, L, I, I, I, ctypes.POINTER(L), ctypes.POINTER(L)]),
    "iq_quantize_k": (I, [P, L, L, L, P, I, I, I, I, I, I, I, P, P, L, L, P, P, P, P, P]),
    "iq_quantize_v": (I, [P, L, L, L, I, I, I, I, I, I, I, P, P, L, L, P, P, P, P, P]),
    "iq_dequant_k": (I, [P, P, L, P, I, I, I, I, I, I, I, I, P, P, L, L, L, P]),
    "iq_dequant_v": (I, [P, P, L, I, I, I, I, I, I, I, I, P, P, L, L, L, P]),
    "iq_dequant_dense": (I, [P, P, P, L, L, L, I, I, I, P, P]),
    "iq_unpack_k": (I, [P, P, L, I, I, I, I, I, I, I, I, P, P, P, P]),
    "iq_unpack_v": (I, [P, P, L, I, I, I, I, I, I, I, I, P, P, P, P]),
    "iq_key_norm_factor": (I, [P, L, L, L, I, I, I, I, I, P, P]),
    "iq_hybrid_mask": (I, [P, P, P, P, L, I, I, I, I, I, P, P]),
    "iq_hybrid_select": (I, [P, P, P, L, I, I, I, I, I, P, P]),
    "iq_qk_gemv": (I, [P, L, L, P, P, P, L, I, I, I, I, I, I, I, I, I, F, P, L, L, P, S, P]),
    "iq_qk_workspace_bytes": (S, [I, I, I]),
    "iq_av_workspace_bytes": (S, [I, I, I, I, I]),
    "iq_av_gemv": (I, [P, L, L, P, P, L, I, I, I, I, I, I, I, I, I, P, P, L, L, I, P, S, P]),
    "iq_decode_workspace_bytes": (S, [I, I, I, I]),
    "iq_window_append": (I, [ctypes.POINTER(iq_window), ctypes.POINTER(iq_window), I, I, I, P]),
    "iq_decode_attention": (I, [P, L, L, P, ctypes.POINTER(iq_segment), ctypes.POINTER(iq_segment),
                                I, I, I, I, I, F, P, L, L, P, S, P]),
    "iq_decode_attention_splits": (I, [P, L, L, P, ctypes.POINTER(iq_segment), ctypes.POINTER(iq_segment),
                                       I, I, I, I, I, F, P, S, ctypes.POINTER(I), P]),
    "iq_decode_attention_combine": (I, [I, I, I, I, I, P, L, L, P, S, P]),
    "iq_decode_attention_splits_live": (I, [P, L, L, P, ctypes.POINTER(iq_segment), ctypes.POINTER(iq_segment),
                                            I, I, I, I, I, F, P, S, ctypes.POINTER(iq_split_plan), P]),
    "iq_decode_attention_combine_live": (I, [ctypes.POINTER(iq_split_plan), I, I, I, I, P, L, L, P, S, P]),
    "iq_decode_noalloc_max_bytes": (S, []),
    "iq_decode_attention_noalloc": (I, [P, L, L, P, ctypes.POINTER(iq_segment), ctypes.POINTER(iq_segment),
                                        I, I, I, I, I, F, P, L, L, P]),
}

_lib = None
_lock = threading.Lock()


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        with _lock:
            if _lib is None:
                if not os.path.exists(LIB_PATH):
                    raise RuntimeError(
                        f"{LIB_PATH} is missing: build it with `python -m innerq_amd.build` "
                        "(innerq_amd has no CPU fallback)")
                h = ctypes.CDLL(LIB_PATH)
                for name, (res, args) in SIGNATURES.items():
                    f = getattr(h, name)
                    f.restype = res
                    f.argtypes = args
                if h.iq_abi_version() != ABI_VERSION:
                    raise RuntimeError("libinnerq_hip.so ABI version mismatch")
                _lib = h
    return _lib


def strerror(status: int) -> str:
    try:
        return lib().iq_strerror(status).decode()
    except Exception:  # library not loadable
        return STATUS.get(status, "unknown")


def call(name: str, *args) -> int:
    st = getattr(lib(), name)(*args)
    if isinstance(st, int) and st < 0:
        raise IQError(name, st)
    return st
