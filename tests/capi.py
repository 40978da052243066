"""ctypes binding of include/turboquant_hip.h for tests (device pointers from torch)."""

from __future__ import annotations

import ctypes
import os
import re

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "turboquant_hip.h")
LIB = os.path.join(ROOT, "turboquant-kv_amd", "turboquant_kv", "_lib", "libturboquant_hip.so")

TQ_F32, TQ_F16, TQ_BF16 = 0, 1, 2

_lib = None


def lib():
    global _lib
    if _lib is None:
        _lib = ctypes.CDLL(LIB)
        _lib.tq_last_error.restype = ctypes.c_char_p
        for name in ("tq_scan_workspace_bytes", "tq_values_workspace_bytes",
                     "tq_decode_workspace_bytes", "tq_decode_dl_workspace_bytes"):
            getattr(_lib, name).restype = ctypes.c_size_t
        _lib.tq_decode_dl_workspace_bytes.argtypes = [ctypes.c_int32, ctypes.c_int32,
                                                      ctypes.c_int32, ctypes.c_int64]
        _lib.tq_scan_workspace_bytes.argtypes = [ctypes.c_int64, ctypes.c_int32, ctypes.c_int32,
                                                 ctypes.c_int64, ctypes.c_int32]
        _lib.tq_values_workspace_bytes.argtypes = [ctypes.c_int64, ctypes.c_int32, ctypes.c_int64]
        _lib.tq_scan_pairs_workspace_bytes.restype = ctypes.c_size_t
        _lib.tq_scan_pairs_workspace_bytes.argtypes = [ctypes.c_int64, ctypes.c_int32, ctypes.c_int64,
                                                       ctypes.c_int32]
        _lib.tq_scan_pair_rows_workspace_bytes.restype = ctypes.c_size_t
        _lib.tq_scan_pair_rows_workspace_bytes.argtypes = [ctypes.c_int64, ctypes.c_int32, ctypes.c_int32,
                                                           ctypes.c_int64, ctypes.c_int32]
        _lib.tq_decode_workspace_bytes.argtypes = [ctypes.c_int32, ctypes.c_int32, ctypes.c_int32,
                                                   ctypes.c_int64]
        _lib.tq_decode_paged_workspace_bytes.restype = ctypes.c_size_t
        _lib.tq_decode_paged_workspace_bytes.argtypes = [ctypes.c_int] + [ctypes.c_int32] * 8
    return _lib


def declared_symbols():
    """Function names declared in the public header."""
    text = open(HEADER).read()
    return sorted(set(re.findall(r"\b(tq_[a-z0-9_]+)\s*\(", text)))


def p(t):
    """Device (or null) pointer of a tensor."""
    return ctypes.c_void_p(0 if t is None else t.data_ptr())


def stream():
    import torch
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def check(rc):
    if rc != 0:
        raise RuntimeError(f"tq error {rc}: {lib().tq_last_error().decode()}")


def i64(v):
    return ctypes.c_int64(int(v))


def i32(v):
    return ctypes.c_int32(int(v))
