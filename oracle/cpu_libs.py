"""ctypes bindings for the CPU checkers built by oracle/Makefile.

TEST INFRASTRUCTURE ONLY (tests/, smoke(), bench.py cpu_baseline).

  port: oracle/libtq_oracle_cpu.so  -- this repo's C restatement (tq_cpu.c)
  ref:  oracle/_ref/libtqcore_ref.so -- the reference's csrc/core compiled from its
        own sources (exists only where the reference checkout was present at build)
        oracle/_ref/libquant_cpu_ref.so -- its csrc/cpu/quant_cpu.cpp, likewise
"""

from __future__ import annotations

import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
PORT_LIB = os.path.join(HERE, "libtq_oracle_cpu.so")
REF_LIB = os.path.join(HERE, "_ref", "libtqcore_ref.so")
# the reference's csrc/cpu kernels (quant_cpu.cpp) compiled against the installed torch
REF_CPU_LIB = os.path.join(HERE, "_ref", "libquant_cpu_ref.so")

_P = ctypes.c_void_p
_libs: dict = {}


def _load(path):
    if path not in _libs:
        _libs[path] = ctypes.CDLL(path)
    return _libs[path]


def have_port() -> bool:
    return os.path.exists(PORT_LIB)


def have_ref() -> bool:
    return os.path.exists(REF_LIB)


def have_ref_cpu() -> bool:
    return os.path.exists(REF_CPU_LIB)


def _ptr(a):
    return a.ctypes.data_as(_P)


def search_packed(queries, packed, norms, R, cen, bits, k, which="port"):
    """Top-k IP search on packed codes; returns (scores f32 [Q,k], ids i64 [Q,k])."""
    q = np.ascontiguousarray(queries, np.float32)
    p = np.ascontiguousarray(packed, np.uint8)
    n = np.ascontiguousarray(norms, np.float32)
    R = np.ascontiguousarray(R, np.float32)
    c = np.ascontiguousarray(cen, np.float32)
    Q, d = q.shape
    N = p.shape[0]
    os_ = np.empty((Q, k), np.float32)
    oi = np.empty((Q, k), np.int64)
    if which == "ref":
        lib = _load(REF_LIB)
        lib.ref_search_packed(_ptr(q), ctypes.c_int(Q), _ptr(p), _ptr(n), ctypes.c_int(N),
                              ctypes.c_int(d), ctypes.c_int(bits), _ptr(R), _ptr(c),
                              ctypes.c_int(k), _ptr(os_), _ptr(oi))
    else:
        lib = _load(PORT_LIB)
        lib.tqo_search_packed(_ptr(q), ctypes.c_int(Q), _ptr(p), _ptr(n), ctypes.c_int64(N),
                              ctypes.c_int(d), ctypes.c_int(bits), _ptr(R), _ptr(c),
                              ctypes.c_int(k), _ptr(os_), _ptr(oi))
    return os_, oi


def rotate_and_quantize(x, R, bnd, bits):
    """quant_cpu.cpp:44-118 restated; returns (packed u8, norms f32)."""
    x = np.ascontiguousarray(x, np.float32)
    R = np.ascontiguousarray(R, np.float32)
    b = np.ascontiguousarray(bnd, np.float32)
    n, d = x.shape
    packed = np.empty((n, bits * ((d + 7) // 8)), np.uint8)
    norms = np.empty(n, np.float32)
    lib = _load(PORT_LIB)
    lib.tqo_rotate_and_quantize(_ptr(x), ctypes.c_int64(n), ctypes.c_int(d), _ptr(R), _ptr(b),
                                ctypes.c_int(bits), _ptr(packed), _ptr(norms))
    return packed, norms


def ref_pack_codes(codes, bits):
    c = np.ascontiguousarray(codes, np.uint8)
    n, d = c.shape
    out = np.empty((n, bits * ((d + 7) // 8)), np.uint8)
    _load(REF_LIB).ref_pack_codes(_ptr(c), ctypes.c_int(n), ctypes.c_int(d), ctypes.c_int(bits),
                                  _ptr(out))
    return out


def ref_unpack_codes(packed, bits, d):
    p = np.ascontiguousarray(packed, np.uint8)
    n = p.shape[0]
    out = np.empty((n, d), np.uint8)
    _load(REF_LIB).ref_unpack_codes(_ptr(p), ctypes.c_int(n), ctypes.c_int(d), ctypes.c_int(bits),
                                    _ptr(out))
    return out


# ---- the reference's CPU kernels (quant_cpu.cpp), through oracle/ref_quant_cpu_shim.cpp
def _ref_cpu():
    return _load(REF_CPU_LIB)


def ref_cpu_rotate_and_quantize(x, R, bnd, bits):
    """rotate_and_quantize_cpu (quant_cpu.cpp:44-118); returns (packed u8, norms f32)."""
    x = np.ascontiguousarray(x, np.float32)
    R = np.ascontiguousarray(R, np.float32)
    b = np.ascontiguousarray(bnd, np.float32)
    n, d = x.shape
    packed = np.empty((n, bits * ((d + 7) // 8)), np.uint8)
    norms = np.empty(n, np.float32)
    rc = _ref_cpu().ref_cpu_rotate_and_quantize(_ptr(x), ctypes.c_int64(n), ctypes.c_int(d), _ptr(R),
                                                _ptr(b), ctypes.c_int(bits), _ptr(packed), _ptr(norms))
    assert rc == 0, "rotate_and_quantize_cpu failed"
    return packed, norms


def ref_cpu_attention_scores(q, packed, norms, cen, R, bits):
    """attention_scores_packed_cpu (quant_cpu.cpp:125-197): q [batch, heads, d] ->
    scores [batch, heads, T]."""
    q = np.ascontiguousarray(q, np.float32)
    p = np.ascontiguousarray(packed, np.uint8)
    n = np.ascontiguousarray(norms, np.float32)
    c = np.ascontiguousarray(cen, np.float32)
    R = np.ascontiguousarray(R, np.float32)
    B, H, d = q.shape
    T = p.shape[0]
    out = np.empty((B, H, T), np.float32)
    rc = _ref_cpu().ref_cpu_attention_scores(_ptr(q), ctypes.c_int(B), ctypes.c_int(H), ctypes.c_int(d),
                                             _ptr(p), _ptr(n), ctypes.c_int64(T), _ptr(c), _ptr(R),
                                             ctypes.c_int(bits), _ptr(out))
    assert rc == 0, "attention_scores_packed_cpu failed"
    return out


def ref_cpu_attention_values(w, packed, norms, cen, R_T, bits, d):
    """attention_values_packed_cpu (quant_cpu.cpp:199-266): w [batch, heads, T] ->
    out [batch, heads, d]."""
    w = np.ascontiguousarray(w, np.float32)
    p = np.ascontiguousarray(packed, np.uint8)
    n = np.ascontiguousarray(norms, np.float32)
    c = np.ascontiguousarray(cen, np.float32)
    Rt = np.ascontiguousarray(R_T, np.float32)
    B, H, T = w.shape
    out = np.empty((B, H, d), np.float32)
    rc = _ref_cpu().ref_cpu_attention_values(_ptr(w), ctypes.c_int(B), ctypes.c_int(H), ctypes.c_int64(T),
                                             _ptr(p), _ptr(n), ctypes.c_int(d), _ptr(c), _ptr(Rt),
                                             ctypes.c_int(bits), _ptr(out))
    assert rc == 0, "attention_values_packed_cpu failed"
    return out
