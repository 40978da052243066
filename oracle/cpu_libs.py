"""ctypes bindings for the CPU checkers built by oracle/Makefile.

TEST INFRASTRUCTURE ONLY (tests/, smoke(), bench.py cpu_baseline).

  port: oracle/libtq_oracle_cpu.so  -- this repo's C restatement (tq_cpu.c)
  ref:  oracle/_ref/libtqcore_ref.so -- the reference's csrc/core compiled from its
        own sources (exists only where the reference checkout was present at build)
"""

from __future__ import annotations

import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
PORT_LIB = os.path.join(HERE, "libtq_oracle_cpu.so")
REF_LIB = os.path.join(HERE, "_ref", "libtqcore_ref.so")

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
