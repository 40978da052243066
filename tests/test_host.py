"""CPU tests of the product's host side: setup code bit-exact with the reference,
the C ABI library exports what the header declares, the torch.ops schemas
register, and CPU tensors are refused (no CPU kernels, no fallback)."""

import ctypes
import os
import struct

import numpy as np
import pytest
import torch

import capi


def _built():
    from turboquant_kv import _lib
    return os.path.exists(_lib.HIP_LIB) and os.path.exists(_lib.TORCH_LIB)


def test_product_codebook_rotation_qjl_bits(golden):
    from turboquant_kv.codebook import (lloyd_max_codebook, make_qjl_matrix, make_rht_rotation,
                                        make_rotation_matrix)
    cb, rot, qj = golden("codebook"), golden("rotation"), golden("qjl")
    for b in range(1, 6):
        for d in (64, 128, 200):
            bnd, cen = lloyd_max_codebook(b, d)
            assert np.array_equal(bnd.numpy().view(np.uint32), cb[f"bnd_b{b}_d{d}"].view(np.uint32))
            assert np.array_equal(cen.numpy().view(np.uint32), cb[f"cen_b{b}_d{d}"].view(np.uint32))
    for d in (64, 128, 200):
        for s in (42, 43):
            assert np.array_equal(make_rotation_matrix(d, s).numpy(), rot[f"R_d{d}_s{s}"])
            assert np.array_equal(make_qjl_matrix(d, d, s).numpy(), qj[f"S_d{d}_s{s}"])
    for d in (64, 128):
        assert np.array_equal(make_rht_rotation(d, 42).numpy(), rot[f"RHT_d{d}_s42"])
    with pytest.raises(ValueError):
        make_rotation_matrix(8, 1, "nope")


def test_config_defaults():
    from turboquant_kv import TurboQuantConfig
    c = TurboQuantConfig()
    assert (c.key_bits, c.value_bits, c.mode, c.rotation, c.seed) == (4, 2, "mse", "dense_qr", 42)


@pytest.mark.skipif(not _built(), reason="native library not built")
def test_capi_exports_every_declared_symbol():
    lib = ctypes.CDLL(capi.LIB)
    syms = capi.declared_symbols()
    assert len(syms) >= 14
    for s in syms:
        assert hasattr(lib, s), s
    lib.tq_abi_version.restype = ctypes.c_int
    assert lib.tq_abi_version() == 3


@pytest.mark.skipif(not _built(), reason="native library not built")
def test_capi_rejects_bad_arguments_without_launching():
    lib = capi.lib()
    z = ctypes.c_void_p(0)
    rc = lib.tq_rotate_and_quantize(z, 0, 0, capi.i64(4), capi.i32(64), z, z, capi.i32(7), z, z, z)
    assert rc == 1 and b"bit_width" in lib.tq_last_error()
    rc = lib.tq_rotate_and_quantize(z, 0, 0, capi.i64(4), capi.i32(300), z, z, capi.i32(4), z, z, z)
    assert rc == 1 and b"dim" in lib.tq_last_error()
    rc = lib.tq_ip_scan_topk(z, 0, capi.i64(1), capi.i32(64), z, z, capi.i64(10), z, z,
                             capi.i32(4), capi.i32(100), z, z, z, ctypes.c_size_t(0), z)
    assert rc == 1 and b"k must be" in lib.tq_last_error()
    rc = lib.tq_decode_attention_packed(z, 0, capi.i32(1), capi.i32(6), capi.i32(4), capi.i32(64),
                                        z, z, z, z, capi.i64(8), z, z, z, z, z, capi.i32(4),
                                        capi.i32(2), ctypes.c_float(1.0), z, z, z, ctypes.c_size_t(0), z)
    assert rc == 1 and b"multiple" in lib.tq_last_error()
    # empty inputs are valid no-ops
    assert lib.tq_rotate_and_quantize(z, 0, 0, capi.i64(0), capi.i32(64), z, z, capi.i32(4), z, z, z) == 0


@pytest.mark.skipif(not _built(), reason="native library not built")
def test_torch_ops_schemas_registered():
    from turboquant_kv._lib import ops
    t = ops()
    for name in ("rotate_and_quantize", "attention_scores_packed", "attention_values_packed",
                 "pack_codes", "unpack_codes", "quantize_mse_packed", "quantize_prod_packed",
                 "dequantize_mse_packed", "dequantize_prod_packed", "ip_scan_topk",
                 "decode_attention_packed"):
        assert hasattr(t, name), name


@pytest.mark.skipif(not _built(), reason="native library not built")
def test_cpu_tensors_are_refused():
    from turboquant_kv import quantize_mse
    from turboquant_kv._lib import ops
    with pytest.raises(RuntimeError, match="HIP device"):
        quantize_mse(torch.randn(4, 64), 4)
    with pytest.raises((RuntimeError, NotImplementedError)):
        ops().pack_codes(torch.zeros(2, 8, dtype=torch.uint8), 2)


def test_index_file_format_header():
    # The reference's Python format: <BII header + mode byte (search.py:29-34, 254-275)
    from turboquant_kv.search import HEADER_FORMAT, HEADER_SIZE
    assert HEADER_FORMAT == "<BII" and HEADER_SIZE == 9
    assert struct.pack(HEADER_FORMAT, 4, 128, 3) == b"\x04\x80\x00\x00\x00\x03\x00\x00\x00"
