"""CPU tests of the product's host side: setup code bit-exact with the reference,
the C ABI library exports what the header declares, the torch.ops schemas
register, CPU tensors reach CPU kernels only for the five reference schemas (which the
reference registers for the CPU key too) and are refused everywhere else (no fallback)."""

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
        # The RHT matrix is re-orthogonalized by torch.linalg.qr (reference.py:174), whose
        # float32 LAPACK bits depend on the host's kernels: the fixture host and an MI355X
        # box differ by up to ~30 ulp (4e-7 at d = 64).  Pinned here at the scale of float32
        # Householder QR's backward error, d * 2^-24 entrywise, with the same signs and
        # orthogonality; tests/test_gpu_api.py checks the codes quantized with it.
        got, want = make_rht_rotation(d, 42).numpy(), rot[f"RHT_d{d}_s42"]
        assert got.dtype == np.float32 and got.shape == (d, d)
        assert np.array_equal(np.sign(got), np.sign(want))
        tol = d * 2.0 ** -24
        assert np.abs(got.astype(np.float64) - want).max() <= tol
        g64 = got.astype(np.float64)
        assert np.abs(g64 @ g64.T - np.eye(d)).max() <= 2 * tol
        # before the QR every entry is +-1/sqrt(d) (d a power of two: H D is already
        # orthogonal), and the QR only fixes rounding
        assert np.abs(np.abs(g64) - 1 / np.sqrt(d)).max() <= tol
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
    assert lib.tq_abi_version() == 4


@pytest.mark.skipif(not _built(), reason="native library not built")
def test_capi_rejects_bad_arguments_without_launching():
    lib = capi.lib()
    z = ctypes.c_void_p(0)
    rc = lib.tq_rotate_and_quantize(z, 0, 0, capi.i64(4), capi.i32(64), z, z, capi.i32(7), z, z, z)
    assert rc == 1 and b"bit_width" in lib.tq_last_error()
    rc = lib.tq_rotate_and_quantize(z, 0, 0, capi.i64(4), capi.i32(300), z, z, capi.i32(4), z, z, z)
    assert rc == 1 and b"dim" in lib.tq_last_error()
    rc = lib.tq_ip_scan_topk(z, 0, capi.i64(1), capi.i32(64), z, z, capi.i64(10), z, z,
                             capi.i32(4), capi.i32(129), z, z, z, ctypes.c_size_t(0), z)
    assert rc == 1 and b"k must be in [1, 128]" in lib.tq_last_error()
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
                 "decode_attention_packed", "ip_scan_topk_prod", "attention_scores_prod",
                 "paged_store", "paged_gather", "decode_attention_paged", "core_rotation",
                 "core_codebook"):
        assert hasattr(t, name), name


@pytest.mark.skipif(not _built(), reason="native library not built")
def test_cpu_tensors_are_refused():
    from turboquant_kv import quantize_mse
    from turboquant_kv._lib import ops
    with pytest.raises(RuntimeError, match="HIP device"):
        quantize_mse(torch.randn(4, 64), 4)
    # the new ops have HIP kernels only: no CPU dispatch entry
    with pytest.raises((RuntimeError, NotImplementedError)):
        ops().quantize_mse_packed(torch.randn(4, 64), torch.eye(64), torch.zeros(15), 4)
    with pytest.raises((RuntimeError, NotImplementedError)):
        ops().ip_scan_topk(torch.randn(1, 64), torch.zeros(8, 32, dtype=torch.uint8), torch.ones(8),
                           torch.zeros(16), torch.eye(64), 4, 2)


def test_index_file_format_header():
    # The reference's Python format: <BII header + mode byte (search.py:29-34, 254-275)
    from turboquant_kv.search import HEADER_FORMAT, HEADER_SIZE
    assert HEADER_FORMAT == "<BII" and HEADER_SIZE == 9
    assert struct.pack(HEADER_FORMAT, 4, 128, 3) == b"\x04\x80\x00\x00\x00\x03\x00\x00\x00"


# ------------------------------------------------------------------ TQIX (the C++ core's files)
@pytest.mark.skipif(not _built(), reason="native library not built")
def test_core_tables_bit_exact_with_reference_core(golden):
    # tq_core_rotation / tq_core_codebook (host code) against the matrices and codebooks
    # the reference's compiled core produced (tests/golden/make_tqix_golden.py)
    z = golden("tqix")
    lib = capi.lib()
    for key in [k for k in z.files if k.startswith("R_d")]:
        d, seed = (int(v) for v in key[3:].split("_s"))
        R = np.zeros((d, d), np.float32)
        assert lib.tq_core_rotation(capi.i32(d), capi.i32(seed), R.ctypes.data_as(ctypes.c_void_p)) == 0
        assert np.array_equal(R.view(np.uint32), z[key].view(np.uint32)), key
        assert np.allclose(R.T.astype(np.float64) @ R, np.eye(d), atol=1e-5)
    for b in (1, 2, 3, 4):
        for d in (64, 128, 200):
            bnd = np.zeros((1 << b) - 1, np.float32)
            cen = np.zeros(1 << b, np.float32)
            assert lib.tq_core_codebook(capi.i32(b), capi.i32(d), bnd.ctypes.data_as(ctypes.c_void_p),
                                        cen.ctypes.data_as(ctypes.c_void_p)) == 0
            assert np.array_equal(bnd.view(np.uint32), z[f"bnd_b{b}_d{d}"].view(np.uint32)), (b, d)
            assert np.array_equal(cen.view(np.uint32), z[f"cen_b{b}_d{d}"].view(np.uint32)), (b, d)
    # the same tables through the Python API
    from turboquant_kv.codebook import core_codebook, make_rotation_matrix
    assert np.array_equal(make_rotation_matrix(64, 7, "core").numpy(), z["R_d64_s7"])
    assert np.array_equal(core_codebook(3, 64)[1].numpy(), z["cen_b3_d64"])


def test_tqix_read_write_byte_exact_and_errors(tmp_path):
    from turboquant_kv.formats import TQIX_MAGIC, read_tqix, write_tqix
    src = os.path.join(os.path.dirname(__file__), "golden", "core_d64_b3_s7.tqix")
    raw = open(src, "rb").read()
    assert struct.unpack("<6I", raw[:24]) == (TQIX_MAGIC, 1, 64, 3, 7, 300) and raw[:4] == b"XIQT"
    f = read_tqix(src)
    assert (f.dim, f.bit_width, f.seed, f.n_vectors) == (64, 3, 7, 300)
    assert f.packed.shape == (300, 24) and f.norms.dtype == np.float32
    assert f.norms[5] == 0.0  # the fixture's zero vector
    out = tmp_path / "copy.tqix"
    write_tqix(str(out), f.dim, f.bit_width, f.seed, f.packed, f.norms)
    assert out.read_bytes() == raw
    empty = tmp_path / "empty.tqix"
    write_tqix(str(empty), 128, 4, -1, np.zeros((0, 64), np.uint8), np.zeros(0, np.float32))
    e = read_tqix(str(empty))
    assert (e.dim, e.bit_width, e.seed, e.n_vectors) == (128, 4, -1, 0)
    for name, data, msg in (("magic", b"QTIX" + raw[4:], "bad magic"),
                            ("version", raw[:4] + struct.pack("<I", 2) + raw[8:], "version"),
                            ("short", raw[:-1], "truncated"), ("head", raw[:10], "truncated")):
        p = tmp_path / f"{name}.tqix"
        p.write_bytes(data)
        with pytest.raises(ValueError, match=msg):
            read_tqix(str(p))


def test_oracle_reproduces_reference_core_search_on_tqix_file(golden):
    # the fixture's search results are the core's arithmetic: the oracle's LUT form
    # (csrc/core/turboquant_core.cpp:407-514) over the file with the core's tables
    import tq_oracle as O
    from turboquant_kv.formats import read_tqix
    z = golden("tqix")
    f = read_tqix(os.path.join(os.path.dirname(__file__), "golden", "core_d64_b3_s7.tqix"))
    s, i = O.search_topk(z["queries"], f.packed, f.norms, z["cen_b3_d64"], z["R_d64_s7"], 3, 10)
    assert np.array_equal(i, z["ids"])
    assert np.array_equal(s.view(np.uint32), z["scores"].view(np.uint32))


# ------------------------------------------------------------------ Huffman code storage
@pytest.mark.skipif(not _built(), reason="native library not built")
def test_huffman_code_words_and_streams_match_reference(golden):
    # code words and byte streams written by the reference's entropy module
    # (tests/golden/make_entropy_golden.py)
    from turboquant_kv.entropy import EntropyPackedStorage, HuffmanCoder, compute_codeword_probabilities
    z = golden("entropy")
    for bits in (1, 2, 3, 4, 5):
        for dim in (64, 128):
            assert np.allclose(compute_codeword_probabilities(bits, dim), z[f"probs_b{bits}_d{dim}"],
                               rtol=1e-12, atol=0)
            c = HuffmanCoder(bits, dim)
            words = [c.codebook[s] for s in range(1 << bits)]
            assert [len(w) for w in words] == z[f"lens_b{bits}_d{dim}"].tolist(), (bits, dim)
            assert [int(w, 2) for w in words] == z[f"words_b{bits}_d{dim}"].tolist(), (bits, dim)
            # Kraft equality: a complete prefix code
            assert abs(sum(2.0 ** -len(w) for w in words) - 1.0) < 1e-12
            assert c.entropy() <= c.avg_code_length() < c.entropy() + 1
    i = 0
    while f"case{i}_meta" in z.files:
        bits, dim = z[f"case{i}_meta"].tolist()
        codes = torch.from_numpy(z[f"case{i}_codes"])
        st = EntropyPackedStorage.from_codes(codes, bits, dim)
        assert st._data == z[f"case{i}_bytes"].tobytes(), i
        assert torch.equal(st.to_codes(), torch.from_numpy(z[f"case{i}_decoded"]))
        assert abs(st.savings_pct - float(z[f"case{i}_savings"])) < 1e-12
        i += 1
    assert i == 5
    assert HuffmanCoder(4, 64).encode(torch.zeros(0, dtype=torch.uint8)) == z["empty_bytes"].tobytes()


@pytest.mark.skipif(not _built(), reason="native library not built")
def test_huffman_round_trip_limits_and_short_streams():
    from turboquant_kv.entropy import EntropyPackedStorage, HuffmanCoder
    rs = np.random.RandomState(9)
    c = HuffmanCoder(4, 128)
    probs = c.probs
    codes = torch.from_numpy(rs.choice(16, 200000, p=probs).astype(np.uint8))
    data = c.encode(codes)
    n, nbits = struct.unpack("<II", data[:8])
    assert n == 200000
    assert nbits == int(sum(np.bincount(codes.numpy(), minlength=16)[s] * len(c.codebook[s]) for s in range(16)))
    assert len(data) == 8 + (nbits + 7) // 8
    assert torch.equal(c.decode(data), codes)
    assert torch.equal(c.decode(data, 1000), codes[:1000])
    # a stream cut short decodes the symbols it still holds
    cut = c.decode(data[:8 + 100])
    assert 0 < cut.numel() < 200000 and torch.equal(cut, codes[:cut.numel()])
    st = EntropyPackedStorage.from_codes(codes.view(-1, 100), 4, 128)
    assert st.to_codes().shape == (2000, 100)
    assert 0 < st.savings_pct < 10  # ~3.8 bits/code against 4


def test_paged_pool_layout_selection():
    # Decode-layout pools take mse K4/V2 at head_dim 64 and power-of-two block sizes >= 16;
    # anything else is refused up front (before any allocation), and the vLLM cache config's
    # "auto" resolves to the decode layout exactly where it applies.
    from turboquant_kv.config import TurboQuantConfig
    from turboquant_kv.vllm_plugin.paged import PagedKVPools
    ok = PagedKVPools.decode_layout_supported
    mse = TurboQuantConfig(key_bits=4, value_bits=2)
    assert ok(mse, 64, 16) and ok(mse, 64, 32) and ok(mse, 64, 64) and ok(mse, 64, 256)
    assert not ok(mse, 64, 8) and not ok(mse, 64, 48) and not ok(mse, 128, 16)
    assert not ok(TurboQuantConfig(key_bits=3, value_bits=2), 64, 16)
    assert not ok(TurboQuantConfig(key_bits=4, value_bits=2, mode="prod"), 64, 16)
    for cfg, d, bs in ((TurboQuantConfig(mode="prod"), 64, 16), (mse, 64, 24), (mse, 128, 64)):
        with pytest.raises(ValueError, match="layout='decode'"):
            PagedKVPools(cfg, 1, 4, bs, 2, d, device="cpu", layout="decode")
    with pytest.raises(ValueError, match="Unknown layout"):
        PagedKVPools(mse, 1, 4, 16, 2, 64, device="cpu", layout="tiles")


def test_huffman_window_table_decoder_equals_bit_walk():
    # Streams decoded through the window table (longest word <= 20 bits) and through the
    # per-bit walk (forced by one extra 24-bit word that never occurs) give the same
    # symbols, for a table with a prefix relation ("0" and "000") and a duplicate word
    # (the later entry wins), and for truncated streams.
    from turboquant_kv._lib import ops
    words = torch.tensor([0b0, 0b10, 0b110, 0b111, 0b000, 0b10], dtype=torch.int64)
    lens = torch.tensor([1, 2, 3, 3, 3, 2], dtype=torch.uint8)
    syms = torch.tensor([0, 1, 2, 3, 4, 5], dtype=torch.int32)
    long_w = torch.cat([words, torch.tensor([0xABCDEF], dtype=torch.int64)])
    long_l = torch.cat([lens, torch.tensor([24], dtype=torch.uint8)])
    long_s = torch.cat([syms, torch.tensor([6], dtype=torch.int32)])
    rs = np.random.RandomState(4)
    for nbytes in (0, 1, 2, 7, 64, 1000):
        body = rs.randint(0, 256, nbytes).astype(np.uint8)
        for nbits in (nbytes * 8, max(nbytes * 8 - 5, 0)):
            hdr = np.array([1 << 20, nbits], np.uint32).view(np.uint8)
            data = torch.from_numpy(np.concatenate([hdr, body]))
            a = ops().huffman_decode(data, -1, words, lens, syms)
            b = ops().huffman_decode(data, -1, long_w, long_l, long_s)
            assert torch.equal(a, b), (nbytes, nbits)
            assert not (a == 1).any() and not (a == 4).any()   # replaced / shadowed words


def test_large_k_topk_keeps_the_lowest_index_among_ties():
    # The k > 32 search path selects with torch.topk, whose order among ties is
    # unspecified; the helper must return the reference core's heap order (score
    # descending, lower index first on a tie) and never list NaN, over integer-valued
    # scores full of ties, -inf and NaN, against the oracle's lexsort order.
    from turboquant_kv.search import _topk_lowest_index
    import tq_oracle as O
    rs = np.random.RandomState(0)
    for trial in range(300):
        Q, N = rs.randint(1, 4), rs.randint(1, 300)
        k = rs.randint(1, N + 1)
        s = rs.randint(-5, 5, size=(Q, N)).astype(np.float32)
        if trial % 3 == 0:
            s[rs.rand(Q, N) < 0.2] = np.nan
        if trial % 5 == 0:
            s[rs.rand(Q, N) < 0.2] = -np.inf
        v, i = _topk_lowest_index(torch.from_numpy(s), k)
        sc = np.where(np.isnan(s), -np.inf, s)
        want_s, want_i = O.topk_desc(sc, N)
        for q in range(Q):
            ids = [j for j in want_i[q] if not np.isnan(s[q, j])][:k]
            ei = np.full(k, -1)
            ei[:len(ids)] = ids
            es = np.full(k, -np.inf, np.float32)
            es[:len(ids)] = s[q, ids]
            assert np.array_equal(i[q].numpy(), ei), (trial, q)
            assert np.array_equal(v[q].numpy(), es), (trial, q)
