"""GPU tests of the drop-in Python API (quantize_* functions, TurboQuantIndex,
QuantizedKVCache, torch.ops schemas) against the reference's golden vectors,
mirroring the reference's own tests (tests/test_reference.py, tests/test_cache.py)."""

import math
import os

import numpy as np
import pytest
import torch

import tq_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"


def T(a):
    return torch.from_numpy(np.ascontiguousarray(a)).to(DEV)


def test_native_library_is_what_runs():
    from turboquant_kv import _lib
    _lib.load()
    maps = open("/proc/self/maps").read()
    assert os.path.basename(_lib.HIP_LIB) in maps and os.path.basename(_lib.TORCH_LIB) in maps


def test_quantize_mse_api_vs_reference(golden):
    from turboquant_kv import quantize_mse, dequantize_mse
    from turboquant_kv.reference import make_rotation_matrix, lloyd_max_codebook
    m = golden("quant_mse")
    x = m["d128_x"]
    for b in (2, 3, 4):
        packed, norms = quantize_mse(T(x), b)  # default rotation seed 42, default codebook
        codes = O.unpack_codes(packed.cpu().numpy(), b, 128)
        ref = O.unpack_codes(m[f"d128_b{b}_packed"], b, 128)
        O.check_codes(codes, ref, x, make_rotation_matrix(128, 42).numpy(),
                      lloyd_max_codebook(b, 128)[0].numpy())
        assert norms.dtype == torch.float32
        rec = dequantize_mse(T(m[f"d128_b{b}_packed"][:64]), T(m[f"d128_b{b}_norms"][:64]), b, 128)
        assert np.allclose(rec.cpu().numpy(), m[f"d128_b{b}_deq64"], rtol=1e-5, atol=2e-6)
    # bf16 input keeps bf16 norms, as reference.py does
    xb = torch.from_numpy(m["bf16_d64_x_u16"].view(np.int16)).to(DEV).view(torch.bfloat16)
    packed, norms = quantize_mse(xb, 4)
    assert norms.dtype == torch.bfloat16
    assert np.array_equal(norms.float().cpu().numpy(), O.bf16_bits_to_f32(m["bf16_d64_b4_norms_u16"]))


def test_quantize_with_rht_rotation_vs_reference_matrix(golden):
    """rotation="rht": the product builds its RHT matrix on this host with torch.linalg.qr,
    whose float32 bits differ between hosts (up to ~30 ulp against the fixture host).  The
    codes are bit-exact with the oracle under the matrix the product built (outside the
    fp32 decision band), and equal the reference's codes under the reference-written matrix
    except where the matrices' difference can move a coordinate across a boundary."""
    from turboquant_kv import TurboQuantMSE
    from turboquant_kv.reference import lloyd_max_codebook
    rot = golden("rotation")
    m = golden("quant_mse")
    for d in (64, 128):
        x = m["d128_x"][:, :d].copy() if d == 64 else m["d128_x"]
        R_ref = rot[f"RHT_d{d}_s42"]
        for b in (2, 4):
            tq = TurboQuantMSE(d, b, seed=42, rotation="rht", device=DEV)
            R_own = tq.rotation.cpu().numpy()
            dev = float(np.abs(R_own.astype(np.float64) - R_ref).max())
            assert dev <= d * 2.0 ** -24
            packed, norms = tq.quantize(T(x))
            codes = O.unpack_codes(packed.cpu().numpy(), b, d)
            bnd = lloyd_max_codebook(b, d)[0].numpy()
            _, n_o, c_own = O.quantize_mse(x, b, R_own, bnd)
            O.check_codes(codes, c_own, x, R_own, bnd)
            assert np.allclose(norms.cpu().numpy(), n_o, rtol=1e-6, atol=0)
            # against the reference's matrix: |y - y_ref| <= sum_k |u_k| |dR_jk|, and
            # |R_jk| = 1/sqrt(d), so the band widens by sqrt(d) * dev relative
            _, _, c_ref = O.quantize_mse(x, b, R_ref, bnd)
            amb = O.code_margin(x, R_ref, bnd, rel=2.0 ** -20 + np.sqrt(d) * dev)
            assert not ((codes != c_ref) & ~amb).any()


def test_quantize_prod_api_roundtrip(golden):
    from turboquant_kv import quantize_prod, dequantize_prod
    pr = golden("quant_prod")
    x = pr["d128_x"]
    mp, sg, rn, nm = quantize_prod(T(x), 4)
    assert mp.shape == (1024, 48) and sg.shape == (1024, 16)
    rec = dequantize_prod(T(pr["d128_mse_packed"][:64]), T(pr["d128_signs"][:64]),
                          T(pr["d128_res_norms"][:64]), T(pr["d128_norms"][:64]), 4, 128)
    ref = pr["d128_deq64"]
    assert np.max(np.abs(rec.cpu().numpy() - ref)) <= 2e-5 * np.max(np.abs(ref))
    with pytest.raises(ValueError):
        quantize_prod(T(x), 1)


def test_torch_ops_reference_schemas(golden):
    ops = torch.ops.turboquant
    m, rot = golden("quant_mse"), golden("rotation")
    R = T(rot["R_d128_s42"])
    bnd, cen = O.lloyd_max_codebook(4, 128)
    packed, norms = ops.rotate_and_quantize(T(m["d128_x"]), R, T(bnd), 4)
    assert packed.shape == (1024, 64) and norms.dtype == torch.float32
    codes = ops.unpack_codes(packed, 4, 128)
    assert torch.equal(ops.pack_codes(codes, 4), packed)
    q = torch.randn(2, 3, 128, device=DEV)
    s = ops.attention_scores_packed(q, packed, norms, T(cen), R, 4)
    assert s.shape == (2, 3, 1024)
    w = torch.softmax(s, -1)
    o = ops.attention_values_packed(w, packed, norms, T(cen), R, 4)
    assert o.shape == (2, 3, 128)
    with pytest.raises(RuntimeError, match="bit_width"):
        ops.rotate_and_quantize(T(m["d128_x"]), R, T(bnd), 7)
    with pytest.raises(RuntimeError, match="packed dim mismatch"):
        ops.unpack_codes(packed, 3, 128)


def test_reference_schemas_cpu_and_gpu_agree(golden):
    """The same call on host tensors (CPU kernels) and on device tensors (gfx950 kernels):
    pack/unpack and scores bit-identical, codes equal outside the decision band (the MFMA
    contraction and the CPU kernel's sequential sum round differently), values within the
    fp32 bound."""
    ops = torch.ops.turboquant
    m, rot = golden("quant_mse"), golden("rotation")
    x, R = m["d64_x"][2:], rot["R_d64_s42"]  # rows of norm > 1e-10
    bnd, cen = O.lloyd_max_codebook(3, 64)
    tc = lambda a: torch.from_numpy(np.ascontiguousarray(a))
    pc, nc = ops.rotate_and_quantize(tc(x), tc(R), tc(bnd), 3)
    pg, ng = ops.rotate_and_quantize(T(x), T(R), T(bnd), 3)
    O.check_codes(O.unpack_codes(pg.cpu().numpy(), 3, 64), O.unpack_codes(pc.numpy(), 3, 64), x, R, bnd)
    assert np.allclose(nc.numpy(), ng.cpu().numpy(), rtol=4e-6, atol=0)
    assert torch.equal(ops.unpack_codes(pc, 3, 64), ops.unpack_codes(pc.to(DEV), 3, 64).cpu())
    codes = ops.unpack_codes(pc, 3, 64)
    assert torch.equal(ops.pack_codes(codes, 3), ops.pack_codes(codes.to(DEV), 3).cpu())
    q = np.random.RandomState(0).randn(2, 4, 64).astype(np.float32)
    sc = ops.attention_scores_packed(tc(q), pc, nc, tc(cen), tc(R), 3)
    sg = ops.attention_scores_packed(T(q), pc.to(DEV), nc.to(DEV), T(cen), T(R), 3)
    assert np.array_equal(sc.numpy().view(np.uint32), sg.cpu().numpy().view(np.uint32))
    w = torch.softmax(sc, -1)
    oc = ops.attention_values_packed(w, pc, nc, tc(cen), tc(R), 3)
    og = ops.attention_values_packed(w.to(DEV), pc.to(DEV), nc.to(DEV), T(cen), T(R), 3)
    assert np.allclose(oc.numpy(), og.cpu().numpy(), rtol=1e-5, atol=1e-5 * oc.abs().max().item())


def test_index_vs_reference(golden, tmp_path):
    from turboquant_kv import TurboQuantIndex
    ix, m = golden("index"), golden("quant_mse")
    db = T(m["d128_x"])
    for b in (2, 3, 4):
        index = TurboQuantIndex.from_vectors(db, bit_width=b, mode="mse")
        s, i = index.search(T(ix["queries"]), k=10)
        assert np.array_equal(i.cpu().numpy(), ix[f"b{b}_ids"]), b
        assert np.allclose(s.cpu().numpy(), ix[f"b{b}_scores"], rtol=1e-5, atol=1e-6)
        path = str(tmp_path / f"idx{b}.tq")
        index.save(path)
        back = TurboQuantIndex.load(path)
        assert back.n_vectors == 1024
        s2, i2 = back.search(T(ix["queries"]), k=10)
        assert torch.equal(i2, i)
    # incremental add == one add; k > n clamps to n
    inc = TurboQuantIndex(128, bit_width=4)
    for c in range(0, 1024, 300):
        inc.add(db[c:c + 300])
    s3, i3 = inc.search(T(ix["queries"]), k=10)
    assert np.array_equal(i3.cpu().numpy(), ix["b4_ids"])
    small = TurboQuantIndex.from_vectors(db[:3], bit_width=4)
    assert small.search(db[0], k=10)[1].shape == (1, 3)


def test_index_top1_matches_brute_force():
    # reference tests/test_reference.py:295-316
    from turboquant_kv import TurboQuantIndex
    torch.manual_seed(42)
    db = torch.randn(500, 64, device=DEV)
    q = torch.randn(10, 64, device=DEV)
    exact = (q @ db.t()).argmax(-1)
    idx = TurboQuantIndex.from_vectors(db, bit_width=4, mode="mse")
    _, top = idx.search(q, k=1)
    assert (top.squeeze(-1) == exact).float().mean().item() >= 0.5
    prod = TurboQuantIndex.from_vectors(db, bit_width=4, mode="prod")
    _, top = prod.search(q, k=1)
    assert (top.squeeze(-1) == exact).float().mean().item() >= 0.5


def test_prod_index_search_scores_without_reconstruction():
    # TurboQuantIndex prod search scores the packed rows; the reference dequantizes every
    # row and multiplies (search.py:229-252).  Both against the float64 composition.
    from turboquant_kv import TurboQuantIndex
    rs = np.random.RandomState(4)
    for d, b in ((128, 4), (200, 3), (64, 2)):
        db = rs.randn(3000, d).astype(np.float32)
        idx = TurboQuantIndex.from_vectors(T(db), bit_width=b, mode="prod")
        q = rs.randn(6, d).astype(np.float32)
        rows = [t.cpu().numpy() for t in (idx._bitplane_codes(), idx._qjl_signs,
                                          idx._residual_norms, idx._norms)]
        R, S = idx._rot_dev.cpu().numpy(), idx._S_dev.cpu().numpy()
        ref = O.prod_scores_f64(q, *rows, b, d, R, idx._cen.cpu().numpy(), S)
        # fp32 sums of d terms against float64: d * 2^-24 of the summed magnitude
        # |q| n (1 + 2 gamma)
        tol = d * 2.0 ** -24 * np.linalg.norm(q, axis=1)[:, None] * rows[3][None, :] * (1 + 2 * rows[2][None, :])
        recon = torch.ops.turboquant.dequantize_prod_packed(
            idx._bitplane_codes(), idx._qjl_signs, idx._residual_norms, idx._norms, idx._cen,
            idx._rot_dev, idx._S_dev, b, d)
        composed = (T(q) @ recon.t()).cpu().numpy()
        assert np.all(np.abs(composed - ref) <= tol)
        for k in (10, 50):  # scan + merge; all scores + torch.topk
            s, i = idx.search(T(q), k=k)
            s, i = s.cpu().numpy(), i.cpu().numpy()
            assert np.all(np.abs(s - np.take_along_axis(ref, i, 1)) <= np.take_along_axis(tol, i, 1))
            _, io = O.topk_desc(ref, k)
            diff = i != io
            a, o = np.take_along_axis(ref, i, 1), np.take_along_axis(ref, io, 1)
            ta, to = np.take_along_axis(tol, i, 1), np.take_along_axis(tol, io, 1)
            assert np.all(~diff | (np.abs(a - o) <= ta + to)), (d, b, k)


def test_prod_cache_scores_without_reconstruction():
    from turboquant_kv import QuantizedKVCache, TurboQuantConfig
    torch.manual_seed(3)
    B, Hq, H, d = 2, 4, 2, 128
    kv = QuantizedKVCache(TurboQuantConfig(key_bits=4, value_bits=3, mode="prod"), 1, 300, H, d,
                          device=DEV, batch_size=B)
    kv.append(0, torch.randn(B, H, 130, d, device=DEV), torch.randn(B, H, 130, d, device=DEV))
    kv.append(0, torch.randn(B, H, 7, d, device=DEV), torch.randn(B, H, 7, d, device=DEV))
    q = torch.randn(B, Hq, 3, d, device=DEV)
    logits = kv.attention_scores(0, q)
    keys = kv._dequantize_keys(0).repeat_interleave(Hq // H, dim=1)   # (B, Hq, T, d)
    ref = torch.matmul(q.double(), keys.double().transpose(-2, -1)) / math.sqrt(d)
    scale = q.double().norm(dim=-1, keepdim=True) * keys.double().norm(dim=-1)[:, :, None, :]
    # both sides carry fp32 sums of d terms (the prod scan; the dequantize kernel): 2 d 2^-24
    assert ((logits.double() - ref).abs() <= 2 * d * 2.0 ** -24 * scale / math.sqrt(d) + 1e-7).all()


def test_tqix_index_from_reference_core_file(golden, tmp_path):
    # A TQIX file written by the reference's C++ core (TurboQuantIndex::save after add):
    # loaded here, the GPU scan returns the core's own search results bit for bit, and
    # save_tqix writes the same bytes back.
    from turboquant_kv import TurboQuantIndex
    z = golden("tqix")
    src = os.path.join(os.path.dirname(__file__), "golden", "core_d64_b3_s7.tqix")
    idx = TurboQuantIndex.load_tqix(src)
    assert (idx.dim, idx.bit_width, idx.seed, idx.n_vectors, idx.rotation_method) == (64, 3, 7, 300, "core")
    s, i = idx.search(T(z["queries"]), k=10)
    assert np.array_equal(i.cpu().numpy(), z["ids"])
    assert np.array_equal(s.cpu().numpy().view(np.uint32), z["scores"].view(np.uint32))
    out = tmp_path / "rt.tqix"
    idx.save_tqix(str(out))
    assert out.read_bytes() == open(src, "rb").read()
    # an index built here with the core's tables: codes equal the core's outside the
    # fp32 ambiguity band (its quantize multiplies by 1/norm), and TQIX round-trips
    own = TurboQuantIndex(64, bit_width=3, rotation="core", seed=7)
    own.add(T(z["vectors"]))
    got = O.unpack_codes(own._bitplane_codes().cpu().numpy(), 3, 64)
    want = O.unpack_codes(open_tqix_codes(src), 3, 64)
    O.check_codes(got, want, z["vectors"], z["R_d64_s7"], z["bnd_b3_d64"])
    own.save_tqix(str(tmp_path / "own.tqix"))
    back = TurboQuantIndex.load_tqix(str(tmp_path / "own.tqix"))
    assert torch.equal(back._packed_codes, own._packed_codes) and torch.equal(back._norms, own._norms)
    with pytest.raises(ValueError, match="core"):
        TurboQuantIndex(64, bit_width=3).save_tqix(str(tmp_path / "x.tqix"))


def open_tqix_codes(path):
    from turboquant_kv.formats import read_tqix
    return read_tqix(path).packed


def test_cache_vs_reference(golden):
    from turboquant_kv import QuantizedKVCache, TurboQuantConfig
    c = golden("cache")
    cfg = TurboQuantConfig(key_bits=4, value_bits=2, mode="mse")
    kv = QuantizedKVCache(cfg, 1, 128, 4, 64, device=DEV)
    kv.append(0, T(c["keys"][:, :100]), T(c["values"][:, :100]))
    kv.append(0, T(c["keys"][:, 100:]), T(c["values"][:, 100:]))
    assert kv.seq_lens[0].item() == 128
    assert np.array_equal(kv._key_packed[0][0].cpu().numpy(), c["key_packed"])
    assert np.array_equal(kv._val_packed[0][0].cpu().numpy(), c["val_packed"])
    logits = kv.attention_scores(0, T(c["query"]))
    assert np.max(np.abs(logits.cpu().numpy() - c["logits"])) <= 1e-5 * np.abs(c["logits"]).max()
    w = torch.softmax(logits, -1)
    out = kv.attention_values(0, w)
    assert np.max(np.abs(out.cpu().numpy() - c["output"])) <= 1e-5 * np.abs(c["output"]).max()
    fused = kv.decode_attention(0, T(c["query"][:, 0])[None])
    assert np.max(np.abs(fused[0].cpu().numpy() - c["output"][:, 0])) <= 1e-4 * np.abs(c["output"]).max()
    assert kv.memory_bytes() == int(c["memory_bytes"])


def test_cache_reference_behaviours():
    # reference tests/test_cache.py
    from turboquant_kv import QuantizedKVCache, TurboQuantConfig
    torch.manual_seed(0)
    cfg = TurboQuantConfig(key_bits=4, value_bits=4, mode="mse")
    cache = QuantizedKVCache(cfg, 2, 128, 4, 64, device=DEV)
    keys, values = torch.randn(4, 32, 64, device=DEV), torch.randn(4, 32, 64, device=DEV)
    cache.append(0, keys, values)
    q = torch.randn(4, 1, 64, device=DEV)
    logits = cache.attention_scores(0, q)
    exact = torch.matmul(q, keys.transpose(-2, -1)) / 8.0
    for h in range(4):
        assert torch.corrcoef(torch.stack([logits[h, 0], exact[h, 0]]))[0, 1] > 0.8
    ratio_cfg = TurboQuantConfig(key_bits=4, value_bits=2)
    c2 = QuantizedKVCache(ratio_cfg, 1, 100, 1, 128, device=DEV)
    c2.append(0, torch.randn(1, 50, 128, device=DEV), torch.randn(1, 50, 128, device=DEV))
    assert 3.0 < c2.compression_ratio < 10.0
    prot = QuantizedKVCache(TurboQuantConfig(protected_layers=2), 4, 64, 2, 32, device=DEV)
    k, v = torch.randn(2, 8, 32, device=DEV), torch.randn(2, 8, 32, device=DEV)
    prot.append(0, k, v)
    prot.append(2, k, v)
    qq = torch.randn(2, 1, 32, device=DEV)
    lp = prot.attention_scores(0, qq)
    ex = torch.matmul(qq, k.half().float().transpose(-2, -1)) / math.sqrt(32)
    assert (lp - ex).abs().max().item() < 0.05
    prodc = QuantizedKVCache(TurboQuantConfig(key_bits=4, value_bits=3, mode="prod"), 1, 64, 2, 64,
                             device=DEV)
    prodc.append(0, torch.randn(2, 20, 64, device=DEV), torch.randn(2, 20, 64, device=DEV))
    w = torch.softmax(prodc.attention_scores(0, torch.randn(2, 1, 64, device=DEV)), -1)
    assert prodc.attention_values(0, w).shape == (2, 1, 64)


@pytest.mark.parametrize("d,vb", [(64, 2), (128, 2), (128, 3)])
def test_cache_gqa_batched_decode_matches_composition(d, vb):
    # the fused decode (decode layout: head_dim 64 and 128) against scores, softmax and
    # values composed from the cache's own ops
    from turboquant_kv import QuantizedKVCache, TurboQuantConfig
    torch.manual_seed(1)
    B, Hq, H, T_ = 2, 8, 2, 700
    kv = QuantizedKVCache(TurboQuantConfig(key_bits=4, value_bits=vb), 1, 1024, H, d, device=DEV,
                          batch_size=B)
    assert kv._dl
    kv.append(0, torch.randn(B, H, 500, d, device=DEV), torch.randn(B, H, 500, d, device=DEV))
    kv.append(0, torch.randn(B, H, T_ - 500, d, device=DEV), torch.randn(B, H, T_ - 500, d, device=DEV))
    q = torch.randn(B, Hq, d, device=DEV)
    fused = kv.decode_attention(0, q)
    logits = kv.attention_scores(0, q.unsqueeze(2))
    ref = kv.attention_values(0, torch.softmax(logits, -1)).squeeze(2)
    assert (fused - ref).abs().max().item() <= 1e-4 * ref.abs().max().item()


@pytest.mark.parametrize("bits,d,mode", [(4, 128, "mse"), (3, 200, "mse"), (4, 64, "prod")])
def test_index_search_k_above_32_ties_and_order(bits, d, mode):
    # k up to 128 runs the fused top-k scans, k above scores every row and selects; both
    # give the core's heap order (score descending, lower index first on a tie): 200
    # duplicated rows tie exactly.
    from turboquant_kv import TurboQuantIndex
    rs = np.random.RandomState(bits * 7 + d)
    db = rs.randn(6000, d).astype(np.float32)
    db[rs.choice(6000, 200, replace=False)] = db[17]
    idx = TurboQuantIndex.from_vectors(torch.from_numpy(db).to(DEV), bit_width=bits, mode=mode)
    q = rs.randn(3, d).astype(np.float32)
    q[0] = db[17]
    for k in (64, 100, 128, 300):
        s, i = idx.search(torch.from_numpy(q).to(DEV), k=k)
        s, i = s.cpu().numpy(), i.cpu().numpy()
        if mode == "mse":
            want_s, want_i = O.search_topk(q, idx._bitplane_codes().cpu().numpy(), idx._norms.cpu().numpy(),
                                           idx._cen.cpu().numpy(), idx._rot_dev.cpu().numpy(), bits, k)
            assert np.array_equal(i, want_i), k
            assert np.array_equal(s.view(np.uint32), want_s.view(np.uint32)), k
        else:  # prod: the heap order over the scan's own scores
            full = idx.search(torch.from_numpy(q).to(DEV), k=6000)[0].cpu().numpy()
            assert (np.diff(s, axis=1) <= 0).all()
            for r in range(3):
                for a in range(k - 1):
                    if s[r, a] == s[r, a + 1]:
                        assert i[r, a] < i[r, a + 1]
            assert np.array_equal(s, full[:, :k])


def test_index_search_many_queries_in_chunks(monkeypatch):
    # A batch larger than one launch's query chunk runs as consecutive launches: the same
    # results as the oracle, for the fused top-k and for k above 32 (whose [Q, N] score
    # matrix is chunked by bytes).
    from turboquant_kv import TurboQuantIndex
    from turboquant_kv import search as S
    monkeypatch.setattr(S, "_SEARCH_CHUNK", 96)
    monkeypatch.setattr(S, "_SCORE_BYTES", 4 * 3000 * 40)
    rs = np.random.RandomState(5)
    db = rs.randn(3000, 128).astype(np.float32)
    idx = TurboQuantIndex.from_vectors(torch.from_numpy(db).to(DEV), bit_width=4)
    q = rs.randn(250, 128).astype(np.float32)
    for k in (10, 40):
        s, i = idx.search(torch.from_numpy(q).to(DEV), k=k)
        want_s, want_i = O.search_topk(q, idx._bitplane_codes().cpu().numpy(), idx._norms.cpu().numpy(),
                                       idx._cen.cpu().numpy(), idx._rot_dev.cpu().numpy(), 4, k)
        assert s.shape == (250, k) and i.shape == (250, k)
        assert np.array_equal(i.cpu().numpy(), want_i), k
        assert np.array_equal(s.cpu().numpy().view(np.uint32), want_s.view(np.uint32)), k
