"""CPU tests: the oracle pinned against the reference's golden vectors, closed forms and
invariants; the C restatement and the reference's compiled core against the oracle.

A failing test here means the checker itself is wrong, so every GPU parity claim
that relies on it would be void.
"""

import math

import numpy as np
import pytest

import tq_oracle as O
import cpu_libs

CASES = {"d128": (128, (2, 3, 4)), "d200": (200, (3, 4)), "d64": (64, (2, 3, 4))}


# ------------------------------------------------------------------ codebook
def test_codebook_bits_match_reference(golden):
    cb = golden("codebook")
    for b in range(1, 6):
        for d in (64, 128, 200):
            bnd, cen = O.lloyd_max_codebook(b, d)
            assert np.array_equal(bnd.view(np.uint32), cb[f"bnd_b{b}_d{d}"].view(np.uint32)), (b, d)
            assert np.array_equal(cen.view(np.uint32), cb[f"cen_b{b}_d{d}"].view(np.uint32)), (b, d)


def test_codebook_closed_form_b1():
    # b=1: centroids +-E|X| = +-sqrt(2/pi), scaled by 1/sqrt(d) (test_reference.py:31-44)
    for d in (64, 128, 256):
        _, c = O.lloyd_max_codebook(1, d)
        assert abs(c[1] - math.sqrt(2 / math.pi) / math.sqrt(d)) < 1e-7
        assert c[0] == -c[1]


def test_codebook_converged_b2_is_lloyd_fixed_point():
    # b=2 converges: centroids equal the conditional means of their cells, and the
    # values sit near Max (1960)'s table (+-0.4528, +-1.510).
    from scipy.stats import norm
    b, c = O.lloyd_max_unscaled(2)
    e = np.concatenate([[-np.inf], b, [np.inf]])
    cm = (norm.pdf(e[:-1]) - norm.pdf(e[1:])) / (norm.cdf(e[1:]) - norm.cdf(e[:-1]))
    assert np.max(np.abs(cm - c)) < 1e-11
    assert np.allclose(c, [-1.510, -0.4528, 0.4528, 1.510], atol=1e-3)


def test_codebook_sorted_and_symmetric():
    for b in (1, 2, 3, 4):
        bnd, cen = O.lloyd_max_codebook(b, 128)
        assert np.all(np.diff(bnd) > 0) and np.all(np.diff(cen) > 0)
        assert np.allclose(cen, -cen[::-1], atol=1e-6)


# ------------------------------------------------------------------ rotation / qjl
def test_rotation_and_qjl_bits_match_reference(golden):
    rot, qj = golden("rotation"), golden("qjl")
    for d in (64, 128, 200):
        for s in (42, 43):
            assert np.array_equal(O.dense_qr_rotation(d, s), rot[f"R_d{d}_s{s}"])
            assert np.array_equal(O.qjl_matrix(d, d, s), qj[f"S_d{d}_s{s}"])


def test_rotation_orthogonal(golden):
    rot = golden("rotation")
    for key in rot.files:
        R = rot[key].astype(np.float64)
        assert np.allclose(R @ R.T, np.eye(R.shape[0]), atol=1e-4 if "RHT" in key else 1e-5), key


# ------------------------------------------------------------------ packing
def test_pack_known_answer():
    # codes 0..7 at b=3, d=8: plane0 = bits0 = 0,1,0,1,0,1,0,1 -> 0b01010101
    codes = np.arange(8, dtype=np.uint8)[None, :]
    assert O.pack_codes(codes, 3).tolist() == [[0x55, 0x33, 0x0F]]
    # d=10 pads bits of the second byte with zeros; dim 8 -> bit 7, dim 9 -> bit 6
    c = np.zeros((1, 10), np.uint8)
    c[0, 8] = 1
    c[0, 0] = 1
    assert O.pack_codes(c, 1).tolist() == [[0x80, 0x80]]
    c[0, 9] = 1
    assert O.pack_codes(c, 1).tolist() == [[0x80, 0xC0]]


def test_pack_unpack_brute_force_tiny():
    # every 2-dim code pair at b=2 and d=3 (one pad bit pattern per row)
    rows = np.array([[a, b, c] for a in range(4) for b in range(4) for c in range(4)], np.uint8)
    packed = O.pack_codes(rows, 2)
    assert packed.shape == (64, 2)
    for r, pk in zip(rows, packed):
        expect0 = ((r[0] & 1) << 7) | ((r[1] & 1) << 6) | ((r[2] & 1) << 5)
        expect1 = ((r[0] >> 1) << 7) | ((r[1] >> 1) << 6) | ((r[2] >> 1) << 5)
        assert pk.tolist() == [expect0, expect1]
    assert np.array_equal(O.unpack_codes(packed, 2, 3), rows)


@pytest.mark.parametrize("bits", [1, 2, 3, 4, 8])
@pytest.mark.parametrize("d", [1, 7, 32, 64, 100, 200, 256])
def test_pack_roundtrip(bits, d):
    rs = np.random.RandomState(bits * 1000 + d)
    codes = rs.randint(0, 1 << bits, (50, d)).astype(np.uint8)
    assert np.array_equal(O.unpack_codes(O.pack_codes(codes, bits), bits, d), codes)


@pytest.mark.skipif(not cpu_libs.have_ref(), reason="reference core not built here")
def test_pack_matches_reference_core():
    rs = np.random.RandomState(3)
    for bits, d in ((1, 64), (3, 200), (4, 128)):
        codes = rs.randint(0, 1 << bits, (40, d)).astype(np.uint8)
        assert np.array_equal(cpu_libs.ref_pack_codes(codes, bits), O.pack_codes(codes, bits))


# ------------------------------------------------------------------ the reference's CPU kernels
# csrc/cpu/quant_cpu.cpp compiled from the reference's source against the installed torch
# (oracle/_ref/libquant_cpu_ref.so, through oracle/ref_quant_cpu_shim.cpp).
_REF_CPU = pytest.mark.skipif(not cpu_libs.have_ref_cpu(), reason="reference CPU kernels not built here")


@_REF_CPU
def test_quantize_port_bit_exact_with_reference_cpu_kernel():
    # rotate_and_quantize_cpu (quant_cpu.cpp:44-118): the C restatement timed as the config-0
    # CPU baseline returns its codes and norms bit for bit; the numpy oracle's codes agree
    # outside their ambiguity band.  Heavy-tailed rows, a zero row and a 1e-12-scaled row.
    rs = np.random.RandomState(21)
    for d, b in ((64, 2), (128, 4), (200, 3), (128, 1)):
        R = O.dense_qr_rotation(d, 42)
        bnd, _ = O.lloyd_max_codebook(b, d)
        x = (rs.randn(700, d) * rs.lognormal(size=(1, d))).astype(np.float32)
        x[3] = 0.0
        x[5] *= np.float32(1e-12)
        pr, nr = cpu_libs.ref_cpu_rotate_and_quantize(x, R, bnd, b)
        pp, npo = cpu_libs.rotate_and_quantize(x, R, bnd, b)
        assert np.array_equal(pp, pr), (d, b)
        assert np.array_equal(npo.view(np.uint32), nr.view(np.uint32)), (d, b)
        _, n, codes = O.quantize_mse(x, b, R, bnd)
        refc = O.unpack_codes(pr, b, d)
        # rows of norm <= 1e-10: the CPU kernel multiplies them by 0 (quant_cpu.cpp:83, the
        # code of 0 everywhere) where reference.py divides by max(n, 1e-10) (the oracle)
        tiny = nr <= np.float32(1e-10)
        assert tiny[3] and tiny[5] and tiny.sum() == 2
        assert (refc[tiny] == np.searchsorted(bnd, np.float32(0.0), side="left")).all()
        O.check_codes(codes[~tiny], refc[~tiny], x[~tiny], R, bnd)
        # norms: d squares summed in another order (numpy's pairwise sum vs the kernel's loop)
        assert np.allclose(n, nr, rtol=d * 2.0 ** -24, atol=0)


@_REF_CPU
def test_scores_oracle_bit_exact_with_reference_cpu_kernel():
    # attention_scores_packed_cpu (quant_cpu.cpp:125-197) against the oracle's exact-fp32
    # LUT scores (the arithmetic the GPU scans are held to), batch x heads queries
    rs = np.random.RandomState(22)
    for d, b in ((64, 3), (128, 4), (200, 2)):
        R = O.dense_qr_rotation(d, 42)
        bnd, cen = O.lloyd_max_codebook(b, d)
        packed, norms, _ = O.quantize_mse(rs.randn(900, d).astype(np.float32), b, R, bnd)
        q = rs.randn(2, 3, d).astype(np.float32)
        got = cpu_libs.ref_cpu_attention_scores(q, packed, norms, cen, R, b)
        want = O.lut_scores_f32(q.reshape(6, d), packed, norms, cen, R, b).reshape(2, 3, -1)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (d, b)


@_REF_CPU
def test_values_oracle_matches_reference_cpu_kernel():
    # attention_values_packed_cpu (quant_cpu.cpp:199-266), fp32, against the oracle's
    # float64 closed form with M = R (what the reference's `rotation_T` argument is given)
    rs = np.random.RandomState(23)
    for d, b in ((64, 2), (128, 3), (200, 4)):
        R = O.dense_qr_rotation(d, 43)
        bnd, cen = O.lloyd_max_codebook(b, d)
        packed, norms, _ = O.quantize_mse(rs.randn(500, d).astype(np.float32), b, R, bnd)
        w = rs.rand(2, 2, 500).astype(np.float32)
        w /= w.sum(-1, keepdims=True)
        got = cpu_libs.ref_cpu_attention_values(w, packed, norms, cen, R, b, d)
        want = O.values_f64(w.reshape(4, 500), packed, norms, cen, R, b).reshape(2, 2, d)
        assert np.allclose(got, want, rtol=1e-5, atol=1e-5 * np.abs(want).max()), (d, b)
        wrong = O.values_f64(w.reshape(4, 500), packed, norms, cen, R.T.copy(), b).reshape(2, 2, d)
        assert np.abs(got - wrong).max() > 0.1 * np.abs(want).max()


# ------------------------------------------------------------------ quantize
def test_searchsorted_tie_goes_low():
    bnd = np.array([-1.0, 0.0, 1.0], np.float32)
    y = np.array([[-1.0, 0.0, 1.0, 1.0000001, -2.0, 2.0]], np.float32)
    assert np.searchsorted(bnd, y, side="left").tolist() == [[0, 1, 2, 3, 0, 3]]


def test_quantize_mse_fp32_matches_reference(golden):
    m, rot = golden("quant_mse"), golden("rotation")
    for name, (d, bl) in CASES.items():
        x, R = m[f"{name}_x"], rot[f"R_d{d}_s42"]
        for b in bl:
            bnd, _ = O.lloyd_max_codebook(b, d)
            _, n, codes = O.quantize_mse(x, b, R, bnd)
            ref = O.unpack_codes(m[f"{name}_b{b}_packed"], b, d)
            info = O.check_codes(codes, ref, x, R, bnd)
            print(name, b, info)
            assert info["band"] < 2e-4 * info["coords"]
            assert np.allclose(n, m[f"{name}_b{b}_norms"], rtol=2e-7, atol=0)


def test_quantize_mse_bf16_matches_reference(golden):
    m, rot = golden("quant_mse"), golden("rotation")
    x = O.bf16_bits_to_f32(m["bf16_d64_x_u16"])
    R = rot["R_d64_s42"]
    for b in (2, 3, 4):
        bnd, _ = O.lloyd_max_codebook(b, 64)
        _, n, codes = O.quantize_mse(x, b, R, bnd, "bf16")
        ref = O.unpack_codes(m[f"bf16_d64_b{b}_packed"], b, 64)
        O.check_codes(codes, ref, x, R, bnd, "bf16")
        assert np.array_equal(n, O.bf16_bits_to_f32(m[f"bf16_d64_b{b}_norms_u16"]))


def test_zero_and_tiny_rows_fixed_by_fixture(golden):
    # zero row: every rotated coordinate is 0 -> code #{bnd < 0}; the middle
    # boundary is ~1e-17, not 0, so b=2 gives 2 and b=3/4 give 2^(b-1)-1.
    m = golden("quant_mse")
    for b, expect in ((2, 2), (3, 3), (4, 7)):
        ref = O.unpack_codes(m[f"d128_b{b}_packed"][:1], b, 128)
        assert np.all(ref == expect), b
        assert m[f"d128_b{b}_norms"][0] == 0.0


def test_margin_catches_planted_mistake(golden):
    # An oracle that forgets to normalize the second time in prod mode, or that
    # rotates with R instead of R^T, must disagree with the reference outside the band.
    m, rot = golden("quant_mse"), golden("rotation")
    x, R = m["d128_x"], rot["R_d128_s42"]
    bnd, _ = O.lloyd_max_codebook(4, 128)
    ref = O.unpack_codes(m["d128_b4_packed"], 4, 128)
    amb = O.code_margin(x, R, bnd)
    _, _, wrong = O.quantize_mse(x, 4, R.T.copy(), bnd)  # transposed operand
    assert np.sum((wrong != ref) & ~amb) > 1000


def test_quantize_prod_matches_reference(golden):
    pr, rot, qj = golden("quant_prod"), golden("rotation"), golden("qjl")
    for name, d in (("d128", 128), ("d200", 200)):
        x, R, S = pr[f"{name}_x"], rot[f"R_d{d}_s42"], qj[f"S_d{d}_s42"]
        bnd, cen = O.lloyd_max_codebook(3, d)
        mp, sg, g, n, codes, proj64 = O.quantize_prod(x, 4, R, bnd, cen, S)
        assert np.array_equal(mp, pr[f"{name}_mse_packed"])
        assert np.array_equal(sg, pr[f"{name}_signs"])
        assert np.allclose(g, pr[f"{name}_res_norms"], rtol=1e-6)
        assert np.allclose(n, pr[f"{name}_norms"], rtol=1e-6)


def test_dequantize_matches_reference(golden):
    m, pr, rot, qj = golden("quant_mse"), golden("quant_prod"), golden("rotation"), golden("qjl")
    for name, (d, bl) in CASES.items():
        R = rot[f"R_d{d}_s42"]
        for b in bl:
            _, cen = O.lloyd_max_codebook(b, d)
            got = O.dequantize_mse(m[f"{name}_b{b}_packed"][:64], m[f"{name}_b{b}_norms"][:64], b, d, R, cen)
            assert np.allclose(got, m[f"{name}_b{b}_deq64"], rtol=1e-5, atol=1e-5)
    for name, d in (("d128", 128), ("d200", 200)):
        R, S = rot[f"R_d{d}_s42"], qj[f"S_d{d}_s42"]
        _, cen = O.lloyd_max_codebook(3, d)
        got = O.dequantize_prod(pr[f"{name}_mse_packed"][:64], pr[f"{name}_signs"][:64],
                                pr[f"{name}_res_norms"][:64], pr[f"{name}_norms"][:64], 4, d, R, cen, S)
        ref = pr[f"{name}_deq64"]
        assert np.max(np.abs(got - ref)) <= 1e-5 * np.max(np.abs(ref))


def test_prod_scores_match_reference_reconstruction(golden):
    # prod_scores_f64 against queries @ (the reference's own dequantize_prod output)^T
    pr, rot, qj = golden("quant_prod"), golden("rotation"), golden("qjl")
    rs = np.random.RandomState(5)
    for name, d in (("d128", 128), ("d200", 200)):
        R, S = rot[f"R_d{d}_s42"], qj[f"S_d{d}_s42"]
        _, cen = O.lloyd_max_codebook(3, d)
        q = rs.randn(6, d).astype(np.float32)
        got = O.prod_scores_f64(q, pr[f"{name}_mse_packed"][:64], pr[f"{name}_signs"][:64],
                                pr[f"{name}_res_norms"][:64], pr[f"{name}_norms"][:64], 4, d,
                                R, cen, S)
        ref = q.astype(np.float64) @ pr[f"{name}_deq64"].astype(np.float64).T
        # row 0 of the fixture is the zero vector (norm 0): its scores are exactly 0
        scale = np.linalg.norm(q, axis=1)[:, None] * pr[f"{name}_norms"][None, :64]
        assert np.all(np.abs(got - ref) <= 1e-5 * scale)


def _prod_fused_f64(q, mp, sg, g, n, bits, d, R, cen, S):
    """The scan kernels' rearrangement: n * (<R q, c[codes]> + sqrt(pi/2)/d * g * <S q, +-1>)."""
    codes = O.unpack_codes(mp, bits - 1, d)
    sgn = 2.0 * O.unpack_codes(sg, 1, d).astype(np.float64) - 1.0
    q64 = np.asarray(q, np.float64)
    qr, qs = q64 @ np.asarray(R, np.float64).T, q64 @ np.asarray(S, np.float64).T
    mse = qr @ np.asarray(cen, np.float64)[codes].T
    corr = math.sqrt(math.pi / 2) / d * g[None, :].astype(np.float64) * (qs @ sgn.T)
    return (mse + corr) * n[None, :].astype(np.float64)


def test_prod_scores_rearrangement_and_special_cases(golden):
    pr, rot, qj = golden("quant_prod"), golden("rotation"), golden("qjl")
    d, R, S = 128, rot["R_d128_s42"], qj["S_d128_s42"]
    _, cen = O.lloyd_max_codebook(3, d)
    mp, sg = pr["d128_mse_packed"], pr["d128_signs"]
    g, n = pr["d128_res_norms"], pr["d128_norms"]
    q = np.random.RandomState(9).randn(4, d).astype(np.float32)
    ref = O.prod_scores_f64(q, mp, sg, g, n, 4, d, R, cen, S)
    scale = np.max(np.abs(ref))
    # the scan kernels' form of the same score
    assert np.max(np.abs(_prod_fused_f64(q, mp, sg, g, n, 4, d, R, cen, S) - ref)) <= 1e-12 * scale
    # gamma = 0 leaves the (bits-1)-bit MSE score
    z = np.zeros_like(g)
    assert np.allclose(O.prod_scores_f64(q, mp, sg, z, n, 4, d, R, cen, S),
                       O.scores_f64(q, mp, n, cen, R, 3), rtol=0, atol=1e-12 * scale)
    # flipping every sign negates the residual term
    mse = O.scores_f64(q, mp, n, cen, R, 3)
    flip = O.prod_scores_f64(q, mp, (~sg).astype(np.uint8), g, n, 4, d, R, cen, S)
    assert np.allclose(flip - mse, -(ref - mse), rtol=0, atol=1e-10 * scale)
    # a transposed S in the rearrangement is caught
    bad = _prod_fused_f64(q, mp, sg, g, n, 4, d, R, cen, S.T.copy())
    assert np.max(np.abs(bad - ref)) > 1e-3 * scale


def test_mse_distortion_bound():
    # mean over vectors of mean_j (x - x_hat)^2 < 2 * sqrt(3 pi)/2 * 4^-b
    # (reference tests/test_reference.py:74-100)
    rs = np.random.RandomState(0)
    d = 128
    R = O.dense_qr_rotation(d, 42)
    x = rs.randn(500, d).astype(np.float32)
    x /= np.linalg.norm(x, axis=1, keepdims=True)
    for b in (1, 2, 3, 4):
        bnd, cen = O.lloyd_max_codebook(b, d)
        p, n, _ = O.quantize_mse(x, b, R, bnd)
        rec = O.dequantize_mse(p, n, b, d, R, cen)
        avg = float(np.mean(np.mean((x - rec) ** 2, axis=1)))
        assert avg < 2 * math.sqrt(3 * math.pi) / 2 * 4.0 ** (-b), b


# ------------------------------------------------------------------ scoring
def test_index_search_matches_reference(golden):
    ix, m, rot = golden("index"), golden("quant_mse"), golden("rotation")
    R, q = rot["R_d128_s42"], ix["queries"]
    for b in (2, 3, 4):
        _, cen = O.lloyd_max_codebook(b, 128)
        s, i = O.search_topk(q, ix[f"b{b}_packed"], m[f"d128_b{b}_norms"], cen, R, b, 10)
        assert np.array_equal(i, ix[f"b{b}_ids"]), b
        assert np.allclose(s, ix[f"b{b}_scores"], rtol=1e-5, atol=1e-6)


def test_lut_scores_equal_closed_form():
    rs = np.random.RandomState(5)
    d, b = 64, 3
    R = O.dense_qr_rotation(d, 42)
    bnd, cen = O.lloyd_max_codebook(b, d)
    x = rs.randn(300, d).astype(np.float32)
    p, n, _ = O.quantize_mse(x, b, R, bnd)
    q = rs.randn(4, d).astype(np.float32)
    s32 = O.lut_scores_f32(q, p, n, cen, R, b)
    s64 = O.scores_f64(q, p, n, cen, R, b)
    assert np.max(np.abs(s32 - s64)) <= 1e-5 * np.max(np.abs(s64))
    # and the closed form equals q . dequantize(x) exactly in exact arithmetic
    rec = O.dequantize_mse(p, n, b, d, R, cen).astype(np.float64)
    assert np.allclose(s64, q.astype(np.float64) @ rec.T, rtol=1e-5, atol=1e-5)


def test_topk_tie_order_and_padding():
    s = np.array([[1.0, 3.0, 3.0, 2.0, 3.0]], np.float32)
    ts, ti = O.topk_desc(s, 7)
    assert ti.tolist() == [[1, 2, 4, 3, 0, -1, -1]]
    assert np.isneginf(ts[0, 5:]).all()


@pytest.mark.parametrize("which", ["port", "ref"])
def test_c_search_bit_exact_with_oracle(golden, which):
    if which == "ref" and not cpu_libs.have_ref():
        pytest.skip("reference core not built here")
    ix, m, rot = golden("index"), golden("quant_mse"), golden("rotation")
    R, q = rot["R_d128_s42"], ix["queries"]
    for b in (2, 3, 4):
        _, cen = O.lloyd_max_codebook(b, 128)
        p, n = ix[f"b{b}_packed"], m[f"d128_b{b}_norms"]
        s0, i0 = O.search_topk(q, p, n, cen, R, b, 10)
        s1, i1 = cpu_libs.search_packed(q, p, n, R, cen, b, 10, which)
        assert np.array_equal(i0, i1)
        assert np.array_equal(s0.view(np.uint32), s1.view(np.uint32))


def test_c_search_port_tie_order_equals_oracle():
    # Exactly tied scores (duplicated rows) and k past the ties: the C restatement lists
    # them as the oracle does, score descending then lower index first.
    rs = np.random.RandomState(8)
    d, b, N = 64, 4, 3000
    R = O.dense_qr_rotation(d, 42)
    bnd, cen = O.lloyd_max_codebook(b, d)
    x = rs.randn(N, d).astype(np.float32)
    p, n, _ = O.quantize_mse(x, b, R, bnd)
    q = rs.randn(3, d).astype(np.float32)
    top = np.argsort(-O.lut_scores_f32(q, p, n, cen, R, b), axis=1)[:, :3]
    for r in range(3):
        for j in range(3):
            dst = rs.choice(N, 7, replace=False)
            p[dst], n[dst] = p[top[r, j]], n[top[r, j]]
    for k in (5, 16, 32):
        s0, i0 = O.search_topk(q, p, n, cen, R, b, k)
        s1, i1 = cpu_libs.search_packed(q, p, n, R, cen, b, k, "port")
        assert np.array_equal(i0, i1), k
        assert np.array_equal(s0.view(np.uint32), s1.view(np.uint32)), k


def test_cache_fixture_matches_oracle(golden):
    c, rot = golden("cache"), golden("rotation")
    R, Rv = rot["R_d64_s42"], rot["R_d64_s43"]
    bk, ck = O.lloyd_max_codebook(4, 64)
    bv, cv = O.lloyd_max_codebook(2, 64)
    for h in range(4):
        assert np.array_equal(O.quantize_mse(c["keys"][h], 4, R, bk)[0], c["key_packed"][h])
        assert np.array_equal(O.quantize_mse(c["values"][h], 2, Rv, bv)[0], c["val_packed"][h])
    out = O.decode_attention_f64(c["query"][None, :, 0], c["key_packed"][None], c["key_norms"][None],
                                 c["val_packed"][None], c["val_norms"][None], [128], ck, cv, R, Rv,
                                 4, 2, 1 / 8)
    assert np.max(np.abs(out[0] - c["output"][:, 0])) <= 1e-5 * np.max(np.abs(c["output"]))


# ------------------------------------------------------------------ paged KV
def _to_pool(rows, bs, table, nblocks):
    """[H, T, ...] rows -> a pool [nblocks, H, bs, ...] holding token t in block
    table[t // bs] at slot t % bs (a plain loop, independent of paged_rows)."""
    H, T = rows.shape[:2]
    pool = np.zeros((nblocks, H, bs) + rows.shape[2:], rows.dtype)
    for t in range(T):
        pool[table[t // bs], :, t % bs] = rows[:, t]
    return pool


def test_paged_oracle_matches_reference_cache_output(golden):
    # The reference's own QuantizedKVCache output (128 tokens, 4 heads) from rows placed
    # in scattered blocks of 16: one new token at position 127 sees every token.
    c, rot = golden("cache"), golden("rotation")
    R, Rv = rot["R_d64_s42"], rot["R_d64_s43"]
    _, ck = O.lloyd_max_codebook(4, 64)
    _, cv = O.lloyd_max_codebook(2, 64)
    table = np.random.RandomState(0).permutation(20)[:8]
    pools = [_to_pool(c[k], 16, table, 20) for k in ("key_packed", "key_norms", "val_packed", "val_norms")]
    out = O.paged_attention_f64(c["query"][:, 0][None], *pools, table, 128, ck, cv, R, Rv, 4, 2, 1 / 8)
    assert np.max(np.abs(out[0] - c["output"][:, 0])) <= 1e-5 * np.max(np.abs(c["output"]))


def test_paged_oracle_causal_rows_and_block_invariance(golden):
    c, rot = golden("cache"), golden("rotation")
    R, Rv = rot["R_d64_s42"], rot["R_d64_s43"]
    _, ck = O.lloyd_max_codebook(4, 64)
    _, cv = O.lloyd_max_codebook(2, 64)
    rs = np.random.RandomState(1)
    q = rs.randn(6, 8, 64)                       # 6 new tokens, 8 query heads on 4 kv heads (GQA)
    T = 100
    keys = ("key_packed", "key_norms", "val_packed", "val_norms")
    t1 = rs.permutation(16)[:7]
    t2 = rs.permutation(16)[:7]
    p1 = [_to_pool(c[k][:, :T], 16, t1, 16) for k in keys]
    p2 = [_to_pool(c[k][:, :T], 16, t2, 16) for k in keys]
    a = O.paged_attention_f64(q, *p1, t1, T, ck, cv, R, Rv, 4, 2, 0.125)
    b = O.paged_attention_f64(q, *p2, t2, T, ck, cv, R, Rv, 4, 2, 0.125)
    assert np.allclose(a, b, rtol=0, atol=1e-12)            # physical placement is invisible
    # row i = one-token decode over the first T-6+i+1 tokens, kv head h // 2
    for i in range(6):
        vis = T - 6 + i + 1
        qq = q[i][None]
        dec = O.decode_attention_f64(qq, c["key_packed"][None, :, :vis],
                                     c["key_norms"][None, :, :vis], c["val_packed"][None, :, :vis],
                                     c["val_norms"][None, :, :vis], [vis], ck, cv, R, Rv, 4, 2, 0.125)
        assert np.allclose(a[i], dec[0], rtol=0, atol=1e-10), i
    # a planted mistake -- tokens addressed as (slot, block) instead of (block, slot) --
    # reorders the context, which the causal rows see
    def swapped(x):
        return np.swapaxes(x.reshape(4, 6, 16, *x.shape[2:]), 1, 2).reshape(x.shape)
    right = O.paged_attention_f64(q, *[_to_pool(c[k][:, :96], 16, t1, 16) for k in keys],
                                  t1, 96, ck, cv, R, Rv, 4, 2, 0.125)
    wrong = O.paged_attention_f64(q, *[_to_pool(swapped(c[k][:, :96]), 16, t1, 16) for k in keys],
                                  t1, 96, ck, cv, R, Rv, 4, 2, 0.125)
    assert np.max(np.abs(wrong - right)) > 1e-3


def test_values_f64_equals_weights_times_dequantized_rows():
    # attention_values_packed's closed form (quant_cpu.cpp:199-266) with M = R is the
    # attention weights times the dequantized rows (reference.py:320-367); with R^T (the
    # mistake the reference's `rotation_T` name invites) it is not.
    rs = np.random.RandomState(12)
    for d, b in ((64, 2), (128, 3), (200, 4)):
        R = O.dense_qr_rotation(d, 43)
        bnd, cen = O.lloyd_max_codebook(b, d)
        x = rs.randn(300, d).astype(np.float32)
        packed, norms, _ = O.quantize_mse(x, b, R, bnd)
        w = rs.rand(5, 300)
        got = O.values_f64(w, packed, norms, cen, R, b)
        want = w @ O.dequantize_mse(packed, norms, b, d, R, cen).astype(np.float64)
        assert np.allclose(got, want, rtol=1e-5, atol=1e-6 * np.abs(want).max())
        wrong = O.values_f64(w, packed, norms, cen, R.T.copy(), b)
        assert np.abs(wrong - want).max() > 0.1 * np.abs(want).max()
        # linear in the weights
        assert np.allclose(O.values_f64(2 * w[:1] + w[1:2], packed, norms, cen, R, b),
                           2 * got[:1] + got[1:2], rtol=1e-12, atol=1e-12)


def test_bf16_reference_emulation_rounds_only_where_the_reference_does():
    # The emulation departs from the float64 closed form by bf16-sized amounts (its
    # history and output are rounded to bf16), no less and not much more, and its
    # outputs are bf16 values.
    rs = np.random.RandomState(13)
    d, B, Hq, Hkv, T = 64, 2, 4, 2, 50
    Rk, Rv = O.dense_qr_rotation(d, 42), O.dense_qr_rotation(d, 43)
    bk, ck = O.lloyd_max_codebook(4, d)
    bv, cv = O.lloyd_max_codebook(2, d)
    K = rs.randn(B * Hkv * T, d).astype(np.float32)
    V = rs.randn(B * Hkv * T, d).astype(np.float32)
    kp, kn, _ = O.quantize_mse(K, 4, Rk, bk)
    vp, vn, _ = O.quantize_mse(V, 2, Rv, bv)
    kp, vp = kp.reshape(B, Hkv, T, -1), vp.reshape(B, Hkv, T, -1)
    kn, vn = kn.reshape(B, Hkv, T), vn.reshape(B, Hkv, T)
    q = O.round_bf16(rs.randn(B, Hq, d).astype(np.float32))
    exact = O.decode_attention_f64(q, kp, kn, vp, vn, [T, 17], ck, cv, Rk, Rv, 4, 2, 0.125)
    emul = O.decode_attention_bf16_reference(q, kp, kn, vp, vn, [T, 17], ck, cv, Rk, Rv, 4, 2, 0.125)
    rel = np.abs(emul - exact).max() / np.abs(exact).max()
    assert 1e-4 < rel < 5e-2, rel
    assert np.array_equal(emul, O.round_bf16(emul.astype(np.float32)))  # bf16 outputs
