"""CPU kernels of the five reference schemas (the CPU dispatch key the reference also
registers, csrc/registration.cpp:106-112; kernels csrc/cpu/quant_cpu.cpp).

They must give the reference CPU path's bits:
  * rotate_and_quantize: bit-exact against the C restatement of quant_cpu.cpp:44-118
    (oracle/tq_cpu.c), which is itself pinned here against the reference.py golden codes
    (every code outside the decision band, oracle.check_codes) and against float64 norms
    within the sequential sum's error bound;
  * attention_scores_packed: bit-exact against the oracle's exact-fp32 LUT scores (the
    same sequential sums, quant_cpu.cpp:125-192), within 1e-5 of the float64 closed form;
  * attention_values_packed: bit-exact against an fp32 step-by-step restatement of
    quant_cpu.cpp:199-266 below, within 1e-5 of the float64 closed form values_f64;
  * pack_codes / unpack_codes: bit-exact against the oracle and the reference core's own
    packer (oracle/_ref, where built).
"""

import numpy as np
import pytest
import torch

import cpu_libs
import tq_oracle as O


def _ops():
    from turboquant_kv._lib import HIP_LIB, TORCH_LIB, ops
    import os
    if not (os.path.exists(HIP_LIB) and os.path.exists(TORCH_LIB)):
        pytest.skip("native library not built")
    return ops()


def _t(a):
    return torch.from_numpy(np.ascontiguousarray(a))


@pytest.mark.parametrize("d", [3, 17, 64, 128, 200])
@pytest.mark.parametrize("bits", [1, 2, 3, 4])
def test_rotate_and_quantize_cpu_matches_c_restatement(d, bits):
    if not cpu_libs.have_port():
        pytest.skip("oracle C restatement not built")
    ops = _ops()
    rs = np.random.RandomState(d * 10 + bits)
    x = rs.randn(300, d).astype(np.float32)
    x[0] = 0.0                      # zero row: norm 0, codes of y = 0
    x[1] *= 1e-12                   # below the 1e-10 norm cut
    x[2] *= 1e6
    R = O.dense_qr_rotation(d, 7)
    bnd, _ = O.lloyd_max_codebook(bits, d)
    p, n = ops.rotate_and_quantize(_t(x), _t(R), _t(bnd), bits)
    pw, nw = cpu_libs.rotate_and_quantize(x, R, bnd, bits)
    assert np.array_equal(p.numpy(), pw)
    assert np.array_equal(n.numpy().view(np.uint32), nw.view(np.uint32))


def test_rotate_and_quantize_cpu_other_dtypes_upcast():
    ops = _ops()
    rs = np.random.RandomState(3)
    x = rs.randn(64, 64).astype(np.float32)
    R = O.dense_qr_rotation(64, 42)
    bnd, _ = O.lloyd_max_codebook(3, 64)
    xb = torch.from_numpy(x).to(torch.bfloat16)
    p1, n1 = ops.rotate_and_quantize(xb, _t(R), _t(bnd), 3)
    p2, n2 = ops.rotate_and_quantize(xb.float(), _t(R), _t(bnd), 3)
    assert torch.equal(p1, p2) and torch.equal(n1, n2)


@pytest.mark.parametrize("name,d,bits", [("d64", 64, 2), ("d128", 128, 4), ("d200", 200, 3)])
def test_c_restatement_pinned_by_reference_codes(golden, name, d, bits):
    """The C restatement's codes equal the codes reference.py wrote (golden fixture)
    outside the decision band, and its norms equal the float64 norms within the bound of a
    sequential fp32 sum: a dropped
    term, a transposed R or an off-by-one boundary test moves codes far outside the band."""
    if not cpu_libs.have_port():
        pytest.skip("oracle C restatement not built")
    m, rot = golden("quant_mse"), golden("rotation")
    x, R = m[f"{name}_x"].astype(np.float32), rot[f"R_d{d}_s42"].astype(np.float32)
    bnd, _ = O.lloyd_max_codebook(bits, d)
    pw, nw = cpu_libs.rotate_and_quantize(x, R, bnd, bits)
    want = O.unpack_codes(m[f"{name}_b{bits}_packed"], bits, d)
    got = O.unpack_codes(pw, bits, d)
    n64 = np.sqrt((x.astype(np.float64) ** 2).sum(1))
    # Rows of norm <= 1e-10 are where the reference's two paths part: reference.py divides
    # by max(n, 1e-10) (reference.py:294-295), the CPU kernel multiplies by 0
    # (quant_cpu.cpp:83), so every coordinate is y = 0 and takes the code of 0: the number
    # of boundaries below 0.
    tiny = n64 <= 1e-10
    assert tiny.any() and (~tiny).sum() > 100
    assert (got[tiny] == int((bnd < 0).sum())).all()
    O.check_codes(got[~tiny], want[~tiny], x[~tiny], R, bnd)
    # sequential fp32 sum of d squares: relative error <= (d + 1) u (u = 2^-24); the square
    # root halves it and adds u
    assert np.allclose(nw, n64, rtol=((d + 1) / 2 + 1) * 2.0 ** -24, atol=0)
    # planted mistake: R transposed gives codes far outside the band
    pt, _ = cpu_libs.rotate_and_quantize(x, np.ascontiguousarray(R.T), bnd, bits)
    with pytest.raises(AssertionError):
        O.check_codes(O.unpack_codes(pt, bits, d)[~tiny], want[~tiny], x[~tiny], R, bnd)


@pytest.mark.parametrize("d,bits", [(64, 4), (128, 3), (50, 2), (9, 1)])
def test_attention_scores_cpu(d, bits):
    ops = _ops()
    rs = np.random.RandomState(d + bits)
    B, H, T = 2, 3, 130
    R = O.dense_qr_rotation(d, 42)
    bnd, cen = O.lloyd_max_codebook(bits, d)
    k = rs.randn(T, d).astype(np.float32)
    packed, norms, _ = O.quantize_mse(k, bits, R, bnd)
    q = rs.randn(B, H, d).astype(np.float32)
    s = ops.attention_scores_packed(_t(q), _t(packed), _t(norms), _t(cen), _t(R), bits).numpy()
    want = O.lut_scores_f32(q.reshape(B * H, d), packed, norms, cen, R, bits).reshape(B, H, T)
    assert np.array_equal(s.view(np.uint32), want.view(np.uint32))
    f64 = O.scores_f64(q.reshape(B * H, d), packed, norms, cen, R, bits).reshape(B, H, T)
    assert np.allclose(s, f64, rtol=1e-5, atol=1e-5 * np.abs(f64).max())


def _values_f32_steps(w, packed, norms, cen, RT, bits):
    """quant_cpu.cpp:199-266 step by step in float32: r_j = sum_t (w_t c[code_tj]) n_t in t
    order, out_k = sum_j r_j RT[j][k] in j order (one rounding per operation)."""
    d = RT.shape[0]
    codes = O.unpack_codes(packed, bits, d)
    cen = np.asarray(cen, np.float32)
    acc = np.zeros((w.shape[0], d), np.float32)
    for t in range(w.shape[1]):
        acc = (acc + ((w[:, t:t + 1] * cen[codes[t]][None, :]).astype(np.float32)
                      * np.float32(norms[t])).astype(np.float32)).astype(np.float32)
    out = np.zeros((w.shape[0], d), np.float32)
    for j in range(d):
        out = (out + (acc[:, j:j + 1] * RT[j][None, :]).astype(np.float32)).astype(np.float32)
    return out


@pytest.mark.parametrize("d,bits", [(64, 2), (128, 4), (33, 3)])
def test_attention_values_cpu(d, bits):
    ops = _ops()
    rs = np.random.RandomState(5 * d + bits)
    B, H, T = 2, 2, 97
    R = O.dense_qr_rotation(d, 43)
    bnd, cen = O.lloyd_max_codebook(bits, d)
    v = rs.randn(T, d).astype(np.float32)
    packed, norms, _ = O.quantize_mse(v, bits, R, bnd)
    w = rs.rand(B, H, T).astype(np.float32)
    w /= w.sum(-1, keepdims=True)
    out = ops.attention_values_packed(_t(w), _t(packed), _t(norms), _t(cen), _t(R), bits).numpy()
    steps = _values_f32_steps(w.reshape(B * H, T), packed, norms, cen, R, bits).reshape(B, H, d)
    assert np.array_equal(out.view(np.uint32), steps.view(np.uint32))
    f64 = O.values_f64(w.reshape(B * H, T), packed, norms, cen, R, bits).reshape(B, H, d)
    assert np.allclose(out, f64, rtol=1e-5, atol=1e-5 * np.abs(f64).max())
    # a transposed rotation is a different answer (the check above would catch it)
    bad = O.values_f64(w.reshape(B * H, T), packed, norms, cen, R.T, bits).reshape(B, H, d)
    assert not np.allclose(out, bad, rtol=1e-3, atol=1e-3 * np.abs(f64).max())


@pytest.mark.parametrize("bits", [1, 2, 3, 4, 8])
@pytest.mark.parametrize("d", [1, 8, 13, 64, 200])
def test_pack_unpack_cpu(bits, d):
    ops = _ops()
    rs = np.random.RandomState(bits * 1000 + d)
    codes = rs.randint(0, 1 << bits, size=(37, d)).astype(np.uint8)
    p = ops.pack_codes(_t(codes), bits).numpy()
    assert np.array_equal(p, O.pack_codes(codes, bits))
    if cpu_libs.have_ref() and bits <= 4:
        assert np.array_equal(p, cpu_libs.ref_pack_codes(codes, bits))
    u = ops.unpack_codes(_t(p), bits, d).numpy()
    assert np.array_equal(u, codes)


def test_cpu_kernels_reject_bad_shapes():
    ops = _ops()
    with pytest.raises(RuntimeError, match="packed dim mismatch"):
        ops.unpack_codes(torch.zeros(2, 5, dtype=torch.uint8), 4, 64)
    with pytest.raises(RuntimeError, match="bit_width"):
        ops.rotate_and_quantize(torch.randn(2, 8), torch.eye(8), torch.zeros(31), 5)
    with pytest.raises(RuntimeError, match="packed dim mismatch"):
        ops.attention_scores_packed(torch.randn(1, 1, 64), torch.zeros(4, 8, dtype=torch.uint8),
                                    torch.ones(4), torch.zeros(16), torch.eye(64), 4)
    with pytest.raises(RuntimeError, match="seq_len"):
        ops.attention_values_packed(torch.rand(1, 1, 4), torch.zeros(3, 16, dtype=torch.uint8),
                                    torch.ones(3), torch.zeros(4), torch.eye(64), 2)
