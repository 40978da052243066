"""GPU parity tests of the C ABI (include/turboquant_hip.h) against the oracle and the
reference's golden vectors.  Tolerances are written in each test:

* codes / sign bits / packed bytes / top-k ids: bit-exact, except codes whose fp64
  distance to a decision point is inside the fp32 band of tq_oracle.code_margin
  (those are counted and bounded);
* ADC scores: bit-exact with the oracle's exact-float32 LUT evaluation (same order
  of operations as the reference's C++ core);
* float outputs (norms, dequantized vectors, values, attention): relative bounds.
"""

import ctypes
import math

import numpy as np
import pytest
import torch

import capi
import tq_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"
L = capi.lib


_ALIVE = []


def T(a, dtype=None):
    """Device copy of a numpy array, kept alive until the next wrapper call: a pointer
    handed to the C ABI must outlive the asynchronous kernel that reads it."""
    t = torch.from_numpy(np.ascontiguousarray(a)).to(DEV)
    t = t if dtype is None else t.to(dtype)
    _ALIVE.append(t)
    return t


def sync():
    torch.cuda.synchronize()
    _ALIVE.clear()


# ------------------------------------------------------------------ wrappers
def k_quantize(x_t, R, bnd, bits, in_dt=capi.TQ_F32, rdt=capi.TQ_F32):
    n, d = x_t.shape
    packed = torch.empty(n, bits * ((d + 7) // 8), dtype=torch.uint8, device=DEV)
    norms = torch.empty(n, dtype=torch.float32, device=DEV)
    capi.check(L().tq_rotate_and_quantize(capi.p(x_t), in_dt, rdt, capi.i64(n), capi.i32(d),
                                          capi.p(T(R)), capi.p(T(bnd)), capi.i32(bits),
                                          capi.p(packed), capi.p(norms), capi.stream()))
    sync()
    return packed.cpu().numpy(), norms.cpu().numpy()


def k_prod(x, R, bnd, cen, S, bits):
    n, d = x.shape
    bpp = (d + 7) // 8
    mp = torch.empty(n, (bits - 1) * bpp, dtype=torch.uint8, device=DEV)
    sg = torch.empty(n, bpp, dtype=torch.uint8, device=DEV)
    rn = torch.empty(n, dtype=torch.float32, device=DEV)
    nm = torch.empty(n, dtype=torch.float32, device=DEV)
    capi.check(L().tq_quantize_prod(capi.p(T(x)), capi.TQ_F32, capi.TQ_F32, capi.i64(n), capi.i32(d),
                                    capi.p(T(R)), capi.p(T(bnd)), capi.p(T(cen)), capi.p(T(S)),
                                    capi.i32(bits), capi.p(mp), capi.p(sg), capi.p(rn), capi.p(nm),
                                    capi.stream()))
    sync()
    return mp.cpu().numpy(), sg.cpu().numpy(), rn.cpu().numpy(), nm.cpu().numpy()


def k_scan(q, packed, norms, cen, R, bits, k, q_dt=capi.TQ_F32):
    qt = T(q)
    Q, d = q.shape
    N = packed.shape[0]
    os_ = torch.empty(Q, k, dtype=torch.float32, device=DEV)
    oi = torch.empty(Q, k, dtype=torch.int64, device=DEV)
    ws_bytes = L().tq_scan_workspace_bytes(Q, d, bits, N, k)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=DEV)
    pk = T(packed) if N else torch.empty(0, bits * ((d + 7) // 8), dtype=torch.uint8, device=DEV)
    nt = T(norms) if N else torch.empty(0, dtype=torch.float32, device=DEV)
    capi.check(L().tq_ip_scan_topk(capi.p(qt), q_dt, capi.i64(Q), capi.i32(d), capi.p(pk), capi.p(nt),
                                   capi.i64(N), capi.p(T(cen)), capi.p(T(R)), capi.i32(bits),
                                   capi.i32(k), capi.p(os_), capi.p(oi), capi.p(ws),
                                   ctypes.c_size_t(ws.numel()), capi.stream()))
    sync()
    return os_.cpu().numpy(), oi.cpu().numpy()


def k_scores(q, packed, norms, cen, R, bits):
    Q, d = q.shape
    N = packed.shape[0]
    out = torch.empty(Q, N, dtype=torch.float32, device=DEV)
    ws = torch.empty(max(L().tq_scan_workspace_bytes(Q, d, bits, N, 0), 1), dtype=torch.uint8, device=DEV)
    capi.check(L().tq_attention_scores_packed(capi.p(T(q)), capi.TQ_F32, capi.i64(Q), capi.i32(d),
                                              capi.p(T(packed)), capi.p(T(norms)), capi.i64(N),
                                              capi.p(T(cen)), capi.p(T(R)), capi.i32(bits),
                                              capi.p(out), capi.p(ws), ctypes.c_size_t(ws.numel()),
                                              capi.stream()))
    sync()
    return out.cpu().numpy()


def k_values(w, packed, norms, cen, M, bits):
    Q, N = w.shape
    d = M.shape[0]
    out = torch.empty(Q, d, dtype=torch.float32, device=DEV)
    ws = torch.empty(max(L().tq_values_workspace_bytes(Q, d, N), 1), dtype=torch.uint8, device=DEV)
    capi.check(L().tq_attention_values_packed(capi.p(T(w)), capi.i64(Q), capi.i64(N),
                                              capi.p(T(packed)), capi.p(T(norms)), capi.p(T(cen)),
                                              capi.p(T(M)), capi.i32(d), capi.i32(bits), capi.p(out),
                                              capi.p(ws), ctypes.c_size_t(ws.numel()), capi.stream()))
    sync()
    return out.cpu().numpy()


def k_decode(q_t, kp, kn, vp, vn, seq_lens, kc, vc, Rk, Rv, kb, vb, scale):
    B, Hq, d = q_t.shape
    Hkv, Tm = kp.shape[1], kp.shape[2]
    out = torch.empty_like(q_t)
    lse = torch.empty(B, Hq, dtype=torch.float32, device=DEV)
    ws = torch.empty(max(L().tq_decode_workspace_bytes(B, Hq, d, Tm), 1), dtype=torch.uint8, device=DEV)
    dt = {torch.float32: capi.TQ_F32, torch.bfloat16: capi.TQ_BF16, torch.float16: capi.TQ_F16}[q_t.dtype]
    sl = T(np.asarray(seq_lens, np.int32))
    capi.check(L().tq_decode_attention_packed(
        capi.p(q_t), dt, capi.i32(B), capi.i32(Hq), capi.i32(Hkv), capi.i32(d), capi.p(T(kp)),
        capi.p(T(kn)), capi.p(T(vp)), capi.p(T(vn)), capi.i64(Tm), capi.p(sl), capi.p(T(kc)),
        capi.p(T(vc)), capi.p(T(Rk)), capi.p(T(Rv)), capi.i32(kb), capi.i32(vb), ctypes.c_float(scale),
        capi.p(out), capi.p(lse), capi.p(ws), ctypes.c_size_t(ws.numel()), capi.stream()))
    sync()
    return out.float().cpu().numpy(), lse.cpu().numpy()


def k_pack_pairs(packed, d):
    """Bit-plane 4-bit rows [N, d/2] -> pair-layout rows (tq_pack_decode_layout, one stream)."""
    N = packed.shape[0]
    out = torch.zeros(max(N, 1), d // 2, dtype=torch.uint8, device=DEV)
    if N:
        capi.check(L().tq_pack_decode_layout(capi.p(T(packed)), capi.i64(1), capi.i64(N), capi.i32(d),
                                             capi.i32(4), capi.i32(0), capi.p(out), capi.i64(N),
                                             capi.i64(0), capi.stream()))
        sync()
    return out[:N]


def k_scan_pairs(q, pairs, norms, cen, R, k, q_dt=capi.TQ_F32, exact=False):
    """tq_ip_scan_topk_pairs; with two or more queries the full workspace runs the
    multi-query filtered scan, exact=True the exact multi-query scan (smaller workspace)."""
    Q, d = q.shape
    N = pairs.shape[0]
    os_ = torch.empty(Q, k, dtype=torch.float32, device=DEV)
    oi = torch.empty(Q, k, dtype=torch.int64, device=DEV)
    wsb = (L().tq_scan_workspace_bytes(Q, d, 4, N, k) if exact
           else L().tq_scan_pairs_workspace_bytes(Q, d, N, k))
    ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device=DEV)
    nt = norms if torch.is_tensor(norms) else (T(norms) if N else torch.empty(0, dtype=torch.float32, device=DEV))
    capi.check(L().tq_ip_scan_topk_pairs(capi.p(T(q)), q_dt, capi.i64(Q), capi.i32(d), capi.p(pairs),
                                         capi.p(nt), capi.i64(N), capi.p(T(cen)), capi.p(T(R)),
                                         capi.i32(k), capi.p(os_), capi.p(oi), capi.p(ws),
                                         ctypes.c_size_t(ws.numel()), capi.stream()))
    sync()
    return os_.cpu().numpy(), oi.cpu().numpy()


def k_scores_pairs(q, pairs, norms, cen, R):
    Q, d = q.shape
    N = pairs.shape[0]
    out = torch.empty(Q, N, dtype=torch.float32, device=DEV)
    ws = torch.empty(max(L().tq_scan_workspace_bytes(Q, d, 4, N, 0), 1), dtype=torch.uint8, device=DEV)
    capi.check(L().tq_attention_scores_pairs(capi.p(T(q)), capi.TQ_F32, capi.i64(Q), capi.i32(d),
                                             capi.p(pairs), capi.p(T(norms)), capi.i64(N),
                                             capi.p(T(cen)), capi.p(T(R)), capi.p(out), capi.p(ws),
                                             ctypes.c_size_t(ws.numel()), capi.stream()))
    sync()
    return out.cpu().numpy()


def k_pack_dl(packed, t_cap, pos, values, cache=None, vbits=2, d=64):
    """Bit-plane rows [S, n, P] -> decode-layout cache (created zeroed when None)."""
    S, n, _ = packed.shape
    bits = vbits if values else 4
    if cache is None:
        shape = (S, t_cap // 64, 8 * vbits * d) if values else (S, t_cap, d // 2)
        cache = torch.zeros(shape, dtype=torch.uint8, device=DEV)
    capi.check(L().tq_pack_decode_layout(capi.p(T(packed)), capi.i64(S), capi.i64(n), capi.i32(d),
                                         capi.i32(bits), capi.i32(values), capi.p(cache),
                                         capi.i64(t_cap), capi.i64(pos), capi.stream()))
    sync()
    return cache


def k_unpack_dl(cache, t_cap, t0, n, values, vbits=2, d=64):
    S = cache.shape[0]
    bits = vbits if values else 4
    out = torch.empty(S, n, bits * (d // 8), dtype=torch.uint8, device=DEV)
    capi.check(L().tq_unpack_decode_layout(capi.p(cache), capi.i64(S), capi.i64(t_cap), capi.i64(t0),
                                           capi.i64(n), capi.i32(d), capi.i32(bits), capi.i32(values),
                                           capi.p(out), capi.stream()))
    sync()
    return out.cpu().numpy()


_DT = {torch.float32: capi.TQ_F32, torch.bfloat16: capi.TQ_BF16, torch.float16: capi.TQ_F16}


def k_decode_dl(q_t, kcache, kn, vcache, vn, seq_lens, kc, vc, Rk, Rv, scale, vbits=2,
                seq_starts=None, norm_dtype=None):
    """tq_decode_attention_dl; with seq_starts or norm_dtype (the norms cast to that torch
    dtype) tq_decode_attention_dl_window."""
    B, Hq, d = q_t.shape
    Hkv, Tc = kn.shape[1], kn.shape[2]
    out = torch.empty_like(q_t)
    lse = torch.empty(B, Hq, dtype=torch.float32, device=DEV)
    ws = torch.empty(L().tq_decode_dl_workspace_bytes(B, Hq, Hkv, Tc), dtype=torch.uint8, device=DEV)
    dt = _DT[q_t.dtype]
    sl = T(np.asarray(seq_lens, np.int32))
    rest = (capi.p(T(kc)), capi.p(T(vc)), capi.p(T(Rk)), capi.p(T(Rv)), capi.i32(4), capi.i32(vbits),
            ctypes.c_float(scale), capi.p(out), capi.p(lse), capi.p(ws), ctypes.c_size_t(ws.numel()),
            capi.stream())
    head = (capi.p(q_t), dt, capi.i32(B), capi.i32(Hq), capi.i32(Hkv), capi.i32(d), capi.p(kcache))
    if seq_starts is None and norm_dtype is None:
        capi.check(L().tq_decode_attention_dl(*head, capi.p(T(kn)), capi.p(vcache), capi.p(T(vn)),
                                              capi.i64(Tc), capi.p(sl), *rest))
    else:
        nd = norm_dtype or torch.float32
        knt, vnt = T(kn, nd), T(vn, nd)
        st = capi.p(None) if seq_starts is None else capi.p(T(np.asarray(seq_starts, np.int32)))
        capi.check(L().tq_decode_attention_dl_window(*head, capi.p(knt), capi.p(vcache), capi.p(vnt),
                                                     _DT[nd], capi.i64(Tc), capi.p(sl), st, *rest))
    sync()
    return out.float().cpu().numpy(), lse.cpu().numpy()


CASES = {"d128": (128, (2, 3, 4)), "d200": (200, (3, 4)), "d64": (64, (2, 3, 4))}


# ------------------------------------------------------------------ quantize
def test_quantize_mse_fp32_vs_reference(golden):
    m, rot = golden("quant_mse"), golden("rotation")
    for name, (d, bl) in CASES.items():
        x, R = m[f"{name}_x"], rot[f"R_d{d}_s42"]
        for b in bl:
            bnd, _ = O.lloyd_max_codebook(b, d)
            packed, norms = k_quantize(T(x), R, bnd, b)
            codes = O.unpack_codes(packed, b, d)
            ref = O.unpack_codes(m[f"{name}_b{b}_packed"], b, d)
            print(f"quantize parity {name} b={b}:", O.check_codes(codes, ref, x, R, bnd))
            assert np.array_equal(O.pack_codes(codes, b), packed)  # pad bits zero
            assert np.allclose(norms, m[f"{name}_b{b}_norms"], rtol=5e-7, atol=0)


def test_quantize_mse_bf16_vs_reference(golden):
    m, rot = golden("quant_mse"), golden("rotation")
    xb = torch.from_numpy(m["bf16_d64_x_u16"].view(np.int16)).to(DEV).view(torch.bfloat16)
    x = O.bf16_bits_to_f32(m["bf16_d64_x_u16"])
    R = rot["R_d64_s42"]
    for b in (2, 3, 4):
        bnd, _ = O.lloyd_max_codebook(b, 64)
        packed, norms = k_quantize(xb, R, bnd, b, capi.TQ_BF16, capi.TQ_BF16)
        codes = O.unpack_codes(packed, b, 64)
        ref = O.unpack_codes(m[f"bf16_d64_b{b}_packed"], b, 64)
        print(f"quantize parity bf16 b={b}:", O.check_codes(codes, ref, x, R, bnd, "bf16"))
        assert np.array_equal(norms, O.bf16_bits_to_f32(m[f"bf16_d64_b{b}_norms_u16"]))


def test_quantize_zero_tiny_and_empty_rows():
    d, b = 128, 4
    R = O.dense_qr_rotation(d, 42)
    bnd, _ = O.lloyd_max_codebook(b, d)
    x = np.zeros((3, d), np.float32)
    x[1] = 1e-12
    packed, norms = k_quantize(T(x), R, bnd, b)
    _, n_o, c_o = O.quantize_mse(x, b, R, bnd)
    assert np.array_equal(O.unpack_codes(packed, b, d), c_o)
    assert norms[0] == 0.0
    k_quantize(T(np.zeros((0, d), np.float32)), R, bnd, b)  # no launch, no error


@pytest.mark.parametrize("d", [64, 128])
def test_quantize_unaligned_outputs_equal_aligned(d):
    # Outputs aligned to whole bit planes take one 16-byte (d 64: 8-byte) store per plane
    # through LDS; outputs at other offsets take 2-byte stores.  Both give the same bytes
    # (MSE codes, prod codes and sign bits), on a ragged row count (a partial last tile).
    rs = np.random.RandomState(90 + d)
    n = 1000 + 37
    x = rs.randn(n, d).astype(np.float32)
    R = O.dense_qr_rotation(d, 42)
    S = O.qjl_matrix(d, d, 43)
    bpp = d // 8
    for bits in (2, 3, 4):
        bnd, _ = O.lloyd_max_codebook(bits, d)
        want, wn = k_quantize(T(x), R, bnd, bits)
        buf = torch.zeros(n * bits * bpp + 16, dtype=torch.uint8, device=DEV)
        out = buf[2:2 + n * bits * bpp]
        norms = torch.empty(n, dtype=torch.float32, device=DEV)
        capi.check(L().tq_rotate_and_quantize(capi.p(T(x)), capi.TQ_F32, capi.TQ_F32, capi.i64(n),
                                              capi.i32(d), capi.p(T(R)), capi.p(T(bnd)), capi.i32(bits),
                                              capi.p(out), capi.p(norms), capi.stream()))
        sync()
        assert np.array_equal(out.cpu().numpy().reshape(n, -1), want), bits
        assert np.array_equal(norms.cpu().numpy(), wn), bits
    for bits in (3, 4):
        bnd, cen = O.lloyd_max_codebook(bits - 1, d)
        mp, sg, rn, nm = k_prod(x, R, bnd, cen, S, bits)
        b1 = torch.zeros(n * (bits - 1) * bpp + 16, dtype=torch.uint8, device=DEV)
        b2 = torch.zeros(n * bpp + 16, dtype=torch.uint8, device=DEV)
        mpo, sgo = b1[2:2 + n * (bits - 1) * bpp], b2[6:6 + n * bpp]
        rno = torch.empty(n, dtype=torch.float32, device=DEV)
        nmo = torch.empty(n, dtype=torch.float32, device=DEV)
        capi.check(L().tq_quantize_prod(capi.p(T(x)), capi.TQ_F32, capi.TQ_F32, capi.i64(n), capi.i32(d),
                                        capi.p(T(R)), capi.p(T(bnd)), capi.p(T(cen)), capi.p(T(S)),
                                        capi.i32(bits), capi.p(mpo), capi.p(sgo), capi.p(rno), capi.p(nmo),
                                        capi.stream()))
        sync()
        assert np.array_equal(mpo.cpu().numpy().reshape(n, -1), mp), bits
        assert np.array_equal(sgo.cpu().numpy().reshape(n, -1), sg), bits
        assert np.array_equal(rno.cpu().numpy(), rn) and np.array_equal(nmo.cpu().numpy(), nm), bits


def test_quantize_prod_vs_reference(golden):
    pr, rot, qj = golden("quant_prod"), golden("rotation"), golden("qjl")
    for name, d in (("d128", 128), ("d200", 200)):
        x, R, S = pr[f"{name}_x"], rot[f"R_d{d}_s42"], qj[f"S_d{d}_s42"]
        bnd, cen = O.lloyd_max_codebook(3, d)
        mp, sg, rn, nm = k_prod(x, R, bnd, cen, S, 4)
        _, _, _, _, _, proj64 = O.quantize_prod(x, 4, R, bnd, cen, S)
        u = x / np.maximum(np.linalg.norm(x.astype(np.float64), axis=1), 1e-10)[:, None]
        codes = O.unpack_codes(mp, 3, d)
        ref = O.unpack_codes(pr[f"{name}_mse_packed"], 3, d)
        print(f"quantize_prod parity {name}:", O.check_codes(codes, ref, u.astype(np.float32), R, bnd))
        same_rows = ~(codes != ref).any(axis=1)
        sign_band = np.abs(proj64) <= 2.0 ** -16 * np.max(np.abs(proj64), axis=1, keepdims=True)
        s_k = O.unpack_codes(sg, 1, d)
        s_r = O.unpack_codes(pr[f"{name}_signs"], 1, d)
        bad = (s_k != s_r) & ~sign_band & same_rows[:, None]
        print(f"{name}: sign mismatches {np.sum(s_k != s_r)}; outside band {bad.sum()}")
        assert not bad.any()
        assert np.allclose(nm, pr[f"{name}_norms"], rtol=5e-7)
        ok = same_rows
        assert np.allclose(rn[ok], pr[f"{name}_res_norms"][ok], rtol=2e-5, atol=1e-7)


@pytest.mark.parametrize("d", [64, 128, 132, 160, 200, 256])
def test_quantize_mfma_ragged_vs_oracle(d):
    # fp32 inputs run the MFMA kernel (64-row tiles; d 64/128 with register-resident
    # operands, d of 132-256 padded to 192/208/256 with operands reloaded per contraction):
    # ragged row counts, every bit width of both modes, against the oracle's float64
    # decision margins.
    rs = np.random.RandomState(900 + d)
    R = O.dense_qr_rotation(d, 42)
    S = O.qjl_matrix(d, d, 42)
    for n in (1, 63, 65, 1000, 4099):
        x = (rs.randn(n, d) * np.exp(rs.randn(1, d))).astype(np.float32)
        x[n // 2] = 0.0  # a zero row
        for b in (1, 2, 3, 4):
            bnd, _ = O.lloyd_max_codebook(b, d)
            packed, norms = k_quantize(T(x), R, bnd, b)
            _, n_o, c_o = O.quantize_mse(x, b, R, bnd)
            codes = O.unpack_codes(packed, b, d)
            O.check_codes(codes, c_o, x, R, bnd)
            assert np.array_equal(O.pack_codes(codes, b), packed)
            assert np.allclose(norms, n_o, rtol=5e-7, atol=0), (d, n, b)
        for b in (2, 3, 4):
            bnd, cen = O.lloyd_max_codebook(b - 1, d)
            mp, sg, rn, nm = k_prod(x, R, bnd, cen, S, b)
            mp_o, sg_o, rn_o, nm_o, c_o, proj64 = O.quantize_prod(x, b, R, bnd, cen, S)
            u = x / np.maximum(np.linalg.norm(x.astype(np.float64), axis=1), 1e-10)[:, None]
            codes = O.unpack_codes(mp, b - 1, d)
            O.check_codes(codes, c_o, u.astype(np.float32), R, bnd)
            same = ~(codes != c_o).any(axis=1)
            sign_band = np.abs(proj64) <= 2.0 ** -16 * np.max(np.abs(proj64), axis=1, keepdims=True)
            s_k, s_o = O.unpack_codes(sg, 1, d), O.unpack_codes(sg_o, 1, d)
            assert not ((s_k != s_o) & ~sign_band & same[:, None]).any(), (d, n, b)
            assert np.allclose(nm, nm_o, rtol=5e-7), (d, n, b)
            assert np.allclose(rn[same], rn_o[same], rtol=2e-5, atol=1e-7), (d, n, b)


# ------------------------------------------------------------------ pack / unpack
@pytest.mark.parametrize("bits", [1, 2, 3, 4, 8])
@pytest.mark.parametrize("d", [1, 7, 64, 100, 128, 200, 256])
def test_pack_unpack_vs_oracle(bits, d):
    rs = np.random.RandomState(bits * 31 + d)
    codes = rs.randint(0, 1 << bits, (333, d)).astype(np.uint8)
    P = bits * ((d + 7) // 8)
    packed = torch.empty(333, P, dtype=torch.uint8, device=DEV)
    capi.check(L().tq_pack_codes(capi.p(T(codes)), capi.i64(333), capi.i32(d), capi.i32(bits),
                                 capi.p(packed), capi.stream()))
    back = torch.empty(333, d, dtype=torch.uint8, device=DEV)
    capi.check(L().tq_unpack_codes(capi.p(packed), capi.i64(333), capi.i32(d), capi.i32(bits),
                                   capi.p(back), capi.stream()))
    sync()
    assert np.array_equal(packed.cpu().numpy(), O.pack_codes(codes, bits))
    assert np.array_equal(back.cpu().numpy(), codes)


# ------------------------------------------------------------------ dequantize
def test_dequantize_mse_vs_reference(golden):
    m, rot = golden("quant_mse"), golden("rotation")
    for name, (d, bl) in CASES.items():
        R = rot[f"R_d{d}_s42"]
        for b in bl:
            _, cen = O.lloyd_max_codebook(b, d)
            pk, nm = m[f"{name}_b{b}_packed"][:64], m[f"{name}_b{b}_norms"][:64]
            out = torch.empty(64, d, dtype=torch.float32, device=DEV)
            capi.check(L().tq_dequantize_mse(capi.p(T(pk)), capi.p(T(nm)), capi.i64(64), capi.i32(d),
                                             capi.i32(b), capi.p(T(cen)), capi.p(T(R)), capi.TQ_F32,
                                             capi.p(out), capi.stream()))
            sync()
            assert np.allclose(out.cpu().numpy(), m[f"{name}_b{b}_deq64"], rtol=1e-5, atol=2e-6)


def test_dequantize_prod_vs_reference(golden):
    pr, rot, qj = golden("quant_prod"), golden("rotation"), golden("qjl")
    for name, d in (("d128", 128), ("d200", 200)):
        R, S = rot[f"R_d{d}_s42"], qj[f"S_d{d}_s42"]
        _, cen = O.lloyd_max_codebook(3, d)
        args = [pr[f"{name}_{k}"][:64] for k in ("mse_packed", "signs", "res_norms", "norms")]
        out = torch.empty(64, d, dtype=torch.float32, device=DEV)
        capi.check(L().tq_dequantize_prod(*[capi.p(T(a)) for a in args], capi.i64(64), capi.i32(d),
                                          capi.i32(4), capi.p(T(cen)), capi.p(T(R)), capi.p(T(S)),
                                          capi.TQ_F32, capi.p(out), capi.stream()))
        sync()
        ref = pr[f"{name}_deq64"]
        assert np.max(np.abs(out.cpu().numpy() - ref)) <= 2e-5 * np.max(np.abs(ref))


# ------------------------------------------------------------------ scores / values
def _db(rs, n, d, b, seed=42):
    R = O.dense_qr_rotation(d, seed)
    bnd, cen = O.lloyd_max_codebook(b, d)
    x = rs.randn(n, d).astype(np.float32)
    p, nm, _ = O.quantize_mse(x, b, R, bnd)
    return R, cen, p, nm


@pytest.mark.parametrize("d", [64, 128, 200])
@pytest.mark.parametrize("b", [1, 2, 3, 4])
def test_attention_scores_bit_exact(d, b):
    rs = np.random.RandomState(d + b)
    R, cen, p, nm = _db(rs, 1500, d, b)
    for Q in (1, 3, 6):
        q = rs.randn(Q, d).astype(np.float32)
        got = k_scores(q, p, nm, cen, R, b)
        want = O.lut_scores_f32(q, p, nm, cen, R, b)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (d, b, Q)


@pytest.mark.parametrize("d,b", [(64, 2), (128, 4), (200, 3)])
def test_attention_values_vs_f64(d, b):
    rs = np.random.RandomState(7 * d + b)
    R, cen, p, nm = _db(rs, 2500, d, b, seed=43)
    w = rs.rand(5, 2500).astype(np.float32)
    w /= w.sum(1, keepdims=True)
    got = k_values(w, p, nm, cen, R, b)
    want = O.values_f64(w, p, nm, cen, R, b)
    assert np.max(np.abs(got - want)) <= 1e-5 * np.max(np.abs(want))


# ------------------------------------------------------------------ top-k scan
def test_scan_vs_reference_index(golden):
    ix, m, rot = golden("index"), golden("quant_mse"), golden("rotation")
    R, q = rot["R_d128_s42"], ix["queries"]
    for b in (2, 3, 4):
        _, cen = O.lloyd_max_codebook(b, 128)
        s, i = k_scan(q, ix[f"b{b}_packed"], m[f"d128_b{b}_norms"], cen, R, b, 10)
        assert np.array_equal(i, ix[f"b{b}_ids"]), b
        assert np.allclose(s, ix[f"b{b}_scores"], rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("d", [64, 128, 200])
@pytest.mark.parametrize("b", [2, 3, 4])
def test_scan_topk_bit_exact(d, b):
    rs = np.random.RandomState(3 * d + b)
    R, cen, p, nm = _db(rs, 20000, d, b)
    for Q, k in ((1, 10), (4, 1), (7, 32)):
        q = rs.randn(Q, d).astype(np.float32)
        s, i = k_scan(q, p, nm, cen, R, b, k)
        so, io = O.search_topk(q, p, nm, cen, R, b, k)
        assert np.array_equal(i, io), (d, b, Q, k)
        assert np.array_equal(s.view(np.uint32), so.view(np.uint32))


def pair_rows_np(codes, bits):
    """Independent numpy packing of codes [N, d] into pair rows (include/turboquant_hip.h):
    2 bits: byte b = c[4b] << 6 | c[4b+1] << 4 | c[4b+2] << 2 | c[4b+3]; 3 bits: per 32 dims
    12 bytes, byte 4i + k = pair (4i + k)'s index c[2p] << 3 | c[2p+1] in bits 0-5 and bits
    2i, 2i+1 of pair (12 + k)'s index in bits 6-7; 4 bits: byte p = c[2p] << 4 | c[2p+1]."""
    c = codes.astype(np.uint32)
    N, d = c.shape
    if bits == 4:
        return ((c[:, 0::2] << 4) | c[:, 1::2]).astype(np.uint8)
    if bits == 2:
        return ((c[:, 0::4] << 6) | (c[:, 1::4] << 4) | (c[:, 2::4] << 2) | c[:, 3::4]).astype(np.uint8)
    idx = (c[:, 0::2] << 3) | c[:, 1::2]                     # [N, d/2] pair indices
    out = np.zeros((N, d * 3 // 8), np.uint32)
    for t in range(d // 32):
        for i in range(3):
            for k in range(4):
                lo = idx[:, 16 * t + 4 * i + k]
                hi = idx[:, 16 * t + 12 + k]
                out[:, 12 * t + 4 * i + k] = lo | (((hi >> (2 * i)) & 3) << 6)
    return out.astype(np.uint8)


def k_pair_rows(packed, d, bits):
    N = packed.shape[0]
    out = torch.zeros(max(N, 1), d * bits // 8, dtype=torch.uint8, device=DEV)
    capi.check(L().tq_pack_pair_rows(capi.p(T(packed)), capi.i64(N), capi.i32(d), capi.i32(bits),
                                     capi.p(out), capi.stream()))
    sync()
    return out[:N]


@pytest.mark.parametrize("bits", [2, 3, 4])
@pytest.mark.parametrize("d", [64, 128])
def test_pair_rows_pack_roundtrip(bits, d):
    rs = np.random.RandomState(60 + 7 * bits + d)
    codes = rs.randint(0, 1 << bits, (333, d))
    packed = O.pack_codes(codes, bits)
    rows = k_pair_rows(packed, d, bits)
    assert np.array_equal(rows.cpu().numpy(), pair_rows_np(codes, bits))
    back = torch.empty(333, bits * d // 8, dtype=torch.uint8, device=DEV)
    capi.check(L().tq_unpack_pair_rows(capi.p(rows), capi.i64(333), capi.i32(d), capi.i32(bits),
                                       capi.p(back), capi.stream()))
    sync()
    assert np.array_equal(back.cpu().numpy(), packed)
    if bits == 3:  # a planted mistake in the numpy packing (pairs 12-15 dropped) fails
        bad = codes.copy()
        bad[:, 24:32] = 0
        assert not np.array_equal(rows.cpu().numpy(), pair_rows_np(bad, bits))


def k_scan_pair_rows(q, rows, norms, cen, R, bits, k, q_dt=capi.TQ_F32, exact=False):
    """tq_ip_scan_topk_pair_rows; with two or more queries the full workspace runs the
    multi-query filtered scan, exact=True the exact scans (smaller workspace)."""
    Q, d = q.shape
    N = rows.shape[0]
    os_ = torch.empty(Q, k, dtype=torch.float32, device=DEV)
    oi = torch.empty(Q, k, dtype=torch.int64, device=DEV)
    wsb = (L().tq_scan_workspace_bytes(Q, d, bits, N, k) if exact
           else L().tq_scan_pair_rows_workspace_bytes(Q, d, bits, N, k))
    ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device=DEV)
    nt = norms if torch.is_tensor(norms) else T(norms)
    capi.check(L().tq_ip_scan_topk_pair_rows(capi.p(T(q)), q_dt, capi.i64(Q), capi.i32(d), capi.p(rows),
                                             capi.p(nt), capi.i64(N), capi.p(T(cen)), capi.p(T(R)),
                                             capi.i32(bits), capi.i32(k), capi.p(os_), capi.p(oi),
                                             capi.p(ws), ctypes.c_size_t(ws.numel()), capi.stream()))
    sync()
    return os_.cpu().numpy(), oi.cpu().numpy()


@pytest.mark.parametrize("bits", [2, 3])
@pytest.mark.parametrize("d", [64, 128])
def test_pair_rows_scan_bit_exact(bits, d):
    # ragged N; one, several and many queries (one query per block row at 2-3 bits)
    rs = np.random.RandomState(80 + 7 * bits + d)
    N = 20000 + 37
    R, cen, p, nm = _db(rs, N, d, bits)
    rows = k_pair_rows(p, d, bits)
    for Q, k in ((1, 10), (4, 1), (9, 32)):
        q = rs.randn(Q, d).astype(np.float32)
        so, io = O.search_topk(q, p, nm, cen, R, bits, k)
        for exact in (False, True):  # the multi-query filter (Q > 1) and the exact scan
            s, i = k_scan_pair_rows(q, rows, nm, cen, R, bits, k, exact=exact)
            assert np.array_equal(i, io), (Q, k, exact)
            assert np.array_equal(s.view(np.uint32), so.view(np.uint32)), (Q, k, exact)
    q = rs.randn(3, d).astype(np.float32)
    out = torch.empty(3, 1500, dtype=torch.float32, device=DEV)
    ws = torch.empty(max(L().tq_scan_workspace_bytes(3, d, bits, 1500, 0), 1), dtype=torch.uint8, device=DEV)
    capi.check(L().tq_attention_scores_pair_rows(capi.p(T(q)), capi.TQ_F32, capi.i64(3), capi.i32(d),
                                                 capi.p(rows), capi.p(T(nm[:1500])), capi.i64(1500),
                                                 capi.p(T(cen)), capi.p(T(R)), capi.i32(bits), capi.p(out),
                                                 capi.p(ws), ctypes.c_size_t(ws.numel()), capi.stream()))
    sync()
    want = O.lut_scores_f32(q, p[:1500], nm[:1500], cen, R, bits)
    assert np.array_equal(out.cpu().numpy().view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("b,layout", [(4, "pairs"), (4, "bitplane"), (3, "bitplane"), (2, "bitplane"),
                                      (3, "pairs"), (2, "pairs")])
def test_scan_q64_batch_vs_oracle(b, layout):
    # A config-2 query batch (64 normalized fp16 queries, k = 10) over N = 100,003 unit
    # rows: the multi-query scan (four queries per block) must return the oracle's ids
    # and float32 scores bit for bit.
    rs = np.random.RandomState(70 + b)
    d, N = 128, 100_003
    R = O.dense_qr_rotation(d, 42)
    bnd, cen = O.lloyd_max_codebook(b, d)
    x = rs.randn(N, d).astype(np.float32)
    x /= np.linalg.norm(x, axis=1, keepdims=True)
    p, nm, _ = O.quantize_mse(x, b, R, bnd)
    qf = rs.randn(64, d).astype(np.float32)
    qf /= np.linalg.norm(qf, axis=1, keepdims=True)
    q16 = qf.astype(np.float16)
    if layout == "pairs" and b == 4:
        s, i = k_scan_pairs(q16, k_pack_pairs(p, d), nm, cen, R, 10, q_dt=capi.TQ_F16)
    elif layout == "pairs":
        s, i = k_scan_pair_rows(q16, k_pair_rows(p, d, b), nm, cen, R, b, 10, q_dt=capi.TQ_F16)
    else:
        s, i = k_scan(q16, p, nm, cen, R, b, 10, q_dt=capi.TQ_F16)
    so, io = O.search_topk(q16.astype(np.float32), p, nm, cen, R, b, 10)
    assert np.array_equal(i, io)
    assert np.array_equal(s.view(np.uint32), so.view(np.uint32))


def test_scan_ties_padding_and_fp16_queries():
    rs = np.random.RandomState(11)
    d, b = 128, 4
    R, cen, p, nm = _db(rs, 40, d, b)
    p = np.concatenate([p, p[:7], p[:7]])  # duplicated rows tie exactly
    nm = np.concatenate([nm, nm[:7], nm[:7]])
    q = rs.randn(3, d).astype(np.float32)
    s, i = k_scan(q, p, nm, cen, R, b, 30)
    so, io = O.search_topk(q, p, nm, cen, R, b, 30)
    assert np.array_equal(i, io)
    s, i = k_scan(q, p[:5], nm[:5], cen, R, b, 8)  # k > N pads (-inf, -1)
    assert (i[:, 5:] == -1).all() and np.isneginf(s[:, 5:]).all()
    q16 = q.astype(np.float16)
    s, i = k_scan(q16, p, nm, cen, R, b, 10, capi.TQ_F16)
    so, io = O.search_topk(q16.astype(np.float32), p, nm, cen, R, b, 10)
    assert np.array_equal(i, io)


@pytest.mark.parametrize("d", [64, 128])
def test_pairs_layout_scan_bit_exact(d):
    rs = np.random.RandomState(5 * d)
    N = 20000 + 37  # ragged: not a multiple of the 64-row step
    R, cen, p, nm = _db(rs, N, d, 4)
    pairs = k_pack_pairs(p, d)
    codes = O.unpack_codes(p, 4, d).astype(np.uint8)
    assert np.array_equal(pairs.cpu().numpy(), (codes[:, 0::2] << 4) | codes[:, 1::2])
    for Q, k in ((1, 10), (4, 1), (7, 32)):
        q = rs.randn(Q, d).astype(np.float32)
        s, i = k_scan_pairs(q, pairs, nm, cen, R, k)
        so, io = O.search_topk(q, p, nm, cen, R, 4, k)
        assert np.array_equal(i, io), (d, Q, k)
        assert np.array_equal(s.view(np.uint32), so.view(np.uint32))
    q = rs.randn(3, d).astype(np.float32)
    got = k_scores_pairs(q, pairs[:1500], nm[:1500], cen, R)
    want = O.lut_scores_f32(q, p[:1500], nm[:1500], cen, R, 4)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    q16 = q.astype(np.float16)
    s, i = k_scan_pairs(q16, pairs, nm, cen, R, 10, capi.TQ_F16)
    so, io = O.search_topk(q16.astype(np.float32), p, nm, cen, R, 4, 10)
    assert np.array_equal(i, io)


@pytest.mark.parametrize("N", [600_000, 2_200_000])
def test_scan_many_blocks_merge(N):
    # Enough rows for hundreds of block lists (up to the full 1024-block grid), so the
    # merge's group maxima span several blocks per thread.
    rs = np.random.RandomState(N % 1000)
    d = 64
    R, cen, p, nm = _db(rs, N, d, 4)
    q = rs.randn(3, d).astype(np.float32)
    pairs = k_pack_pairs(p, d)
    s32, i32 = O.search_topk(q, p, nm, cen, R, 4, 32)  # top-k for smaller k is its prefix
    for k in (1, 10, 32):
        so, io = s32[:, :k], i32[:, :k]
        s, i = k_scan(q, p, nm, cen, R, 4, k)
        assert np.array_equal(i, io), k
        assert np.array_equal(s.view(np.uint32), so.view(np.uint32))
        s, i = k_scan_pairs(q, pairs, nm, cen, R, k)
        assert np.array_equal(i, io), k


def test_pairs_scan_ties_padding_and_golden(golden):
    rs = np.random.RandomState(13)
    d = 128
    R, cen, p, nm = _db(rs, 40, d, 4)
    p = np.concatenate([p, p[:7], p[:7]])  # duplicated rows tie exactly
    nm = np.concatenate([nm, nm[:7], nm[:7]])
    pairs = k_pack_pairs(p, d)
    q = rs.randn(3, d).astype(np.float32)
    s, i = k_scan_pairs(q, pairs, nm, cen, R, 30)
    so, io = O.search_topk(q, p, nm, cen, R, 4, 30)
    assert np.array_equal(i, io)
    s, i = k_scan_pairs(q, pairs[:5], nm[:5], cen, R, 8)  # k > N pads (-inf, -1)
    assert (i[:, 5:] == -1).all() and np.isneginf(s[:, 5:]).all()
    s, i = k_scan_pairs(q, pairs[:0], nm[:0], cen, R, 4)  # empty database
    assert (i == -1).all() and np.isneginf(s).all()
    ix, m, rot = golden("index"), golden("quant_mse"), golden("rotation")
    _, cen4 = O.lloyd_max_codebook(4, 128)
    s, i = k_scan_pairs(ix["queries"], k_pack_pairs(ix["b4_packed"], 128), m["d128_b4_norms"], cen4,
                        rot["R_d128_s42"], 10)
    assert np.array_equal(i, ix["b4_ids"])
    assert np.allclose(s, ix["b4_scores"], rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("d", [64, 128])
def test_pairs_scan_one_query(d):
    # One query per call runs the pair-byte kernel (both centroids of a byte from one
    # table read, products formed in registers, a block-wide bound after each wave's
    # first 64 rows).  Scores stay bit-exact.
    rs = np.random.RandomState(70 + d)
    N = 300_000 + 29
    R, cen, p, nm = _db(rs, N, d, 4)
    pairs = k_pack_pairs(p, d)
    q = rs.randn(1, d).astype(np.float32)
    s32, i32 = O.search_topk(q, p, nm, cen, R, 4, 32)
    for k in (1, 10, 32):  # k = 32: the block list merge ranks more than 128 entries
        s, i = k_scan_pairs(q, pairs, nm, cen, R, k)
        assert np.array_equal(i, i32[:, :k]), k
        assert np.array_equal(s.view(np.uint32), s32[:, :k].view(np.uint32)), k
    # small and ragged databases: waves without rows, a partial last step, k > N
    for n in (1, 5, 63, 64, 65, 700, 769, 5000):
        s, i = k_scan_pairs(q, pairs[:n], nm[:n], cen, R, 10)
        so, io = O.search_topk(q, p[:n], nm[:n], cen, R, 4, 10)
        assert np.array_equal(i, io), n
        assert np.array_equal(s.view(np.uint32), so.view(np.uint32)), n
    q16 = q.astype(np.float16)
    s, i = k_scan_pairs(q16, pairs, nm, cen, R, 10, capi.TQ_F16)
    so, io = O.search_topk(q16.astype(np.float32), p, nm, cen, R, 4, 10)
    assert np.array_equal(i, io)
    assert np.array_equal(s.view(np.uint32), so.view(np.uint32))
    got = k_scores_pairs(q, pairs[:20000], nm[:20000], cen, R)  # every score, one query
    want = O.lut_scores_f32(q, p[:20000], nm[:20000], cen, R, 4)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_pairs_scan_one_query_ties():
    # 3000 copies of the best row tie exactly: the block bound and the wave lists must
    # keep the lowest ids among them (and the merge takes its exact fallback).
    rs = np.random.RandomState(17)
    d = 128
    R, cen, p, nm = _db(rs, 30000, d, 4)
    q = rs.randn(1, d).astype(np.float32)
    top = int(np.argmax(O.lut_scores_f32(q, p, nm, cen, R, 4)))
    idx = rs.choice(30000, 3000, replace=False)
    p[idx] = p[top]
    nm[idx] = nm[top]
    pairs = k_pack_pairs(p, d)
    for k in (4, 16, 32):
        s, i = k_scan_pairs(q, pairs, nm, cen, R, k)
        so, io = O.search_topk(q, p, nm, cen, R, 4, k)
        assert np.array_equal(i, io), k
        assert np.array_equal(s.view(np.uint32), so.view(np.uint32)), k


def _topk_no_nan(scores, k):
    # the scan never lists a NaN score; the remaining rows in the oracle's order
    sc = np.where(np.isnan(scores), -np.inf, scores)
    keep = ~np.isnan(scores)
    so, io = O.topk_desc(sc, sc.shape[1])
    out_s = np.full((sc.shape[0], k), -np.inf, np.float32)
    out_i = np.full((sc.shape[0], k), -1, np.int64)
    for r in range(sc.shape[0]):
        ids = [j for j in io[r] if keep[r, j]][:k]
        out_i[r, :len(ids)] = ids
        out_s[r, :len(ids)] = scores[r, ids]
    return out_s, out_i


def test_pairs_scan_one_query_special_norms():
    # The one-query scan scores rows approximately first; rows whose norms are zero,
    # negative, huge, tiny or infinite (inf * 0 = NaN rows are never listed) must still
    # come out exactly as the reference's arithmetic orders them.
    rs = np.random.RandomState(23)
    d = 128
    N = 150_000
    R, cen, p, nm = _db(rs, N, d, 4)
    nm = nm.copy()
    idx = rs.permutation(N)
    nm[idx[:2000]] = 0.0
    nm[idx[2000:4000]] *= -1.0
    nm[idx[4000:4010]] = 1e30
    nm[idx[4010:4020]] = -1e30
    nm[idx[4020:4030]] = 1e-38
    nm[idx[4030:4036]] = np.inf
    nm[idx[4036:4040]] = -np.inf
    pairs = k_pack_pairs(p, d)
    q = rs.randn(1, d).astype(np.float32)
    want = O.lut_scores_f32(q, p, nm, cen, R, 4)
    for k in (1, 10, 32):
        s, i = k_scan_pairs(q, pairs, nm, cen, R, k)
        so, io = _topk_no_nan(want, k)
        assert np.array_equal(i, io), k
        assert np.array_equal(s.view(np.uint32), so.view(np.uint32)), k


@pytest.mark.parametrize("qscale", [0.0, 1e-36, 1e-20, 1e20, 1e34])
def test_pairs_scan_one_query_extreme_queries(qscale):
    # Queries that are zero (every score ties at 0: the lowest ids win) or whose scale
    # leaves the fp16 filter's range (every row is rescored exactly) or nearly does.
    rs = np.random.RandomState(31)
    d = 64
    N = 40_000
    R, cen, p, nm = _db(rs, N, d, 4)
    pairs = k_pack_pairs(p, d)
    q = (rs.randn(1, d) * qscale).astype(np.float32)
    want = O.lut_scores_f32(q, p, nm, cen, R, 4)
    for k in (3, 10):
        s, i = k_scan_pairs(q, pairs, nm, cen, R, k)
        so, io = _topk_no_nan(want, k)
        assert np.array_equal(i, io), (qscale, k)
        assert np.array_equal(s.view(np.uint32), so.view(np.uint32)), (qscale, k)


def test_pairs_scan_one_query_ulp_ties():
    # 600 copies of the best row whose norms differ from it by a few ulps: their
    # approximate scores cannot tell them apart, their exact scores can.
    rs = np.random.RandomState(41)
    d = 128
    N = 80_000
    R, cen, p, nm = _db(rs, N, d, 4)
    q = rs.randn(1, d).astype(np.float32)
    top = int(np.argmax(O.lut_scores_f32(q, p, nm, cen, R, 4)))
    idx = rs.choice(N, 600, replace=False)
    p[idx] = p[top]
    steps = rs.randint(-3, 4, size=600).astype(np.int32)
    nm[idx] = (nm[top].view(np.int32) + steps).view(np.float32)
    pairs = k_pack_pairs(p, d)
    for k in (5, 32):
        s, i = k_scan_pairs(q, pairs, nm, cen, R, k)
        so, io = O.search_topk(q, p, nm, cen, R, 4, k)
        assert np.array_equal(i, io), k
        assert np.array_equal(s.view(np.uint32), so.view(np.uint32)), k


def test_pairs_scan_one_query_past_4gib():
    # 67.1M rows of d = 128 (4.3 GB of codes): rows past byte 2^32 are addressed with
    # 64-bit bases.  Random codes, norm 0 except 200 planted rows spread over the whole
    # range (most past 2^32 bytes); the answer is the planted rows with positive scores,
    # then zero-score rows by lowest id.  Only the planted rows go through the oracle.
    rs = np.random.RandomState(53)
    d = 128
    N = (1 << 26) + 1017
    R = O.dense_qr_rotation(d, 42)
    _, cen = O.lloyd_max_codebook(4, d)
    g = torch.Generator(device=DEV)
    g.manual_seed(5)
    pairs = torch.randint(0, 256, (N, d // 2), dtype=torch.uint8, device=DEV, generator=g)
    norms = torch.zeros(N, dtype=torch.float32, device=DEV)
    planted = np.sort(rs.choice(np.arange(1000, N), 200, replace=False))
    planted[-1] = N - 1
    codes = rs.randint(0, 16, size=(200, d)).astype(np.uint8)
    pn = (rs.rand(200) * 2 + 0.5).astype(np.float32)
    pt = torch.from_numpy((codes[:, 0::2] << 4) | codes[:, 1::2]).to(DEV)
    it = torch.from_numpy(planted).to(DEV)
    pairs[it] = pt
    norms[it] = torch.from_numpy(pn).to(DEV)
    q = rs.randn(1, d).astype(np.float32)
    ps = O.lut_scores_f32(q, O.pack_codes(codes, 4), pn, cen, R, 4)[0]
    pos = [(float(ps[j]), int(planted[j])) for j in range(200) if ps[j] > 0]
    pos.sort(key=lambda t: (-t[0], t[1]))
    assert len(pos) >= 32
    zero_ids = [j for j in range(64) if j not in set(planted.tolist())]
    for k in (10, 32):
        s, i = k_scan_pairs(q, pairs, norms, cen, R, k)
        want_i = [t[1] for t in pos][:k]
        want_s = np.array([t[0] for t in pos][:k], np.float32)
        assert np.array_equal(i[0], np.array(want_i)), k
        assert np.array_equal(s[0].view(np.uint32), want_s.view(np.uint32)), k
    # three positive rows left: then the zero-score rows (norm 0) by lowest id
    keep3 = {t[1] for t in pos[:3]}
    drop = [int(planted[j]) for j in range(200) if ps[j] > 0 and int(planted[j]) not in keep3]
    norms[torch.tensor(drop, device=DEV)] = 0.0
    s, i = k_scan_pairs(q, pairs, norms, cen, R, 10)
    want_i = [t[1] for t in pos[:3]] + zero_ids[:7]
    assert np.array_equal(i[0], np.array(want_i))
    assert np.array_equal(s[0, :3].view(np.uint32), np.array([t[0] for t in pos[:3]], np.float32).view(np.uint32))
    assert (s[0, 3:] == 0).all()
    del pairs, norms
    torch.cuda.empty_cache()


@pytest.mark.parametrize("bits", [2, 3])
def test_pair_rows_one_query_past_4gib(bits):
    # One query over 2-/3-bit pair rows of d = 128 past 2^32 bytes (4.3 GB of codes): rows
    # there are addressed with 64-bit bases.  Random codes, norm 0 except
    # 200 planted rows spread over the whole range; the answer is the planted rows with
    # positive scores (only they go through the oracle), then zero-score rows by lowest id.
    rs = np.random.RandomState(57 + bits)
    d = 128
    rb = d * bits // 8
    N = (1 << 32) // rb + 1017
    R = O.dense_qr_rotation(d, 42)
    _, cen = O.lloyd_max_codebook(bits, d)
    g = torch.Generator(device=DEV)
    g.manual_seed(7 + bits)
    rows = torch.randint(0, 256, (N, rb), dtype=torch.uint8, device=DEV, generator=g)
    norms = torch.zeros(N, dtype=torch.float32, device=DEV)
    planted = np.sort(rs.choice(np.arange(1000, N), 200, replace=False))
    planted[-1] = N - 1
    codes = rs.randint(0, 1 << bits, size=(200, d)).astype(np.uint8)
    packed = O.pack_codes(codes, bits)
    pn = (rs.rand(200) * 2 + 0.5).astype(np.float32)
    it = torch.from_numpy(planted).to(DEV)
    rows[it] = k_pair_rows(packed, d, bits)
    norms[it] = torch.from_numpy(pn).to(DEV)
    q = rs.randn(1, d).astype(np.float32)
    ps = O.lut_scores_f32(q, packed, pn, cen, R, bits)[0]
    pos = [(float(ps[j]), int(planted[j])) for j in range(200) if ps[j] > 0]
    pos.sort(key=lambda t: (-t[0], t[1]))
    assert len(pos) >= 32
    print(f"pair rows past 4 GiB: {bits} bits, {N} rows", flush=True)
    for k in (10, 32):
        s, i = k_scan_pair_rows(q, rows, norms, cen, R, bits, k)
        want_i = [t[1] for t in pos][:k]
        want_s = np.array([t[0] for t in pos][:k], np.float32)
        assert np.array_equal(i[0], np.array(want_i)), k
        assert np.array_equal(s[0].view(np.uint32), want_s.view(np.uint32)), k
    keep3 = {t[1] for t in pos[:3]}
    drop = [int(planted[j]) for j in range(200) if ps[j] > 0 and int(planted[j]) not in keep3]
    norms[torch.tensor(drop, device=DEV)] = 0.0
    s, i = k_scan_pair_rows(q, rows, norms, cen, R, bits, 10)
    zero_ids = [j for j in range(64) if j not in set(planted.tolist())]
    assert np.array_equal(i[0], np.array([t[1] for t in pos[:3]] + zero_ids[:7]))
    assert (s[0, 3:] == 0).all()
    del rows, norms
    torch.cuda.empty_cache()


# ------------------------------------------------------------------ multi-query filtered scan
def _cpu_search(q, p, nm, cen, R, k):
    """The C restatement of the reference core's search (oracle/tq_cpu.c, OpenMP) over
    bit-plane rows, for batches the numpy oracle is too slow for.  tests/test_oracle.py
    holds it bit-exact with the reference's compiled core and with the numpy oracle,
    including the oracle's order of exactly tied scores (lower index first; the core's own
    heap leaves the order of tied scores unspecified)."""
    import cpu_libs
    return cpu_libs.search_packed(q, p, nm, R, cen, 4, k, "port")


@pytest.mark.parametrize("d", [64, 128])
def test_mq_scan_vs_oracle_and_exact_path(d):
    # Batches of 2, 64 and 130 queries (one, one and three 64-query tiles, the last two
    # partly filled) over ~100k unit rows: ids and scores bit-identical to the oracle and
    # to the exact multi-query scan, for k = 1, 10, 32, fp32 and fp16 queries.
    rs = np.random.RandomState(90 + d)
    N = 100_003 if d == 128 else 60_001
    R, cen, p, nm = _db(rs, N, d, 4)
    nm = nm / np.float32(np.sqrt(d))  # unit-scale rows
    pairs = k_pack_pairs(p, d)
    for Q in (2, 64, 130):
        q = rs.randn(Q, d).astype(np.float32)
        q /= np.linalg.norm(q, axis=1, keepdims=True)
        s32, i32 = _cpu_search(q, p, nm, cen, R, 32)
        if Q == 2:
            so, io = O.search_topk(q, p, nm, cen, R, 4, 32)
            assert np.array_equal(io, i32) and np.array_equal(so.view(np.uint32), s32.view(np.uint32))
        for k in (1, 10, 32):
            s, i = k_scan_pairs(q, pairs, nm, cen, R, k)
            assert np.array_equal(i, i32[:, :k]), (Q, k)
            assert np.array_equal(s.view(np.uint32), s32[:, :k].view(np.uint32)), (Q, k)
            se, ie = k_scan_pairs(q, pairs, nm, cen, R, k, exact=True)
            assert np.array_equal(ie, i) and np.array_equal(se.view(np.uint32), s.view(np.uint32))
        q16 = q.astype(np.float16)
        s, i = k_scan_pairs(q16, pairs, nm, cen, R, 10, capi.TQ_F16)
        so, io = _cpu_search(q16.astype(np.float32), p, nm, cen, R, 10)
        assert np.array_equal(i, io) and np.array_equal(s.view(np.uint32), so.view(np.uint32))


def test_mq_scan_q1024_with_ties():
    # configs[1]'s largest batch: 1024 normalized fp16 queries over 100,003 rows in which 40
    # rows appear 25 times each (exact ties across and within blocks), k = 10 and 32:
    # bit-identical to the reference core's search.
    rs = np.random.RandomState(1024)
    d, N = 128, 100_003
    R, cen, p, nm = _db(rs, N, d, 4)
    nm = nm / np.float32(np.sqrt(d))
    src = rs.choice(N, 40, replace=False)
    for j, r in enumerate(src):
        dst = rs.choice(N, 24, replace=False)
        p[dst] = p[r]
        nm[dst] = nm[r]
    pairs = k_pack_pairs(p, d)
    q = rs.randn(1024, d).astype(np.float32)
    q = (q / np.linalg.norm(q, axis=1, keepdims=True)).astype(np.float16)
    # the tied rows are the answer of some queries: queries 0-39 point at them
    q[:40] = (O.dequantize_mse(p[src], np.ones(40, np.float32), 4, d, R, cen)).astype(np.float16)
    qf = q.astype(np.float32)
    s32, i32 = _cpu_search(qf, p, nm, cen, R, 32)
    for k in (10, 32):
        s, i = k_scan_pairs(q, pairs, nm, cen, R, k, capi.TQ_F16)
        assert np.array_equal(i, i32[:, :k]), k
        assert np.array_equal(s.view(np.uint32), s32[:, :k].view(np.uint32)), k


def test_mq_scan_overflowing_lists_take_the_exact_fallback():
    # 3000 copies of query 0's best row: its lists overflow (the query is answered by the
    # exact scan), the other queries of the tile stay on the filter; all bit-exact.
    rs = np.random.RandomState(77)
    d = 128
    R, cen, p, nm = _db(rs, 30000, d, 4)
    q = rs.randn(5, d).astype(np.float32)
    top = int(np.argmax(O.lut_scores_f32(q[:1], p, nm, cen, R, 4)[0]))
    idx = rs.choice(30000, 3000, replace=False)
    p[idx] = p[top]
    nm[idx] = nm[top]
    pairs = k_pack_pairs(p, d)
    for k in (4, 32):
        s, i = k_scan_pairs(q, pairs, nm, cen, R, k)
        so, io = O.search_topk(q, p, nm, cen, R, 4, k)
        assert np.array_equal(i, io), k
        assert np.array_equal(s.view(np.uint32), so.view(np.uint32)), k


def test_mq_scan_special_norms():
    # zero, negative, huge, tiny and infinite norms (inf * 0 = NaN rows never listed)
    rs = np.random.RandomState(29)
    d = 128
    N = 150_000
    R, cen, p, nm = _db(rs, N, d, 4)
    nm = nm.copy()
    idx = rs.permutation(N)
    nm[idx[:2000]] = 0.0
    nm[idx[2000:4000]] *= -1.0
    nm[idx[4000:4010]] = 1e30
    nm[idx[4010:4020]] = -1e30
    nm[idx[4020:4030]] = 1e-38
    nm[idx[4030:4036]] = np.inf
    nm[idx[4036:4040]] = -np.inf
    pairs = k_pack_pairs(p, d)
    q = rs.randn(6, d).astype(np.float32)
    want = O.lut_scores_f32(q, p, nm, cen, R, 4)
    for k in (1, 10, 32):
        s, i = k_scan_pairs(q, pairs, nm, cen, R, k)
        so, io = _topk_no_nan(want, k)
        assert np.array_equal(i, io), k
        assert np.array_equal(s.view(np.uint32), so.view(np.uint32)), k


@pytest.mark.parametrize("qscale", [0.0, 1e-36, 1e-20, 1e20, 1e34])
def test_mq_scan_extreme_query_in_tile(qscale):
    # One query of the tile is zero or far outside the fp16 filter's range: the tile's
    # bound turns the filter off and every query is answered by the exact scan.
    rs = np.random.RandomState(37)
    d = 64
    N = 40_000
    R, cen, p, nm = _db(rs, N, d, 4)
    pairs = k_pack_pairs(p, d)
    q = rs.randn(4, d).astype(np.float32)
    q[2] *= np.float32(qscale)
    want = O.lut_scores_f32(q, p, nm, cen, R, 4)
    for k in (3, 10):
        s, i = k_scan_pairs(q, pairs, nm, cen, R, k)
        so, io = _topk_no_nan(want, k)
        assert np.array_equal(i, io), (qscale, k)
        assert np.array_equal(s.view(np.uint32), so.view(np.uint32)), (qscale, k)


def test_mq_scan_ulp_ties():
    # 600 copies of query 0's best row with norms a few ulps apart: the approximate scores
    # cannot order them, the exact rescoring does.
    rs = np.random.RandomState(43)
    d = 128
    N = 80_000
    R, cen, p, nm = _db(rs, N, d, 4)
    q = rs.randn(3, d).astype(np.float32)
    top = int(np.argmax(O.lut_scores_f32(q[:1], p, nm, cen, R, 4)[0]))
    idx = rs.choice(N, 600, replace=False)
    p[idx] = p[top]
    steps = rs.randint(-3, 4, size=600).astype(np.int32)
    nm[idx] = (nm[top].view(np.int32) + steps).view(np.float32)
    pairs = k_pack_pairs(p, d)
    for k in (5, 32):
        s, i = k_scan_pairs(q, pairs, nm, cen, R, k)
        so, io = O.search_topk(q, p, nm, cen, R, 4, k)
        assert np.array_equal(i, io), k
        assert np.array_equal(s.view(np.uint32), so.view(np.uint32)), k


def test_mq_scan_past_4gib_equals_exact_path():
    # 67.1M random rows of d = 128 (4.3 GB of codes, 64-bit row bases in the filter): the
    # filtered batch equals the exact multi-query scan bit for bit, and the answer rows'
    # scores equal the oracle's arithmetic on them.
    rs = np.random.RandomState(59)
    d = 128
    N = (1 << 26) + 1017
    R = O.dense_qr_rotation(d, 42)
    _, cen = O.lloyd_max_codebook(4, d)
    g = torch.Generator(device=DEV)
    g.manual_seed(7)
    pairs = torch.randint(0, 256, (N, d // 2), dtype=torch.uint8, device=DEV, generator=g)
    norms = (torch.rand(N, device=DEV, generator=g) + 0.5).float()
    q = rs.randn(3, d).astype(np.float32)
    s, i = k_scan_pairs(q, pairs, norms, cen, R, 10)
    se, ie = k_scan_pairs(q, pairs, norms, cen, R, 10, exact=True)
    assert np.array_equal(i, ie) and np.array_equal(s.view(np.uint32), se.view(np.uint32))
    for r in range(3):
        rows = pairs[torch.from_numpy(i[r]).to(DEV)].cpu().numpy()
        codes = np.empty((10, d), np.uint8)
        codes[:, 0::2], codes[:, 1::2] = rows >> 4, rows & 15
        want = O.lut_scores_f32(q[r:r + 1], O.pack_codes(codes, 4), norms[torch.from_numpy(i[r]).to(DEV)].cpu().numpy(),
                                cen, R, 4)[0]
        assert np.array_equal(s[r].view(np.uint32), want.view(np.uint32))
    del pairs, norms
    torch.cuda.empty_cache()


def _cpu_search_bits(q, p, nm, cen, R, bits, k):
    import cpu_libs
    return cpu_libs.search_packed(q, p, nm, R, cen, bits, k, "port")


@pytest.mark.parametrize("bits", [2, 3])
@pytest.mark.parametrize("d", [64, 128])
def test_mq_pair_rows_vs_oracle_and_exact_path(bits, d):
    # 2- and 3-bit pair rows: batches of 2, 64 and 130 queries over ~100k unit rows (ragged
    # N), fp32 and fp16 queries, k = 1, 10, 32 and 100: the multi-query filtered scan's ids
    # and scores bit-identical to the oracle (C restatement of the reference core) and to
    # the exact pair-row scan.
    rs = np.random.RandomState(300 + 10 * bits + d)
    N = 100_003 if d == 128 else 60_001
    R, cen, p, nm = _db(rs, N, d, bits)
    nm = nm / np.float32(np.sqrt(d))
    rows = k_pair_rows(p, d, bits)
    for Q in (2, 64, 130):
        q = rs.randn(Q, d).astype(np.float32)
        q /= np.linalg.norm(q, axis=1, keepdims=True)
        s100, i100 = _cpu_search_bits(q, p, nm, cen, R, bits, 100)
        if Q == 2:
            so, io = O.search_topk(q, p, nm, cen, R, bits, 100)
            assert np.array_equal(io, i100) and np.array_equal(so.view(np.uint32), s100.view(np.uint32))
        for k in (1, 10, 32, 100):
            s, i = k_scan_pair_rows(q, rows, nm, cen, R, bits, k)
            assert np.array_equal(i, i100[:, :k]), (Q, k)
            assert np.array_equal(s.view(np.uint32), s100[:, :k].view(np.uint32)), (Q, k)
            if k == 10:
                se, ie = k_scan_pair_rows(q, rows, nm, cen, R, bits, k, exact=True)
                assert np.array_equal(ie, i) and np.array_equal(se.view(np.uint32), s.view(np.uint32))
        q16 = q.astype(np.float16)
        s, i = k_scan_pair_rows(q16, rows, nm, cen, R, bits, 10, q_dt=capi.TQ_F16)
        so, io = _cpu_search_bits(q16.astype(np.float32), p, nm, cen, R, bits, 10)
        assert np.array_equal(i, io) and np.array_equal(s.view(np.uint32), so.view(np.uint32))


@pytest.mark.parametrize("bits", [2, 3])
def test_mq_pair_rows_q1024_with_ties(bits):
    # configs[1]'s 1024-query batch at 3 and 2 bits: normalized fp16 queries over 100,003
    # rows in which 40 rows appear 25 times each (queries 0-39 point at them), k = 10 and
    # 32: bit-identical to the reference core's search.
    rs = np.random.RandomState(1024 + bits)
    d, N = 128, 100_003
    R, cen, p, nm = _db(rs, N, d, bits)
    nm = nm / np.float32(np.sqrt(d))
    src = rs.choice(N, 40, replace=False)
    for r in src:
        dst = rs.choice(N, 24, replace=False)
        p[dst] = p[r]
        nm[dst] = nm[r]
    rows = k_pair_rows(p, d, bits)
    q = rs.randn(1024, d).astype(np.float32)
    q = (q / np.linalg.norm(q, axis=1, keepdims=True)).astype(np.float16)
    q[:40] = (O.dequantize_mse(p[src], np.ones(40, np.float32), bits, d, R, cen)).astype(np.float16)
    s32, i32 = _cpu_search_bits(q.astype(np.float32), p, nm, cen, R, bits, 32)
    for k in (10, 32):
        s, i = k_scan_pair_rows(q, rows, nm, cen, R, bits, k, q_dt=capi.TQ_F16)
        assert np.array_equal(i, i32[:, :k]), k
        assert np.array_equal(s.view(np.uint32), s32[:, :k].view(np.uint32)), k


@pytest.mark.parametrize("bits,d", [(2, 128), (3, 64)])
def test_mq_pair_rows_fallback_special_norms_and_ulp_ties(bits, d):
    # Query 0's best row copied over 3000 rows (its lists overflow: the exact pair-row scan
    # answers it, flagged alone), 600 more copies of query 1's best row with norms a few
    # ulps apart, and zero, negative, huge, tiny and infinite norms: all bit-exact.
    rs = np.random.RandomState(88 + bits)
    N = 80_000
    R, cen, p, nm = _db(rs, N, d, bits)
    nm = nm.copy()
    q = rs.randn(5, d).astype(np.float32)
    sc = O.lut_scores_f32(q[:2], p, nm, cen, R, bits)
    top0, top1 = int(np.argmax(sc[0])), int(np.argmax(sc[1]))
    perm = rs.permutation(np.setdiff1d(np.arange(N), [top0, top1]))
    a, b = perm[:3000], perm[3000:3600]
    p[a] = p[top0]
    nm[a] = nm[top0]
    p[b] = p[top1]
    nm[b] = (nm[top1].view(np.int32) + rs.randint(-3, 4, size=600).astype(np.int32)).view(np.float32)
    sp = perm[3600:]
    nm[sp[:2000]] = 0.0
    nm[sp[2000:4000]] *= -1.0
    nm[sp[4000:4010]] = 1e30
    nm[sp[4010:4020]] = -1e30
    nm[sp[4020:4030]] = 1e-38
    nm[sp[4030:4036]] = np.inf
    nm[sp[4036:4040]] = -np.inf
    rows = k_pair_rows(p, d, bits)
    want = O.lut_scores_f32(q, p, nm, cen, R, bits)
    for k in (4, 32):
        s, i = k_scan_pair_rows(q, rows, nm, cen, R, bits, k)
        so, io = _topk_no_nan(want, k)
        assert np.array_equal(i, io), k
        assert np.array_equal(s.view(np.uint32), so.view(np.uint32)), k


@pytest.mark.parametrize("qscale", [0.0, 1e-36, 1e20])
def test_mq_pair_rows_extreme_query_in_tile(qscale):
    # a zero or out-of-range query turns the tile's filter off: the exact scan answers all
    rs = np.random.RandomState(41)
    d, bits, N = 128, 3, 30_000
    R, cen, p, nm = _db(rs, N, d, bits)
    rows = k_pair_rows(p, d, bits)
    q = rs.randn(4, d).astype(np.float32)
    q[1] *= np.float32(qscale)
    want = O.lut_scores_f32(q, p, nm, cen, R, bits)
    s, i = k_scan_pair_rows(q, rows, nm, cen, R, bits, 10)
    so, io = _topk_no_nan(want, 10)
    assert np.array_equal(i, io) and np.array_equal(s.view(np.uint32), so.view(np.uint32))


# ------------------------------------------------------------------ top-k above 32
def _plant_ties(rs, p, nm, nsrc, copies):
    """Copy each of nsrc random rows (codes and norm) over `copies` other rows: exact ties."""
    N = p.shape[0]
    src = rs.choice(N, nsrc, replace=False)
    for r in src:
        dst = rs.choice(N, copies, replace=False)
        p[dst] = p[r]
        nm[dst] = nm[r]
    return src


@pytest.mark.parametrize("d,b", [(64, 1), (128, 2), (200, 3), (128, 4), (64, 4)])
def test_scan_large_k_bit_exact_with_ties(d, b):
    # k = 33, 100 and 128 over bit-plane rows (the exact scan's lists sized for k, the
    # long-list block merge, the large-k merge), one and several queries, 40 rows appearing
    # six times each (query 0 points at one of them), and a table of 77 rows (k > N pads
    # with (-inf, -1)): bit-identical to the oracle, tie order included.
    rs = np.random.RandomState(700 + d + b)
    N = 20_011
    R, cen, p, nm = _db(rs, N, d, b)
    nm = nm.copy()
    src = _plant_ties(rs, p, nm, 40, 5)
    for Q in (1, 5):
        q = rs.randn(Q, d).astype(np.float32)
        q[0] = O.dequantize_mse(p[src[:1]], np.ones(1, np.float32), b, d, R, cen)[0]
        so, io = O.search_topk(q, p, nm, cen, R, b, 128)
        for k in (33, 100, 128):
            s, i = k_scan(q, p, nm, cen, R, b, k)
            assert np.array_equal(i, io[:, :k]), (Q, k)
            assert np.array_equal(s.view(np.uint32), so[:, :k].view(np.uint32)), (Q, k)
        s, i = k_scan(q, p[:77], nm[:77], cen, R, b, 100)
        so, io = O.search_topk(q, p[:77], nm[:77], cen, R, b, 100)
        assert np.array_equal(i, io) and np.array_equal(s.view(np.uint32), so.view(np.uint32))


@pytest.mark.parametrize("bits,d", [(2, 64), (3, 128)])
def test_pair_rows_scan_large_k_with_ties(bits, d):
    # 2-/3-bit pair rows (one query per block row of the pair scan: twelve wave lists of up
    # to k entries merged by binary search), k = 64, 100, 128, with exact ties.
    rs = np.random.RandomState(710 + bits + d)
    N = 30_007
    R, cen, p, nm = _db(rs, N, d, bits)
    nm = nm.copy()
    src = _plant_ties(rs, p, nm, 40, 5)
    rows = k_pair_rows(p, d, bits)
    for Q in (1, 3):
        q = rs.randn(Q, d).astype(np.float32)
        q[0] = O.dequantize_mse(p[src[:1]], np.ones(1, np.float32), bits, d, R, cen)[0]
        so, io = O.search_topk(q, p, nm, cen, R, bits, 128)
        for k in (64, 100, 128):
            s, i = k_scan_pair_rows(q, rows, nm, cen, R, bits, k)
            assert np.array_equal(i, io[:, :k]), (Q, k)
            assert np.array_equal(s.view(np.uint32), so[:, :k].view(np.uint32)), (Q, k)


@pytest.mark.parametrize("d", [64, 128])
def test_pairs_scan_large_k_with_ties(d):
    # 4-bit pair rows, k = 64, 100 and 128: the multi-query filtered scan (a single query
    # included: above k = 32 it takes one query too), the exact multi-query scan and the
    # one-query pair scan, over 300k unit rows in which 60 rows appear eight times each
    # (queries 0-9 point at them): bit-identical to the C restatement of the reference core.
    rs = np.random.RandomState(128 + d)
    N = 300_007
    R, cen, p, nm = _db(rs, N, d, 4)
    nm = nm / np.float32(np.sqrt(d))
    src = _plant_ties(rs, p, nm, 60, 7)
    pairs = k_pack_pairs(p, d)
    for Q in (1, 64, 130):
        q = rs.randn(Q, d).astype(np.float32)
        q /= np.linalg.norm(q, axis=1, keepdims=True)
        t = min(Q, 10)
        q[:t] = O.dequantize_mse(p[src[:t]], np.ones(t, np.float32), 4, d, R, cen)
        s128, i128 = _cpu_search(q, p, nm, cen, R, 128)
        for k in (64, 100, 128):
            s, i = k_scan_pairs(q, pairs, nm, cen, R, k)
            assert np.array_equal(i, i128[:, :k]), (Q, k)
            assert np.array_equal(s.view(np.uint32), s128[:, :k].view(np.uint32)), (Q, k)
        se, ie = k_scan_pairs(q, pairs, nm, cen, R, 100, exact=True)
        assert np.array_equal(ie, i128[:, :100]), Q
        assert np.array_equal(se.view(np.uint32), s128[:, :100].view(np.uint32)), Q


# ------------------------------------------------------------------ decode attention
@pytest.mark.parametrize("d,kb,vb", [(64, 4, 2), (128, 3, 4), (64, 2, 3)])
def test_decode_attention_vs_f64(d, kb, vb):
    rs = np.random.RandomState(d + 10 * kb + vb)
    B, Hq, Hkv, Tm = 3, 8, 2, 2600
    seq = [37, 0, 2600]
    Rk, Rv = O.dense_qr_rotation(d, 42), O.dense_qr_rotation(d, 43)
    bk, ck = O.lloyd_max_codebook(kb, d)
    bv, cv = O.lloyd_max_codebook(vb, d)
    K = rs.randn(B * Hkv * Tm, d).astype(np.float32)
    K[:, rs.choice(d, 4, replace=False)] *= 20.0
    V = rs.randn(B * Hkv * Tm, d).astype(np.float32)
    kp, kn, _ = O.quantize_mse(K, kb, Rk, bk)
    vp, vn, _ = O.quantize_mse(V, vb, Rv, bv)
    kp, vp = kp.reshape(B, Hkv, Tm, -1), vp.reshape(B, Hkv, Tm, -1)
    kn, vn = kn.reshape(B, Hkv, Tm), vn.reshape(B, Hkv, Tm)
    q = rs.randn(B, Hq, d).astype(np.float32)
    scale = 1.0 / math.sqrt(d)
    want, want_lse = O.decode_attention_f64(q, kp, kn, vp, vn, seq, ck, cv, Rk, Rv, kb, vb, scale,
                                            return_lse=True)
    got, lse = k_decode(T(q), kp, kn, vp, vn, seq, ck, cv, Rk, Rv, kb, vb, scale)
    assert np.all(got[1] == 0) and np.isneginf(lse[1]).all()  # empty sequence
    assert np.max(np.abs(got - want)) <= 1e-3 * np.max(np.abs(want))
    ok = np.isfinite(want_lse)
    assert np.max(np.abs(lse[ok] - want_lse[ok])) <= 1e-4 * np.max(np.abs(want_lse[ok]))
    qb = torch.from_numpy(q).to(DEV).to(torch.bfloat16)
    want_b = O.decode_attention_f64(qb.float().cpu().numpy(), kp, kn, vp, vn, seq, ck, cv, Rk, Rv,
                                    kb, vb, scale)
    got_b, _ = k_decode(qb, kp, kn, vp, vn, seq, ck, cv, Rk, Rv, kb, vb, scale)
    assert np.max(np.abs(got_b - want_b)) <= 1e-2 * np.max(np.abs(want_b))


@pytest.mark.parametrize("kb,vb", [(4, 2), (3, 1), (2, 2), (1, 1), (4, 1)])
@pytest.mark.parametrize("G", [1, 3, 4])
def test_fused_decode_ragged_vs_f64(kb, vb, G):
    # head_dim 64, fp16/bf16 queries: the single-kernel MFMA path.  Ragged lengths cover
    # empty, sub-tile, tile-boundary and multi-split sequences and a capacity that is not
    # a multiple of 4; the second query set is scaled up so the softmax is peaky and the
    # running maximum moves.
    rs = np.random.RandomState(100 * kb + 10 * vb + G)
    d, Hkv, Tm = 64, 2, 5003
    seq = [0, 1, 3, 63, 64, 65, 257, 5003]
    B, Hq = len(seq), Hkv * G
    Rk, Rv = O.dense_qr_rotation(d, 42), O.dense_qr_rotation(d, 43)
    bk, ck = O.lloyd_max_codebook(kb, d)
    bv, cv = O.lloyd_max_codebook(vb, d)
    K = rs.randn(B * Hkv * Tm, d).astype(np.float32) * rs.uniform(0.2, 3.0, (B * Hkv * Tm, 1)).astype(np.float32)
    V = rs.randn(B * Hkv * Tm, d).astype(np.float32) * rs.uniform(0.2, 3.0, (B * Hkv * Tm, 1)).astype(np.float32)
    kp, kn, _ = O.quantize_mse(K, kb, Rk, bk)
    vp, vn, _ = O.quantize_mse(V, vb, Rv, bv)
    kp, vp = kp.reshape(B, Hkv, Tm, -1), vp.reshape(B, Hkv, Tm, -1)
    kn, vn = kn.reshape(B, Hkv, Tm), vn.reshape(B, Hkv, Tm)
    for qscale in (1.0, 6.0):
        q = (rs.randn(B, Hq, d) * qscale).astype(np.float32)
        for dt, tol in ((torch.bfloat16, 1e-2), (torch.float16, 3e-3)):
            qt = torch.from_numpy(q).to(DEV).to(dt)
            qf = qt.float().cpu().numpy()
            want, want_lse = O.decode_attention_f64(qf, kp, kn, vp, vn, seq, ck, cv, Rk, Rv, kb, vb,
                                                    0.125, return_lse=True)
            got, lse = k_decode(qt, kp, kn, vp, vn, seq, ck, cv, Rk, Rv, kb, vb, 0.125)
            assert np.all(got[0] == 0) and np.isneginf(lse[0]).all()
            for bi in range(1, B):
                err = np.max(np.abs(got[bi] - want[bi])) / np.max(np.abs(want[bi]))
                assert err <= tol, (qscale, dt, seq[bi], err)
            ok = np.isfinite(want_lse)
            assert np.max(np.abs(lse[ok] - want_lse[ok]) / np.maximum(1.0, np.abs(want_lse[ok]))) <= 1e-4


@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("vb", [2, 3, 4])
@pytest.mark.parametrize("dt", ["bf16", "f16"])
def test_cache_append_dl_equals_quantize_then_pack(d, vb, dt):
    # tq_cache_append_dl (one token per stream, one launch) against tq_rotate_and_quantize
    # (rounding in the input type) followed by tq_pack_decode_layout, bit for bit: caches
    # that start as random bytes (the other tokens' bits must survive), positions on both
    # sides of tile boundaries, fp32 and 16-bit norm caches, outlier channels.
    tdt, cdt = (torch.bfloat16, capi.TQ_BF16) if dt == "bf16" else (torch.float16, capi.TQ_F16)
    rs = np.random.RandomState(500 + 10 * vb + d)
    S, t_cap = 37, 192
    Rk, Rv = O.dense_qr_rotation(d, 42), O.dense_qr_rotation(d, 43)
    bk, _ = O.lloyd_max_codebook(4, d)
    bv, _ = O.lloyd_max_codebook(vb, d)
    scales = np.ones(d, np.float32)
    scales[rs.choice(d, 4, replace=False)] = 20.0
    g = torch.Generator(device=DEV)
    g.manual_seed(vb * 1000 + d)
    kp0 = torch.randint(0, 256, (S, t_cap, d // 2), dtype=torch.uint8, device=DEV, generator=g)
    vp0 = torch.randint(0, 256, (S, t_cap // 64, 8 * vb * d), dtype=torch.uint8, device=DEV, generator=g)
    for ndt, ncode in ((torch.float32, capi.TQ_F32), (tdt, cdt)):
        kn0 = torch.randn(S, t_cap, device=DEV, generator=g).to(ndt)
        vn0 = torch.randn(S, t_cap, device=DEV, generator=g).to(ndt)
        fused = [kp0.clone(), kn0.clone(), vp0.clone(), vn0.clone()]
        ref = [kp0.clone(), kn0.clone(), vp0.clone(), vn0.clone()]
        for pos in (0, 1, 62, 63, 64, 65, 127, 128, 191):
            k = torch.from_numpy(rs.randn(S, d).astype(np.float32) * scales).to(DEV).to(tdt)
            v = torch.from_numpy(rs.randn(S, d).astype(np.float32) * scales).to(DEV).to(tdt)
            if pos == 65:
                k[3] = 0  # a zero row: norm 0, the code of 0 everywhere
            capi.check(L().tq_cache_append_dl(
                capi.p(k), capi.p(v), cdt, capi.i64(S), capi.i32(d), capi.p(T(Rk)), capi.p(T(bk)),
                capi.p(T(Rv)), capi.p(T(bv)), capi.i32(vb), capi.p(fused[0]), capi.p(fused[1]),
                capi.p(fused[2]), capi.p(fused[3]), ncode, capi.i64(t_cap), capi.i64(pos), capi.stream()))
            kq, kn = k_quantize(k, Rk, bk, 4, cdt, cdt)
            vq, vn = k_quantize(v, Rv, bv, vb, cdt, cdt)
            k_pack_dl(kq.reshape(S, 1, -1), t_cap, pos, 0, cache=ref[0], d=d)
            k_pack_dl(vq.reshape(S, 1, -1), t_cap, pos, 1, cache=ref[2], vbits=vb, d=d)
            ref[1][:, pos] = torch.from_numpy(kn).to(DEV).to(ndt)
            ref[3][:, pos] = torch.from_numpy(vn).to(DEV).to(ndt)
        sync()
        for name, a, b in zip(("kpairs", "knorms", "vtiles", "vnorms"), fused, ref):
            ai = a.view(torch.uint8) if a.dtype == torch.uint8 else a.view(torch.int16 if a.element_size() == 2 else torch.int32)
            bi = b.view(torch.uint8) if b.dtype == torch.uint8 else b.view(torch.int16 if b.element_size() == 2 else torch.int32)
            assert torch.equal(ai, bi), (name, ndt)
        # untouched positions keep their bytes
        keep = [t for t in range(t_cap) if t not in (0, 1, 62, 63, 64, 65, 127, 128, 191)]
        assert torch.equal(fused[0][:, keep], kp0[:, keep])


def test_cache_append_dl_refusals():
    k = torch.zeros(4, 64, dtype=torch.float32, device=DEV)
    buf = torch.zeros(4096, dtype=torch.uint8, device=DEV)
    R = T(O.dense_qr_rotation(64, 42))
    bk, _ = O.lloyd_max_codebook(4, 64)
    args = lambda dt, d, vb, t_cap, pos: (capi.p(k), capi.p(k), dt, capi.i64(4), capi.i32(d), capi.p(R), capi.p(T(bk)),
                                          capi.p(R), capi.p(T(bk)), capi.i32(vb), capi.p(buf), capi.p(buf),
                                          capi.p(buf), capi.p(buf), capi.TQ_F32, capi.i64(t_cap), capi.i64(pos),
                                          capi.stream())
    for bad in ((capi.TQ_F32, 64, 2, 64, 0), (capi.TQ_BF16, 96, 2, 64, 0), (capi.TQ_BF16, 64, 5, 64, 0),
                (capi.TQ_BF16, 64, 2, 60, 0), (capi.TQ_BF16, 64, 2, 64, 64)):
        assert L().tq_cache_append_dl(*args(*bad)) != 0, bad


def test_decode_layout_pack_roundtrip():
    # Appends in uneven pieces (partial value blocks are merged with their earlier tokens);
    # the layout bytes are checked against an independent numpy packing of the codes and
    # the unpacked rows must equal the bit-plane input.
    rs = np.random.RandomState(21)
    S, t_cap, d = 3, 128, 64
    kcodes = rs.randint(0, 16, (S, t_cap, d))
    vcodes = rs.randint(0, 4, (S, t_cap, d))
    kp = np.stack([O.pack_codes(kcodes[s], 4) for s in range(S)])
    vp = np.stack([O.pack_codes(vcodes[s], 2) for s in range(S)])
    kc = vc = None
    for pos, n in ((0, 5), (5, 1), (6, 7), (13, 3), (16, 21), (37, 11), (48, 30), (78, 50)):
        kc = k_pack_dl(np.ascontiguousarray(kp[:, pos:pos + n]), t_cap, pos, 0, kc)
        vc = k_pack_dl(np.ascontiguousarray(vp[:, pos:pos + n]), t_cap, pos, 1, vc)
    want_k = (kcodes[:, :, 0::2] << 4) | kcodes[:, :, 1::2]
    assert np.array_equal(kc.cpu().numpy(), want_k.astype(np.uint8))
    # values: tiles of 64 tokens; byte 16*(16*sl + c) + 4*m + dg holds dim 16*dg + c of
    # tokens 64*tile + 4*(4*m + sl) + t at bits 2t
    vb = vcodes.reshape(S, t_cap // 64, 4, 4, 4, 4, 16)  # [S, tile, m, sl, t, dg, c]
    packed_v = vb[:, :, :, :, 0] | (vb[:, :, :, :, 1] << 2) | (vb[:, :, :, :, 2] << 4) | (vb[:, :, :, :, 3] << 6)
    want_v = packed_v.transpose(0, 1, 3, 5, 2, 4).reshape(S, t_cap // 64, 1024)  # [S, tile, sl, c, m, dg]
    assert np.array_equal(vc.cpu().numpy(), want_v.astype(np.uint8))
    assert np.array_equal(k_unpack_dl(kc, t_cap, 0, t_cap, 0), kp)
    assert np.array_equal(k_unpack_dl(vc, t_cap, 7, 30, 1), vp[:, 7:37])
    assert np.array_equal(k_unpack_dl(vc, t_cap, 60, 68, 1), vp[:, 60:128])


@pytest.mark.parametrize("G", [1, 2, 4])
def test_decode_layout_attention_vs_f64(G):
    # Same cases as the bit-plane kernel, through the decode layout; fp32 queries take
    # the exact value product.
    rs = np.random.RandomState(300 + G)
    d, Hkv, Tc = 64, 2, 5056
    seq = [0, 1, 3, 63, 64, 65, 257, 513, 5004]
    B, Hq = len(seq), Hkv * G
    Rk, Rv = O.dense_qr_rotation(d, 42), O.dense_qr_rotation(d, 43)
    bk, ck = O.lloyd_max_codebook(4, d)
    bv, cv = O.lloyd_max_codebook(2, d)
    n = B * Hkv * Tc
    K = rs.randn(n, d).astype(np.float32) * rs.uniform(0.2, 3.0, (n, 1)).astype(np.float32)
    V = rs.randn(n, d).astype(np.float32) * rs.uniform(0.2, 3.0, (n, 1)).astype(np.float32)
    kp, kn, _ = O.quantize_mse(K, 4, Rk, bk)
    vp, vn, _ = O.quantize_mse(V, 2, Rv, bv)
    kc = k_pack_dl(kp.reshape(B * Hkv, Tc, -1), Tc, 0, 0)
    vc = k_pack_dl(vp.reshape(B * Hkv, Tc, -1), Tc, 0, 1)
    kp, vp = kp.reshape(B, Hkv, Tc, -1), vp.reshape(B, Hkv, Tc, -1)
    kn, vn = kn.reshape(B, Hkv, Tc), vn.reshape(B, Hkv, Tc)
    for qscale in (1.0, 6.0):
        q = (rs.randn(B, Hq, d) * qscale).astype(np.float32)
        for dt, tol in ((torch.float32, 1e-3), (torch.bfloat16, 1e-2), (torch.float16, 3e-3)):
            qt = torch.from_numpy(q).to(DEV).to(dt)
            qf = qt.float().cpu().numpy()
            want, want_lse = O.decode_attention_f64(qf, kp, kn, vp, vn, seq, ck, cv, Rk, Rv, 4, 2,
                                                    0.125, return_lse=True)
            got, lse = k_decode_dl(qt, kc, kn, vc, vn, seq, ck, cv, Rk, Rv, 0.125)
            assert np.all(got[0] == 0) and np.isneginf(lse[0]).all()
            for bi in range(1, B):
                err = np.max(np.abs(got[bi] - want[bi])) / np.max(np.abs(want[bi]))
                assert err <= (1e-4 if dt == torch.float32 else tol), (qscale, dt, seq[bi], err)
            ok = np.isfinite(want_lse)
            # bf16 queries score with one fp16 product per term (2^-11 per operand, finer
            # than bf16 arithmetic); fp32 / fp16 queries use hi + lo parts
            lse_tol = 2e-3 if dt == torch.bfloat16 else 1e-5
            assert np.max(np.abs(lse[ok] - want_lse[ok]) / np.maximum(1.0, np.abs(want_lse[ok]))) <= lse_tol


def dl_value_tiles_np(codes, vb):
    """Independent numpy packing of 2/3/4-bit value codes [S, t_cap, 64] into decode-layout
    tiles [S, t_cap/64, 512*vb]: lane L = 16 sl + c owns words 0-3 at byte 16 L and the
    rest at 1024 + (8 vb - 16) L; byte k = 2 (m % 2) + t // 2 of word w holds the pair
    (tokens t = 2p, 2p + 1 of block 4m + sl, dim j): vb 4: w = 4 (m // 2) + j // 16, codes
    at bits 0-3 / 4-7; vb 3: dims j < 48 at w = 3 (m // 2) + j // 16, bits 0-2 / 3-5, and
    dims 48-63's 6-bit pair index spread two bits at a time over bits 6-7 of words
    3 (m // 2) + 0, 1, 2."""
    S, tc, d = codes.shape
    nt = tc // 64
    if vb == 2:  # byte 16 (16 sl + c) + 4 m + dg: dim 16 dg + c of four tokens at bits 2 t
        v = codes.reshape(S, nt, 4, 4, 4, 4, 16).astype(np.uint32)  # [S, tile, m, sl, t, dg, c]
        packed = v[:, :, :, :, 0] | (v[:, :, :, :, 1] << 2) | (v[:, :, :, :, 2] << 4) | (v[:, :, :, :, 3] << 6)
        return packed.transpose(0, 1, 3, 5, 2, 4).reshape(S, nt, 1024).astype(np.uint8)
    x = codes.reshape(S, nt, 4, 4, 4, d).astype(np.uint32)  # [S, tile, m, sl, t, j]
    out = np.zeros((S, nt, 512 * vb), np.uint32)

    def off(L, w, k):
        return 16 * L + 4 * w + k if w < 4 else 1024 + (8 * vb - 16) * L + 4 * (w - 4) + k

    for sl in range(4):
        for c in range(16):
            L = 16 * sl + c
            for m in range(4):
                G, mm = divmod(m, 2)
                for pp in range(2):
                    k = 2 * mm + pp
                    e0, e1 = x[:, :, m, sl, 2 * pp], x[:, :, m, sl, 2 * pp + 1]  # [S, nt, j]
                    if vb == 4:
                        for dg in range(4):
                            j = 16 * dg + c
                            out[:, :, off(L, 4 * G + dg, k)] = e0[..., j] | (e1[..., j] << 4)
                    else:
                        i3 = e0[..., 48 + c] | (e1[..., 48 + c] << 3)
                        for i in range(3):
                            j = 16 * i + c
                            out[:, :, off(L, 3 * G + i, k)] = (e0[..., j] | (e1[..., j] << 3) |
                                                               (((i3 >> (2 * i)) & 3) << 6))
    return out.astype(np.uint8)


@pytest.mark.parametrize("vb", [3, 4])
def test_decode_layout_value_tiles_pack_roundtrip(vb):
    # Appends in uneven pieces that straddle pairs, blocks and tiles; the tile bytes must
    # equal the independent numpy packing and unpack to the bit-plane input.
    rs = np.random.RandomState(40 + vb)
    S, t_cap, d = 3, 192, 64
    codes = rs.randint(0, 1 << vb, (S, t_cap, d))
    vp = np.stack([O.pack_codes(codes[s], vb) for s in range(S)])
    vc = None
    for pos, n in ((0, 1), (1, 2), (3, 6), (9, 30), (39, 25), (64, 65), (129, 63)):
        vc = k_pack_dl(np.ascontiguousarray(vp[:, pos:pos + n]), t_cap, pos, 1, vc, vbits=vb)
    assert np.array_equal(vc.cpu().numpy(), dl_value_tiles_np(codes, vb))
    assert np.array_equal(k_unpack_dl(vc, t_cap, 0, t_cap, 1, vbits=vb), vp)
    assert np.array_equal(k_unpack_dl(vc, t_cap, 5, 70, 1, vbits=vb), vp[:, 5:75])
    # a planted transposition in the numpy packing (dims 48-63 swapped with 32-47) must
    # not pass: the dim group 3 bits are where the 3-bit layout differs
    if vb == 3:
        bad = codes.copy()
        bad[:, :, 32:48], bad[:, :, 48:64] = codes[:, :, 48:64], codes[:, :, 32:48]
        assert not np.array_equal(vc.cpu().numpy(), dl_value_tiles_np(bad, vb))


@pytest.mark.parametrize("vb,G", [(3, 1), (3, 4), (4, 4), (3, 8), (2, 7), (2, 8), (4, 5)])
def test_decode_layout_vbits_and_groups_vs_f64(vb, G):
    # 3- and 4-bit value tiles and more than four query heads per KV head (launched four
    # heads at a time); ragged lengths, fp32 / bf16 / fp16 queries.
    rs = np.random.RandomState(500 + 10 * vb + G)
    d, Hkv, Tc = 64, 2, 2112
    seq = [0, 1, 63, 64, 65, 513, 2100]
    B, Hq = len(seq), Hkv * G
    Rk, Rv = O.dense_qr_rotation(d, 42), O.dense_qr_rotation(d, 43)
    bk, ck = O.lloyd_max_codebook(4, d)
    bv, cv = O.lloyd_max_codebook(vb, d)
    n = B * Hkv * Tc
    K = rs.randn(n, d).astype(np.float32) * rs.uniform(0.2, 3.0, (n, 1)).astype(np.float32)
    V = rs.randn(n, d).astype(np.float32) * rs.uniform(0.2, 3.0, (n, 1)).astype(np.float32)
    kp, kn, _ = O.quantize_mse(K, 4, Rk, bk)
    vp, vn, _ = O.quantize_mse(V, vb, Rv, bv)
    kc = k_pack_dl(kp.reshape(B * Hkv, Tc, -1), Tc, 0, 0)
    vc = k_pack_dl(vp.reshape(B * Hkv, Tc, -1), Tc, 0, 1, vbits=vb)
    kp, vp = kp.reshape(B, Hkv, Tc, -1), vp.reshape(B, Hkv, Tc, -1)
    kn, vn = kn.reshape(B, Hkv, Tc), vn.reshape(B, Hkv, Tc)
    q = (rs.randn(B, Hq, d) * 3.0).astype(np.float32)
    for dt, tol in ((torch.float32, 1e-4), (torch.bfloat16, 1e-2), (torch.float16, 3e-3)):
        qt = torch.from_numpy(q).to(DEV).to(dt)
        qf = qt.float().cpu().numpy()
        want, want_lse = O.decode_attention_f64(qf, kp, kn, vp, vn, seq, ck, cv, Rk, Rv, 4, vb,
                                                0.125, return_lse=True)
        got, lse = k_decode_dl(qt, kc, kn, vc, vn, seq, ck, cv, Rk, Rv, 0.125, vbits=vb)
        assert np.all(got[0] == 0) and np.isneginf(lse[0]).all()
        for bi in range(1, B):
            err = np.max(np.abs(got[bi] - want[bi])) / np.max(np.abs(want[bi]))
            assert err <= tol, (dt, seq[bi], err)
        ok = np.isfinite(want_lse)
        # bf16 queries: one fp16 product per q.K term (2^-11 per operand), so the lse is
        # held to the bf16 output tolerance; fp32 / fp16 queries use hi + lo parts
        lse_tol = 1e-2 if dt == torch.bfloat16 else 1e-5
        assert np.max(np.abs(lse[ok] - want_lse[ok]) / np.maximum(1.0, np.abs(want_lse[ok]))) <= lse_tol


@pytest.mark.parametrize("vb", [2, 3, 4])
@pytest.mark.parametrize("case", ["516x4", "515x8"])
def test_decode_layout_two_streams_per_workgroup_vs_f64(vb, case):
    # At least two streams per CU (B * hkv >= 512 on the 256-CU MI355X) the kernel runs two
    # streams per workgroup, four waves each: 516 streams (G = 4) and an odd 515 (G = 8:
    # two launches of four heads; the last workgroup's second stream does not exist), with
    # ragged and empty sequences, window starts, fp32 and bf16 norms, fp32 / bf16 queries.
    rs = np.random.RandomState(900 + vb + (0 if case == "516x4" else 50))
    d = 64
    if case == "516x4":
        B, Hkv, G, Tc = 129, 4, 4, 192
    else:
        B, Hkv, G, Tc = 515, 1, 8, 128
    Hq = Hkv * G
    seq = rs.randint(0, Tc + 1, size=B)
    seq[:6] = [0, 1, 63, 64, 65, Tc]
    starts = np.minimum(rs.randint(0, 40, size=B), seq)
    starts[:6] = 0
    Rk, Rv = O.dense_qr_rotation(d, 42), O.dense_qr_rotation(d, 43)
    bk, ck = O.lloyd_max_codebook(4, d)
    bv, cv = O.lloyd_max_codebook(vb, d)
    n = B * Hkv * Tc
    K = rs.randn(n, d).astype(np.float32) * rs.uniform(0.2, 3.0, (n, 1)).astype(np.float32)
    V = rs.randn(n, d).astype(np.float32) * rs.uniform(0.2, 3.0, (n, 1)).astype(np.float32)
    kp, kn, _ = O.quantize_mse(K, 4, Rk, bk)
    vp, vn, _ = O.quantize_mse(V, vb, Rv, bv)
    kc = k_pack_dl(kp.reshape(B * Hkv, Tc, -1), Tc, 0, 0)
    vc = k_pack_dl(vp.reshape(B * Hkv, Tc, -1), Tc, 0, 1, vbits=vb)
    kp, vp = kp.reshape(B, Hkv, Tc, -1), vp.reshape(B, Hkv, Tc, -1)
    kn, vn = kn.reshape(B, Hkv, Tc), vn.reshape(B, Hkv, Tc)
    q = (rs.randn(B, Hq, d) * 3.0).astype(np.float32)
    for dt, tol, nd in ((torch.float32, 1e-4, None), (torch.bfloat16, 1e-2, torch.bfloat16)):
        qt = torch.from_numpy(q).to(DEV).to(dt)
        qf = qt.float().cpu().numpy()
        knr = T(kn, nd).float().cpu().numpy() if nd is not None else kn
        vnr = T(vn, nd).float().cpu().numpy() if nd is not None else vn
        for st in (None, starts):
            got, lse = k_decode_dl(qt, kc, kn, vc, vn, seq, ck, cv, Rk, Rv, 0.125, vbits=vb,
                                   seq_starts=st, norm_dtype=nd)
            lo = np.zeros(B, np.int64) if st is None else st
            for bi in range(B):
                if seq[bi] - lo[bi] <= 0:
                    assert np.all(got[bi] == 0) and np.isneginf(lse[bi]).all(), (dt, bi)
                    continue
                rows = slice(int(lo[bi]), int(seq[bi]))
                want, want_lse = O.decode_attention_f64(
                    qf[bi:bi + 1], kp[bi:bi + 1, :, rows], knr[bi:bi + 1, :, rows], vp[bi:bi + 1, :, rows],
                    vnr[bi:bi + 1, :, rows], [seq[bi] - lo[bi]], ck, cv, Rk, Rv, 4, vb, 0.125, return_lse=True)
                err = np.max(np.abs(got[bi] - want[0])) / np.max(np.abs(want[0]))
                assert err <= tol, (dt, case, bi, err)
                lse_tol = 1e-2 if dt == torch.bfloat16 else 1e-5
                assert np.max(np.abs(lse[bi] - want_lse[0]) / np.maximum(1.0, np.abs(want_lse[0]))) <= lse_tol


@pytest.mark.parametrize("vb", [2, 3])
def test_decode_layout_window_vs_f64(vb):
    # Windows [start, len) of each sequence (left-padded batches): tokens before start are
    # masked; starts inside a 64-token tile, on a tile edge, at 0, at len - 1 and at len
    # (an empty window: zeros and lse -inf).  Against float64 attention over the window's
    # rows alone.
    rs = np.random.RandomState(700 + vb)
    d, Hkv, G, Tc = 64, 2, 4, 2112
    seq = [700, 1500, 64, 2100, 3, 513, 90]
    starts = [0, 37, 63, 1290, 2, 513, 64]
    B, Hq = len(seq), Hkv * G
    Rk, Rv = O.dense_qr_rotation(d, 42), O.dense_qr_rotation(d, 43)
    bk, ck = O.lloyd_max_codebook(4, d)
    bv, cv = O.lloyd_max_codebook(vb, d)
    n = B * Hkv * Tc
    K = rs.randn(n, d).astype(np.float32)
    V = rs.randn(n, d).astype(np.float32)
    kp, kn, _ = O.quantize_mse(K, 4, Rk, bk)
    vp, vn, _ = O.quantize_mse(V, vb, Rv, bv)
    kc = k_pack_dl(kp.reshape(B * Hkv, Tc, -1), Tc, 0, 0)
    vc = k_pack_dl(vp.reshape(B * Hkv, Tc, -1), Tc, 0, 1, vbits=vb)
    kp, vp = kp.reshape(B, Hkv, Tc, -1), vp.reshape(B, Hkv, Tc, -1)
    kn, vn = kn.reshape(B, Hkv, Tc), vn.reshape(B, Hkv, Tc)
    # stale norms before each window must not reach the output
    for b in range(B):
        kn[b, :, :starts[b]] = np.nan
        vn[b, :, :starts[b]] = np.nan
    q = (rs.randn(B, Hq, d) * 3.0).astype(np.float32)
    for dt, tol in ((torch.float32, 1e-4), (torch.bfloat16, 1e-2)):
        qt = torch.from_numpy(q).to(DEV).to(dt)
        qf = qt.float().cpu().numpy()
        got, lse = k_decode_dl(qt, kc, kn, vc, vn, seq, ck, cv, Rk, Rv, 0.125, vbits=vb,
                               seq_starts=starts)
        for b in range(B):
            s0, t = starts[b], seq[b]
            if s0 >= t:
                assert np.all(got[b] == 0) and np.isneginf(lse[b]).all()
                continue
            want = O.decode_attention_f64(qf[b:b + 1], kp[b:b + 1, :, s0:t], kn[b:b + 1, :, s0:t],
                                          vp[b:b + 1, :, s0:t], vn[b:b + 1, :, s0:t], [t - s0], ck, cv,
                                          Rk, Rv, 4, vb, 0.125)[0]
            err = np.max(np.abs(got[b] - want)) / np.max(np.abs(want))
            assert err <= tol, (dt, b, err)
    # starts of 0 equal the plain entry point bit for bit
    qt = torch.from_numpy(q).to(DEV).to(torch.bfloat16)
    kn0, vn0 = np.nan_to_num(kn), np.nan_to_num(vn)
    a, la = k_decode_dl(qt, kc, kn0, vc, vn0, seq, ck, cv, Rk, Rv, 0.125, vbits=vb, seq_starts=[0] * B)
    b_, lb = k_decode_dl(qt, kc, kn0, vc, vn0, seq, ck, cv, Rk, Rv, 0.125, vbits=vb)
    assert np.array_equal(a, b_) and np.array_equal(la, lb)


@pytest.mark.parametrize("nd", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("vb", [2, 3, 4])
def test_decode_layout_16bit_norms(nd, vb):
    # A 16-bit model's cache keeps its norms in that dtype (the reference's quantize returns
    # them so): the kernel reads them as 16-bit values.  With norms that are exactly
    # representable in nd, the output equals the fp32-norm call's up to the compiler's
    # contraction choices (an fp16 norm can enter a mixed-precision fma directly): within
    # 1e-5 of the output's maximum, lse within 1e-6.
    rs = np.random.RandomState(800 + vb)
    d, Hkv, G, Tc = 64, 2, 4, 1088
    seq = [1000, 5, 64, 1088]
    B, Hq = len(seq), Hkv * G
    Rk, Rv = O.dense_qr_rotation(d, 42), O.dense_qr_rotation(d, 43)
    _, ck = O.lloyd_max_codebook(4, d)
    _, cv = O.lloyd_max_codebook(vb, d)
    kp = rs.randint(0, 256, (B * Hkv, Tc, 32)).astype(np.uint8)
    vp = rs.randint(0, 256, (B * Hkv, Tc, 8 * vb)).astype(np.uint8)
    kc = k_pack_dl(kp, Tc, 0, 0)  # any bytes are valid bit-plane rows
    vc = k_pack_dl(vp, Tc, 0, 1, vbits=vb)
    to16 = lambda x: torch.from_numpy(x).to(nd).float().numpy()
    kn = to16(rs.uniform(0.3, 3.0, (B, Hkv, Tc)).astype(np.float32))
    vn = to16(rs.uniform(0.3, 3.0, (B, Hkv, Tc)).astype(np.float32))
    for qdt in (torch.float32, torch.bfloat16):
        qt = torch.from_numpy(rs.randn(B, Hq, d).astype(np.float32)).to(DEV).to(qdt)
        a, la = k_decode_dl(qt, kc, kn, vc, vn, seq, ck, cv, Rk, Rv, 0.125, vbits=vb)
        b_, lb = k_decode_dl(qt, kc, kn, vc, vn, seq, ck, cv, Rk, Rv, 0.125, vbits=vb, norm_dtype=nd)
        assert np.max(np.abs(a - b_)) <= 1e-5 * np.max(np.abs(a)), qdt
        ok = np.isfinite(la)
        assert np.array_equal(ok, np.isfinite(lb))
        assert np.max(np.abs(la[ok] - lb[ok])) <= 1e-6 * max(1.0, np.max(np.abs(la[ok]))), qdt


@pytest.mark.parametrize("vb,T", [(2, 2048), (3, 1024)])
def test_decode_layout_config_shape_vs_f64(vb, T):
    # The benchmarked launch: B = 32, Hq = 32, Hkv = 8 (256 streams, one split per stream,
    # so the kernel applies R_v and writes the output itself), bf16 K/V with four outlier
    # channels per KV head scaled x20, bf16 queries, scale 1/8.
    rs = np.random.RandomState(7 + vb)
    B, Hq, Hkv, d = 32, 32, 8, 64
    assert L().tq_decode_dl_workspace_bytes(B, Hq, Hkv, T) >= 256
    Rk, Rv = O.dense_qr_rotation(d, 42), O.dense_qr_rotation(d, 43)
    bk, ck = O.lloyd_max_codebook(4, d)
    bv, cv = O.lloyd_max_codebook(vb, d)
    K = rs.randn(B, Hkv, T, d).astype(np.float32)
    V = rs.randn(B, Hkv, T, d).astype(np.float32)
    for h in range(Hkv):
        ch = rs.choice(d, 4, replace=False)
        K[:, h, :, ch] *= 20.0
        V[:, h, :, ch] *= 20.0
    K = torch.from_numpy(K).to(torch.bfloat16).float().numpy().reshape(-1, d)
    V = torch.from_numpy(V).to(torch.bfloat16).float().numpy().reshape(-1, d)
    kp, kn, _ = O.quantize_mse(K, 4, Rk, bk)
    vp, vn, _ = O.quantize_mse(V, vb, Rv, bv)
    kc = k_pack_dl(kp.reshape(B * Hkv, T, -1), T, 0, 0)
    vc = k_pack_dl(vp.reshape(B * Hkv, T, -1), T, 0, 1, vbits=vb)
    kp, vp = kp.reshape(B, Hkv, T, -1), vp.reshape(B, Hkv, T, -1)
    kn, vn = kn.reshape(B, Hkv, T), vn.reshape(B, Hkv, T)
    qt = torch.from_numpy(rs.randn(B, Hq, d).astype(np.float32)).to(DEV).to(torch.bfloat16)
    seq = [T] * B
    want = O.decode_attention_f64(qt.float().cpu().numpy(), kp, kn, vp, vn, seq, ck, cv, Rk, Rv,
                                  4, vb, 0.125)
    got, _ = k_decode_dl(qt, kc, kn, vc, vn, seq, ck, cv, Rk, Rv, 0.125, vbits=vb)
    # the bf16 output tolerance per batch row (max |error| over its heads and dims against
    # its largest output), as the other decode tests
    err = max(np.max(np.abs(got[b] - want[b])) / np.max(np.abs(want[b])) for b in range(B))
    assert err <= 1e-2, err
    # per head: well inside what the reference's own bf16 arithmetic gives on these rows
    # (history rounded to bf16, bf16 output; about 0.1 here against float64)
    ref = O.decode_attention_bf16_reference(qt.float().cpu().numpy(), kp, kn, vp, vn, seq, ck, cv,
                                            Rk, Rv, 4, vb, 0.125)
    head = lambda x: np.max(np.max(np.abs(x - want), axis=-1) / np.max(np.abs(want), axis=-1))
    assert head(got) <= 0.5 * head(ref), (head(got), head(ref))


@pytest.mark.parametrize("vb", [2, 3, 4])
def test_decode_layout_d128_pack_roundtrip(vb):
    # head_dim 128: key rows of 64 pair bytes; value tiles of two 64-dim halves, each the
    # 64-dim tile of its dims (the independent numpy packing per half), from appends in
    # uneven pieces
    rs = np.random.RandomState(80 + vb)
    S, t_cap, d = 2, 192, 128
    codes = rs.randint(0, 1 << vb, (S, t_cap, d))
    vp = np.stack([O.pack_codes(codes[s], vb) for s in range(S)])
    vc = None
    for pos, n in ((0, 3), (3, 61), (64, 65), (129, 63)):
        vc = k_pack_dl(np.ascontiguousarray(vp[:, pos:pos + n]), t_cap, pos, 1, vc, vbits=vb, d=d)
    tiles = vc.cpu().numpy().reshape(S, t_cap // 64, 2, 512 * vb)
    for h in range(2):
        assert np.array_equal(tiles[:, :, h].reshape(S, t_cap // 64, -1),
                              dl_value_tiles_np(codes[:, :, 64 * h:64 * h + 64], vb)), h
    assert np.array_equal(k_unpack_dl(vc, t_cap, 0, t_cap, 1, vbits=vb, d=d), vp)
    assert np.array_equal(k_unpack_dl(vc, t_cap, 7, 100, 1, vbits=vb, d=d), vp[:, 7:107])
    kcodes = rs.randint(0, 16, (S, t_cap, d))
    kpk = np.stack([O.pack_codes(kcodes[s], 4) for s in range(S)])
    kc = k_pack_dl(kpk, t_cap, 0, 0, d=d)
    pairs = kc.cpu().numpy()
    assert np.array_equal(pairs, ((kcodes[:, :, 0::2] << 4) | kcodes[:, :, 1::2]).astype(np.uint8))
    assert np.array_equal(k_unpack_dl(kc, t_cap, 0, t_cap, 0, d=d), kpk)


@pytest.mark.parametrize("vb,G", [(2, 4), (3, 4), (4, 4), (2, 1), (3, 6)])
def test_decode_layout_d128_vs_f64(vb, G):
    # head_dim 128 (two 64-dim halves per operand): Hq 32 / Hkv 8 at G = 4, ragged lengths
    # (several splits for the long rows), fp32 / bf16 / fp16 queries against the float64
    # decode oracle, output and log-sum-exp.
    rs = np.random.RandomState(900 + 10 * vb + G)
    d, Hkv, Tc = 128, 8 if G == 4 else 2, 2112
    seq = [0, 1, 65, 700, 2100]
    B, Hq = len(seq), Hkv * G
    Rk, Rv = O.dense_qr_rotation(d, 42), O.dense_qr_rotation(d, 43)
    bk, ck = O.lloyd_max_codebook(4, d)
    bv, cv = O.lloyd_max_codebook(vb, d)
    n = B * Hkv * Tc
    K = rs.randn(n, d).astype(np.float32) * rs.uniform(0.2, 3.0, (n, 1)).astype(np.float32)
    V = rs.randn(n, d).astype(np.float32) * rs.uniform(0.2, 3.0, (n, 1)).astype(np.float32)
    K[:, rs.choice(d, 4, replace=False)] *= 20.0
    kp, kn, _ = O.quantize_mse(K, 4, Rk, bk)
    vp, vn, _ = O.quantize_mse(V, vb, Rv, bv)
    kc = k_pack_dl(kp.reshape(B * Hkv, Tc, -1), Tc, 0, 0, d=d)
    vc = k_pack_dl(vp.reshape(B * Hkv, Tc, -1), Tc, 0, 1, vbits=vb, d=d)
    kp, vp = kp.reshape(B, Hkv, Tc, -1), vp.reshape(B, Hkv, Tc, -1)
    kn, vn = kn.reshape(B, Hkv, Tc), vn.reshape(B, Hkv, Tc)
    q = (rs.randn(B, Hq, d) * 3.0).astype(np.float32)
    print(f"decode d=128 vb={vb} G={G}", flush=True)
    for dt, tol in ((torch.float32, 1e-4), (torch.bfloat16, 1e-2), (torch.float16, 3e-3)):
        qt = torch.from_numpy(q).to(DEV).to(dt)
        qf = qt.float().cpu().numpy()
        want, want_lse = O.decode_attention_f64(qf, kp, kn, vp, vn, seq, ck, cv, Rk, Rv, 4, vb,
                                                0.125, return_lse=True)
        got, lse = k_decode_dl(qt, kc, kn, vc, vn, seq, ck, cv, Rk, Rv, 0.125, vbits=vb)
        assert np.all(got[0] == 0) and np.isneginf(lse[0]).all()
        for bi in range(1, B):
            err = np.max(np.abs(got[bi] - want[bi])) / np.max(np.abs(want[bi]))
            assert err <= tol, (dt, seq[bi], err)
        ok = np.isfinite(want_lse)
        # the scores' rounding error follows the products q_j k_j, not the score (outlier
        # channels make them large where a score is near 0): the log-sum-exp is held to the
        # tolerance relative to its batch row's largest magnitude
        scale = np.maximum(1.0, np.max(np.where(ok, np.abs(want_lse), 0.0), axis=1, keepdims=True))
        lse_tol = 1e-2 if dt == torch.bfloat16 else 1e-5
        rel = np.abs(np.where(ok, lse - want_lse, 0.0)) / scale
        assert np.max(rel) <= lse_tol, (dt, np.max(rel))


@pytest.mark.parametrize("vb", [2, 3])
def test_decode_layout_d128_config_shape_vs_f64(vb):
    # B = 32, Hq = 32, Hkv = 8, head_dim 128, T = 1024 (one split per stream: the kernel
    # applies R_v and writes the output itself), bf16 queries and K/V with outlier channels
    rs = np.random.RandomState(17 + vb)
    B, Hq, Hkv, d, T_ = 32, 32, 8, 128, 1024
    Rk, Rv = O.dense_qr_rotation(d, 42), O.dense_qr_rotation(d, 43)
    bk, ck = O.lloyd_max_codebook(4, d)
    bv, cv = O.lloyd_max_codebook(vb, d)
    K = rs.randn(B, Hkv, T_, d).astype(np.float32)
    V = rs.randn(B, Hkv, T_, d).astype(np.float32)
    for h in range(Hkv):
        ch = rs.choice(d, 4, replace=False)
        K[:, h, :, ch] *= 20.0
        V[:, h, :, ch] *= 20.0
    K = torch.from_numpy(K).to(torch.bfloat16).float().numpy().reshape(-1, d)
    V = torch.from_numpy(V).to(torch.bfloat16).float().numpy().reshape(-1, d)
    kp, kn, _ = O.quantize_mse(K, 4, Rk, bk)
    vp, vn, _ = O.quantize_mse(V, vb, Rv, bv)
    kc = k_pack_dl(kp.reshape(B * Hkv, T_, -1), T_, 0, 0, d=d)
    vc = k_pack_dl(vp.reshape(B * Hkv, T_, -1), T_, 0, 1, vbits=vb, d=d)
    kp, vp = kp.reshape(B, Hkv, T_, -1), vp.reshape(B, Hkv, T_, -1)
    kn, vn = kn.reshape(B, Hkv, T_), vn.reshape(B, Hkv, T_)
    qt = torch.from_numpy(rs.randn(B, Hq, d).astype(np.float32)).to(DEV).to(torch.bfloat16)
    seq = [T_] * B
    want = O.decode_attention_f64(qt.float().cpu().numpy(), kp, kn, vp, vn, seq, ck, cv, Rk, Rv,
                                  4, vb, 0.125)
    got, _ = k_decode_dl(qt, kc, kn, vc, vn, seq, ck, cv, Rk, Rv, 0.125, vbits=vb)
    err = max(np.max(np.abs(got[b] - want[b])) / np.max(np.abs(want[b])) for b in range(B))
    assert err <= 1e-2, err


def test_scan_many_exact_ties_take_fallback():
    # 3000 identical rows tie exactly; more survivors than the merge's sort buffer, so
    # the exact k-round fallback must return the lowest ids among the tied rows.
    rs = np.random.RandomState(12)
    d, b = 128, 4
    R, cen, p, nm = _db(rs, 20000, d, b)
    best = int(np.argmax(O.lut_scores_f32(rs.randn(1, d).astype(np.float32), p, nm, cen, R, b)))
    q = rs.randn(2, d).astype(np.float32)
    top = int(np.argmax(O.lut_scores_f32(q[:1], p, nm, cen, R, b)))
    idx = rs.choice(20000, 3000, replace=False)
    p[idx] = p[top]
    nm[idx] = nm[top]
    s, i = k_scan(q, p, nm, cen, R, b, 16)
    so, io = O.search_topk(q, p, nm, cen, R, b, 16)
    assert np.array_equal(i, io)
    assert np.array_equal(s.view(np.uint32), so.view(np.uint32))


# ------------------------------------------------------------------ prod-mode scoring
def k_scan_prod(q, mp, sg, rn, nm, cen, R, S, bits, k, sg_offset_rows=0):
    """tq_ip_scan_topk_prod; sg_offset_rows > 0 passes the sign rows at that row offset
    of a larger buffer (a base that is not 16-byte aligned when bpp % 16 != 0)."""
    Q, d = q.shape
    N = mp.shape[0]
    os_ = torch.empty(Q, k, dtype=torch.float32, device=DEV)
    oi = torch.empty(Q, k, dtype=torch.int64, device=DEV)
    ws = torch.empty(max(L().tq_scan_workspace_bytes(Q, d, bits, N, k), 1), dtype=torch.uint8, device=DEV)
    sgt = T(np.concatenate([np.zeros((sg_offset_rows, sg.shape[1]), np.uint8), sg]))[sg_offset_rows:]
    capi.check(L().tq_ip_scan_topk_prod(capi.p(T(q)), capi.TQ_F32, capi.i64(Q), capi.i32(d),
                                        capi.p(T(mp)), capi.p(sgt), capi.p(T(rn)), capi.p(T(nm)),
                                        capi.i64(N), capi.p(T(cen)), capi.p(T(R)), capi.p(T(S)),
                                        capi.i32(bits), capi.i32(k), capi.p(os_), capi.p(oi),
                                        capi.p(ws), ctypes.c_size_t(ws.numel()), capi.stream()))
    sync()
    return os_.cpu().numpy(), oi.cpu().numpy()


def k_scores_prod(q, mp, sg, rn, nm, cen, R, S, bits):
    Q, d = q.shape
    N = mp.shape[0]
    out = torch.empty(Q, N, dtype=torch.float32, device=DEV)
    ws = torch.empty(max(L().tq_scan_workspace_bytes(Q, d, bits, N, 0), 1), dtype=torch.uint8, device=DEV)
    capi.check(L().tq_attention_scores_prod(capi.p(T(q)), capi.TQ_F32, capi.i64(Q), capi.i32(d),
                                            capi.p(T(mp)), capi.p(T(sg)), capi.p(T(rn)),
                                            capi.p(T(nm)), capi.i64(N), capi.p(T(cen)), capi.p(T(R)),
                                            capi.p(T(S)), capi.i32(bits), capi.p(out), capi.p(ws),
                                            ctypes.c_size_t(ws.numel()), capi.stream()))
    sync()
    return out.cpu().numpy()


def _prod_db(rs, n, d, b, seed=42):
    R, S = O.dense_qr_rotation(d, seed), O.qjl_matrix(d, d, seed + 12345)
    bnd, cen = O.lloyd_max_codebook(b - 1, d)
    x = (rs.randn(n, d) * rs.uniform(0.5, 2.0, (n, 1))).astype(np.float32)
    mp, sg, g, nm, _, _ = O.quantize_prod(x, b, R, bnd, cen, S)
    return R, S, cen, mp, sg, g, nm


def _prod_scale(q, nm, g):
    """|q| * n * (1 + 2 gamma): bounds the magnitudes summed in a prod score (the MSE term
    |<R q, c[codes]>| <= |q| |c[codes]| ~ |q|, the QJL term sqrt(pi/2)/d * gamma *
    sum_j |(S q)_j| <= ~1.3 gamma |q|), times the row norm."""
    return np.linalg.norm(q, axis=1)[:, None] * nm[None, :] * (1.0 + 2.0 * g[None, :])


def _prod_tol(q, nm, g):
    """fp32 sums of d terms (the rotations R q, S q and the two dot products) against
    float64: d * 2^-24 of the summed magnitude."""
    d = q.shape[1]
    return d * 2.0 ** -24 * _prod_scale(q, nm, g)


def _prod_err_units(got, ref, q, nm, g):
    """Largest |got - ref| in units of 2^-24 * the summed magnitude (d bounds it)."""
    return float(np.max(np.abs(got - ref) / (2.0 ** -24 * _prod_scale(q, nm, g))))


def _check_prod_topk(s, i, ref, tol, k):
    """Scores within tol of the float64 reference; ids equal the float64 top-k except
    where a swapped pair's float64 scores lie within the tolerance of each other."""
    so, io = O.topk_desc(ref, k)
    for qi in range(ref.shape[0]):
        n_valid = min(k, ref.shape[1])
        assert np.all(i[qi, n_valid:] == -1) and np.all(np.isneginf(s[qi, n_valid:]))
        ids = i[qi, :n_valid]
        assert len(set(ids.tolist())) == n_valid
        assert np.all(np.diff(s[qi, :n_valid]) <= 0)
        assert np.all(np.abs(s[qi, :n_valid] - ref[qi, ids]) <= tol[qi, ids])
        for r in range(n_valid):
            if ids[r] != io[qi, r]:
                a, bb = ids[r], io[qi, r]
                assert abs(ref[qi, a] - ref[qi, bb]) <= tol[qi, a] + tol[qi, bb], (qi, r)


@pytest.mark.parametrize("d", [64, 96, 128, 200])
@pytest.mark.parametrize("b", [2, 3, 4])
def test_prod_scan_topk_vs_f64(d, b):
    rs = np.random.RandomState(5 * d + b)
    R, S, cen, mp, sg, g, nm = _prod_db(rs, 12000, d, b)
    for Q, k in ((1, 10), (4, 1), (7, 32), (1, 100), (3, 128)):
        q = rs.randn(Q, d).astype(np.float32)
        s, i = k_scan_prod(q, mp, sg, g, nm, cen, R, S, b, k)
        ref = O.prod_scores_f64(q, mp, sg, g, nm, b, d, R, cen, S)
        _check_prod_topk(s, i, ref, _prod_tol(q, nm, g), k)


@pytest.mark.parametrize("d,b", [(64, 2), (96, 3), (128, 4), (200, 4)])
def test_prod_attention_scores_vs_f64(d, b):
    rs = np.random.RandomState(17 * d + b)
    R, S, cen, mp, sg, g, nm = _prod_db(rs, 3000, d, b, seed=43)
    for Q in (1, 3, 8):
        q = rs.randn(Q, d).astype(np.float32)
        got = k_scores_prod(q, mp, sg, g, nm, cen, R, S, b)
        ref = O.prod_scores_f64(q, mp, sg, g, nm, b, d, R, cen, S)
        print(f"prod scores d={d} b={b} Q={Q}: max error {_prod_err_units(got, ref, q, nm, g):.1f} "
              f"x 2^-24 of the summed magnitude (bound {d})")
        assert np.all(np.abs(got - ref) <= _prod_tol(q, nm, g)), (d, b, Q)


def test_prod_scan_reference_rows(golden):
    # The reference's own quantize_prod outputs (fixture) as the database (the d128 set
    # holds a zero vector at row 0).
    pr, rot, qj = golden("quant_prod"), golden("rotation"), golden("qjl")
    rs = np.random.RandomState(23)
    for name, d in (("d128", 128), ("d200", 200)):
        R, S = rot[f"R_d{d}_s42"], qj[f"S_d{d}_s42"]
        _, cen = O.lloyd_max_codebook(3, d)
        rows = [pr[f"{name}_{k}"] for k in ("mse_packed", "signs", "res_norms", "norms")]
        q = rs.randn(5, d).astype(np.float32)
        ref = O.prod_scores_f64(q, *rows, 4, d, R, cen, S)
        tol = _prod_tol(q, rows[3], rows[2])
        s, i = k_scan_prod(q, *rows, cen, R, S, 4, 10)
        _check_prod_topk(s, i, ref, tol, 10)
        got = k_scores_prod(q, *rows, cen, R, S, 4)
        assert np.all(np.abs(got - ref) <= tol)
        # zero rows score exactly 0
        zero = rows[3] == 0
        assert zero.sum() == (1 if d == 128 else 0) and np.all(got[:, zero] == 0)


def test_prod_scan_ties_padding_and_unaligned_signs():
    rs = np.random.RandomState(31)
    d, b = 64, 4
    R, S, cen, mp, sg, g, nm = _prod_db(rs, 5000, d, b)
    q = rs.randn(3, d).astype(np.float32)
    ref = O.prod_scores_f64(q, mp, sg, g, nm, b, d, R, cen, S)
    top = int(np.argmax(ref[0]))
    # 40 exact copies of the best row tie exactly: the lowest ids come first
    idx = np.sort(rs.choice(5000, 40, replace=False))
    for a in (mp, sg, g, nm):
        a[idx] = a[top]
    ref = O.prod_scores_f64(q, mp, sg, g, nm, b, d, R, cen, S)
    s, i = k_scan_prod(q, mp, sg, g, nm, cen, R, S, b, 16)
    tied = np.unique(np.concatenate([idx, [top]]))[:16]
    assert np.array_equal(i[0], tied)
    assert np.all(s[0] == s[0, 0])
    _check_prod_topk(s, i, ref, _prod_tol(q, nm, g), 16)
    # sign rows at an 8-byte offset (not 16-byte aligned): the generic loader, same results
    s2, i2 = k_scan_prod(q, mp, sg, g, nm, cen, R, S, b, 16, sg_offset_rows=1)
    assert np.array_equal(i2, i) and np.array_equal(s2.view(np.uint32), s.view(np.uint32))
    # k above N pads with (-inf, -1)
    s3, i3 = k_scan_prod(q, mp[:7], sg[:7], g[:7], nm[:7], cen, R, S, b, 12)
    _check_prod_topk(s3, i3, ref[:, :7], _prod_tol(q, nm[:7], g[:7]), 12)
    # empty key set: nothing to write
    assert k_scores_prod(q, mp[:0], sg[:0], g[:0], nm[:0], cen, R, S, b).shape == (3, 0)


def test_prod_scan_rejects_bad_bits():
    q = np.zeros((1, 64), np.float32)
    for bits in (1, 5):
        with pytest.raises(RuntimeError, match="bit_width"):
            k_scan_prod(q, np.zeros((4, 8 * max(bits - 1, 1)), np.uint8), np.zeros((4, 8), np.uint8),
                        np.ones(4, np.float32), np.ones(4, np.float32), np.zeros(2, np.float32),
                        np.eye(64, dtype=np.float32), np.eye(64, dtype=np.float32), bits, 4)


@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("dt", ["bf16", "f16"])
def test_quantize_few_rows_equals_tiled_kernel(d, dt):
    """A call of at most 16384 bf16/fp16 rows of d 64/128 (a decode step's append) runs one
    wave per row; its codes and norms equal the tiled kernel's -- the same rows inside a
    call of 20,000 rows -- bit for bit, and the oracle's outside the decision band."""
    g = torch.Generator(device=DEV).manual_seed(d)
    x = torch.randn(20000, d, generator=g, device=DEV) * 3
    x[5] = 0.0
    tdt = torch.bfloat16 if dt == "bf16" else torch.float16
    cdt = capi.TQ_BF16 if dt == "bf16" else capi.TQ_F16
    xt = x.to(tdt).contiguous()
    R = O.dense_qr_rotation(d, 42)
    for bits in (1, 2, 3, 4):
        bnd, _ = O.lloyd_max_codebook(bits, d)
        big_p, big_n = k_quantize(xt, R, bnd, bits, cdt, cdt)
        for n in (1, 37, 512):
            p, nm = k_quantize(xt[:n].contiguous(), R, bnd, bits, cdt, cdt)
            assert np.array_equal(p, big_p[:n]), (bits, n)
            assert np.array_equal(nm.view(np.uint32), big_n[:n].view(np.uint32)), (bits, n)
        # against the oracle: identical outside the decision band (inside it the reduced-
        # precision sums flip often -- the tiled kernel these equal is the one pinned to
        # reference.py's own bf16 codes by the golden test above)
        xf = xt[:512].float().cpu().numpy()
        O.check_codes(O.unpack_codes(p, bits, d), O.quantize_mse(xf, bits, R, bnd, dt)[2], xf, R,
                      bnd, dt, max_rate=1.0)


@pytest.mark.parametrize("d,b", [(128, 4), (64, 4), (128, 3), (64, 3)])
def test_prod_pair_rows_equal_bitplane_prod_scan(d, b):
    """Prod scoring with the MSE half as pair rows is the bit-plane prod scan bit for bit:
    top-k ids and scores (one query and several), and every score of the all-rows op."""
    from turboquant_kv._lib import ops
    g = torch.Generator(device=DEV).manual_seed(d + b)
    N = 70_001
    x = torch.randn(N, d, generator=g, device=DEV)
    x[7] = 0.0
    R = T(O.dense_qr_rotation(d, 42))
    bnd, cen = O.lloyd_max_codebook(b - 1, d)
    S = T(O.qjl_matrix(d, d, 42))
    mp, sg, rn, nm = ops().quantize_prod_packed(x, R, T(bnd), T(cen), S, b)
    rows = ops().pack_pair_rows(mp, b - 1, d)
    for Q in (1, 5):
        q = torch.randn(Q, d, generator=g, device=DEV).half()
        for k in (10, 100):
            s0, i0 = ops().ip_scan_topk_prod(q, mp, sg, rn, nm, T(cen), R, S, b, k)
            s1, i1 = ops().ip_scan_topk_prod_pair_rows(q, rows, sg, rn, nm, T(cen), R, S, b, k)
            assert torch.equal(i0, i1), (Q, k)
            assert torch.equal(s0.view(torch.int32), s1.view(torch.int32)), (Q, k)
    qa = torch.randn(2, 3, d, generator=g, device=DEV)
    a0 = ops().attention_scores_prod(qa, mp[:5000], sg[:5000], rn[:5000], nm[:5000], T(cen), R, S, b)
    a1 = ops().attention_scores_prod_pair_rows(qa, rows[:5000], sg[:5000], rn[:5000], nm[:5000],
                                               T(cen), R, S, b)
    assert torch.equal(a0.view(torch.int32), a1.view(torch.int32))


@pytest.mark.parametrize("bits,d", [(3, 128), (3, 64), (2, 128), (2, 64)])
def test_pair_rows_one_query_filter_cases(bits, d):
    """One query over 2-/3-bit pair rows: ids and scores equal the oracle's bit for bit on
    ragged N, fp16 unit queries, duplicated best rows (exact ties), special norms (zero,
    negative, huge, tiny, infinite: NaN rows are never listed) and zero / huge / tiny
    query scales."""
    rs = np.random.RandomState(300 + 10 * bits + d)
    N = 130_001
    R, cen, p, nm = _db(rs, N, d, bits)
    nm = nm.copy()
    # ties: 500 copies of the best row for a fixed query
    q0 = rs.randn(1, d).astype(np.float32)
    top = int(np.argmax(O.lut_scores_f32(q0, p, nm, cen, R, bits)))
    idx = rs.permutation(N)
    p[idx[:500]] = p[top]
    nm[idx[:500]] = nm[top]
    nm[idx[500:1500]] = 0.0
    nm[idx[1500:2500]] *= -1.0
    nm[idx[2500:2510]] = 1e30
    nm[idx[2510:2520]] = 1e-38
    nm[idx[2520:2526]] = np.inf
    nm[idx[2526:2530]] = -np.inf
    rows = k_pair_rows(p, d, bits)
    qn = rs.randn(1, d).astype(np.float32)
    qn /= np.linalg.norm(qn)
    cases = [(q0, capi.TQ_F32), (qn.astype(np.float16), capi.TQ_F16)]
    cases += [((rs.randn(1, d) * sc).astype(np.float32), capi.TQ_F32) for sc in (0.0, 1e-36, 1e34)]
    for q, qdt in cases:
        qf = q.astype(np.float32)
        want = O.lut_scores_f32(qf, p, nm, cen, R, bits)
        for k in (1, 10, 32):
            s, i = k_scan_pair_rows(q, rows, nm, cen, R, bits, k, q_dt=qdt)
            so, io = _topk_no_nan(want, k)
            assert np.array_equal(i, io), (k, qdt)
            assert np.array_equal(s.view(np.uint32), so.view(np.uint32)), (k, qdt)
