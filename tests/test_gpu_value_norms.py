"""GPU tests of the attention kernels at value norms far outside fp16's range.

The decode and prefill kernels hand the weights p |v| to the matrix cores as fp16; a
per-wave power-of-two scale keeps them inside fp16's range whatever the norms' fp32
magnitude.  Two checks, through every kernel that forms such weights (the decode-layout
kernel at head_dim 64 and 128 with one and two streams per workgroup and split and unsplit
sequences, the bit-plane fused decode kernel, the paged decode-layout kernel and the paged
prefill kernel):

* scaling: attention is linear in the value norms, and every step of these kernels commutes
  with a power-of-two scale, so norms times 2^k give outputs exactly 2^k times the unscaled
  ones, bit for bit, for k from -100 to 100 (unscaled fp16 weights underflow or overflow
  long before);
* mixed magnitudes: norms spread over 10^-4 .. 10^5 at random per token, or ramped from
  10^-4 to 10^6 along the sequence (the scale moves in the middle of a stream), against
  the float64 oracle, each batch row relative to its own largest output.

Queries are fp32 or bf16 (outputs of fp16 queries are fp16, whose range bounds the outputs
themselves)."""

import ctypes

import numpy as np
import pytest
import torch

import capi
import tq_oracle as O
from test_gpu_capi import T, k_decode, k_decode_dl, k_pack_dl, sync
from test_gpu_paged import _dl_pools

pytestmark = pytest.mark.gpu
DEV = "cuda"
L = capi.lib
_DT = {torch.float32: capi.TQ_F32, torch.bfloat16: capi.TQ_BF16, torch.float16: capi.TQ_F16}
SHIFTS = [-100, -40, 24, 100]
# fp32 queries: fp16 hi + lo parts of every operand (about 1e-6 relative); bf16 queries:
# one fp16 product per term
QDT = [(torch.float32, 2e-5), (torch.bfloat16, 1e-2)]


def _vmul(profile, pos, rs):
    """Multiplier of each token's value norm by its position."""
    pos = np.asarray(pos)
    if profile == "mixed":
        return 10.0 ** rs.uniform(-4.0, 5.0, pos.shape)
    return 10.0 ** (-4.0 + 10.0 * pos / 2100.0)  # ramp


def _check_scaled(base, got, k, what):
    assert np.all(np.isfinite(got)), what
    want = np.ldexp(base.astype(np.float64), k).astype(np.float32)
    assert np.array_equal(got, want), (what, np.max(np.abs(got - want)))


def _check_rows(got, want, tol, what):
    """Every batch row within tol of the float64 row, relative to the row's largest |x|;
    rows of empty sequences are exactly 0."""
    assert np.all(np.isfinite(got)), what
    g, w = got.reshape(got.shape[0], -1), want.reshape(want.shape[0], -1)
    num, den = np.abs(g - w).max(axis=1), np.abs(w).max(axis=1)
    live = den > 0
    assert np.all(g[~live] == 0), what
    err = np.max(num[live] / den[live])
    assert err <= tol, (what, err)


def _dl_case(rs, d, vb, B, Hkv, G, Tc):
    Rk, Rv = O.dense_qr_rotation(d, 42), O.dense_qr_rotation(d, 43)
    bk, ck = O.lloyd_max_codebook(4, d)
    bv, cv = O.lloyd_max_codebook(vb, d)
    n = B * Hkv * Tc
    kp, kn, _ = O.quantize_mse(rs.randn(n, d).astype(np.float32), 4, Rk, bk)
    vp, vn, _ = O.quantize_mse(rs.randn(n, d).astype(np.float32), vb, Rv, bv)
    kc = k_pack_dl(kp.reshape(B * Hkv, Tc, -1), Tc, 0, 0, d=d)
    vc = k_pack_dl(vp.reshape(B * Hkv, Tc, -1), Tc, 0, 1, vbits=vb, d=d)
    return (kc, vc, kp.reshape(B, Hkv, Tc, -1), kn.reshape(B, Hkv, Tc), vp.reshape(B, Hkv, Tc, -1),
            vn.reshape(B, Hkv, Tc), ck, cv, Rk, Rv, rs.randn(B, Hkv * G, d).astype(np.float32))


# 8 streams: several splits per long sequence (partials through the combine kernel);
# 516 streams: two streams per workgroup, one split each
DL_CASES = {"d64": (64, 3, [0, 37, 700, 2100], 2, 4, 2112),
            "d128": (128, 2, [0, 37, 700, 2100], 2, 4, 2112),
            "d64x516": (64, 2, None, 2, 4, 192)}


def _dl_setup(case, seed):
    d, vb, seq, Hkv, G, Tc = DL_CASES[case]
    rs = np.random.RandomState(seed)
    if seq is None:
        seq = list(rs.randint(0, 190, 258))
        seq[3] = 0
    return rs, d, vb, seq, _dl_case(rs, d, vb, len(seq), Hkv, G, Tc)


@pytest.mark.parametrize("case", list(DL_CASES))
def test_decode_layout_value_norm_scaling(case):
    rs, d, vb, seq, (kc, vc, kp, kn, vp, vn, ck, cv, Rk, Rv, q) = _dl_setup(case, 5 + len(case))
    print(f"decode layout value-norm scaling {case}", flush=True)
    for dt, tol in QDT:
        qt = torch.from_numpy(q).to(DEV).to(dt)
        base, base_lse = k_decode_dl(qt, kc, kn, vc, vn, seq, ck, cv, Rk, Rv, 0.125, vbits=vb)
        want = O.decode_attention_f64(qt.float().cpu().numpy(), kp, kn, vp, vn, seq, ck, cv, Rk, Rv,
                                      4, vb, 0.125)
        _check_rows(base, want, tol, (case, dt))
        for k in SHIFTS:
            got, lse = k_decode_dl(qt, kc, kn, vc, np.ldexp(vn, k), seq, ck, cv, Rk, Rv, 0.125, vbits=vb)
            _check_scaled(base, got, k, (case, dt, k))
            assert np.array_equal(lse, base_lse)


@pytest.mark.parametrize("case", list(DL_CASES))
@pytest.mark.parametrize("profile", ["mixed", "ramp"])
def test_decode_layout_value_norm_mixed(case, profile):
    rs, d, vb, seq, (kc, vc, kp, kn, vp, vn, ck, cv, Rk, Rv, q) = _dl_setup(case, 9 + len(case))
    Tc = kn.shape[2]
    # the ramp spans 10^-4 .. 10^6 over the longest sequence
    vn = (vn * _vmul(profile, np.arange(Tc) * (2100.0 / max(seq)), rs)).astype(np.float32)
    print(f"decode layout value norms {case} {profile}", flush=True)
    for dt, tol in QDT:
        qt = torch.from_numpy(q).to(DEV).to(dt)
        want = O.decode_attention_f64(qt.float().cpu().numpy(), kp, kn, vp, vn, seq, ck, cv, Rk, Rv,
                                      4, vb, 0.125)
        got, _ = k_decode_dl(qt, kc, kn, vc, vn, seq, ck, cv, Rk, Rv, 0.125, vbits=vb)
        _check_rows(got, want, tol, (case, profile, dt))


def test_fused_decode_value_norms():
    # bit-plane caches, head_dim 64: bf16 queries take the fused MFMA kernel, fp32 queries
    # the split scan path
    rs = np.random.RandomState(21)
    d, kb, vb, Hkv, G, Tm = 64, 4, 2, 2, 4, 2600
    seq = [0, 37, 700, 2600]
    B, Hq = len(seq), Hkv * G
    Rk, Rv = O.dense_qr_rotation(d, 42), O.dense_qr_rotation(d, 43)
    bk, ck = O.lloyd_max_codebook(kb, d)
    bv, cv = O.lloyd_max_codebook(vb, d)
    n = B * Hkv * Tm
    kp, kn, _ = O.quantize_mse(rs.randn(n, d).astype(np.float32), kb, Rk, bk)
    vp, vn, _ = O.quantize_mse(rs.randn(n, d).astype(np.float32), vb, Rv, bv)
    kp, vp = kp.reshape(B, Hkv, Tm, -1), vp.reshape(B, Hkv, Tm, -1)
    kn, vn = kn.reshape(B, Hkv, Tm), vn.reshape(B, Hkv, Tm)
    q = rs.randn(B, Hq, d).astype(np.float32)
    print("fused decode value norms", flush=True)
    for dt, tol in QDT:
        qt = torch.from_numpy(q).to(DEV).to(dt)
        qf = qt.float().cpu().numpy()
        base, _ = k_decode(qt, kp, kn, vp, vn, seq, ck, cv, Rk, Rv, kb, vb, 0.125)
        for k in SHIFTS:
            got, _ = k_decode(qt, kp, kn, vp, np.ldexp(vn, k), seq, ck, cv, Rk, Rv, kb, vb, 0.125)
            _check_scaled(base, got, k, ("fused", dt, k))
        for profile in ("mixed", "ramp"):
            vm = (vn * _vmul(profile, np.arange(Tm), rs)).astype(np.float32)
            want = O.decode_attention_f64(qf, kp, kn, vp, vm, seq, ck, cv, Rk, Rv, kb, vb, 0.125)
            got, _ = k_decode(qt, kp, kn, vp, vm, seq, ck, cv, Rk, Rv, kb, vb, 0.125)
            _check_rows(got, want, tol, ("fused", profile, dt))


def _paged_run(pools, lens, bs, vb, nb, width, Hkv, q, qp, Tq, ck, cv, Rk, Rv):
    """(paged decode outputs, prefill outputs of sequence 1's last positions)"""
    tab, kp, knp, vt, vnp = pools
    B, Hq, _ = q.shape
    n = qp.shape[0]
    Tc = width * bs
    out = torch.empty_like(q)
    lse = torch.empty(B, Hq, dtype=torch.float32, device=DEV)
    ws = torch.empty(L().tq_decode_dl_workspace_bytes(B, Hq, Hkv, Tc), dtype=torch.uint8, device=DEV)
    capi.check(L().tq_decode_attention_paged_dl(
        capi.p(q), _DT[q.dtype], capi.i32(B), capi.i32(Hq), capi.i32(Hkv), capi.i32(64), capi.p(kp),
        capi.p(knp), capi.p(vt), capi.p(vnp), capi.i64(nb), capi.i32(bs), capi.i32(vb), capi.p(T(tab)),
        capi.i32(width), capi.p(T(np.asarray(lens, np.int32))), capi.p(T(ck)), capi.p(T(cv)),
        capi.p(T(Rk)), capi.p(T(Rv)), ctypes.c_float(0.125), capi.p(out), capi.p(lse), capi.p(ws),
        ctypes.c_size_t(ws.numel()), capi.stream()))
    outp = torch.empty(n, Hq, 64, dtype=torch.float32, device=DEV)
    capi.check(L().tq_prefill_attention_paged_dl(
        capi.p(qp), _DT[qp.dtype], capi.i32(n), capi.i64(Tq), capi.i32(Hq), capi.i32(Hkv), capi.i32(64),
        capi.p(kp), capi.p(knp), capi.p(vt), capi.p(vnp), capi.i64(nb), capi.i32(bs), capi.i32(vb),
        capi.p(T(tab[1])), capi.i32(width), capi.p(T(ck)), capi.p(T(cv)), capi.p(T(Rk)), capi.p(T(Rv)),
        ctypes.c_float(0.125), capi.p(outp), capi.stream()))
    sync()
    return out.float().cpu().numpy(), outp.cpu().numpy()


@pytest.mark.parametrize("bs,vb", [(16, 2), (64, 3)])
def test_paged_decode_and_prefill_value_norms(bs, vb):
    # paged decode-layout pools (16-token sub-blocks at block size 16, 64-token tiles at
    # 64): the decode kernel over three sequences and the prefill kernel over the long
    # sequence's last 100 positions
    rs = np.random.RandomState(31 * bs + vb)
    Hkv, G = 2, 4
    Hq = Hkv * G
    lens = [37, 2100, 700]
    B, n, Tq = len(lens), 100, lens[1]
    width = (max(lens) + bs - 1) // bs + 1
    nb = sum((n_ + bs - 1) // bs for n_ in lens) + 4
    Rk, Rv = O.dense_qr_rotation(64, 42), O.dense_qr_rotation(64, 43)
    _, ck = O.lloyd_max_codebook(4, 64)
    _, cv = O.lloyd_max_codebook(vb, 64)
    Tc = width * bs
    print(f"paged decode + prefill value norms bs={bs} vb={vb}", flush=True)
    for profile in (None, "mixed", "ramp"):
        prs = np.random.RandomState(7)  # the same pools for every profile
        vmul = None if profile is None else (lambda pos: _vmul(profile, pos, rs))
        tab, kp, knp, vt, vnp, seqs = _dl_pools(prs, lens, bs, nb, width, Hkv, vb, vmul=vmul)
        pools = (tab, kp, knp, vt, vnp)
        kc_ = np.zeros((B, Hkv, Tc, 32), np.uint8)
        vc_ = np.zeros((B, Hkv, Tc, 8 * vb), np.uint8)
        kn_, vn_ = np.zeros((B, Hkv, Tc), np.float32), np.zeros((B, Hkv, Tc), np.float32)
        for b, n_ in enumerate(lens):
            kc_[b, :, :n_], kn_[b, :, :n_], vc_[b, :, :n_], vn_[b, :, :n_] = seqs[b]
        kr, knr, vr, vnr = seqs[1]
        bc = lambda x: np.broadcast_to(x[None], (n,) + x.shape)
        pos = np.arange(Tq - n + 1, Tq + 1)
        for dt, tol in QDT:
            q = torch.from_numpy(rs.randn(B, Hq, 64).astype(np.float32)).to(DEV).to(dt)
            qp = torch.from_numpy(rs.randn(n, Hq, 64).astype(np.float32)).to(DEV).to(dt)
            got, gotp = _paged_run(pools, lens, bs, vb, nb, width, Hkv, q, qp, Tq, ck, cv, Rk, Rv)
            want = O.decode_attention_f64(q.float().cpu().numpy(), kc_, kn_, vc_, vn_, lens, ck, cv, Rk,
                                          Rv, 4, vb, 0.125)
            wantp = O.decode_attention_f64(qp.float().cpu().numpy(), bc(kr), bc(knr), bc(vr), bc(vnr), pos,
                                           ck, cv, Rk, Rv, 4, vb, 0.125)
            _check_rows(got, want, tol, ("paged decode", profile, dt))
            _check_rows(gotp, wantp, 5e-3 if dt == torch.bfloat16 else tol, ("prefill", profile, dt))
            if profile is not None:
                continue
            for k in SHIFTS:
                vk = vnp.clone()
                vk.mul_(2.0 ** k)
                g2, g2p = _paged_run((tab, kp, knp, vt, vk), lens, bs, vb, nb, width, Hkv, q, qp, Tq, ck, cv,
                                     Rk, Rv)
                _check_scaled(got, g2, k, ("paged decode", dt, k))
                _check_scaled(gotp, g2p, k, ("prefill", dt, k))
