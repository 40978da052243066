"""CPU oracle for turboquant-kv's quantize-and-score path.

TEST INFRASTRUCTURE ONLY.  Imported by tests/, by __graft_entry__.smoke() and by
bench.py's cpu_baseline leg, always as the checker.  The product package
(turboquant-kv_amd/turboquant_kv) never imports it.

A numpy restatement of the reference algorithm, each function citing the
reference file:line it follows (paths relative to the reference checkout).
Floating-point behaviour is stated per function:

* codebook / rotation / QJL matrix: same arithmetic as the reference
  (scipy normal cdf/pdf; numpy RandomState + LAPACK QR; torch CPU generator).
  Pinned by tests/golden/{codebook,rotation,qjl}.npz.
* quantize (fp32): numpy float32 arithmetic.  The reference's GEMM summation
  order is its BLAS's, so codes can differ only where the rotated coordinate
  lies within the fp32 error band of a boundary; `code_margin` measures that
  band in float64 and tests require exact equality outside it.
* quantize (bf16/fp16 inputs): every rounding point of reference.py emulated
  (norm, division, GEMM output, boundaries).  Pinned by quant_mse.npz bf16 cases.
* scores / search: the LUT form of csrc/core/turboquant_core.cpp:407-514 in exact
  float32 (sequential j, one rounding per add), so scores are bit-reproducible;
  float64 closed forms are given for tolerance checks.
* prod scores / search: float64 closed form of search.py:229-252 (q @ dequantize_prod^T);
  pinned by the reference's dequantize_prod output in quant_prod.npz.
* decode attention: float64 closed form of cache.py:282-339 + softmax, with GQA.
"""

from __future__ import annotations

import math

import numpy as np

# ----------------------------------------------------------------- rounding helpers


def round_bf16(x):
    """float32 -> nearest bf16 (ties to even), returned as float32."""
    a = np.asarray(x, dtype=np.float32)
    u = a.view(np.uint32).astype(np.uint64)
    nan = np.isnan(a)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    out = u.astype(np.uint32).view(np.float32)
    return np.where(nan, a, out).astype(np.float32)


def round_f16(x):
    return np.asarray(x, dtype=np.float32).astype(np.float16).astype(np.float32)


def round_to(x, dtype: str):
    if dtype == "bf16":
        return round_bf16(x)
    if dtype == "f16":
        return round_f16(x)
    return np.asarray(x, dtype=np.float32)


def bf16_bits_to_f32(u16):
    return (np.asarray(u16, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


# ----------------------------------------------------------------- codebook


def lloyd_max_unscaled(bits: int, max_iter: int = 200, tol: float = 1e-12):
    """Lloyd-Max for N(0,1) (reference.py:26-54): centroids start at linspace(-3, 3),
    at most `max_iter` updates, stop when the largest centroid move is below `tol`
    (the loop leaves before adopting that last update), boundaries = midpoints."""
    from scipy.stats import norm

    L = 1 << bits
    c = np.linspace(-3.0, 3.0, L)
    for _ in range(max_iter):
        b = (c[:-1] + c[1:]) / 2.0
        e = np.concatenate([[-np.inf], b, [np.inf]])
        nc = np.zeros(L, dtype=np.float64)
        for i in range(L):
            lo, hi = e[i], e[i + 1]
            p = norm.cdf(hi) - norm.cdf(lo)
            nc[i] = c[i] if p < 1e-15 else (norm.pdf(lo) - norm.pdf(hi)) / p
        if np.max(np.abs(nc - c)) < tol:
            break
        c = nc
    return (c[:-1] + c[1:]) / 2.0, c


def lloyd_max_codebook(bits: int, dim: int):
    """Scaled by 1/sqrt(dim) in float64, then float32 (reference.py:57-73)."""
    b, c = lloyd_max_unscaled(bits)
    s = 1.0 / math.sqrt(dim)
    return (b * s).astype(np.float32), (c * s).astype(np.float32)


# ----------------------------------------------------------------- rotations


def dense_qr_rotation(dim: int, seed: int = 42) -> np.ndarray:
    """reference.py:100-109: RandomState(seed).randn(d, d) as float32, LAPACK QR,
    columns multiplied by sign(diag(R)) (zeros -> +1)."""
    g = np.random.RandomState(seed).randn(dim, dim).astype(np.float32)
    q, r = np.linalg.qr(g)
    s = np.sign(np.diag(r))
    s[s == 0] = 1.0
    return (q * s[None, :]).astype(np.float32)


def qjl_matrix(dim: int, n_sign_bits: int, seed: int) -> np.ndarray:
    """reference.py:375-389: torch CPU generator seeded with seed + 12345, randn."""
    import torch

    g = torch.Generator(device="cpu").manual_seed(seed + 12345)
    return torch.randn(n_sign_bits, dim, generator=g, dtype=torch.float32).numpy()


# ----------------------------------------------------------------- packing


def pack_codes(codes: np.ndarray, bits: int) -> np.ndarray:
    """reference.py:191-224: planes of ceil(d/8) bytes, plane i = bit i, dim j at
    bit 7-(j&7) of byte j>>3, pad bits zero."""
    codes = np.asarray(codes, dtype=np.uint8)
    n, d = codes.shape
    bpp = (d + 7) // 8
    out = np.zeros((n, bits * bpp), dtype=np.uint8)
    for i in range(bits):
        plane = ((codes >> i) & 1).astype(np.uint8)
        padded = np.zeros((n, bpp * 8), dtype=np.uint8)
        padded[:, :d] = plane
        out[:, i * bpp:(i + 1) * bpp] = np.packbits(padded, axis=1, bitorder="big")
    return out


def unpack_codes(packed: np.ndarray, bits: int, dim: int) -> np.ndarray:
    """reference.py:227-255."""
    packed = np.asarray(packed, dtype=np.uint8)
    bpp = (dim + 7) // 8
    codes = np.zeros((packed.shape[0], dim), dtype=np.uint8)
    for i in range(bits):
        plane = np.unpackbits(packed[:, i * bpp:(i + 1) * bpp], axis=1, bitorder="big")[:, :dim]
        codes |= (plane << i).astype(np.uint8)
    return codes


# ----------------------------------------------------------------- quantize


def _rowdot(u, M):
    """u @ M.T in float64 (u, M given in float32)."""
    return np.asarray(u, np.float64) @ np.asarray(M, np.float64).T


def quantize_mse(x, bits, R, bnd, dtype: str = "f32"):
    """reference.py:263-317 for x of `dtype` ('f32', 'bf16', 'f16' given as float32
    values).  Returns (packed u8, norms float32, codes u8)."""
    x = np.asarray(x, dtype=np.float32)
    if dtype == "f32":
        n = np.sqrt(np.sum(x.astype(np.float32) ** 2, axis=-1, dtype=np.float32)).astype(np.float32)
        u = (x / np.maximum(n, np.float32(1e-10))[:, None]).astype(np.float32)
        y = (u @ np.asarray(R, np.float32).T).astype(np.float32)
        codes = np.searchsorted(np.asarray(bnd, np.float32), y, side="left").astype(np.uint8)
    else:
        n = round_to(np.sqrt(np.sum(x.astype(np.float64) ** 2, axis=-1)).astype(np.float32), dtype)
        eps = round_to(np.float32(1e-10), dtype)
        u = round_to(x / np.maximum(n, eps)[:, None], dtype)
        Rr = round_to(R, dtype)
        y = round_to(_rowdot(u, Rr).astype(np.float32), dtype)
        codes = np.searchsorted(round_to(bnd, dtype), y, side="left").astype(np.uint8)
    return pack_codes(codes, bits), n, codes


def code_margin(x, R, bnd, dtype: str = "f32", rel: float | None = None):
    """Per-coordinate ambiguity flags for quantize_mse.

    Returns a bool array [n, d]: True where the reference's own fp32 arithmetic
    (any summation order, norm off by an ulp) could land on either side of a
    decision point, so the code is not fixed by the algorithm.  For fp32 inputs
    the decision points are the boundaries; for bf16/fp16 inputs they are also
    the rounding midpoints of the GEMM output and of the norm.
    """
    x = np.asarray(x, dtype=np.float32)
    bnd = np.asarray(bnd, np.float32)
    if rel is None:
        rel = 2.0 ** -20 if dtype == "f32" else 2.0 ** -21
    if dtype == "f32":
        # rel * sum_k |u_k R_jk| covers two fp32 dot products of d terms summed in
        # different orders (each about sqrt(d) * 2^-25 of that sum, 2^-21.5 at d = 128);
        # 2^-22 |y| covers the norm and the division landing an ulp or two apart.
        n = np.sqrt(np.sum(x.astype(np.float64) ** 2, axis=-1))
        u = x / np.maximum(n, 1e-10)[:, None]
        y = _rowdot(u, R)
        band = rel * (np.abs(u) @ np.abs(np.asarray(R, np.float64)).T) + 2.0 ** -22 * np.abs(y)
        d = np.min(np.abs(y[..., None] - bnd.astype(np.float64)), axis=-1)
        return d <= band
    n32 = np.sqrt(np.sum(x.astype(np.float64) ** 2, axis=-1))
    lo = round_to((n32 * (1 - 2.0 ** -20)).astype(np.float32), dtype)
    hi = round_to((n32 * (1 + 2.0 ** -20)).astype(np.float32), dtype)
    row_amb = lo != hi
    n = round_to(n32.astype(np.float32), dtype)
    eps = round_to(np.float32(1e-10), dtype)
    u = round_to(x / np.maximum(n, eps)[:, None], dtype)
    Rr = round_to(R, dtype)
    y = _rowdot(u, Rr)
    band = rel * (np.abs(u).astype(np.float64) @ np.abs(Rr.astype(np.float64)).T)
    amb = round_to((y - band).astype(np.float32), dtype) != round_to((y + band).astype(np.float32), dtype)
    return amb | row_amb[:, None]


def boundary_distance(x, R, bnd):
    """Per coordinate, the float64 distance of y = (x/|x|) R^T from its nearest decision
    boundary in units of sum_k |u_k R_jk| -- the scale of fp32 dot-product rounding, so
    a code two fp32 computations disagree on has a small value here."""
    x = np.asarray(x, dtype=np.float32)
    n = np.sqrt(np.sum(x.astype(np.float64) ** 2, axis=-1))
    u = x / np.maximum(n, 1e-10)[:, None]
    y = _rowdot(u, R)
    scale = np.abs(u) @ np.abs(np.asarray(R, np.float64)).T
    d = np.min(np.abs(y[..., None] - np.asarray(bnd, np.float64)), axis=-1)
    return d / np.maximum(scale, 1e-300)


def check_codes(got, want, x, R, bnd, dtype: str = "f32", max_rate: float = 2e-5):
    """Parity of quantize codes (the summation-order policy): codes outside the ambiguity
    band must be identical; inside it they may differ, but no more often than `max_rate`
    per coordinate (about 10x the flip rate two fp32 summation orders give near the
    boundaries, ~1-2e-6).  Returns a summary dict; raises AssertionError otherwise."""
    amb = code_margin(x, R, bnd, dtype)
    diff = np.asarray(got) != np.asarray(want)
    outside = diff & ~amb
    info = {"coords": int(diff.size), "band": int(amb.sum()), "mismatches": int(diff.sum()),
            "outside_band": int(outside.sum())}
    if dtype == "f32" and diff.any():
        info["max_mismatch_distance"] = float(boundary_distance(x, R, bnd)[diff].max())
    assert not outside.any(), ("codes differ outside the ambiguity band", info,
                               np.argwhere(outside)[:5])
    assert info["mismatches"] <= max(2, max_rate * diff.size), ("too many in-band flips", info)
    return info


def dequantize_mse(packed, norms, bits, dim, R, cen, dtype: str = "f32"):
    """reference.py:320-367: (c[codes] @ R) * n, in `dtype` rounding."""
    codes = unpack_codes(packed, bits, dim)
    c = round_to(cen, dtype)[codes]
    rec = round_to(_rowdot(c, round_to(np.asarray(R, np.float32).T, dtype)).astype(np.float32), dtype)
    return round_to(rec * np.asarray(norms, np.float32)[:, None], dtype)


def quantize_prod(x, bits, R, bnd, cen, S):
    """reference.py:392-469 (fp32): n, u = x/max(n,1e-10); MSE at bits-1 on u (which
    normalizes again, reference.py:441 -> 294-295); r = u - c[codes] R;
    gamma = ||r||; signs = (r S^T >= 0).  Returns (mse_packed, signs_packed,
    gamma, n, codes, proj64) -- proj64 is r S^T in float64 for margin checks."""
    x = np.asarray(x, dtype=np.float32)
    n = np.sqrt(np.sum(x ** 2, axis=-1, dtype=np.float32)).astype(np.float32)
    u = (x / np.maximum(n, np.float32(1e-10))[:, None]).astype(np.float32)
    mp, _, codes = quantize_mse(u, bits - 1, R, bnd)
    rec = (np.asarray(cen, np.float32)[codes] @ np.asarray(R, np.float32)).astype(np.float32)
    r = (u - rec).astype(np.float32)
    g = np.sqrt(np.sum(r ** 2, axis=-1, dtype=np.float32)).astype(np.float32)
    proj = (r @ np.asarray(S, np.float32).T).astype(np.float32)
    signs = (proj >= 0).astype(np.uint8)
    proj64 = _rowdot(r, S)
    return mp, pack_codes(signs, 1), g, n, codes, proj64


def dequantize_prod(mse_packed, signs_packed, gamma, norms, bits, dim, R, cen, S):
    """reference.py:472-533 in float64: (c[codes] R + sqrt(pi/2)/d * gamma * (s S)) * n."""
    codes = unpack_codes(mse_packed, bits - 1, dim)
    rec = np.asarray(cen, np.float64)[codes] @ np.asarray(R, np.float64)
    s = 2.0 * unpack_codes(signs_packed, 1, dim).astype(np.float64) - 1.0
    corr = math.sqrt(math.pi / 2.0) / dim * np.asarray(gamma, np.float64)[:, None] * (s @ np.asarray(S, np.float64))
    return (rec + corr) * np.asarray(norms, np.float64)[:, None]


# ----------------------------------------------------------------- scoring


def rotate_queries_f32(q, R):
    """q_rot[j] = sum_k q[k] * R[j][k], float32, k ascending, separate multiply and
    add roundings (csrc/core/turboquant_core.cpp:429-437)."""
    q = np.asarray(q, np.float32)
    R = np.asarray(R, np.float32)
    acc = np.zeros((q.shape[0], R.shape[0]), dtype=np.float32)
    for k in range(R.shape[1]):
        acc = (acc + (q[:, k:k + 1] * R[None, :, k]).astype(np.float32)).astype(np.float32)
    return acc


def lut_scores_f32(q, packed, norms, cen, R, bits):
    """scores[q, i] = norms[i] * sum_j LUT[j][code_ij] in exact float32 with j ascending
    (core.cpp:440-483; triton_kernels.py:264-310).  Returns float32 [Q, N]."""
    d = np.asarray(R).shape[0]
    qr = rotate_queries_f32(q, R)                          # [Q, d]
    lut = (qr[:, :, None] * np.asarray(cen, np.float32)[None, None, :]).astype(np.float32)
    codes = unpack_codes(packed, bits, d).astype(np.int64)  # [N, d]
    out = np.zeros((qr.shape[0], codes.shape[0]), dtype=np.float32)
    for qi in range(qr.shape[0]):
        acc = np.zeros(codes.shape[0], dtype=np.float32)
        for j in range(d):
            acc = (acc + lut[qi, j][codes[:, j]]).astype(np.float32)
        out[qi] = (acc * np.asarray(norms, np.float32)).astype(np.float32)
    return out


def topk_desc(scores, k):
    """Top-k by score descending, equal scores ordered by lower index; pads with
    (-inf, -1) when k exceeds the row count (core.cpp:498-512)."""
    scores = np.asarray(scores)
    Q, N = scores.shape
    out_s = np.full((Q, k), -np.inf, dtype=np.float32)
    out_i = np.full((Q, k), -1, dtype=np.int64)
    idx = np.arange(N)
    for q in range(Q):
        order = np.lexsort((idx, -scores[q].astype(np.float64)))[:k]
        out_s[q, :len(order)] = scores[q, order]
        out_i[q, :len(order)] = order
    return out_s, out_i


def prod_scores_f64(q, mse_packed, signs_packed, gamma, norms, bits, dim, R, cen, S):
    """Prod-mode index scores in float64: queries @ dequantize_prod(rows)^T, the
    computation of TurboQuantIndex._search_prod (search.py:229-252) without its fp32
    roundings.  Returns float64 [Q, N]."""
    rec = dequantize_prod(mse_packed, signs_packed, gamma, norms, bits, dim, R, cen, S)
    return np.asarray(q, np.float64) @ rec.T


def search_topk(q, packed, norms, cen, R, bits, k):
    """Index search (search.py:178-227 semantics, core.cpp:407-514 arithmetic)."""
    return topk_desc(lut_scores_f32(q, packed, norms, cen, R, bits), k)


def scores_f64(q, packed, norms, cen, R, bits):
    """float64 closed form: s = n * (R q) . c[codes]  (reference ops.py:182-194)."""
    d = np.asarray(R).shape[0]
    codes = unpack_codes(packed, bits, d)
    qr = np.asarray(q, np.float64) @ np.asarray(R, np.float64).T
    return (qr @ np.asarray(cen, np.float64)[codes].T) * np.asarray(norms, np.float64)[None, :]


def values_f64(w, packed, norms, cen, M, bits):
    """float64 closed form of attention_values_packed (quant_cpu.cpp:199-266):
    (sum_t w_t n_t c[code_t]) @ M."""
    d = np.asarray(M).shape[0]
    codes = unpack_codes(packed, bits, d)
    v = np.asarray(cen, np.float64)[codes] * np.asarray(norms, np.float64)[:, None]
    return (np.asarray(w, np.float64) @ v) @ np.asarray(M, np.float64)


def decode_attention_f64(q, kpacked, knorms, vpacked, vnorms, seq_lens, kc, vc, Rk, Rv, kbits,
                         vbits, scale, return_lse=False):
    """float64 GQA decode attention over packed K/V (cache.py:282-339 + softmax,
    vllm_plugin/__init__.py:400), q head h reading kv head h // (Hq / Hkv).
    q [B, Hq, d]; kpacked [B, Hkv, T, Pk]; knorms [B, Hkv, T]; -> [B, Hq, d]."""
    q = np.asarray(q, np.float64)
    B, Hq, d = q.shape
    Hkv = kpacked.shape[1]
    G = Hq // Hkv
    out = np.zeros((B, Hq, d))
    lse = np.full((B, Hq), -np.inf)
    for b in range(B):
        T = int(seq_lens[b])
        if T == 0:
            continue
        for g in range(Hkv):
            kcod = unpack_codes(kpacked[b, g, :T], kbits, d)
            vcod = unpack_codes(vpacked[b, g, :T], vbits, d)
            K = (np.asarray(kc, np.float64)[kcod] @ np.asarray(Rk, np.float64)) * np.asarray(knorms[b, g, :T], np.float64)[:, None]
            V = (np.asarray(vc, np.float64)[vcod] @ np.asarray(Rv, np.float64)) * np.asarray(vnorms[b, g, :T], np.float64)[:, None]
            for h in range(g * G, (g + 1) * G):
                s = (K @ q[b, h]) * scale
                p = np.exp(s - s.max())
                lse[b, h] = s.max() + np.log(p.sum())
                p /= p.sum()
                out[b, h] = p @ V
    return (out, lse) if return_lse else out


def decode_attention_bf16_reference(q, kpacked, knorms, vpacked, vnorms, seq_lens, kc, vc, Rk,
                                    Rv, kbits, vbits, scale):
    """The reference's own rounding for a bf16 model's cache, with float64 sums elsewhere:
    the history is dequantized in the norms' dtype, so every K/V element is rounded to
    bf16 (reference.py:356-365 computes c[codes] @ R * n in norms.dtype), handed to SDPA
    in bf16 (hf_integration.py:372-390), and the output is rounded to bf16.  Not the
    product's parity target: it measures how far the reference's bf16 arithmetic itself
    sits from decode_attention_f64, the bar the kernels' bf16 paths are held under."""
    q = round_bf16(np.asarray(q, np.float32)).astype(np.float64)
    B, Hq, d = q.shape
    Hkv = kpacked.shape[1]
    G = Hq // Hkv
    out = np.zeros((B, Hq, d))
    for b in range(B):
        T = int(seq_lens[b])
        if T == 0:
            continue
        for g in range(Hkv):
            K = round_bf16(dequantize_mse(kpacked[b, g, :T], knorms[b, g, :T], kbits, d, Rk, kc)).astype(np.float64)
            V = round_bf16(dequantize_mse(vpacked[b, g, :T], vnorms[b, g, :T], vbits, d, Rv, vc)).astype(np.float64)
            for h in range(g * G, (g + 1) * G):
                s = (K @ q[b, h]) * scale
                p = np.exp(s - s.max())
                out[b, h] = round_bf16(((p / p.sum()) @ V).astype(np.float32))
    return out


# ----------------------------------------------------------------- paged KV (vLLM block tables)


def paged_rows(pool, block_table, T):
    """Rows of tokens 0..T-1 of one sequence from a block pool [num_blocks, H, bs, ...]:
    token t sits in block block_table[t // bs] at slot t % bs (vLLM's paging).
    Returns [H, T, ...]."""
    pool = np.asarray(pool)
    bs = pool.shape[2]
    t = np.arange(T)
    blk = np.asarray(block_table, np.int64)[t // bs]
    return np.stack([pool[blk[i], :, t[i] % bs] for i in range(T)], axis=1) if T else \
        np.zeros((pool.shape[1], 0) + pool.shape[3:], pool.dtype)


def paged_attention_f64(q, kpool, knorm_pool, vpool, vnorm_pool, block_table, T, kc, vc, Rk, Rv,
                        kbits, vbits, scale, kprod=None, vprod=None):
    """float64 attention of one sequence's n new tokens q [n, Hq, d] -- positions
    T-n .. T-1 -- over its first T cached tokens, causally (token i sees positions
    <= T-n+i), with GQA (q head h reads kv head h // (Hq/Hkv)).  K/V are the
    dequantized pool rows (reference.py:320-367; with kprod/vprod = (sign_pool,
    res_pool, S) the prod reconstruction of reference.py:472-533 at bits-1 codes).
    The reference's vLLM step (vllm_plugin/__init__.py:380-412) is this with n = 1 and
    one sequence.  Returns [n, Hq, d]."""
    q = np.asarray(q, np.float64)
    n, Hq, d = q.shape
    Hkv = kpool.shape[1]
    G = Hq // Hkv

    def deq(pool, npool, cen, R, bits, prod):
        rows, nrm = paged_rows(pool, block_table, T), paged_rows(npool, block_table, T)
        out = []
        for g in range(Hkv):
            if prod is None:
                codes = unpack_codes(rows[g], bits, d)
                x = (np.asarray(cen, np.float64)[codes] @ np.asarray(R, np.float64)) * nrm[g].astype(np.float64)[:, None]
            else:
                sg, rs = paged_rows(prod[0], block_table, T)[g], paged_rows(prod[1], block_table, T)[g]
                x = dequantize_prod(rows[g], sg, rs, nrm[g], bits, d, R, cen, prod[2])
            out.append(x)
        return out

    K = deq(kpool, knorm_pool, kc, Rk, kbits, kprod)
    V = deq(vpool, vnorm_pool, vc, Rv, vbits, vprod)
    out = np.zeros((n, Hq, d))
    for i in range(n):
        vis = T - n + i + 1
        for h in range(Hq):
            g = h // G
            s = (K[g][:vis] @ q[i, h]) * scale
            p = np.exp(s - s.max())
            out[i, h] = (p / p.sum()) @ V[g][:vis]
    return out
