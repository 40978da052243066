"""GPU tests of the paged (vLLM block-table) KV path: slot-mapped stores and gathers
bit-exact against numpy, paged decode against the contiguous decode kernels and the
float64 oracle, and the vLLM attention step (mixed prefill + decode batches, causal
prefill, GQA, prod mode, protected layers) against the float64 paged oracle."""

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
    t = torch.from_numpy(np.ascontiguousarray(a)).to(DEV)
    t = t if dtype is None else t.to(dtype)
    _ALIVE.append(t)
    return t


def sync():
    torch.cuda.synchronize()
    _ALIVE.clear()


def _tables(rs, lens, bs, nblocks, width):
    """Block tables of distinct random blocks; entries past a sequence's blocks are -1."""
    perm = rs.permutation(nblocks)
    tab = np.full((len(lens), width), -1, np.int32)
    used = 0
    for i, n in enumerate(lens):
        k = (n + bs - 1) // bs
        tab[i, :k] = perm[used:used + k]
        used += k
    return tab


def _np_store(rows, norms, slots, pool, npool):
    bs = pool.shape[2]
    for t, s in enumerate(slots):
        if 0 <= s < pool.shape[0] * bs:
            pool[s // bs, :, s % bs] = rows[t]
            npool[s // bs, :, s % bs] = norms[t]


@pytest.mark.parametrize("P", [32, 25])
def test_paged_store_and_gather_bit_exact(P):
    rs = np.random.RandomState(P)
    nb, H, bs = 12, 3, 16
    pool = np.zeros((nb, H, bs, P), np.uint8)
    npool = np.zeros((nb, H, bs), np.float32)
    pt, nt = T(pool), T(npool)
    lens = [37, 5, 0]
    tab = _tables(rs, lens, bs, nb, 4)
    # every token of the three sequences, in shuffled order, plus two padding slots
    slots = [tab[i, t // bs] * bs + t % bs for i, n in enumerate(lens) for t in range(n)]
    slots = np.array(slots + [-1, nb * bs + 3], np.int64)[rs.permutation(len(slots) + 2)]
    rows = rs.randint(0, 256, (len(slots), H, P)).astype(np.uint8)
    norms = rs.rand(len(slots), H).astype(np.float32)
    capi.check(L().tq_paged_store(capi.p(T(rows)), capi.p(T(norms)), capi.i64(len(slots)), capi.i32(H),
                                  capi.i32(P), capi.p(T(slots)), capi.p(pt), capi.p(nt), capi.i64(nb),
                                  capi.i32(bs), capi.stream()))
    sync()
    _np_store(rows, norms, slots, pool, npool)
    assert np.array_equal(pt.cpu().numpy(), pool) and np.array_equal(nt.cpu().numpy(), npool)
    tmax = 48
    out = torch.empty(3, H, tmax, P, dtype=torch.uint8, device=DEV)
    onr = torch.empty(3, H, tmax, dtype=torch.float32, device=DEV)
    tab[0, 3] = 99  # past sequence 0's tokens anyway; must not be read
    capi.check(L().tq_paged_gather(capi.p(pt), capi.p(nt), capi.i64(nb), capi.i32(H), capi.i32(bs),
                                   capi.i32(P), capi.p(T(tab)), capi.i32(tab.shape[1]),
                                   capi.p(T(np.array(lens, np.int32))), capi.i32(3), capi.i64(tmax),
                                   capi.p(out), capi.p(onr), capi.stream()))
    sync()
    o, on = out.cpu().numpy(), onr.cpu().numpy()
    for i, n in enumerate(lens):
        assert np.array_equal(o[i, :, :n], O.paged_rows(pool, tab[i], n))
        assert np.array_equal(on[i, :, :n], O.paged_rows(npool, tab[i], n))
        assert not o[i, :, n:].any() and not on[i, :, n:].any()


def k_decode_paged(q_t, kpool, knp, vpool, vnp, tab, lens, kc, vc, Rk, Rv, kb, vb, scale):
    B, Hq, d = q_t.shape
    nb, Hkv, bs = kpool.shape[:3]
    dt = {torch.float32: capi.TQ_F32, torch.bfloat16: capi.TQ_BF16, torch.float16: capi.TQ_F16}[q_t.dtype]
    out = torch.empty_like(q_t)
    lse = torch.empty(B, Hq, dtype=torch.float32, device=DEV)
    wsb = L().tq_decode_paged_workspace_bytes(dt, B, Hq, Hkv, d, kb, vb, tab.shape[1], bs)
    ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device=DEV)
    capi.check(L().tq_decode_attention_paged(
        capi.p(q_t), dt, capi.i32(B), capi.i32(Hq), capi.i32(Hkv), capi.i32(d), capi.p(T(kpool)),
        capi.p(T(knp)), capi.p(T(vpool)), capi.p(T(vnp)), capi.i64(nb), capi.i32(bs), capi.p(T(tab)),
        capi.i32(tab.shape[1]), capi.p(T(np.asarray(lens, np.int32))), capi.p(T(kc)), capi.p(T(vc)),
        capi.p(T(Rk)), capi.p(T(Rv)), capi.i32(kb), capi.i32(vb), ctypes.c_float(scale), capi.p(out),
        capi.p(lse), capi.p(ws), ctypes.c_size_t(ws.numel()), capi.stream()))
    sync()
    return out.float().cpu().numpy(), lse.cpu().numpy()


def k_decode(q_t, kp, kn, vp, vn, seq_lens, kc, vc, Rk, Rv, kb, vb, scale):
    B, Hq, d = q_t.shape
    Hkv, Tm = kp.shape[1], kp.shape[2]
    out = torch.empty_like(q_t)
    lse = torch.empty(B, Hq, dtype=torch.float32, device=DEV)
    ws = torch.empty(max(L().tq_decode_workspace_bytes(B, Hq, d, Tm), 1), dtype=torch.uint8, device=DEV)
    dt = {torch.float32: capi.TQ_F32, torch.bfloat16: capi.TQ_BF16, torch.float16: capi.TQ_F16}[q_t.dtype]
    capi.check(L().tq_decode_attention_packed(
        capi.p(q_t), dt, capi.i32(B), capi.i32(Hq), capi.i32(Hkv), capi.i32(d), capi.p(T(kp)),
        capi.p(T(kn)), capi.p(T(vp)), capi.p(T(vn)), capi.i64(Tm), capi.p(T(np.asarray(seq_lens, np.int32))),
        capi.p(T(kc)), capi.p(T(vc)), capi.p(T(Rk)), capi.p(T(Rv)), capi.i32(kb), capi.i32(vb),
        ctypes.c_float(scale), capi.p(out), capi.p(lse), capi.p(ws), ctypes.c_size_t(ws.numel()),
        capi.stream()))
    sync()
    return out.float().cpu().numpy(), lse.cpu().numpy()


@pytest.mark.parametrize("d,kb,vb,G,bs,qdt", [(64, 4, 2, 4, 16, torch.bfloat16),
                                              (64, 3, 1, 2, 64, torch.float16),
                                              (64, 4, 2, 1, 8, torch.bfloat16),
                                              (128, 4, 2, 2, 16, torch.bfloat16),   # gathered path
                                              (64, 4, 2, 4, 16, torch.float32)])    # gathered path
def test_decode_paged_vs_contiguous_and_f64(d, kb, vb, G, bs, qdt):
    rs = np.random.RandomState(d + kb * 10 + bs)
    Hkv, B = 2, 4
    Hq = G * Hkv
    lens = [0, 3, 700, 1500]
    width = (max(lens) + bs - 1) // bs + 1
    nb = sum((n + bs - 1) // bs for n in lens) + 5
    tab = _tables(rs, lens, bs, nb, width)
    Rk, Rv = O.dense_qr_rotation(d, 42), O.dense_qr_rotation(d, 43)
    _, ck = O.lloyd_max_codebook(kb, d)
    _, cv = O.lloyd_max_codebook(vb, d)
    bpp = d // 8
    kpool = rs.randint(0, 256, (nb, Hkv, bs, kb * bpp)).astype(np.uint8)
    vpool = rs.randint(0, 256, (nb, Hkv, bs, vb * bpp)).astype(np.uint8)
    knp = rs.uniform(0.5, 2.0, (nb, Hkv, bs)).astype(np.float32)
    vnp = rs.uniform(0.5, 2.0, (nb, Hkv, bs)).astype(np.float32)
    # stale slots past each sequence's end in its last block hold NaN norms: masked
    # tokens must not reach the output
    for b, n in enumerate(lens):
        if n % bs:
            knp[tab[b, (n - 1) // bs], :, n % bs:] = np.nan
            vnp[tab[b, (n - 1) // bs], :, n % bs:] = np.nan
    q = torch.from_numpy(rs.randn(B, Hq, d).astype(np.float32)).to(DEV).to(qdt)
    scale = 1.0 / math.sqrt(d)
    got, lse = k_decode_paged(q, kpool, knp, vpool, vnp, tab, lens, ck, cv, Rk, Rv, kb, vb, scale)
    assert np.all(np.isfinite(got))
    # the same tokens laid out contiguously, through the contiguous decode entry point
    Tm = width * bs
    kc_, kn_, vc_, vn_ = (np.zeros((B, Hkv, Tm) + p.shape[3:], p.dtype) for p in (kpool, knp, vpool, vnp))
    for b, n in enumerate(lens):
        for arr, pool in ((kc_, kpool), (kn_, knp), (vc_, vpool), (vn_, vnp)):
            arr[b, :, :n] = O.paged_rows(pool, tab[b], n)
    ref, ref_lse = k_decode(q, kc_, kn_, vc_, vn_, lens, ck, cv, Rk, Rv, kb, vb, scale)
    if d == 64 and qdt != torch.float32:   # same fused kernel and split plan: identical sums
        assert np.array_equal(got, ref) and np.array_equal(lse, ref_lse)
    else:
        assert np.max(np.abs(got - ref)) <= 1e-5 * np.max(np.abs(ref))
    want = O.decode_attention_f64(q.float().cpu().numpy(), kc_, kn_, vc_, vn_, lens, ck, cv, Rk, Rv,
                                  kb, vb, scale)
    assert np.all(got[0] == 0)
    tol = 1e-2 if qdt != torch.float32 else 1e-3
    assert np.max(np.abs(got - want)) <= tol * np.max(np.abs(want))


def _step_meta(blocks, before, n_new, bs, host_copies=False):
    """One vLLM-ordered batch: sequences with n_new > 1 are prefills (listed first), the
    rest decode one token.  blocks[i] = sequence i's physical blocks for all its tokens.
    host_copies: the metadata also carries host lists of query_start_loc and seq_lens."""
    from turboquant_kv.vllm_plugin import TurboQuantAttentionMetadata
    order = sorted(range(len(n_new)), key=lambda i: n_new[i] == 1)
    width = max(len(b) for b in blocks)
    tab = np.full((len(order), width), -1, np.int32)
    slots, qsl, lens = [], [0], []
    for j, i in enumerate(order):
        tab[j, :len(blocks[i])] = blocks[i]
        lens.append(before[i] + n_new[i])
        slots += [blocks[i][t // bs] * bs + t % bs for t in range(before[i], lens[-1])]
        qsl.append(qsl[-1] + n_new[i])
    md = TurboQuantAttentionMetadata(
        slot_mapping=torch.tensor(slots, dtype=torch.long, device=DEV),
        seq_lens=torch.tensor(lens, dtype=torch.int32, device=DEV),
        block_tables=torch.from_numpy(tab).to(DEV),
        query_start_loc=torch.tensor(qsl, dtype=torch.int32, device=DEV),
        num_prefills=sum(1 for i in order if n_new[i] > 1),
        query_start_loc_cpu=list(qsl) if host_copies else None,
        seq_lens_cpu=list(lens) if host_copies else None)
    return md, order, lens, tab


def _bitplane_pools(pools, tab, lens):
    """The layer-0 pools as numpy arrays; decode-layout pools are converted to bit-plane
    rows (through the pools' own gather + unpack) at the sequences' blocks."""
    st = pools.layers[0]
    P = {key: t.cpu().numpy() for key, t in st.items()}
    if "kp" not in st:
        return P
    nb, H, bs = st["kn"].shape
    out = {"k": np.zeros((nb, H, bs, 32), np.uint8), "v": np.zeros((nb, H, bs, 8 * pools.vbits), np.uint8),
           "kn": np.zeros((nb, H, bs), np.float32), "vn": np.zeros((nb, H, bs), np.float32)}
    for j, n in enumerate(lens):
        bt = torch.from_numpy(tab[j]).to(DEV)
        for kind in ("k", "v"):
            rows, norms = pools._gather(st, kind, bt, n)
            rows, norms = rows.cpu().numpy(), norms.cpu().numpy()
            for t in range(n):
                out[kind][tab[j, t // bs], :, t % bs] = rows[:, t]
                out[kind + "n"][tab[j, t // bs], :, t % bs] = norms[:, t]
    return out


@pytest.mark.parametrize("mode,kb,vb,d,G,layout", [("mse", 4, 2, 64, 4, "bitplane"),
                                                   ("mse", 4, 2, 64, 4, "auto"),
                                                   ("mse", 4, 2, 64, 8, "auto"),
                                                   ("mse", 4, 2, 64, 7, "auto"),
                                                   ("mse", 4, 3, 64, 4, "auto"),
                                                   ("mse", 4, 4, 64, 2, "auto"),
                                                   ("mse", 3, 2, 128, 2, "auto"),
                                                   ("prod", 4, 3, 64, 2, "auto")])
def test_vllm_paged_step_vs_f64(mode, kb, vb, d, G, layout):
    # Two steps through the vLLM entry: a batch of prompts (prefill), then a mixed batch
    # -- a chunked prefill continuing one sequence and single-token decodes of the
    # others -- each checked against the float64 paged oracle (causal, GQA).
    from turboquant_kv.vllm_plugin import (TurboQuantKVCacheConfig, TurboQuantPagedKVCache,
                                           paged_attention_step)
    rs = np.random.RandomState(kb * 7 + d)
    Hkv, bs, nb = 2, 16, 64
    Hq = G * Hkv
    cfg = TurboQuantKVCacheConfig(key_bits=kb, value_bits=vb, mode=mode, block_size=bs,
                                  num_gpu_blocks=nb, pool_layout=layout)
    kv = TurboQuantPagedKVCache(cfg, num_layers=1, num_heads=Hkv, head_dim=d, device=DEV)
    pools = kv.pools()
    assert pools.layout == ("decode" if (mode, kb, d, layout) == ("mse", 4, 64, "auto")
                            else "bitplane")
    scale = 1.0 / math.sqrt(d)
    steps = [[40, 17, 70, 5], [30, 1, 1, 1]]   # new tokens per sequence in each step
    final = [sum(s[i] for s in steps) for i in range(4)]
    perm = [int(b) for b in rs.permutation(nb)]
    blocks, used = [], 0
    for n in final:
        k = (n + bs - 1) // bs
        blocks.append(perm[used:used + k])
        used += k
    before = [0, 0, 0, 0]
    for step, n_new in enumerate(steps):
        md, order, lens, tab = _step_meta(blocks, before, n_new, bs)
        n_tok = sum(n_new)
        q = torch.randn(n_tok, Hq, d, device=DEV, dtype=torch.bfloat16)
        k = torch.randn(n_tok, Hkv, d, device=DEV, dtype=torch.bfloat16)
        v = torch.randn(n_tok, Hkv, d, device=DEV, dtype=torch.bfloat16)
        out = paged_attention_step(q, k, v, kv, md, scale)
        assert out.shape == q.shape and out.dtype == q.dtype
        P = _bitplane_pools(pools, tab, lens)
        kc, vc = pools.kcen.cpu().numpy(), pools.vcen.cpu().numpy()
        Rk, Rv = pools.R_k.cpu().numpy(), pools.R_v.cpu().numpy()
        kprod = vprod = None
        if mode == "prod":
            kprod = (P["ks"], P["kr"], pools.S_k.cpu().numpy())
            vprod = (P["vs"], P["vr"], pools.S_v.cpu().numpy())
        qsl = md.query_start_loc.tolist()
        for j in range(len(order)):
            a, b = qsl[j], qsl[j + 1]
            want = O.paged_attention_f64(q[a:b].float().cpu().numpy(), P["k"], P["kn"], P["v"],
                                         P["vn"], tab[j], lens[j], kc, vc, Rk, Rv,
                                         pools.kbits if mode == "mse" else kb,
                                         pools.vbits if mode == "mse" else vb, scale, kprod, vprod)
            got = out[a:b].float().cpu().numpy()
            assert np.max(np.abs(got - want)) <= 2e-2 * np.max(np.abs(want)), (step, j)
        before = [before[i] + n_new[i] for i in range(4)]


def test_vllm_paged_protected_layer_and_padding():
    from turboquant_kv.vllm_plugin import (TurboQuantAttentionMetadata, TurboQuantKVCacheConfig,
                                           TurboQuantPagedKVCache, paged_attention_step)
    rs = np.random.RandomState(3)
    Hkv, Hq, d, bs, nb = 2, 4, 64, 16, 16
    cfg = TurboQuantKVCacheConfig(key_bits=4, value_bits=2, block_size=bs, num_gpu_blocks=nb,
                                  protected_layers=1)
    kv = TurboQuantPagedKVCache(cfg, num_layers=2, num_heads=Hkv, head_dim=d, device=DEV)
    tab = np.array([[5, 2, 9]], np.int32)
    n = 35
    slots = [tab[0, t // bs] * bs + t % bs for t in range(n)] + [-1, -1]   # two padding tokens
    q = torch.randn(n + 2, Hq, d, device=DEV)
    k = torch.randn(n + 2, Hkv, d, device=DEV)
    v = torch.randn(n + 2, Hkv, d, device=DEV)
    md = TurboQuantAttentionMetadata(torch.tensor(slots, device=DEV), torch.tensor([n], dtype=torch.int32),
                                     torch.from_numpy(tab).to(DEV), torch.tensor([0, n]), 1, layer_id=0)
    out = paged_attention_step(q, k, v, kv, md, 0.125)
    # protected layer: fp16 K/V, causal softmax attention in float64
    qf = q[:n].double().transpose(0, 1).contiguous()                          # [Hq, n, d]
    kf = k[:n].half().double().repeat_interleave(2, dim=1).transpose(0, 1).contiguous()
    vf = v[:n].half().double().repeat_interleave(2, dim=1).transpose(0, 1).contiguous()
    s = torch.matmul(qf, kf.transpose(1, 2).contiguous()) * 0.125
    s = s.masked_fill(torch.triu(torch.ones(n, n, dtype=torch.bool, device=DEV), 1), float("-inf"))
    want = torch.matmul(torch.softmax(s, -1), vf).transpose(0, 1)
    assert (out[:n].double() - want).abs().max().item() <= 1e-4 * want.abs().max().item()
    # padding slots wrote nothing: only the sequence's three blocks hold data
    fp = kv.pools().layers[0]["k_fp"]
    used = torch.zeros(nb, dtype=torch.bool)
    used[[5, 2, 9]] = True
    assert fp[~used.to(DEV)].abs().sum().item() == 0


# ------------------------------------------------------------------ decode-layout pools
def _dl_pools(rs, lens, bs, nb, width, Hkv, vb=2, vmul=None):
    """Random 4-bit key / vb-bit value bit-plane rows of every token, stored into
    decode-layout block pools through the C ABI (values in two shuffled calls, so tiles are
    filled piecewise).  vmul(positions) scales the value norms per token.  Returns the
    pools and each sequence's contiguous rows and norms."""
    from turboquant_kv import ops
    tab = _tables(rs, lens, bs, nb, width)
    slots = np.array([tab[i, t // bs] * bs + t % bs for i, n in enumerate(lens) for t in range(n)],
                     np.int64)
    n = len(slots)
    krows = rs.randint(0, 256, (n, Hkv, 32)).astype(np.uint8)
    vrows = rs.randint(0, 256, (n, Hkv, 8 * vb)).astype(np.uint8)
    kn = rs.uniform(0.5, 2.0, (n, Hkv)).astype(np.float32)
    vn = rs.uniform(0.5, 2.0, (n, Hkv)).astype(np.float32)
    if vmul is not None:
        pos = np.concatenate([np.arange(L_) for L_ in lens])
        vn = (vn * vmul(pos)[:, None]).astype(np.float32)
    kp = torch.zeros(nb, Hkv, bs, 32, dtype=torch.uint8, device=DEV)
    knp = torch.zeros(nb, Hkv, bs, dtype=torch.float32, device=DEV)
    vt = (torch.zeros(nb, Hkv, bs // 64, 512 * vb, dtype=torch.uint8, device=DEV) if bs >= 64 else
          torch.zeros(nb, Hkv, bs // 16, 128 * vb, dtype=torch.uint8, device=DEV))
    vnp = torch.zeros(nb, Hkv, bs, dtype=torch.float32, device=DEV)
    pairs = torch.empty(n * Hkv, 1, 32, dtype=torch.uint8, device=DEV)
    ops.pack_decode_layout(T(krows).view(n * Hkv, 1, 32), pairs, 64, 4, False, 0)
    capi.check(L().tq_paged_store(capi.p(pairs), capi.p(T(kn)), capi.i64(n), capi.i32(Hkv), capi.i32(32),
                                  capi.p(T(slots)), capi.p(kp), capi.p(knp), capi.i64(nb), capi.i32(bs),
                                  capi.stream()))
    order = rs.permutation(n)
    for part in (order[: n // 2], order[n // 2:]):
        sp = np.concatenate([slots[part], [-1]]).astype(np.int64)       # plus one padding slot
        rp = np.concatenate([vrows[part], vrows[:1]])
        npart = np.concatenate([vn[part], vn[:1]])
        capi.check(L().tq_paged_store_value_tiles(capi.p(T(rp)), capi.p(T(npart)), capi.i64(len(sp)),
                                                  capi.i32(Hkv), capi.p(T(sp)), capi.p(vt), capi.p(vnp),
                                                  capi.i64(nb), capi.i32(bs), capi.i32(vb), capi.stream()))
    sync()
    seqs, o = [], 0
    for L_ in lens:
        seqs.append((krows[o:o + L_].transpose(1, 0, 2), kn[o:o + L_].T, vrows[o:o + L_].transpose(1, 0, 2),
                     vn[o:o + L_].T))
        o += L_
    return tab, kp, knp, vt, vnp, seqs


@pytest.mark.parametrize("vb", [2, 3, 4])
@pytest.mark.parametrize("bs", [16, 32, 64, 128])
def test_paged_dl_store_round_trip(bs, vb):
    # every bit of every token's value code lands where the decode kernel reads it: the
    # pools gathered back into the contiguous decode layout unpack to the stored rows
    from turboquant_kv import ops
    from turboquant_kv.vllm_plugin.paged import gather_value_tiles
    rs = np.random.RandomState(bs + vb)
    Hkv, lens = 2, [130, 64, 1, 0]
    width = (max(lens) + bs - 1) // bs + 1
    nb = sum((n + bs - 1) // bs for n in lens) + 3
    tab, kp, knp, vt, vnp, seqs = _dl_pools(rs, lens, bs, nb, width, Hkv, vb)
    for b, n in enumerate(lens):
        if n == 0:
            continue
        one = lambda v: torch.tensor([v], dtype=torch.int32, device=DEV)
        bt = T(tab[b:b + 1])
        pr, pn = ops.paged_gather(kp, knp, bt, one(n), n)
        tiles = gather_value_tiles(vt, bt, n)
        _, vnn = ops.paged_gather(kp, vnp, bt, one(n), n)
        kr, knr, vr, vnr = seqs[b]
        assert np.array_equal(ops.unpack_decode_layout(pr[0], 64, 4, False, 0, n).cpu().numpy(), kr)
        assert np.array_equal(ops.unpack_decode_layout(tiles, 64, vb, True, 0, n).cpu().numpy(), vr)
        assert np.array_equal(pn[0].cpu().numpy(), knr) and np.array_equal(vnn[0].cpu().numpy(), vnr)


@pytest.mark.parametrize("bs,G,qdt,vb", [(64, 4, torch.bfloat16, 2), (128, 2, torch.float16, 2),
                                         (64, 1, torch.float32, 2), (16, 4, torch.bfloat16, 2),
                                         (32, 2, torch.float16, 2), (16, 1, torch.float32, 2),
                                         (16, 8, torch.bfloat16, 2), (64, 6, torch.float32, 2),
                                         (16, 4, torch.bfloat16, 3), (64, 4, torch.bfloat16, 3),
                                         (32, 6, torch.float32, 3), (128, 1, torch.float16, 3),
                                         (16, 2, torch.float16, 4), (64, 8, torch.float32, 4),
                                         (32, 4, torch.bfloat16, 4)])
def test_decode_paged_dl_vs_contiguous_and_f64(bs, G, qdt, vb):
    # The paged decode-layout kernel (16-token sub-blocks below block size 64, 64-token
    # tiles from 64 on) equals the contiguous kernel over the same tokens bit for bit, and
    # the float64 oracle within the query type's tolerance.
    from turboquant_kv import ops
    rs = np.random.RandomState(bs + G + 100 * vb)
    Hkv = 2
    Hq = G * Hkv
    lens = [0, 3, 700, 1500, 64]
    B = len(lens)
    width = (max(lens) + bs - 1) // bs + 1
    width = -(-width * bs // 64) * 64 // bs   # the contiguous reference needs t_cap % 64 == 0
    nb = sum((n + bs - 1) // bs for n in lens) + 4
    tab, kp, knp, vt, vnp, seqs = _dl_pools(rs, lens, bs, nb, width, Hkv, vb)
    tab[0, 0] = 7   # a block id past sequence 0's (empty) context: never read
    Rk, Rv = O.dense_qr_rotation(64, 42), O.dense_qr_rotation(64, 43)
    _, ck = O.lloyd_max_codebook(4, 64)
    _, cv = O.lloyd_max_codebook(vb, 64)
    q = torch.from_numpy(rs.randn(B, Hq, 64).astype(np.float32)).to(DEV).to(qdt)
    scale = 0.125
    dt = {torch.float32: capi.TQ_F32, torch.bfloat16: capi.TQ_BF16, torch.float16: capi.TQ_F16}[qdt]
    out = torch.empty_like(q)
    lse = torch.empty(B, Hq, dtype=torch.float32, device=DEV)
    Tc = width * bs
    ws = torch.empty(L().tq_decode_dl_workspace_bytes(B, Hq, Hkv, Tc), dtype=torch.uint8, device=DEV)
    capi.check(L().tq_decode_attention_paged_dl(
        capi.p(q), dt, capi.i32(B), capi.i32(Hq), capi.i32(Hkv), capi.i32(64), capi.p(kp), capi.p(knp),
        capi.p(vt), capi.p(vnp), capi.i64(nb), capi.i32(bs), capi.i32(vb), capi.p(T(tab)), capi.i32(width),
        capi.p(T(np.asarray(lens, np.int32))), capi.p(T(ck)), capi.p(T(cv)), capi.p(T(Rk)), capi.p(T(Rv)),
        ctypes.c_float(scale), capi.p(out), capi.p(lse), capi.p(ws), ctypes.c_size_t(ws.numel()),
        capi.stream()))
    sync()
    got, got_lse = out.float().cpu().numpy(), lse.cpu().numpy()
    # the same tokens in contiguous decode-layout caches of the same capacity
    kc_ = np.zeros((B, Hkv, Tc, 32), np.uint8)
    vc_ = np.zeros((B, Hkv, Tc, 8 * vb), np.uint8)
    kn_, vn_ = np.zeros((B, Hkv, Tc), np.float32), np.zeros((B, Hkv, Tc), np.float32)
    for b, n in enumerate(lens):
        kc_[b, :, :n], kn_[b, :, :n], vc_[b, :, :n], vn_[b, :, :n] = seqs[b]
    kpairs = torch.empty(B * Hkv, Tc, 32, dtype=torch.uint8, device=DEV)
    vblocks = torch.zeros(B * Hkv, Tc // 64, 512 * vb, dtype=torch.uint8, device=DEV)
    ops.pack_decode_layout(T(kc_).view(B * Hkv, Tc, 32), kpairs, 64, 4, False, 0)
    ops.pack_decode_layout(T(vc_).view(B * Hkv, Tc, 8 * vb), vblocks, 64, vb, True, 0)
    ref, ref_lse = ops.decode_attention_dl(q, kpairs.view(B, Hkv, Tc, 32), T(kn_),
                                           vblocks.view(B, Hkv, Tc // 64, 512 * vb), T(vn_),
                                           T(np.asarray(lens, np.int32)), T(ck), T(cv), T(Rk), T(Rv),
                                           scale, return_lse=True)
    # same kernel, same split plan: identical sums
    assert np.array_equal(got, ref.float().cpu().numpy())
    assert np.array_equal(got_lse, ref_lse.cpu().numpy())
    want = O.decode_attention_f64(q.float().cpu().numpy(), kc_, kn_, vc_, vn_, lens, ck, cv, Rk, Rv,
                                  4, vb, scale)
    assert np.all(got[0] == 0) and np.all(np.isneginf(got_lse[0]))
    tol = 1e-2 if qdt != torch.float32 else 1e-4
    assert np.max(np.abs(got - want)) <= tol * np.max(np.abs(want))


@pytest.mark.parametrize("vb", [2, 3, 4])
@pytest.mark.parametrize("bs", [64, 16])
def test_vllm_paged_step_decode_layout_vs_bitplane_and_f64(bs, vb):
    # The vLLM step (chunked prefill + decodes) on decode-layout pools: the stored codes
    # equal the bit-plane pools' and outputs match the float64 paged oracle (K4/V3 is
    # configs[4]'s cache).
    from turboquant_kv.vllm_plugin import PagedKVPools
    from turboquant_kv.config import TurboQuantConfig
    rs = np.random.RandomState(11 + vb)
    Hkv, Hq, d, nb = 2, 8, 64, 24 * 64 // bs
    cfg = TurboQuantConfig(key_bits=4, value_bits=vb)
    bp = PagedKVPools(cfg, 1, nb, bs, Hkv, d, DEV)
    dl = PagedKVPools(cfg, 1, nb, bs, Hkv, d, DEV, layout="decode")
    steps = [[100, 17, 200, 5], [70, 1, 1, 1]]
    final = [sum(s[i] for s in steps) for i in range(4)]
    perm = [int(b) for b in rs.permutation(nb)]
    blocks, used = [], 0
    for n in final:
        k = (n + bs - 1) // bs
        blocks.append(perm[used:used + k])
        used += k
    before = [0, 0, 0, 0]
    scale = 0.125
    for step, n_new in enumerate(steps):
        md, order, lens, tab = _step_meta(blocks, before, n_new, bs, host_copies=step == 0)
        n_tok = sum(n_new)
        q = torch.randn(n_tok, Hq, d, device=DEV, dtype=torch.bfloat16)
        k = torch.randn(n_tok, Hkv, d, device=DEV, dtype=torch.bfloat16)
        v = torch.randn(n_tok, Hkv, d, device=DEV, dtype=torch.bfloat16)
        out_bp = bp.forward(q, k, v, md, scale)
        out_dl = dl.forward(q, k, v, md, scale)
        P = {key: t.cpu().numpy() for key, t in bp.layers[0].items()}
        kc, vc = bp.kcen.cpu().numpy(), bp.vcen.cpu().numpy()
        Rk, Rv = bp.R_k.cpu().numpy(), bp.R_v.cpu().numpy()
        qsl = md.query_start_loc.tolist()
        for j in range(len(order)):
            bt = md.block_tables[j]
            for kind in ("k", "v"):
                r_bp, n_bp = bp._gather(bp.layers[0], kind, bt, lens[j])
                r_dl, n_dl = dl._gather(dl.layers[0], kind, bt, lens[j])
                assert torch.equal(r_bp, r_dl) and torch.equal(n_bp, n_dl), (step, j, kind)
            a, b = qsl[j], qsl[j + 1]
            want = O.paged_attention_f64(q[a:b].float().cpu().numpy(), P["k"], P["kn"], P["v"], P["vn"],
                                         tab[j], lens[j], kc, vc, Rk, Rv, 4, vb, scale)
            got = out_dl[a:b].float().cpu().numpy()
            assert np.max(np.abs(got - want)) <= 2e-2 * np.max(np.abs(want)), (step, j)
            ref = out_bp[a:b].float().cpu().numpy()
            assert np.max(np.abs(got - ref)) <= 2e-2 * np.max(np.abs(want)), (step, j)
        before = [before[i] + n_new[i] for i in range(4)]


@pytest.mark.parametrize("vb", [2, 3, 4])
def test_decode_layout_prefill_kernel_vs_per_token_decode(vb):
    # PagedKVPools.prefill over decode-layout pools runs the tiled prefill kernel.  A whole
    # 1200-token prompt (T = n, block size 16, shuffled blocks) against the per-token
    # decode kernel over the same pools (fp32 queries: both paths fp32-accurate) and the
    # float64 paged oracle.
    from turboquant_kv import ops
    from turboquant_kv.vllm_plugin import PagedKVPools
    from turboquant_kv.config import TurboQuantConfig
    Hkv, Hq, d, bs, nb, n = 2, 8, 64, 16, 80, 1200
    pools = PagedKVPools(TurboQuantConfig(value_bits=vb), 1, nb, bs, Hkv, d, DEV, layout="decode")
    g = torch.Generator(device=DEV).manual_seed(6)
    table = torch.randperm(nb, generator=g, device=DEV)[:(n + bs - 1) // bs].to(torch.int32)
    slots = (table.long()[torch.arange(n, device=DEV) // bs] * bs + torch.arange(n, device=DEV) % bs)
    k = torch.randn(n, Hkv, d, generator=g, device=DEV)
    v = torch.randn(n, Hkv, d, generator=g, device=DEV)
    pools.write(0, k, v, slots)
    q = torch.randn(n, Hq, d, generator=g, device=DEV)
    got = pools.prefill(0, q, table, n, 0.125).cpu().numpy()
    st = pools.layers[0]
    per_token = ops.decode_attention_paged_dl(
        q, st["kp"], st["kn"], st["vt"], st["vn"], table[None].expand(n, -1).contiguous(),
        torch.arange(1, n + 1, dtype=torch.int32, device=DEV), pools.kcen, pools.vcen, pools.R_k,
        pools.R_v, 0.125).cpu().numpy()
    P = _bitplane_pools(pools, table.cpu().numpy()[None], [n])
    want = O.paged_attention_f64(q.cpu().numpy(), P["k"], P["kn"], P["v"], P["vn"],
                                 table.cpu().numpy(), n, pools.kcen.cpu().numpy(),
                                 pools.vcen.cpu().numpy(), pools.R_k.cpu().numpy(),
                                 pools.R_v.cpu().numpy(), 4, vb, 0.125)
    # both kernels fp32-accurate, their sums in different orders
    assert np.max(np.abs(got - want)) <= 1e-4 * np.max(np.abs(want))
    assert np.max(np.abs(got - per_token)) <= 4e-5 * np.max(np.abs(want))


@pytest.mark.parametrize("bs,G,n,qdt,vb", [(16, 4, 300, torch.bfloat16, 2), (32, 7, 77, torch.float16, 2),
                                           (64, 1, 200, torch.float32, 2), (128, 8, 129, torch.bfloat16, 2),
                                           (64, 4, 1, torch.float32, 2), (16, 4, 300, torch.bfloat16, 3),
                                           (64, 2, 200, torch.float32, 3), (32, 7, 77, torch.float16, 4),
                                           (128, 4, 129, torch.bfloat16, 4), (16, 1, 65, torch.float32, 4)])
def test_prefill_kernel_capi_vs_per_token_decode_and_f64(bs, G, n, qdt, vb):
    # tq_prefill_attention_paged_dl: sequence 1's last n tokens (positions T-n .. T-1, so
    # T-n tokens of history) against the per-token decode-layout kernel (B = n rows, row i's
    # context ending at its own position, fp32 queries) and the float64 decode oracle per
    # row.  Query rows per KV head n*G are ragged against the kernel's 64-row tiles; the
    # sequence's stale slots past T hold NaN norms and its block-table entries past T are
    # -1 (clamped into the pool, masked): neither may reach the output.
    from turboquant_kv import ops
    rs = np.random.RandomState(bs * 31 + G + n + 1000 * vb)
    Hkv = 2
    Hq = G * Hkv
    lens = [37, 1100 + bs, 5]
    width = (max(lens) + bs - 1) // bs + 2
    nb = sum((L + bs - 1) // bs for L in lens) + 4
    tab, kp, knp, vt, vnp, seqs = _dl_pools(rs, lens, bs, nb, width, Hkv, vb)
    Tq = lens[1]
    row = tab[1].copy()
    nblk = (Tq + bs - 1) // bs
    for t in range(Tq, nblk * bs):
        knp[int(row[nblk - 1]), :, t % bs] = float("nan")
        vnp[int(row[nblk - 1]), :, t % bs] = float("nan")
    row[nblk:] = -1
    Rk, Rv = O.dense_qr_rotation(64, 42), O.dense_qr_rotation(64, 43)
    _, ck = O.lloyd_max_codebook(4, 64)
    _, cv = O.lloyd_max_codebook(vb, 64)
    q = torch.from_numpy(rs.randn(n, Hq, 64).astype(np.float32)).to(DEV).to(qdt)
    scale = 0.125
    dt = {torch.float32: capi.TQ_F32, torch.bfloat16: capi.TQ_BF16, torch.float16: capi.TQ_F16}[qdt]
    out = torch.empty(n, Hq, 64, dtype=torch.float32, device=DEV)
    print(f"prefill capi bs={bs} G={G} n={n} T={Tq} {qdt} vb={vb}", flush=True)
    capi.check(L().tq_prefill_attention_paged_dl(
        capi.p(q), dt, capi.i32(n), capi.i64(Tq), capi.i32(Hq), capi.i32(Hkv), capi.i32(64), capi.p(kp),
        capi.p(knp), capi.p(vt), capi.p(vnp), capi.i64(nb), capi.i32(bs), capi.i32(vb), capi.p(T(row)),
        capi.i32(width),
        capi.p(T(ck)), capi.p(T(cv)), capi.p(T(Rk)), capi.p(T(Rv)), ctypes.c_float(scale), capi.p(out),
        capi.stream()))
    sync()
    got = out.cpu().numpy()
    assert np.all(np.isfinite(got))
    qf = q.float()
    bt = T(row)[None].expand(n, -1).contiguous()
    pos = torch.arange(Tq - n + 1, Tq + 1, dtype=torch.int32, device=DEV)
    per_token = ops.decode_attention_paged_dl(qf, kp, knp, vt, vnp, bt, pos, T(ck), T(cv), T(Rk), T(Rv),
                                              scale).cpu().numpy()
    kr, kn_, vr, vn_ = seqs[1]
    bc = lambda x: np.broadcast_to(x[None], (n,) + x.shape)
    want = O.decode_attention_f64(qf.cpu().numpy(), bc(kr), bc(kn_), bc(vr), bc(vn_), pos.cpu().numpy(),
                                  ck, cv, Rk, Rv, 4, vb, scale)
    # fp32 / fp16 queries: hi + lo operand parts, fp32-accurate; bf16 queries: one fp16
    # product per term (outputs consumed in bf16, whose rounding is 2^-9)
    # (outputs average many values, so their maximum sits far below the summed terms':
    # both bars are relative to the float64 output's maximum)
    tol_f64, tol_tok = (1e-4, 1e-4) if qdt != torch.bfloat16 else (5e-3, 5e-3)
    assert np.max(np.abs(got - want)) <= tol_f64 * np.max(np.abs(want))
    assert np.max(np.abs(got - per_token)) <= tol_tok * np.max(np.abs(want))


def test_prefill_kernel_capi_refusals():
    # bad shapes are refused before any launch
    z = torch.zeros(64, dtype=torch.float32, device=DEV)
    zb = torch.zeros(64, dtype=torch.uint8, device=DEV)
    tab = torch.zeros(4, dtype=torch.int32, device=DEV)
    args = lambda n, T_, bs, d=64, hq=8, vb=2: (
        capi.p(z), capi.TQ_F32, capi.i32(n), capi.i64(T_), capi.i32(hq), capi.i32(2), capi.i32(d),
        capi.p(zb), capi.p(z), capi.p(zb), capi.p(z), capi.i64(1), capi.i32(bs), capi.i32(vb), capi.p(tab),
        capi.i32(4), capi.p(z), capi.p(z), capi.p(z), capi.p(z), ctypes.c_float(1.0), capi.p(z), capi.stream())
    assert L().tq_prefill_attention_paged_dl(*args(1, 1, 16, d=128)) != 0      # head_dim 64 only
    assert L().tq_prefill_attention_paged_dl(*args(1, 1, 24)) != 0             # block size
    assert L().tq_prefill_attention_paged_dl(*args(5, 4, 16)) != 0            # n > T
    assert L().tq_prefill_attention_paged_dl(*args(1, 65, 16)) != 0            # T past the table
    assert L().tq_prefill_attention_paged_dl(*args(1, 1, 16, hq=7)) != 0       # GQA groups
    assert L().tq_prefill_attention_paged_dl(*args(1, 1, 16, vb=5)) != 0       # value width


# ------------------------------------------------------------------ pools past 2 GiB
def _high_tables(lens, bs, nb, width):
    """Block tables using the pool's last blocks (past the 2 GiB mark of the key pool),
    in descending order; entries past a sequence's blocks are -1."""
    tab = np.full((len(lens), width), -1, np.int32)
    nxt = nb - 1
    for i, n in enumerate(lens):
        for j in range((n + bs - 1) // bs):
            tab[i, j] = nxt
            nxt -= 1
    return tab


@pytest.mark.parametrize("layout,vb,bs", [("decode", 2, 64), ("decode", 3, 64), ("decode", 4, 16),
                                          ("bitplane", 2, 64)])
def test_paged_pools_past_2gib(layout, vb, bs):
    # Key pools of 2.46 GB (76.8M rows of 32 B): the sequences' blocks sit past byte 2^31,
    # which 32-bit buffer offsets cannot reach, so these calls take the 64-bit-address
    # kernels (64-token value tiles, and 16-token sub-blocks at block size 16).  Same sums
    # as the contiguous kernels over the same rows, and the float64 oracle within the bf16
    # tolerance.
    from turboquant_kv import ops
    rs = np.random.RandomState(77 + vb + bs)
    Hkv, G = 2, 4
    Hq = G * Hkv
    lens = [700, 1, 1500]
    B = len(lens)
    nb = 600_000 * 64 // bs
    assert nb * Hkv * bs * 32 >= 2 ** 31
    width = (max(lens) + bs - 1) // bs + 1
    tab = _high_tables(lens, bs, nb, width)
    assert int(tab[tab >= 0].min()) * Hkv * bs * 32 >= 2 ** 31
    slots = np.array([tab[i, t // bs] * bs + t % bs for i, n in enumerate(lens) for t in range(n)],
                     np.int64)
    n = len(slots)
    krows = rs.randint(0, 256, (n, Hkv, 32)).astype(np.uint8)
    vrows = rs.randint(0, 256, (n, Hkv, 8 * vb)).astype(np.uint8)
    kn = rs.uniform(0.5, 2.0, (n, Hkv)).astype(np.float32)
    vn = rs.uniform(0.5, 2.0, (n, Hkv)).astype(np.float32)
    Rk, Rv = O.dense_qr_rotation(64, 42), O.dense_qr_rotation(64, 43)
    _, ck = O.lloyd_max_codebook(4, 64)
    _, cv = O.lloyd_max_codebook(vb, 64)
    q = torch.from_numpy(rs.randn(B, Hq, 64).astype(np.float32)).to(DEV).to(torch.bfloat16)
    scale = 0.125
    Tc = -(-width * bs // 64) * 64   # the contiguous reference needs t_cap % 64 == 0
    kc_ = np.zeros((B, Hkv, Tc, 32), np.uint8)
    vc_ = np.zeros((B, Hkv, Tc, 8 * vb), np.uint8)
    kn_, vn_ = np.zeros((B, Hkv, Tc), np.float32), np.zeros((B, Hkv, Tc), np.float32)
    o = 0
    for b, L_ in enumerate(lens):
        kc_[b, :, :L_] = krows[o:o + L_].transpose(1, 0, 2)
        vc_[b, :, :L_] = vrows[o:o + L_].transpose(1, 0, 2)
        kn_[b, :, :L_], vn_[b, :, :L_] = kn[o:o + L_].T, vn[o:o + L_].T
        o += L_
    lens_t = T(np.asarray(lens, np.int32))
    out = torch.empty_like(q)
    lse = torch.empty(B, Hq, dtype=torch.float32, device=DEV)
    knp = torch.zeros(nb, Hkv, bs, dtype=torch.float32, device=DEV)
    vnp = torch.zeros(nb, Hkv, bs, dtype=torch.float32, device=DEV)
    if layout == "decode":
        kp = torch.zeros(nb, Hkv, bs, 32, dtype=torch.uint8, device=DEV)
        vt = (torch.zeros(nb, Hkv, bs // 64, 512 * vb, dtype=torch.uint8, device=DEV) if bs >= 64 else
              torch.zeros(nb, Hkv, bs // 16, 128 * vb, dtype=torch.uint8, device=DEV))
        pairs = torch.empty(n * Hkv, 1, 32, dtype=torch.uint8, device=DEV)
        ops.pack_decode_layout(T(krows).view(n * Hkv, 1, 32), pairs, 64, 4, False, 0)
        capi.check(L().tq_paged_store(capi.p(pairs), capi.p(T(kn)), capi.i64(n), capi.i32(Hkv),
                                      capi.i32(32), capi.p(T(slots)), capi.p(kp), capi.p(knp),
                                      capi.i64(nb), capi.i32(bs), capi.stream()))
        capi.check(L().tq_paged_store_value_tiles(capi.p(T(vrows)), capi.p(T(vn)), capi.i64(n),
                                                  capi.i32(Hkv), capi.p(T(slots)), capi.p(vt),
                                                  capi.p(vnp), capi.i64(nb), capi.i32(bs), capi.i32(vb),
                                                  capi.stream()))
        ws = torch.empty(L().tq_decode_dl_workspace_bytes(B, Hq, Hkv, width * bs), dtype=torch.uint8,
                         device=DEV)
        print(f"paged decode past 2 GiB vb={vb} bs={bs}", flush=True)
        capi.check(L().tq_decode_attention_paged_dl(
            capi.p(q), capi.TQ_BF16, capi.i32(B), capi.i32(Hq), capi.i32(Hkv), capi.i32(64), capi.p(kp),
            capi.p(knp), capi.p(vt), capi.p(vnp), capi.i64(nb), capi.i32(bs), capi.i32(vb), capi.p(T(tab)),
            capi.i32(width), capi.p(lens_t), capi.p(T(ck)), capi.p(T(cv)), capi.p(T(Rk)), capi.p(T(Rv)),
            ctypes.c_float(scale), capi.p(out), capi.p(lse), capi.p(ws), ctypes.c_size_t(ws.numel()),
            capi.stream()))
        sync()
        got = out.float().cpu().numpy()
        del kp, vt
        kpairs = torch.empty(B * Hkv, Tc, 32, dtype=torch.uint8, device=DEV)
        vblocks = torch.zeros(B * Hkv, Tc // 64, 512 * vb, dtype=torch.uint8, device=DEV)
        ops.pack_decode_layout(T(kc_).view(B * Hkv, Tc, 32), kpairs, 64, 4, False, 0)
        ops.pack_decode_layout(T(vc_).view(B * Hkv, Tc, 8 * vb), vblocks, 64, vb, True, 0)
        ref, _ = ops.decode_attention_dl(q, kpairs.view(B, Hkv, Tc, 32), T(kn_),
                                         vblocks.view(B, Hkv, Tc // 64, 512 * vb), T(vn_), lens_t, T(ck),
                                         T(cv), T(Rk), T(Rv), scale, return_lse=True)
        ref = ref.float().cpu().numpy()
    else:
        kpool = torch.zeros(nb, Hkv, bs, 32, dtype=torch.uint8, device=DEV)
        vpool = torch.zeros(nb, Hkv, bs, 16, dtype=torch.uint8, device=DEV)
        for rows, norms, pool, npool in ((krows, kn, kpool, knp), (vrows, vn, vpool, vnp)):
            capi.check(L().tq_paged_store(capi.p(T(rows)), capi.p(T(norms)), capi.i64(n), capi.i32(Hkv),
                                          capi.i32(rows.shape[2]), capi.p(T(slots)), capi.p(pool),
                                          capi.p(npool), capi.i64(nb), capi.i32(bs), capi.stream()))
        wsb = L().tq_decode_paged_workspace_bytes(capi.TQ_BF16, B, Hq, Hkv, 64, 4, 2, width, bs)
        ws = torch.empty(max(wsb, 1), dtype=torch.uint8, device=DEV)
        capi.check(L().tq_decode_attention_paged(
            capi.p(q), capi.TQ_BF16, capi.i32(B), capi.i32(Hq), capi.i32(Hkv), capi.i32(64),
            capi.p(kpool), capi.p(knp), capi.p(vpool), capi.p(vnp), capi.i64(nb), capi.i32(bs),
            capi.p(T(tab)), capi.i32(width), capi.p(lens_t), capi.p(T(ck)), capi.p(T(cv)), capi.p(T(Rk)),
            capi.p(T(Rv)), capi.i32(4), capi.i32(2), ctypes.c_float(scale), capi.p(out), capi.p(lse),
            capi.p(ws), ctypes.c_size_t(ws.numel()), capi.stream()))
        sync()
        got = out.float().cpu().numpy()
        del kpool, vpool
        ref, _ = k_decode(q, kc_, kn_, vc_, vn_, lens, ck, cv, Rk, Rv, 4, 2, scale)
    del knp, vnp
    torch.cuda.empty_cache()
    assert np.array_equal(got, ref)  # same arithmetic and split plan as the contiguous kernel
    want = O.decode_attention_f64(q.float().cpu().numpy(), kc_, kn_, vc_, vn_, lens, ck, cv, Rk, Rv,
                                  4, vb, scale)
    assert np.max(np.abs(got - want)) <= 1e-2 * np.max(np.abs(want))
