"""GPU tests of the callers: the HF TurboQuantCache (transformers 5.x Cache API, plain and
fused-attention modes) and the vLLM attention step."""

import math

import numpy as np
import pytest
import torch

import tq_oracle as O

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _tiny_llama(seed=0, dtype=torch.float32):
    from transformers import LlamaConfig, LlamaForCausalLM
    torch.manual_seed(seed)
    cfg = LlamaConfig(hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                      num_attention_heads=8, num_key_value_heads=2, head_dim=64,
                      vocab_size=1000, max_position_embeddings=512, tie_word_embeddings=True)
    cfg._attn_implementation = "sdpa"
    return LlamaForCausalLM(cfg).to(DEV, dtype).eval()


def test_hf_update_returns_dequantized_history_plus_exact_new():
    from turboquant_kv import TurboQuantCache
    torch.manual_seed(0)
    cache = TurboQuantCache(key_bits=4, value_bits=2)
    k1, v1 = torch.randn(2, 2, 5, 64, device=DEV), torch.randn(2, 2, 5, 64, device=DEV)
    K, V = cache.update(k1, v1, 0)
    assert torch.equal(K, k1) and torch.equal(V, v1)          # empty history: exact
    k2, v2 = torch.randn(2, 2, 1, 64, device=DEV), torch.randn(2, 2, 1, 64, device=DEV)
    K, V = cache.update(k2, v2, 0)
    assert K.shape == (2, 2, 6, 64) and torch.equal(K[:, :, 5:], k2)
    layer = cache.layers[0]
    # stored codes equal the oracle's quantization of the history (outside the fp32 band)
    R = O.dense_qr_rotation(64, 42)
    bnd, cen = O.lloyd_max_codebook(4, 64)
    x = k1.reshape(-1, 64).cpu().numpy()
    _, _, codes = O.quantize_mse(x, 4, R, bnd)
    rows = layer.rows(False, 5).reshape(-1, 32).cpu().numpy()   # bit-plane rows
    got = O.unpack_codes(rows, 4, 64)
    O.check_codes(got, codes, x, R, bnd)
    deq = O.dequantize_mse(rows, layer.kn[:, :, :5].reshape(-1).float().cpu().numpy(), 4, 64, R, cen)
    assert np.allclose(K[:, :, :5].reshape(-1, 64).cpu().numpy(), deq, rtol=1e-5, atol=1e-5)
    assert cache.get_seq_length(0) == 6 and cache.memory_bytes() == 2 * 2 * 6 * (32 + 16 + 8)


def _tiny_llama_gqa4(seed=0, dtype=torch.float32):
    """Two layers, 16 query heads over 4 KV heads of 64 dims (the group size of the
    end-to-end config)."""
    from transformers import LlamaConfig, LlamaForCausalLM
    torch.manual_seed(seed)
    cfg = LlamaConfig(hidden_size=1024, intermediate_size=2048, num_hidden_layers=2,
                      num_attention_heads=16, num_key_value_heads=4, head_dim=64,
                      vocab_size=1000, max_position_embeddings=1024, tie_word_embeddings=True)
    cfg._attn_implementation = "sdpa"
    return LlamaForCausalLM(cfg).to(DEV, dtype).eval()


def test_hf_fused_decode_logits_match_reference_semantics():
    # A K4/V3 TurboQuantCache through a prefill of 512 tokens and three decode steps:
    # the fused steps (packed history by the decode kernel + exact new token by
    # log-sum-exp) against the reference's rule run by the general path (dequantized
    # history + exact new tokens, then SDPA).  fp32 model: the paths differ only in
    # summation order, so the logits agree tightly.
    from turboquant_kv import TurboQuantCache
    from turboquant_kv.hf_integration import enable_fused_attention
    model = _tiny_llama_gqa4()
    g = torch.Generator(DEV).manual_seed(1)
    ids = torch.randint(0, 1000, (4, 512), device=DEV, generator=g)
    nxt = torch.randint(0, 1000, (4, 3), device=DEV, generator=g)

    def run(fused):
        cache = TurboQuantCache(key_bits=4, value_bits=3, fused_attention=fused)
        if fused:
            enable_fused_attention(model)
        else:
            model.set_attn_implementation("sdpa")
        logits = []
        with torch.no_grad():
            model(input_ids=ids, past_key_values=cache, use_cache=True)
            for i in range(3):
                out = model(input_ids=nxt[:, i:i + 1], past_key_values=cache, use_cache=True)
                logits.append(out.logits[:, -1].float())
        return torch.stack(logits), cache

    ref, c_ref = run(False)
    got, c_got = run(True)
    assert c_got.layers[0].dl and c_got.get_seq_length(0) == 515
    err = ((got - ref).abs().amax(-1) / ref.abs().amax(-1)).max().item()
    assert err <= 1e-3, err
    # cache bytes: 4-bit keys + 3-bit values + two fp32 norms per (token, kv head)
    assert c_got.memory_bytes() == 2 * 4 * 4 * 515 * (32 + 24 + 8)
    with torch.no_grad():
        out = model.generate(ids[:, :40], past_key_values=TurboQuantCache(4, 3, fused_attention=True),
                             max_new_tokens=6, do_sample=False)
    assert out.shape == (4, 46)


def test_hf_fused_decode_left_padded_generate():
    # generate() on a left-padded batch (prompts of 300, 211, 40 and 299 tokens): every
    # decode step carries an attention mask.  The fused steps (decode-layout kernel over
    # each sequence's window after its padding + the exact new token) against the
    # reference's rule run by the general path (dequantized history + SDPA with the mask):
    # per-step logits within 1e-3 of the maximum, the same greedy tokens.
    from turboquant_kv import TurboQuantCache
    from turboquant_kv.hf_integration import enable_fused_attention
    model = _tiny_llama_gqa4()
    g = torch.Generator(DEV).manual_seed(3)
    lens = [300, 211, 40, 299]
    L_ = max(lens)
    ids = torch.randint(1, 1000, (4, L_), device=DEV, generator=g)
    mask = torch.zeros(4, L_, dtype=torch.long, device=DEV)
    for b, n in enumerate(lens):
        ids[b, :L_ - n] = 0
        mask[b, L_ - n:] = 1

    def run(fused):
        if fused:
            enable_fused_attention(model)
        else:
            model.set_attn_implementation("sdpa")
        cache = TurboQuantCache(key_bits=4, value_bits=3, fused_attention=fused)
        with torch.no_grad():
            out = model.generate(input_ids=ids, attention_mask=mask, past_key_values=cache,
                                 max_new_tokens=5, do_sample=False, output_scores=True,
                                 return_dict_in_generate=True, pad_token_id=0)
        return out.sequences, torch.stack([s.float() for s in out.scores]), cache

    seq_ref, sc_ref, _ = run(False)
    seq_got, sc_got, cache = run(True)
    assert cache.layers[0].dl
    err = ((sc_got - sc_ref).abs().amax(-1) / sc_ref.abs().amax(-1)).max().item()
    assert err <= 1e-3, err
    assert torch.equal(seq_got, seq_ref)


def test_hf_window_starts_from_masks():
    # The mask -> window reading: left padding gives the first attended position; a hole in
    # the middle, a masked current token or a fully masked row give None (general path).
    from turboquant_kv.hf_integration import _window_starts
    m = torch.ones(3, 1, 1, 9, dtype=torch.bool, device=DEV)
    m[1, ..., :4] = False
    m[2, ..., :8] = False
    assert _window_starts(m, 3, 8).tolist() == [0, 4, 8]
    f = torch.zeros(3, 1, 1, 9, device=DEV)
    f[1, ..., :4] = float("-inf")
    assert _window_starts(f, 3, 8).tolist() == [0, 4, 0]
    h = m.clone()
    h[0, ..., 5] = False
    assert _window_starts(h, 3, 8) is None
    c = m.clone()
    c[0, ..., 8] = False
    assert _window_starts(c, 3, 8) is None
    assert _window_starts(m, 3, 9) is None  # a mask of another length


@pytest.mark.parametrize("vb,G", [(3, 4), (2, 4), (4, 2), (3, 8)])
def test_hf_fused_decode_step_vs_f64(vb, G):
    # One decode step of a bf16 layer: the attention function's output against float64
    # attention over the stored history (dequantized from the cache's own rows) followed
    # by the exact new token -- the reference's update rule (hf_integration.py:372-390)
    # and SDPA, with GQA (query head h reads KV head h // G).
    from turboquant_kv import TurboQuantCache
    from turboquant_kv.hf_integration import turboquant_attention
    torch.manual_seed(10 * vb + G)
    B, Hkv, d, T = 4, 4, 64, 512
    Hq = G * Hkv
    cache = TurboQuantCache(key_bits=4, value_bits=vb, fused_attention=True)
    k0 = (torch.randn(B, Hkv, T, d, device=DEV) * 2).to(torch.bfloat16)
    v0 = torch.randn(B, Hkv, T, d, device=DEV).to(torch.bfloat16)
    cache.update(k0, v0, 0)
    k1 = torch.randn(B, Hkv, 1, d, device=DEV).to(torch.bfloat16)
    v1 = torch.randn(B, Hkv, 1, d, device=DEV).to(torch.bfloat16)
    q = torch.randn(B, Hq, 1, d, device=DEV).to(torch.bfloat16)
    K, V = cache.update(k1, v1, 0)

    class M:
        layer_idx = 0
    got, _ = turboquant_attention(M(), q, K, V, None, scaling=1 / 8)
    got = got.float().cpu().numpy()[:, 0]                       # [B, Hq, d]
    layer = cache.layers[0]
    assert layer.dl
    # a bf16 model's cache keeps bf16 norms, counted as the reference counts them
    assert layer.kn.dtype == torch.bfloat16 and layer.vn.dtype == torch.bfloat16
    assert cache.memory_bytes() == B * Hkv * (T + 1) * (32 + 8 * vb + 2 * 2)
    Rk, Rv = O.dense_qr_rotation(d, 42), O.dense_qr_rotation(d, 43)
    _, ck = O.lloyd_max_codebook(4, d)
    _, cv = O.lloyd_max_codebook(vb, d)
    kr = layer.rows(False, T).cpu().numpy()
    vr = layer.rows(True, T).cpu().numpy()
    kn = layer.kn[:, :, :T].float().cpu().numpy()
    vn = layer.vn[:, :, :T].float().cpu().numpy()
    qf = q.float().cpu().numpy()[:, :, 0].astype(np.float64)
    k1f = k1.float().cpu().numpy()[:, :, 0].astype(np.float64)
    v1f = v1.float().cpu().numpy()[:, :, 0].astype(np.float64)
    want = np.zeros((B, Hq, d))
    for b in range(B):
        for g in range(Hkv):
            Kh = O.dequantize_mse(kr[b, g], kn[b, g], 4, d, Rk, ck).astype(np.float64)
            Vh = O.dequantize_mse(vr[b, g], vn[b, g], vb, d, Rv, cv).astype(np.float64)
            Ka = np.concatenate([Kh, k1f[b, g][None]])
            Va = np.concatenate([Vh, v1f[b, g][None]])
            for h in range(g * G, (g + 1) * G):
                s = Ka @ qf[b, h] / 8
                p = np.exp(s - s.max())
                want[b, h] = (p / p.sum()) @ Va
    err = np.max(np.abs(got - want), axis=-1) / np.max(np.abs(want), axis=-1)
    assert err.max() <= 1e-2, err.max()


def test_hf_fused_step_matches_plain_step():
    from turboquant_kv import TurboQuantCache
    from turboquant_kv.hf_integration import turboquant_attention
    torch.manual_seed(3)
    B, Hq, Hkv, d = 2, 8, 2, 64
    plain, fused = TurboQuantCache(4, 2), TurboQuantCache(4, 2, fused_attention=True)
    k0, v0 = torch.randn(B, Hkv, 300, d, device=DEV), torch.randn(B, Hkv, 300, d, device=DEV)
    plain.update(k0, v0, 0)
    fused.update(k0, v0, 0)
    k1, v1 = torch.randn(B, Hkv, 1, d, device=DEV), torch.randn(B, Hkv, 1, d, device=DEV)
    q = torch.randn(B, Hq, 1, d, device=DEV)
    Kp, Vp = plain.update(k1, v1, 0)
    Kf, Vf = fused.update(k1, v1, 0)

    class M:
        layer_idx = 0
    ref, _ = turboquant_attention(M(), q, Kp, Vp, None, scaling=1 / 8)
    got, _ = turboquant_attention(M(), q, Kf, Vf, None, scaling=1 / 8)
    assert (got - ref).abs().max().item() <= 1e-4 * ref.abs().max().item()


def test_vllm_attention_step_gqa():
    from turboquant_kv.vllm_plugin import (TurboQuantAttentionBackend, TurboQuantKVCacheConfig,
                                           TurboQuantPagedKVCache, attention_step, register)
    register()
    assert TurboQuantAttentionBackend.get_name() == "turboquant"
    assert TurboQuantAttentionBackend.get_kv_cache_shape(10, 16, 8, 64) == (2, 10, 16, 8, 64)
    torch.manual_seed(4)
    cfg = TurboQuantKVCacheConfig(key_bits=4, value_bits=2, num_gpu_blocks=64, block_size=16)
    kv = TurboQuantPagedKVCache(cfg, num_layers=1, num_heads=2, head_dim=64, device=DEV)
    kv2 = TurboQuantPagedKVCache(cfg, num_layers=1, num_heads=2, head_dim=64, device=DEV)
    q0, k0, v0 = (torch.randn(20, 8, 64, device=DEV), torch.randn(20, 2, 64, device=DEV),
                  torch.randn(20, 2, 64, device=DEV))
    attention_step(q0, k0, v0, kv, 0, 0.125)
    attention_step(q0, k0, v0, kv2, 0, 0.125)
    q1, k1, v1 = (torch.randn(1, 8, 64, device=DEV), torch.randn(1, 2, 64, device=DEV),
                  torch.randn(1, 2, 64, device=DEV))
    fused = attention_step(q1, k1, v1, kv, 0, 0.125)              # single token: fused kernel
    kv2.append(0, k1.transpose(0, 1), v1.transpose(0, 1))
    c = kv2._cache
    logits = c.attention_scores(0, q1.transpose(0, 1)) * (0.125 * 8)
    ref = c.attention_values(0, torch.softmax(logits, -1)).transpose(0, 1)
    assert (fused - ref).abs().max().item() <= 1e-4 * ref.abs().max().item()
    assert kv.get_seq_length(0) == 21 and kv.memory_bytes() > 0


@pytest.mark.parametrize("dt,kvdt", [(torch.float32, torch.float32), (torch.bfloat16, torch.bfloat16),
                                      (torch.float16, torch.bfloat16)])
def test_decode_merge_token_vs_float64(dt, kvdt):
    """tq_decode_merge_token against the log-sum-exp merge of hf_integration.py:372-390 in
    float64, including a row whose history is empty (lse = -inf: the output is v_new) and
    queries that dominate either side."""
    from turboquant_kv._lib import ops
    g = torch.Generator(device="cuda").manual_seed(3)
    B, Hq, Hkv, d, scale = 3, 8, 2, 64, 0.125
    q = torch.randn(B, Hq, d, generator=g, device="cuda").to(dt)
    o = torch.randn(B, Hq, d, generator=g, device="cuda").to(dt)
    lse = torch.randn(B, Hq, generator=g, device="cuda") * 4
    lse[0, 1] = -math.inf
    k = (torch.randn(B, Hkv, d, generator=g, device="cuda") * 3).to(kvdt)
    v = torch.randn(B, Hkv, d, generator=g, device="cuda").to(kvdt)
    out = ops().decode_merge_token(o, lse, q, k, v, scale)
    assert out.dtype == dt and out.shape == (B, Hq, d)
    G = Hq // Hkv
    kd = k.double().repeat_interleave(G, 1)
    vd = v.double().repeat_interleave(G, 1)
    s = (q.double() * kd).sum(-1) * scale
    m = torch.maximum(lse.double(), s)
    wh, wn = torch.exp(lse.double() - m), torch.exp(s - m)
    want = (o.double() * wh[..., None] + vd * wn[..., None]) / (wh + wn)[..., None]
    tol = 1e-5 if dt == torch.float32 else (1e-2 if dt == torch.bfloat16 else 2e-3)
    err = (out.double() - want).abs().max().item()
    assert err <= tol * want.abs().max().item(), err
    assert torch.allclose(out[0, 1].double(), vd[0, 1], rtol=tol, atol=tol)


@pytest.mark.parametrize("dt", [torch.bfloat16, torch.float32])
def test_decode_attention_dl_merged_equals_two_ops(dt):
    """decode_attention_dl_merged (the HF decode step's one op) equals
    decode_attention_dl_lse followed by decode_merge_token bit for bit, with and without
    window starts."""
    from turboquant_kv._lib import ops
    rs = np.random.RandomState(8)
    g = torch.Generator(device="cuda").manual_seed(8)
    B, Hq, Hkv, d, Tc, vb, scale = 3, 8, 2, 64, 256, 3, 0.125
    kp = torch.randint(0, 256, (B, Hkv, Tc, d // 2), dtype=torch.uint8, device="cuda", generator=g)
    vp = torch.randint(0, 256, (B, Hkv, Tc // 64, 8 * vb * d), dtype=torch.uint8, device="cuda",
                       generator=g)
    kn = torch.rand(B, Hkv, Tc, device="cuda", generator=g) + 0.5
    vn = torch.rand(B, Hkv, Tc, device="cuda", generator=g) + 0.5
    R = torch.from_numpy(O.dense_qr_rotation(d, 42)).cuda()
    _, kc = O.lloyd_max_codebook(4, d)
    _, vc = O.lloyd_max_codebook(vb, d)
    kc, vc = torch.from_numpy(kc).cuda(), torch.from_numpy(vc).cuda()
    seq = torch.tensor([200, 1, 256], dtype=torch.int32, device="cuda")
    q = torch.randn(B, Hq, d, generator=g, device="cuda").to(dt)
    kv_new = [torch.randn(B, Hkv, d, generator=g, device="cuda").to(dt) for _ in range(2)]
    for starts in (None, torch.tensor([3, 0, 70], dtype=torch.int32, device="cuda")):
        o, lse = ops().decode_attention_dl_lse(q, kp, kn, vp, vn, seq, kc, vc, R, R, scale, starts)
        want = ops().decode_merge_token(o, lse, q, kv_new[0], kv_new[1], scale)
        got = ops().decode_attention_dl_merged(q, kp, kn, vp, vn, seq, kc, vc, R, R, scale, starts,
                                               kv_new[0], kv_new[1])
        assert got.dtype == want.dtype and torch.equal(got, want)
