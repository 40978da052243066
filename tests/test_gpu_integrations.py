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
    got = O.unpack_codes(layer.kp[:, :, :5].reshape(-1, 32).cpu().numpy(), 4, 64)
    assert not ((got != codes) & ~O.code_margin(x, R, bnd)).any()
    deq = O.dequantize_mse(layer.kp[:, :, :5].reshape(-1, 32).cpu().numpy(),
                           layer.kn[:, :, :5].reshape(-1).cpu().numpy(), 4, 64, R, cen)
    assert np.allclose(K[:, :, :5].reshape(-1, 64).cpu().numpy(), deq, rtol=1e-5, atol=1e-5)
    assert cache.get_seq_length(0) == 6 and cache.memory_bytes() == 2 * 2 * 6 * (32 + 16 + 8)


def test_hf_generate_plain_and_fused_agree():
    from turboquant_kv import TurboQuantCache
    from turboquant_kv.hf_integration import enable_fused_attention
    model = _tiny_llama()
    ids = torch.randint(0, 1000, (2, 40), device=DEV, generator=torch.Generator(DEV).manual_seed(1))
    with torch.no_grad():
        plain = model.generate(ids, past_key_values=TurboQuantCache(key_bits=4, value_bits=4),
                               max_new_tokens=12, do_sample=False)
        enable_fused_attention(model)
        fused = model.generate(ids, past_key_values=TurboQuantCache(key_bits=4, value_bits=4,
                                                                     fused_attention=True),
                               max_new_tokens=12, do_sample=False)
    assert plain.shape == fused.shape == (2, 52)
    # Same prompt handling; decode steps differ only by fp32 summation order.
    agree = (plain[:, 40:] == fused[:, 40:]).float().mean().item()
    assert agree >= 0.9, agree


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
