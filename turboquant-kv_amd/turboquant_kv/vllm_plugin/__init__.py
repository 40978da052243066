"""TurboQuant vLLM out-of-tree plugin (API of turboquant_kv/vllm_plugin/__init__.py:1-528).

Same classes and entry point as the reference: TurboQuantKVCacheConfig,
TurboQuantPagedKVCache, TurboQuantAttentionImpl, TurboQuantAttentionBackend, register().
When vLLM is not installed the attention classes derive from stub bases and
TurboQuantAttentionImpl refuses construction, as the reference does (vllm_plugin:35-59,
340-345); the cache and the attention step itself (`attention_step`) work without vLLM.

Differences from the reference, all on the compute side: the cache lives in packed
device storage and is read by the HIP kernels (no per-step dequantization); query heads
may be a multiple of the KV heads (grouped-query attention, which the reference cannot
express, cache.py:294-307); a single-token step runs the fused decode kernel.

Paged operation (what vLLM's cache engine and scheduler provide, which the reference's
backend ignores): TurboQuantPagedKVCache.pools() holds K/V in block pools
(vllm_plugin/paged.py), and TurboQuantAttentionImpl.forward with metadata that carries
`block_tables` and `slot_mapping` stores the new tokens at their slots, runs causal
prefill per prefill sequence and one paged decode launch for the decode sequences.
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Any, Dict, List, Optional, Tuple, Type

import torch

from turboquant_kv.cache import QuantizedKVCache
from turboquant_kv.config import TurboQuantConfig
from turboquant_kv.vllm_plugin.paged import PagedKVPools, TurboQuantAttentionMetadata

_VLLM_AVAILABLE = False
try:  # pragma: no cover - vLLM is not installed in this image
    from vllm.attention.backends.abstract import (AttentionBackend, AttentionImpl,
                                                  AttentionMetadata, AttentionType)
    _VLLM_AVAILABLE = True
except ImportError:
    class AttentionBackend:  # type: ignore[no-redef]
        pass

    class AttentionImpl:  # type: ignore[no-redef]
        pass

    class AttentionMetadata:  # type: ignore[no-redef]
        pass

    class AttentionType:  # type: ignore[no-redef]
        pass


@dataclass
class TurboQuantKVCacheConfig:
    """vLLM-side configuration (vllm_plugin:67-106)."""

    key_bits: int = 4
    value_bits: int = 2
    mode: str = "mse"
    rotation: str = "dense_qr"
    block_size: int = 16
    num_gpu_blocks: int = 0
    num_cpu_blocks: int = 0
    protected_layers: int = 0
    seed: int = 42
    # block pool layout: "bitplane", "decode" (the MFMA decode kernel's layout: mse, 4-bit
    # keys, 2-4 bit values, head_dim 64, power-of-two block_size >= 16) or "auto" (decode
    # where it applies)
    pool_layout: str = "auto"

    def to_turboquant_config(self) -> TurboQuantConfig:
        return TurboQuantConfig(key_bits=self.key_bits, value_bits=self.value_bits, mode=self.mode,
                                rotation=self.rotation, protected_layers=self.protected_layers,
                                quantize_on_append=True, seed=self.seed)


class TurboQuantPagedKVCache:
    """Packed KV storage sized in vLLM blocks (vllm_plugin:114-304): capacity
    num_gpu_blocks * block_size tokens per layer, backed by a QuantizedKVCache."""

    def __init__(self, config: TurboQuantKVCacheConfig, num_layers: int, num_heads: int,
                 head_dim: int, dtype: torch.dtype = torch.float16, device: str = "cuda") -> None:
        self.config = config
        self.tq_config = config.to_turboquant_config()
        self.num_layers = num_layers
        self.num_heads = num_heads
        self.head_dim = head_dim
        self.dtype = dtype
        self.device = torch.device(device)
        self.block_size = config.block_size
        self._total_blocks = config.num_gpu_blocks
        self._max_tokens = self._total_blocks * self.block_size
        # The single-sequence cache of the reference's API (append / attention_scores /
        # attention_values) and the paged pools are each built on first use.
        self._cache: Optional[QuantizedKVCache] = None
        self._pools: Optional[PagedKVPools] = None
        self._block_offsets: Dict[int, List[int]] = {}

    def allocate(self, num_layers: int, num_heads: int, head_dim: int, num_gpu_blocks: int,
                 num_cpu_blocks: int, dtype: torch.dtype, device: str) -> None:
        self.config.num_gpu_blocks = num_gpu_blocks
        self.config.num_cpu_blocks = num_cpu_blocks
        self._total_blocks = num_gpu_blocks
        self._max_tokens = num_gpu_blocks * self.block_size
        self.num_layers, self.num_heads, self.head_dim = num_layers, num_heads, head_dim
        self.dtype, self.device = dtype, torch.device(device)
        self._cache = QuantizedKVCache(self.tq_config, num_layers, self._max_tokens, num_heads,
                                       head_dim, device=device)
        self._pools = None

    def _require(self) -> QuantizedKVCache:
        if self._cache is None:
            if self._max_tokens <= 0:
                raise RuntimeError("TurboQuantPagedKVCache has not been allocated. Call allocate() first.")
            self._cache = QuantizedKVCache(self.tq_config, self.num_layers, self._max_tokens,
                                           self.num_heads, self.head_dim, device=self.device)
        return self._cache

    def pools(self) -> PagedKVPools:
        """The block pools: num_gpu_blocks blocks of block_size tokens per layer."""
        if self._pools is None:
            if self._total_blocks <= 0:
                raise RuntimeError("TurboQuantPagedKVCache has no blocks. Call allocate() first.")
            layout = self.config.pool_layout
            if layout == "auto":
                layout = ("decode" if PagedKVPools.decode_layout_supported(
                    self.tq_config, self.head_dim, self.block_size) else "bitplane")
            self._pools = PagedKVPools(self.tq_config, self.num_layers, self._total_blocks,
                                       self.block_size, self.num_heads, self.head_dim, self.device,
                                       layout=layout)
        return self._pools

    def append(self, layer_id: int, key: torch.Tensor, value: torch.Tensor) -> None:
        self._require().append(layer_id, key, value)

    def get_keys(self, layer_id: int) -> torch.Tensor:
        if self._cache is None:
            return torch.zeros(self.num_heads, 0, self.head_dim, dtype=torch.float32, device=self.device)
        return self._cache._dequantize_keys(layer_id)

    def get_values(self, layer_id: int) -> torch.Tensor:
        if self._cache is None:
            return torch.zeros(self.num_heads, 0, self.head_dim, dtype=torch.float32, device=self.device)
        return self._cache._dequantize_values(layer_id)

    def attention_scores(self, layer_id: int, query: torch.Tensor) -> torch.Tensor:
        return self._require().attention_scores(layer_id, query)

    def attention_values(self, layer_id: int, attn_weights: torch.Tensor) -> torch.Tensor:
        return self._require().attention_values(layer_id, attn_weights)

    def get_seq_length(self, layer_id: int) -> int:
        return 0 if self._cache is None else int(self._cache.seq_lens[layer_id].item())

    def memory_bytes(self) -> int:
        """Packed bytes of the single-sequence cache (the reference's count); with pools
        allocated, their bytes are added."""
        n = 0 if self._cache is None else self._cache.memory_bytes()
        return n + (0 if self._pools is None else self._pools.memory_bytes())

    @property
    def compression_ratio(self) -> float:
        return 0.0 if self._cache is None else self._cache.compression_ratio


def attention_step(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                   kv_cache: TurboQuantPagedKVCache, layer_id: int, scale: float,
                   output: Optional[torch.Tensor] = None) -> torch.Tensor:
    """One attention step through the packed cache (the body of vllm_plugin:350-412):
    append the new K/V, then softmax(q K^T * scale) V over everything cached.
    query (num_tokens, Hq, d); key/value (num_tokens, Hkv, d) -> (num_tokens, Hq, d)."""
    kv_cache.append(layer_id, key.transpose(0, 1), value.transpose(0, 1))
    cache = kv_cache._require()
    num_tokens = query.shape[0]
    if num_tokens == 1 and not cache._is_prod and not cache._is_protected_layer(layer_id):
        out = cache.decode_attention(layer_id, query, scale=scale)        # (1, Hq, d)
        out = out.to(query.dtype)
    else:
        q = query.transpose(0, 1)                                       # (Hq, Nt, d)
        logits = cache.attention_scores(layer_id, q) * (scale * math.sqrt(cache.head_dim))
        attn = torch.softmax(logits, dim=-1)
        out = cache.attention_values(layer_id, attn).transpose(0, 1).to(query.dtype)
    if output is not None:
        output.copy_(out.reshape(output.shape))
        return output
    return out


class TurboQuantAttentionImpl(AttentionImpl):
    """vLLM attention implementation over a TurboQuantPagedKVCache (vllm_plugin:312-412)."""

    def __init__(self, num_heads: int, head_dim: int, scale: float, num_kv_heads: int,
                 alibi_slopes: Optional[List[float]] = None, sliding_window: Optional[int] = None,
                 kv_cache_dtype: str = "turboquant", blocksparse_params: Optional[Dict[str, Any]] = None,
                 logits_soft_cap: Optional[float] = None, **kwargs: Any) -> None:
        if not _VLLM_AVAILABLE:
            raise ImportError("vLLM is required for TurboQuantAttentionImpl. Install with: pip install vllm")
        super().__init__()  # pragma: no cover
        self.num_heads = num_heads
        self.head_dim = head_dim
        self.scale = scale
        self.num_kv_heads = num_kv_heads
        self.alibi_slopes = alibi_slopes
        self.sliding_window = sliding_window
        self.logits_soft_cap = logits_soft_cap

    def forward(self, query, key, value, kv_cache: TurboQuantPagedKVCache, attn_metadata,
                k_scale: float = 1.0, v_scale: float = 1.0, attn_type: Any = None,
                output: Optional[torch.Tensor] = None, **kwargs: Any) -> torch.Tensor:  # pragma: no cover
        if getattr(attn_metadata, "block_tables", None) is not None:
            return kv_cache.pools().forward(query, key, value, attn_metadata, self.scale, output)
        layer_id: int = getattr(attn_metadata, "layer_id", 0)
        return attention_step(query, key, value, kv_cache, layer_id, self.scale, output)


class TurboQuantAttentionBackend(AttentionBackend):
    """vLLM backend entry (vllm_plugin:420-458)."""

    @staticmethod
    def get_name() -> str:
        return "turboquant"

    @staticmethod
    def get_impl_cls() -> Type[TurboQuantAttentionImpl]:
        return TurboQuantAttentionImpl

    @staticmethod
    def get_metadata_cls() -> Type[AttentionMetadata]:
        return AttentionMetadata

    @staticmethod
    def get_kv_cache_shape(num_blocks: int, block_size: int, num_kv_heads: int,
                           head_size: int) -> Tuple[int, ...]:
        # logical shape for vLLM's bookkeeping (vllm_plugin:440-453)
        return (2, num_blocks, block_size, num_kv_heads, head_size)

    @staticmethod
    def get_supported_head_sizes() -> List[int]:
        return [32, 64, 96, 128, 160, 192, 224, 256]


_REGISTERED = False


def register() -> None:
    """vLLM general-plugin entry point; idempotent; a no-op without vLLM (vllm_plugin:469-515)."""
    global _REGISTERED
    if _REGISTERED or not _VLLM_AVAILABLE:
        return
    try:  # pragma: no cover
        from vllm.attention import selector as _selector
        if hasattr(_selector, "register_backend"):
            _selector.register_backend("turboquant", TurboQuantAttentionBackend)
    except (ImportError, AttributeError):  # pragma: no cover
        pass
    _REGISTERED = True


def paged_attention_step(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                         kv_cache: TurboQuantPagedKVCache, metadata: TurboQuantAttentionMetadata,
                         scale: float, output: Optional[torch.Tensor] = None) -> torch.Tensor:
    """TurboQuantAttentionImpl.forward on paged metadata, callable without vLLM."""
    return kv_cache.pools().forward(query, key, value, metadata, scale, output)


__all__ = ["TurboQuantKVCacheConfig", "TurboQuantPagedKVCache", "TurboQuantAttentionBackend",
           "TurboQuantAttentionImpl", "TurboQuantAttentionMetadata", "PagedKVPools",
           "attention_step", "paged_attention_step", "register"]
