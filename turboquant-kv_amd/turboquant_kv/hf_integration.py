"""HuggingFace Transformers integration: TurboQuantCache (API of hf_integration.py:272-555).

Targets the layer-based Cache of transformers 5.x: each transformer layer gets a
`TurboQuantLayer` holding packed device storage + fp32 norms [B, H_kv, capacity] that
grows geometrically; every `update` quantizes all (batch, head, token) rows of the new
states in one kernel launch (the reference loops over batch items and heads in Python,
hf_integration.py:370-415).  MSE caches with 4-bit keys, 2-4 bit values and head_dim 64 or
128 (the default K4/V2 and the K4/V3 of the end-to-end config) keep their codes in the
decode layout -- key pair bytes [B, H_kv, capacity, d/2], 64-token value tiles [B, H_kv,
capacity/64, 8*value_bits*d] -- that the fused decode kernel streams; other shapes keep
the reference's bit-plane rows [B, H_kv, capacity, P].

Semantics kept from the reference (hf_integration.py:319-421):
  * protected layers (index < protected_layers) keep exact K/V;
  * an update returns the dequantized history followed by the *exact* new tokens, so
    the current token carries no quantization error;
  * keys use `seed`, values `seed + 1`; prod mode uses the (bits-1)-bit codebook and
    QJL matrices seeded `seed + 12345` / `seed + 1 + 12345`.

Fused attention (new): construct the cache with `fused_attention=True` and run the model
with `attn_implementation="turboquant"` (registered here; see `enable_fused_attention`).
Updates then return only the new tokens, and the attention function attends to the
packed history with the fused decode kernel, merging the exact new token by log-sum-exp
-- no dequantized copy of the history is materialized.  Single-token MSE steps without
an attention mask run it (decode-layout storage: any number of query heads per KV head;
bit-plane rows: the shapes tq_decode_attention_packed fuses, else its split kernels);
prefill chunks, masked steps and prod-mode storage take the general path (dequantize the
history, then SDPA), which has the reference's numerics.
"""

from __future__ import annotations

import math
import threading
from typing import Any, Dict, List, Optional, Tuple

import torch

from turboquant_kv import ops
from turboquant_kv._lib import ops as _ops
from turboquant_kv.codebook import lloyd_max_codebook, make_qjl_matrix, make_rotation_matrix
from turboquant_kv.config import TurboQuantConfig

try:
    from transformers.cache_utils import Cache as _HFCache, CacheLayerMixin as _HFLayer
    from transformers import AttentionInterface as _AttnIf
    _TRANSFORMERS_AVAILABLE = True
except ImportError:  # pragma: no cover - transformers is installed in this image
    _HFCache, _HFLayer, _AttnIf = object, object, None
    _TRANSFORMERS_AVAILABLE = False

_PENDING = threading.local()


def _pending() -> Dict[int, Any]:
    if not hasattr(_PENDING, "d"):
        _PENDING.d = {}
    return _PENDING.d


class _Quantizer:
    """Device-resident rotation / codebook / QJL state of one of K or V."""

    def __init__(self, head_dim: int, bits: int, seed: int, cfg: TurboQuantConfig, device):
        self.prod = cfg.mode == "prod"
        self.bits = bits
        self.code_bits = bits - 1 if self.prod else bits
        self.d = head_dim
        self.R = make_rotation_matrix(head_dim, seed=seed, method=cfg.rotation).to(device)
        bnd, cen = lloyd_max_codebook(self.code_bits, head_dim)
        self.bnd, self.cen = bnd.to(device), cen.to(device)
        self.S = make_qjl_matrix(head_dim, head_dim, seed, device) if self.prod else None

    def quantize(self, flat: torch.Tensor):
        if self.prod:
            return _ops().quantize_prod_packed(flat, self.R, self.bnd, self.cen, self.S, self.bits)
        return _ops().quantize_mse_packed(flat, self.R, self.bnd, self.bits)

    def dequantize(self, packed, norms, signs=None, res=None, dtype=torch.float32):
        if self.prod:
            out = _ops().dequantize_prod_packed(packed, signs, res, norms.float(), self.cen, self.R,
                                                self.S, self.bits, self.d)
            return out.to(dtype)
        return _ops().dequantize_mse_packed(packed, norms.to(dtype), self.cen, self.R, self.bits,
                                            self.d)


class TurboQuantLayer(_HFLayer):
    """Packed KV storage of one transformer layer."""

    is_sliding = False
    is_compileable = False

    def __init__(self, tq_config: TurboQuantConfig, protected: bool = False,
                 fused_attention: bool = False):
        if _TRANSFORMERS_AVAILABLE:
            super().__init__()
        else:
            self.keys = self.values = None
            self.is_initialized = False
        self.tq_config = tq_config
        self.protected = protected
        self.fused_attention = fused_attention and not protected
        self.seq_len = 0
        self.cap = 0
        self.dl = False

    # ------------------------------------------------------------ storage
    def lazy_initialization(self, key_states: torch.Tensor, value_states: torch.Tensor) -> None:
        self.dtype, self.device = key_states.dtype, key_states.device
        B, H, _, d = key_states.shape
        self.batch, self.num_heads, self.head_dim = B, H, d
        if self.protected:
            self.keys = key_states.new_zeros(B, H, 0, d)
            self.values = value_states.new_zeros(B, H, 0, d)
        else:
            cfg = self.tq_config
            self.kq = _Quantizer(d, cfg.key_bits, cfg.seed, cfg, self.device)
            self.vq = _Quantizer(d, cfg.value_bits, cfg.seed + 1, cfg, self.device)
            self.keys = self.values = None
            # decode layout: mse, 4-bit keys, 2-4 bit values, head_dim 64 or 128
            self.dl = (not self.kq.prod and self.kq.code_bits == 4 and
                       2 <= self.vq.code_bits <= 4 and d in (64, 128))
            # norms in the model's dtype for 16-bit models, as the reference's cache keeps
            # them (quantize returns them in the input dtype; hf_integration.py:512-525
            # counts them so); the decode-layout kernel reads 16-bit norms directly.  Other
            # layouts keep fp32 norms for their kernels.
            self.norm_dtype = (self.dtype if self.dl and self.dtype in (torch.bfloat16, torch.float16)
                               else torch.float32)
        self.is_initialized = True

    def _grow(self, need: int) -> None:
        if need <= self.cap:
            return
        cap = max(need, 2 * self.cap, 256)
        if self.dl:
            cap = (cap + 63) // 64 * 64  # whole 64-token value tiles
        B, H, d = self.batch, self.num_heads, self.head_dim
        bpp = (d + 7) // 8
        dev = self.device
        prod = self.kq.prod

        def grown(old, *tail, dtype, per_tile=False):
            n = cap // 64 if per_tile else cap
            t = torch.zeros(B, H, n, *tail, dtype=dtype, device=dev)
            used = (self.seq_len + 63) // 64 if per_tile else self.seq_len
            if old is not None and used:
                t[:, :, :used] = old[:, :, :used]
            return t

        if self.dl:
            self.kp = grown(getattr(self, "kp", None), d // 2, dtype=torch.uint8)
            self.vp = grown(getattr(self, "vp", None), 8 * self.vq.code_bits * d, dtype=torch.uint8,
                            per_tile=True)
        else:
            self.kp = grown(getattr(self, "kp", None), self.kq.code_bits * bpp, dtype=torch.uint8)
            self.vp = grown(getattr(self, "vp", None), self.vq.code_bits * bpp, dtype=torch.uint8)
        self.kn = grown(getattr(self, "kn", None), dtype=self.norm_dtype)
        self.vn = grown(getattr(self, "vn", None), dtype=self.norm_dtype)
        if prod:
            self.ks = grown(getattr(self, "ks", None), bpp, dtype=torch.uint8)
            self.vs = grown(getattr(self, "vs", None), bpp, dtype=torch.uint8)
            self.kr = grown(getattr(self, "kr", None), dtype=torch.float32)
            self.vr = grown(getattr(self, "vr", None), dtype=torch.float32)
        self.cap = cap

    def _append(self, key_states, value_states) -> None:
        B, H, s, d = key_states.shape
        self._grow(self.seq_len + s)
        if self.dl and not self.kq.prod:  # K and V quantized, packed and stored in one op
            _ops().cache_append_dl(key_states, value_states, self.kp, self.kn, self.vp, self.vn,
                                   self.seq_len, self.kq.R, self.kq.bnd, self.vq.R, self.vq.bnd,
                                   self.kq.bits, self.vq.bits)
            self.seq_len += s
            return
        sl = slice(self.seq_len, self.seq_len + s)
        for vals, (q, x, p, n, sg, rs) in enumerate(
                ((self.kq, key_states, self.kp, self.kn, "ks", "kr"),
                 (self.vq, value_states, self.vp, self.vn, "vs", "vr"))):
            out = q.quantize(x.reshape(-1, d))
            if self.dl:
                _ops().pack_decode_layout(out[0].view(B * H, s, -1), p.view(B * H, p.shape[2], -1),
                                          d, q.code_bits, vals, self.seq_len)
            else:
                p[:, :, sl] = out[0].view(B, H, s, -1)
            n[:, :, sl].copy_(out[-1].view(B, H, s))  # one cast-and-copy kernel
            if q.prod:
                getattr(self, sg)[:, :, sl] = out[1].view(B, H, s, -1)
                getattr(self, rs)[:, :, sl].copy_(out[2].view(B, H, s))
        self.seq_len += s

    def dequantized(self, upto: Optional[int] = None) -> Tuple[torch.Tensor, torch.Tensor]:
        """History [0, upto) as (B, H, T, d) tensors in the cache dtype."""
        T = self.seq_len if upto is None else upto
        B, H, d = self.batch, self.num_heads, self.head_dim
        if T == 0:
            z = torch.zeros(B, H, 0, d, dtype=self.dtype, device=self.device)
            return z, z.clone()
        res = []
        for q, p, n, sg, rs in ((self.kq, self.kp, self.kn, "ks", "kr"),
                                (self.vq, self.vp, self.vn, "vs", "vr")):
            flat_p = self.rows(p is self.vp, T).reshape(B * H * T, -1)
            flat_n = n[:, :, :T].reshape(-1)
            if q.prod:
                out = q.dequantize(flat_p, flat_n, getattr(self, sg)[:, :, :T].reshape(B * H * T, -1),
                                   getattr(self, rs)[:, :, :T].reshape(-1), self.dtype)
            else:
                out = q.dequantize(flat_p, flat_n.to(self.dtype) if self.dtype != torch.float32 else flat_n,
                                   dtype=self.dtype)
            res.append(out.view(B, H, T, d).to(self.dtype))
        return res[0], res[1]

    def rows(self, values: bool, T: Optional[int] = None) -> torch.Tensor:
        """Bit-plane packed rows [B, H, T, P] of tokens 0..T-1 (reference.py:191-224),
        whatever the storage layout."""
        T = self.seq_len if T is None else T
        p = self.vp if values else self.kp
        if not self.dl:
            return p[:, :, :T]
        B, H = self.batch, self.num_heads
        q = self.vq if values else self.kq
        r = _ops().unpack_decode_layout(p.view(B * H, p.shape[2], -1), self.head_dim, q.code_bits,
                                        int(values), 0, T)
        return r.view(B, H, T, -1)

    # ------------------------------------------------------------ Cache layer API
    def update(self, key_states: torch.Tensor, value_states: torch.Tensor, *args, **kwargs):
        if not self.is_initialized:
            self.lazy_initialization(key_states, value_states)
        if self.protected:
            self.keys = torch.cat([self.keys, key_states], dim=-2)
            self.values = torch.cat([self.values, value_states], dim=-2)
            self.seq_len = self.keys.shape[-2]
            return self.keys, self.values
        if key_states.shape[0] != self.batch:
            raise ValueError(f"batch changed from {self.batch} to {key_states.shape[0]}")
        t_hist = self.seq_len
        if self.fused_attention:
            self._append(key_states, value_states)
            return _FusedKV(key_states, self, t_hist), value_states
        k_old, v_old = self.dequantized()
        self._append(key_states, value_states)
        return (torch.cat([k_old, key_states.to(self.dtype)], dim=-2),
                torch.cat([v_old, value_states.to(self.dtype)], dim=-2))

    def get_mask_sizes(self, query_length: int) -> Tuple[int, int]:
        return self.seq_len + query_length, 0

    def get_seq_length(self) -> int:
        return self.seq_len

    def get_max_length(self) -> int:
        return -1

    def reorder(self, beam_idx: torch.LongTensor) -> None:
        """Reorder the batch dimension (beam search); packed rows move as they are."""
        if self.protected:
            self.keys = self.keys.index_select(0, beam_idx.to(self.keys.device))
            self.values = self.values.index_select(0, beam_idx.to(self.values.device))
            return
        if not self.is_initialized or self.cap == 0:
            return
        idx = beam_idx.to(self.device)
        for name in ("kp", "vp", "kn", "vn", "ks", "vs", "kr", "vr"):
            t = getattr(self, name, None)
            if t is not None:
                setattr(self, name, t.index_select(0, idx))

    def memory_bytes(self) -> int:
        """Packed codes + norms actually stored (hf_integration.py:512-525 counts the same)."""
        if self.protected or not self.is_initialized:
            return 0
        B, H, T = self.batch, self.num_heads, self.seq_len
        bpp = (self.head_dim + 7) // 8
        nsz = torch.finfo(self.norm_dtype).bits // 8
        per = (self.kq.code_bits + self.vq.code_bits) * bpp + 2 * nsz
        if self.kq.prod:
            per += 2 * bpp + 8
        return B * H * T * per


class _FusedKV(torch.Tensor):
    """Key tensor of the new tokens that also carries its layer and history length, so
    the registered "turboquant" attention function can reach the packed history."""

    @staticmethod
    def __new__(cls, data, layer, t_hist):
        t = torch.Tensor._make_subclass(cls, data, False)
        t._tq_layer = layer
        t._tq_hist = t_hist
        return t

    @classmethod
    def __torch_function__(cls, func, types, args=(), kwargs=None):
        # Any torch op on it behaves like on the plain tensor (and returns plain tensors).
        kwargs = kwargs or {}
        args = [a.as_subclass(torch.Tensor) if isinstance(a, _FusedKV) else a for a in args]
        return func(*args, **kwargs)


def _sdpa_gqa(query, key, value, attention_mask, scaling):
    G = query.shape[1] // key.shape[1]
    if G > 1:
        key = key.repeat_interleave(G, dim=1)
        value = value.repeat_interleave(G, dim=1)
    is_causal = attention_mask is None and query.shape[2] > 1
    out = torch.nn.functional.scaled_dot_product_attention(
        query, key, value, attn_mask=attention_mask, is_causal=is_causal, scale=scaling)
    return out.transpose(1, 2).contiguous()


_HIST_LENS: Dict[Any, torch.Tensor] = {}


def _history_lengths(B: int, t_hist: int, device) -> torch.Tensor:
    """[B] int32 tensor of t_hist, shared by every layer of a decode step (one fill per
    step instead of one per layer)."""
    key = (B, t_hist, str(device))
    t = _HIST_LENS.get(key)
    if t is None:
        _HIST_LENS.clear()
        t = _HIST_LENS[key] = torch.full((B,), t_hist, dtype=torch.int32, device=device)
    return t


_WINDOW: Dict[Any, Optional[torch.Tensor]] = {}


def _window_starts(mask: torch.Tensor, B: int, t_hist: int) -> Optional[torch.Tensor]:
    """Left-padding starts of a decode step from its attention mask [B, 1, 1, t_hist + 1]
    (bool, True = attend, as transformers' sdpa_mask builds it; or additive float, 0 =
    attend): per sequence the first attended position, when every position from it through
    the current token is attended -- the form generate() gives left-padded batches.  None
    for any other mask (the caller takes the general path).  One host read per mask: every
    layer of a step shares the step's mask tensor."""
    key = (id(mask), mask.data_ptr(), tuple(mask.shape), t_hist)
    if key in _WINDOW:
        return _WINDOW[key]
    _WINDOW.clear()
    m = mask[:, 0, -1, :] if mask.dim() == 4 else mask.reshape(mask.shape[0], -1)
    vis = m if m.dtype == torch.bool else (m == 0)
    res = None
    if vis.shape[-1] == t_hist + 1:
        vis = vis.expand(B, -1)
        first = vis.int().argmax(-1)  # the first attended position (0 when none is)
        ok = ((vis.sum(-1) == vis.shape[-1] - first) & vis[:, -1]).all()
        if bool(ok):
            res = first.to(torch.int32)
    _WINDOW[key] = res
    return res


def turboquant_attention(module, query, key, value, attention_mask, scaling=None, dropout=0.0,
                         **kwargs):
    """Attention function registered as "turboquant" with transformers."""
    if scaling is None:
        scaling = 1.0 / math.sqrt(query.shape[-1])
    layer = getattr(key, "_tq_layer", None)
    if layer is None:
        k = key.as_subclass(torch.Tensor) if isinstance(key, _FusedKV) else key
        return _sdpa_gqa(query, k, value, attention_mask, scaling), None
    t_hist = key._tq_hist
    k_new = key.as_subclass(torch.Tensor)
    B, Hq, sq, d = query.shape
    # a padded batch's mask (left padding, as generate() pads) becomes per-sequence window
    # starts of the decode-layout kernel; any other mask takes the general path
    starts = None
    if sq == 1 and attention_mask is not None and t_hist > 0 and layer.dl and not layer.kq.prod:
        starts = _window_starts(attention_mask, B, t_hist)
    if sq == 1 and (attention_mask is None or starts is not None) and t_hist > 0 \
            and not layer.kq.prod:
        q = query[:, :, 0, :]
        seq = _history_lengths(B, t_hist, query.device)
        # the token being decoded attends to its own exact key and value: merged with the
        # history by log-sum-exp in one kernel (the eager composition of
        # hf_integration.py:372-390); the decode layout takes both in one op
        if layer.dl:
            out = _ops().decode_attention_dl_merged(
                q, layer.kp, layer.kn, layer.vp, layer.vn, seq, layer.kq.cen, layer.vq.cen,
                layer.kq.R, layer.vq.R, float(scaling), starts, k_new[:, :, 0, :],
                value[:, :, 0, :])
        else:
            o_h, lse_h = _ops().decode_attention_packed_lse(
                q, layer.kp, layer.kn, layer.vp, layer.vn, seq, layer.kq.cen, layer.vq.cen,
                layer.kq.R, layer.vq.R, layer.kq.bits, layer.vq.bits, float(scaling))
            out = _ops().decode_merge_token(o_h, lse_h, q, k_new[:, :, 0, :], value[:, :, 0, :],
                                            float(scaling))
        return out.to(query.dtype).unsqueeze(1), None
    k_old, v_old = layer.dequantized(upto=t_hist)
    k_all = torch.cat([k_old, k_new.to(k_old.dtype)], dim=-2)
    v_all = torch.cat([v_old, value.to(v_old.dtype)], dim=-2)
    return _sdpa_gqa(query, k_all, v_all, attention_mask, scaling), None


def enable_fused_attention(model) -> None:
    """Run `model`'s attention through the "turboquant" function (pair it with a
    TurboQuantCache(fused_attention=True))."""
    if hasattr(model, "set_attn_implementation"):
        model.set_attn_implementation("turboquant")
    else:
        model.config._attn_implementation = "turboquant"


if _TRANSFORMERS_AVAILABLE:
    _AttnIf.register("turboquant", turboquant_attention)
    try:
        from transformers.masking_utils import AttentionMaskInterface, sdpa_mask
        AttentionMaskInterface.register("turboquant", sdpa_mask)
    except ImportError:  # pragma: no cover
        pass


class TurboQuantCache(_HFCache):
    """Drop-in quantized KV cache for `model.generate` (hf_integration.py:272-555)."""

    def __init__(self, key_bits: int = 4, value_bits: int = 2, mode: str = "mse",
                 rotation: str = "dense_qr", protected_layers: int = 0, seed: int = 42,
                 fused_attention: bool = False, **kwargs: Any) -> None:
        self.tq_config = TurboQuantConfig(key_bits=key_bits, value_bits=value_bits, mode=mode,
                                          rotation=rotation, protected_layers=protected_layers,
                                          quantize_on_append=True, seed=seed)
        if mode not in ("mse", "prod"):
            raise ValueError(f"Unknown mode: {mode}")
        self._protected_layers = protected_layers
        self.fused_attention = fused_attention
        counter = [0]

        def make_layer():
            idx = counter[0]
            counter[0] += 1
            return TurboQuantLayer(self.tq_config, protected=idx < protected_layers,
                                   fused_attention=fused_attention)

        if _TRANSFORMERS_AVAILABLE:
            super().__init__(layer_class_to_replicate=make_layer, **kwargs)
        else:
            self.layers: List[TurboQuantLayer] = []
            self.layer_class_to_replicate = make_layer

    @classmethod
    def from_config(cls, key_bits: int = 4, value_bits: int = 2, mode: str = "mse",
                    rotation: str = "dense_qr", protected_layers: int = 0,
                    seed: int = 42) -> "TurboQuantCache":
        return cls(key_bits=key_bits, value_bits=value_bits, mode=mode, rotation=rotation,
                   protected_layers=protected_layers, seed=seed)

    def update(self, key_states, value_states, layer_idx: int, cache_kwargs=None, *args, **kwargs):
        while len(self.layers) <= layer_idx:
            self.layers.append(self.layer_class_to_replicate())
        return self.layers[layer_idx].update(key_states, value_states)

    def get_seq_length(self, layer_idx: int = 0) -> int:
        if layer_idx >= len(self.layers):
            return 0
        return self.layers[layer_idx].get_seq_length()

    def get_max_length(self) -> Optional[int]:
        return None

    def get_usable_length(self, new_seq_length: int, layer_idx: int = 0) -> int:
        return self.get_seq_length(layer_idx)

    def reorder_cache(self, beam_idx: torch.LongTensor) -> None:
        for layer in self.layers:
            layer.reorder(beam_idx)

    @property
    def seen_tokens(self) -> int:
        return max([l.get_seq_length() for l in self.layers] or [0])

    def memory_bytes(self) -> int:
        """Bytes of packed codes + norms of the quantized layers (protected layers excluded,
        as in hf_integration.py:512-525)."""
        return sum(l.memory_bytes() for l in self.layers)

    def __len__(self) -> int:
        return len(self.layers)

    def __getitem__(self, layer_idx: int) -> Tuple[torch.Tensor, torch.Tensor]:
        if layer_idx >= len(self.layers) or not self.layers[layer_idx].is_initialized:
            raise IndexError(f"No cached data for layer {layer_idx}")
        layer = self.layers[layer_idx]
        if layer.protected:
            return layer.keys, layer.values
        return layer.dequantized()

    def __iter__(self):
        for i in range(len(self.layers)):
            if self.layers[i].is_initialized:
                yield self[i]


__all__ = ["TurboQuantCache", "TurboQuantLayer", "turboquant_attention", "enable_fused_attention"]
