"""QuantizedKVCache on packed device storage (API of turboquant_kv/cache.py:29-381).

Storage per layer is [B, H, max_seq_len, packed_bytes] uint8 plus [B, H, max_seq_len]
float32 norms on the device.  `batch_size` defaults to 1, which reproduces the
reference's behaviour of keeping batch 0 of a 4-D append (cache.py:157-160); with
batch_size > 1 every sequence is stored.  Appends quantize every (batch, head, token)
row in one kernel launch instead of a Python loop over heads (cache.py:174-207).

Scores and values read the packed codes directly (attention_scores_packed /
attention_values_packed kernels); `decode_attention` runs the fused GQA decode
kernel.  Query heads may be a multiple of the KV heads (head h reads KV head
h // (Hq / H), as HF's repeat_kv does); the reference only handles equal counts.

For 4-bit keys and 2-4 bit values at head_dim 64 or 128 (MSE mode) the codes are kept in
the decode layout (same bytes per token, arranged for the decode kernel: key bytes hold two
4-bit codes, value bytes hold one dim of four consecutive tokens); the reference keeps
its packed storage private (cache.py:81-130), so only `_key_packed` / `_val_packed`,
which return the bit-plane rows, see the difference.
"""

from __future__ import annotations

import math
from typing import Optional

import torch

from turboquant_kv import ops
from turboquant_kv._lib import ops as _ops
from turboquant_kv.codebook import lloyd_max_codebook, make_qjl_matrix, make_rotation_matrix
from turboquant_kv.config import TurboQuantConfig


class QuantizedKVCache:
    def __init__(
        self,
        config: TurboQuantConfig,
        num_layers: int,
        max_seq_len: int,
        num_heads: int,
        head_dim: int,
        device: str = "cuda",
        batch_size: int = 1,
    ):
        self.config = config
        self.num_layers = num_layers
        self.max_seq_len = max_seq_len
        self.num_heads = num_heads
        self.head_dim = head_dim
        self.batch_size = batch_size
        self.device = torch.device(device)
        self.seq_lens = torch.zeros(num_layers, dtype=torch.long)
        dev = self.device

        # keys use seed, values seed + 1 (cache.py:56-61)
        self._key_rotation = make_rotation_matrix(head_dim, seed=config.seed,
                                                  method=config.rotation).to(dev)
        self._val_rotation = make_rotation_matrix(head_dim, seed=config.seed + 1,
                                                  method=config.rotation).to(dev)
        self._key_codebook = lloyd_max_codebook(config.key_bits, head_dim)
        self._val_codebook = lloyd_max_codebook(config.value_bits, head_dim)
        self._has_outliers = config.outlier_channels > 0
        if self._has_outliers:  # built for parity with cache.py:66-70; not used by any path
            self._key_codebook_outlier = lloyd_max_codebook(config.key_bits + 1, head_dim)
            self._val_codebook_outlier = lloyd_max_codebook(config.value_bits + 1, head_dim)

        self._is_prod = config.mode == "prod"
        if config.mode not in ("mse", "prod"):
            raise ValueError(f"Unknown mode: {config.mode}")
        kb, vb = config.key_bits, config.value_bits
        if self._is_prod:
            self._key_S = make_qjl_matrix(head_dim, head_dim, config.seed, dev)
            self._val_S = make_qjl_matrix(head_dim, head_dim, config.seed + 1, dev)
            self._key_codebook_prod = lloyd_max_codebook(kb - 1, head_dim)
            self._val_codebook_prod = lloyd_max_codebook(vb - 1, head_dim)
            kb, vb = kb - 1, vb - 1
        self._kbits_stored, self._vbits_stored = kb, vb
        kcb = self._key_codebook_prod if self._is_prod else self._key_codebook
        vcb = self._val_codebook_prod if self._is_prod else self._val_codebook
        self._kbnd, self._kcen = kcb[0].to(dev), kcb[1].to(dev)
        self._vbnd, self._vcen = vcb[0].to(dev), vcb[1].to(dev)

        bpp = (head_dim + 7) // 8
        # 4-bit keys and 2-4 bit values of head_dim 64 or 128 are kept in the decode layout
        self._dl = (not self._is_prod and kb == 4 and 2 <= vb <= 4 and head_dim in (64, 128))
        # decode-layout value tiles hold 64 tokens: capacity rounded up to a multiple of 64
        self._t_cap = (max_seq_len + 63) // 64 * 64 if self._dl else max_seq_len
        B, H, T = batch_size, num_heads, self._t_cap
        u8 = dict(dtype=torch.uint8, device=dev)
        f32 = dict(dtype=torch.float32, device=dev)
        self._protected = config.protected_layers > 0
        self._kstore, self._key_norms, self._vstore, self._val_norms = [], [], [], []
        self._key_qjl_signs, self._key_res_norms, self._val_qjl_signs, self._val_res_norms = [], [], [], []
        self._key_fp, self._val_fp = [], []
        for layer in range(num_layers):
            if self._protected and layer < config.protected_layers:
                self._key_fp.append(torch.zeros(B, H, T, head_dim, dtype=torch.float16, device=dev))
                self._val_fp.append(torch.zeros(B, H, T, head_dim, dtype=torch.float16, device=dev))
                for lst in (self._kstore, self._key_norms, self._vstore, self._val_norms):
                    lst.append(None)
                continue
            if self._dl:
                self._kstore.append(torch.zeros(B, H, T, head_dim // 2, **u8))
                self._vstore.append(torch.zeros(B, H, T // 64, 8 * vb * head_dim, **u8))
            else:
                self._kstore.append(torch.zeros(B, H, T, kb * bpp, **u8))
                self._vstore.append(torch.zeros(B, H, T, vb * bpp, **u8))
            self._key_norms.append(torch.zeros(B, H, T, **f32))
            self._val_norms.append(torch.zeros(B, H, T, **f32))
            if self._is_prod:
                self._key_qjl_signs.append(torch.zeros(B, H, T, bpp, **u8))
                self._key_res_norms.append(torch.zeros(B, H, T, **f32))
                self._val_qjl_signs.append(torch.zeros(B, H, T, bpp, **u8))
                self._val_res_norms.append(torch.zeros(B, H, T, **f32))

    # ------------------------------------------------------------------ helpers
    def _is_protected_layer(self, layer_id: int) -> bool:
        return self._protected and layer_id < self.config.protected_layers

    def _rows(self, layer_id: int, values: bool, T: int) -> torch.Tensor:
        """Bit-plane packed rows [B, H, T, P] of tokens 0..T-1 (reference.py:191-224)."""
        st = (self._vstore if values else self._kstore)[layer_id]
        if not self._dl:
            return st[:, :, :T]
        B, H = self.batch_size, self.num_heads
        bits = self._vbits_stored if values else self._kbits_stored
        r = ops.unpack_decode_layout(st.view(B * H, st.shape[2], st.shape[3]), self.head_dim, bits,
                                     values, 0, T)
        return r.view(B, H, T, -1)

    @property
    def _key_packed(self):
        """Per layer: packed key rows [B, H, max_seq_len, P] (None for protected layers)."""
        return [None if st is None else self._rows(l, False, self.max_seq_len)
                for l, st in enumerate(self._kstore)]

    @property
    def _val_packed(self):
        return [None if st is None else self._rows(l, True, self.max_seq_len)
                for l, st in enumerate(self._vstore)]

    def _as_bhsd(self, t: torch.Tensor) -> torch.Tensor:
        if t.dim() == 3:
            t = t.unsqueeze(0)
        if t.dim() != 4:
            raise ValueError(f"Expected 3D or 4D key/value, got {t.dim()}D")
        if t.shape[0] != self.batch_size:
            if self.batch_size == 1:
                t = t[:1]  # reference behaviour: keep batch 0 (cache.py:157-160)
            else:
                raise ValueError(f"batch {t.shape[0]} != cache batch_size {self.batch_size}")
        if t.shape[1] != self.num_heads or t.shape[3] != self.head_dim:
            raise ValueError(f"expected (B, {self.num_heads}, S, {self.head_dim}), got {tuple(t.shape)}")
        return t.to(self.device)

    # ------------------------------------------------------------------ append
    def append(self, layer_id: int, key: torch.Tensor, value: torch.Tensor):
        """Quantize and store new tokens.  key/value: (B, H, S, d) or (H, S, d)."""
        key, value = self._as_bhsd(key), self._as_bhsd(value)
        B, H, s, d = key.shape
        pos = int(self.seq_lens[layer_id].item())
        if pos + s > self.max_seq_len:
            raise ValueError(f"layer {layer_id}: {pos}+{s} tokens exceed max_seq_len {self.max_seq_len}")
        sl = slice(pos, pos + s)
        if self._is_protected_layer(layer_id):
            self._key_fp[layer_id][:, :, sl] = key.half()
            self._val_fp[layer_id][:, :, sl] = value.half()
            self.seq_lens[layer_id] += s
            return
        T = self._ops_quantize(key, self._key_rotation, self._kbnd, self._kcen,
                               getattr(self, "_key_S", None), self.config.key_bits)
        self._store(layer_id, False, T[0].view(B * H, s, -1), pos)
        self._key_norms[layer_id][:, :, sl] = T[-1].float().view(B, H, s)
        if self._is_prod:
            self._key_qjl_signs[layer_id][:, :, sl] = T[1].view(B, H, s, -1)
            self._key_res_norms[layer_id][:, :, sl] = T[2].float().view(B, H, s)
        V = self._ops_quantize(value, self._val_rotation, self._vbnd, self._vcen,
                               getattr(self, "_val_S", None), self.config.value_bits)
        self._store(layer_id, True, V[0].view(B * H, s, -1), pos)
        self._val_norms[layer_id][:, :, sl] = V[-1].float().view(B, H, s)
        if self._is_prod:
            self._val_qjl_signs[layer_id][:, :, sl] = V[1].view(B, H, s, -1)
            self._val_res_norms[layer_id][:, :, sl] = V[2].float().view(B, H, s)
        self.seq_lens[layer_id] += s

    def _store(self, layer_id: int, values: bool, rows: torch.Tensor, pos: int) -> None:
        """Write bit-plane rows [B*H, s, P] at tokens pos..pos+s of every (batch, head)."""
        st = (self._vstore if values else self._kstore)[layer_id]
        B, H = self.batch_size, self.num_heads
        s = rows.shape[1]
        if self._dl:
            bits = self._vbits_stored if values else self._kbits_stored
            ops.pack_decode_layout(rows, st.view(B * H, st.shape[2], st.shape[3]), self.head_dim,
                                   bits, values, pos)
        else:
            st[:, :, pos:pos + s] = rows.view(B, H, s, -1)

    def _ops_quantize(self, x, R, bnd, cen, S, bits):
        flat = x.reshape(-1, self.head_dim)
        if self._is_prod:
            return _ops().quantize_prod_packed(flat, R, bnd, cen, S, bits)
        return _ops().quantize_mse_packed(flat, R, bnd, bits)

    # ------------------------------------------------------------------ dequantize
    def _dequant(self, layer_id, values, norms, signs, res, R, cen, S, bits):
        T = int(self.seq_lens[layer_id].item())
        B, H, d = self.batch_size, self.num_heads, self.head_dim
        if T == 0:
            out = torch.zeros(B, H, 0, d, dtype=torch.float32, device=self.device)
        else:
            p = self._rows(layer_id, values, T).reshape(B * H * T, -1)
            n = norms[layer_id][:, :, :T].reshape(-1)
            if self._is_prod:
                out = _ops().dequantize_prod_packed(
                    p, signs[layer_id][:, :, :T].reshape(B * H * T, -1),
                    res[layer_id][:, :, :T].reshape(-1), n, cen, R, S, bits, d)
            else:
                out = _ops().dequantize_mse_packed(p, n, cen, R, bits, d)
            out = out.view(B, H, T, d)
        return out[0] if B == 1 else out

    def _dequantize_keys(self, layer_id: int) -> torch.Tensor:
        """(H, T, d) for batch_size 1, else (B, H, T, d), float32."""
        if self._is_protected_layer(layer_id):
            T = int(self.seq_lens[layer_id].item())
            k = self._key_fp[layer_id][:, :, :T].float()
            return k[0] if self.batch_size == 1 else k
        return self._dequant(layer_id, False, self._key_norms, self._key_qjl_signs,
                             self._key_res_norms, self._key_rotation, self._kcen,
                             getattr(self, "_key_S", None), self.config.key_bits)

    def _dequantize_values(self, layer_id: int) -> torch.Tensor:
        if self._is_protected_layer(layer_id):
            T = int(self.seq_lens[layer_id].item())
            v = self._val_fp[layer_id][:, :, :T].float()
            return v[0] if self.batch_size == 1 else v
        return self._dequant(layer_id, True, self._val_norms, self._val_qjl_signs,
                             self._val_res_norms, self._val_rotation, self._vcen,
                             getattr(self, "_val_S", None), self.config.value_bits)

    # ------------------------------------------------------------------ attention
    def _query_groups(self, q4: torch.Tensor):
        Hq = q4.shape[1]
        if Hq % self.num_heads != 0:
            raise ValueError(f"query heads {Hq} not a multiple of KV heads {self.num_heads}")
        return Hq // self.num_heads

    def _kv_batch(self, qb: int, b: int) -> int:
        return 0 if self.batch_size == 1 else b

    def attention_scores(self, layer_id: int, query: torch.Tensor) -> torch.Tensor:
        """Scaled logits q K^T / sqrt(d) from packed keys (cache.py:282-315).
        query: (batch, Hq, seq_q, d) or (Hq, seq_q, d) -> (..., Hq, seq_q, T)."""
        has_batch = query.dim() == 4
        q4 = (query if has_batch else query.unsqueeze(0)).to(self.device)
        Bq, Hq, sq, d = q4.shape
        if self.batch_size != 1 and Bq != self.batch_size:
            raise ValueError(f"query batch {Bq} != cache batch_size {self.batch_size}")
        G = self._query_groups(q4)
        T = int(self.seq_lens[layer_id].item())
        scale = 1.0 / math.sqrt(self.head_dim)
        if self._is_protected_layer(layer_id) or (self._is_prod and self.config.key_bits > 4):
            keys = self._dequantize_keys(layer_id)
            keys = keys.unsqueeze(0) if keys.dim() == 3 else keys
            keys = keys.repeat_interleave(G, dim=1) if G > 1 else keys
            logits = torch.matmul(q4.float(), keys.expand(Bq, -1, -1, -1).transpose(-2, -1)) * scale
        else:
            logits = torch.empty(Bq, Hq, sq, T, dtype=torch.float32, device=self.device)
            if T > 0:
                rows = self._rows(layer_id, False, T)
                qf = q4.float()
                for kvb in range(self.batch_size):
                    qbs = slice(None) if self.batch_size == 1 else slice(kvb, kvb + 1)
                    for g in range(self.num_heads):
                        qs = qf[qbs, g * G:(g + 1) * G]            # (b', G, sq, d)
                        if self._is_prod:
                            # <q, dequantize_prod(k_t)> scored from the packed rows.
                            s = ops.attention_scores_prod(
                                qs.reshape(1, -1, d), rows[kvb, g],
                                self._key_qjl_signs[layer_id][kvb, g, :T],
                                self._key_res_norms[layer_id][kvb, g, :T],
                                self._key_norms[layer_id][kvb, g, :T], self._kcen,
                                self._key_rotation, self._key_S, self.config.key_bits)
                        else:
                            s = ops.attention_scores_packed(
                                qs.reshape(1, -1, d), rows[kvb, g],
                                self._key_norms[layer_id][kvb, g, :T], self._kcen,
                                self._key_rotation, self.config.key_bits)
                        logits[qbs, g * G:(g + 1) * G] = s.view(qs.shape[0], G, sq, T)
                logits = logits * scale
        return logits if has_batch else logits.squeeze(0)

    def attention_values(self, layer_id: int, attn_weights: torch.Tensor) -> torch.Tensor:
        """attn_weights @ V from packed values (cache.py:317-339).
        attn_weights: (batch, Hq, seq_q, T) or (Hq, seq_q, T) -> (..., Hq, seq_q, d)."""
        has_batch = attn_weights.dim() == 4
        w4 = (attn_weights if has_batch else attn_weights.unsqueeze(0)).to(self.device)
        Bq, Hq, sq, T = w4.shape
        G = self._query_groups(w4)
        d = self.head_dim
        if self._is_protected_layer(layer_id) or self._is_prod:
            vals = self._dequantize_values(layer_id)
            vals = vals.unsqueeze(0) if vals.dim() == 3 else vals
            vals = vals.repeat_interleave(G, dim=1) if G > 1 else vals
            out = torch.matmul(w4.float(), vals.expand(Bq, -1, -1, -1))
        else:
            out = torch.empty(Bq, Hq, sq, d, dtype=torch.float32, device=self.device)
            rows = self._rows(layer_id, True, T) if T > 0 else None
            wf = w4.float()
            for kvb in range(self.batch_size):
                qbs = slice(None) if self.batch_size == 1 else slice(kvb, kvb + 1)
                for g in range(self.num_heads):
                    ws = wf[qbs, g * G:(g + 1) * G]
                    o = ops.attention_values_packed(
                        ws.reshape(1, -1, T), rows[kvb, g],
                        self._val_norms[layer_id][kvb, g, :T], self._vcen, self._val_rotation,
                        self.config.value_bits)
                    out[qbs, g * G:(g + 1) * G] = o.view(ws.shape[0], G, sq, d)
        return out if has_batch else out.squeeze(0)

    def decode_attention(self, layer_id: int, query: torch.Tensor,
                         scale: Optional[float] = None,
                         seq_lens: Optional[torch.Tensor] = None) -> torch.Tensor:
        """Fused single-token attention softmax(q K^T * scale) V over the packed cache.
        query: (B, Hq, d) with Hq a multiple of the KV heads; returns (B, Hq, d) in
        query.dtype.  seq_lens (B,) int32 on the device overrides the layer length."""
        if self._is_protected_layer(layer_id) or self._is_prod:
            raise NotImplementedError("decode_attention covers MSE-mode quantized layers")
        q = query.to(self.device)
        if q.dim() != 3:
            raise ValueError("query must be (B, Hq, d)")
        B = q.shape[0]
        if B != self.batch_size:
            raise ValueError(f"query batch {B} != cache batch_size {self.batch_size}")
        if scale is None:
            scale = 1.0 / math.sqrt(self.head_dim)
        if seq_lens is None:
            seq_lens = torch.full((B,), int(self.seq_lens[layer_id].item()), dtype=torch.int32,
                                  device=self.device)
        if self._dl and q.shape[1] % self.num_heads == 0:
            return ops.decode_attention_dl(
                q, self._kstore[layer_id], self._key_norms[layer_id], self._vstore[layer_id],
                self._val_norms[layer_id], seq_lens, self._kcen, self._vcen, self._key_rotation,
                self._val_rotation, scale)
        Tc = self._t_cap
        return ops.decode_attention_packed(
            q, self._rows(layer_id, False, Tc), self._key_norms[layer_id],
            self._rows(layer_id, True, Tc), self._val_norms[layer_id], seq_lens, self._kcen,
            self._vcen, self._key_rotation, self._val_rotation, self.config.key_bits,
            self.config.value_bits, scale)

    # ------------------------------------------------------------------ accounting
    def memory_bytes(self) -> int:
        """Packed bytes + 4-byte norms per stored token (cache.py:341-366)."""
        total = 0
        bpp = (self.head_dim + 7) // 8
        for layer_id in range(self.num_layers):
            T = int(self.seq_lens[layer_id].item())
            if T == 0:
                continue
            rows = self.batch_size * self.num_heads * T
            if self._is_protected_layer(layer_id):
                total += 2 * rows * self.head_dim * 2
                continue
            per = self.config.key_bits * bpp + self.config.value_bits * bpp + 8
            if self._is_prod:
                per += 2 * bpp + 8
            total += rows * per
        return total

    @property
    def compression_ratio(self) -> float:
        """fp16 K+V bytes / memory_bytes() (cache.py:368-381)."""
        fp16 = sum(2 * self.batch_size * self.num_heads * int(self.seq_lens[l].item()) *
                   self.head_dim * 2 for l in range(self.num_layers))
        actual = self.memory_bytes()
        return 0.0 if actual == 0 else fp16 / actual
