"""Paged packed KV storage for the vLLM backend: block pools, slot-mapped writes, decode
through block tables, causal prefill.

vLLM hands an attention backend a flat batch of tokens with a slot per new token
(`slot_mapping`), a block table per sequence and the sequences' context lengths.  The
reference's backend (turboquant_kv/vllm_plugin/__init__.py:114-304, 350-412) ignores
them: it appends every token to one contiguous QuantizedKVCache and attends over all of
it, with no causal mask for prefill and no notion of separate sequences.  Here a layer's
K and V live in block pools laid out as vLLM lays out its blocks,
[num_blocks, num_kv_heads, block_size, packed_bytes] uint8 plus fp32 norms
[num_blocks, num_kv_heads, block_size]; new tokens are quantized in one launch and
scattered to their slots (`paged_store`); decode tokens of all sequences run one fused
kernel that reads the pools through the block tables (`decode_attention_paged`); a
prefill sequence gathers its rows (`paged_gather`) and attends causally: the i-th of
its n new tokens sees the first T - n + i + 1 tokens of its context.

Keys use `seed`, values `seed + 1`, prod mode the (bits-1)-bit codebook and the QJL
matrices of seed + 12345 / seed + 1 + 12345 -- the QuantizedKVCache conventions
(cache.py:56-76).  Protected layers keep fp16 rows in pools of the same block layout.

layout="decode" (mse mode, 4-bit keys, 2-, 3- or 4-bit values, head_dim 64, block_size a
power of two >= 16) keeps the quantized layers in the decode layout instead: key pair bytes
[num_blocks, H, block_size, 32] and value tiles -- [num_blocks, H, block_size/64, 512 vb]
(64-token tiles) for block sizes >= 64, [num_blocks, H, block_size/16, 128 vb] (16-token
sub-blocks) below -- read by the MFMA decode kernel through the block tables
(`decode_attention_paged_dl`); a prefill sequence runs the causal prefill kernel over the
same pools (`prefill_attention_paged_dl`).
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import List, Optional

import torch

from turboquant_kv import ops
from turboquant_kv._lib import ops as _ops
from turboquant_kv.codebook import lloyd_max_codebook, make_qjl_matrix, make_rotation_matrix
from turboquant_kv.config import TurboQuantConfig


@dataclass
class TurboQuantAttentionMetadata:
    """The fields of vLLM's attention metadata this backend reads.

    Tokens are ordered prefill sequences first, then decode sequences (one token each),
    as vLLM batches them.
      slot_mapping     [num_tokens] int64: flat slot of each new token (-1: padding, skipped)
      seq_lens         [num_seqs] int32: context length of each sequence after this step
      block_tables     [num_seqs, max_blocks] int32
      query_start_loc  [num_seqs + 1]: first token of each sequence in the batch
      num_prefills     number of leading prefill sequences
      query_start_loc_cpu, seq_lens_cpu  optional host copies of the two (vLLM keeps
                       them beside the device tensors); a step with prefill sequences
                       reads them instead of copying the device tensors back
    """

    slot_mapping: torch.Tensor
    seq_lens: torch.Tensor
    block_tables: torch.Tensor
    query_start_loc: torch.Tensor
    num_prefills: int
    layer_id: int = 0
    query_start_loc_cpu: Optional[List[int]] = None
    seq_lens_cpu: Optional[List[int]] = None


def gather_value_tiles(vt_pool: torch.Tensor, block_table: torch.Tensor, T: int) -> torch.Tensor:
    """Value tiles of tokens 0..T-1 of one sequence from a decode-layout pool, in the
    contiguous decode layout [H, ceil(T/64), 512 vb] (unpack_decode_layout's input)."""
    nb, H, per_block, width = vt_pool.shape
    dev = vt_pool.device
    tiles64 = width >= 1024
    vb = width // (512 if tiles64 else 128)
    n = (T + 63) // 64 if tiles64 else (T + 15) // 16
    tiles, _ = ops.paged_gather(vt_pool, None, block_table.view(1, -1),
                                torch.tensor([n], dtype=torch.int32, device=dev), n)
    if tiles64:
        return tiles[0]
    # 16-token sub-blocks: sub-block m of a tile holds group m's share of the tile words
    nt = (T + 63) // 64
    sub = torch.zeros(H, nt * 4, width, dtype=torch.uint8, device=dev)
    sub[:, :n] = tiles[0]
    if vb == 2:  # word m of each lane
        return sub.view(H, nt, 4, 64, 4).permute(0, 1, 3, 2, 4).reshape(H, nt, 1024)
    if vb == 4:  # bytes 2 (m % 2) .. + 1 of tile word 4 (m / 2) + dg: lane L's 8 bytes
        w = sub.view(H, nt, 2, 2, 64, 4, 2)              # [G, m % 2, L, dg, byte]
        return w.permute(0, 1, 2, 4, 5, 3, 6).reshape(H, nt, 2048)
    a = sub[..., :256].reshape(H, nt, 2, 2, 64, 2, 2)      # words 3G + 0, 1: [G, m % 2, L, i, byte]
    b = sub[..., 256:].reshape(H, nt, 2, 2, 64, 1, 2)      # word 3G + 2
    w = torch.cat([a, b], dim=5).permute(0, 1, 4, 2, 5, 3, 6).reshape(H, nt, 64, 6, 4)
    return torch.cat([w[:, :, :, :4].reshape(H, nt, 1024), w[:, :, :, 4:].reshape(H, nt, 512)], dim=2)


class PagedKVPools:
    """A model's paged packed KV storage: per layer, K/V block pools and norms."""

    def __init__(self, config: TurboQuantConfig, num_layers: int, num_blocks: int, block_size: int,
                 num_kv_heads: int, head_dim: int, device="cuda", layout: str = "bitplane"):
        if config.mode not in ("mse", "prod"):
            raise ValueError(f"Unknown mode: {config.mode}")
        if layout not in ("bitplane", "decode"):
            raise ValueError(f"Unknown layout: {layout}")
        if layout == "decode" and not self.decode_layout_supported(config, head_dim, block_size):
            raise ValueError("layout='decode' needs mse mode, 4-bit keys, 2-4 bit values, "
                             "head_dim 64 and a power-of-two block_size >= 16")
        self.layout = layout
        self.config = config
        self.num_layers = num_layers
        self.num_blocks = num_blocks
        self.block_size = block_size
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim
        self.device = torch.device(device)
        dev = self.device
        self.prod = config.mode == "prod"
        self.R_k = make_rotation_matrix(head_dim, seed=config.seed, method=config.rotation).to(dev)
        self.R_v = make_rotation_matrix(head_dim, seed=config.seed + 1, method=config.rotation).to(dev)
        kb, vb = config.key_bits, config.value_bits
        if self.prod:
            self.S_k = make_qjl_matrix(head_dim, head_dim, config.seed, dev)
            self.S_v = make_qjl_matrix(head_dim, head_dim, config.seed + 1, dev)
            kb, vb = kb - 1, vb - 1
        self.kbits, self.vbits = kb, vb  # stored code widths
        self.kbnd, self.kcen = [t.to(dev) for t in lloyd_max_codebook(kb, head_dim)]
        self.vbnd, self.vcen = [t.to(dev) for t in lloyd_max_codebook(vb, head_dim)]
        bpp = (head_dim + 7) // 8
        nb, H, bs = num_blocks, num_kv_heads, block_size
        u8 = dict(dtype=torch.uint8, device=dev)
        f32 = dict(dtype=torch.float32, device=dev)
        self.layers: List[dict] = []
        for layer in range(num_layers):
            if layer < config.protected_layers:
                self.layers.append({"k_fp": torch.zeros(nb, H, bs, head_dim, dtype=torch.float16, device=dev),
                                    "v_fp": torch.zeros(nb, H, bs, head_dim, dtype=torch.float16, device=dev)})
                continue
            if layout == "decode":
                self.layers.append({"kp": torch.zeros(nb, H, bs, head_dim // 2, **u8),
                                    "kn": torch.zeros(nb, H, bs, **f32),
                                    "vt": (torch.zeros(nb, H, bs // 64, 512 * vb, **u8) if bs >= 64
                                           else torch.zeros(nb, H, bs // 16, 128 * vb, **u8)),
                                    "vn": torch.zeros(nb, H, bs, **f32)})
                continue
            st = {"k": torch.zeros(nb, H, bs, kb * bpp, **u8), "kn": torch.zeros(nb, H, bs, **f32),
                  "v": torch.zeros(nb, H, bs, vb * bpp, **u8), "vn": torch.zeros(nb, H, bs, **f32)}
            if self.prod:
                st.update(ks=torch.zeros(nb, H, bs, bpp, **u8), kr=torch.zeros(nb, H, bs, **f32),
                          vs=torch.zeros(nb, H, bs, bpp, **u8), vr=torch.zeros(nb, H, bs, **f32))
            self.layers.append(st)

    @staticmethod
    def decode_layout_supported(config: TurboQuantConfig, head_dim: int, block_size: int) -> bool:
        return (config.mode == "mse" and config.key_bits == 4 and 2 <= config.value_bits <= 4
                and head_dim == 64 and block_size >= 16 and block_size & (block_size - 1) == 0)

    # ------------------------------------------------------------------ writes
    def _quantize(self, x: torch.Tensor, R, bnd, cen, S, bits_total):
        flat = x.reshape(-1, self.head_dim)
        if self.prod:
            return _ops().quantize_prod_packed(flat, R, bnd, cen, S, bits_total)
        return _ops().quantize_mse_packed(flat, R, bnd, bits_total)

    def write(self, layer: int, key: torch.Tensor, value: torch.Tensor,
              slot_mapping: torch.Tensor) -> None:
        """Quantize key/value [n, num_kv_heads, head_dim] and store token i at slot
        slot_mapping[i] (negative slots are skipped)."""
        n, H = key.shape[0], self.num_kv_heads
        if n == 0:
            return
        st = self.layers[layer]
        sm = slot_mapping.to(self.device, torch.long)
        if "k_fp" in st:
            self._write_fp(st["k_fp"], key, sm)
            self._write_fp(st["v_fp"], value, sm)
            return
        kq = self._quantize(key.to(self.device), self.R_k, self.kbnd, self.kcen,
                            getattr(self, "S_k", None), self.config.key_bits)
        vq = self._quantize(value.to(self.device), self.R_v, self.vbnd, self.vcen,
                            getattr(self, "S_v", None), self.config.value_bits)
        if "kp" in st:
            pairs = torch.empty(n * H, 1, self.head_dim // 2, dtype=torch.uint8, device=self.device)
            ops.pack_decode_layout(kq[0].view(n * H, 1, -1), pairs, self.head_dim, 4, False, 0)
            ops.paged_store(pairs.view(n, H, -1), kq[-1].float().view(n, H), sm, st["kp"], st["kn"])
            ops.paged_store_value_tiles(vq[0].view(n, H, -1), vq[-1].float().view(n, H), sm,
                                        st["vt"], st["vn"])
            return
        ops.paged_store(kq[0].view(n, H, -1), kq[-1].float().view(n, H), sm, st["k"], st["kn"])
        ops.paged_store(vq[0].view(n, H, -1), vq[-1].float().view(n, H), sm, st["v"], st["vn"])
        if self.prod:
            ops.paged_store(kq[1].view(n, H, -1), kq[2].float().view(n, H), sm, st["ks"], st["kr"])
            ops.paged_store(vq[1].view(n, H, -1), vq[2].float().view(n, H), sm, st["vs"], st["vr"])

    def _write_fp(self, pool: torch.Tensor, x: torch.Tensor, sm: torch.Tensor) -> None:
        nb, H, bs, d = pool.shape
        ok = (sm >= 0) & (sm < nb * bs)
        sm, x = sm[ok], x.to(self.device)[ok]
        idx = ((sm // bs)[:, None] * H + torch.arange(H, device=self.device)[None, :]) * bs + (sm % bs)[:, None]
        pool.view(-1, d)[idx.reshape(-1)] = x.reshape(-1, d).half()

    # ------------------------------------------------------------------ reads
    def _gather_fp(self, pool: torch.Tensor, block_table: torch.Tensor, T: int) -> torch.Tensor:
        """fp16 rows of tokens 0..T-1 of one sequence -> [H, T, d] float32."""
        nb, H, bs, d = pool.shape
        t = torch.arange(T, device=self.device)
        blk = block_table.to(self.device, torch.long)[t // bs]
        idx = (blk[None, :] * H + torch.arange(H, device=self.device)[:, None]) * bs + (t % bs)[None, :]
        return pool.view(-1, d)[idx].float()

    def _gather(self, st: dict, key: str, block_table: torch.Tensor, T: int):
        """Rows and norms of tokens 0..T-1 of one sequence: ([H, T, P], [H, T])."""
        if "kp" in st:  # decode layout: back to bit-plane rows
            d = self.head_dim
            one = lambda v: torch.tensor([v], dtype=torch.int32, device=self.device)
            if key == "k":
                pairs, norms = ops.paged_gather(st["kp"], st["kn"], block_table.view(1, -1), one(T), T)
                return ops.unpack_decode_layout(pairs[0], d, 4, False, 0, T), norms[0]
            tiles = gather_value_tiles(st["vt"], block_table, T)
            _, norms = ops.paged_gather(st["kp"], st["vn"], block_table.view(1, -1), one(T), T)
            return ops.unpack_decode_layout(tiles, d, self.vbits, True, 0, T), norms[0]
        norm_key = {"k": "kn", "v": "vn", "ks": "kr", "vs": "vr"}[key]
        rows, norms = ops.paged_gather(st[key], st[norm_key], block_table.view(1, -1),
                                       torch.tensor([T], dtype=torch.int32, device=self.device), T)
        return rows[0], norms[0]

    def sequence_kv(self, layer: int, block_table: torch.Tensor, T: int):
        """Dequantized K and V of tokens 0..T-1 of one sequence: ([H, T, d], [H, T, d]) fp32."""
        st = self.layers[layer]
        if "k_fp" in st:
            return (self._gather_fp(st["k_fp"], block_table, T),
                    self._gather_fp(st["v_fp"], block_table, T))
        d, H = self.head_dim, self.num_kv_heads
        out = []
        for kind, R, cen, bits in (("k", self.R_k, self.kcen, self.config.key_bits),
                                   ("v", self.R_v, self.vcen, self.config.value_bits)):
            rows, norms = self._gather(st, kind, block_table, T)
            if self.prod:
                signs, res = self._gather(st, kind + "s", block_table, T)
                S = self.S_k if kind == "k" else self.S_v
                x = _ops().dequantize_prod_packed(rows.reshape(H * T, -1), signs.reshape(H * T, -1),
                                                  res.reshape(-1), norms.reshape(-1), cen, R, S,
                                                  bits, d)
            else:
                x = _ops().dequantize_mse_packed(rows.reshape(H * T, -1), norms.reshape(-1), cen, R,
                                                 bits, d)
            out.append(x.view(H, T, d))
        return out[0], out[1]

    # ------------------------------------------------------------------ attention
    def prefill(self, layer: int, q: torch.Tensor, block_table: torch.Tensor, T: int,
                scale: float) -> torch.Tensor:
        """Causal attention of one sequence's n new tokens q [n, Hq, d] (positions
        T-n .. T-1 of its context) over its first T tokens -> [n, Hq, d] fp32."""
        n, Hq, d = q.shape
        H = self.num_kv_heads
        G = Hq // H
        st = self.layers[layer]
        if "kp" in st:
            # one kernel: each 64-token tile of the history read once per 48 query rows
            return ops.prefill_attention_paged_dl(q.to(self.device), st["kp"], st["kn"], st["vt"],
                                                  st["vn"], block_table.to(self.device), T, self.kcen,
                                                  self.vcen, self.R_k, self.R_v, float(scale))
        qf = q.to(self.device).float()
        pos = torch.arange(T - n, T, device=self.device)
        mask = torch.arange(T, device=self.device)[None, :] > pos[:, None]       # [n, T]
        out = torch.empty(n, Hq, d, dtype=torch.float32, device=self.device)
        packed = "k_fp" not in st
        if packed:
            krows, kn = self._gather(st, "k", block_table, T)
            vrows, vn = self._gather(st, "v", block_table, T)
            if self.prod:
                ks, kr = self._gather(st, "ks", block_table, T)
                _, vals = self.sequence_kv(layer, block_table, T)
        else:
            keys, vals = self.sequence_kv(layer, block_table, T)
        for g in range(H):
            qg = qf[:, g * G:(g + 1) * G].transpose(0, 1).reshape(1, G * n, d)   # heads x tokens
            if not packed:
                s = (qg[0] @ keys[g].t()).view(G, n, T)
            elif self.prod:
                s = ops.attention_scores_prod(qg, krows[g], ks[g], kr[g], kn[g], self.kcen, self.R_k,
                                              self.S_k, self.config.key_bits)[0].view(G, n, T)
            else:
                s = ops.attention_scores_packed(qg, krows[g], kn[g], self.kcen, self.R_k,
                                                self.config.key_bits)[0].view(G, n, T)
            s = (s * scale).masked_fill(mask[None], float("-inf"))
            w = torch.softmax(s, dim=-1)
            if packed and not self.prod:
                o = ops.attention_values_packed(w.reshape(1, G * n, T), vrows[g], vn[g], self.vcen,
                                                self.R_v, self.config.value_bits)[0]
            else:
                o = w.reshape(G * n, T) @ vals[g]
            out[:, g * G:(g + 1) * G] = o.view(G, n, d).transpose(0, 1)
        return out

    def decode(self, layer: int, q: torch.Tensor, block_tables: torch.Tensor,
               seq_lens: torch.Tensor, scale: float) -> torch.Tensor:
        """One new token per sequence: q [B, Hq, d] over each sequence's first seq_lens[b]
        tokens -> [B, Hq, d] in q's dtype."""
        st = self.layers[layer]
        if "kp" in st:
            return self._decode_dl(st, q.to(self.device), block_tables, seq_lens, scale)
        if "k_fp" not in st and not self.prod:
            out, _ = _ops().decode_attention_paged(
                q.to(self.device), st["k"], st["kn"], st["v"], st["vn"], block_tables, seq_lens,
                self.kcen, self.vcen, self.R_k, self.R_v, self.config.key_bits,
                self.config.value_bits, float(scale))
            return out
        lens = seq_lens.tolist()
        return torch.cat([self.prefill(layer, q[b:b + 1], block_tables[b], int(lens[b]), scale)
                          for b in range(q.shape[0])]).to(q.dtype)

    def _decode_dl(self, st: dict, q, block_tables, seq_lens, scale) -> torch.Tensor:
        return ops.decode_attention_paged_dl(q, st["kp"], st["kn"], st["vt"], st["vn"], block_tables,
                                             seq_lens, self.kcen, self.vcen, self.R_k, self.R_v,
                                             float(scale))

    def forward(self, query: torch.Tensor, key: torch.Tensor, value: torch.Tensor,
                md: TurboQuantAttentionMetadata, scale: float,
                output: Optional[torch.Tensor] = None) -> torch.Tensor:
        """vLLM attention step: store the batch's new K/V at their slots, then causal
        prefill for the leading sequences and one fused decode launch for the rest.
        query [num_tokens, Hq, d], key/value [num_tokens, Hkv, d]."""
        layer = md.layer_id
        self.write(layer, key, value, md.slot_mapping)
        out = output if output is not None else torch.empty_like(query)
        npf = md.num_prefills
        if npf > 0:
            # prefill needs each sequence's token range and context length on the host: the
            # metadata's host copies, else one copy of just the prefill sequences' entries
            if md.query_start_loc_cpu is not None and md.seq_lens_cpu is not None:
                qsl, lens = md.query_start_loc_cpu, md.seq_lens_cpu
            else:
                both = torch.cat([md.query_start_loc[:npf + 1].to(torch.int64),
                                  md.seq_lens[:npf].to(torch.int64)]).tolist()
                qsl, lens = both[:npf + 1], both[npf + 1:]
            for i in range(npf):
                a, b = qsl[i], qsl[i + 1]
                if b > a:
                    out[a:b] = self.prefill(layer, query[a:b], md.block_tables[i], int(lens[i]),
                                            scale).to(out.dtype)
        # decode sequences hold one token each and come last: their count and position
        # follow from the shapes, with no host copy of the device metadata
        nd = md.block_tables.shape[0] - npf
        if nd > 0:
            d0 = query.shape[0] - nd
            out[d0:] = self.decode(layer, query[d0:], md.block_tables[npf:],
                                   md.seq_lens[npf:].to(self.device, torch.int32),
                                   scale).to(out.dtype)
        return out

    def memory_bytes(self) -> int:
        return sum(t.numel() * t.element_size() for st in self.layers for t in st.values())
