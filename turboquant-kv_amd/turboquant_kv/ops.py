"""Direct wrappers of torch.ops.turboquant (mirrors turboquant_kv/ops.py:49-246).

Unlike the reference's dispatch chain (Triton -> torch.ops -> Python, with every
error swallowed, ops.py:51-56,159-179), each function here calls exactly one op
and lets errors propagate.  The five reference schemas (pack_codes, unpack_codes,
rotate_and_quantize, attention_scores_packed, attention_values_packed) take tensors on
a HIP device (gfx950 kernels) or in host memory (the CPU kernels the reference also
registers, registration.cpp:106-112); every other op needs HIP-device tensors.
"""

from __future__ import annotations

from typing import Tuple

import torch

from turboquant_kv._lib import ops as _ops, require_device as _require_device
from turboquant_kv._lib import require_tensor as _require_tensor


def pack_codes(codes: torch.Tensor, bit_width: int) -> torch.Tensor:
    _require_tensor(codes, "codes")
    return _ops().pack_codes(codes, bit_width)


def unpack_codes(packed: torch.Tensor, bit_width: int, dim: int) -> torch.Tensor:
    _require_tensor(packed, "packed")
    return _ops().unpack_codes(packed, bit_width, dim)


def rotate_and_quantize(vectors: torch.Tensor, rotation: torch.Tensor, boundaries: torch.Tensor,
                        bit_width: int) -> Tuple[torch.Tensor, torch.Tensor]:
    """(packed, norms fp32) of fp32-upcast vectors (ops.py:74-104)."""
    _require_tensor(vectors, "vectors")
    return _ops().rotate_and_quantize(vectors, rotation, boundaries, bit_width)


def attention_scores_packed(query, packed_keys, key_norms, centroids, rotation, bit_width):
    """scores[b, h, t] = n_t * (R q_bh) . c[code_t], no 1/sqrt(d) (ops.py:131-194)."""
    _require_tensor(query, "query")
    return _ops().attention_scores_packed(query, packed_keys, key_norms, centroids, rotation,
                                          bit_width)


def attention_values_packed(attn_weights, packed_values, value_norms, centroids, rotation_T,
                            bit_width):
    """out[b, h] = (sum_t w n_t c[code_t]) @ rotation_T; pass R itself to invert the
    rotation (ops.py:202-246)."""
    _require_tensor(attn_weights, "attn_weights")
    return _ops().attention_values_packed(attn_weights, packed_values, value_norms, centroids,
                                          rotation_T, bit_width)


def ip_scan_topk(queries, packed, norms, centroids, rotation, bit_width, k):
    """Top-k inner-product search over packed codes: (scores f32 [Q,k], ids i64 [Q,k])."""
    _require_device(queries, "queries")
    return _ops().ip_scan_topk(queries, packed, norms, centroids, rotation, bit_width, k)


def ip_scan_topk_pairs(queries, pairs, norms, centroids, rotation, k):
    """ip_scan_topk over 4-bit pair-layout rows [N, d/2] (byte p = code[2p] << 4 |
    code[2p+1]; d = 64 or 128): the same scores and ids."""
    _require_device(queries, "queries")
    return _ops().ip_scan_topk_pairs(queries, pairs, norms, centroids, rotation, k)


def attention_scores_pairs(query, pairs, key_norms, centroids, rotation):
    """attention_scores_packed over 4-bit pair-layout rows [T, d/2] (d = 64 or 128)."""
    _require_device(query, "query")
    return _ops().attention_scores_pairs(query, pairs, key_norms, centroids, rotation)


def pack_pair_rows(packed, bit_width, dim):
    """Bit-plane rows [n, bits*ceil(d/8)] -> pair rows [n, d*bits/8] (2-4 bits, d 64/128):
    one table index per pair of dims (layout in include/turboquant_hip.h)."""
    _require_device(packed, "packed")
    return _ops().pack_pair_rows(packed, bit_width, dim)


def unpack_pair_rows(rows, bit_width, dim):
    """Pair rows back to the reference's bit-plane rows (reference.py:191-224)."""
    _require_device(rows, "rows")
    return _ops().unpack_pair_rows(rows, bit_width, dim)


def ip_scan_topk_pair_rows(queries, rows, norms, centroids, rotation, bit_width, k):
    """ip_scan_topk over pair rows: identical scores and ids."""
    _require_device(queries, "queries")
    return _ops().ip_scan_topk_pair_rows(queries, rows, norms, centroids, rotation, bit_width, k)


def attention_scores_pair_rows(query, rows, key_norms, centroids, rotation, bit_width):
    """attention_scores_packed over pair rows: identical scores."""
    _require_device(query, "query")
    return _ops().attention_scores_pair_rows(query, rows, key_norms, centroids, rotation, bit_width)


def ip_scan_topk_prod(queries, mse_packed, signs, res_norms, norms, centroids, rotation, qjl,
                      bit_width, k):
    """Top-k of <q, dequantize_prod(row)> (search.py:229-252) scored from the packed rows:
    n * (sum_j (R q)_j c[code_j] + sqrt(pi/2)/d * gamma * sum_j (S q)_j (+-1)_j).
    bit_width is the prod bit budget (2-4); centroids are the (bit_width-1)-bit codebook."""
    _require_device(queries, "queries")
    return _ops().ip_scan_topk_prod(queries, mse_packed, signs, res_norms, norms, centroids,
                                    rotation, qjl, bit_width, k)


def attention_scores_prod(query, mse_packed, signs, res_norms, key_norms, centroids, rotation,
                          qjl, bit_width):
    """<q, dequantize_prod(key_t)> for query [B, H, d] -> [B, H, T] fp32 (no 1/sqrt(d))."""
    _require_device(query, "query")
    return _ops().attention_scores_prod(query, mse_packed, signs, res_norms, key_norms, centroids,
                                        rotation, qjl, bit_width)


def ip_scan_topk_prod_pair_rows(queries, mse_rows, signs, res_norms, norms, centroids, rotation,
                                qjl, bit_width, k):
    """ip_scan_topk_prod with the MSE half as pair rows (bit_width 3 or 4, d 64/128):
    the same scores bit for bit."""
    _require_device(queries, "queries")
    return _ops().ip_scan_topk_prod_pair_rows(queries, mse_rows, signs, res_norms, norms, centroids,
                                              rotation, qjl, bit_width, k)


def attention_scores_prod_pair_rows(query, mse_rows, signs, res_norms, key_norms, centroids,
                                    rotation, qjl, bit_width):
    _require_device(query, "query")
    return _ops().attention_scores_prod_pair_rows(query, mse_rows, signs, res_norms, key_norms,
                                                  centroids, rotation, qjl, bit_width)


def decode_attention_packed(q, kpacked, knorms, vpacked, vnorms, seq_lens, kcentroids,
                            vcentroids, krotation, vrotation, kbits, vbits, scale):
    """Fused GQA decode attention over packed K/V -> [B, Hq, d] in q.dtype."""
    _require_device(q, "q")
    return _ops().decode_attention_packed(q, kpacked, knorms, vpacked, vnorms, seq_lens,
                                          kcentroids, vcentroids, krotation, vrotation, kbits,
                                          vbits, float(scale))


def decode_attention_packed_lse(q, kpacked, knorms, vpacked, vnorms, seq_lens, kcentroids,
                                vcentroids, krotation, vrotation, kbits, vbits, scale):
    """decode_attention_packed plus the per-head log-sum-exp of the scores ([B, Hq] fp32),
    for merging more tokens afterwards."""
    _require_device(q, "q")
    return _ops().decode_attention_packed_lse(q, kpacked, knorms, vpacked, vnorms, seq_lens,
                                              kcentroids, vcentroids, krotation, vrotation, kbits,
                                              vbits, float(scale))


def pack_decode_layout(packed: torch.Tensor, cache: torch.Tensor, dim: int, bit_width: int,
                       values: bool, pos: int) -> None:
    """Write bit-plane rows [streams, n, P] into a decode-layout cache at tokens pos..pos+n
    (keys: [streams, t_cap, dim/2] pair bytes, 4-bit; values: [streams, t_cap/64,
    8*bit_width*dim] tile bytes, 2-4 bit; dim 64)."""
    _require_device(cache, "cache")
    _ops().pack_decode_layout(packed, cache, dim, bit_width, int(values), pos)


def unpack_decode_layout(cache: torch.Tensor, dim: int, bit_width: int, values: bool, t0: int,
                         n: int) -> torch.Tensor:
    """Tokens t0..t0+n of a decode-layout cache as bit-plane rows [streams, n, P]."""
    _require_device(cache, "cache")
    return _ops().unpack_decode_layout(cache, dim, bit_width, int(values), t0, n)


def decode_attention_dl(q, kpairs, knorms, vblocks, vnorms, seq_lens, kcentroids, vcentroids,
                        krotation, vrotation, scale, return_lse: bool = False):
    """decode_attention_packed over a decode-layout cache (4-bit keys, 2-4 bit values --
    the width of the value tiles names it --, head_dim 64 or 128, any number of query heads per
    KV head): [B, Hq, d] in q.dtype (and the [B, Hq] log-sum-exp with return_lse)."""
    _require_device(q, "q")
    if return_lse:
        return _ops().decode_attention_dl_lse(q, kpairs, knorms, vblocks, vnorms, seq_lens,
                                              kcentroids, vcentroids, krotation, vrotation,
                                              float(scale))
    return _ops().decode_attention_dl(q, kpairs, knorms, vblocks, vnorms, seq_lens, kcentroids,
                                      vcentroids, krotation, vrotation, float(scale))


def paged_store(rows, norms, slot_mapping, pool, norm_pool):
    """Scatter rows [n, hkv, P] (+ norms [n, hkv]) to the flat slots slot_mapping [n] of a
    block pool [num_blocks, hkv, block_size, P] (+ [num_blocks, hkv, block_size]); slots
    outside the pool (vLLM's -1 padding) are skipped."""
    _require_device(pool, "pool")
    _ops().paged_store(rows, norms, slot_mapping, pool, norm_pool)


def paged_gather(pool, norm_pool, block_tables, seq_lens, t_max):
    """Rows [B, hkv, t_max, P] and norms [B, hkv, t_max] of each sequence's first
    seq_lens[b] tokens, read through block_tables [B, max_blocks] (zeros past the end)."""
    _require_device(pool, "pool")
    return _ops().paged_gather(pool, norm_pool, block_tables, seq_lens, t_max)


def decode_attention_paged(q, kpool, knorm_pool, vpool, vnorm_pool, block_tables, seq_lens,
                           kcentroids, vcentroids, krotation, vrotation, kbits, vbits, scale,
                           return_lse=False):
    """decode_attention_packed over paged block pools: batch row b attends to its first
    seq_lens[b] tokens, found through block_tables [B, max_blocks]."""
    _require_device(q, "q")
    out, lse = _ops().decode_attention_paged(q, kpool, knorm_pool, vpool, vnorm_pool, block_tables,
                                             seq_lens, kcentroids, vcentroids, krotation, vrotation,
                                             kbits, vbits, scale)
    return (out, lse) if return_lse else out


def paged_store_value_tiles(rows, norms, slot_mapping, vtile_pool, vnorm_pool):
    """Write vb-bit value rows [n, hkv, 8 vb] (bit planes of d = 64, vb = 2-4) and norms
    [n, hkv] into the value tiles vtile_pool -- [num_blocks, hkv, block_size/64, 512 vb] for
    block sizes >= 64, [num_blocks, hkv, block_size/16, 128 vb] for 16 and 32; vb is read
    from the pool's width -- (+ norms [num_blocks, hkv, block_size]) at the flat slots
    slot_mapping [n]; other tokens of a tile keep their bits, slots outside the pool are
    skipped."""
    _require_device(vtile_pool, "vtile_pool")
    _ops().paged_store_value_tiles(rows, norms, slot_mapping, vtile_pool, vnorm_pool)


def decode_attention_paged_dl(q, kpairs_pool, knorm_pool, vtile_pool, vnorm_pool, block_tables,
                              seq_lens, kcentroids, vcentroids, krotation, vrotation, scale,
                              return_lse=False):
    """decode_attention_dl over paged pools in the decode layout (block_size a power of two
    >= 16, 2-4 bit value tiles as paged_store_value_tiles writes them): batch row b attends
    to its first seq_lens[b] tokens through block_tables."""
    _require_device(q, "q")
    out, lse = _ops().decode_attention_paged_dl(q, kpairs_pool, knorm_pool, vtile_pool, vnorm_pool,
                                                block_tables, seq_lens, kcentroids, vcentroids,
                                                krotation, vrotation, float(scale))
    return (out, lse) if return_lse else out


def prefill_attention_paged_dl(q, kpairs_pool, knorm_pool, vtile_pool, vnorm_pool, block_table, T,
                               kcentroids, vcentroids, krotation, vrotation, scale):
    """Causal prefill of one sequence over decode-layout paged pools: its n new tokens
    q [n, Hq, 64] sit at positions T-n .. T-1 and new token i attends to tokens
    0 .. T-n+i, read through block_table [max_blocks].  -> [n, Hq, 64] fp32.  One kernel
    streams each 64-token tile once per 48 query rows (32 for fp32 / fp16 queries)."""
    _require_device(q, "q")
    return _ops().prefill_attention_paged_dl(q, kpairs_pool, knorm_pool, vtile_pool, vnorm_pool,
                                             block_table, int(T), kcentroids, vcentroids,
                                             krotation, vrotation, float(scale))
