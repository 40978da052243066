"""Huffman-coded storage of code indices (API of turboquant_kv/entropy.py:37-373).

For disk, not for scoring: the scan and attention kernels read fixed-width bit-plane
rows.  The code is built from the a-priori probabilities of the Lloyd-Max cells of
N(0, 1) (paper Section 3.1), so encoder and decoder share it without storing it.

Stream format (entropy.py:162-195): uint32 LE symbol count, uint32 LE bit count, then the
code words most significant bit first, zero-padded to a byte.  The tree is built exactly
as the reference builds it -- a min-heap of (probability, insertion counter), two pops
merged into a node that takes the next counter -- so the code words, and the bytes, are
the reference's.  The per-symbol bit packing and prefix decoding run in the native
library (tq_huffman_encode / tq_huffman_decode) instead of Python string handling.
"""

from __future__ import annotations

import heapq
import math
from typing import Dict, List, Optional, Tuple

import numpy as np
import torch

from turboquant_kv.codebook import _lloyd_max_unscaled


def compute_codeword_probabilities(bits: int, dim: int) -> np.ndarray:
    """P(code = k) = Phi(b_{k+1}) - Phi(b_k) over the unscaled N(0, 1) Lloyd-Max cells
    (edges -inf, b_1..b_{L-1}, +inf), renormalized to sum to 1 (entropy.py:37-70).  dim
    does not change the cells (the 1/sqrt(d) scale cancels)."""
    from scipy.stats import norm

    bnd, _ = _lloyd_max_unscaled(bits)
    edges = np.concatenate([[-np.inf], bnd, [np.inf]])
    probs = np.zeros(1 << bits, dtype=np.float64)
    for i in range(1 << bits):
        probs[i] = norm.cdf(edges[i + 1]) - norm.cdf(edges[i])
    probs /= probs.sum()
    return probs


class _Node:
    __slots__ = ("key", "symbol", "left", "right")

    def __init__(self, freq: float, counter: int, symbol=None, left=None, right=None):
        self.key = (freq, counter)
        self.symbol, self.left, self.right = symbol, left, right

    def __lt__(self, other: "_Node") -> bool:
        return self.key < other.key


class HuffmanCoder:
    """Prefix code for 2^bits code indices (entropy.py:87-269).  `codebook` maps each
    symbol to its code word as a '0'/'1' string; symbols of probability 0 get the word of
    bits + 8 zeros."""

    def __init__(self, bits: int, dim: int):
        self.bits = bits
        self.dim = dim
        self.n_levels = 1 << bits
        self.probs = compute_codeword_probabilities(bits, dim)
        self.codebook: Dict[int, str] = {}
        self._assign(self._build_tree(), "")
        for i in range(self.n_levels):
            if i not in self.codebook:
                self.codebook[i] = "0" * (bits + 8)
        # decode table: code word -> symbol, later symbols replacing earlier ones for a
        # repeated word, in the codebook's insertion order (entropy.py:121-124)
        self._decode_table = {code: sym for sym, code in self.codebook.items()}
        self._enc = (torch.tensor([int(self.codebook[s], 2) for s in range(self.n_levels)],
                                  dtype=torch.int64),
                     torch.tensor([len(self.codebook[s]) for s in range(self.n_levels)],
                                  dtype=torch.uint8))
        words = list(self._decode_table.items())
        self._dec = (torch.tensor([int(w, 2) for w, _ in words], dtype=torch.int64),
                     torch.tensor([len(w) for w, _ in words], dtype=torch.uint8),
                     torch.tensor([s for _, s in words], dtype=torch.int32))

    def _build_tree(self) -> _Node:
        heap: List[_Node] = []
        counter = 0
        for i in range(self.n_levels):
            if self.probs[i] > 0:
                heapq.heappush(heap, _Node(self.probs[i], counter, symbol=i))
                counter += 1
        if len(heap) == 1:
            only = heapq.heappop(heap)
            return _Node(only.key[0], counter, left=only)
        while len(heap) > 1:
            a = heapq.heappop(heap)
            b = heapq.heappop(heap)
            heapq.heappush(heap, _Node(a.key[0] + b.key[0], counter, left=a, right=b))
            counter += 1
        return heap[0]

    def _assign(self, node: _Node, prefix: str) -> None:
        if node.symbol is not None:
            self.codebook[node.symbol] = prefix if prefix else "0"
            return
        if node.left is not None:
            self._assign(node.left, prefix + "0")
        if node.right is not None:
            self._assign(node.right, prefix + "1")

    def encode(self, codes: torch.Tensor) -> bytes:
        """Code indices (any shape, flattened) -> header + packed code words."""
        from turboquant_kv._lib import ops
        flat = codes.detach().cpu().to(torch.uint8).reshape(-1)
        return bytes(ops().huffman_encode(flat, *self._enc).numpy().tobytes())

    def decode(self, data: bytes, n_symbols: Optional[int] = None) -> torch.Tensor:
        """Header + packed code words -> 1-D uint8 code indices (at most n_symbols, default
        the header's count)."""
        from turboquant_kv._lib import ops
        buf = torch.frombuffer(bytearray(data), dtype=torch.uint8)
        return ops().huffman_decode(buf, -1 if n_symbols is None else int(n_symbols), *self._dec)

    def compression_ratio(self) -> float:
        h = self.entropy()
        return 1.0 if h == 0 else self.bits / h

    def entropy(self) -> float:
        return -sum(p * math.log2(p) for p in self.probs if p > 0)

    def avg_code_length(self) -> float:
        return float(sum(self.probs[i] * len(self.codebook[i]) for i in range(self.n_levels)))

    def __repr__(self) -> str:
        return (f"HuffmanCoder(bits={self.bits}, dim={self.dim}, entropy={self.entropy():.3f}, "
                f"avg_len={self.avg_code_length():.3f})")


class EntropyPackedStorage:
    """Huffman-compressed code tensor (entropy.py:272-373)."""

    def __init__(self, compressed_data: bytes, shape: Tuple[int, ...], bits: int, dim: int,
                 coder: HuffmanCoder):
        self._data = compressed_data
        self.shape = shape
        self.bits = bits
        self.dim = dim
        self._coder = coder

    @classmethod
    def from_codes(cls, codes: torch.Tensor, bits: int, dim: int) -> "EntropyPackedStorage":
        coder = HuffmanCoder(bits, dim)
        return cls(coder.encode(codes), tuple(codes.shape), bits, dim, coder)

    def to_codes(self) -> torch.Tensor:
        return self._coder.decode(self._data).reshape(self.shape)

    @property
    def nbytes(self) -> int:
        return len(self._data)

    @property
    def fixed_width_nbytes(self) -> int:
        n = 1
        for s in self.shape:
            n *= s
        return (n * self.bits + 7) // 8

    @property
    def savings_pct(self) -> float:
        fixed = self.fixed_width_nbytes
        return 0.0 if fixed == 0 else 100.0 * (1.0 - self.nbytes / fixed)

    def __repr__(self) -> str:
        return (f"EntropyPackedStorage(shape={self.shape}, bits={self.bits}, "
                f"compressed={self.nbytes} bytes, savings={self.savings_pct:.1f}%)")


__all__ = ["compute_codeword_probabilities", "HuffmanCoder", "EntropyPackedStorage"]
