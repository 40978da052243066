"""TurboQuantMSE / TurboQuantProd: the two algorithms as objects.

The reference names them in its README (README.md:120-121) but exposes only free
functions (reference.py:263-533).  These classes hold the device-resident rotation,
codebook and QJL matrix once and call the same kernels as the free functions.
"""

from __future__ import annotations

import math
from typing import Tuple

import torch

from turboquant_kv import ops
from turboquant_kv._lib import ops as _ops, require_device as _require_device
from turboquant_kv.codebook import lloyd_max_codebook, make_qjl_matrix, make_rotation_matrix


class TurboQuantMSE:
    """Algorithm 1: rotate, scalar Lloyd-Max quantize, bit-plane pack."""

    def __init__(self, dim: int, bits: int, seed: int = 42, rotation: str = "dense_qr",
                 device="cuda"):
        self.dim, self.bits, self.seed = dim, bits, seed
        self.device = torch.device(device)
        self.rotation = make_rotation_matrix(dim, seed=seed, method=rotation).to(self.device)
        bnd, cen = lloyd_max_codebook(bits, dim)
        self.boundaries = bnd.to(self.device)
        self.centroids = cen.to(self.device)

    @property
    def packed_dim(self) -> int:
        return self.bits * ((self.dim + 7) // 8)

    def quantize(self, x: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
        _require_device(x, "x")
        return _ops().quantize_mse_packed(x.reshape(-1, self.dim), self.rotation,
                                          self.boundaries, self.bits)

    def dequantize(self, packed: torch.Tensor, norms: torch.Tensor) -> torch.Tensor:
        return _ops().dequantize_mse_packed(packed, norms, self.centroids, self.rotation,
                                            self.bits, self.dim)

    def scores(self, queries: torch.Tensor, packed: torch.Tensor, norms: torch.Tensor) -> torch.Tensor:
        """<q, x_hat> for every (query, row): [Q, N] fp32."""
        q = queries.reshape(1, -1, self.dim)
        return ops.attention_scores_packed(q, packed, norms, self.centroids, self.rotation,
                                           self.bits)[0]

    def search(self, queries: torch.Tensor, packed: torch.Tensor, norms: torch.Tensor, k: int):
        return ops.ip_scan_topk(queries.reshape(-1, self.dim), packed, norms, self.centroids,
                                self.rotation, self.bits, k)


class TurboQuantProd:
    """Algorithm 2: MSE at bits-1 plus a 1-bit QJL sign sketch of the residual."""

    def __init__(self, dim: int, bits: int, seed: int = 42, rotation: str = "dense_qr",
                 device="cuda"):
        if bits < 2:
            raise ValueError(f"Prod mode requires bits >= 2, got {bits}")
        self.dim, self.bits, self.seed = dim, bits, seed
        self.device = torch.device(device)
        self.rotation = make_rotation_matrix(dim, seed=seed, method=rotation).to(self.device)
        bnd, cen = lloyd_max_codebook(bits - 1, dim)
        self.boundaries = bnd.to(self.device)
        self.centroids = cen.to(self.device)
        self.S = make_qjl_matrix(dim, dim, seed, self.device)

    def quantize(self, x: torch.Tensor):
        """(mse_packed, signs, residual_norms, norms)."""
        _require_device(x, "x")
        return _ops().quantize_prod_packed(x.reshape(-1, self.dim), self.rotation,
                                           self.boundaries, self.centroids, self.S, self.bits)

    def dequantize(self, mse_packed, signs, residual_norms, norms) -> torch.Tensor:
        return _ops().dequantize_prod_packed(mse_packed, signs, residual_norms, norms,
                                             self.centroids, self.rotation, self.S, self.bits,
                                             self.dim)

    @property
    def qjl_scale(self) -> float:
        return math.sqrt(math.pi / 2.0) / self.dim
