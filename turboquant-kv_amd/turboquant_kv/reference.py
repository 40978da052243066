"""TurboQuant quantize / dequantize with the reference's Python signatures.

Drop-in for turboquant_kv/reference.py: the same public functions and arguments,
computed by the gfx950 kernels behind torch.ops.turboquant.  Tensors to quantize
must live on a HIP device (there is no CPU path).  Host-side setup (codebooks,
rotations, QJL matrices) is re-exported from turboquant_kv.codebook.

Numerics follow reference.py: intermediates are rounded to the input dtype
(bf16/fp16 inputs quantize in bf16/fp16), a value equal to a boundary takes the
lower code, quantize_prod normalizes twice (reference.py:431,441).
"""

from __future__ import annotations

from typing import Optional, Tuple

import torch

from turboquant_kv._lib import ops as _ops, require_device as _require_device
from turboquant_kv.codebook import (  # noqa: F401  (re-exported API)
    lloyd_max_codebook,
    make_rht_rotation,
    make_rotation_matrix,
)
from turboquant_kv.codebook import make_qjl_matrix


def _make_qjl_matrix(dim: int, n_sign_bits: int, seed: int, device) -> torch.Tensor:
    """reference.py:375-389 signature."""
    return make_qjl_matrix(dim, n_sign_bits, seed, device)


def pack_codes(codes: torch.Tensor, bits: int) -> torch.Tensor:
    """(N, d) uint8 codes -> (N, bits * ceil(d/8)) bit planes (reference.py:191-224)."""
    _require_device(codes, "codes")
    return _ops().pack_codes(codes.to(torch.uint8), bits)


def unpack_codes(packed: torch.Tensor, bits: int, dim: int) -> torch.Tensor:
    """Inverse of pack_codes (reference.py:227-255)."""
    _require_device(packed, "packed")
    return _ops().unpack_codes(packed, bits, dim)


def _resolve(vectors_device, d, bits, rotation, codebook, seed, rotation_method):
    if rotation is None:
        rotation = make_rotation_matrix(d, seed=seed, method=rotation_method)
    if codebook is None:
        codebook = lloyd_max_codebook(bits, d)
    return rotation.to(vectors_device), codebook


def quantize_mse(
    vectors: torch.Tensor,
    bits: int,
    dim: Optional[int] = None,
    rotation: Optional[torch.Tensor] = None,
    codebook: Optional[Tuple[torch.Tensor, torch.Tensor]] = None,
    seed: int = 42,
    rotation_method: str = "dense_qr",
) -> Tuple[torch.Tensor, torch.Tensor]:
    """TurboQuant_MSE (reference.py:263-317).  Returns (packed (N, bits*ceil(d/8)) uint8,
    norms (N,) in vectors.dtype)."""
    _require_device(vectors, "vectors")
    d = dim if dim is not None else vectors.shape[-1]
    flat = vectors.reshape(-1, d)
    rotation, codebook = _resolve(flat.device, d, bits, rotation, codebook, seed, rotation_method)
    boundaries = codebook[0]
    return _ops().quantize_mse_packed(flat, rotation, boundaries.to(flat.device), bits)


def dequantize_mse(
    packed_codes: torch.Tensor,
    norms: torch.Tensor,
    bits: int,
    dim: int,
    rotation: Optional[torch.Tensor] = None,
    codebook: Optional[Tuple[torch.Tensor, torch.Tensor]] = None,
    seed: int = 42,
    rotation_method: str = "dense_qr",
) -> torch.Tensor:
    """(c[codes] @ R) * norms in norms.dtype (reference.py:320-367)."""
    _require_device(packed_codes, "packed_codes")
    rotation, codebook = _resolve(packed_codes.device, dim, bits, rotation, codebook, seed,
                                  rotation_method)
    centroids = codebook[1].to(packed_codes.device)
    return _ops().dequantize_mse_packed(packed_codes, norms.to(packed_codes.device), centroids,
                                        rotation, bits, dim)


def quantize_prod(
    vectors: torch.Tensor,
    bits: int,
    dim: Optional[int] = None,
    rotation: Optional[torch.Tensor] = None,
    codebook: Optional[Tuple[torch.Tensor, torch.Tensor]] = None,
    S_matrix: Optional[torch.Tensor] = None,
    seed: int = 42,
    rotation_method: str = "dense_qr",
) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    """TurboQuant_prod (reference.py:392-469): MSE at bits-1 plus 1-bit QJL residual signs.
    Returns (mse_packed, qjl_signs, residual_norms, norms)."""
    _require_device(vectors, "vectors")
    if bits - 1 < 1:
        raise ValueError(f"Prod mode requires bits >= 2, got {bits}")
    d = dim if dim is not None else vectors.shape[-1]
    flat = vectors.reshape(-1, d)
    rotation, codebook = _resolve(flat.device, d, bits - 1, rotation, codebook, seed,
                                  rotation_method)
    if S_matrix is None:
        S_matrix = make_qjl_matrix(d, d, seed)
    dev = flat.device
    return _ops().quantize_prod_packed(flat, rotation, codebook[0].to(dev), codebook[1].to(dev),
                                       S_matrix.to(dev), bits)


def dequantize_prod(
    mse_packed: torch.Tensor,
    qjl_signs: torch.Tensor,
    residual_norms: torch.Tensor,
    norms: torch.Tensor,
    bits: int,
    dim: int,
    rotation: Optional[torch.Tensor] = None,
    codebook: Optional[Tuple[torch.Tensor, torch.Tensor]] = None,
    S_matrix: Optional[torch.Tensor] = None,
    seed: int = 42,
    rotation_method: str = "dense_qr",
) -> torch.Tensor:
    """(c[codes] @ R + sqrt(pi/2)/d * gamma * (s @ S)) * norms (reference.py:472-533)."""
    _require_device(mse_packed, "mse_packed")
    dev = mse_packed.device
    rotation, codebook = _resolve(dev, dim, bits - 1, rotation, codebook, seed, rotation_method)
    if S_matrix is None:
        S_matrix = make_qjl_matrix(dim, dim, seed)
    return _ops().dequantize_prod_packed(mse_packed, qjl_signs.to(dev), residual_norms.to(dev),
                                         norms.to(dev), codebook[1].to(dev), rotation,
                                         S_matrix.to(dev), bits, dim)


__all__ = [
    "lloyd_max_codebook",
    "make_rotation_matrix",
    "make_rht_rotation",
    "pack_codes",
    "unpack_codes",
    "quantize_mse",
    "dequantize_mse",
    "quantize_prod",
    "dequantize_prod",
]
