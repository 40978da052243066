"""Host-side setup shared by every quantizer: codebooks, rotations, QJL matrices.

These run once on the host (as in the reference) and are then moved to the GPU.
Each reproduces the reference's bits exactly; tests pin them against golden
vectors written from the reference.
"""

from __future__ import annotations

import math
from functools import lru_cache
from typing import Tuple

import numpy as np
import torch


def _lloyd_max_unscaled(bits: int, max_iter: int = 200, tol: float = 1e-12):
    """Lloyd-Max quantizer of N(0, 1) (reference.py:26-54).

    Start from `2^bits` evenly spaced centroids on [-3, 3]; each iteration sets the
    boundaries to centroid midpoints and moves every centroid to the conditional
    mean of its cell, E[X | lo < X < hi] = (pdf(lo) - pdf(hi)) / P(cell) (a cell of
    probability below 1e-15 keeps its centroid).  The loop stops before adopting an
    update whose largest move is below `tol`, or after `max_iter` iterations (the
    4- and 5-bit schedules end at that cap).  Returns float64 (boundaries, centroids).
    """
    from scipy.stats import norm

    levels = 1 << bits
    cent = np.linspace(-3.0, 3.0, levels)
    for _ in range(max_iter):
        mids = 0.5 * (cent[:-1] + cent[1:])
        lo = np.concatenate([[-np.inf], mids])
        hi = np.concatenate([mids, [np.inf]])
        prob = norm.cdf(hi) - norm.cdf(lo)
        upd = cent.copy()
        ok = prob >= 1e-15
        upd[ok] = (norm.pdf(lo[ok]) - norm.pdf(hi[ok])) / prob[ok]
        if np.max(np.abs(upd - cent)) < tol:
            break
        cent = upd
    return 0.5 * (cent[:-1] + cent[1:]), cent


@lru_cache(maxsize=16)
def lloyd_max_codebook(bits: int, dim: int) -> Tuple[torch.Tensor, torch.Tensor]:
    """(boundaries[2^b - 1], centroids[2^b]) float32: the N(0,1) codebook scaled by
    1/sqrt(dim) in float64 before the cast (reference.py:57-73).  The returned
    tensors are shared between calls; do not modify them in place."""
    b, c = _lloyd_max_unscaled(bits)
    s = 1.0 / math.sqrt(dim)
    return (torch.tensor(b * s, dtype=torch.float32), torch.tensor(c * s, dtype=torch.float32))


def make_rotation_matrix(dim: int, seed: int = 42, method: str = "dense_qr") -> torch.Tensor:
    """Orthogonal (dim, dim) float32 matrix (reference.py:81-97).  method "core" gives the
    reference C++ core's matrix for the same seed (turboquant_core.cpp:137-213), the one
    its TQIX index files are written with."""
    if method == "dense_qr":
        return _dense_qr(dim, seed)
    if method == "rht":
        return make_rht_rotation(dim, seed)
    if method == "core":
        return core_rotation(dim, seed)
    raise ValueError(f"Unknown rotation method: {method}")


def core_rotation(dim: int, seed: int) -> torch.Tensor:
    """The reference C++ core's rotation (std::mt19937 Gaussian draw, two-pass modified
    Gram-Schmidt, non-negative diagonal; turboquant_core.cpp:137-213), built by the native
    library's tq_core_rotation."""
    from turboquant_kv._lib import ops
    return ops().core_rotation(dim, seed)


@lru_cache(maxsize=16)
def core_codebook(bits: int, dim: int) -> Tuple[torch.Tensor, torch.Tensor]:
    """The reference C++ core's Lloyd-Max codebook (turboquant_core.cpp:71-132), scaled
    (boundaries[2^b - 1], centroids[2^b]) float32, built by tq_core_codebook.  Shared
    tensors: do not modify them in place."""
    from turboquant_kv._lib import ops
    return tuple(ops().core_codebook(bits, dim))


def _dense_qr(dim: int, seed: int) -> torch.Tensor:
    """QR of a float32 Gaussian matrix from numpy's RandomState(seed), columns
    sign-fixed so diag(R) > 0 (reference.py:100-109)."""
    gauss = np.random.RandomState(seed).randn(dim, dim).astype(np.float32)
    q, r = np.linalg.qr(gauss)
    sign = np.sign(np.diag(r))
    sign[sign == 0] = 1.0
    return torch.from_numpy(np.ascontiguousarray(q * sign[None, :]))


def make_rht_rotation(dim: int, seed: int = 42) -> torch.Tensor:
    """Randomized-Hadamard rotation as an explicit matrix (reference.py:142-183):
    random +-1 diagonal from torch's CPU generator, normalized Sylvester Hadamard
    matrix of the next power of two, H @ D cropped to (dim, dim), re-orthogonalized
    by QR with the same sign fix.  torch's QR result depends on its thread count,
    so it runs single-threaded here: the matrix is the same in every process on one
    host.  Across hosts it is not bit-stable, in the reference as here: the float32
    LAPACK kernels behind torch.linalg.qr differ by CPU, and two hosts' matrices differ
    by an ulp or two per entry (both orthogonal to 1e-6)."""
    nthreads = torch.get_num_threads()
    torch.set_num_threads(1)
    try:
        return _rht(dim, seed)
    finally:
        torch.set_num_threads(nthreads)


def _rht(dim: int, seed: int) -> torch.Tensor:
    gen = torch.Generator().manual_seed(seed)
    n = 1
    while n < dim:
        n <<= 1
    bitsv = torch.randint(0, 2, (n,), generator=gen).bool()
    diag = torch.where(bitsv, torch.ones(n), -torch.ones(n))
    had = torch.ones(1, 1)
    while had.shape[0] < n:
        had = torch.cat([torch.cat([had, had], 1), torch.cat([had, -had], 1)], 0)
    had = had / math.sqrt(n)
    m = (had @ torch.diag(diag))[:dim, :dim]
    q, r = torch.linalg.qr(m)
    s = torch.sign(torch.diag(r))
    s[s == 0] = 1.0
    return (q * s.unsqueeze(0)).float()


def make_qjl_matrix(dim: int, n_sign_bits: int, seed: int, device=None) -> torch.Tensor:
    """QJL projection S (n_sign_bits, dim): standard normal draws from torch's CPU
    generator seeded with seed + 12345 (reference.py:375-389)."""
    gen = torch.Generator(device="cpu").manual_seed(seed + 12345)
    s = torch.randn(n_sign_bits, dim, generator=gen, dtype=torch.float32)
    return s.to(device) if device is not None else s
