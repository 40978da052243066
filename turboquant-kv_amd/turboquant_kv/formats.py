"""TQIX v1: the index file format of the reference's standalone C++ core
(csrc/core/turboquant_core.cpp:559-618).

    header  6 x uint32 little-endian: magic 0x54514958 ("TQIX"), version 1, dim,
            bit_width, seed, n_vectors                                   (24 bytes)
    body    n_vectors x bit_width*ceil(dim/8) bytes of bit-plane packed codes,
            then n_vectors x float32 norms

The codes are quantized with the core's own rotation and codebook for (dim, seed) and
(bit_width, dim), which the file does not store: a reader rebuilds them
(`codebook.core_rotation`, `codebook.core_codebook`).  TurboQuantIndex.save_tqix /
load_tqix use this module; an index built with rotation="core" is what the core writes.
The reference's Python index format (search.py:254-317) is TurboQuantIndex.save / load.
"""

from __future__ import annotations

import struct
from dataclasses import dataclass

import numpy as np

TQIX_MAGIC = 0x54514958
TQIX_VERSION = 1
_HEADER = struct.Struct("<6I")


@dataclass
class TqixFile:
    dim: int
    bit_width: int
    seed: int
    packed: np.ndarray   # [n, bit_width * ceil(dim/8)] uint8
    norms: np.ndarray    # [n] float32

    @property
    def n_vectors(self) -> int:
        return int(self.norms.shape[0])


def packed_width(dim: int, bit_width: int) -> int:
    return bit_width * ((dim + 7) // 8)


def write_tqix(path: str, dim: int, bit_width: int, seed: int, packed, norms) -> None:
    """Write a TQIX v1 file (turboquant_core.cpp:559-578); seed is stored as uint32."""
    packed = np.ascontiguousarray(np.asarray(packed, dtype=np.uint8))
    norms = np.ascontiguousarray(np.asarray(norms, dtype=np.float32))
    n = norms.shape[0]
    if packed.shape != (n, packed_width(dim, bit_width)):
        raise ValueError(f"packed must be [{n}, {packed_width(dim, bit_width)}], got {packed.shape}")
    with open(path, "wb") as f:
        f.write(_HEADER.pack(TQIX_MAGIC, TQIX_VERSION, dim, bit_width, seed & 0xFFFFFFFF, n))
        f.write(packed.tobytes())
        f.write(norms.astype("<f4").tobytes())


def read_tqix(path: str) -> TqixFile:
    """Read a TQIX v1 file; raises ValueError for a bad magic, an unsupported version or a
    truncated body, as the core's loader refuses them (turboquant_core.cpp:580-618)."""
    with open(path, "rb") as f:
        head = f.read(_HEADER.size)
        if len(head) < 4 or struct.unpack("<I", head[:4])[0] != TQIX_MAGIC:
            raise ValueError("Invalid TQIDX file (bad magic)")
        if len(head) < 8 or struct.unpack("<I", head[4:8])[0] != TQIX_VERSION:
            raise ValueError("Unsupported TQIDX version")
        if len(head) != _HEADER.size:
            raise ValueError(f"Read error / truncated file: {path}")
        _, _, dim, bit_width, seed, n = _HEADER.unpack(head)
        pw = packed_width(dim, bit_width)
        body = f.read(n * pw + 4 * n)
    if len(body) != n * pw + 4 * n:
        raise ValueError(f"Read error / truncated file: {path}")
    packed = np.frombuffer(body, dtype=np.uint8, count=n * pw).reshape(n, pw).copy()
    norms = np.frombuffer(body, dtype="<f4", count=n, offset=n * pw).astype(np.float32)
    seed_signed = seed - (1 << 32) if seed >= (1 << 31) else seed  # the core reads an int
    return TqixFile(dim, bit_width, seed_signed, packed, norms)
