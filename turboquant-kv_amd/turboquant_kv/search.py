"""TurboQuantIndex: brute-force inner-product search over packed codes on the GPU.

API of turboquant_kv/search.py:37-317.  The database lives on the device in a
buffer that grows geometrically (the reference re-concatenates on every add,
search.py:145-176).  MSE-mode search runs the fused ADC scan + top-k kernel: the
query is rotated, a per-dimension query x centroid table is built, every packed
row is scored from that table and the top k are kept with equal scores ordered by
lower index (the order of the reference's C++ heap, turboquant_core.cpp:487-494).
Queries are upcast to fp32 before rotation, as the reference's op and C++ paths do
(ops.py:188; bindings.cpp:105); the reference's Python fallback computes in the query
dtype (search.py:209-221).  Prod mode scores against dequantized vectors, as the
reference does (search.py:229-252).

4-bit MSE databases of dim 64 or 128 are kept in the pair layout (row byte p =
code[2p] << 4 | code[2p+1]): the same bytes per row as the bit-plane format, arranged so
that every code is one masked nibble, which the scan turns into a table address with a
single instruction.  Scores and ids are identical to the bit-plane scan.

save/load use the reference's Python file format (search.py:29-34, 254-317); the pair
layout is converted back to bit planes on save and from them on load.  save_tqix /
load_tqix read and write the C++ core's TQIX v1 files (turboquant_core.cpp:559-618):
rotation="core" builds the core's rotation and codebook for the seed, so an index loaded
from a file the core wrote returns the core's own search results.
"""

from __future__ import annotations

import struct
from typing import Optional, Tuple

import numpy as np
import torch

from turboquant_kv import ops
from turboquant_kv._lib import ops as _ops
from turboquant_kv.codebook import (core_codebook, lloyd_max_codebook, make_qjl_matrix,
                                    make_rotation_matrix)
from turboquant_kv.formats import read_tqix, write_tqix

HEADER_FORMAT = "<BII"  # bit_width u8, dim u32, n_vectors u32
HEADER_SIZE = struct.calcsize(HEADER_FORMAT)
MODE_MSE = 0
MODE_PROD = 1
_SCAN_MAX_K = 128  # the fused top-k kernels' per-call limit
# Queries per scan launch at k <= 32 (k above: proportionally fewer): the scans' per-block
# candidate lists grow with queries x k (and a launch takes at most 65,535 queries);
# larger batches run as consecutive launches.
_SEARCH_CHUNK = 4096
# k above _SCAN_MAX_K scores every row into a [Q, N] fp32 matrix: at most this many
# score bytes per launch
_SCORE_BYTES = 1 << 30


def _topk_lowest_index(s: torch.Tensor, k: int) -> Tuple[torch.Tensor, torch.Tensor]:
    """Top k of each row of s [Q, N] (k <= N) by score descending, equal scores in
    increasing index order -- the order of the reference core's heap, which keeps the
    earlier row on a tie (turboquant_core.cpp:487-512) -- and NaN scores never listed
    ((-inf, -1) pads in their place, as the fused scan).  torch.topk alone leaves the order
    of ties unspecified: its k-th value sets a threshold, every score above it is taken,
    then the lowest-index entries at it, and the k winners are sorted stably."""
    nan = torch.isnan(s)
    sc = torch.where(nan, torch.full_like(s, float("-inf")), s)
    kth = torch.topk(sc, k, dim=-1).values[:, -1:]
    above = sc > kth
    tie = (sc == kth) & ~nan
    tie_nan = (sc == kth) & nan  # a NaN ranks below every real score, -inf included
    need = k - above.sum(dim=-1, keepdim=True)
    need_nan = need - tie.sum(dim=-1, keepdim=True)
    take = (above | (tie & (torch.cumsum(tie.to(torch.int32), dim=-1) <= need)) |
            (tie_nan & (torch.cumsum(tie_nan.to(torch.int32), dim=-1) <= need_nan)))
    idx = take.nonzero()[:, 1].view(s.shape[0], k)  # row-major: ascending index per row
    vals = sc.gather(1, idx)
    vals, order = torch.sort(vals, dim=-1, descending=True, stable=True)
    idx = idx.gather(1, order)
    was_nan = nan.gather(1, idx)
    if bool(was_nan.any()):  # NaN rows sit among the -inf ones: make them pads, last
        vals = torch.where(was_nan, torch.full_like(vals, float("-inf")), vals)
        idx = torch.where(was_nan, torch.full_like(idx, -1), idx)
        key = was_nan.to(torch.int32)
        key, order = torch.sort(key, dim=-1, stable=True)
        vals, idx = vals.gather(1, order), idx.gather(1, order)
    return vals, idx


class TurboQuantIndex:
    def __init__(self, dim: int, bit_width: int = 3, mode: str = "mse", rotation: str = "dense_qr",
                 seed: int = 42, device="cuda"):
        if mode not in ("mse", "prod"):
            raise ValueError(f"Unknown mode: {mode}")
        self.dim = dim
        self.bit_width = bit_width
        self.mode = mode
        self.rotation_method = rotation
        self.seed = seed
        self.device = torch.device(device)
        self._use_cpp = False  # attribute of the reference API; the C++ core is not used
        if rotation == "core" and mode != "mse":
            raise ValueError('rotation="core" (the C++ core\'s tables) has no prod mode')
        self._rotation = make_rotation_matrix(dim, seed=seed, method=rotation)
        self._rot_dev = self._rotation.to(self.device)
        if mode == "mse":
            self._codebook = (core_codebook(bit_width, dim) if rotation == "core"
                              else lloyd_max_codebook(bit_width, dim))
            self._code_bits = bit_width
        else:
            self._codebook = lloyd_max_codebook(bit_width - 1, dim)
            self._code_bits = bit_width - 1
            self._S_matrix = make_qjl_matrix(dim, dim, seed)
            self._S_dev = self._S_matrix.to(self.device)
        # 2-4 bit MSE rows of 64/128 dims, and the 2-3 bit MSE halves of prod rows, live as
        # pair rows (same row width): one table read per pair of dims in the scan.
        self._pairs = 2 <= self._code_bits <= (4 if mode == "mse" else 3) and dim in (64, 128)
        self._bnd = self._codebook[0].to(self.device)
        self._cen = self._codebook[1].to(self.device)
        self.n_vectors = 0
        self._cap = 0
        self._packed_buf: Optional[torch.Tensor] = None
        self._norm_buf: Optional[torch.Tensor] = None
        self._sign_buf: Optional[torch.Tensor] = None
        self._res_buf: Optional[torch.Tensor] = None

    # ------------------------------------------------------------------ storage views
    @property
    def _packed_codes(self) -> Optional[torch.Tensor]:
        return None if self._packed_buf is None else self._packed_buf[: self.n_vectors]

    def _bitplane_codes(self) -> Optional[torch.Tensor]:
        """The database rows in the reference's bit-plane format [n, b*ceil(d/8)]."""
        if self._packed_buf is None or not self._pairs:
            return self._packed_codes
        return ops.unpack_pair_rows(self._packed_codes, self._code_bits, self.dim)

    def _store_codes(self, packed: torch.Tensor, pos: int) -> None:
        """Write bit-plane rows at rows pos.. of the database buffer."""
        if self._pairs:
            self._packed_buf[pos: pos + packed.shape[0]] = ops.pack_pair_rows(packed, self._code_bits,
                                                                               self.dim)
        else:
            self._packed_buf[pos: pos + packed.shape[0]] = packed

    @property
    def _norms(self) -> Optional[torch.Tensor]:
        return None if self._norm_buf is None else self._norm_buf[: self.n_vectors]

    @property
    def _qjl_signs(self) -> Optional[torch.Tensor]:
        return None if self._sign_buf is None else self._sign_buf[: self.n_vectors]

    @property
    def _residual_norms(self) -> Optional[torch.Tensor]:
        return None if self._res_buf is None else self._res_buf[: self.n_vectors]

    def _reserve(self, n_total: int) -> None:
        if n_total <= self._cap:
            return
        cap = max(n_total, 2 * self._cap, 1024)
        bpp = (self.dim + 7) // 8
        dev = self.device

        def grow(old, shape, dtype):
            new = torch.empty(shape, dtype=dtype, device=dev)
            if old is not None and self.n_vectors:
                new[: self.n_vectors] = old[: self.n_vectors]
            return new

        self._packed_buf = grow(self._packed_buf, (cap, self._code_bits * bpp), torch.uint8)
        self._norm_buf = grow(self._norm_buf, (cap,), torch.float32)
        if self.mode == "prod":
            self._sign_buf = grow(self._sign_buf, (cap, bpp), torch.uint8)
            self._res_buf = grow(self._res_buf, (cap,), torch.float32)
        self._cap = cap

    @classmethod
    def from_vectors(cls, vectors: torch.Tensor, bit_width: int = 3, mode: str = "mse",
                     rotation: str = "dense_qr", seed: int = 42, device=None) -> "TurboQuantIndex":
        if device is None:
            device = vectors.device if vectors.is_cuda else "cuda"
        idx = cls(dim=vectors.shape[-1], bit_width=bit_width, mode=mode, rotation=rotation,
                  seed=seed, device=device)
        idx.add(vectors)
        return idx

    def add(self, vectors: torch.Tensor) -> None:
        """Quantize (N, dim) or (dim,) vectors on the device and append them."""
        if vectors.dim() == 1:
            vectors = vectors.unsqueeze(0)
        if vectors.shape[-1] != self.dim:
            raise ValueError(f"expected dim {self.dim}, got {vectors.shape[-1]}")
        x = vectors.to(self.device)
        if x.dtype not in (torch.float32, torch.float16, torch.bfloat16):
            x = x.float()
        n = x.shape[0]
        if n == 0:
            return
        self._reserve(self.n_vectors + n)
        sl = slice(self.n_vectors, self.n_vectors + n)
        if self.mode == "mse":
            p, nm = _ops().quantize_mse_packed(x, self._rot_dev, self._bnd, self.bit_width)
            self._store_codes(p, self.n_vectors)
            self._norm_buf[sl] = nm.float()
        else:
            mp, sg, rn, nm = _ops().quantize_prod_packed(x, self._rot_dev, self._bnd, self._cen,
                                                         self._S_dev, self.bit_width)
            self._store_codes(mp, self.n_vectors)
            self._sign_buf[sl] = sg
            self._res_buf[sl] = rn.float()
            self._norm_buf[sl] = nm.float()
        self.n_vectors += n

    def search(self, queries: torch.Tensor, k: int = 10) -> Tuple[torch.Tensor, torch.Tensor]:
        """Top-k inner products: (scores (Q, k'), indices (Q, k')) with k' = min(k, n_vectors).
        Any number of queries: large batches run in consecutive launches."""
        if queries.dim() == 1:
            queries = queries.unsqueeze(0)
        assert self.n_vectors > 0, "Index is empty"
        q = queries.to(self.device)
        k = min(k, self.n_vectors)
        fused = k <= _SCAN_MAX_K and (self.mode == "mse" or self.bit_width <= 4)
        step = (max(1, _SEARCH_CHUNK * 32 // max(k, 32)) if fused
                else max(1, min(_SEARCH_CHUNK, _SCORE_BYTES // (4 * self.n_vectors))))
        recon = None
        if self.mode == "prod" and self.bit_width > 4:  # built once for every chunk
            recon = _ops().dequantize_prod_packed(self._bitplane_codes(), self._qjl_signs,
                                                  self._residual_norms, self._norms, self._cen,
                                                  self._rot_dev, self._S_dev, self.bit_width,
                                                  self.dim)
        if q.shape[0] <= step:
            return self._search(q, k, recon)
        parts = [self._search(q[i:i + step], k, recon) for i in range(0, q.shape[0], step)]
        return torch.cat([p[0] for p in parts]), torch.cat([p[1] for p in parts])

    def _search(self, q: torch.Tensor, k: int,
                recon: Optional[torch.Tensor] = None) -> Tuple[torch.Tensor, torch.Tensor]:
        if self.mode == "mse":
            if k <= _SCAN_MAX_K:
                if self._pairs:
                    return ops.ip_scan_topk_pair_rows(q, self._packed_codes, self._norms, self._cen,
                                                      self._rot_dev, self.bit_width, k)
                return ops.ip_scan_topk(q, self._packed_codes, self._norms, self._cen,
                                        self._rot_dev, self.bit_width, k)
            if self._pairs:
                s = ops.attention_scores_pair_rows(q.float().unsqueeze(0), self._packed_codes,
                                                   self._norms, self._cen, self._rot_dev,
                                                   self.bit_width)[0]
            else:
                s = ops.attention_scores_packed(q.float().unsqueeze(0), self._packed_codes,
                                                self._norms, self._cen, self._rot_dev,
                                                self.bit_width)[0]
            return _topk_lowest_index(s, k)
        if self.bit_width <= 4:
            # Scored from the packed rows: <q, dequantize_prod(row)> rearranged as
            # n * (<R q, c[codes]> + sqrt(pi/2)/d * gamma * <S q, +-1>).
            scan = ops.ip_scan_topk_prod_pair_rows if self._pairs else ops.ip_scan_topk_prod
            scores_of = (ops.attention_scores_prod_pair_rows if self._pairs
                         else ops.attention_scores_prod)
            if k <= _SCAN_MAX_K:
                return scan(q, self._packed_codes, self._qjl_signs, self._residual_norms,
                            self._norms, self._cen, self._rot_dev, self._S_dev, self.bit_width, k)
            s = scores_of(q.float().unsqueeze(0), self._packed_codes, self._qjl_signs,
                          self._residual_norms, self._norms, self._cen, self._rot_dev, self._S_dev,
                          self.bit_width)[0]
            return _topk_lowest_index(s, k)
        if recon is None:
            recon = _ops().dequantize_prod_packed(self._bitplane_codes(), self._qjl_signs,
                                                  self._residual_norms, self._norms, self._cen,
                                                  self._rot_dev, self._S_dev, self.bit_width,
                                                  self.dim)
        scores = q.float() @ recon.t()
        return _topk_lowest_index(scores, k)

    # ------------------------------------------------------------------ persistence
    def save(self, path: str) -> None:
        """header <BII (bit_width, dim, n) + mode byte + packed + norms f32
        [+ signs + residual norms f32] (search.py:254-275)."""
        mode_byte = MODE_MSE if self.mode == "mse" else MODE_PROD
        with open(path, "wb") as f:
            f.write(struct.pack(HEADER_FORMAT, self.bit_width, self.dim, self.n_vectors))
            f.write(struct.pack("<B", mode_byte))
            if self.n_vectors:
                f.write(self._bitplane_codes().cpu().numpy().tobytes())
                f.write(self._norms.cpu().numpy().astype(np.float32).tobytes())
                if self.mode == "prod":
                    f.write(self._qjl_signs.cpu().numpy().tobytes())
                    f.write(self._residual_norms.cpu().numpy().astype(np.float32).tobytes())

    def save_tqix(self, path: str) -> None:
        """Write the index as a TQIX v1 file (turboquant_core.cpp:559-578).  The file keeps
        only (dim, bit_width, seed): a reader rebuilds the C++ core's rotation and codebook,
        so only indexes built with rotation="core" (MSE mode) can be written."""
        if self.mode != "mse" or self.rotation_method != "core":
            raise ValueError('TQIX files hold MSE indexes built with rotation="core"')
        n = self.n_vectors
        packed = (self._bitplane_codes().cpu().numpy() if n else
                  np.zeros((0, self._code_bits * ((self.dim + 7) // 8)), np.uint8))
        norms = self._norms.cpu().numpy() if n else np.zeros(0, np.float32)
        write_tqix(path, self.dim, self.bit_width, self.seed, packed, norms)

    @classmethod
    def load_tqix(cls, path: str, device="cuda") -> "TurboQuantIndex":
        """An index from a TQIX v1 file written by the C++ core (or save_tqix), with the
        core's rotation and codebook for its seed (turboquant_core.cpp:580-618)."""
        f = read_tqix(path)
        idx = cls(dim=f.dim, bit_width=f.bit_width, mode="mse", rotation="core", seed=f.seed,
                  device=device)
        n = f.n_vectors
        if n:
            idx._reserve(n)
            idx._store_codes(torch.from_numpy(f.packed).to(idx.device), 0)
            idx._norm_buf[:n] = torch.from_numpy(f.norms).to(idx.device)
        idx.n_vectors = n
        return idx

    @classmethod
    def load(cls, path: str, rotation: str = "dense_qr", seed: int = 42,
             device="cuda") -> "TurboQuantIndex":
        with open(path, "rb") as f:
            head = f.read(HEADER_SIZE)
            if len(head) != HEADER_SIZE:
                raise ValueError(f"{path}: truncated header")
            bit_width, dim, n = struct.unpack(HEADER_FORMAT, head)
            mb = f.read(1)
            if len(mb) != 1:
                raise ValueError(f"{path}: truncated header")
            mode = "mse" if mb[0] == MODE_MSE else "prod"
            bpp = (dim + 7) // 8
            code_bits = bit_width if mode == "mse" else bit_width - 1

            def take(nbytes):
                buf = f.read(nbytes)
                if len(buf) != nbytes:
                    raise ValueError(f"{path}: truncated body")
                return buf

            packed = np.frombuffer(take(code_bits * bpp * n), dtype=np.uint8).reshape(n, -1)
            norms = np.frombuffer(take(4 * n), dtype=np.float32)
            if mode == "prod":
                signs = np.frombuffer(take(bpp * n), dtype=np.uint8).reshape(n, -1)
                res = np.frombuffer(take(4 * n), dtype=np.float32)
        idx = cls(dim=dim, bit_width=bit_width, mode=mode, rotation=rotation, seed=seed,
                  device=device)
        if n:
            idx._reserve(n)
            idx._store_codes(torch.from_numpy(packed.copy()).to(idx.device), 0)
            idx._norm_buf[:n] = torch.from_numpy(norms.copy()).to(idx.device)
            if mode == "prod":
                idx._sign_buf[:n] = torch.from_numpy(signs.copy()).to(idx.device)
                idx._res_buf[:n] = torch.from_numpy(res.copy()).to(idx.device)
        idx.n_vectors = n
        return idx
