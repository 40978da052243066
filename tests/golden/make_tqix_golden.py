"""Write the fixtures that pin TQIX v1 interchange with the reference's C++ core.

Run in the build container after `make -C oracle ref` (which compiles the reference's
csrc/core/turboquant_core.cpp, from where it lies, into oracle/_ref/libtqcore_ref.so):

    python tests/golden/make_tqix_golden.py

Everything written is data produced by the reference core itself:
  * core_d64_b3_s7.tqix -- a file written by turboquant::TurboQuantIndex::save
    (turboquant_core.cpp:559-578) after add() of 300 fixed vectors (dim 64, 3 bits,
    seed 7);
  * tqix.npz -- the vectors, 5 queries and what TurboQuantIndex::load + search returned
    for them (k = 10), and the core's rotation matrices (make_rotation_matrix,
    turboquant_core.cpp:137-213) and codebooks (Codebook, :71-132) for the (dim, seed) and
    (bits, dim) pairs the tests use.
"""

import ctypes
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(os.path.dirname(os.path.dirname(HERE)), "oracle", "_ref", "libtqcore_ref.so")


def main() -> None:
    if not os.path.exists(LIB):
        sys.exit(f"{LIB} is missing: run `make -C oracle ref` first")
    lib = ctypes.CDLL(LIB)
    P = lambda a: a.ctypes.data_as(ctypes.c_void_p)
    rs = np.random.RandomState(11)
    dim, bits, seed, n = 64, 3, 7, 300
    x = (rs.randn(n, dim) * rs.uniform(0.2, 3.0, (n, 1))).astype(np.float32)
    x[5] = 0.0  # a zero vector
    path = os.path.join(HERE, "core_d64_b3_s7.tqix")
    assert lib.ref_index_build_save(dim, bits, seed, P(x), n, path.encode()) == 0
    q = rs.randn(5, dim).astype(np.float32)
    k = 10
    s = np.zeros((5, k), np.float32)
    ids = np.zeros((5, k), np.int64)
    assert lib.ref_index_load_search(path.encode(), P(q), 5, k, P(s), P(ids)) == 0
    out = {"vectors": x, "queries": q, "scores": s, "ids": ids}
    for d, sd in ((64, 7), (128, 42), (200, 3)):
        R = np.zeros((d, d), np.float32)
        lib.ref_make_rotation(d, sd, P(R))
        out[f"R_d{d}_s{sd}"] = R
    for b in (1, 2, 3, 4):
        for d in (64, 128, 200):
            bnd = np.zeros((1 << b) - 1, np.float32)
            cen = np.zeros(1 << b, np.float32)
            lib.ref_codebook(b, d, P(bnd), P(cen))
            out[f"bnd_b{b}_d{d}"] = bnd
            out[f"cen_b{b}_d{d}"] = cen
    np.savez_compressed(os.path.join(HERE, "tqix.npz"), **out)
    print("wrote", path, "and tqix.npz")


if __name__ == "__main__":
    main()
