"""Write the golden vectors that pin the parts of the reference no closed form pins.

Run ONCE, in the build container that has the reference checked out at
/root/reference (it never travels to the GPU box):

    python tests/golden/make_golden.py /root/reference

It imports the reference's own Python (turboquant_kv.reference, .search, .cache)
and records inputs and outputs as small ``.npz`` files next to this script.
Only data is written: inputs, and what the reference returned for them.

What is pinned here and why no closed form does it:
  * ``lloyd_max_codebook`` float32 bits (reference.py:26-73). The 4- and 5-bit
    iterations stop at the 200-iteration cap, so the bits are an iterate of
    that exact schedule, not a textbook table.
  * ``make_rotation_matrix`` (reference.py:100-109): numpy RandomState + LAPACK
    QR; the bits depend on the LAPACK build.
  * ``_make_qjl_matrix`` (reference.py:375-389): torch CPU generator stream.
  * ``quantize_mse`` / ``quantize_prod`` / ``dequantize_*`` outputs
    (reference.py:263-533) on fixed inputs: the fp32 GEMM summation order is
    the library's, so only the reference's own run fixes its codes.
  * ``TurboQuantIndex.search`` (search.py:206-227) and
    ``QuantizedKVCache.attention_scores/values`` (cache.py:282-339).
"""

import os
import sys

import numpy as np


def main(ref_root: str) -> None:
    sys.path.insert(0, ref_root)
    import torch
    from turboquant_kv import reference as R
    from turboquant_kv.search import TurboQuantIndex
    from turboquant_kv.cache import QuantizedKVCache
    from turboquant_kv.config import TurboQuantConfig

    out_dir = os.path.dirname(os.path.abspath(__file__))
    torch.set_num_threads(1)

    # ---------------- codebooks ----------------
    cb = {}
    for b in range(1, 6):
        for d in (64, 128, 200):
            bnd, cen = R.lloyd_max_codebook(b, d)
            cb[f"bnd_b{b}_d{d}"] = bnd.numpy().astype(np.float32)
            cb[f"cen_b{b}_d{d}"] = cen.numpy().astype(np.float32)
    np.savez_compressed(os.path.join(out_dir, "codebook.npz"), **cb)

    # ---------------- rotations and QJL matrices ----------------
    rot = {}
    qjl = {}
    for d in (64, 128, 200):
        for s in (42, 43):
            rot[f"R_d{d}_s{s}"] = R.make_rotation_matrix(d, seed=s).numpy()
            qjl[f"S_d{d}_s{s}"] = R._make_qjl_matrix(d, d, s, torch.device("cpu")).numpy()
    for d in (64, 128):
        rot[f"RHT_d{d}_s42"] = R.make_rht_rotation(d, seed=42).numpy()
    np.savez_compressed(os.path.join(out_dir, "rotation.npz"), **rot)
    np.savez_compressed(os.path.join(out_dir, "qjl.npz"), **qjl)

    # ---------------- quantize_mse, fp32 inputs ----------------
    rs = np.random.RandomState(2024)

    def special_rows(x):
        x[0] = 0.0                                  # zero vector: code #{bnd < 0}
        x[1] = rs.randn(x.shape[1]) * 1e-12         # norm below the 1e-10 clamp
        x[2] = 0.0
        x[2, 3] = 5.0                               # one-hot: rotated row = a column of R
        return x

    mse = {}
    cases = {"d128": (1024, 128, (2, 3, 4)), "d200": (512, 200, (3, 4)), "d64": (1024, 64, (2, 3, 4))}
    for name, (n, d, bits_list) in cases.items():
        x = special_rows(rs.randn(n, d).astype(np.float32))
        mse[f"{name}_x"] = x
        Rm = R.make_rotation_matrix(d, seed=42)
        xt = torch.from_numpy(x)
        for b in bits_list:
            cbk = R.lloyd_max_codebook(b, d)
            packed, norms = R.quantize_mse(xt, b, rotation=Rm, codebook=cbk)
            mse[f"{name}_b{b}_packed"] = packed.numpy()
            mse[f"{name}_b{b}_norms"] = norms.numpy()
            deq = R.dequantize_mse(packed[:64], norms[:64], b, d, rotation=Rm, codebook=cbk)
            mse[f"{name}_b{b}_deq64"] = deq.numpy()

    # bf16 inputs: the reference quantizes in bf16 (R and boundaries cast to bf16)
    d = 64
    xb = special_rows(rs.randn(1024, d).astype(np.float32))
    xb[3:16] *= 20.0                                # a few outlier-scale rows
    xbt = torch.from_numpy(xb).to(torch.bfloat16)
    mse["bf16_d64_x_u16"] = xbt.view(torch.int16).numpy().view(np.uint16)
    Rm = R.make_rotation_matrix(d, seed=42)
    for b in (2, 3, 4):
        cbk = R.lloyd_max_codebook(b, d)
        packed, norms = R.quantize_mse(xbt, b, rotation=Rm, codebook=cbk)
        mse[f"bf16_d64_b{b}_packed"] = packed.numpy()
        mse[f"bf16_d64_b{b}_norms_u16"] = norms.view(torch.int16).numpy().view(np.uint16)
    np.savez_compressed(os.path.join(out_dir, "quant_mse.npz"), **mse)

    # ---------------- quantize_prod ----------------
    prod = {}
    # heavy-tailed non-negative integers 0..255 (config 3a distribution, small N)
    xh = np.clip(np.floor(np.abs(rs.randn(1024, 128) * 40.0)), 0, 255).astype(np.float32)
    xh[0] = 0.0
    # per-dimension log-normal scales (config 3b distribution, small N)
    g = rs.randn(200)
    xl = (rs.randn(512, 200) * np.exp(g)[None, :]).astype(np.float32)
    for name, x in (("d128", xh), ("d200", xl)):
        d = x.shape[1]
        Rm = R.make_rotation_matrix(d, seed=42)
        S = R._make_qjl_matrix(d, d, 42, torch.device("cpu"))
        cbk = R.lloyd_max_codebook(3, d)
        xt = torch.from_numpy(x)
        mp, sg, rn, nm = R.quantize_prod(xt, 4, rotation=Rm, codebook=cbk, S_matrix=S)
        prod[f"{name}_x"] = x
        prod[f"{name}_mse_packed"] = mp.numpy()
        prod[f"{name}_signs"] = sg.numpy()
        prod[f"{name}_res_norms"] = rn.numpy()
        prod[f"{name}_norms"] = nm.numpy()
        deq = R.dequantize_prod(mp[:64], sg[:64], rn[:64], nm[:64], 4, d,
                                rotation=Rm, codebook=cbk, S_matrix=S)
        prod[f"{name}_deq64"] = deq.numpy()
    np.savez_compressed(os.path.join(out_dir, "quant_prod.npz"), **prod)

    # ---------------- TurboQuantIndex.search (Python path) ----------------
    idx = {}
    db = torch.from_numpy(mse["d128_x"])
    q = torch.from_numpy(rs.randn(16, 128).astype(np.float32))
    idx["queries"] = q.numpy()
    for b in (2, 3, 4):
        index = TurboQuantIndex.from_vectors(db, bit_width=b, mode="mse")
        assert not index._use_cpp
        sc, ids = index.search(q, k=10)
        idx[f"b{b}_scores"] = sc.numpy()
        idx[f"b{b}_ids"] = ids.numpy()
        idx[f"b{b}_packed"] = index._packed_codes.numpy()
    np.savez_compressed(os.path.join(out_dir, "index.npz"), **idx)

    # ---------------- QuantizedKVCache scores / values ----------------
    cache = {}
    H, T, d = 4, 128, 64
    k = rs.randn(H, T, d).astype(np.float32)
    v = rs.randn(H, T, d).astype(np.float32)
    qq = rs.randn(H, 1, d).astype(np.float32)
    cfg = TurboQuantConfig(key_bits=4, value_bits=2, mode="mse")
    kv = QuantizedKVCache(cfg, 1, T, H, d, device="cpu")
    kv.append(0, torch.from_numpy(k[:, :100]), torch.from_numpy(v[:, :100]))
    kv.append(0, torch.from_numpy(k[:, 100:]), torch.from_numpy(v[:, 100:]))
    logits = kv.attention_scores(0, torch.from_numpy(qq))
    w = torch.softmax(logits, dim=-1)
    o = kv.attention_values(0, w)
    cache.update(keys=k, values=v, query=qq, logits=logits.numpy(), weights=w.numpy(),
                 output=o.numpy(), key_packed=kv._key_packed[0].numpy(),
                 key_norms=kv._key_norms[0].numpy(), val_packed=kv._val_packed[0].numpy(),
                 val_norms=kv._val_norms[0].numpy(), memory_bytes=np.int64(kv.memory_bytes()))
    np.savez_compressed(os.path.join(out_dir, "cache.npz"), **cache)

    total = sum(os.path.getsize(os.path.join(out_dir, f)) for f in os.listdir(out_dir)
                if f.endswith(".npz"))
    print(f"wrote fixtures: {total / 1e6:.2f} MB")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
