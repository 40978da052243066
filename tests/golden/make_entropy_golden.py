"""Write the fixtures that pin the Huffman code storage (turboquant_kv/entropy.py).

Run in the build container, which has the reference checked out:

    python tests/golden/make_entropy_golden.py /root/reference

It imports the reference's own entropy module -- nothing else fixes its code words (the
tree's tie-breaking) or its byte stream -- and records, as data: the codeword
probabilities and code words for bits 1-5 at dims 64 and 128, and for a few fixed code
arrays the bytes HuffmanCoder.encode returned and what decode returned for them.
"""

import os
import sys

import numpy as np


def main(ref_root: str) -> None:
    sys.path.insert(0, ref_root)
    import torch
    from turboquant_kv.entropy import EntropyPackedStorage, HuffmanCoder, compute_codeword_probabilities

    out = {}
    for bits in (1, 2, 3, 4, 5):
        for dim in (64, 128):
            out[f"probs_b{bits}_d{dim}"] = compute_codeword_probabilities(bits, dim)
            coder = HuffmanCoder(bits, dim)
            words = [coder.codebook[s] for s in range(1 << bits)]
            out[f"lens_b{bits}_d{dim}"] = np.array([len(w) for w in words], np.int32)
            out[f"words_b{bits}_d{dim}"] = np.array([int(w, 2) for w in words], np.int64)
    rs = np.random.RandomState(2)
    cases = [(4, 128, (300, 128)), (3, 64, (7, 64)), (2, 128, (1, 5)), (1, 64, (33,)), (5, 128, (40, 16))]
    for i, (bits, dim, shape) in enumerate(cases):
        codes = rs.randint(0, 1 << bits, shape).astype(np.uint8)
        st = EntropyPackedStorage.from_codes(torch.from_numpy(codes), bits, dim)
        out[f"case{i}_meta"] = np.array([bits, dim], np.int32)
        out[f"case{i}_codes"] = codes
        out[f"case{i}_bytes"] = np.frombuffer(st._data, np.uint8).copy()
        out[f"case{i}_decoded"] = st.to_codes().numpy()
        out[f"case{i}_savings"] = np.array(st.savings_pct)
    empty = HuffmanCoder(4, 64).encode(torch.zeros(0, dtype=torch.uint8))
    out["empty_bytes"] = np.frombuffer(empty, np.uint8).copy()
    np.savez_compressed(os.path.join(os.path.dirname(os.path.abspath(__file__)), "entropy.npz"), **out)
    print("wrote entropy.npz")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
