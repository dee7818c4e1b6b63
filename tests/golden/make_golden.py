"""Write the golden fixtures of the PECO hot path (small, seeded) from the CPU oracle.

    python tests/golden/make_golden.py

The oracle is pinned independently (tests/test_oracle.py); these fixtures freeze its
outputs so that later changes to the oracle or to the HIP kernels are caught against
committed data. Inputs are bf16-representable values stored as float32.
"""
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))

from oracle import canonical  # noqa: E402


def bf16_round(a):
    u = np.ascontiguousarray(a, np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) >> 16 << 16
    return u.astype(np.uint32).view(np.float32)


def main():
    rng = np.random.default_rng(2024)
    # k-means: 2 heads, 300 tokens, D=64, 8 clusters (two of them duplicates), 5 iterations.
    means = rng.normal(size=(2, 6, 64))
    means = means / np.linalg.norm(means, axis=-1, keepdims=True) * 8
    comp = rng.integers(0, 6, size=(2, 300))
    x = bf16_round(np.take_along_axis(means, comp[..., None], 1) + 1.5 * rng.normal(size=(2, 300, 64)))
    idx = rng.integers(0, 300, size=(2, 8))
    idx[:, 3] = idx[:, 2]
    init = np.take_along_axis(x, idx[..., None], 1).copy()
    labels, centers, counts, indices, offsets = canonical.kmeans_fit(x, init, 5)
    np.savez_compressed(HERE / "kmeans_d64.npz", x=x, init=init, iterations=np.int32(5), labels=labels,
                        centers=centers, counts=counts, indices=indices, offsets=offsets)
    # Base-Offset 4-bit and 8-bit: 2 heads, 100 tokens, D=128 against the fitted centres.
    xq = bf16_round(rng.normal(size=(2, 100, 128)) * 2)
    cq = rng.normal(size=(2, 5, 128)).astype(np.float32)
    lq = rng.integers(0, 5, size=(2, 100)).astype(np.int32)
    out = {"x": xq, "centroids": cq, "labels": lq}
    for bits in (4, 8):
        codes, low, scale, xhat = canonical.base_offset(xq, lq, cq, bits)
        out.update({f"codes{bits}": codes, f"low{bits}": low, f"scale{bits}": scale,
                    f"xhat{bits}": bf16_round(xhat)})
    np.savez_compressed(HERE / "base_offset_d128.npz", **out)
    # Sparse attention: 2 heads, 96 queries, 112 keys, D=64, 4 query / 5 key clusters.
    q = bf16_round(rng.normal(size=(2, 96, 64)))
    k = bf16_round(rng.normal(size=(2, 112, 64)))
    v = bf16_round(rng.normal(size=(2, 112, 64)))
    qs = np.array([[30, 0, 40, 26], [10, 20, 30, 36]], np.int32)
    ks = np.array([[20, 30, 0, 40, 22], [12, 25, 25, 25, 25]], np.int32)
    m = rng.random((2, 4, 5)) < 0.5
    m[0, 3] = False
    o = canonical.sparse_attention(q, k, v, m, qs, ks)
    np.savez_compressed(HERE / "sparse_attention_d64.npz", q=q, k=k, v=v, map=m, q_sizes=qs, k_sizes=ks, out=o)


if __name__ == "__main__":
    main()
