"""Committed golden fixtures (tests/golden/make_golden.py): the oracle reproduces them on
the CPU, and the HIP path reproduces them on the GPU (bit-exact for integer/byte and
fixed-order fp32 results, tolerance for attention)."""
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import canonical

GOLDEN = Path(__file__).resolve().parent / "golden"


def _load(name):
    with np.load(GOLDEN / name, allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


def test_oracle_reproduces_kmeans_fixture():
    g = _load("kmeans_d64.npz")
    labels, centers, counts, indices, offsets = canonical.kmeans_fit(g["x"], g["init"], int(g["iterations"]))
    for name, val in (("labels", labels), ("counts", counts), ("indices", indices), ("offsets", offsets)):
        assert np.array_equal(val, g[name]), name
    assert np.array_equal(centers.view(np.int32), g["centers"].view(np.int32))


def test_oracle_reproduces_base_offset_fixture():
    g = _load("base_offset_d128.npz")
    for bits in (4, 8):
        codes, low, scale, xhat = canonical.base_offset(g["x"], g["labels"], g["centroids"], bits)
        assert np.array_equal(codes, g[f"codes{bits}"])
        assert np.array_equal(low.view(np.int32), g[f"low{bits}"].view(np.int32))
        assert np.array_equal(scale.view(np.int32), g[f"scale{bits}"].view(np.int32))
        assert np.array_equal(torch.from_numpy(xhat).bfloat16().float().numpy(), g[f"xhat{bits}"])


def test_oracle_reproduces_attention_fixture():
    g = _load("sparse_attention_d64.npz")
    out = canonical.sparse_attention(g["q"], g["k"], g["v"], g["map"], g["q_sizes"], g["k_sizes"])
    assert np.allclose(out, g["out"], atol=1e-6)


@pytest.mark.gpu
def test_hip_path_reproduces_fixtures():
    from peco_amd import attention_cuda, clustering_cuda, quantization

    dev = "cuda:0"
    g = _load("kmeans_d64.npz")
    x = torch.from_numpy(g["x"]).bfloat16().to(dev)
    (labels, centers, counts, indices, offsets), = clustering_cuda.kmeans_fit(
        [clustering_cuda.KMeansProblem(x, torch.from_numpy(g["init"]).to(dev))], int(g["iterations"]))
    assert np.array_equal(labels.cpu().numpy(), g["labels"])
    assert np.array_equal(indices.cpu().numpy(), g["indices"])
    assert np.array_equal(centers.cpu().numpy().view(np.int32), g["centers"].view(np.int32))
    g = _load("base_offset_d128.npz")
    xq = torch.from_numpy(g["x"]).bfloat16().to(dev)
    for bits in (4, 8):
        enc = quantization.quantize_base_offset(xq, torch.from_numpy(g["labels"]).to(dev),
                                                torch.from_numpy(g["centroids"]).to(dev), bits)
        assert np.array_equal(enc.codes.cpu().numpy(), g[f"codes{bits}"])
        assert np.array_equal(enc.dequantize().float().cpu().numpy(), g[f"xhat{bits}"])
    g = _load("sparse_attention_d64.npz")
    t = [torch.from_numpy(g[n]).bfloat16()[None].to(dev) for n in ("q", "k", "v")]
    out = attention_cuda.sparse_attention(*t, torch.from_numpy(g["map"])[None].to(dev),
                                          torch.from_numpy(g["q_sizes"])[None].to(dev),
                                          torch.from_numpy(g["k_sizes"])[None].to(dev))
    err = np.abs(out[0].float().cpu().numpy() - g["out"])
    assert err.max() <= 2e-2 and err.mean() <= 2e-3
