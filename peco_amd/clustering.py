"""Group similar tokens and select the cluster pairs used by PECO attention.

Same interface as peco/clustering.py. Each batch/head is clustered independently on
the GPU by the fused HIP k-means (clustering_cuda.kmeans_fit); labels follow the
fixed-order fp32 definition documented in peco_amd/csrc/kmeans.hip. Inputs must be
GPU tensors: CPU execution of this path exists only in the test oracle.
"""
from __future__ import annotations

import math

import torch

from . import clustering_cuda


def _require_gpu(*tensors):
    if any(not t.is_cuda for t in tensors if t is not None):
        raise ValueError("peco_amd clustering runs on GPU tensors; CPU tensors are not supported")


@torch.no_grad()
def fit_token_clusters(x, n_clusters, max_iters=100, tol=1e-4, init_centroids=None, *, chunk_size=1024):
    """Run Euclidean Lloyd updates independently for each batch/head.

    Input features have shape [BH,N,D]. Optional initial centers [BH,K,D] allow reuse
    across denoising steps. Returns labels [BH,N] int32, centers [BH,K,D] fp32, counts
    [BH,K] int32 and the iteration count (peco/clustering.py:17-89). ``tol=0`` runs the
    fixed iteration count with no host synchronization; ``tol>0`` stops once the largest
    centre displacement is <= tol (one host sync per iteration). ``chunk_size`` is
    validated for compatibility; the MFMA assignment needs no token chunking.
    """
    if x.ndim != 3 or not x.is_floating_point():
        raise ValueError("x must be a floating tensor with shape [batch_heads, tokens, dims]")
    batch, tokens, dims = x.shape
    if min(batch, tokens, dims) <= 0:
        raise ValueError("x dimensions must be nonzero")
    if not isinstance(n_clusters, int) or not 1 <= n_clusters <= tokens:
        raise ValueError("n_clusters must be an integer in [1, tokens]")
    if not isinstance(max_iters, int) or max_iters < 1:
        raise ValueError("max_iters must be a positive integer")
    if tol < 0 or not math.isfinite(tol):
        raise ValueError("tol must be finite and nonnegative")
    if not isinstance(chunk_size, int) or chunk_size < 1:
        raise ValueError("chunk_size must be a positive integer")
    _require_gpu(x, init_centroids)
    if x.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        x = x.float()
    if x.stride(2) != 1 or x.stride(1) != dims:
        x = x.contiguous()
    if init_centroids is None:
        indices = torch.randint(tokens, (batch, n_clusters), device=x.device)
        centers = x.float().gather(1, indices[..., None].expand(-1, -1, dims)).contiguous()
    else:
        if init_centroids.shape != (batch, n_clusters, dims) or init_centroids.device != x.device:
            raise ValueError("init_centroids must match [batch_heads, n_clusters, dims] and x.device")
        centers = init_centroids.float().contiguous()
    if tol == 0:
        labels, centers, counts, _, _ = clustering_cuda.kmeans_fit(
            [clustering_cuda.KMeansProblem(x, centers)], max_iters)[0]
        return labels, centers, counts, max_iters
    iteration = 0
    for iteration in range(1, max_iters + 1):
        labels, means, counts, _, _ = clustering_cuda.kmeans_fit([clustering_cuda.KMeansProblem(x, centers)], 1)[0]
        shift = torch.linalg.vector_norm(means - centers, dim=-1).max().item()
        centers = means
        if shift <= tol:
            break
    return labels, centers, counts, iteration


def _prepare_sequence_indices(tensor, labels, dim, sorted_indices):
    """Validate token reordering and return contiguous int32 indices [BH,N] (peco/clustering.py:92-108)."""
    if tensor.ndim != 4 or dim not in (2, -2):
        raise ValueError("permutation expects [batch, heads, tokens, dims] with dim=2")
    if tensor.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        raise ValueError("permutation supports float16, bfloat16, and float32")
    batch, heads, tokens, _ = tensor.shape
    if min(tensor.shape) <= 0:
        raise ValueError("permutation tensor dimensions must be nonzero")
    if sorted_indices is None:
        if labels is None or labels.numel() != batch * heads * tokens or labels.device != tensor.device:
            raise ValueError("labels must contain one cluster ID per token on the same device")
        # Stable sort keeps the original order inside each cluster.
        sorted_indices = torch.argsort(labels.reshape(batch * heads, tokens), dim=-1, stable=True)
    if sorted_indices.numel() != batch * heads * tokens or sorted_indices.device != tensor.device:
        raise ValueError("sorted_indices must contain one index per token on the same device")
    return sorted_indices.reshape(batch * heads, tokens).to(torch.int32).contiguous()


@torch.no_grad()
def gather_clustered_tokens(tensor, labels, dim=2, sorted_indices=None):
    """Pack [B,H,N,D] features into cluster order and return the gather indices.

    ``indices[bh, j]`` is the original token at packed position ``j``; pass them when
    packing V to reuse exactly the K ordering.
    """
    indices = _prepare_sequence_indices(tensor, labels, dim, sorted_indices)
    _require_gpu(tensor)
    return clustering_cuda.reorder_token_features(tensor, indices), indices


@torch.no_grad()
def restore_sequence_order(tensor, sorted_indices, dim=2):
    """Scatter packed features back to the original sequence using gather indices."""
    indices = _prepare_sequence_indices(tensor, None, dim, sorted_indices)
    _require_gpu(tensor)
    return clustering_cuda.reorder_token_features(tensor, indices, inverse=True)


@torch.no_grad()
def compute_cluster_weights(scores, weights):
    """softmax(scores + log(counts)) over key clusters in FP32 (peco/clustering.py:140-151).

    Empty clusters contribute zero mass; an entirely empty row returns zeros.
    """
    scores, weights = scores.float(), weights.float()
    logits = scores + torch.where(weights > 0, weights.log(), -torch.inf)
    row_max = logits.max(dim=-1, keepdim=True).values
    row_max = torch.where(torch.isfinite(row_max), row_max, torch.zeros_like(row_max))
    mass = torch.exp(logits - row_max)
    return mass / mass.sum(dim=-1, keepdim=True).clamp_min(torch.finfo(torch.float32).tiny)


@torch.no_grad()
def select_cluster_connections(query_centroids, key_centroids, q_cluster_sizes, k_cluster_sizes, p, min_kc_ratio=0):
    """Choose nonempty query/key cluster pairs from estimated attention mass.

    Centroids are [B,H,C,D], sizes [B,H,C]. For each query cluster keep the smallest
    descending-probability prefix reaching ``p``, and at least ceil(min_kc_ratio*CK) key
    clusters. Returns a bool [B,H,CQ,CK] map; empty clusters never pair
    (peco/clustering.py:155-186). Runs as one HIP launch (peco_select_cluster_connections).
    """
    if not 0 <= p <= 1 or not 0 <= min_kc_ratio <= 1:
        raise ValueError("p and min_kc_ratio must be in [0, 1]")
    _require_gpu(query_centroids, key_centroids, q_cluster_sizes, k_cluster_sizes)
    minimum = math.ceil(min_kc_ratio * key_centroids.shape[-2])
    dynamic_map, _, _ = clustering_cuda.select_connections(query_centroids, key_centroids, q_cluster_sizes,
                                                           k_cluster_sizes, p, minimum)
    return dynamic_map
