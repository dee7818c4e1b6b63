"""The reference's CPU torch path, restated with the same torch operations.

TEST INFRASTRUCTURE ONLY (the CPU baseline that bench.py times, and the pin for
oracle.canonical). Each function names the reference lines it follows; the
reference's CUDA branches are replaced by its CPU branches, and its CUDA-only
sparse attention (peco/attention_cuda.py:98-99 has no CPU path) by a
block-sparse torch attention with the documented semantics.
"""
from __future__ import annotations

import math

import torch
import torch.nn.functional as F


@torch.no_grad()
def fit_token_clusters(x, n_clusters, iterations, init_centroids, *, chunk_size=1024, tol=0.0):
    """Lloyd's k-means, CPU branch of peco/clustering.py:45-89 (explicit initial centres).

    Returns (labels int32 [BH,N], centers fp32 [BH,K,D], counts int32 [BH,K], iteration).
    """
    x = x.float().contiguous()
    batch, tokens, dims = x.shape
    centers = init_centroids.float().contiguous().clone()
    labels = torch.empty((batch, tokens), dtype=torch.int32)
    counts = torch.empty((batch, n_clusters), dtype=torch.int32)
    sums = torch.empty_like(centers)
    means = torch.empty_like(centers)
    chunk_size = min(chunk_size, tokens)
    iteration = 0
    for iteration in range(1, iterations + 1):
        norms = centers.square().sum(-1).unsqueeze(1)
        for start in range(0, tokens, chunk_size):
            part = x[:, start:start + chunk_size]
            distance = -2 * torch.bmm(part, centers.transpose(1, 2))
            distance += norms
            labels[:, start:start + chunk_size] = distance.argmin(-1).to(torch.int32)
        sums.zero_()
        counts.zero_()
        index = labels.long()
        sums.scatter_add_(1, index[..., None].expand(-1, -1, dims), x)
        counts.scatter_add_(1, index, torch.ones_like(labels))
        means.copy_(torch.where(counts[..., None] > 0, sums / counts[..., None].clamp_min(1), centers))
        shift = torch.linalg.vector_norm(means - centers, dim=-1).max().item() if tol > 0 else None
        centers, means = means, centers
        if tol > 0 and shift <= tol:
            break
    return labels, centers, counts, iteration


def stable_indices(labels):
    """int32 [BH,N]: original token at each packed position (peco/clustering.py:105)."""
    return torch.argsort(labels, dim=-1, stable=True).to(torch.int32)


def gather_tokens(tensor, indices):
    """[B,H,N,D] packed into cluster order (peco/clustering.py:121-123)."""
    b, h, n, d = tensor.shape
    return tensor.gather(2, indices.long().view(b, h, n, 1).expand(-1, -1, -1, d))


def restore_tokens(tensor, indices):
    """Inverse of gather_tokens (peco/clustering.py:133-136)."""
    b, h, n, d = tensor.shape
    out = torch.empty_like(tensor)
    out.scatter_(2, indices.long().view(b, h, n, 1).expand(-1, -1, -1, d), tensor)
    return out


def cluster_weights(scores, weights):
    """softmax(scores + log(weights)) with empty clusters at zero (peco/clustering.py:146-151)."""
    scores, weights = scores.float(), weights.float()
    logits = scores + torch.where(weights > 0, weights.log(), -torch.inf)
    top = logits.max(dim=-1, keepdim=True).values
    top = torch.where(torch.isfinite(top), top, torch.zeros_like(top))
    mass = torch.exp(logits - top)
    return mass / mass.sum(dim=-1, keepdim=True).clamp_min(torch.finfo(torch.float32).tiny)


def select_connections(q_centroids, k_centroids, q_sizes, k_sizes, p, min_kc_ratio=0.0):
    """Boolean [B,H,CQ,CK] map of kept cluster pairs (peco/clustering.py:167-186)."""
    scores = torch.matmul(q_centroids.float(), k_centroids.float().transpose(-1, -2))
    scores *= q_centroids.shape[-1] ** -0.5
    probs = cluster_weights(scores, k_sizes.unsqueeze(-2))
    ordered, order = probs.sort(dim=-1, descending=True, stable=True)
    before = ordered.cumsum(-1) - ordered
    keep = before < p
    if p == 1:
        keep.fill_(True)
    keep[..., 0] = True
    minimum = math.ceil(min_kc_ratio * k_centroids.shape[-2])
    if minimum:
        keep[..., :minimum] = True
    dynamic_map = torch.zeros_like(probs, dtype=torch.bool)
    dynamic_map.scatter_(-1, order, keep)
    dynamic_map &= k_sizes.unsqueeze(-2) > 0
    dynamic_map &= q_sizes.unsqueeze(-1) > 0
    return dynamic_map


def quantize(x, labels, centroids, bits):
    """(codes uint8 [BH,N,D], low fp32 [BH,N,1], scale fp32 [BH,N,1]) (peco/quantization.py:111-118)."""
    n, d = x.shape[-2:]
    flat = x.reshape(-1, n, d)
    idx = labels.to(torch.int64)
    cent = centroids.float()
    base = cent.gather(1, idx.unsqueeze(-1).expand(-1, -1, d))
    residual = flat.float() - base
    low = residual.amin(dim=-1, keepdim=True)
    high = residual.amax(dim=-1, keepdim=True)
    levels = (1 << bits) - 1
    raw = (high - low) / levels
    scale = torch.where(raw > 0, raw, torch.ones_like(raw))
    codes = ((residual - low) / scale).round().clamp_(0, levels).to(torch.uint8)
    return codes, low, scale


def dequantize(codes, low, scale, labels, centroids, dtype, shape):
    """Reconstruction of quantize's payload (peco/quantization.py:134-136)."""
    d = codes.shape[-1]
    idx = labels.to(torch.int64)
    base = centroids.float().gather(1, idx.unsqueeze(-1).expand(-1, -1, d))
    residual = low + scale * codes.float()
    return (base + residual).to(dtype).reshape(shape)


def fake_quantize(x, labels, centroids, bits):
    """peco/quantization.py:140-150; bits=0 returns x itself."""
    if bits == 0:
        return x
    codes, low, scale = quantize(x, labels, centroids, bits)
    return dequantize(codes, low, scale, labels, centroids, x.dtype, tuple(x.shape))


def extend_text_partition(dynamic_map, q_sizes, k_sizes, valid_text, text_length):
    """Append [valid text, padding] groups to the cluster partition (peco/processor.py:68-84)."""
    dynamic_map = F.pad(dynamic_map, (0, 2, 0, 2), value=False)
    dynamic_map[..., -2, :-1] = True
    dynamic_map[..., :-1, -2] = True
    dynamic_map[..., -1, -1] = True
    extra = torch.tensor([valid_text, text_length - valid_text], dtype=torch.int32)
    extra = extra.expand(*q_sizes.shape[:-1], 2)
    return (dynamic_map.contiguous(), torch.cat((q_sizes, extra), -1).to(torch.int32).contiguous(),
            torch.cat((k_sizes, extra), -1).to(torch.int32).contiguous())


@torch.no_grad()
def sparse_attention(q, k, v, dynamic_map, q_sizes, k_sizes):
    """Block-sparse CPU attention with the semantics of peco/attention_cuda.py:75-83.

    q [B,H,SQ,D], k/v [B,H,SK,D]; fp32 arithmetic; fully masked rows are zero.
    """
    b, h, sq, d = q.shape
    sk = k.shape[2]
    qf, kf, vf = (t.float().reshape(b * h, -1, d) for t in (q, k, v))
    out = torch.zeros((b * h, sq, d), dtype=torch.float32)
    m = dynamic_map.reshape(b * h, q_sizes.shape[-1], k_sizes.shape[-1])
    qs = q_sizes.reshape(b * h, -1).tolist()
    ks = k_sizes.reshape(b * h, -1).tolist()
    scale = d ** -0.5
    for i in range(b * h):
        kpre = [0]
        for s in ks[i]:
            kpre.append(kpre[-1] + max(0, min(s, sk - kpre[-1])))
        qoff = 0
        for c, s in enumerate(qs[i]):
            s = max(0, min(s, sq - qoff))
            if s:
                kept = torch.nonzero(m[i, c]).flatten().tolist()
                ranges = [torch.arange(kpre[j], kpre[j + 1]) for j in kept if kpre[j + 1] > kpre[j]]
                if ranges:
                    rows = torch.cat(ranges)
                    scores = (qf[i, qoff:qoff + s] @ kf[i, rows].T) * scale
                    out[i, qoff:qoff + s] = torch.softmax(scores, dim=-1) @ vf[i, rows]
            qoff += s
    return out.reshape(b, h, sq, d).to(q.dtype)


@torch.no_grad()
def peco_layer(query, key, value, *, num_q_centroids, num_k_centroids, iterations, q_init, k_init,
               top_p, min_kc_ratio, bits, text_length, valid_text, attention=None, fit=None, stages=None):
    """The sparse (non-warm-up) branch of PecoAttention.attention, peco/processor.py:129-157.

    ``q_init``/``k_init`` are explicit initial centroids [BH,K,D] (the layer's cached state).
    ``attention`` overrides the block-sparse attention (e.g. the float64 C oracle) and
    ``fit(x, clusters, iterations, init)`` the k-means (e.g. the fixed-order C oracle).
    ``stages`` (dict, optional) receives the intermediate tensors.
    Returns the attention output [B,H,S,D] in the input dtype.
    """
    batch, heads, length, dim = query.shape
    n = length - text_length
    q_video = query[:, :, :n].contiguous()
    k_video = key[:, :, :n].contiguous()
    v_video = value[:, :, :n].contiguous()
    bh = batch * heads
    fit = fit or fit_token_clusters
    q_labels, q_cent, q_sizes, _ = fit(q_video.reshape(bh, n, dim), num_q_centroids, iterations, q_init)
    k_labels, k_cent, k_sizes, _ = fit(k_video.reshape(bh, n, dim), num_k_centroids, iterations, k_init)
    q_sizes = q_sizes.reshape(batch, heads, -1)
    k_sizes = k_sizes.reshape(batch, heads, -1)
    dynamic_map = select_connections(q_cent.reshape(batch, heads, -1, dim), k_cent.reshape(batch, heads, -1, dim),
                                     q_sizes, k_sizes, top_p, min_kc_ratio)
    q_hat = fake_quantize(q_video, q_labels, q_cent, bits)
    k_hat = fake_quantize(k_video, k_labels, k_cent, bits)
    q_idx = stable_indices(q_labels)
    k_idx = stable_indices(k_labels)
    q_sorted = gather_tokens(q_hat, q_idx)
    k_sorted = gather_tokens(k_hat, k_idx)
    v_sorted = gather_tokens(v_video, k_idx)
    q_perm = torch.cat((q_sorted, query[:, :, n:]), 2).contiguous()
    k_perm = torch.cat((k_sorted, key[:, :, n:]), 2).contiguous()
    v_perm = torch.cat((v_sorted, value[:, :, n:]), 2).contiguous()
    ext_map, ext_q, ext_k = extend_text_partition(dynamic_map, q_sizes, k_sizes, valid_text, text_length)
    text_idx = torch.arange(n, length, dtype=torch.int32)
    indices = torch.cat((q_idx.reshape(bh, n), text_idx.expand(bh, -1)), -1)
    attend = attention or sparse_attention
    out_perm = attend(q_perm, k_perm, v_perm, ext_map, ext_q, ext_k)
    output = restore_tokens(out_perm, indices)
    if stages is not None:
        stages.update(q_labels=q_labels, k_labels=k_labels, q_centroids=q_cent, k_centroids=k_cent,
                      q_sizes=q_sizes, k_sizes=k_sizes, dynamic_map=dynamic_map, q_hat=q_hat, k_hat=k_hat,
                      q_indices=q_idx, k_indices=k_idx, q_perm=q_perm, k_perm=k_perm, v_perm=v_perm,
                      ext_map=ext_map, ext_q_sizes=ext_q, ext_k_sizes=ext_k, indices=indices, out_perm=out_perm)
    return output


def processor_prologue(attn, hidden_states, encoder_hidden_states, image_rotary_emb, rotary):
    """q, k, v [B,H,S,D] that PecoAttention.__call__ hands to attention (peco/processor.py:163-187).

    Single-stream blocks (no add_q_proj) project [video, text] with the same weights and
    rotate only the video rows; double-stream blocks project the text with the added
    projections and norms. ``rotary(x, freqs)`` is the rotary function.
    """
    text_length = 0 if encoder_hidden_states is None else encoder_hidden_states.shape[1]
    if attn.add_q_proj is None and text_length:
        hidden_states = torch.cat((hidden_states, encoder_hidden_states), 1)

    def split_heads(x):
        return x.unflatten(2, (attn.heads, -1)).transpose(1, 2)

    query, key, value = (split_heads(proj(hidden_states)) for proj in (attn.to_q, attn.to_k, attn.to_v))
    if attn.norm_q is not None:
        query = attn.norm_q(query)
    if attn.norm_k is not None:
        key = attn.norm_k(key)
    if image_rotary_emb is not None:
        if attn.add_q_proj is None and text_length:
            query = torch.cat((rotary(query[:, :, :-text_length], image_rotary_emb), query[:, :, -text_length:]), 2)
            key = torch.cat((rotary(key[:, :, :-text_length], image_rotary_emb), key[:, :, -text_length:]), 2)
        else:
            query, key = (rotary(x, image_rotary_emb) for x in (query, key))
    if attn.add_q_proj is not None and text_length:
        eq, ek, ev = (split_heads(proj(encoder_hidden_states))
                      for proj in (attn.add_q_proj, attn.add_k_proj, attn.add_v_proj))
        if attn.norm_added_q is not None:
            eq = attn.norm_added_q(eq)
        if attn.norm_added_k is not None:
            ek = attn.norm_added_k(ek)
        query, key, value = torch.cat((query, eq), 2), torch.cat((key, ek), 2), torch.cat((value, ev), 2)
    return query.contiguous(), key.contiguous(), value.contiguous()


def processor_epilogue(attn, output, encoder_hidden_states):
    """(video output, text output) of PecoAttention.__call__ from the attention output
    [B,H,S,D] (peco/processor.py:188-197): no output projections when there is no text."""
    text_length = 0 if encoder_hidden_states is None else encoder_hidden_states.shape[1]
    output = output.transpose(1, 2).flatten(2, 3)
    if not text_length:
        return output, encoder_hidden_states
    output, encoder_output = output[:, :-text_length], output[:, -text_length:]
    if getattr(attn, "to_out", None) is not None:
        output = attn.to_out[1](attn.to_out[0](output))
    if getattr(attn, "to_add_out", None) is not None:
        encoder_output = attn.to_add_out(encoder_output)
    return output, encoder_output


def rotary_embedding(x, freqs_cis):
    """diffusers' apply_rotary_emb(x, (cos, sin), use_real=True, use_real_unbind_dim=-1):
    channel pairs (2i, 2i+1) rotated by the tables [S, D] (HunyuanVideo's call)."""
    cos, sin = freqs_cis
    cos, sin = cos[None, None], sin[None, None]
    real, imag = x.reshape(*x.shape[:-1], -1, 2).unbind(-1)
    rotated = torch.stack([-imag, real], dim=-1).flatten(3)
    return (x.float() * cos + rotated.float() * sin).to(x.dtype)
