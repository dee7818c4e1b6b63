"""HunyuanVideo attention processor with PECO cluster-sparse attention (peco/processor.py interface).

The sparse path of ``PecoAttention.attention`` runs as three groups of device launches:
  1. fused Q+K k-means (clustering_cuda.kmeans_fit): labels, centres, sizes and the
     stable cluster permutation of both tensors. With Base-Offset on, a token-parallel
     launch after the last update writes Q and K fake-quantized against their final
     centres, row for row in original order (text rows copied);
  2. one selection launch (clustering_cuda.select_work): cluster-pair selection with the
     text partition appended, each query cluster's kept key segments and the attention's
     cost-ordered work items;
  3. the MFMA sparse attention, which reads Q, K (or their fake-quantized copies) and V
     through the sort permutations and writes every video row straight back to its original
     sequence position.
No cluster-order Q/K/V copies and no concatenations are made.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import torch
import torch.nn.functional as F
from torch.nn.attention import SDPBackend, sdpa_kernel

from . import clustering_cuda
from .attention_cuda import base_offset_attention, sparse_attention, sparse_attention_work
from .quantization import _validate_bits


@dataclass(frozen=True)
class PecoConfig:
    num_q_centroids: int = 100
    num_k_centroids: int = 500
    top_p: float = 0.9
    min_kc_ratio: float = 0.1
    kmeans_iter_init: int = 50
    kmeans_iter_step: int = 2
    warmup_steps: int = 2
    warmup_layers: int = 0
    zero_step_kmeans_init: bool = True
    base_offset_bits: int = 4

    def __post_init__(self):
        if min(self.num_q_centroids, self.num_k_centroids, self.kmeans_iter_init, self.kmeans_iter_step) < 1:
            raise ValueError("Cluster counts and KMeans iteration counts must be positive")
        if not 0 < self.top_p <= 1 or not 0 <= self.min_kc_ratio <= 1:
            raise ValueError("top_p must be in (0, 1], min_kc_ratio in [0, 1]")
        if self.base_offset_bits not in (0, 4, 8):
            raise ValueError("base_offset_bits must be 0, 4 or 8")
        if self.warmup_steps < 0 or self.warmup_layers < 0:
            raise ValueError("Warmup counts must be nonnegative")


@dataclass
class InferenceContext:
    """Shared by processors in one pipeline; filled once per transformer call."""

    step: int = -1
    text_length: int = 0
    valid_text_length: int = 0


def dense_attention(query, key, value, valid_length):
    """Dense SDPA over [0, valid_length) and the padding segment separately (peco/processor.py:52-65)."""
    output = torch.empty_like(query)
    backend = [SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION, SDPBackend.MATH] if query.is_cuda \
        else [SDPBackend.MATH]
    with sdpa_kernel(backend):
        for start, end in ((0, valid_length), (valid_length, query.shape[2])):
            if start < end:
                output[:, :, start:end] = F.scaled_dot_product_attention(
                    query[:, :, start:end].contiguous(),
                    key[:, :, start:end].contiguous(),
                    value[:, :, start:end].contiguous(),
                    dropout_p=0.0,
                )
    return output


def extend_text_partition(dynamic_map, q_sizes, k_sizes, valid_text, text_length):
    """Append valid-text and padding groups to the video-cluster partition.

    Valid text and video tokens attend to each other; padding forms a separate sequence
    excluded from every video/text interaction (peco/processor.py:68-84).
    """
    dynamic_map = F.pad(dynamic_map, (0, 2, 0, 2), value=False)
    dynamic_map[..., -2, :-1] = True
    dynamic_map[..., :-1, -2] = True
    dynamic_map[..., -1, -1] = True
    extra = torch.tensor([valid_text, text_length - valid_text], device=q_sizes.device, dtype=torch.int32)
    extra = extra.expand(*q_sizes.shape[:-1], 2)
    return (
        dynamic_map.contiguous(),
        torch.cat((q_sizes, extra), -1).to(torch.int32).contiguous(),
        torch.cat((k_sizes, extra), -1).to(torch.int32).contiguous(),
    )


def _rotary_function():
    """diffusers' apply_rotary_emb when diffusers is installed, else the restatement below."""
    try:
        from diffusers.models.embeddings import apply_rotary_emb
    except ImportError:
        return _apply_rotary_emb
    return apply_rotary_emb


def _apply_rotary_emb(x, freqs_cis):
    """Rotary embedding with (cos, sin) tables [S, D] over interleaved channel pairs.

    Used when diffusers is not installed; it restates diffusers' published
    ``apply_rotary_emb(x, freqs_cis, use_real=True, use_real_unbind_dim=-1)``.
    """
    cos, sin = freqs_cis
    cos, sin = cos[None, None].to(x.device), sin[None, None].to(x.device)
    real, imag = x.reshape(*x.shape[:-1], -1, 2).unbind(-1)
    rotated = torch.stack([-imag, real], dim=-1).flatten(3)
    return (x.float() * cos + rotated.float() * sin).to(x.dtype)


class _FitResult:
    """One call's fit: labels, sizes [B,H,K] and stable permutations of Q and K, and the
    keys the last update fake-quantized (None when not asked for)."""

    __slots__ = ("q_labels", "k_labels", "q_sizes", "k_sizes", "q_idx", "k_idx", "pack", "q_hat")

    def __init__(self, q_labels, k_labels, q_sizes, k_sizes, q_idx, k_idx, pack, q_hat=None):
        self.q_labels, self.k_labels, self.q_sizes, self.k_sizes = q_labels, k_labels, q_sizes, k_sizes
        self.q_idx, self.k_idx, self.pack, self.q_hat = q_idx, k_idx, pack, q_hat


class PecoAttention:
    def __init__(self, layer_idx, config: PecoConfig, context: InferenceContext):
        self.layer_idx = layer_idx
        self.config = config
        self.context = context
        self.q_centroids = None
        self.k_centroids = None
        # Opt-in extension, not part of the reference's configuration: with Base-Offset on,
        # score video rows against video keys from the codes on the integer MFMA
        # (attention_cuda.base_offset_attention) instead of the fake-quantized rows.
        self.integer_scores = False
        # Diagnostics: when True, the last call's permutations (q_idx, k_idx) stay in
        # _last_fit and its fake-quantized keys in _last_pack. Off by default, so a layer
        # holds nothing between calls but its centroids (as the reference's does).
        self.record_intermediates = False
        self._last_fit = None
        self._last_pack = None

    def reset(self):
        self.q_centroids = self.k_centroids = None
        self._last_fit = None
        self._last_pack = None

    def _update_cluster_state(self, query, key):
        """Fit Q/K partitions, reusing this layer's centres after initialization
        (peco/processor.py:97-113).

        query/key are the video parts [B,H,N,D]; returns (q_labels, k_labels, q_sizes, k_sizes)
        with sizes [B,H,K]. Both fits run in one library call (four chains of launches).
        """
        fit = self._fit_clusters(query, key)
        return fit.q_labels, fit.k_labels, fit.q_sizes, fit.k_sizes

    def _fit_clusters(self, query, key, pack_keys=None, pack_order="cluster", query_full=None):
        """``_update_cluster_state`` returning a _FitResult. With ``pack_keys = (bits, key_full,
        value_full)`` ([B,H,S,D], key the tensor whose video part is ``key``; value_full None
        for ``pack_order="original"``) the fit also writes K Base-Offset fake-quantized
        against its final centres, with the text rows after the video rows: in the final key
        cluster order together with V, or each row at its own position
        (``pack_order="original"``, no V). A fourth entry ``True`` adds the keys' codes, lows
        and scales in the same order. The result's ``pack`` holds these tensors. With
        ``pack_order="original"``, ``query_full`` ([B,H,S,D], the tensor whose video part is
        ``query``) makes the fit write Q fake-quantized the same way (``q_hat``).
        """
        batch, heads, length, dim = query.shape
        initializing = self.q_centroids is None
        iterations = self.config.kmeans_iter_init if initializing else self.config.kmeans_iter_step
        q_flat = query.reshape(batch * heads, length, dim)
        k_flat = key.reshape(batch * heads, length, dim)
        if not query.is_cuda:
            raise ValueError("peco_amd attention runs on GPU tensors; CPU tensors are not supported")
        if q_flat.stride(2) != 1 or q_flat.stride(1) != dim:
            q_flat = q_flat.contiguous()
        if k_flat.stride(2) != 1 or k_flat.stride(1) != dim:
            k_flat = k_flat.contiguous()
        q_init = self._initial_centers(q_flat, self.q_centroids, self.config.num_q_centroids)
        k_init = self._initial_centers(k_flat, self.k_centroids, self.config.num_k_centroids)
        if q_flat.dtype not in (torch.float16, torch.bfloat16, torch.float32) or q_flat.dtype != k_flat.dtype:
            q_flat, k_flat = q_flat.float(), k_flat.float()
        pack = q_hat = None
        if pack_keys is None:
            problems = [clustering_cuda.KMeansProblem(q_flat, q_init), clustering_cuda.KMeansProblem(k_flat, k_init)]
            outs = clustering_cuda.kmeans_fit(problems, iterations)
        else:
            # The key rows are fitted in place in the full [B*H, S, D] tensor, whose rows past
            # the video part (the text) the packing copies.
            bits, key_full, value_full = pack_keys[:3]
            with_codes = len(pack_keys) > 3 and pack_keys[3]
            full = key_full.shape[2]
            if key_full.dtype != k_flat.dtype or not key_full.is_contiguous() or \
                    (value_full is not None and not value_full.is_contiguous()):
                raise ValueError("the packed key and value must be contiguous [B,H,S,D] tensors like key")
            k_rows = key_full.reshape(batch * heads, full, dim)[:, :length]
            value_flat = None if value_full is None else value_full.reshape(batch * heads, full, dim)
            q_pack = None
            if query_full is not None:
                if pack_order != "original" or query_full.shape != key_full.shape or \
                        query_full.dtype != k_flat.dtype or not query_full.is_contiguous():
                    raise ValueError("the packed query must be a contiguous [B,H,S,D] tensor like key, packed in "
                                     "original order")
                q_flat = query_full.reshape(batch * heads, full, dim)[:, :length]
                q_pack = (bits, full, None)
            problems = [clustering_cuda.KMeansProblem(q_flat, q_init), clustering_cuda.KMeansProblem(k_rows, k_init)]
            outs, packed = clustering_cuda.kmeans_fit(problems, iterations,
                                                      pack=[q_pack, (bits, full, value_flat, with_codes)],
                                                      pack_order=pack_order)
            k_hat, v_perm = packed[1][:2]
            pack = (k_hat.view(batch, heads, full, dim),
                    None if v_perm is None else v_perm.view(batch, heads, full, dim), *packed[1][2:])
            if q_pack is not None:
                q_hat = packed[0][0].view(batch, heads, full, dim)
        (q_labels, q_cent, q_sizes, q_idx, _), (k_labels, k_cent, k_sizes, k_idx, _) = outs
        self.q_centroids, self.k_centroids = q_cent, k_cent
        if self.record_intermediates:
            self._last_fit, self._last_pack = (q_idx, k_idx), pack
        return _FitResult(q_labels, k_labels, q_sizes.reshape(batch, heads, -1), k_sizes.reshape(batch, heads, -1),
                          q_idx, k_idx, pack, q_hat)

    @staticmethod
    def _initial_centers(x, cached, clusters):
        if cached is not None:
            # A cache from a call with other heads, dims or device must not reach the kernels,
            # which size every centre buffer from x (peco/clustering.py:51-52).
            if tuple(cached.shape) != (x.shape[0], clusters, x.shape[2]) or cached.device != x.device:
                raise ValueError("init_centroids must match [batch_heads, n_clusters, dims] and x.device")
            return cached
        tokens = x.shape[1]
        if not 1 <= clusters <= tokens:
            raise ValueError("n_clusters must be an integer in [1, tokens]")
        # Seeded-random tokens with replacement, as peco/clustering.py:48-49.
        indices = torch.randint(tokens, (x.shape[0], clusters), device=x.device)
        return x.float().gather(1, indices[..., None].expand(-1, -1, x.shape[2])).contiguous()

    def attention(self, query, key, value):
        batch, heads, length, dim = query.shape
        if batch != 1:
            raise ValueError("This minimal HunyuanVideo entry supports one prompt per call")
        text_length = self.context.text_length
        video_length = length - text_length
        valid_text = self.context.valid_text_length
        if video_length <= 0 or not 0 <= valid_text <= text_length:
            raise ValueError("Invalid video/text lengths in transformer context")
        warmup = self.context.step < self.config.warmup_steps or self.layer_idx < self.config.warmup_layers
        if warmup:
            if self.config.zero_step_kmeans_init and self.layer_idx >= self.config.warmup_layers:
                self._update_cluster_state(query[:, :, :video_length], key[:, :, :video_length])
            return dense_attention(query, key, value, video_length + valid_text)

        bits = self.config.base_offset_bits
        _validate_bits(bits, allow_bypass=True)
        query, key, value = query.contiguous(), key.contiguous(), value.contiguous()
        integer = bool(bits) and self.integer_scores
        if integer:
            # Extension: video x video scores from the Base-Offset codes (see __init__). The
            # last update writes K fake-quantized, V and K's codes in key-cluster order.
            fit = self._fit_clusters(query[:, :, :video_length], key[:, :, :video_length],
                                     pack_keys=(bits, key, value, True))
            dynamic_map, ext_q, ext_k = clustering_cuda.select_connections(
                self.q_centroids.reshape(batch, heads, -1, dim), self.k_centroids.reshape(batch, heads, -1, dim),
                fit.q_sizes, fit.k_sizes, self.config.top_p,
                math.ceil(self.config.min_kc_ratio * self.config.num_k_centroids), (valid_text, text_length))
            k_perm, v_perm, k_codes, k_low, k_scale = fit.pack
            return base_offset_attention(query, k_perm, v_perm, dynamic_map, ext_q, ext_k, out_index=fit.q_idx,
                                         q_centroids=self.q_centroids, k_centroids=self.k_centroids,
                                         k_codes=k_codes, k_low=k_low, k_scale=k_scale, bits=bits)
        # With Base-Offset on, the fit ends with a launch that writes Q and K fake-quantized
        # against their final centres, each row at its own position (stage 2 in the fit).
        fit = self._fit_clusters(query[:, :, :video_length], key[:, :, :video_length],
                                 pack_keys=(bits, key, None) if bits else None, pack_order="original",
                                 query_full=query if bits else None)
        # Cluster connectivity from the floating-point centres, extended with the text
        # partition (select_cluster_connections + extend_text_partition), in one launch that
        # also writes each query cluster's kept key segments and the attention's work items.
        work = clustering_cuda.select_work(
            self.q_centroids.reshape(batch, heads, -1, dim), self.k_centroids.reshape(batch, heads, -1, dim),
            fit.q_sizes, fit.k_sizes, self.config.top_p,
            math.ceil(self.config.min_kc_ratio * self.config.num_k_centroids), (valid_text, text_length),
            length, length)
        # The attention reads Q/K/V through the sort permutations (stage 3 fused into its
        # loads) and writes the output in original order, so no cluster-order copy is made.
        # With Base-Offset on, Q and K come fake-quantized from the fit.
        q_in, k_in = (query, key) if bits == 0 else (fit.q_hat, fit.pack[0])
        return sparse_attention_work(q_in, k_in, value, work, out_index=fit.q_idx, out_index_rows=video_length,
                                     k_index=fit.k_idx)

    @torch.no_grad()
    def __call__(self, attn, hidden_states, encoder_hidden_states=None, attention_mask=None, image_rotary_emb=None):
        """diffusers attention-processor entry (peco/processor.py:159-197).

        ``attention_mask`` is ignored: which text rows are valid comes from the shared
        InferenceContext. The sequence is [video rows, text rows]. Each projection of each
        part is written once, head-major, into its slot of one [3, B, H, S, D] buffer (the
        copy that splits the heads also places the rows), so no concatenation copies are
        made. Video rows get the rotary embedding; text rows never do. Double-stream blocks
        (``add_q_proj`` set) project the text with their added projections and norms,
        single-stream blocks with the same ones as the video.
        """
        rotary = _rotary_function()
        text = 0 if encoder_hidden_states is None else encoder_hidden_states.shape[1]
        parts = [(hidden_states, (attn.to_q, attn.to_k, attn.to_v), (attn.norm_q, attn.norm_k),
                  image_rotary_emb)]
        if text:
            if attn.add_q_proj is not None:
                parts.append((encoder_hidden_states, (attn.add_q_proj, attn.add_k_proj, attn.add_v_proj),
                              (attn.norm_added_q, attn.norm_added_k), None))
            else:
                parts.append((encoder_hidden_states, (attn.to_q, attn.to_k, attn.to_v), (attn.norm_q, attn.norm_k),
                              None))
        length = hidden_states.shape[1] + text
        qkv = None
        first = 0
        for source, projections, norms, freqs in parts:
            rows = source.shape[1]
            for slot, proj in enumerate(projections):
                part = proj(source).unflatten(2, (attn.heads, -1)).transpose(1, 2)  # [B, H, rows, D] view
                if slot < 2:
                    if norms[slot] is not None:
                        part = norms[slot](part)
                    if freqs is not None:
                        part = rotary(part, freqs)
                if qkv is None:
                    batch, heads, _, dim = part.shape
                    qkv = torch.empty((3, batch, heads, length, dim), dtype=part.dtype, device=part.device)
                qkv[slot, :, :, first:first + rows] = part
            first += rows
        output = self.attention(qkv[0], qkv[1], qkv[2]).transpose(1, 2)  # [B, S, H, D] view
        video = hidden_states.shape[1]
        if not text:
            return output.flatten(2, 3), encoder_hidden_states
        video_out = output[:, :video].flatten(2, 3)
        text_out = output[:, video:].flatten(2, 3)
        if getattr(attn, "to_out", None) is not None:
            video_out = attn.to_out[1](attn.to_out[0](video_out))
        if getattr(attn, "to_add_out", None) is not None:
            text_out = attn.to_add_out(text_out)
        return video_out, text_out
