"""HunyuanVideo attention processor with PECO cluster-sparse attention (peco/processor.py interface).

The sparse path of ``PecoAttention.attention`` runs as four groups of device launches:
  1. fused Q+K k-means (clustering_cuda.kmeans_fit): labels, centres, sizes and the
     stable cluster permutation of both tensors;
  2. one selection launch: cluster-pair map with the text partition appended
     (select_cluster_connections + extend_text_partition);
  3. one pack launch that fake-quantizes Q/K (Base-Offset, when enabled), gathers Q/K/V
     into cluster order and appends the text rows (no slice copies, no concatenations);
  4. the HIP work-list builder and MFMA sparse attention, whose epilogue writes every
     video row straight back to its original sequence position.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import torch
import torch.nn.functional as F
from torch.nn.attention import SDPBackend, sdpa_kernel

from . import clustering_cuda
from .attention_cuda import sparse_attention, sparse_attention_indexed
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


def _extend_partition_on_device(dynamic_map, q_sizes, k_sizes, valid_text, text_length):
    """extend_text_partition without the host-to-device copy of the two extra sizes."""
    dynamic_map = F.pad(dynamic_map, (0, 2, 0, 2), value=False)
    dynamic_map[..., -2, :-1] = True
    dynamic_map[..., :-1, -2] = True
    dynamic_map[..., -1, -1] = True
    lead = q_sizes.shape[:-1]
    extra = torch.empty((*lead, 2), dtype=torch.int32, device=q_sizes.device)
    extra[..., 0] = valid_text
    extra[..., 1] = text_length - valid_text
    return (dynamic_map.contiguous(), torch.cat((q_sizes.to(torch.int32), extra), -1).contiguous(),
            torch.cat((k_sizes.to(torch.int32), extra), -1).contiguous())


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


class PecoAttention:
    def __init__(self, layer_idx, config: PecoConfig, context: InferenceContext):
        self.layer_idx = layer_idx
        self.config = config
        self.context = context
        self.q_centroids = None
        self.k_centroids = None
        self._last_fit = None

    def reset(self):
        self.q_centroids = self.k_centroids = None
        self._last_fit = None

    def _update_cluster_state(self, query, key):
        """Fit Q/K partitions, reusing this layer's centres after initialization.

        query/key are the video parts [B,H,N,D]; returns (q_labels, k_labels, q_sizes, k_sizes)
        with sizes [B,H,K]. Both fits run in the same launches.
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
        (q_labels, q_cent, q_sizes, q_idx, _), (k_labels, k_cent, k_sizes, k_idx, _) = clustering_cuda.kmeans_fit(
            [clustering_cuda.KMeansProblem(q_flat, q_init), clustering_cuda.KMeansProblem(k_flat, k_init)],
            iterations)
        self.q_centroids, self.k_centroids = q_cent, k_cent
        self._last_fit = (q_idx, k_idx)
        return q_labels, k_labels, q_sizes.reshape(batch, heads, -1), k_sizes.reshape(batch, heads, -1)

    @staticmethod
    def _initial_centers(x, cached, clusters):
        if cached is not None:
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
        q_labels, k_labels, q_sizes, k_sizes = self._update_cluster_state(
            query[:, :, :video_length], key[:, :, :video_length])
        q_idx, k_idx = self._last_fit
        # Cluster connectivity from the floating-point centres, extended with the text
        # partition (select_cluster_connections + extend_text_partition in one launch).
        dynamic_map, q_sizes, k_sizes, kept = clustering_cuda.select_connections(
            self.q_centroids.reshape(batch, heads, -1, dim), self.k_centroids.reshape(batch, heads, -1, dim),
            q_sizes, k_sizes, self.config.top_p,
            math.ceil(self.config.min_kc_ratio * self.config.num_k_centroids), text=(valid_text, text_length),
            with_kept=True)
        if bits == 0:
            # No fake quantization: attention reads Q/K/V through the sort permutations and
            # writes the output in original order, so no packed copy is made.
            return sparse_attention_indexed(query, key, value, dynamic_map, q_sizes, k_sizes, q_idx, k_idx,
                                            video_length, validate_sizes=False, kept_keys=kept)
        # Fake-quantize Q/K against their centroids while packing Q/K/V into cluster order.
        q_perm, k_perm, v_perm = clustering_cuda.pack_clustered(
            [query, key, value], [q_idx, k_idx, k_idx], [q_labels, k_labels, None],
            [self.q_centroids, self.k_centroids, None], [bits, bits, 0], video_length)
        # Video rows return to their original positions; text rows keep theirs.
        return sparse_attention(q_perm, k_perm, v_perm, dynamic_map, q_sizes, k_sizes, validate_sizes=False,
                                out_index=q_idx, out_index_rows=video_length, kept_keys=kept)

    @torch.no_grad()
    def __call__(self, attn, hidden_states, encoder_hidden_states=None, attention_mask=None, image_rotary_emb=None):
        """diffusers attention-processor entry (peco/processor.py:159-197)."""
        try:
            from diffusers.models.embeddings import apply_rotary_emb
        except ImportError:
            apply_rotary_emb = _apply_rotary_emb

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
                query = torch.cat((apply_rotary_emb(query[:, :, :-text_length], image_rotary_emb),
                                   query[:, :, -text_length:]), 2)
                key = torch.cat((apply_rotary_emb(key[:, :, :-text_length], image_rotary_emb),
                                 key[:, :, -text_length:]), 2)
            else:
                query, key = (apply_rotary_emb(x, image_rotary_emb) for x in (query, key))
        if attn.add_q_proj is not None and text_length:
            eq, ek, ev = (split_heads(proj(encoder_hidden_states))
                          for proj in (attn.add_q_proj, attn.add_k_proj, attn.add_v_proj))
            if attn.norm_added_q is not None:
                eq = attn.norm_added_q(eq)
            if attn.norm_added_k is not None:
                ek = attn.norm_added_k(ek)
            query, key, value = torch.cat((query, eq), 2), torch.cat((key, ek), 2), torch.cat((value, ev), 2)
        output = self.attention(query.contiguous(), key.contiguous(), value.contiguous())
        output = output.transpose(1, 2).flatten(2, 3).to(query.dtype)
        if not text_length:
            return output, encoder_hidden_states
        output, encoder_output = output[:, :-text_length], output[:, -text_length:]
        if getattr(attn, "to_out", None) is not None:
            output = attn.to_out[1](attn.to_out[0](output))
        if getattr(attn, "to_add_out", None) is not None:
            encoder_output = attn.to_add_out(encoder_output)
        return output, encoder_output
