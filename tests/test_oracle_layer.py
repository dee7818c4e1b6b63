"""Pins of the oracle's end-to-end layer, reference_path.peco_layer (no GPU).

peco_layer restates the orchestration of peco/processor.py:129-157: slicing, k-means,
selection, fake quantization, cluster sort and gather, text concatenation, the text
partition (processor.py:68-84), the restore index assembly and the restore. Each test
below checks it against a closed form that shares none of that machinery:
  - keeping every cluster pair (top_p = 1, min_kc_ratio = 1) makes the layer dense
    attention over [video + valid text] plus a separate padding segment, i.e. the
    processor's own dense_attention (processor.py:52-65) computed by library SDPA;
  - the same with Base-Offset on, where Q/K video rows are the C oracle's quantizer output;
  - for any selection, every output row in ORIGINAL token order equals softmax attention
    under the mask built directly from the labels and the cluster map (no permutation,
    no sizes, no extended map).
A slip in any of the assembly steps (a dropped or duplicated text row, a wrong restore
index, V gathered with Q's permutation, the padding attending to valid tokens, the map
transposed) fails at least one of them.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import canonical, reference_path


def _inputs(seed, heads=2, video=300, text=16, dim=32):
    g = torch.Generator().manual_seed(seed)
    # Mixture-shaped Q/K so the clusters are meaningful; V plain normal.
    means = torch.randn(heads, 6, dim, generator=g) * 3
    pick = torch.randint(6, (heads, video + text), generator=g)
    q = means.gather(1, pick[..., None].expand(-1, -1, dim)) + torch.randn(heads, video + text, dim, generator=g)
    pick = torch.randint(6, (heads, video + text), generator=g)
    k = means.gather(1, pick[..., None].expand(-1, -1, dim)) + torch.randn(heads, video + text, dim, generator=g)
    v = torch.randn(heads, video + text, dim, generator=g)
    q, k, v = (t[None].contiguous() for t in (q, k, v))
    q_init = q[0, :, :video][:, torch.randint(video, (8,), generator=g)].contiguous()
    k_init = k[0, :, :video][:, torch.randint(video, (12,), generator=g)].contiguous()
    return q, k, v, q_init, k_init


def _layer(q, k, v, q_init, k_init, *, text, valid, top_p, ratio, bits, stages=None):
    return reference_path.peco_layer(q, k, v, num_q_centroids=q_init.shape[1], num_k_centroids=k_init.shape[1],
                                     iterations=3, q_init=q_init, k_init=k_init, top_p=top_p, min_kc_ratio=ratio,
                                     bits=bits, text_length=text, valid_text=valid, stages=stages)


def _two_segment_sdpa(q, k, v, valid_length):
    out = torch.empty_like(q)
    for a, b in ((0, valid_length), (valid_length, q.shape[2])):
        if a < b:
            out[:, :, a:b] = F.scaled_dot_product_attention(q[:, :, a:b], k[:, :, a:b], v[:, :, a:b])
    return out


@pytest.mark.parametrize("valid", [16, 11, 0])
def test_keep_all_pairs_is_dense_attention_with_padding_segment(valid):
    q, k, v, qi, ki = _inputs(1)
    video, text = 300, 16
    out = _layer(q, k, v, qi, ki, text=text, valid=valid, top_p=1.0, ratio=1.0, bits=0)
    ref = _two_segment_sdpa(q, k, v, video + valid)
    assert out.shape == q.shape and out.dtype == q.dtype
    assert torch.allclose(out, ref, atol=2e-5, rtol=1e-5), (out - ref).abs().max()


@pytest.mark.parametrize("bits", [4, 8])
def test_keep_all_pairs_with_base_offset_attends_to_quantized_video(bits):
    q, k, v, qi, ki = _inputs(2)
    video, text, valid = 300, 16, 13
    st = {}
    out = _layer(q, k, v, qi, ki, text=text, valid=valid, top_p=1.0, ratio=1.0, bits=bits, stages=st)
    # Quantized video rows from the C oracle's quantizer, given the layer's own partition.
    qh = canonical.base_offset(q[0, :, :video].numpy(), st["q_labels"].numpy(), st["q_centroids"].numpy(), bits)[3]
    kh = canonical.base_offset(k[0, :, :video].numpy(), st["k_labels"].numpy(), st["k_centroids"].numpy(), bits)[3]
    q2 = torch.cat((torch.from_numpy(qh)[None], q[:, :, video:]), 2)
    k2 = torch.cat((torch.from_numpy(kh)[None], k[:, :, video:]), 2)
    ref = _two_segment_sdpa(q2, k2, v, video + valid)
    assert torch.allclose(out, ref, atol=2e-5, rtol=1e-5), (out - ref).abs().max()
    # And it is not the unquantized result.
    plain = _two_segment_sdpa(q, k, v, video + valid)
    assert (out - plain).abs().max() > 1e-4


def _masked_attention_original_order(q, k, v, q_labels, k_labels, cmap, video, valid):
    """Attention in original order under mask[i, j] built from labels and the cluster map."""
    _, heads, length, dim = q.shape
    out = torch.zeros_like(q)
    for h in range(heads):
        mask = torch.zeros(length, length, dtype=torch.bool)
        ql, kl = q_labels[h].long(), k_labels[h].long()
        mask[:video, :video] = cmap[h][ql][:, kl]            # video query -> kept key clusters
        mask[:video + valid, video:video + valid] = True     # everyone but padding -> valid text
        mask[video:video + valid, :video] = True              # valid text -> all video
        mask[video + valid:, video + valid:] = True           # padding -> padding only
        s = (q[0, h] @ k[0, h].T) * dim ** -0.5
        s = s.masked_fill(~mask, float("-inf"))
        p = torch.softmax(s, -1)
        p = torch.nan_to_num(p, nan=0.0)                       # fully masked rows are zero
        out[0, h] = p @ v[0, h]
    return out


@pytest.mark.parametrize("top_p,ratio,valid", [(1e-9, 0.25, 16), (0.6, 0.0, 9), (0.9, 0.1, 0)])
def test_sparse_layer_equals_label_mask_attention_in_original_order(top_p, ratio, valid):
    q, k, v, qi, ki = _inputs(3)
    video, text = 300, 16
    st = {}
    out = _layer(q, k, v, qi, ki, text=text, valid=valid, top_p=top_p, ratio=ratio, bits=0, stages=st)
    cmap = st["dynamic_map"][0]
    assert not cmap.all(), "the selection should drop some pairs here"
    ref = _masked_attention_original_order(q, k, v, st["q_labels"], st["k_labels"], cmap, video, valid)
    assert torch.allclose(out, ref, atol=2e-5, rtol=1e-5), (out - ref).abs().max()


def test_label_mask_check_fails_on_a_planted_restore_slip():
    """The original-order check above detects a layer whose restore uses K's permutation."""
    q, k, v, qi, ki = _inputs(4)
    video, text, valid = 300, 16, 16
    st = {}
    _layer(q, k, v, qi, ki, text=text, valid=valid, top_p=1e-9, ratio=0.25, bits=0, stages=st)
    wrong = torch.cat((st["k_indices"].reshape(2, video), torch.arange(video, video + text, dtype=torch.int32)
                       .expand(2, -1)), -1)
    slipped = reference_path.restore_tokens(st["out_perm"], wrong)
    ref = _masked_attention_original_order(q, k, v, st["q_labels"], st["k_labels"], st["dynamic_map"][0], video,
                                           valid)
    assert not torch.allclose(slipped, ref, atol=1e-3)
