"""PecoAttention.__call__, the diffusers processor entry (peco/processor.py:159-197), and the
dense warm-up branch (processor.py:52-65,124-128).

CPU tests pin the oracle's restatement of the prologue/epilogue against closed forms and
check __call__'s assembly against it with the attention itself stubbed out. GPU tests run
__call__ end to end through the HIP path for both block types (single-stream: text projected
with the video's weights and left unrotated; double-stream: text through the added
projections and norms) and run the warm-up branch on the GPU.

The rotary embedding follows diffusers' published apply_rotary_emb (use_real=True,
use_real_unbind_dim=-1); diffusers is not installed here, so its own outputs are not
available. It is pinned to the closed form it implements: each channel pair (2i, 2i+1) is a
complex number multiplied by cos + i sin.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import canonical, reference_path
from peco_amd import processor

DEV = "cuda:0"


class _Attn(torch.nn.Module):
    """Stands in for a diffusers Attention module of HunyuanVideo."""

    def __init__(self, heads, head_dim, dual, seed=0, norms=True):
        super().__init__()
        torch.manual_seed(seed)
        dim = heads * head_dim
        self.heads = heads
        lin = lambda: torch.nn.Linear(dim, dim)  # noqa: E731
        norm = (lambda: torch.nn.RMSNorm(head_dim, eps=1e-6)) if norms else (lambda: None)  # noqa: E731
        self.to_q, self.to_k, self.to_v = lin(), lin(), lin()
        self.norm_q, self.norm_k = norm(), norm()
        if dual:
            self.add_q_proj, self.add_k_proj, self.add_v_proj = lin(), lin(), lin()
            self.norm_added_q, self.norm_added_k = norm(), norm()
            self.to_add_out = lin()
        else:
            self.add_q_proj = None
        self.to_out = torch.nn.ModuleList([lin(), torch.nn.Dropout(0.0)])
        if norms:
            for m in self.modules():
                if isinstance(m, torch.nn.RMSNorm):
                    torch.nn.init.uniform_(m.weight, 0.5, 1.5)


def _rotary_tables(length, dim, seed=0):
    g = torch.Generator().manual_seed(seed)
    theta = torch.rand(length, dim // 2, generator=g) * 6.3
    # HunyuanVideo's tables repeat each angle for the two channels of a pair.
    return theta.cos().repeat_interleave(2, -1), theta.sin().repeat_interleave(2, -1)


# ------------------------------------------------------------------------------- CPU

def test_rotary_embedding_is_complex_rotation():
    x = torch.randn(1, 2, 10, 8, dtype=torch.float64)
    cos, sin = _rotary_tables(10, 8)
    cos, sin = cos.double(), sin.double()
    z = torch.view_as_complex(x.reshape(1, 2, 10, 4, 2).contiguous())
    w = torch.complex(cos[:, ::2], sin[:, ::2])
    expect = torch.view_as_real(z * w).reshape(1, 2, 10, 8)
    for fn in (reference_path.rotary_embedding, processor._apply_rotary_emb):
        got = fn(x.float(), (cos.float(), sin.float()))
        assert torch.allclose(got.double(), expect, atol=1e-5)
    # Identity and quarter turn.
    one, zero = torch.ones(10, 8), torch.zeros(10, 8)
    xf = x.float()
    assert torch.equal(reference_path.rotary_embedding(xf, (one, zero)), xf)
    quarter = reference_path.rotary_embedding(xf, (zero, one))
    assert torch.equal(quarter[..., 0::2], -xf[..., 1::2]) and torch.equal(quarter[..., 1::2], xf[..., 0::2])


def _identity_attn(dual):
    attn = _Attn(2, 8, dual, norms=False)
    for m in attn.modules():
        if isinstance(m, torch.nn.Linear):
            torch.nn.init.eye_(m.weight)
            torch.nn.init.zeros_(m.bias)
    return attn


@pytest.mark.parametrize("dual", [False, True])
def test_oracle_prologue_closed_form(dual):
    """Identity projections, no norms, quarter-turn rotary: q/k are the input rows split into
    heads, the video rows rotated and the text rows not."""
    attn = _identity_attn(dual)
    h, e = torch.randn(1, 12, 16), torch.randn(1, 5, 16)
    zero, one = torch.zeros(12, 8), torch.ones(12, 8)
    q, k, v = reference_path.processor_prologue(attn, h, e, (zero, one), reference_path.rotary_embedding)
    rows = torch.cat((h, e), 1).unflatten(2, (2, 8)).transpose(1, 2)
    assert torch.equal(v, rows)
    for t in (q, k):
        assert torch.equal(t[:, :, 12:], rows[:, :, 12:])
        assert torch.equal(t[:, :, :12, 0::2], -rows[:, :, :12, 1::2])
        assert torch.equal(t[:, :, :12, 1::2], rows[:, :, :12, 0::2])
    out, enc = reference_path.processor_epilogue(attn, rows, e)
    assert torch.equal(out, h) and (torch.equal(enc, e) if dual else torch.equal(enc, rows.transpose(1, 2)
                                                                                     .flatten(2)[:, 12:]))


def _stubbed_call(attn, hidden, enc, freqs, video, text):
    """Runs __call__ with the attention replaced by a fixed function of its inputs."""
    ctx = processor.InferenceContext(step=5, text_length=text, valid_text_length=text)
    layer = processor.PecoAttention(0, processor.PecoConfig(warmup_steps=0), ctx)
    seen = {}

    def attention(q, k, v):
        seen.update(q=q.clone(), k=k.clone(), v=v.clone())
        return q * 0.5 + k * 0.25 - v
    layer.attention = attention
    out = layer(attn, hidden, enc, image_rotary_emb=freqs)
    return out, seen


@pytest.mark.parametrize("dual", [False, True])
@pytest.mark.parametrize("with_text", [True, False])
def test_call_assembly_matches_oracle_on_cpu(dual, with_text):
    heads, hd, video, text = 2, 16, 20, 6
    attn = _Attn(heads, hd, dual, seed=3)
    hidden = torch.randn(1, video, heads * hd)
    enc = torch.randn(1, text, heads * hd) if with_text else None
    freqs = _rotary_tables(video, hd)
    with torch.no_grad():
        (out, enc_out), seen = _stubbed_call(attn, hidden, enc, freqs, video, text if with_text else 0)
        q, k, v = reference_path.processor_prologue(attn, hidden, enc, freqs, reference_path.rotary_embedding)
        ref_out, ref_enc = reference_path.processor_epilogue(attn, q * 0.5 + k * 0.25 - v, enc)
    tol = dict(atol=1e-5, rtol=1e-5)
    for name, ref in (("q", q), ("k", k), ("v", v)):
        assert seen[name].shape == ref.shape and torch.allclose(seen[name], ref, **tol), name
    assert torch.allclose(out, ref_out, **tol)
    if with_text:
        assert torch.allclose(enc_out, ref_enc, **tol)
    else:
        assert enc_out is None


# ------------------------------------------------------------------------------- GPU

def _bf16_ulps(a, b):
    """max |a - b| in units of b's bf16 spacing."""
    a, b = a.float(), b.float()
    spacing = torch.ldexp(torch.ones_like(b), torch.frexp(b.abs().clamp_min(1e-30))[1] - 8)
    return ((a - b).abs() / spacing).max().item()


@pytest.mark.gpu
@pytest.mark.parametrize("dual", [False, True])
def test_call_sparse_path_on_gpu(announce, dual):
    heads, hd, video, text, valid = 2, 128, 2048, 64, 50
    announce(f"dual={dual} heads={heads} video={video} text={text} valid={valid}")
    attn = _Attn(heads, hd, dual, seed=7).to(DEV, torch.bfloat16)
    g = torch.Generator().manual_seed(11)
    hidden = torch.randn(1, video, heads * hd, generator=g).to(DEV, torch.bfloat16)
    enc = torch.randn(1, text, heads * hd, generator=g).to(DEV, torch.bfloat16)
    cos, sin = _rotary_tables(video, hd, seed=5)
    freqs = (cos.to(DEV), sin.to(DEV))
    cfg = processor.PecoConfig(num_q_centroids=16, num_k_centroids=32, top_p=0.9, min_kc_ratio=0.25,
                               kmeans_iter_init=4, kmeans_iter_step=2, warmup_steps=0, base_offset_bits=4)
    ctx = processor.InferenceContext(step=0, text_length=text, valid_text_length=valid)
    layer = processor.PecoAttention(0, cfg, ctx)
    qv = hidden.float()[0].reshape(video, heads, hd).transpose(0, 1)  # a deterministic initial state
    layer.q_centroids = qv[:, ::video // 16][:, :16].contiguous()
    layer.k_centroids = qv[:, ::video // 32][:, :32].contiguous()
    init = (layer.q_centroids.cpu(), layer.k_centroids.cpu())
    seen = {}
    sparse = layer.attention

    def attention(q, k, v):
        seen.update(q=q.clone(), k=k.clone(), v=v.clone())
        seen["o"] = sparse(q, k, v)
        return seen["o"]
    layer.attention = attention
    with torch.no_grad():
        out, enc_out = layer(attn, hidden, enc, image_rotary_emb=freqs)
        q, k, v = reference_path.processor_prologue(attn, hidden, enc, freqs, processor._rotary_function())
        ref_out, ref_enc = reference_path.processor_epilogue(attn, seen["o"], enc)
    torch.cuda.synchronize()
    # Prologue: double-stream blocks run the reference's own projections (exact); single-stream
    # blocks project video and text in separate GEMMs, which may round differently.
    for name, ref in (("q", q), ("k", k), ("v", v)):
        ulps = _bf16_ulps(seen[name], ref)
        print(f"[call] dual={dual} {name}: {ulps:.1f} bf16 ulps", flush=True)
        assert ulps <= (0 if dual else 2), name
    # Attention on those inputs against the oracle's layer.
    oracle_out = reference_path.peco_layer(
        seen["q"].cpu(), seen["k"].cpu(), seen["v"].cpu(), num_q_centroids=16, num_k_centroids=32, iterations=2,
        q_init=init[0], k_init=init[1], top_p=0.9, min_kc_ratio=0.25, bits=4, text_length=text, valid_text=valid,
        fit=lambda x, c, it, i0: _canonical_fit(x, it, i0),
        attention=lambda *a: _canonical_attention(*a))
    err = (seen["o"].float().cpu() - oracle_out.float()).abs()
    print(f"[call] dual={dual} attention: max {err.max():.3e} mean {err.mean():.3e}", flush=True)
    assert err.max().item() <= 2e-2 and err.mean().item() <= 2e-3
    # Epilogue: the output projections of the reference on the same attention output.
    assert _bf16_ulps(out, ref_out) <= 1 and _bf16_ulps(enc_out, ref_enc) <= 1


def _canonical_fit(x, iterations, init):
    labels, centers, counts, _, _ = canonical.kmeans_fit(x.float().numpy(), init.numpy(), iterations)
    return torch.from_numpy(labels), torch.from_numpy(centers), torch.from_numpy(counts), iterations


def _canonical_attention(q, k, v, m, qs, ks):
    o = canonical.sparse_attention(q[0].float().numpy(), k[0].float().numpy(), v[0].float().numpy(), m[0].numpy(),
                                   qs[0].numpy(), ks[0].numpy())
    return torch.from_numpy(o)[None].to(q.dtype)


@pytest.mark.gpu
@pytest.mark.parametrize("valid", [64, 40])
def test_dense_warmup_branch_on_gpu(announce, valid):
    """Warm-up steps run dense SDPA in two segments on the GPU, and (zero_step_kmeans_init)
    fit the layer's clusters on the way, bit-exact against the oracle."""
    heads, hd, video, text = 2, 128, 2048, 64
    announce(f"warm-up: heads={heads} video={video} text={text} valid={valid}")
    g = torch.Generator().manual_seed(21)
    q, k, v = (torch.randn(1, heads, video + text, hd, generator=g).bfloat16() for _ in range(3))
    cfg = processor.PecoConfig(num_q_centroids=16, num_k_centroids=32, kmeans_iter_init=3, warmup_steps=2)
    ctx = processor.InferenceContext(step=1, text_length=text, valid_text_length=valid)
    layer = processor.PecoAttention(0, cfg, ctx)
    qi = q[0, :, :video:128].float()[:, :16].contiguous()
    ki = k[0, :, :video:64].float()[:, :32].contiguous()
    layer.q_centroids, layer.k_centroids = qi.to(DEV), ki.to(DEV)
    with torch.no_grad():
        out = layer.attention(q.to(DEV), k.to(DEV), v.to(DEV))
    torch.cuda.synchronize()
    ref = torch.empty(q.shape)
    for a, b in ((0, video + valid), (video + valid, video + text)):
        ref[:, :, a:b] = F.scaled_dot_product_attention(q[:, :, a:b].float(), k[:, :, a:b].float(),
                                                        v[:, :, a:b].float())
    err = (out.float().cpu() - ref).abs()
    print(f"[warm-up] valid={valid}: max {err.max():.3e} mean {err.mean():.3e}", flush=True)
    assert out.dtype == torch.bfloat16
    assert err.max().item() <= 2e-2 and err.mean().item() <= 2e-3
    # The warm-up fit started from the cached centroids with kmeans_iter_step iterations.
    _, qc, _, _, _ = canonical.kmeans_fit(q[0, :, :video].float().numpy(), qi.numpy(), cfg.kmeans_iter_step)
    _, kc, _, _, _ = canonical.kmeans_fit(k[0, :, :video].float().numpy(), ki.numpy(), cfg.kmeans_iter_step)
    assert np.array_equal(layer.q_centroids.cpu().numpy().view(np.int32), qc.view(np.int32))
    assert np.array_equal(layer.k_centroids.cpu().numpy().view(np.int32), kc.view(np.int32))
