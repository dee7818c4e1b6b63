"""Host-side behaviour of the drop-in API (no GPU): validation, text partition, wiring."""
import pytest
import torch

from oracle import reference_path
from peco_amd import attention_cuda, clustering, model, processor, quantization


def test_peco_config_validation_matches_reference():
    processor.PecoConfig()
    with pytest.raises(ValueError, match="positive"):
        processor.PecoConfig(num_q_centroids=0)
    with pytest.raises(ValueError, match="top_p"):
        processor.PecoConfig(top_p=0)
    with pytest.raises(ValueError, match="top_p"):
        processor.PecoConfig(min_kc_ratio=1.5)
    with pytest.raises(ValueError, match="base_offset_bits"):
        processor.PecoConfig(base_offset_bits=2)
    with pytest.raises(ValueError, match="nonnegative"):
        processor.PecoConfig(warmup_steps=-1)


def test_fit_token_clusters_argument_errors():
    x = torch.randn(2, 10, 8)
    with pytest.raises(ValueError, match="floating tensor"):
        clustering.fit_token_clusters(x[0], 2)
    with pytest.raises(ValueError, match="n_clusters"):
        clustering.fit_token_clusters(x, 11)
    with pytest.raises(ValueError, match="max_iters"):
        clustering.fit_token_clusters(x, 2, max_iters=0)
    with pytest.raises(ValueError, match="tol"):
        clustering.fit_token_clusters(x, 2, tol=-1)
    with pytest.raises(ValueError, match="chunk_size"):
        clustering.fit_token_clusters(x, 2, chunk_size=0)
    with pytest.raises(ValueError, match="GPU"):
        clustering.fit_token_clusters(x, 2)


def test_permutation_argument_errors():
    t = torch.randn(1, 2, 5, 4)
    with pytest.raises(ValueError, match="dim=2"):
        clustering.gather_clustered_tokens(t, torch.zeros(2, 5), dim=1)
    with pytest.raises(ValueError, match="one cluster ID"):
        clustering.gather_clustered_tokens(t, torch.zeros(2, 4))
    with pytest.raises(ValueError, match="one index"):
        clustering.restore_sequence_order(t, torch.zeros(2, 4, dtype=torch.int32))


def test_quantization_argument_errors():
    x = torch.randn(2, 5, 64)
    lab = torch.zeros(2, 5, dtype=torch.int32)
    c = torch.randn(2, 3, 64)
    with pytest.raises(ValueError, match="bits"):
        quantization.quantize_base_offset(x, lab, c, bits=0)
    with pytest.raises(ValueError, match="bits"):
        quantization.fake_quantize_base_offset(x, lab, c, bits=3)
    assert quantization.fake_quantize_base_offset(x, lab, c, bits=0) is x
    with pytest.raises(TypeError, match="int32 or int64"):
        quantization.quantize_base_offset(x, lab.float(), c)
    with pytest.raises(ValueError, match="labels must have shape"):
        quantization.quantize_base_offset(x, lab[:, :4], c)
    with pytest.raises(ValueError, match="centroids must have shape"):
        quantization.quantize_base_offset(x, lab, c[:, :, :32])
    with pytest.raises(ValueError, match="GPU"):
        quantization.quantize_base_offset(x, lab, c)


def test_sparse_attention_argument_errors():
    q = torch.randn(1, 2, 8, 64, dtype=torch.bfloat16)
    qs = torch.tensor([[[8], [8]]], dtype=torch.int32)
    m = torch.ones(1, 2, 1, 1, dtype=torch.bool)
    with pytest.raises(TypeError, match="torch tensors"):
        attention_cuda.sparse_attention(q, q, q, m, qs, None)
    with pytest.raises(ValueError, match="head dimensions"):
        attention_cuda.sparse_attention(q[..., :32], q[..., :32], q[..., :32], m, qs, qs)
    with pytest.raises(TypeError, match="dtype"):
        attention_cuda.sparse_attention(q.float(), q.float(), q.float(), m, qs, qs)
    with pytest.raises(ValueError, match="GPU device"):
        attention_cuda.sparse_attention(q, q, q, m, qs, qs)


def test_extend_text_partition_matches_oracle_fixture():
    m = torch.tensor([[[[True, False], [False, True]]]])
    qs = torch.tensor([[[3, 4]]], dtype=torch.int32)
    ks = torch.tensor([[[5, 2]]], dtype=torch.int32)
    em, eq, ek = processor.extend_text_partition(m, qs, ks, 3, 5)
    rm, rq, rk = reference_path.extend_text_partition(m, qs, ks, 3, 5)
    assert torch.equal(em, rm) and torch.equal(eq, rq) and torch.equal(ek, rk)


def test_attention_rejects_bad_context():
    cfg = processor.PecoConfig(warmup_steps=0)
    ctx = processor.InferenceContext(step=0, text_length=10, valid_text_length=11)
    layer = processor.PecoAttention(0, cfg, ctx)
    q = torch.randn(1, 2, 20, 64)
    with pytest.raises(ValueError, match="video/text"):
        layer.attention(q, q, q)
    with pytest.raises(ValueError, match="one prompt"):
        layer.attention(q.expand(2, -1, -1, -1), q, q)


class _Linear(torch.nn.Linear):
    pass


class _FakeAttn:
    """Stands in for a diffusers Attention module (HunyuanVideo single-stream block)."""

    def __init__(self, dim=64, heads=2):
        torch.manual_seed(0)
        self.heads = heads
        self.to_q, self.to_k, self.to_v = (_Linear(dim, dim) for _ in range(3))
        self.norm_q = self.norm_k = None
        self.add_q_proj = None
        self.to_out = [_Linear(dim, dim), torch.nn.Identity()]
        self.processor = None

    def set_processor(self, p):
        self.processor = p


def test_call_warmup_path_runs_dense_sdpa_on_cpu():
    cfg = processor.PecoConfig(warmup_steps=5, zero_step_kmeans_init=False)
    ctx = processor.InferenceContext(step=0, text_length=4, valid_text_length=3)
    layer = processor.PecoAttention(0, cfg, ctx)
    attn = _FakeAttn()
    hidden = torch.randn(1, 12, 64)
    text = torch.randn(1, 4, 64)
    cos, sin = torch.ones(12, 32), torch.zeros(12, 32)
    out, enc = layer(attn, hidden, text, image_rotary_emb=(cos, sin))
    assert out.shape == (1, 12, 64) and enc.shape == (1, 4, 64)
    # Reference: dense attention over [video + valid text] and over the padding separately.
    h = torch.cat((hidden, text), 1)
    q, k, v = (p(h).unflatten(2, (2, -1)).transpose(1, 2) for p in (attn.to_q, attn.to_k, attn.to_v))
    o = torch.empty_like(q)
    o[:, :, :15] = torch.nn.functional.scaled_dot_product_attention(q[:, :, :15], k[:, :, :15], v[:, :, :15])
    o[:, :, 15:] = torch.nn.functional.scaled_dot_product_attention(q[:, :, 15:], k[:, :, 15:], v[:, :, 15:])
    o = o.transpose(1, 2).flatten(2, 3)
    assert torch.allclose(out, attn.to_out[0](o[:, :12]), atol=1e-5)


def test_install_attention_and_reset_state():
    class Block:
        def __init__(self):
            self.attn = _FakeAttn()

    class Transformer(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.transformer_blocks = [Block(), Block()]
            self.single_transformer_blocks = [Block()]

        def forward(self, hidden_states, encoder_attention_mask=None):
            return hidden_states

    class Pipe:
        transformer = Transformer()

    pipe = Pipe()
    ctx = model.install_attention(pipe, processor.PecoConfig())
    assert all(isinstance(b.attn.processor, processor.PecoAttention)
               for b in pipe.transformer.transformer_blocks + pipe.transformer.single_transformer_blocks)
    pipe.transformer(torch.zeros(1), encoder_attention_mask=torch.tensor([[1, 1, 1, 0]]))
    assert (ctx.step, ctx.text_length, ctx.valid_text_length) == (0, 4, 3)
    with pytest.raises(ValueError, match="right padding"):
        pipe.transformer(torch.zeros(1), encoder_attention_mask=torch.tensor([[1, 0, 1, 0]]))
    processors = pipe.transformer._peco_installation.processors
    assert [p.layer_idx for p in processors] == [0, 1, 2]
    processors[0].q_centroids = torch.zeros(1)
    model.reset_state(pipe)
    assert ctx.step == -1 and processors[0].q_centroids is None
    # Installing again replaces the hook: one transformer call advances the new context once,
    # and the old context no more.
    ctx2 = model.install_attention(pipe, processor.PecoConfig())
    pipe.transformer(torch.zeros(1), encoder_attention_mask=torch.tensor([[1, 1, 0, 0]]))
    assert (ctx2.step, ctx2.text_length, ctx2.valid_text_length) == (0, 4, 2)
    assert ctx.step == -1
    with pytest.raises(ValueError, match="one prompt"):
        pipe.transformer(torch.zeros(1), encoder_attention_mask=torch.ones(2, 4))


def test_reference_import_paths_resolve():
    """The reference's caller imports (generate.py:63-64) and the stage modules resolve
    through the `peco` package to the very modules of peco_amd."""
    from peco.model import install_attention, reset_state
    from peco.processor import PecoConfig
    from peco.clustering import fit_token_clusters, select_cluster_connections
    from peco.quantization import fake_quantize_base_offset
    from peco.attention_cuda import sparse_attention
    import peco.clustering_cuda

    assert PecoConfig is processor.PecoConfig
    assert install_attention is model.install_attention and reset_state is model.reset_state
    assert fit_token_clusters is clustering.fit_token_clusters
    assert select_cluster_connections is clustering.select_cluster_connections
    assert fake_quantize_base_offset is quantization.fake_quantize_base_offset
    assert sparse_attention is attention_cuda.sparse_attention
    import peco_amd.clustering_cuda
    assert peco.clustering_cuda is peco_amd.clustering_cuda
