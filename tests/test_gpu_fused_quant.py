"""Base-Offset fake quantization and the cluster gather fused into their neighbours.

With Base-Offset on, the layer has no cluster-order pack:
- the k-means fit ends with a token-parallel launch that writes Q and K fake-quantized against
  their final centres, each row at its own position with the text rows copied
  (peco_kmeans_fit_pack, hat_order 1); the integer-score extension takes K and V in the final
  key-cluster order from the last update instead (hat_order 0);
- the attention reads Q, K and V through the permutations (peco_sparse_attention_work with
  k_index). Its mode that fake-quantizes Q as it loads the rows (q_centroids) stays an entry
  point of its own.
All must equal the standalone pack launch (itself checked against the oracle's
fake_quantize + gather + concat in test_gpu_stages.py) bit for bit, and the attention over
them must equal the attention over packed inputs bit for bit.
"""
import pytest
import torch

from peco_amd import attention_cuda, clustering_cuda

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _gen(seed):
    g = torch.Generator()
    g.manual_seed(seed)
    return g


def _mixture(g, h, n, d, m, sigma=1.0):
    means = torch.randn(h, m, d, generator=g)
    means = means / means.norm(dim=-1, keepdim=True) * 8.0
    comp = torch.randint(m, (h, n), generator=g)
    return means.gather(1, comp[..., None].expand(-1, -1, d)) + sigma * torch.randn(h, n, d, generator=g)


def _bits_equal(a, b):
    return a.shape == b.shape and torch.equal(a.contiguous().view(torch.int16), b.contiguous().view(torch.int16))


def _fit_inputs(seed, h, n, text, d, dtype, kq, kk):
    g = _gen(seed)
    length = n + text
    q = _mixture(g, h, length, d, 24).to(dtype)[None].to(DEV)
    k = _mixture(g, h, length, d, 24).to(dtype)[None].to(DEV)
    v = torch.randn(1, h, length, d, generator=g).to(dtype).to(DEV)
    qi = torch.randint(n, (h, kq), generator=g)
    ki = torch.randint(n, (h, kk), generator=g)
    q_init = q[0, :, :n].float().gather(1, qi.to(DEV)[..., None].expand(-1, -1, d)).contiguous()
    k_init = k[0, :, :n].float().gather(1, ki.to(DEV)[..., None].expand(-1, -1, d)).contiguous()
    return q, k, v, q_init, k_init


# Wave-mode updates (few members per cluster), a shared-mode update (more than 64 members per
# cluster on average), D = 64 in fp16, 8-bit codes and a sequence without text rows.
@pytest.mark.parametrize("dtype,d,h,n,text,kq,kk,bits,iters", [
    (torch.bfloat16, 128, 3, 2000, 40, 12, 30, 4, 3),
    (torch.bfloat16, 128, 2, 9000, 32, 16, 40, 4, 2),
    (torch.float16, 64, 2, 3000, 16, 10, 20, 8, 2),
    (torch.bfloat16, 128, 2, 1500, 0, 8, 24, 4, 2),
])
def test_fit_packs_keys_and_values_like_the_pack_launch(announce, dtype, d, h, n, text, kq, kk, bits, iters):
    q, k, v, q_init, k_init = _fit_inputs(d + n + bits, h, n, text, d, dtype, kq, kk)
    length = n + text
    announce(f"{dtype} D={d} H={h} N={n} text={text} KQ={kq} KK={kk} bits={bits} iters={iters}")
    problems = [clustering_cuda.KMeansProblem(q[0, :, :n], q_init), clustering_cuda.KMeansProblem(k[0, :, :n], k_init)]
    plain = clustering_cuda.kmeans_fit(problems, iters)
    outs, packed = clustering_cuda.kmeans_fit(problems, iters, pack=[None, (bits, length, v[0])])
    assert packed[0] is None
    for a, b in zip(plain, outs):
        for x, y in zip(a, b):
            assert torch.equal(x, y)
    k_labels, k_cent, _, k_idx, _ = outs[1]
    k_hat, v_out = packed[1]
    ref_k, ref_v = clustering_cuda.pack_clustered([k, v], [k_idx, k_idx], [k_labels, None], [k_cent, None],
                                                  [bits, 0], n)
    torch.cuda.synchronize()
    assert _bits_equal(k_hat.cpu(), ref_k[0].cpu())
    assert _bits_equal(v_out.cpu(), ref_v[0].cpu())


@pytest.mark.parametrize("dtype,d,bits", [(torch.bfloat16, 128, 4), (torch.float16, 64, 8), (torch.bfloat16, 64, 4)])
def test_attention_quantizes_queries_at_load(announce, dtype, d, bits):
    h, n, text, valid, kq, kk = 4, 3000, 48, 37, 16, 48
    q, k, v, q_init, k_init = _fit_inputs(d * 3 + bits, h, n, text, d, dtype, kq, kk)
    length = n + text
    announce(f"{dtype} D={d} bits={bits}")
    problems = [clustering_cuda.KMeansProblem(q[0, :, :n], q_init), clustering_cuda.KMeansProblem(k[0, :, :n], k_init)]
    outs, packed = clustering_cuda.kmeans_fit(problems, 2, pack=[None, (bits, length, v[0])])
    (q_labels, q_cent, q_sizes, q_idx, _), (_, k_cent, k_sizes, _, _) = outs
    k_hat, v_out = (t[None] for t in packed[1])
    work = clustering_cuda.select_work(q_cent[None], k_cent[None], q_sizes[None], k_sizes[None], 0.7, 4,
                                       (valid, text), length, length)
    # Reference: Q fake-quantized and packed by the pack launch, then the packed-input attention.
    (q_hat,) = clustering_cuda.pack_clustered([q], [q_idx], [q_labels], [q_cent], [bits], n)
    ref = attention_cuda.sparse_attention_work(q_hat, k_hat, v_out, work, out_index=q_idx, out_index_rows=n)
    out = attention_cuda.sparse_attention_work(q, k_hat, v_out, work, out_index=q_idx, out_index_rows=n,
                                               q_centroids=q_cent, bits=bits)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)


@pytest.mark.parametrize("dtype,d,h,n,text,kq,kk,bits,iters", [
    (torch.bfloat16, 128, 3, 2000, 40, 12, 30, 4, 3),
    (torch.bfloat16, 128, 2, 9000, 32, 16, 40, 4, 2),
    (torch.float16, 64, 2, 3000, 16, 10, 20, 8, 2),
    (torch.bfloat16, 128, 2, 1500, 0, 8, 24, 4, 2),
])
def test_fit_packs_keys_in_original_order(announce, dtype, d, h, n, text, kq, kk, bits, iters):
    """pack_order="original": row t < N of the packed keys is key row t fake-quantized against
    its final centre (the cluster-order pack scattered back through the permutation), rows
    past N are the text rows unchanged, and the fit itself is unchanged."""
    q, k, v, q_init, k_init = _fit_inputs(d + n + bits + 1, h, n, text, d, dtype, kq, kk)
    length = n + text
    announce(f"{dtype} D={d} H={h} N={n} text={text} KQ={kq} KK={kk} bits={bits} iters={iters}")
    problems = [clustering_cuda.KMeansProblem(q[0, :, :n], q_init), clustering_cuda.KMeansProblem(k[0, :, :n], k_init)]
    plain = clustering_cuda.kmeans_fit(problems, iters)
    outs, packed = clustering_cuda.kmeans_fit(problems, iters, pack=[None, (bits, length, None)],
                                              pack_order="original")
    for a, b in zip(plain, outs):
        for x, y in zip(a, b):
            assert torch.equal(x, y)
    k_labels, k_cent, _, k_idx, _ = outs[1]
    k_hat, v_out = packed[1]
    assert v_out is None
    (ref_k,) = clustering_cuda.pack_clustered([k], [k_idx], [k_labels], [k_cent], [bits], n)
    expect = ref_k[0].clone()
    expect[:, :n] = torch.empty_like(expect[:, :n]).scatter_(
        1, k_idx.long()[..., None].expand(-1, -1, d), ref_k[0, :, :n])
    torch.cuda.synchronize()
    assert _bits_equal(k_hat.cpu(), expect.cpu())
    assert _bits_equal(k_hat[:, n:].cpu(), k[0, :, n:].cpu())
    with pytest.raises(ValueError, match="pack_order"):
        clustering_cuda.kmeans_fit(problems, iters, pack=[None, (bits, length, v[0])], pack_order="original")


@pytest.mark.parametrize("dtype,d,bits", [(torch.bfloat16, 128, 4), (torch.float16, 64, 8), (torch.bfloat16, 64, 4)])
def test_attention_quantizes_queries_with_indexed_keys(announce, dtype, d, bits):
    """The layer's Base-Offset attention (Q quantized at load, K fake-quantized in original
    order, V the input itself, both read through the key permutation) equals the attention
    over the cluster-order pack bit for bit."""
    h, n, text, valid, kq, kk = 4, 3000, 48, 37, 16, 48
    q, k, v, q_init, k_init = _fit_inputs(d * 3 + bits + 1, h, n, text, d, dtype, kq, kk)
    length = n + text
    announce(f"{dtype} D={d} bits={bits}")
    problems = [clustering_cuda.KMeansProblem(q[0, :, :n], q_init), clustering_cuda.KMeansProblem(k[0, :, :n], k_init)]
    outs, packed = clustering_cuda.kmeans_fit(problems, 2, pack=[None, (bits, length, v[0])])
    (q_labels, q_cent, q_sizes, q_idx, _), (_, k_cent, k_sizes, k_idx, _) = outs
    k_perm, v_perm = (t[None] for t in packed[1])
    _, packed_o = clustering_cuda.kmeans_fit(problems, 2, pack=[None, (bits, length, None)], pack_order="original")
    k_hat = packed_o[1][0][None]
    work = clustering_cuda.select_work(q_cent[None], k_cent[None], q_sizes[None], k_sizes[None], 0.7, 4,
                                       (valid, text), length, length)
    ref = attention_cuda.sparse_attention_work(q, k_perm, v_perm, work, out_index=q_idx, out_index_rows=n,
                                               q_centroids=q_cent, bits=bits)
    out = attention_cuda.sparse_attention_work(q, k_hat, v, work, out_index=q_idx, out_index_rows=n,
                                               k_index=k_idx, q_centroids=q_cent, bits=bits)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)


@pytest.mark.parametrize("dtype,d,h,n,text,kq,kk,bits", [
    (torch.bfloat16, 128, 3, 2000, 40, 12, 30, 4),
    (torch.float16, 64, 2, 3000, 16, 10, 20, 8),
    (torch.bfloat16, 128, 2, 1500, 0, 8, 24, 4),
])
def test_fit_packs_queries_and_keys_in_original_order(announce, dtype, d, h, n, text, kq, kk, bits):
    """Both problems packed in original order (the Base-Offset layer's fit): each equals the
    cluster-order pack launch scattered back through its permutation, and the attention over
    the two fake-quantized tensors (indexed inputs) equals the attention that fake-quantizes Q
    as it loads it, bit for bit."""
    q, k, v, q_init, k_init = _fit_inputs(d + n + bits + 2, h, n, text, d, dtype, kq, kk)
    length = n + text
    announce(f"{dtype} D={d} H={h} N={n} text={text} KQ={kq} KK={kk} bits={bits}")
    problems = [clustering_cuda.KMeansProblem(q[0, :, :n], q_init), clustering_cuda.KMeansProblem(k[0, :, :n], k_init)]
    plain = clustering_cuda.kmeans_fit(problems, 2)
    outs, packed = clustering_cuda.kmeans_fit(problems, 2, pack=[(bits, length, None), (bits, length, None)],
                                              pack_order="original")
    for a, b in zip(plain, outs):
        for x, y in zip(a, b):
            assert torch.equal(x, y)
    for src, (labels, cent, _, idx, _), (hat, extra) in zip((q, k), outs, packed):
        assert extra is None
        (ref,) = clustering_cuda.pack_clustered([src], [idx], [labels], [cent], [bits], n)
        expect = ref[0].clone()
        expect[:, :n] = torch.empty_like(expect[:, :n]).scatter_(
            1, idx.long()[..., None].expand(-1, -1, d), ref[0, :, :n])
        torch.cuda.synchronize()
        assert _bits_equal(hat.cpu(), expect.cpu())
    (q_labels, q_cent, q_sizes, q_idx, _), (_, k_cent, k_sizes, k_idx, _) = outs
    q_hat, k_hat = packed[0][0][None], packed[1][0][None]
    work = clustering_cuda.select_work(q_cent[None], k_cent[None], q_sizes[None], k_sizes[None], 0.7, 4,
                                       (max(text - 3, 0), text), length, length)
    ref = attention_cuda.sparse_attention_work(q, k_hat, v, work, out_index=q_idx, out_index_rows=n,
                                               k_index=k_idx, q_centroids=q_cent, bits=bits)
    out = attention_cuda.sparse_attention_work(q_hat, k_hat, v, work, out_index=q_idx, out_index_rows=n,
                                               k_index=k_idx)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)
