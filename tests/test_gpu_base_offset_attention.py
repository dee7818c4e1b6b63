"""Base-Offset scores on the integer MFMA (attention_cuda.base_offset_attention), an extension.

The reference reconstructs Q and K from their Base-Offset payloads, rounds them to the input
dtype and runs floating-point attention (peco/quantization.py:132-150, peco/processor.py:141).
This kernel scores video rows against video keys from the payloads themselves through the
exact expansion of (Cq + a + s u).(Ck + b + t w), so its scores are those of the unrounded
reconstructions. Checked here:
- the codes, lows and scales the fit's packing pass writes equal the oracle's quantize of K
  in cluster order, bit for bit;
- the output equals the oracle's attention over the unrounded reconstructions (text rows
  raw) within the attention tolerance (max 2e-2, mean 2e-3);
- it is closer to that oracle than the kernel over rounded reconstructions is (a dropped or
  mis-signed term of the expansion would make it farther);
- the layer with ``integer_scores`` stays within the tolerance of the reference's own layer
  (peco_layer with bits=4: rounded reconstructions), for bf16 and fp16 inputs. This path is
  outside the parity contract with the reference (it skips the rounding of the
  reconstructions, peco/quantization.py:136); that last check is a bound on how far the
  extension strays, and its margin is printed.
"""
import numpy as np
import pytest
import torch

from oracle import canonical
from oracle import reference_path as ref
from peco_amd import attention_cuda, clustering_cuda, processor, workloads

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


def _inputs(seed, h, n, text, d, dtype, kq, kk):
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


def _exact_reference(q, k, v, q_labels, q_cent, k_labels, k_cent, q_idx, k_idx, ext_map, ext_q, ext_k, n, bits):
    """Oracle attention over the unrounded Base-Offset reconstructions (fp32), text rows raw."""
    h, d = q.shape[1], q.shape[3]
    qv = q[0, :, :n].cpu()
    kv = k[0, :, :n].cpu()

    def exact(x, labels, cent):
        codes, low, scale = ref.quantize(x, labels.cpu(), cent.cpu(), bits)
        return ref.dequantize(codes, low, scale, labels.cpu(), cent.cpu(), torch.float32, tuple(x.shape))

    q_hat = exact(qv, q_labels, q_cent)
    k_hat = exact(kv, k_labels, k_cent)
    qi, ki = q_idx.cpu().long(), k_idx.cpu().long()
    q_perm = torch.cat((q_hat.gather(1, qi[..., None].expand(-1, -1, d)), q[0, :, n:].cpu().float()), 1)
    k_perm = torch.cat((k_hat.gather(1, ki[..., None].expand(-1, -1, d)), k[0, :, n:].cpu().float()), 1)
    v_perm = torch.cat((v[0, :, :n].cpu().gather(1, ki[..., None].expand(-1, -1, d)), v[0, :, n:].cpu()), 1).float()
    out_perm = ref.sparse_attention(q_perm[None], k_perm[None], v_perm[None], ext_map.cpu(), ext_q.cpu(),
                                    ext_k.cpu())
    length = q.shape[2]
    text_idx = torch.arange(n, length, dtype=torch.int32)
    indices = torch.cat((q_idx.cpu().reshape(h, n), text_idx.expand(h, -1)), -1)
    return ref.restore_tokens(out_perm, indices)


@pytest.mark.parametrize("dtype,d,bits,h,n,text,valid", [
    (torch.bfloat16, 128, 4, 3, 2600, 40, 29),
    (torch.bfloat16, 128, 8, 2, 3000, 33, 33),
    (torch.float16, 64, 4, 3, 2200, 24, 0),
    (torch.bfloat16, 64, 8, 2, 1800, 17, 9),
])
def test_integer_scores_match_the_unrounded_reconstructions(announce, dtype, d, bits, h, n, text, valid):
    kq, kk = 12, 40
    q, k, v, q_init, k_init = _inputs(d * 7 + bits + n, h, n, text, d, dtype, kq, kk)
    length = n + text
    announce(f"{dtype} D={d} bits={bits} H={h} N={n} text={text} valid={valid}")
    problems = [clustering_cuda.KMeansProblem(q[0, :, :n], q_init), clustering_cuda.KMeansProblem(k[0, :, :n], k_init)]
    outs, packed = clustering_cuda.kmeans_fit(problems, 2, pack=[None, (bits, length, v[0], True)])
    (q_labels, q_cent, q_sizes, q_idx, _), (k_labels, k_cent, k_sizes, k_idx, _) = outs
    k_hat, v_out, k_codes, k_low, k_scale = packed[1]
    args = (q_cent[None], k_cent[None], q_sizes[None], k_sizes[None], 0.7, 4)
    ext_map, ext_q, ext_k = clustering_cuda.select_connections(*args, text=(valid, text))
    out = attention_cuda.base_offset_attention(
        q, k_hat[None], v_out[None], ext_map, ext_q, ext_k, out_index=q_idx, q_centroids=q_cent,
        k_centroids=k_cent, k_codes=k_codes, k_low=k_low, k_scale=k_scale, bits=bits)
    # The same selection's work list, for the kernel over rounded reconstructions.
    work = clustering_cuda.select_work(*args, (valid, text), length, length)
    rounded = attention_cuda.sparse_attention_work(q, k_hat[None], v_out[None], work, out_index=q_idx,
                                                   out_index_rows=n, q_centroids=q_cent, bits=bits)
    torch.cuda.synchronize()

    # The packing pass's payload is the oracle's quantize of K, in cluster order.
    codes, low, scale = ref.quantize(k[0, :, :n].cpu(), k_labels.cpu(), k_cent.cpu(), bits)
    ki = k_idx.cpu().long()
    assert torch.equal(k_codes.cpu(), codes.gather(1, ki[..., None].expand(-1, -1, d)))
    assert torch.equal(k_low.cpu(), low[..., 0].gather(1, ki))
    assert torch.equal(k_scale.cpu(), scale[..., 0].gather(1, ki))

    exact = _exact_reference(q, k, v, q_labels, q_cent, k_labels, k_cent, q_idx, k_idx, ext_map, ext_q, ext_k, n, bits)
    err = (out[0].float().cpu() - exact.float()).abs()
    err_rounded = (rounded[0].float().cpu() - exact.float()).abs()
    print(f"integer scores: max {err.max().item():.3e} mean {err.mean().item():.3e}; "
          f"rounded rows: max {err_rounded.max().item():.3e} mean {err_rounded.mean().item():.3e}", flush=True)
    assert torch.isfinite(out).all()
    assert err.max().item() <= 2e-2 and err.mean().item() <= 2e-3
    assert err.mean().item() < err_rounded.mean().item()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_layer_with_integer_scores_matches_the_reference_layer(announce, dtype):
    """The 480p Base-Offset configuration at two heads, against the reference path's layer
    (rounded reconstructions) with the fixed-order k-means of the oracle."""
    wl = workloads.make_workload("hunyuan_480p_bo4", heads=2)
    if dtype != wl.query.dtype:
        wl = workloads.Workload(wl.shape, wl.query.to(dtype), wl.key.to(dtype), wl.value.to(dtype), wl.q_init,
                                wl.k_init)
    shape, iters = wl.shape, wl.shape.iterations
    announce(f"{dtype} hunyuan_480p_bo4 heads=2 iters={iters}")
    cfg = processor.PecoConfig(num_q_centroids=shape.num_q_centroids, num_k_centroids=shape.num_k_centroids,
                               top_p=wl.top_p, min_kc_ratio=wl.min_kc_ratio, kmeans_iter_init=iters,
                               kmeans_iter_step=iters, warmup_steps=0, base_offset_bits=shape.bits)
    ctx = processor.InferenceContext(step=0, text_length=shape.text, valid_text_length=shape.text)
    layer = processor.PecoAttention(0, cfg, ctx)
    layer.integer_scores = True
    layer.q_centroids, layer.k_centroids = wl.q_init.to(DEV), wl.k_init.to(DEV)
    with torch.no_grad():
        out = layer.attention(wl.query.to(DEV), wl.key.to(DEV), wl.value.to(DEV))
    torch.cuda.synchronize()

    def fit(x, clusters, iters_, init):
        labels, centers, counts, _, _ = canonical.kmeans_fit(x.float().numpy(), init.numpy(), iters_)
        return torch.from_numpy(labels), torch.from_numpy(centers), torch.from_numpy(counts), iters_

    expected = ref.peco_layer(wl.query, wl.key, wl.value, num_q_centroids=shape.num_q_centroids,
                              num_k_centroids=shape.num_k_centroids, iterations=iters, q_init=wl.q_init,
                              k_init=wl.k_init, top_p=wl.top_p, min_kc_ratio=wl.min_kc_ratio, bits=shape.bits,
                              text_length=shape.text, valid_text=shape.text, fit=fit)
    err = (out.float().cpu() - expected.float()).abs()
    emax, emean = err.max().item(), err.mean().item()
    print(f"layer vs reference: max {emax:.3e} ({emax / 2e-2:.0%} of the 2e-2 bound), "
          f"mean {emean:.3e} ({emean / 2e-3:.0%} of 2e-3)", flush=True)
    assert emax <= 2e-2 and emean <= 2e-3
