"""End-to-end GPU parity of PecoAttention.attention against the oracle's reference path."""
import numpy as np
import pytest
import torch

from oracle import canonical, reference_path
from peco_amd import processor, workloads

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _run_layer(wl, iterations, valid_text=None):
    shape = wl.shape
    valid_text = shape.text if valid_text is None else valid_text
    cfg = processor.PecoConfig(num_q_centroids=shape.num_q_centroids, num_k_centroids=shape.num_k_centroids,
                               top_p=wl.top_p, min_kc_ratio=wl.min_kc_ratio, kmeans_iter_init=iterations,
                               kmeans_iter_step=iterations, warmup_steps=0, base_offset_bits=shape.bits)
    ctx = processor.InferenceContext(step=0, text_length=shape.text, valid_text_length=valid_text)
    layer = processor.PecoAttention(0, cfg, ctx)
    layer.record_intermediates = True
    layer.q_centroids, layer.k_centroids = wl.q_init.to(DEV), wl.k_init.to(DEV)
    with torch.no_grad():
        out = layer.attention(wl.query.to(DEV), wl.key.to(DEV), wl.value.to(DEV))
    torch.cuda.synchronize()
    return layer, out


def _oracle_layer(wl, iterations, valid_text=None):
    shape = wl.shape
    valid_text = shape.text if valid_text is None else valid_text

    def attend(q, k, v, m, qs, ks):
        o = canonical.sparse_attention(q[0].float().numpy(), k[0].float().numpy(), v[0].float().numpy(),
                                       m[0].numpy(), qs[0].numpy(), ks[0].numpy())
        return torch.from_numpy(o)[None]

    def fit(x, clusters, iters, init):
        labels, centers, counts, _, _ = canonical.kmeans_fit(x.float().numpy(), init.numpy(), iters)
        return torch.from_numpy(labels), torch.from_numpy(centers), torch.from_numpy(counts), iters

    stages = {}
    out = reference_path.peco_layer(
        wl.query, wl.key, wl.value, num_q_centroids=shape.num_q_centroids, num_k_centroids=shape.num_k_centroids,
        iterations=iterations, q_init=wl.q_init, k_init=wl.k_init, top_p=wl.top_p, min_kc_ratio=wl.min_kc_ratio,
        bits=shape.bits, text_length=shape.text, valid_text=valid_text, attention=attend, fit=fit, stages=stages)
    return out, stages


@pytest.mark.parametrize("name,heads,video", [
    ("hunyuan_480p", 2, 6750),
    ("hunyuan_480p_bo4", 2, 6750),
    ("cpu_small", 2, 2048),
    # The 720p and 544p Zipf configurations at one head and a shortened sequence: their
    # cluster counts (256/1024 and 128/512), iteration counts, keep ratios, Base-Offset and
    # mixture weights are kept, so small and heavily skewed clusters are exercised.
    ("hunyuan_720p", 1, 12000),
    ("hunyuan_544p_zipf", 1, 16384),
])
def test_layer_matches_oracle(announce, name, heads, video):
    wl = workloads.make_workload(name, heads=heads, video=video)
    if wl.query.dtype == torch.float32:
        # The sparse attention kernel takes fp16/bf16 (as the reference's); run the fp32
        # workload in bf16 end to end.
        wl = workloads.Workload(wl.shape, wl.query.bfloat16(), wl.key.bfloat16(), wl.value.bfloat16(),
                                wl.q_init, wl.k_init)
    iters = wl.shape.iterations
    announce(f"{name} heads={heads} video={video} iters={iters}")
    layer, out = _run_layer(wl, iters)
    ref, st = _oracle_layer(wl, iters)
    # Stage 1 + 3: labels and permutations are bit-exact.
    n = wl.shape.video
    q_idx, k_idx = layer._last_fit
    xq = wl.query[0, :, :n].float().numpy()
    rl, rc, _, ridx, _ = canonical.kmeans_fit(xq, wl.q_init.numpy(), iters)
    assert np.array_equal(q_idx.cpu().numpy(), ridx)
    assert np.array_equal(layer.q_centroids.cpu().numpy().view(np.int32), rc.view(np.int32))
    # K has the larger cluster count, where the saturated-list fallback of the assign runs.
    xk = wl.key[0, :, :n].float().numpy()
    _, kc, _, kidx, _ = canonical.kmeans_fit(xk, wl.k_init.numpy(), iters)
    assert np.array_equal(k_idx.cpu().numpy(), kidx)
    assert np.array_equal(layer.k_centroids.cpu().numpy().view(np.int32), kc.view(np.int32))
    # The torch-literal k-means of the reference path (peco/clustering.py:67-73) agrees with
    # the labels of this layer (equal to the canonical ones above) except at fp32 near-ties,
    # where its bmm summation order (MKL's) decides; a tie settled differently can move later
    # iterations' centres, so the bound is on the fraction after all iterations.
    agreement = {}
    for side, x, init, clusters, labels in (
            ("Q", xq, wl.q_init, wl.shape.num_q_centroids, rl),
            ("K", xk, wl.k_init, wl.shape.num_k_centroids, canonical.kmeans_fit(xk, wl.k_init.numpy(), iters)[0])):
        tl, _, _, _ = reference_path.fit_token_clusters(torch.from_numpy(x), clusters, iters, init)
        agreement[side] = (tl.numpy() == labels).mean()
        assert agreement[side] >= 0.999, f"{side}: reference-path label agreement {agreement[side]}"
    err = (out.float().cpu() - ref.float()).abs()
    print(f"[layer] {name}: max {err.max().item():.3e} mean {err.mean().item():.3e} "
          f"label agreement Q {agreement['Q']:.6f} K {agreement['K']:.6f}", flush=True)
    assert err.mean().item() <= 2e-3
    assert err.max().item() <= 2e-2


def test_layer_warm_start_second_step(announce):
    """Two denoising steps of the skewed (Zipf) workload. Both calls find cached centroids
    (the first the seeded initial ones, the second the first call's result) and so run the
    warm-start iteration count; the second runs on drifted Q/K. Each step's permutations,
    centroids and output are checked against the oracle started from the oracle's own
    previous centroids."""
    wl = workloads.make_workload("hunyuan_544p_zipf", heads=1, video=8192)
    shape = wl.shape
    announce(f"warm start: heads=1 video={shape.video} init={shape.iterations} step={shape.warm_iterations}")
    cfg = processor.PecoConfig(num_q_centroids=shape.num_q_centroids, num_k_centroids=shape.num_k_centroids,
                               top_p=wl.top_p, min_kc_ratio=wl.min_kc_ratio, kmeans_iter_init=shape.iterations,
                               kmeans_iter_step=shape.warm_iterations, warmup_steps=0, base_offset_bits=shape.bits)
    ctx = processor.InferenceContext(step=0, text_length=shape.text, valid_text_length=shape.text)
    layer = processor.PecoAttention(0, cfg, ctx)
    layer.record_intermediates = True
    layer.q_centroids, layer.k_centroids = wl.q_init.to(DEV), wl.k_init.to(DEV)
    n = shape.video
    q_init, k_init = wl.q_init, wl.k_init
    for step, iters in ((0, shape.warm_iterations), (1, shape.warm_iterations)):
        cur = wl if step == 0 else workloads.drift(wl, step)
        with torch.no_grad():
            out = layer.attention(cur.query.to(DEV), cur.key.to(DEV), cur.value.to(DEV))
        torch.cuda.synchronize()
        ref, _ = _oracle_layer(workloads.Workload(shape, cur.query, cur.key, cur.value, q_init, k_init), iters)
        xq = cur.query[0, :, :n].float().numpy()
        xk = cur.key[0, :, :n].float().numpy()
        _, qc, _, qidx, _ = canonical.kmeans_fit(xq, q_init.numpy(), iters)
        _, kc, _, kidx, _ = canonical.kmeans_fit(xk, k_init.numpy(), iters)
        q_idx, k_idx = layer._last_fit
        assert np.array_equal(q_idx.cpu().numpy(), qidx), f"step {step}: Q permutation"
        assert np.array_equal(k_idx.cpu().numpy(), kidx), f"step {step}: K permutation"
        assert np.array_equal(layer.q_centroids.cpu().numpy().view(np.int32), qc.view(np.int32))
        assert np.array_equal(layer.k_centroids.cpu().numpy().view(np.int32), kc.view(np.int32))
        err = (out.float().cpu() - ref.float()).abs()
        print(f"[warm] step {step} ({iters} iterations): max {err.max().item():.3e} "
              f"mean {err.mean().item():.3e}", flush=True)
        assert err.mean().item() <= 2e-3
        assert err.max().item() <= 2e-2
        q_init, k_init = torch.from_numpy(qc), torch.from_numpy(kc)


def test_layer_full_size_heads_independent(announce):
    """The 480p layer at its full size (24 heads). Heads share nothing, so the first two heads
    of the 24-head call equal a call on those two heads alone, bit for bit (output and sort
    permutations); every head's permutation is a permutation of its video tokens; and head 0
    matches the oracle."""
    wl = workloads.make_workload("hunyuan_480p")
    iters = wl.shape.iterations
    n = wl.shape.video
    announce(f"hunyuan_480p full size: heads={wl.shape.heads} video={n} iters={iters}")
    layer, out = _run_layer(wl, iters)
    q_idx, k_idx = (t.cpu() for t in layer._last_fit)
    ar = torch.arange(n, dtype=q_idx.dtype)
    for idx in (q_idx, k_idx):
        assert idx.shape == (wl.shape.heads, n)
        assert torch.equal(idx.sort(dim=-1).values, ar.expand(wl.shape.heads, n))
    assert torch.isfinite(out.float()).all()

    def heads(w, sel):
        shape = workloads.LayerShape(**{**w.shape.__dict__, "heads": len(sel)})
        return workloads.Workload(shape, w.query[:, sel].contiguous(), w.key[:, sel].contiguous(),
                                  w.value[:, sel].contiguous(), w.q_init[sel].contiguous(), w.k_init[sel].contiguous())

    part = heads(wl, [0, 1])
    layer2, out2 = _run_layer(part, iters)
    assert torch.equal(out[:, :2].cpu(), out2.cpu())
    assert torch.equal(q_idx[:2], layer2._last_fit[0].cpu())
    assert torch.equal(k_idx[:2], layer2._last_fit[1].cpu())
    ref, _ = _oracle_layer(heads(wl, [0]), iters)
    err = (out[:, :1].float().cpu() - ref.float()).abs()
    print(f"[full] head 0: max {err.max().item():.3e} mean {err.mean().item():.3e}", flush=True)
    assert err.mean().item() <= 2e-3
    assert err.max().item() <= 2e-2


@pytest.mark.parametrize("name,dtype,pad", [
    ("hunyuan_480p", torch.bfloat16, 100),
    ("hunyuan_480p_bo4", torch.float16, 37),
    ("hunyuan_480p", torch.float16, 0),
    ("hunyuan_480p_bo4", torch.bfloat16, 256),
])
def test_layer_padded_text_and_fp16(announce, name, dtype, pad):
    """Text padding (valid_text < text length: the padding rows attend only to themselves, the
    valid text and video never to them) and fp16 inputs, end to end against the oracle."""
    wl = workloads.make_workload(name, heads=1, video=4096)
    wl = workloads.Workload(wl.shape, wl.query.to(dtype), wl.key.to(dtype), wl.value.to(dtype), wl.q_init, wl.k_init)
    valid = wl.shape.text - pad
    iters = wl.shape.iterations
    announce(f"{name} {dtype} video=4096 text={wl.shape.text} valid_text={valid}")
    layer, out = _run_layer(wl, iters, valid_text=valid)
    ref, _ = _oracle_layer(wl, iters, valid_text=valid)
    assert out.dtype == dtype
    err = (out.float().cpu() - ref.float()).abs()
    print(f"[padded] {name} {dtype} valid {valid}: max {err.max().item():.3e} mean {err.mean().item():.3e}", flush=True)
    assert err.mean().item() <= 2e-3
    assert err.max().item() <= 2e-2


def test_layer_head_bands_bit_exact(announce):
    """At 119056 tokens the attention runs its 8 heads in two bands of 4 (one band's K/V fill
    the MALL); a call on the first two heads runs them in one band. Heads are independent, so
    the two calls agree bit for bit on those heads."""
    wl = workloads.make_workload("hunyuan_720p", heads=8, device=DEV)
    iters = 2
    announce(f"hunyuan_720p heads=8 video={wl.shape.video} iters={iters}")
    _, out = _run_layer(wl, iters)
    shape = workloads.LayerShape(**{**wl.shape.__dict__, "heads": 2})
    part = workloads.Workload(shape, wl.query[:, :2].contiguous(), wl.key[:, :2].contiguous(),
                              wl.value[:, :2].contiguous(), wl.q_init[:2].contiguous(), wl.k_init[:2].contiguous())
    _, out2 = _run_layer(part, iters)
    assert torch.isfinite(out.float()).all()
    assert torch.equal(out[:, :2], out2)


def test_layer_full_length_720p_head_matches_oracle(announce):
    """One head of the 720p layer at its full length (118800 video + 256 text tokens, 256/1024
    clusters, 8 iterations, 15% of key clusters kept, Base-Offset 4-bit). Permutations and
    centroids of Q and K are bit-exact against the C oracle's fit; the output is compared with
    the oracle's layer, whose block-sparse attention runs in fp32 torch on the CPU (the
    float64 brute force would take minutes at this length)."""
    wl = workloads.make_workload("hunyuan_720p", heads=1)
    shape = wl.shape
    iters = shape.iterations
    n = shape.video
    announce(f"hunyuan_720p full length: heads=1 video={n} clusters={shape.num_q_centroids}/"
             f"{shape.num_k_centroids} iters={iters} bits={shape.bits}")
    layer, out = _run_layer(wl, iters)
    q_idx, k_idx = (t.cpu().numpy() for t in layer._last_fit)
    fits = {}
    for name, x, init in (("q", wl.query, wl.q_init), ("k", wl.key, wl.k_init)):
        fits[name] = canonical.kmeans_fit(x[0, :, :n].float().numpy(), init.numpy(), iters)
    assert np.array_equal(q_idx, fits["q"][3]), "Q permutation"
    assert np.array_equal(k_idx, fits["k"][3]), "K permutation"
    assert np.array_equal(layer.q_centroids.cpu().numpy().view(np.int32), fits["q"][1].view(np.int32))
    assert np.array_equal(layer.k_centroids.cpu().numpy().view(np.int32), fits["k"][1].view(np.int32))

    def fit(x, clusters, iterations, init):
        labels, centers, counts, _, _ = fits["q" if clusters == shape.num_q_centroids else "k"]
        return torch.from_numpy(labels), torch.from_numpy(centers), torch.from_numpy(counts), iterations

    ref = reference_path.peco_layer(
        wl.query, wl.key, wl.value, num_q_centroids=shape.num_q_centroids, num_k_centroids=shape.num_k_centroids,
        iterations=iters, q_init=wl.q_init, k_init=wl.k_init, top_p=wl.top_p, min_kc_ratio=wl.min_kc_ratio,
        bits=shape.bits, text_length=shape.text, valid_text=shape.text, fit=fit)
    err = (out.float().cpu() - ref.float()).abs()
    print(f"[720p head] max {err.max().item():.3e} mean {err.mean().item():.3e}", flush=True)
    assert err.mean().item() <= 2e-3
    assert err.max().item() <= 2e-2


def test_layer_544p_zipf_sequence_full_length_matches_oracle(announce):
    """The 10-call denoising sequence of the Zipf workload on one head at its full length
    (32640 video + 256 text tokens, 128/512 clusters, 20% kept, Base-Offset 4-bit): the first
    call fits 10 iterations from the seeded centroids, every later call warm-starts from the
    previous call's centroids with 3 iterations on Q/K drifted by N(0, 0.1^2) per step, as the
    bench's sequence does. Every call's permutations and centroids are bit-exact against the C
    oracle started from the oracle's own previous centroids, and its output is compared with
    the oracle's layer (fp32 torch block-sparse attention on the CPU)."""
    wl = workloads.make_workload("hunyuan_544p_zipf", heads=1)
    shape = wl.shape
    n = shape.video
    announce(f"544p Zipf sequence: heads=1 video={n} calls={shape.steps} init={shape.iterations} "
             f"warm={shape.warm_iterations}")
    cfg = processor.PecoConfig(num_q_centroids=shape.num_q_centroids, num_k_centroids=shape.num_k_centroids,
                               top_p=wl.top_p, min_kc_ratio=wl.min_kc_ratio, kmeans_iter_init=shape.iterations,
                               kmeans_iter_step=shape.iterations, warmup_steps=0, base_offset_bits=shape.bits)
    ctx = processor.InferenceContext(step=0, text_length=shape.text, valid_text_length=shape.text)
    layer = processor.PecoAttention(0, cfg, ctx)
    layer.record_intermediates = True
    layer.q_centroids, layer.k_centroids = wl.q_init.to(DEV), wl.k_init.to(DEV)
    q_init, k_init = wl.q_init, wl.k_init
    worst = 0.0
    for step in range(shape.steps):
        iters = shape.iterations if step == 0 else shape.warm_iterations
        layer.config = processor.PecoConfig(**{**cfg.__dict__, "kmeans_iter_step": iters})
        cur = wl if step == 0 else workloads.drift(wl, step)
        print(f"[case] call {step}: {iters} iterations", flush=True)
        with torch.no_grad():
            out = layer.attention(cur.query.to(DEV), cur.key.to(DEV), cur.value.to(DEV))
        torch.cuda.synchronize()
        fits = {}
        for name, x, init in (("q", cur.query, q_init), ("k", cur.key, k_init)):
            fits[name] = canonical.kmeans_fit(x[0, :, :n].float().numpy(), init.numpy(), iters)
        q_idx, k_idx = (t.cpu().numpy() for t in layer._last_fit)
        assert np.array_equal(q_idx, fits["q"][3]), f"call {step}: Q permutation"
        assert np.array_equal(k_idx, fits["k"][3]), f"call {step}: K permutation"
        assert np.array_equal(layer.q_centroids.cpu().numpy().view(np.int32), fits["q"][1].view(np.int32))
        assert np.array_equal(layer.k_centroids.cpu().numpy().view(np.int32), fits["k"][1].view(np.int32))

        def fit(x, clusters, iterations, init, fits=fits):
            labels, centers, counts, _, _ = fits["q" if clusters == shape.num_q_centroids else "k"]
            return torch.from_numpy(labels), torch.from_numpy(centers), torch.from_numpy(counts), iterations

        ref = reference_path.peco_layer(
            cur.query, cur.key, cur.value, num_q_centroids=shape.num_q_centroids,
            num_k_centroids=shape.num_k_centroids, iterations=iters, q_init=q_init, k_init=k_init, top_p=wl.top_p,
            min_kc_ratio=wl.min_kc_ratio, bits=shape.bits, text_length=shape.text, valid_text=shape.text, fit=fit)
        err = (out.float().cpu() - ref.float()).abs()
        print(f"[544p sequence] call {step}: max {err.max().item():.3e} mean {err.mean().item():.3e}", flush=True)
        assert err.mean().item() <= 2e-3
        assert err.max().item() <= 2e-2
        worst = max(worst, err.max().item())
        q_init, k_init = torch.from_numpy(fits["q"][1]), torch.from_numpy(fits["k"][1])
    print(f"[544p sequence] worst max error over {shape.steps} calls: {worst:.3e}", flush=True)


@pytest.mark.parametrize("bits", [0, 4])
def test_layer_head_dim_64_matches_oracle(announce, bits):
    """The layer at head dimension 64 (the other size the attention and fit kernels take),
    with and without Base-Offset: permutations and centres bit-exact, output within the
    attention tolerance of the oracle's layer."""
    base = workloads.SHAPES["hunyuan_480p_bo4" if bits else "hunyuan_480p"]
    shape = workloads.LayerShape(**{**base.__dict__, "dims": 64, "heads": 2, "video": 3000, "iterations": 6})
    wl = workloads.make_workload(shape)
    iters = shape.iterations
    announce(f"D=64 bits={bits} heads=2 video=3000 iters={iters}")
    layer, out = _run_layer(wl, iters)
    ref, _ = _oracle_layer(wl, iters)
    n = shape.video
    q_idx, k_idx = layer._last_fit
    for x, init, idx, cent in ((wl.query, wl.q_init, q_idx, layer.q_centroids),
                               (wl.key, wl.k_init, k_idx, layer.k_centroids)):
        _, rc, _, ridx, _ = canonical.kmeans_fit(x[0, :, :n].float().numpy(), init.numpy(), iters)
        assert np.array_equal(idx.cpu().numpy(), ridx)
        assert np.array_equal(cent.cpu().numpy().view(np.int32), rc.view(np.int32))
    err = (out.float().cpu() - ref.float()).abs()
    print(f"[D=64] bits={bits}: max {err.max().item():.3e} mean {err.mean().item():.3e}", flush=True)
    assert err.mean().item() <= 2e-3
    assert err.max().item() <= 2e-2


def _near_tie_bound(x, c, best):
    """fp32 near-tie band of the distance |c|^2 - 2 x.c between two summation orders: each
    order's error is at most gamma_D |x||c| (the dot) plus an ulp of the result, so two
    orders differ by under 4 gamma_D |x| max|c| + 4 u |best| (the band test_oracle.py uses
    for the CPU assignment)."""
    u = 2.0 ** -24
    d = x.shape[-1]
    gamma = d * u / (1 - d * u)
    return 4 * gamma * np.linalg.norm(x, axis=-1) * np.linalg.norm(c, axis=-1).max(-1)[..., None] + 4 * u * np.abs(best)


@pytest.mark.parametrize("name", ["hunyuan_480p", "hunyuan_544p_zipf"])
def test_first_assignment_matches_reference_torch_path_up_to_near_ties(announce, name):
    """Lock-step first iteration of the layer's fit against the reference's own torch
    formula (-2 x.c^T by bmm + |c|^2, argmin; peco/clustering.py:67-73) from the same initial
    centroids, Q and K: the GPU labels may differ only where the two candidates' float64
    distances lie within the fp32 near-tie band, and on under 0.1% of the tokens. The second
    case builds near-ties on purpose (centres taken from the tokens, as test_oracle.py does on
    the CPU), so the band check is exercised."""
    from peco_amd import clustering_cuda

    cases = []
    if name == "hunyuan_480p":
        wl = workloads.make_workload(name, heads=4)
        n = wl.shape.video
        cases += [("Q", wl.query[0, :, :n].float(), wl.q_init), ("K", wl.key[0, :, :n].float(), wl.k_init)]
    else:
        g = torch.Generator()
        g.manual_seed(2)
        x = torch.randn(4, 3000, 128, generator=g) * 2
        c = x[:, torch.randint(3000, (200,), generator=g)].contiguous()
        cases.append(("tokens as centres", x, c))
    for side, x, init in cases:
        xb = x.to(torch.bfloat16)
        announce(f"{name} {side}: {tuple(x.shape)} x {tuple(init.shape)}")
        (labels, _, _, _, _), = clustering_cuda.kmeans_fit(
            [clustering_cuda.KMeansProblem(xb.to(DEV), init.to(DEV))], 1)
        gpu = labels.cpu().numpy()
        xf = xb.float()
        dist = -2 * torch.bmm(xf, init.float().transpose(1, 2)) + init.float().square().sum(-1).unsqueeze(1)
        ref = dist.argmin(-1).numpy()
        diff = gpu != ref
        x64, c64 = xf.double().numpy(), init.double().numpy()
        d64 = (c64 ** 2).sum(-1)[:, None, :] - 2 * np.einsum("bnd,bkd->bnk", x64, c64)
        rows = np.arange(d64.shape[0])[:, None]
        cols = np.arange(d64.shape[1])[None, :]
        gap = np.abs(d64[rows, cols, gpu] - d64[rows, cols, ref])
        band = _near_tie_bound(xf.numpy(), init.float().numpy(), d64.min(-1))
        print(f"[first assign] {name} {side}: {diff.sum()} of {diff.size} labels differ", flush=True)
        assert np.all(gap[diff] <= band[diff]), "a disagreement lies outside the fp32 near-tie band"
        assert diff.mean() < 1e-3


def test_layer_keeps_no_intermediates_by_default(announce):
    """After a sparse call a layer holds only its centroids: the permutations and the
    fake-quantized keys of the call are not kept (record_intermediates is off)."""
    wl = workloads.make_workload("hunyuan_480p_bo4", heads=2, video=4096)
    shape = wl.shape
    announce("hunyuan_480p_bo4 heads=2 video=4096")
    cfg = processor.PecoConfig(num_q_centroids=shape.num_q_centroids, num_k_centroids=shape.num_k_centroids,
                               top_p=wl.top_p, min_kc_ratio=wl.min_kc_ratio, kmeans_iter_init=2,
                               kmeans_iter_step=2, warmup_steps=0, base_offset_bits=shape.bits)
    ctx = processor.InferenceContext(step=0, text_length=shape.text, valid_text_length=shape.text)
    layer = processor.PecoAttention(0, cfg, ctx)
    layer.q_centroids, layer.k_centroids = wl.q_init.to(DEV), wl.k_init.to(DEV)
    with torch.no_grad():
        out = layer.attention(wl.query.to(DEV), wl.key.to(DEV), wl.value.to(DEV))
    torch.cuda.synchronize()
    assert torch.isfinite(out.float()).all()
    assert layer._last_fit is None and layer._last_pack is None
    assert layer.q_centroids is not None and layer.k_centroids is not None
