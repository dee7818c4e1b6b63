"""GPU parity of each hot-path stage against the CPU oracle (bit-exact where integer/byte).

Every test feeds the HIP kernel and the oracle the same seeded inputs. Integer and byte
results (labels, permutations, counts, codes) and the fixed-order fp32 results (centres,
norms, Base-Offset reconstructions) must match bit for bit; attention output must be
within max-abs 2e-2 and mean-abs 2e-3 of the float64 oracle.
"""
import ctypes

import numpy as np
import pytest
import torch

from oracle import canonical, reference_path
from peco_amd import _native, attention_cuda, clustering, clustering_cuda, quantization, workloads

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _gen(seed):
    g = torch.Generator()
    g.manual_seed(seed)
    return g


def _mixture(g, bh, n, d, m, sigma=1.0):
    means = torch.randn(bh, m, d, generator=g)
    means = means / means.norm(dim=-1, keepdim=True) * 8.0
    comp = torch.randint(m, (bh, n), generator=g)
    return means.gather(1, comp[..., None].expand(-1, -1, d)) + sigma * torch.randn(bh, n, d, generator=g)


# ---------------------------------------------------------------- stage 3: sort + reorder

# 40000 and 118800 tokens span several 32-tile scan groups (the last one partial).
@pytest.mark.parametrize("clusters,tokens", [(1, 777), (7, 5000), (256, 6750), (1000, 3000), (64, 70), (300, 40000),
                                             (1024, 118800)])
def test_cluster_sort_matches_stable_argsort(announce, clusters, tokens):
    g = _gen(clusters * 31 + tokens)
    labels = torch.randint(clusters, (3, tokens), generator=g, dtype=torch.int32)
    announce(f"K={clusters} N={tokens}")
    idx, counts, offsets = clustering_cuda.cluster_sort(labels.to(DEV), clusters)
    ref_idx, ref_off = canonical.stable_sort(labels.numpy(), clusters)
    assert np.array_equal(idx.cpu().numpy(), ref_idx)
    assert np.array_equal(offsets.cpu().numpy(), ref_off)
    assert np.array_equal(counts.cpu().numpy(), np.diff(ref_off, axis=1))
    torch_idx = torch.argsort(labels, dim=-1, stable=True).to(torch.int32)
    assert torch.equal(idx.cpu(), torch_idx)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("dims", [64, 128, 40])
def test_reorder_roundtrip_bit_exact(announce, dtype, dims):
    g = _gen(dims)
    x = torch.randn(1, 3, 513, dims, generator=g).to(dtype)
    perm = torch.stack([torch.randperm(513, generator=g) for _ in range(3)]).to(torch.int32)
    announce(f"{dtype} D={dims}")
    xd, pd = x.to(DEV), perm.to(DEV)
    fwd = clustering_cuda.reorder_token_features(xd, pd)
    inv = clustering_cuda.reorder_token_features(fwd, pd, inverse=True)
    ref = reference_path.gather_tokens(x, perm)
    assert torch.equal(fwd.cpu().view(torch.int16 if dtype != torch.float32 else torch.int32),
                       ref.view(torch.int16 if dtype != torch.float32 else torch.int32))
    assert torch.equal(inv.cpu(), x)
    assert torch.equal(clustering.restore_sequence_order(fwd, pd).cpu(), x)


# ---------------------------------------------------------------- stage 2: Base-Offset

def _bits_equal(a, b):
    a, b = a.contiguous(), b.contiguous()
    if a.dtype in (torch.bfloat16, torch.float16):
        return torch.equal(a.view(torch.int16), b.view(torch.int16))
    if a.dtype == torch.float32:
        return torch.equal(a.view(torch.int32), b.view(torch.int32))
    return torch.equal(a, b)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("dims", [128, 64])
def test_base_offset_bit_exact(announce, dtype, bits, dims):
    g = _gen(bits * 7 + dims)
    bh, n, k = 3, 1500, 24
    x = _mixture(g, bh, n, dims, 8).to(dtype)
    cent = torch.randn(bh, k, dims, generator=g) * 2
    labels = torch.randint(k, (bh, n), generator=g, dtype=torch.int32)
    # A constant-residual token (scale falls back to 1) and a token equal to its centroid.
    x[0, 0] = (cent[0, labels[0, 0]] + 0.5).to(dtype)
    cent[1, labels[1, 3]] = x[1, 3].float()
    announce(f"{dtype} bits={bits} D={dims}")
    enc = quantization.quantize_base_offset(x.to(DEV), labels.to(DEV), cent.to(DEV), bits)
    codes, low, scale, xhat = canonical.base_offset(x.float().numpy(), labels.numpy(), cent.numpy(), bits)
    assert np.array_equal(enc.codes.cpu().numpy(), codes)
    assert np.array_equal(enc.offset_min.cpu().numpy()[..., 0].view(np.int32), low.view(np.int32))
    assert np.array_equal(enc.scale.cpu().numpy()[..., 0].view(np.int32), scale.view(np.int32))
    ref_hat = torch.from_numpy(xhat).to(dtype)
    assert _bits_equal(enc.dequantize().cpu(), ref_hat)
    fq = quantization.fake_quantize_base_offset(x.to(DEV), labels.to(DEV), cent.to(DEV), bits)
    assert _bits_equal(fq.cpu(), ref_hat)
    # The torch restatement of the reference gives the same bits.
    assert _bits_equal(reference_path.fake_quantize(x, labels, cent, bits), ref_hat)


@pytest.mark.parametrize("bits", [4, 8])
@pytest.mark.parametrize("dims", [128, 64])
def test_base_offset_half_integer_quotients(announce, bits, dims):
    """Residual/scale quotients exactly on a half-integer (round half to even decides) and one
    ulp either side of it, where a reciprocal-based quotient could round the other way."""
    g = _gen(bits + dims + 1)
    bh, n = 2, 256
    levels = (1 << bits) - 1
    lo = (torch.randint(-64, 64, (bh, n, 1), generator=g).float() / 8)
    s = 2.0 ** torch.randint(-6, 3, (bh, n, 1), generator=g).float()       # exact scale: span / levels
    k = torch.randint(0, levels, (bh, n, dims), generator=g).float()
    x = lo + (k + 0.5) * s                                                  # quotient k + 0.5 exactly
    nudge = torch.randint(-1, 2, (bh, n, dims), generator=g)               # -1, 0, +1 ulp
    x = torch.where(nudge == 0, x, torch.nextafter(x, x + nudge.float() * torch.inf))
    x[..., 0:1] = lo                                                        # row minimum
    x[..., 1:2] = lo + levels * s                                           # row maximum (span = levels * s)
    cent = torch.zeros(bh, 1, dims)
    labels = torch.zeros(bh, n, dtype=torch.int32)
    announce(f"bits={bits} D={dims}")
    enc = quantization.quantize_base_offset(x.to(DEV), labels.to(DEV), cent.to(DEV), bits)
    codes, low, scale, xhat = canonical.base_offset(x.numpy(), labels.numpy(), cent.numpy(), bits)
    assert np.array_equal(enc.codes.cpu().numpy(), codes)
    assert np.array_equal(enc.scale.cpu().numpy()[..., 0].view(np.int32), scale.view(np.int32))
    assert _bits_equal(enc.dequantize().cpu(), torch.from_numpy(xhat))
    # Ties really occur (codes at both neighbours of a half-integer).
    assert (torch.from_numpy(codes.astype(np.int64)) % 2 == 0).any() and (torch.from_numpy(codes.astype(np.int64)) % 2 == 1).any()


@pytest.mark.parametrize("bits", [0, 4])
def test_pack_matches_quant_gather_concat(announce, bits):
    g = _gen(bits + 100)
    h, n, t, d, kq, kk = 3, 900, 40, 128, 12, 30
    q = _mixture(g, h, n + t, d, 6).to(torch.bfloat16)[None]
    k = _mixture(g, h, n + t, d, 6).to(torch.bfloat16)[None]
    v = torch.randn(1, h, n + t, d, generator=g).to(torch.bfloat16)
    ql = torch.randint(kq, (h, n), generator=g, dtype=torch.int32)
    kl = torch.randint(kk, (h, n), generator=g, dtype=torch.int32)
    qc = torch.randn(h, kq, d, generator=g)
    kc = torch.randn(h, kk, d, generator=g)
    qi = reference_path.stable_indices(ql)
    ki = reference_path.stable_indices(kl)
    announce(f"bits={bits}")
    outs = clustering_cuda.pack_clustered(
        [q.to(DEV), k.to(DEV), v.to(DEV)], [qi.to(DEV), ki.to(DEV), ki.to(DEV)], [ql.to(DEV), kl.to(DEV), None],
        [qc.to(DEV), kc.to(DEV), None], [bits, bits, 0], n)
    for out, x, lab, cent, idx in ((outs[0], q, ql, qc, qi), (outs[1], k, kl, kc, ki), (outs[2], v, None, None, ki)):
        video = x[:, :, :n]
        if lab is not None:
            video = reference_path.fake_quantize(video, lab, cent, bits).reshape(video.shape)
        ref = torch.cat((reference_path.gather_tokens(video, idx), x[:, :, n:]), 2)
        assert _bits_equal(out.cpu(), ref)


# ---------------------------------------------------------------- stage 1: k-means

def _centres_with_duplicates(g, x, k):
    bh, n, d = x.shape
    idx = torch.randint(n, (bh, k), generator=g)
    idx[:, 1] = idx[:, 0]  # guaranteed duplicate centre -> exact tie, lowest id wins
    return x.float().gather(1, idx[..., None].expand(-1, -1, d)).contiguous()


@pytest.mark.parametrize("dims", [128, 64])
@pytest.mark.parametrize("k", [1, 32, 100, 256])
def test_assign_lockstep_fp32(announce, dims, k):
    g = _gen(k + dims)
    x = _mixture(g, 2, 2048, dims, 16)
    c = _centres_with_duplicates(g, x, k) if k > 1 else x[:, :1].contiguous()
    announce(f"D={dims} K={k}")
    labels = torch.empty(2, 2048, dtype=torch.int32, device=DEV)
    norms = torch.empty(2, k, device=DEV)
    clustering_cuda.assign_tokens_to_centers(x.to(DEV), c.to(DEV), labels, torch.empty(1, device=DEV), norms, 1024)
    ref_norms = canonical.center_norms(c.numpy())
    ref = canonical.assign(x.numpy(), c.numpy(), ref_norms)
    assert np.array_equal(norms.cpu().numpy().view(np.int32), ref_norms.view(np.int32))
    assert np.array_equal(labels.cpu().numpy(), ref)


@pytest.mark.parametrize("dims", [128, 64])
def test_update_lockstep_fp32(announce, dims):
    g = _gen(dims + 5)
    x = _mixture(g, 3, 3000, dims, 10)
    k = 40
    labels = torch.randint(k - 3, (3, 3000), generator=g, dtype=torch.int32)  # last 3 clusters empty
    prev = torch.randn(3, k, dims, generator=g)
    announce(f"D={dims}")
    sums = torch.empty(3, k, dims, device=DEV)
    counts = torch.empty(3, k, dtype=torch.int32, device=DEV)
    means = torch.empty(3, k, dims, device=DEV)
    clustering_cuda.recompute_cluster_centers(x.to(DEV), labels.to(DEV), prev.to(DEV), sums, counts, means)
    rs, rc, rm = canonical.update(x.numpy(), labels.numpy(), prev.numpy())
    assert np.array_equal(counts.cpu().numpy(), rc)
    assert np.array_equal(sums.cpu().numpy().view(np.int32), rs.view(np.int32))
    assert np.array_equal(means.cpu().numpy().view(np.int32), rm.view(np.int32))


@pytest.mark.parametrize("dtype,dims,n,kq,kk,iters", [
    (torch.float32, 128, 2048, 32, 32, 10),
    (torch.bfloat16, 128, 6750, 64, 256, 10),
    (torch.float16, 64, 3000, 20, 50, 6),
    # Sort paths: one fused scan+place launch needs <= 32 tiles of 256 tokens and <= 1024
    # clusters in every problem; otherwise separate scan and place launches run.
    (torch.bfloat16, 64, 8192, 24, 96, 4),     # fused, exactly 32 tiles
    (torch.bfloat16, 64, 4000, 10, 1000, 3),   # fused, clusters span four 256-thread passes
    (torch.bfloat16, 64, 9000, 16, 40, 4),     # 36 tiles: scan + place
    (torch.bfloat16, 64, 5000, 16, 1100, 3),   # 1100 clusters: scan + place
    (torch.bfloat16, 128, 6000, 24, 600, 4),   # D = 128 with 600 centres, duplicated ones among them
])
def test_fused_fit_bit_exact(announce, dtype, dims, n, kq, kk, iters):
    g = _gen(n + kq)
    bh = 2
    q = _mixture(g, bh, n, dims, 32, 1.5).to(dtype)
    k = _mixture(g, bh, n, dims, 64, 1.5).to(dtype)
    qi = _centres_with_duplicates(g, q, kq)
    ki = _centres_with_duplicates(g, k, kk)
    announce(f"{dtype} D={dims} N={n} KQ={kq} KK={kk} iters={iters}")
    (ql, qc, qn, qidx, qoff), (kl, kc, kn, kidx, koff) = clustering_cuda.kmeans_fit(
        [clustering_cuda.KMeansProblem(q.to(DEV), qi.to(DEV)), clustering_cuda.KMeansProblem(k.to(DEV), ki.to(DEV))],
        iters)
    for (lab, cen, cnt, idx, off), x, init in (((ql, qc, qn, qidx, qoff), q, qi), ((kl, kc, kn, kidx, koff), k, ki)):
        rl, rc, rn, ridx, roff = canonical.kmeans_fit(x.float().numpy(), init.numpy(), iters)
        assert np.array_equal(lab.cpu().numpy(), rl)
        assert np.array_equal(cnt.cpu().numpy(), rn)
        assert np.array_equal(cen.cpu().numpy().view(np.int32), rc.view(np.int32))
        assert np.array_equal(idx.cpu().numpy(), ridx)
        assert np.array_equal(off.cpu().numpy(), roff)


def _near_degenerate_centres(g, k, dims, rel):
    """k centres within ~rel (relative) of one point, plus a few well-separated ones."""
    base = torch.randn(1, dims, generator=g) * 3
    cent = base + rel * base.norm() * torch.randn(k, dims, generator=g) / dims ** 0.5
    cent[-4:] = torch.randn(4, dims, generator=g) * 6
    return cent


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("dims,k", [(128, 64), (64, 100)])
def test_assign_saturated_candidate_lists(announce, dtype, dims, k):
    """Centres closer together than the screen's error bound: every token near them is
    flagged with a saturated candidate list and takes the all-centre canonical fallback."""
    g = _gen(dims + k)
    cent = torch.stack([_near_degenerate_centres(g, k, dims, 1e-6) for _ in range(2)])
    x = (cent[:, :1] + torch.randn(2, 1500, dims, generator=g) * 2).to(dtype)
    announce(f"{dtype} D={dims} K={k}")
    if dtype == torch.float32:
        labels = torch.empty(2, 1500, dtype=torch.int32, device=DEV)
        norms = torch.empty(2, k, device=DEV)
        clustering_cuda.assign_tokens_to_centers(x.to(DEV), cent.to(DEV), labels, torch.empty(1, device=DEV), norms,
                                                 1024)
    else:
        labels = clustering_cuda.kmeans_fit([clustering_cuda.KMeansProblem(x.to(DEV), cent.to(DEV))], 1)[0][0]
    ref = canonical.assign(x.float().numpy(), cent.numpy(), canonical.center_norms(cent.numpy()))
    # The near-degenerate group really competes: most tokens pick one of its centres.
    assert (ref < k - 4).mean() > 0.5
    assert np.array_equal(labels.cpu().numpy(), ref)


def test_fit_token_clusters_api(announce):
    g = _gen(77)
    x = _mixture(g, 2, 1000, 128, 8).to(torch.bfloat16)
    init = _centres_with_duplicates(g, x, 16)
    announce()
    labels, centers, counts, it = clustering.fit_token_clusters(x.to(DEV), 16, max_iters=5, tol=0,
                                                                 init_centroids=init.to(DEV))
    rl, rc, rn, _, _ = canonical.kmeans_fit(x.float().numpy(), init.numpy(), 5)
    assert it == 5
    assert np.array_equal(labels.cpu().numpy(), rl)
    assert np.array_equal(centers.cpu().numpy().view(np.int32), rc.view(np.int32))
    # tol>0: stops once the centres stop moving; result is still a fixed point of the oracle.
    labels2, centers2, counts2, it2 = clustering.fit_token_clusters(x.to(DEV), 16, max_iters=100, tol=1e-6,
                                                                    init_centroids=init.to(DEV))
    rl2, rc2, _, _, _ = canonical.kmeans_fit(x.float().numpy(), init.numpy(), it2)
    assert np.array_equal(labels2.cpu().numpy(), rl2)
    assert np.array_equal(centers2.cpu().numpy().view(np.int32), rc2.view(np.int32))


# ---------------------------------------------------------------- stage 4: sparse attention

def _random_partition(g, n, c, empty=0):
    cuts = torch.sort(torch.randint(n + 1, (c - 1,), generator=g)).values
    sizes = torch.diff(torch.cat([torch.tensor([0]), cuts, torch.tensor([n])]))
    if empty:
        sizes[:empty] = 0
        sizes[-1] += n - sizes.sum()
    return sizes.to(torch.int32)


def _check_attention(out, ref):
    err = (out.float().cpu() - torch.from_numpy(ref)).abs()
    assert err.max().item() <= 2e-2, f"max abs error {err.max().item():.3e}"
    assert err.mean().item() <= 2e-3, f"mean abs error {err.mean().item():.3e}"


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("dims", [128, 64])
@pytest.mark.parametrize("density", [0.3, 1.0])
def test_sparse_attention_matches_oracle(announce, dtype, dims, density):
    g = _gen(int(density * 10) + dims)
    h, sq, sk, cq, ck = 3, 1100, 1300, 9, 23
    q = torch.randn(1, h, sq, dims, generator=g).to(dtype)
    k = torch.randn(1, h, sk, dims, generator=g).to(dtype)
    v = torch.randn(1, h, sk, dims, generator=g).to(dtype)
    qs = torch.stack([_random_partition(g, sq, cq, empty=1) for _ in range(h)])[None]
    ks = torch.stack([_random_partition(g, sk, ck, empty=2) for _ in range(h)])[None]
    m = torch.rand(1, h, cq, ck, generator=g) < density
    m[0, 0, 2] = False  # one fully masked query cluster -> zero rows
    announce(f"{dtype} D={dims} density={density}")
    out = attention_cuda.sparse_attention(q.to(DEV), k.to(DEV), v.to(DEV), m.to(DEV), qs.to(DEV), ks.to(DEV))
    ref = canonical.sparse_attention(q[0].float().numpy(), k[0].float().numpy(), v[0].float().numpy(),
                                     m[0].numpy(), qs[0].numpy(), ks[0].numpy())
    _check_attention(out[0], ref)
    off = int(qs[0, 0, :2].sum())
    rows = int(qs[0, 0, 2])
    assert torch.all(out[0, 0, off:off + rows].float() == 0)


def test_sparse_attention_dense_equals_sdpa(announce):
    g = _gen(5)
    q = torch.randn(1, 2, 700, 128, generator=g).to(torch.bfloat16)
    k = torch.randn(1, 2, 900, 128, generator=g).to(torch.bfloat16)
    v = torch.randn(1, 2, 900, 128, generator=g).to(torch.bfloat16)
    qs = torch.tensor([[[300, 400], [700, 0]]], dtype=torch.int32)
    ks = torch.tensor([[[500, 400], [100, 800]]], dtype=torch.int32)
    m = torch.ones(1, 2, 2, 2, dtype=torch.bool)
    announce()
    out = attention_cuda.sparse_attention(q.to(DEV), k.to(DEV), v.to(DEV), m.to(DEV), qs.to(DEV), ks.to(DEV))
    ref = torch.nn.functional.scaled_dot_product_attention(q.double(), k.double(), v.double())
    err = (out.cpu().double() - ref).abs()
    assert err.max().item() <= 2e-2 and err.mean().item() <= 2e-3


def test_sparse_attention_out_index_scatter(announce):
    g = _gen(9)
    h, s, d = 2, 600, 128
    q = torch.randn(1, h, s, d, generator=g).to(torch.bfloat16)
    k = torch.randn(1, h, s, d, generator=g).to(torch.bfloat16)
    v = torch.randn(1, h, s, d, generator=g).to(torch.bfloat16)
    qs = torch.tensor([[[200, 400], [100, 500]]], dtype=torch.int32)
    ks = torch.tensor([[[300, 300], [350, 250]]], dtype=torch.int32)
    m = torch.tensor([[[[True, False], [True, True]], [[False, True], [True, False]]]])
    perm = torch.stack([torch.randperm(s, generator=g) for _ in range(h)]).to(torch.int32)
    announce()
    args = [t.to(DEV) for t in (q, k, v, m, qs, ks)]
    plain = attention_cuda.sparse_attention(*args)
    fused = attention_cuda.sparse_attention(*args, out_index=perm.to(DEV))
    restored = clustering.restore_sequence_order(plain, perm.to(DEV))
    assert torch.equal(fused.cpu().view(torch.int16), restored.cpu().view(torch.int16))
    # kept_keys only orders the work items (here against their true costs), so the result is
    # the same bit for bit, with and without out_index.
    kept = torch.tensor([[[1, 2], [300, 0]]], dtype=torch.int32).to(DEV)
    ordered = attention_cuda.sparse_attention(*args, out_index=perm.to(DEV), kept_keys=kept)
    assert torch.equal(ordered.cpu().view(torch.int16), fused.cpu().view(torch.int16))
    assert torch.equal(attention_cuda.sparse_attention(*args, kept_keys=kept).cpu().view(torch.int16),
                       plain.cpu().view(torch.int16))


def _gather_rows(x, index):
    """x [1,H,S,D] with rows j < R of head h replaced by rows index[h, j]."""
    out = x.clone()
    rows = index.shape[1]
    out[0, :, :rows] = x[0].gather(1, index.long()[..., None].expand(-1, -1, x.shape[-1]))
    return out


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("dims", [128, 64])
@pytest.mark.parametrize("sq,sk,rows", [(1000, 1000, 900), (700, 1100, 650), (300, 300, 300), (260, 260, 0)])
def test_sparse_attention_indexed_equals_packed(announce, dtype, dims, sq, sk, rows):
    """Reading Q/K/V through the sort permutations gives the packed path's output bit for bit."""
    g = _gen(sq + rows + dims)
    h, cq, ck = 3, 7, 11
    q = torch.randn(1, h, sq, dims, generator=g).to(dtype)
    k = torch.randn(1, h, sk, dims, generator=g).to(dtype)
    v = torch.randn(1, h, sk, dims, generator=g).to(dtype)
    qs = torch.stack([_random_partition(g, sq, cq, empty=1) for _ in range(h)])[None]
    ks = torch.stack([_random_partition(g, sk, ck, empty=2) for _ in range(h)])[None]
    m = torch.rand(1, h, cq, ck, generator=g) < 0.4
    m[0, 1, 3] = False  # a fully masked query cluster
    qi = torch.stack([torch.randperm(rows, generator=g) for _ in range(h)]).to(torch.int32)
    ki = torch.stack([torch.randperm(rows, generator=g) for _ in range(h)]).to(torch.int32)
    announce(f"{dtype} D={dims} sq={sq} sk={sk} rows={rows}")
    dev = [t.to(DEV) for t in (q, k, v, m, qs, ks, qi, ki)]
    indexed = attention_cuda.sparse_attention_indexed(*dev[:6], dev[6], dev[7], rows)
    packed = attention_cuda.sparse_attention(_gather_rows(dev[0], dev[6]), _gather_rows(dev[1], dev[7]),
                                             _gather_rows(dev[2], dev[7]), *dev[3:6], out_index=dev[6],
                                             out_index_rows=rows)
    assert torch.equal(indexed.cpu().view(torch.int16), packed.cpu().view(torch.int16))
    # Kept-key counts only order the work items: any counts give the same bits.
    kept = torch.randint(0, 5000, (1, h, cq), generator=g, dtype=torch.int32)
    ordered = attention_cuda.sparse_attention_indexed(*dev[:6], dev[6], dev[7], rows, kept_keys=kept.to(DEV))
    assert torch.equal(ordered.cpu().view(torch.int16), indexed.cpu().view(torch.int16))
    # And against the oracle on the packed inputs, restored to original order.
    pq, pk, pv = (_gather_rows(x, i)[0].float().numpy() for x, i in ((q, qi), (k, ki), (v, ki)))
    ref = canonical.sparse_attention(pq, pk, pv, m[0].numpy(), qs[0].numpy(), ks[0].numpy())
    restored = np.array(ref)
    for head in range(h):
        restored[head, qi[head].long().numpy()] = ref[head, :rows]
    _check_attention(indexed[0], restored)


# ---------------------------------------------------------------- selection + text partition

@pytest.mark.parametrize("p,ratio", [(1e-9, 0.25), (0.5, 0.0), (0.9, 0.1), (1.0, 0.0), (0.0, 0.0)])
@pytest.mark.parametrize("dims,ck", [(128, 70), (64, 70), (128, 256), (128, 1000), (64, 2048), (192, 300)])
def test_select_connections_matches_oracle(announce, p, ratio, dims, ck):
    g = _gen(int(p * 100) + dims + ck)
    b, h, cq = 1, 3, 20
    qc = torch.randn(b, h, cq, dims, generator=g) * 0.5
    kc = torch.randn(b, h, ck, dims, generator=g) * 0.5
    qs = torch.randint(0, 40, (b, h, cq), generator=g, dtype=torch.int32)
    ks = torch.randint(0, 40, (b, h, ck), generator=g, dtype=torch.int32)
    qs[0, 0, :3] = 0
    ks[0, 1, :5] = 0
    announce(f"p={p} ratio={ratio} D={dims} CK={ck}")
    m = clustering.select_cluster_connections(qc.to(DEV), kc.to(DEV), qs.to(DEV), ks.to(DEV), p, ratio)
    ref = reference_path.select_connections(qc, kc, qs, ks, p, ratio)
    assert torch.equal(m.cpu(), ref)


def test_select_with_text_partition_matches_oracle(announce):
    g = _gen(31)
    qc = torch.randn(1, 2, 16, 128, generator=g)
    kc = torch.randn(1, 2, 40, 128, generator=g)
    qs = torch.randint(1, 30, (1, 2, 16), generator=g, dtype=torch.int32)
    ks = torch.randint(0, 30, (1, 2, 40), generator=g, dtype=torch.int32)
    announce()
    m, eq, ek, kept = clustering_cuda.select_connections(qc.to(DEV), kc.to(DEV), qs.to(DEV), ks.to(DEV), 1e-9, 10,
                                                         text=(7, 9), with_kept=True)
    rm, rq, rk = reference_path.extend_text_partition(
        reference_path.select_connections(qc, kc, qs, ks, 1e-9, 0.25), qs, ks, 7, 9)
    assert torch.equal(m.cpu(), rm) and torch.equal(eq.cpu(), rq) and torch.equal(ek.cpu(), rk)
    # Kept key rows of every (extended) map row: the sizes of its kept columns.
    ref_kept = (rm.to(torch.int64) * rk[:, :, None, :].to(torch.int64)).sum(-1).to(torch.int32)
    assert torch.equal(kept.cpu(), ref_kept)


def _threshold_case(m, rows=4, ck=64, dims=128, seed=0):
    """Centroids whose count-weighted probabilities are exactly fl(1/m) for m keys of each
    row and 0 for the others: integer entries make every score exact in any summation order,
    unit counts make the log-count term 0, and the other keys score 226 lower, so their exp
    is exactly 0. Each row is its own head (one query cluster, ck key clusters), with its m
    keys at random positions."""
    g = _gen(seed)
    kc = torch.zeros(1, rows, ck, dims)
    for r in range(rows):
        kc[0, r, torch.randperm(ck, generator=g)[:m]] = 20.0
    qc = torch.ones(1, rows, 1, dims)
    qs = torch.ones(1, rows, 1, dtype=torch.int32)
    ks = torch.ones(1, rows, ck, dtype=torch.int32)
    return qc, kc, qs, ks


@pytest.mark.parametrize("m", [3, 7, 10, 20])
def test_select_near_threshold_matches_oracle(announce, m):
    """Keep decisions where a prefix sum lands within an ulp of top_p. The selection follows
    torch's CPU semantics (the oracle): cumsum accumulated in double and rounded per element,
    `before` = fl(cumsum) - prob in fp32, compared against fp32(top_p). Thresholds are the
    default 0.9, every `before` value of the row, and their fp32 neighbours."""
    qc, kc, qs, ks = _threshold_case(m, seed=m)
    prob = np.float32(1.0) / np.float32(m)
    befores = (np.cumsum(np.full(m, prob, np.float64)).astype(np.float32) - prob).astype(np.float32)
    ps = {0.9}
    for b in befores[1:]:
        for v in (b, np.nextafter(b, np.float32(1)), np.nextafter(b, np.float32(0))):
            if 0 < v <= 1:
                ps.add(float(v))
    announce(f"m={m} thresholds={len(ps)}")
    kept_counts = set()
    for p in sorted(ps):
        got = clustering.select_cluster_connections(qc.to(DEV), kc.to(DEV), qs.to(DEV), ks.to(DEV), p, 0.0).cpu()
        ref = reference_path.select_connections(qc, kc, qs, ks, p, 0.0)
        assert torch.equal(got, ref), f"p={p!r}"
        kept_counts.add(int(ref[0, 0, 0].sum()))
    # The thresholds straddle every crossing: each prefix length 1..m occurs.
    assert kept_counts == set(range(1, m + 1))


# ---------------------------------------------------------------- the assign screen's error model

@pytest.mark.parametrize("name", ["hunyuan_480p", "hunyuan_720p"])
def test_assign_screen_error_within_certification_bound(announce, name):
    """The certified assignment accepts a screened argmin only when its margin exceeds twice
    an a-priori bound E = kappa |x||c| + gamma |c|^2 on |screened - canonical|, which assumes
    the MFMA forms exact products and rounds its fp32 accumulation no worse than fp32 adds.
    AMD does not document gfx950's MFMA accumulation, so this measures the realised screen
    error against exact float64 distances on the k-means shapes of the 480p and 720p layers
    (two heads; K and Q with their cluster counts), and requires it to stay below half of
    kappa |x||c| + gamma |c|^2 (the canonical fp32 chain has its own share of the bound)."""
    lib = _native.library()
    wl = workloads.make_workload(name, heads=2, video=8192)
    n = wl.shape.video
    kappa, gamma = ctypes.c_float(), ctypes.c_float()
    lib.peco_kmeans_screen_bound(128, ctypes.byref(kappa), ctypes.byref(gamma))
    worst = 0.0
    for label, x, init in (("K", wl.key, wl.k_init), ("Q", wl.query, wl.q_init)):
        xv = x[0, :, :n].contiguous()  # bf16 [2, n, 128]
        c = init.contiguous()          # fp32 [2, K, 128]
        b, k = c.shape[0], c.shape[1]
        announce(f"{name} {label}: B={b} N={n} K={k}")
        xg, cg = xv.to(DEV), c.to(DEV)
        norms = torch.empty(b, k, device=DEV)
        labels = torch.empty(b, n, dtype=torch.int32, device=DEV)
        screened = torch.empty(b, n, k, device=DEV)
        status = lib.peco_kmeans_screen(_native.ptr(xg), 1, _native.ptr(cg), _native.ptr(norms), _native.ptr(labels),
                                        _native.ptr(screened), b, n, 128, k, None)
        assert status == 0
        torch.cuda.synchronize()
        x64, c64 = xv.double(), c.double()
        exact = (c64 * c64).sum(-1)[:, None, :] - 2.0 * torch.bmm(x64, c64.transpose(1, 2))
        err = (screened.cpu().double() - exact).abs()
        xn = x64.norm(dim=-1)[:, :, None]
        cn = c64.norm(dim=-1)[:, None, :]
        bound = kappa.value * xn * cn + gamma.value * cn * cn
        ratio = (err / bound).max().item()
        rel = (err / (xn * cn)).max().item()
        worst = max(worst, ratio)
        print(f"[screen] {name} {label}: max |screened - exact| / (|x||c|) = {rel:.3e} "
              f"(kappa {kappa.value:.3e}); max error / bound = {ratio:.4f}", flush=True)
        # The labels of this assignment are the canonical ones.
        ref = canonical.assign(xv.float().numpy(), c.numpy())
        assert np.array_equal(labels.cpu().numpy(), ref)
    assert worst < 0.5
