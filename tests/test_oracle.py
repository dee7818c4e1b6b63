"""Pins of the CPU oracle (no GPU): every oracle function is checked against something
independent of its own formula -- float64 brute force, torch library routines, closed
forms and special cases -- chosen so that a plausible slip (sign, dropped term, wrong
tie rule, wrong rounding, transposed operand) fails at least one test.
"""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import canonical, reference_path

U32 = 2.0 ** -24


def _rng(seed):
    return np.random.default_rng(seed)


def _gamma(n):
    return n * U32 / (1 - n * U32)


# ------------------------------------------------------------------ k-means assignment

def _brute_force(x, c):
    d = ((x[:, :, None, :].astype(np.float64) - c[:, None, :, :].astype(np.float64)) ** 2).sum(-1)
    return d


def test_assign_matches_float64_brute_force():
    rng = _rng(0)
    x = rng.normal(size=(3, 400, 32)).astype(np.float32)
    c = rng.normal(size=(3, 17, 32)).astype(np.float32)
    labels, best, second = canonical.assign(x, c, margins=True)
    d = _brute_force(x, c)
    ref = d.argmin(-1)
    srt = np.sort(d, -1)
    margin = srt[..., 1] - srt[..., 0]
    # Canonical fp32 distance error <= 2*gamma_D*|x||c| + 2u|D|; decide only clear cases.
    bound = 4 * _gamma(32) * np.linalg.norm(x, axis=-1)[..., None] * np.linalg.norm(c, axis=-1).max() + 1e-3
    clear = margin > bound[..., 0]
    assert clear.mean() > 0.99
    assert np.array_equal(labels[clear], ref[clear])
    # The reported best distance is the float64 one shifted by |x|^2 (rank-invariant term).
    shifted = d.min(-1) - (x.astype(np.float64) ** 2).sum(-1)
    assert np.allclose(best, shifted, rtol=1e-5, atol=1e-3)


def test_assign_ties_choose_lowest_id():
    rng = _rng(1)
    x = rng.normal(size=(2, 200, 16)).astype(np.float32)
    c = rng.normal(size=(2, 9, 16)).astype(np.float32)
    c[:, 5] = c[:, 2]
    c[:, 7] = c[:, 2]
    labels, best, second = canonical.assign(x, c, margins=True)
    assert not np.isin(labels, [5, 7]).any()
    assert (labels == 2).any()
    assert np.all(second[labels == 2] == best[labels == 2])


def test_assign_agrees_with_torch_bmm_except_certified_near_ties():
    """The reference's CPU formula (clustering.py:67-73) computed by torch/MKL."""
    rng = _rng(2)
    x = rng.normal(size=(4, 3000, 128)).astype(np.float32) * 2
    c = x[:, rng.integers(0, 3000, 200)].copy()
    labels, best, second = canonical.assign(x, c, margins=True)
    xt, ct = torch.from_numpy(x), torch.from_numpy(c)
    dist = -2 * torch.bmm(xt, ct.transpose(1, 2)) + ct.square().sum(-1).unsqueeze(1)
    tl = dist.argmin(-1).numpy()
    diff = tl != labels
    bound = 4 * _gamma(128) * np.linalg.norm(x, axis=-1) * np.linalg.norm(c, axis=-1).max() + 4 * U32 * np.abs(best)
    assert np.all((second - best)[diff] <= bound[diff]), "disagreement outside the fp32 near-tie band"
    assert diff.mean() < 1e-3


def test_center_norms_exact_on_integers_and_close_otherwise():
    c = np.arange(2 * 3 * 8, dtype=np.float32).reshape(2, 3, 8) - 20
    assert np.array_equal(canonical.center_norms(c), (c.astype(np.int64) ** 2).sum(-1).astype(np.float32))
    rng = _rng(3)
    c = rng.normal(size=(2, 5, 128)).astype(np.float32)
    n = canonical.center_norms(c)
    exact = (c.astype(np.float64) ** 2).sum(-1)
    assert np.all(np.abs(n - exact) <= 2 * _gamma(128) * exact)


# ------------------------------------------------------------------ k-means update / fit

def test_update_matches_scatter_add_and_closed_form_mean():
    rng = _rng(4)
    x = rng.normal(size=(3, 2500, 64)).astype(np.float32)
    labels = rng.integers(0, 29, size=(3, 2500)).astype(np.int32)  # clusters 29..31 empty
    prev = rng.normal(size=(3, 32, 64)).astype(np.float32)
    sums, counts, means = canonical.update(x, labels, prev)
    xt, lt = torch.from_numpy(x), torch.from_numpy(labels).long()
    ts = torch.zeros(3, 32, 64).scatter_add_(1, lt[..., None].expand(-1, -1, 64), xt)
    tc = torch.zeros(3, 32, dtype=torch.int32).scatter_add_(1, lt, torch.ones_like(lt, dtype=torch.int32))
    assert np.array_equal(sums.view(np.int32), ts.numpy().view(np.int32))
    assert np.array_equal(counts, tc.numpy())
    assert np.array_equal(counts.sum(-1), np.full(3, 2500))
    assert np.array_equal(means[:, 29:], prev[:, 29:])
    for b in range(3):
        for k in (0, 13, 28):
            exact = x[b][labels[b] == k].astype(np.float64).mean(0)
            assert np.allclose(means[b, k], exact, rtol=0, atol=1e-5)


def test_fit_objective_does_not_increase_and_matches_reference_path():
    rng = _rng(5)
    means_ = rng.normal(size=(2, 12, 32)) * 3
    comp = rng.integers(0, 12, size=(2, 1500))
    x = (np.take_along_axis(means_, comp[..., None], 1) + rng.normal(size=(2, 1500, 32))).astype(np.float32)
    init = x[:, rng.integers(0, 1500, 10)].copy()
    prev = None
    for it in range(1, 8):
        labels, centers, counts, idx, off = canonical.kmeans_fit(x, init, it)
        # objective of the assignment made at iteration `it` against the centres it used
        obj = 0.0
        c_used = init if it == 1 else canonical.kmeans_fit(x, init, it - 1)[1]
        d = _brute_force(x, c_used)
        obj = np.take_along_axis(d, labels[..., None].astype(np.int64), -1).sum()
        if prev is not None:
            assert obj <= prev * (1 + 1e-9)
        prev = obj
    tl, tc, tn, _ = reference_path.fit_token_clusters(torch.from_numpy(x), 10, 7, torch.from_numpy(init))
    assert np.array_equal(tl.numpy(), labels)
    assert np.array_equal(tc.numpy().view(np.int32), centers.view(np.int32))
    assert np.array_equal(tn.numpy(), counts)
    assert np.array_equal(idx, torch.argsort(tl, dim=-1, stable=True).numpy())
    assert np.array_equal(off[:, 1:] - off[:, :-1], counts)


# ------------------------------------------------------------------ stable sort

@pytest.mark.parametrize("k", [1, 5, 300])
def test_stable_sort_matches_library_argsort(k):
    rng = _rng(k)
    labels = rng.integers(0, k, size=(3, 4000)).astype(np.int32)
    idx, off = canonical.stable_sort(labels, k)
    assert np.array_equal(idx, np.argsort(labels, axis=-1, kind="stable"))
    assert np.array_equal(idx, torch.argsort(torch.from_numpy(labels), dim=-1, stable=True).numpy())
    assert np.array_equal(off[:, -1], np.full(3, 4000))
    assert np.array_equal(np.diff(off, axis=1), np.stack([np.bincount(r, minlength=k) for r in labels]))


# ------------------------------------------------------------------ Base-Offset quantizer

@pytest.mark.parametrize("bits", [4, 8])
def test_base_offset_matches_torch_ops_bit_exact(bits):
    rng = _rng(bits)
    x = rng.normal(size=(2, 700, 128)).astype(np.float32)
    c = rng.normal(size=(2, 9, 128)).astype(np.float32)
    labels = rng.integers(0, 9, size=(2, 700)).astype(np.int32)
    codes, low, scale, xhat = canonical.base_offset(x, labels, c, bits)
    tcodes, tlow, tscale = reference_path.quantize(torch.from_numpy(x), torch.from_numpy(labels),
                                                   torch.from_numpy(c), bits)
    assert np.array_equal(codes, tcodes.numpy())
    assert np.array_equal(low.view(np.int32), tlow.numpy()[..., 0].view(np.int32))
    assert np.array_equal(scale.view(np.int32), tscale.numpy()[..., 0].view(np.int32))
    th = reference_path.dequantize(tcodes, tlow, tscale, torch.from_numpy(labels), torch.from_numpy(c),
                                   torch.float32, (2, 700, 128))
    assert np.array_equal(xhat.view(np.int32), th.numpy().view(np.int32))
    # Reconstruction error is at most half a step (plus fp32 rounding of the three adds).
    base = np.take_along_axis(c, labels[..., None].astype(np.int64), 1)
    step = scale[..., None]
    assert np.all(np.abs(xhat - x) <= step / 2 + 4 * np.finfo(np.float32).eps * (np.abs(x) + np.abs(base) + step * 15))
    assert codes.max() <= (1 << bits) - 1


def test_base_offset_constant_residual_and_half_even():
    c = np.zeros((1, 1, 8), np.float32)
    x = np.full((1, 2, 8), 3.0, np.float32)
    # token 1: residuals 0..15 with exact halves -> ties go to even codes
    x[0, 1] = [0.0, 15.0, 0.5, 1.5, 2.5, 3.5, 14.5, 7.0]
    labels = np.zeros((1, 2), np.int32)
    codes, low, scale, xhat = canonical.base_offset(x, labels, c, 4)
    assert scale[0, 0] == 1.0 and low[0, 0] == 3.0
    assert np.all(codes[0, 0] == 0) and np.all(xhat[0, 0] == 3.0)
    assert scale[0, 1] == 1.0 and low[0, 1] == 0.0
    assert codes[0, 1].tolist() == [0, 15, 0, 2, 2, 4, 14, 7]


# ------------------------------------------------------------------ sparse attention

def _sizes(rng, n, c):
    cuts = np.sort(rng.integers(0, n + 1, c - 1))
    return np.diff(np.concatenate([[0], cuts, [n]])).astype(np.int32)


def test_sparse_attention_all_true_equals_sdpa():
    rng = _rng(10)
    q = rng.normal(size=(2, 150, 64)).astype(np.float32)
    k = rng.normal(size=(2, 170, 64)).astype(np.float32)
    v = rng.normal(size=(2, 170, 64)).astype(np.float32)
    qs = np.stack([_sizes(rng, 150, 4) for _ in range(2)])
    ks = np.stack([_sizes(rng, 170, 5) for _ in range(2)])
    m = np.ones((2, 4, 5), bool)
    out = canonical.sparse_attention(q, k, v, m, qs, ks)
    ref = F.scaled_dot_product_attention(*(torch.from_numpy(t).double() for t in (q, k, v)))
    assert np.allclose(out, ref.numpy(), atol=1e-6)


def test_sparse_attention_block_diagonal_and_masked_rows():
    rng = _rng(11)
    q = rng.normal(size=(1, 90, 32)).astype(np.float32)
    k = rng.normal(size=(1, 90, 32)).astype(np.float32)
    v = rng.normal(size=(1, 90, 32)).astype(np.float32)
    qs = np.array([[30, 20, 40]], np.int32)
    ks = np.array([[25, 35, 30]], np.int32)
    m = np.eye(3, dtype=bool)[None]
    m[0, 1, 1] = False  # query cluster 1 keeps nothing -> zero rows
    out = canonical.sparse_attention(q, k, v, m, qs, ks)
    qo, ko = np.concatenate([[0], np.cumsum(qs[0])]), np.concatenate([[0], np.cumsum(ks[0])])
    for i in (0, 2):
        ref = F.scaled_dot_product_attention(torch.from_numpy(q[:, qo[i]:qo[i + 1]]).double(),
                                             torch.from_numpy(k[:, ko[i]:ko[i + 1]]).double(),
                                             torch.from_numpy(v[:, ko[i]:ko[i + 1]]).double())
        assert np.allclose(out[:, qo[i]:qo[i + 1]], ref.numpy(), atol=1e-6)
    assert np.all(out[:, qo[1]:qo[2]] == 0)


def test_sparse_attention_brute_force_tiny():
    rng = _rng(12)
    q = rng.normal(size=(1, 7, 4)).astype(np.float32)
    k = rng.normal(size=(1, 6, 4)).astype(np.float32)
    v = rng.normal(size=(1, 6, 4)).astype(np.float32)
    qs = np.array([[3, 4]], np.int32)
    ks = np.array([[2, 1, 3]], np.int32)
    m = np.array([[[True, False, True], [False, True, False]]])
    out = canonical.sparse_attention(q, k, v, m, qs, ks)
    kc = [0, 0, 1, 2, 2, 2]
    for r in range(7):
        cq = 0 if r < 3 else 1
        cols = [j for j in range(6) if m[0, cq, kc[j]]]
        s = np.array([q[0, r].astype(np.float64) @ k[0, j] for j in cols]) / 2.0
        p = np.exp(s - s.max())
        p /= p.sum()
        assert np.allclose(out[0, r], p @ v[0, cols].astype(np.float64), atol=1e-6)


def test_reference_path_blockwise_attention_matches_oracle():
    rng = _rng(13)
    q = torch.from_numpy(rng.normal(size=(1, 2, 120, 32)).astype(np.float32))
    k = torch.from_numpy(rng.normal(size=(1, 2, 130, 32)).astype(np.float32))
    v = torch.from_numpy(rng.normal(size=(1, 2, 130, 32)).astype(np.float32))
    qs = torch.from_numpy(np.stack([_sizes(rng, 120, 3) for _ in range(2)]))[None]
    ks = torch.from_numpy(np.stack([_sizes(rng, 130, 4) for _ in range(2)]))[None]
    m = torch.from_numpy(rng.random((1, 2, 3, 4)) < 0.5)
    out = reference_path.sparse_attention(q, k, v, m, qs, ks)
    ref = canonical.sparse_attention(q[0].numpy(), k[0].numpy(), v[0].numpy(), m[0].numpy(), qs[0].numpy(),
                                     ks[0].numpy())
    assert np.allclose(out[0].numpy(), ref, atol=2e-5)


# ------------------------------------------------------------------ selection and text partition

def _centroids(seed, cq=6, ck=10, d=16):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(1, 2, cq, d, generator=g), torch.randn(1, 2, ck, d, generator=g),
            torch.randint(1, 50, (1, 2, cq), generator=g, dtype=torch.int32),
            torch.randint(1, 50, (1, 2, ck), generator=g, dtype=torch.int32))


def test_select_p_one_and_ratio_one_keep_all_nonempty():
    qc, kc, qs, ks = _centroids(0)
    qs[0, 0, 1] = 0
    ks[0, 1, 3] = 0
    for p, r in ((1.0, 0.0), (1e-9, 1.0)):
        m = reference_path.select_connections(qc, kc, qs, ks, p, r)
        expect = (qs[..., :, None] > 0) & (ks[..., None, :] > 0)
        assert torch.equal(m, expect)


def test_select_tiny_p_is_topk_of_count_weighted_scores():
    qc, kc, qs, ks = _centroids(1)
    m = reference_path.select_connections(qc, kc, qs, ks, 1e-9, 0.3)
    logits = (qc @ kc.transpose(-1, -2)) / 4.0 + ks.float().log()[..., None, :]
    top = logits.topk(math.ceil(0.3 * 10), dim=-1).indices
    expect = torch.zeros_like(m).scatter_(-1, top, True)
    assert torch.equal(m, expect)


def test_select_threshold_keeps_the_crossing_cluster():
    # Probabilities proportional to counts when all scores are equal: 0.3, 0.5, 0.2.
    qc = torch.zeros(1, 1, 1, 4)
    kc = torch.zeros(1, 1, 3, 4)
    qs = torch.tensor([[[5]]], dtype=torch.int32)
    ks = torch.tensor([[[30, 50, 20]]], dtype=torch.int32)
    m = reference_path.select_connections(qc, kc, qs, ks, 0.6, 0.0)
    assert m[0, 0, 0].tolist() == [True, True, False]  # mass before cluster 0 is 0.5 < 0.6: kept
    m = reference_path.select_connections(qc, kc, qs, ks, 0.45, 0.0)
    assert m[0, 0, 0].tolist() == [False, True, False]


def test_extend_text_partition_fixture():
    m = torch.tensor([[[[True, False], [False, True]]]])
    qs = torch.tensor([[[3, 4]]], dtype=torch.int32)
    ks = torch.tensor([[[5, 2]]], dtype=torch.int32)
    em, eq, ek = reference_path.extend_text_partition(m, qs, ks, 3, 5)
    expect = torch.tensor([[1, 0, 1, 0], [0, 1, 1, 0], [1, 1, 1, 0], [0, 0, 0, 1]], dtype=torch.bool)
    assert torch.equal(em[0, 0], expect)
    assert eq.tolist() == [[[3, 4, 3, 2]]] and ek.tolist() == [[[5, 2, 3, 2]]]
