"""The fit runs as four chains of launches, three on library streams forked from and joined back
to the caller's stream: by problem (each problem's heads in halves) or, for two problems of at
most 16384 tokens with at least four heads, mixed (each chain a quarter of both problems'
heads). Its results must not depend on the layout, on which stream the caller is on, on calls
queued back to back without a synchronization, or on work the caller queues right after the
call on its own stream."""
import pytest
import torch

from peco_amd import clustering_cuda

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _problems(seed, h=3, n=5000, d=128, kq=16, kk=48):
    g = torch.Generator()
    g.manual_seed(seed)
    out = []
    for k in (kq, kk):
        means = torch.randn(h, 24, d, generator=g) * 3.0
        comp = torch.randint(24, (h, n), generator=g)
        x = (means.gather(1, comp[..., None].expand(-1, -1, d)) + torch.randn(h, n, d, generator=g))
        x = x.to(torch.bfloat16).to(DEV)
        idx = torch.randint(n, (h, k), generator=g).to(DEV)
        init = x.float().gather(1, idx[..., None].expand(-1, -1, d)).contiguous()
        out.append(clustering_cuda.KMeansProblem(x, init))
    return out


def _equal(a, b):
    return all(torch.equal(x, y) for pa, pb in zip(a, b) for x, y in zip(pa, pb))


# Three heads: the by-problem layout; six heads (at most 16384 tokens): the mixed one; 17000
# tokens: by problem again.
LAYOUTS = [(3, 5000), (6, 3000), (4, 17000)]


@pytest.mark.parametrize("h,n", LAYOUTS)
def test_fit_on_a_caller_stream_matches_the_default_stream(announce, h, n):
    announce(f"two-problem fit on a caller stream, consumer on the same stream, H={h} N={n}")
    problems = _problems(1, h=h, n=n)
    ref = clustering_cuda.kmeans_fit(problems, 4)
    torch.cuda.synchronize()
    s = torch.cuda.Stream(device=DEV)
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        out = clustering_cuda.kmeans_fit(problems, 4)
        # Consumers queued on the caller's stream right after the call see finished results.
        total = out[1][2].sum() + out[0][2].sum()
        cent = out[1][1].clone()
    s.synchronize()
    assert _equal(ref, out)
    assert total.item() == 2 * h * n  # every token counted once per problem
    assert torch.equal(cent, ref[1][1])


@pytest.mark.parametrize("h,n", LAYOUTS[:2])
def test_layouts_match_one_problem_fits(announce, h, n):
    """Each problem fitted alone (its heads in halves) equals its part of the two-problem fit."""
    announce(f"two-problem fit against one-problem fits, H={h} N={n}")
    problems = _problems(2, h=h, n=n)
    both = clustering_cuda.kmeans_fit(problems, 3)
    alone = [clustering_cuda.kmeans_fit([p], 3)[0] for p in problems]
    torch.cuda.synchronize()
    assert _equal(both, alone)


def test_fits_queued_back_to_back(announce):
    announce("five two-problem fits queued without synchronization")
    sets = [_problems(10 + i) for i in range(5)]
    refs = []
    for p in sets:
        refs.append(clustering_cuda.kmeans_fit(p, 3))
        torch.cuda.synchronize()
    outs = [clustering_cuda.kmeans_fit(p, 3) for p in sets]
    torch.cuda.synchronize()
    for r, o in zip(refs, outs):
        assert _equal(r, o)
