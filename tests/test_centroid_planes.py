"""The key-centroid planes of the integer-score attention (attention_cuda.centroid_planes).

The kernel computes u.Ck as cs * (u.P0 + u.P1/128 + u.P2/16384) on the integer MFMA, so the
planes must reconstruct every centroid to within 2^-21 of its largest magnitude (the last
plane's half step is 2^-22, the fp32 rounding of C / cs adds about 2^-24), stay inside
int8, and keep a zero centroid exact. Host-side torch code: checked here on the CPU against a
float64 reconstruction and a float64 dot product with 8-bit codes.
"""
import torch

from peco_amd.attention_cuda import centroid_planes


def _centroids(seed):
    g = torch.Generator()
    g.manual_seed(seed)
    c = torch.randn(3, 40, 128, generator=g) * torch.logspace(-3, 3, 40)[None, :, None]
    c[0, 0] = 0.0                        # a zero centroid
    c[1, 1] = 1.0                        # all channels equal
    c[2, 2, 5] = -7.5e3                  # one dominant channel
    return c


def test_planes_reconstruct_each_centroid():
    c = _centroids(0)
    planes, cs, sums = centroid_planes(c)
    assert planes.dtype == torch.int8 and planes.shape == (3, 40, 3, 128)
    assert cs.shape == (3, 40) and bool((cs > 0).all())
    assert int(planes.abs().max()) <= 127
    p = planes.double()
    rec = cs.double()[..., None] * (p[:, :, 0] + p[:, :, 1] / 128 + p[:, :, 2] / 16384)
    err = (rec - c.double()).abs().amax(dim=-1)
    bound = c.double().abs().amax(dim=-1) * 2.0 ** -21
    assert bool((err <= bound).all()), float((err / bound.clamp_min(1e-300)).max())
    assert bool((rec[0, 0] == 0).all())
    assert torch.allclose(sums.double(), c.double().sum(-1), rtol=1e-6, atol=1e-6 * c.abs().sum(-1).max().item())


def test_plane_dot_products_match_the_centroid_dot_products():
    """u.Ck for 8-bit codes u, as the kernel forms it from the planes (integer dot products,
    then the scale), against the float64 product with the centroid itself."""
    c = _centroids(1)
    planes, cs, _ = centroid_planes(c)
    g = torch.Generator()
    g.manual_seed(2)
    u = torch.randint(0, 256, (3, 7, 128), generator=g)
    ints = torch.einsum("bqd,bkpd->bqkp", u.long(), planes.long())      # exact integers
    approx = cs.double()[:, None, :] * (ints[..., 0] + ints[..., 1] / 128.0 + ints[..., 2] / 16384.0).double()
    exact = torch.einsum("bqd,bkd->bqk", u.double(), c.double())
    scale = u.double().abs().sum(-1)[..., None] * c.double().abs().amax(-1)[:, None, :]
    assert bool(((approx - exact).abs() <= scale * 2.0 ** -21).all())
