"""Synthetic PECO attention-layer workloads (Gaussian-mixture Q/K, Gaussian V).

These are the measured configurations of the per-layer hot path:

- ``cpu_small``: 1x4 heads, 2048 video + 64 text tokens, D=128, fp32, 32 mixture
  components (norm 8, sigma 1.0, uniform), KQ=KK=32, 10 iterations, keep 8/32 key
  clusters, Base-Offset off.
- ``hunyuan_480p``: HunyuanVideo 480x720x17f, 1x24 heads, 6750 video + 256 text
  tokens, D=128, bf16, 256 components (sigma 1.5, Dirichlet(1) weights),
  KQ=64, KK=256, 10 iterations, keep 25% of key clusters, Base-Offset off.
- ``hunyuan_480p_bo4``: the same with 4-bit Base-Offset on.
- ``hunyuan_720p``: 720x1280x129f, 118800 video + 256 text tokens, 1024 components,
  KQ=256, KK=1024, 8 iterations, keep 15%, Base-Offset 4-bit.
- ``hunyuan_544p_zipf``: 544x960x61f, 32640 video + 256 text tokens, Zipf(1.2) over
  512 components, KQ=128, KK=512, keep 20%, Base-Offset 4-bit; 10 steps with
  N(0, 0.1^2) drift, warm-started k-means (10 iterations first, then 3).

"Keep top-k" maps onto the reference's selection as a tiny ``top_p`` plus
``min_kc_ratio = k / CK`` (peco/clustering.py:167-181). Initial centroids are video
tokens at seeded random indices drawn with replacement (as peco/clustering.py:48).
All draws use one seeded torch.Generator on the requested device.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import torch

TINY_TOP_P = 1e-9


@dataclass(frozen=True)
class LayerShape:
    name: str
    heads: int
    video: int
    text: int
    dims: int
    dtype: torch.dtype
    components: int
    sigma: float
    weights: str  # "uniform" | "dirichlet" | "zipf"
    num_q_centroids: int
    num_k_centroids: int
    iterations: int
    keep_ratio: float
    bits: int
    steps: int = 1
    warm_iterations: int = 0
    drift: float = 0.0
    zipf_s: float = 1.2

    @property
    def length(self) -> int:
        return self.video + self.text


SHAPES = {
    "cpu_small": LayerShape("cpu_small", 4, 2048, 64, 128, torch.float32, 32, 1.0, "uniform", 32, 32, 10, 0.25, 0),
    "hunyuan_480p": LayerShape("hunyuan_480p", 24, 6750, 256, 128, torch.bfloat16, 256, 1.5, "dirichlet", 64, 256,
                               10, 0.25, 0),
    "hunyuan_480p_bo4": LayerShape("hunyuan_480p_bo4", 24, 6750, 256, 128, torch.bfloat16, 256, 1.5, "dirichlet",
                                   64, 256, 10, 0.25, 4),
    "hunyuan_720p": LayerShape("hunyuan_720p", 24, 118800, 256, 128, torch.bfloat16, 1024, 1.5, "dirichlet", 256,
                               1024, 8, 0.15, 4),
    "hunyuan_544p_zipf": LayerShape("hunyuan_544p_zipf", 24, 32640, 256, 128, torch.bfloat16, 512, 1.5, "zipf", 128,
                                    512, 10, 0.20, 4, steps=10, warm_iterations=3, drift=0.1),
}


@dataclass
class Workload:
    shape: LayerShape
    query: torch.Tensor  # [1,H,S,D]
    key: torch.Tensor
    value: torch.Tensor
    q_init: torch.Tensor  # [H,KQ,D] fp32
    k_init: torch.Tensor  # [H,KK,D] fp32
    extra: dict = field(default_factory=dict)

    @property
    def top_p(self) -> float:
        return TINY_TOP_P

    @property
    def min_kc_ratio(self) -> float:
        return self.shape.keep_ratio


def _weights(gen, heads, m, kind, zipf_s, device):
    if kind == "uniform":
        return torch.ones(heads, m, device=device)
    if kind == "dirichlet":
        # Dirichlet(1) == normalised Exp(1) draws.
        u = torch.rand(heads, m, generator=gen, device=device).clamp_min(1e-12)
        e = -torch.log(u)
        return e / e.sum(-1, keepdim=True)
    if kind == "zipf":
        w = torch.arange(1, m + 1, device=device, dtype=torch.float64).pow(-zipf_s).float()
        return (w / w.sum()).expand(heads, m).contiguous()
    raise ValueError(f"unknown mixture weights {kind!r}")


def _mixture(gen, heads, tokens, dims, m, sigma, weights, device):
    means = torch.randn(heads, m, dims, generator=gen, device=device)
    means = means / means.norm(dim=-1, keepdim=True) * 8.0
    comp = torch.multinomial(weights, tokens, replacement=True, generator=gen)
    x = means.gather(1, comp[..., None].expand(-1, -1, dims))
    return x + sigma * torch.randn(heads, tokens, dims, generator=gen, device=device)


def make_workload(name: str | LayerShape, *, seed: int = 0, device="cpu", heads: int | None = None,
                  video: int | None = None) -> Workload:
    """Draw one layer's inputs. ``heads``/``video`` shrink the shape (for tests)."""
    shape = SHAPES[name] if isinstance(name, str) else name
    if heads is not None or video is not None:
        shape = LayerShape(**{**shape.__dict__, "heads": heads or shape.heads, "video": video or shape.video})
    device = torch.device(device)
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    h, n, t, d = shape.heads, shape.video, shape.text, shape.dims
    s = n + t
    qw = _weights(gen, h, shape.components, shape.weights, shape.zipf_s, device)
    kw = _weights(gen, h, shape.components, shape.weights, shape.zipf_s, device)
    q = _mixture(gen, h, s, d, shape.components, shape.sigma, qw, device)
    k = _mixture(gen, h, s, d, shape.components, shape.sigma, kw, device)
    v = torch.randn(h, s, d, generator=gen, device=device)
    q_idx = torch.randint(n, (h, shape.num_q_centroids), generator=gen, device=device)
    k_idx = torch.randint(n, (h, shape.num_k_centroids), generator=gen, device=device)
    q = q.to(shape.dtype)
    k = k.to(shape.dtype)
    v = v.to(shape.dtype)
    # Initial centroids are the (already cast) video tokens, as x.float().gather(...).
    q_init = q[:, :n].float().gather(1, q_idx[..., None].expand(-1, -1, d)).contiguous()
    k_init = k[:, :n].float().gather(1, k_idx[..., None].expand(-1, -1, d)).contiguous()
    return Workload(shape, q.unsqueeze(0).contiguous(), k.unsqueeze(0).contiguous(), v.unsqueeze(0).contiguous(),
                    q_init, k_init)


def drift(workload: Workload, step: int, seed: int = 0) -> Workload:
    """Next denoising step of a drifting workload: Q/K += N(0, drift^2)."""
    gen = torch.Generator(device=workload.query.device)
    gen.manual_seed(seed * 1000003 + step)
    sd = workload.shape.drift

    def move(x):
        return (x.float() + sd * torch.randn(x.shape, generator=gen, device=x.device)).to(x.dtype)

    return Workload(workload.shape, move(workload.query), move(workload.key), workload.value,
                    workload.q_init, workload.k_init)


def attention_flops(dynamic_map: torch.Tensor, q_sizes: torch.Tensor, k_sizes: torch.Tensor, dims: int) -> float:
    """4*D*sum over kept (i,j) of |Q_i|*|K_j| for an extended map [B,H,CQ,CK]."""
    m = dynamic_map.to(torch.float64)
    qs = q_sizes.to(torch.float64)
    ks = k_sizes.to(torch.float64)
    pairs = torch.einsum("bhij,bhi,bhj->", m, qs, ks)
    return float(4 * dims * pairs.item())
