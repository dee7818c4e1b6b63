"""Cluster-centroid Base-Offset quantization of Q/K (peco/quantization.py interface).

Each token/head has one affine quantizer over its D channels:

    r = x - C[label]
    low = min(r); scale = (max(r) - low) / (2**bits - 1)   (1 when not positive)
    code = clamp(round_half_even((r - low) / scale), 0, 2**bits - 1)
    x_hat = C[label] + (low + scale * code)

computed by HIP kernels in exactly this fp32 order, so codes, low, scale and x_hat are
bit-identical to the reference's torch arithmetic. Codes occupy uint8 containers (not
nibble-packed), as in the reference. Inputs must be GPU tensors.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from . import _native

_DTYPES = {torch.float16: 0, torch.bfloat16: 1, torch.float32: 2}


@dataclass(frozen=True)
class BaseOffsetQuantized:
    """Quantized payload with flattened batch/head axes (peco/quantization.py:33-52).

    ``centroids`` is FP32 [BH,K,D], ``labels`` int64 [BH,N], ``codes`` uint8 [BH,N,D],
    ``offset_min``/``scale`` FP32 [BH,N,1]; ``original_shape`` is [BH,N,D] or [B,H,N,D].
    """

    centroids: torch.Tensor
    labels: torch.Tensor
    codes: torch.Tensor
    offset_min: torch.Tensor
    scale: torch.Tensor
    original_dtype: torch.dtype
    original_shape: tuple[int, ...]
    bits: int

    def dequantize(self) -> torch.Tensor:
        return dequantize_base_offset(self)


def _validate_bits(bits: int, *, allow_bypass: bool) -> None:
    allowed = (0, 4, 8) if allow_bypass else (4, 8)
    if type(bits) is not int or bits not in allowed:
        suffix = "; use fake_quantize_base_offset(..., bits=0) to bypass" if not allow_bypass else ""
        raise ValueError(f"bits must be one of {allowed}{suffix}")


def _flatten_inputs(x, labels, centroids):
    """Checks of peco/quantization.py:62-89; returns (flat x, labels int64, centroids fp32)."""
    if x.ndim not in (3, 4):
        raise ValueError("x must have shape [BH,N,D] or [B,H,N,D]")
    if any(size == 0 for size in x.shape):
        raise ValueError("x dimensions must be nonempty")
    if not x.is_floating_point() or not centroids.is_floating_point():
        raise TypeError("x and centroids must have floating-point dtypes")
    if labels.dtype not in (torch.int32, torch.int64):
        raise TypeError("labels must have dtype int32 or int64")
    if x.device != labels.device or x.device != centroids.device:
        raise ValueError("x, labels and centroids must be on the same device")
    n, d = x.shape[-2:]
    flat = x.reshape(-1, n, d)
    if labels.shape != flat.shape[:2]:
        raise ValueError(f"labels must have shape {tuple(flat.shape[:2])}")
    if centroids.ndim != 3 or centroids.shape[0] != flat.shape[0] or centroids.shape[1] == 0 or centroids.shape[2] != d:
        raise ValueError(f"centroids must have shape [{flat.shape[0]},K,{d}] with K > 0")
    if not x.is_cuda:
        raise ValueError("peco_amd quantization runs on GPU tensors; CPU tensors are not supported")
    if d not in (64, 128):
        raise ValueError("HIP Base-Offset quantization supports head dimensions 64 and 128")
    if x.dtype not in _DTYPES:
        raise TypeError("x must be float16, bfloat16 or float32")
    return flat, labels.to(torch.int64), centroids.float()


def _launch_args(flat, labels, centroids):
    lab32 = labels.to(torch.int32).contiguous()
    return flat.contiguous(), lab32, centroids.contiguous()


@torch.no_grad()
def quantize_base_offset(x, labels, centroids, bits: int = 4) -> BaseOffsetQuantized:
    """Encode Q or K against its assigned cluster's vector centroid (bits 4 or 8)."""
    _validate_bits(bits, allow_bypass=False)
    flat, labels, centroids = _flatten_inputs(x, labels, centroids)
    xs, lab32, cent = _launch_args(flat, labels, centroids)
    bh, n, d = xs.shape
    codes = torch.empty((bh, n, d), dtype=torch.uint8, device=xs.device)
    low = torch.empty((bh, n, 1), dtype=torch.float32, device=xs.device)
    scale = torch.empty((bh, n, 1), dtype=torch.float32, device=xs.device)
    library = _native.library()
    with torch.cuda.device(xs.device):
        status = library.peco_base_offset_encode(
            _native.ptr(xs), _DTYPES[xs.dtype], _native.ptr(lab32), _native.ptr(cent), bh, n, cent.shape[1], d, bits,
            _native.ptr(codes), _native.ptr(low), _native.ptr(scale),
            _native.current_stream(xs.device, xs, lab32, cent, codes, low, scale),
        )
    _native.check(status, "Base-Offset encode")
    return BaseOffsetQuantized(centroids=centroids, labels=labels, codes=codes, offset_min=low, scale=scale,
                               original_dtype=x.dtype, original_shape=tuple(x.shape), bits=bits)


@torch.no_grad()
def dequantize_base_offset(encoded: BaseOffsetQuantized) -> torch.Tensor:
    """Reconstruct a quantized payload to the input shape and dtype."""
    codes = encoded.codes.contiguous()
    bh, n, d = codes.shape
    cent = encoded.centroids.float().contiguous()
    lab32 = encoded.labels.to(torch.int32).contiguous()
    low = encoded.offset_min.float().contiguous()
    scale = encoded.scale.float().contiguous()
    out = torch.empty((bh, n, d), dtype=encoded.original_dtype, device=codes.device)
    library = _native.library()
    with torch.cuda.device(codes.device):
        status = library.peco_base_offset_decode(
            _native.ptr(codes), _native.ptr(low), _native.ptr(scale), _native.ptr(lab32), _native.ptr(cent), bh, n,
            cent.shape[1], d, _DTYPES[encoded.original_dtype], _native.ptr(out),
            _native.current_stream(codes.device, codes, low, scale, lab32, cent, out),
        )
    _native.check(status, "Base-Offset decode")
    return out.reshape(encoded.original_shape)


@torch.no_grad()
def fake_quantize_base_offset(x, labels, centroids, bits: int = 4) -> torch.Tensor:
    """Quantize and dequantize Q or K in one pass; bits=0 returns x itself."""
    _validate_bits(bits, allow_bypass=True)
    if bits == 0:
        return x
    flat, labels, centroids = _flatten_inputs(x, labels, centroids)
    xs, lab32, cent = _launch_args(flat, labels, centroids)
    bh, n, d = xs.shape
    out = torch.empty_like(xs)
    library = _native.library()
    with torch.cuda.device(xs.device):
        status = library.peco_base_offset_fake_quant(
            _native.ptr(xs), _DTYPES[xs.dtype], _native.ptr(lab32), _native.ptr(cent), bh, n, cent.shape[1], d, bits,
            _native.ptr(out), _native.current_stream(xs.device, xs, lab32, cent, out),
        )
    _native.check(status, "Base-Offset fake quantization")
    return out.reshape(x.shape)
