"""Cluster-sparse attention on gfx950 MFMA (peco/attention_cuda.py interface).

QK^T and PV both run on MFMA (v_mfma_f32_32x32x16 bf16/fp16); the online softmax is
FP32. Unlike the reference, which keeps P in FP32 for a CUDA-core PV product, P is
rounded to the input dtype before the PV MFMA. Inference only; backward is unsupported.
"""
from __future__ import annotations

import ctypes

import torch

from . import _native

# Per-launch timing of the work-list attention (for measurement): None, or an object whose
# start(stream) and stop(stream) every sparse_attention_work call invokes immediately around
# its kernel launch (such as _native.LaunchTimer, which records HIP timing events there).
launch_timer = None


def _device_is_gfx950(device) -> bool:
    name = getattr(torch.cuda.get_device_properties(device), "gcnArchName", "")
    return name.split(":")[0] == "gfx950"


def _validate(q, k, v, dynamic_map, q_sizes, k_sizes):
    """Argument checks of peco/attention_cuda.py:84-119 (same messages)."""
    tensors = (q, k, v, dynamic_map, q_sizes, k_sizes)
    if not all(isinstance(tensor, torch.Tensor) for tensor in tensors):
        raise TypeError("All sparse attention inputs must be torch tensors")
    if q.ndim != 4 or k.ndim != 4 or v.shape != k.shape:
        raise ValueError("Expected Q [B,H,SQ,D] and equal-shaped K/V [B,H,SK,D]")
    batch, heads, sq, dim = q.shape
    if batch < 1 or heads < 1 or batch * heads > 65535:
        raise ValueError("B*H must be between 1 and 65535")
    if k.shape[:2] != q.shape[:2] or k.shape[-1] != dim:
        raise ValueError("Q and K/V batch, head, and feature dimensions must match")
    if dim not in (64, 128):
        raise ValueError("HIP attention supports head dimensions 64 and 128")
    if q.dtype not in (torch.float16, torch.bfloat16) or k.dtype != q.dtype or v.dtype != q.dtype:
        raise TypeError("Q/K/V must share dtype torch.float16 or torch.bfloat16")
    if not q.is_cuda or any(t.device != q.device for t in tensors):
        raise ValueError("All sparse attention inputs must reside on the same GPU device")
    if any(not t.is_contiguous() for t in tensors):
        raise ValueError("All sparse attention inputs must be contiguous")
    if q_sizes.ndim != 3 or k_sizes.ndim != 3 or q_sizes.shape[:2] != (batch, heads) or k_sizes.shape[:2] != (batch, heads):
        raise ValueError("Cluster sizes must have shape [B,H,C]")
    cq, ck = q_sizes.shape[-1], k_sizes.shape[-1]
    if cq < 1 or ck < 1 or dynamic_map.shape != (batch, heads, cq, ck):
        raise ValueError("Expected a nonempty cluster axis and dynamic_map [B,H,CQ,CK]")
    if dynamic_map.dtype != torch.bool or q_sizes.dtype != torch.int32 or k_sizes.dtype != torch.int32:
        raise TypeError("dynamic_map must be bool and cluster sizes must be int32")
    if torch.is_grad_enabled() and any(t.requires_grad for t in (q, k, v)):
        raise RuntimeError("PECO HIP sparse attention supports inference only; use torch.no_grad()")
    sk = k.shape[-2]
    capacity = (sq + 15) // 16 + cq
    stride = ck + 2 + 3 * capacity
    if max(sq, sk, cq, ck, capacity, stride) > 2**31 - 1:
        raise ValueError("Sequence/cluster metadata exceeds the int32 indexing limit")
    return batch, heads, sq, dim, sk, cq, ck, stride


def _check_index(index, name, batch, heads, rows):
    if not isinstance(index, torch.Tensor) or index.dtype != torch.int32 or not index.is_contiguous():
        raise ValueError(f"{name} must be a contiguous int32 tensor")
    if index.numel() != batch * heads * rows:
        raise ValueError(f"{name} must hold B*H*{rows} elements")


def _launch(q, k, v, dynamic_map, q_sizes, k_sizes, validate_sizes, out_index, k_index, rows, kept_keys=None):
    batch, heads, sq, dim, sk, cq, ck, stride = _validate(q, k, v, dynamic_map, q_sizes, k_sizes)
    with torch.cuda.device(q.device):
        if not _device_is_gfx950(q.device):
            raise RuntimeError("This HIP build requires an MI355X-class gfx950 GPU")
        if validate_sizes:
            torch._assert_async((q_sizes >= 0).all(), "q_sizes must be nonnegative")
            torch._assert_async((k_sizes >= 0).all(), "k_sizes must be nonnegative")
            torch._assert_async((q_sizes.sum(-1) == sq).all(), "q_sizes must sum to the Q sequence length")
            torch._assert_async((k_sizes.sum(-1) == sk).all(), "k_sizes must sum to the K sequence length")
        output = torch.empty_like(q)
        if sq == 0:
            return output
        rows = sq if rows is None else int(rows)
        if out_index is not None:
            if not 0 <= rows <= sq:
                raise ValueError("out_index_rows must be in [0, SQ]")
            _check_index(out_index, "out_index", batch, heads, rows)
        if k_index is not None:
            if rows > sk:
                raise ValueError("index_rows must be in [0, min(SQ, SK)]")
            _check_index(k_index, "k_index", batch, heads, rows)
            if k_index.device != q.device or out_index.device != q.device:
                raise ValueError("All sparse attention inputs must reside on the same GPU device")
        if kept_keys is not None:
            _check_index(kept_keys, "kept_keys", batch, heads, cq)
            if kept_keys.device != q.device:
                raise ValueError("All sparse attention inputs must reside on the same GPU device")
        # Same footprint as the reference's workspace (peco/attention_cuda.py:112-113,128).
        workspace = torch.empty(batch * heads * stride, dtype=torch.int32, device=q.device)
        library = _native.library()
        stream = _native.current_stream(q.device, q, k, v, dynamic_map, q_sizes, k_sizes, workspace, output,
                                        out_index, k_index, kept_keys)
        dtype = 0 if q.dtype == torch.float16 else 1
        head = (_native.ptr(q), _native.ptr(k), _native.ptr(v), _native.ptr(dynamic_map), _native.ptr(q_sizes),
                _native.ptr(k_sizes), _native.ptr(output))
        tail = (batch * heads, sq, sk, dim, cq, ck, dtype, stream)
        if k_index is None:
            error = library.peco_sparse_attention_ex(*head, _native.ptr(out_index), rows, _native.ptr(kept_keys),
                                                     _native.ptr(workspace), workspace.numel(), *tail)
        else:
            error = library.peco_sparse_attention_indexed(*head, _native.ptr(out_index), _native.ptr(k_index), rows,
                                                          _native.ptr(kept_keys), _native.ptr(workspace),
                                                          workspace.numel(), *tail)
        if error:
            message = library.peco_attention_error_string(error).decode("utf-8", errors="replace")
            raise RuntimeError(f"PECO HIP sparse attention launch failed: {message} ({error})")
        return output


def sparse_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    dynamic_map: torch.Tensor,
    q_sizes: torch.Tensor,
    k_sizes: torch.Tensor,
    *,
    validate_sizes: bool = True,
    out_index: torch.Tensor | None = None,
    out_index_rows: int | None = None,
    kept_keys: torch.Tensor | None = None,
) -> torch.Tensor:
    """Return cluster-masked softmax(QK^T/sqrt(D))V.

    Inputs must be contiguous GPU tensors: Q [B,H,SQ,D], K/V [B,H,SK,D], bool map
    [B,H,CQ,CK] and int32 sizes [B,H,CQ/CK]. Tokens must already be grouped in cluster
    order. Empty clusters and completely masked rows are supported; a completely masked
    row returns zero. Sizes are checked on the stream without copying them to the host.
    ``out_index`` (int32 [B*H, R], optional) writes output row j < R of head b to row
    out_index[b, j] instead (rows j >= R keep their position), fusing the inverse token
    permutation into the epilogue. R is ``out_index_rows`` (default SQ). ``kept_keys`` (int32
    [B,H,CQ], optional) gives the key rows each query cluster keeps, as
    ``select_connections(..., with_kept=True)`` returns them; it only orders the work items.
    """
    return _launch(q, k, v, dynamic_map, q_sizes, k_sizes, validate_sizes, out_index, None, out_index_rows,
                   kept_keys)


def sparse_attention_indexed(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    dynamic_map: torch.Tensor,
    q_sizes: torch.Tensor,
    k_sizes: torch.Tensor,
    q_index: torch.Tensor,
    k_index: torch.Tensor,
    index_rows: int,
    *,
    validate_sizes: bool = True,
    kept_keys: torch.Tensor | None = None,
) -> torch.Tensor:
    """``sparse_attention`` on Q/K/V left in their original token order.

    The cluster order is given by the sort permutations instead of a packed copy: stream
    row j < R of head b is query row q_index[b, j] and key/value row k_index[b, j]
    (R = ``index_rows``, the video length); rows j >= R (text) keep their position. Output
    row j < R is written to row q_index[b, j], so the result is in original order. Equals
    ``sparse_attention(gather(q, q_index), gather(k, k_index), gather(v, k_index), ...,
    out_index=q_index, out_index_rows=R)`` bit for bit, without the gather pass
    (peco/processor.py:143-156 with the reorder of peco/clustering.py:112-136 fused in).
    ``kept_keys`` (int32 [B,H,CQ], optional) gives the key rows each query cluster keeps, as
    ``select_connections(..., with_kept=True)`` returns them; it only orders the work items.
    """
    if q_index is None or k_index is None:
        raise ValueError("q_index and k_index are required")
    return _launch(q, k, v, dynamic_map, q_sizes, k_sizes, validate_sizes, q_index, k_index, index_rows, kept_keys)


def sparse_attention_work(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    work,
    *,
    out_index: torch.Tensor | None = None,
    out_index_rows: int | None = None,
    k_index: torch.Tensor | None = None,
    q_centroids: torch.Tensor | None = None,
    bits: int = 0,
) -> torch.Tensor:
    """``sparse_attention`` over the work list of ``clustering_cuda.select_work``.

    The key stream of every query cluster comes from its kept-segment list, so no map is
    read and no builder runs. Without ``k_index`` Q/K/V are in cluster order (as for
    ``sparse_attention``, with an optional ``out_index`` scatter of the first
    ``out_index_rows`` output rows); with it, Q/K/V are in original order and read through
    ``out_index`` (queries, also the output scatter) and ``k_index`` (keys and values), as
    ``sparse_attention_indexed``. With ``q_centroids`` (fp32 [B*H, CQ, D]; needs
    ``out_index``) Q is in original order, read through ``out_index`` and Base-Offset
    fake-quantized with ``bits`` against its cluster's centroid as it is loaded
    (peco/processor.py:141 and the Q gather fused into the kernel); K/V are then in cluster
    order, or in original order read through ``k_index`` when it is given.
    """
    for name, t in (("q", q), ("k", k), ("v", v)):
        if not isinstance(t, torch.Tensor) or not t.is_cuda or not t.is_contiguous() or t.dim() != 4:
            raise ValueError(f"{name} must be a contiguous 4-D GPU tensor")
    if q.dtype not in (torch.float16, torch.bfloat16) or k.dtype != q.dtype or v.dtype != q.dtype:
        raise ValueError("PECO HIP sparse attention supports float16 and bfloat16")
    batch, heads, sq, dim = q.shape
    sk = k.shape[2]
    if k.shape != (batch, heads, sk, dim) or v.shape != k.shape or dim not in (64, 128):
        raise ValueError("q/k/v shapes must be [B,H,S,D] with D in {64, 128} and matching K/V")
    if work.bh != batch * heads or work.sq != sq or work.sk != sk:
        raise ValueError("the work list was built for another shape")
    if not work.valid():
        raise RuntimeError("the work list was overwritten by a later select_work call of the same shape on this "
                           "stream; call select_work again")
    output = torch.empty_like(q)
    if sq == 0:
        return output
    rows = sq if out_index_rows is None else int(out_index_rows)
    if out_index is not None:
        if not 0 <= rows <= sq:
            raise ValueError("out_index_rows must be in [0, SQ]")
        _check_index(out_index, "out_index", batch, heads, rows)
    if k_index is not None:
        if out_index is None or rows > sk:
            raise ValueError("k_index needs out_index and index rows in [0, min(SQ, SK)]")
        _check_index(k_index, "k_index", batch, heads, rows)
    q_clusters = 0
    if q_centroids is not None:
        if out_index is None or bits not in (4, 8):
            raise ValueError("q_centroids needs out_index and bits in {4, 8}")
        if q_centroids.dtype != torch.float32 or not q_centroids.is_contiguous() or q_centroids.dim() != 3 \
                or q_centroids.shape[0] != batch * heads or q_centroids.shape[2] != dim \
                or not 1 <= q_centroids.shape[1] <= work.rows or q_centroids.device != q.device:
            raise ValueError("q_centroids must be contiguous fp32 [B*H, CQ, D] on the device of q")
        q_clusters = q_centroids.shape[1]
    with torch.cuda.device(q.device):
        if not _device_is_gfx950(q.device):
            raise RuntimeError("This HIP build requires an MI355X-class gfx950 GPU")
        library = _native.library()
        stream = _native.current_stream(q.device, q, k, v, work.buffer, out_index, k_index, q_centroids)
        timer = launch_timer
        if timer is not None:
            timer.start(stream)
        error = library.peco_sparse_attention_work(
            _native.ptr(q), _native.ptr(k), _native.ptr(v), _native.ptr(output), _native.ptr(out_index), rows,
            _native.ptr(k_index), _native.ptr(q_centroids), q_clusters, int(bits) if q_centroids is not None else 0,
            _native.ptr(work.buffer), work.ints, batch * heads, sq, sk, dim, work.rows, work.cols,
            0 if q.dtype == torch.float16 else 1, stream)
        if timer is not None:
            timer.stop(stream)
        if error:
            message = library.peco_attention_error_string(error).decode("utf-8", errors="replace")
            raise RuntimeError(f"PECO HIP sparse attention launch failed: {message} ({error})")
    return output


def centroid_planes(centroids: torch.Tensor):
    """Key centroids [BH, K, D] fp32 as three int8 planes and a scale per centroid:
    C = cs * (P0 + P1/128 + P2/16384) to within 2^-21 * max|C| of each centroid (the last
    plane's half step, 2^-22, plus the fp32 rounding of C / cs), plus Sum(C).

    Returns (planes int8 [BH, K, 3, D], cs fp32 [BH, K], sums fp32 [BH, K]). cs = max|C|/127
    (1 for a zero centroid); each plane is the rounded remainder of the one before, scaled
    by 128.
    """
    c = centroids.float()
    cs = c.abs().amax(dim=-1) / 127.0
    cs = torch.where(cs > 0, cs, torch.ones_like(cs))
    x = c / cs[..., None]
    p0 = torch.round(x).clamp_(-127, 127)
    r1 = (x - p0) * 128.0
    p1 = torch.round(r1).clamp_(-127, 127)
    r2 = (r1 - p1) * 128.0
    p2 = torch.round(r2).clamp_(-127, 127)
    planes = torch.stack((p0, p1, p2), dim=-2).to(torch.int8).contiguous()
    return planes, cs.contiguous(), c.sum(dim=-1).contiguous()


def base_offset_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    dynamic_map: torch.Tensor,
    q_sizes: torch.Tensor,
    k_sizes: torch.Tensor,
    *,
    out_index: torch.Tensor,
    q_centroids: torch.Tensor,
    k_centroids: torch.Tensor,
    k_codes: torch.Tensor,
    k_low: torch.Tensor,
    k_scale: torch.Tensor,
    bits: int,
) -> torch.Tensor:
    """Cluster-sparse attention with Base-Offset scores on the integer MFMA (an extension: the
    reference reconstructs Q/K and runs floating-point attention, peco/quantization.py:1-22,
    README.md:18).

    Video query rows against video key clusters score through the exact expansion of
    (Cq + a + s u).(Ck + b + t w) with u.w on v_mfma_i32_32x32x32_i8; text scores use the
    fake-quantized bf16 rows as the reference does. Inputs: ``q`` [B,H,S,D] in original
    order (its first N = ``out_index.shape[-1]`` video rows Base-Offset quantized at load
    against ``q_centroids`` [B*H, KQ, D], rows j < N of the cluster order read from
    ``out_index[j]``, which also places the output); ``k`` (video rows fake-quantized), ``v``
    [B,H,S,D] and ``k_codes`` uint8 [B*H, N, D], ``k_low``/``k_scale`` fp32 [B*H, N] in key
    cluster order, as ``clustering_cuda.kmeans_fit`` packs them (``k_centroids`` [B*H, KK, D]);
    the extended map [B,H,KQ+2,KK+2] and sizes of ``clustering_cuda.select_connections`` with
    the text partition.
    """
    for name, t in (("q", q), ("k", k), ("v", v)):
        if not isinstance(t, torch.Tensor) or not t.is_cuda or not t.is_contiguous() or t.dim() != 4:
            raise ValueError(f"{name} must be a contiguous 4-D GPU tensor")
    if q.dtype not in (torch.float16, torch.bfloat16) or k.dtype != q.dtype or v.dtype != q.dtype:
        raise ValueError("PECO HIP sparse attention supports float16 and bfloat16")
    batch, heads, sq, dim = q.shape
    sk = k.shape[2]
    bh = batch * heads
    if k.shape != (batch, heads, sk, dim) or v.shape != k.shape or dim not in (64, 128):
        raise ValueError("q/k/v shapes must be [B,H,S,D] with D in {64, 128} and matching K/V")
    if bits not in (4, 8):
        raise ValueError("bits must be 4 or 8")
    if dynamic_map.dtype != torch.bool or dynamic_map.dim() != 4 or dynamic_map.shape[:2] != (batch, heads):
        raise ValueError("dynamic_map must be bool [B,H,CQ,CK]")
    cq, ck = dynamic_map.shape[2:]
    if tuple(q_sizes.shape) != (batch, heads, cq) or tuple(k_sizes.shape) != (batch, heads, ck):
        raise ValueError("q_sizes/k_sizes must be [B,H,CQ] and [B,H,CK]")
    rows = out_index.shape[-1]
    _check_index(out_index, "out_index", batch, heads, rows)
    if not 1 <= rows <= min(sq, sk):
        raise ValueError("out_index must cover between 1 and min(SQ, SK) video rows")
    kq, kk = q_centroids.shape[1], k_centroids.shape[1]
    for name, t, shape in (("q_centroids", q_centroids, (bh, kq, dim)), ("k_centroids", k_centroids, (bh, kk, dim)),
                           ("k_low", k_low, (bh, rows)), ("k_scale", k_scale, (bh, rows))):
        if t.dtype != torch.float32 or not t.is_contiguous() or tuple(t.shape) != shape or t.device != q.device:
            raise ValueError(f"{name} must be contiguous fp32 {list(shape)} on the device of q")
    if k_codes.dtype != torch.uint8 or not k_codes.is_contiguous() or tuple(k_codes.shape) != (bh, rows, dim):
        raise ValueError("k_codes must be contiguous uint8 [B*H, N, D]")
    if not 1 <= kq <= cq or not 1 <= kk <= ck:
        raise ValueError("the centroids must describe the first clusters of the map")
    output = torch.empty_like(q)
    with torch.cuda.device(q.device):
        if not _device_is_gfx950(q.device):
            raise RuntimeError("This HIP build requires an MI355X-class gfx950 GPU")
        library = _native.library()
        planes, cs, csum = centroid_planes(k_centroids)
        qk_dot = torch.bmm(k_centroids.double(), q_centroids.double().transpose(1, 2).contiguous()).float()
        smap = dynamic_map.contiguous().view(torch.uint8)
        qs = q_sizes.to(torch.int32).contiguous()
        ks = k_sizes.to(torch.int32).contiguous()
        ws_ints = library.peco_sparse_attention_workspace_size(bh, sq, sk, cq, ck)
        workspace = torch.empty(ws_ints, dtype=torch.int32, device=q.device)
        stream = _native.current_stream(q.device, q, k, v, output, out_index, q_centroids, k_codes, k_low, k_scale,
                                        planes, cs, csum, qk_dot, smap, qs, ks, workspace)
        error = library.peco_base_offset_attention(
            _native.ptr(q), _native.ptr(out_index), _native.ptr(q_centroids), kq, _native.ptr(k), _native.ptr(v),
            _native.ptr(k_codes), _native.ptr(k_low), _native.ptr(k_scale), _native.ptr(planes), _native.ptr(cs),
            _native.ptr(csum), _native.ptr(qk_dot), kk, int(bits), _native.ptr(smap), _native.ptr(qs),
            _native.ptr(ks), _native.ptr(output), _native.ptr(workspace), ws_ints, bh, sq, sk, rows, dim, cq, ck,
            0 if q.dtype == torch.float16 else 1, stream)
        if error:
            message = library.peco_attention_error_string(error).decode("utf-8", errors="replace")
            raise RuntimeError(f"PECO HIP Base-Offset attention launch failed: {message} ({error})")
    return output
