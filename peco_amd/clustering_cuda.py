"""PECO clustering kernels on gfx950 through the C-ABI (peco/clustering_cuda.py interface).

The module name is kept from the reference so callers can switch imports unchanged.
Clustering reads FP32/BF16/FP16 features and writes FP32 centres with int32
labels/counts; token reordering copies FP16/BF16/FP32 feature bits unchanged.
Every call is asynchronous on torch's current stream.
"""
from __future__ import annotations

import collections
import ctypes

import torch

from . import _native

_DTYPES = {torch.float16: 0, torch.bfloat16: 1, torch.float32: 2}


def build_cluster_library():
    """Build the HIP library when missing or older than its sources; return its path."""
    return _native.build_library()


def _library():
    return _native.library()


def _raise_cluster_error(status):
    """Raise for an immediate launch failure (peco/clustering_cuda.py:76-80)."""
    if status:
        message = _library().peco_cluster_error_message(status).decode("utf-8", errors="replace")
        raise RuntimeError(f"HIP clustering failed: {message} (status {status})")


def _retain_on_current_stream(device, *tensors):
    return _native.current_stream(device, *tensors)


def assign_tokens_to_centers(x, centers, labels, scratch, center_norms, chunk_size):
    """Assign FP32 x [B,N,D] to centers [B,C,D], writing int32 labels [B,N].

    ``center_norms`` [B,C] receives the centre norms. ``scratch`` and ``chunk_size``
    are accepted for interface compatibility; the MFMA kernel needs no N-by-C scratch.
    """
    library = _library()
    batch, tokens, dims = x.shape
    clusters = centers.shape[1]
    with torch.cuda.device(x.device):
        status = library.peco_assign_tokens_to_centers(
            _native.ptr(x), _native.ptr(centers), _native.ptr(labels), _native.ptr(scratch),
            _native.ptr(center_norms), batch, tokens, dims, clusters, chunk_size,
            _retain_on_current_stream(x.device, x, centers, labels, scratch, center_norms),
        )
    _raise_cluster_error(status)


def recompute_cluster_centers(x, labels, previous, sums, counts, means):
    """Write FP32 means [B,C,D] and int32 counts [B,C] for labels [B,N].

    ``sums`` [B,C,D] receives the per-cluster sums; empty clusters keep ``previous``.
    """
    library = _library()
    batch, tokens, dims = x.shape
    with torch.cuda.device(x.device):
        status = library.peco_recompute_cluster_centers(
            _native.ptr(x), _native.ptr(labels), _native.ptr(previous), _native.ptr(sums),
            _native.ptr(counts), _native.ptr(means), batch, tokens, dims, previous.shape[1],
            _retain_on_current_stream(x.device, x, labels, previous, sums, counts, means),
        )
    _raise_cluster_error(status)


def reorder_token_features(tensor, indices, inverse=False):
    """Reorder features [B,H,N,D] using original token IDs [B*H,N].

    Forward gathers original IDs into sorted order; inverse scatters sorted rows back.
    """
    library = _library()
    tensor = tensor.contiguous()
    indices = indices.to(dtype=torch.int32).contiguous()
    batch, heads, tokens, dims = tensor.shape
    result = torch.empty_like(tensor)
    with torch.cuda.device(tensor.device):
        status = library.peco_reorder_token_features(
            _native.ptr(tensor), _native.ptr(indices), _native.ptr(result), batch * heads, tokens, dims,
            tensor.element_size(), int(inverse), _retain_on_current_stream(tensor.device, tensor, indices, result),
        )
    _raise_cluster_error(status)
    return result


def cluster_sort(labels, clusters):
    """Stable sort of int32 labels [B,N] with values in [0, clusters).

    Returns (indices [B,N], counts [B,C], offsets [B,C+1]) where indices[b, j] is the
    original token at sorted position j (== torch.argsort(labels, stable=True)).
    """
    library = _library()
    labels = labels.to(torch.int32).contiguous()
    batch, tokens = labels.shape
    dev = labels.device
    indices = torch.empty((batch, tokens), dtype=torch.int32, device=dev)
    counts = torch.empty((batch, clusters), dtype=torch.int32, device=dev)
    offsets = torch.empty((batch, clusters + 1), dtype=torch.int32, device=dev)
    ws_bytes = library.peco_cluster_sort_workspace_size(batch, tokens, clusters)
    ws = torch.empty(max(ws_bytes, 4), dtype=torch.uint8, device=dev)
    with torch.cuda.device(dev):
        status = library.peco_cluster_sort(
            _native.ptr(labels), batch, tokens, clusters, _native.ptr(indices), None, _native.ptr(counts),
            _native.ptr(offsets), _native.ptr(ws), ws.numel(),
            _retain_on_current_stream(dev, labels, indices, counts, offsets, ws),
        )
    _raise_cluster_error(status)
    return indices, counts, offsets


class KMeansProblem:
    """One k-means problem for :func:`kmeans_fit`: x [B,N,D] (rows may have a batch stride)."""

    def __init__(self, x, init_centers):
        if x.ndim != 3 or x.stride(2) != 1 or x.stride(1) != x.shape[2]:
            raise ValueError("x must be [B,N,D] with contiguous token rows")
        if init_centers.ndim != 3 or init_centers.shape[0] != x.shape[0] or init_centers.shape[2] != x.shape[2] \
                or not 1 <= init_centers.shape[1] <= x.shape[1] or init_centers.device != x.device:
            raise ValueError("init_centroids must match [batch_heads, n_clusters, dims] and x.device")
        self.x = x
        self.init = init_centers.float().contiguous()
        self.batch, self.tokens, self.dims = x.shape
        self.clusters = self.init.shape[1]


def kmeans_fit(problems, iterations, pack=None, pack_order="cluster"):
    """Fused Lloyd fit of one or two problems (their heads run as four chains of launches, three
    on library streams forked from and joined back to the current stream).

    Returns, per problem, (labels int32 [B,N], centers fp32 [B,K,D], counts int32 [B,K],
    indices int32 [B,N], offsets int32 [B,K+1]); indices is the stable sort of labels.

    ``pack`` (optional, one entry per problem, None or ``(bits, length, with_tensor)``) makes
    the last update also pack that problem (peco/processor.py:141-149 fused into the fit):
    hat [B, length, D] receives x's rows in the final cluster order, Base-Offset
    fake-quantized with ``bits`` against the final centres, then x's rows [N, length) (the
    text, which x's batch stride must cover); ``with_tensor`` ([B, length, D] or None) is
    gathered in the same order into a new tensor. Then returns (outs, packed) with packed[i] =
    (hat, with_out) or None. An entry ``(bits, length, with_tensor, True)`` also returns the
    Base-Offset payload of hat's first N rows in that order: packed[i] = (hat, with_out,
    codes uint8 [B, N, D], low fp32 [B, N], scale fp32 [B, N]), the values
    quantize_base_offset computes (peco/quantization.py:97-128).

    ``pack_order="original"`` writes hat's rows [0, N) (and the payload) at each token's own
    position instead of in cluster order, so hat is x with its video rows fake-quantized;
    no ``with_tensor`` is gathered then.
    """
    library = _library()
    if not 1 <= len(problems) <= 2:
        raise ValueError("kmeans_fit takes one or two problems")
    dims = problems[0].dims
    dtype = problems[0].x.dtype
    dev = problems[0].x.device
    if any(p.dims != dims or p.x.dtype != dtype or p.x.device != dev for p in problems):
        raise ValueError("kmeans_fit problems must share dims, dtype and device")
    if pack is not None and len(pack) != len(problems):
        raise ValueError("pack needs one entry per problem")
    if pack_order not in ("cluster", "original"):
        raise ValueError("pack_order must be 'cluster' or 'original'")
    outs = []
    ws_bytes = 0
    for p in problems:
        outs.append((
            torch.empty((p.batch, p.tokens), dtype=torch.int32, device=dev),
            torch.empty((p.batch, p.clusters, dims), dtype=torch.float32, device=dev),
            torch.empty((p.batch, p.clusters), dtype=torch.int32, device=dev),
            torch.empty((p.batch, p.tokens), dtype=torch.int32, device=dev),
            torch.empty((p.batch, p.clusters + 1), dtype=torch.int32, device=dev),
        ))
        ws_bytes += library.peco_kmeans_workspace_size(p.batch, p.tokens, p.clusters, dims)
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    strides = (ctypes.c_int64 * len(problems))(*[p.x.stride(0) for p in problems])
    # Only the caller's tensors need recording: the outputs and the workspace are allocated
    # here, on the stream the launches run on.
    tensors = [p.x for p in problems] + [p.init for p in problems]
    common = (
        len(problems),
        _native.ptr_array([p.x for p in problems]), ctypes.cast(strides, ctypes.c_void_p),
        _native.ptr_array([p.init for p in problems]),
        _native.ptr_array([o[1] for o in outs]), _native.ptr_array([o[0] for o in outs]),
        _native.ptr_array([o[2] for o in outs]), _native.ptr_array([o[3] for o in outs]),
        _native.ptr_array([o[4] for o in outs]),
        _native.int_array([p.batch for p in problems]), _native.int_array([p.tokens for p in problems]),
        _native.int_array([p.clusters for p in problems]), dims, _DTYPES[dtype], int(iterations),
    )
    if pack is None:
        with torch.cuda.device(dev):
            status = library.peco_kmeans_fit(*common, _native.ptr(ws), ws_bytes,
                                             _retain_on_current_stream(dev, *tensors))
        _raise_cluster_error(status)
        return outs
    length = None
    hats, withs_in, withs_out, bits, payloads = [], [], [], [], []
    for p, spec in zip(problems, pack):
        if spec is None:
            hats.append(None), withs_in.append(None), withs_out.append(None), bits.append(0)
            payloads.append(None)
            continue
        b, n, w = spec[:3]
        want_codes = len(spec) > 3 and bool(spec[3])
        if length is not None and n != length:
            raise ValueError("packed problems must share one length")
        length = int(n)
        if length < p.tokens or (length > p.tokens and p.x.stride(0) < length * dims):
            raise ValueError("x's batch stride must cover the packed length")
        hats.append(torch.empty((p.batch, length, dims), dtype=dtype, device=dev))
        if w is not None:
            if pack_order != "cluster":
                raise ValueError("a gathered companion needs pack_order='cluster'")
            if w.shape != (p.batch, length, dims) or w.dtype != dtype or not w.is_contiguous() or w.device != dev:
                raise ValueError("the gathered companion must be a contiguous [B, length, D] tensor like x")
            withs_out.append(torch.empty_like(w))
        else:
            withs_out.append(None)
        withs_in.append(w)
        bits.append(int(b))
        payloads.append((torch.empty((p.batch, p.tokens, dims), dtype=torch.uint8, device=dev),
                         torch.empty((p.batch, p.tokens), dtype=torch.float32, device=dev),
                         torch.empty((p.batch, p.tokens), dtype=torch.float32, device=dev)) if want_codes else None)
    codes, lows, scales = ([None if q is None else q[i] for q in payloads] for i in range(3))
    extra = [t for t in withs_in if t is not None]
    with torch.cuda.device(dev):
        status = library.peco_kmeans_fit_pack(
            *common, _native.ptr_array(hats), _native.int_array(bits), _native.ptr_array(withs_in),
            _native.ptr_array(withs_out), _native.ptr_array(codes), _native.ptr_array(lows),
            _native.ptr_array(scales), int(length or 0), int(pack_order == "original"), _native.ptr(ws), ws_bytes,
            _retain_on_current_stream(dev, *tensors, *extra))
    _raise_cluster_error(status)
    packed = [None if h is None else ((h, w) if q is None else (h, w, *q))
              for h, w, q in zip(hats, withs_out, payloads)]
    return outs, packed


def select_connections(query_centroids, key_centroids, q_counts, k_counts, p, minimum, text=None, *,
                       with_kept=False):
    """Cluster-pair map of select_cluster_connections in one launch.

    Centroids [..., C, D], counts [..., C]. With ``text=(valid_text, text_length)`` the map
    is extended with the text partition and the extended size vectors are returned too.
    Returns (map bool [..., CQ(+2), CK(+2)], ext_q_sizes or None, ext_k_sizes or None), and
    with ``with_kept`` also int32 [..., CQ(+2)]: the key rows each map row keeps.
    """
    library = _library()
    lead = query_centroids.shape[:-2]
    cq, dims = query_centroids.shape[-2:]
    ck = key_centroids.shape[-2]
    bh = 1
    for n in lead:
        bh *= n
    dev = query_centroids.device
    qc = query_centroids.float().reshape(bh, cq, dims).contiguous()
    kc = key_centroids.float().reshape(bh, ck, dims).contiguous()
    qn = q_counts.to(torch.int32).reshape(bh, cq).contiguous()
    kn = k_counts.to(torch.int32).reshape(bh, ck).contiguous()
    extend = text is not None
    re, ce = (cq + 2, ck + 2) if extend else (cq, ck)
    dmap = torch.empty((*lead, re, ce), dtype=torch.bool, device=dev)
    ext_q = torch.empty((*lead, re), dtype=torch.int32, device=dev) if extend else None
    ext_k = torch.empty((*lead, ce), dtype=torch.int32, device=dev) if extend else None
    kept = torch.empty((*lead, re), dtype=torch.int32, device=dev) if with_kept else None
    valid_text, text_length = text if extend else (0, 0)
    with torch.cuda.device(dev):
        status = library.peco_select_cluster_connections(
            _native.ptr(qc), _native.ptr(kc), _native.ptr(qn), _native.ptr(kn), bh, cq, ck, dims, float(p),
            int(minimum), int(extend), int(valid_text), int(text_length), _native.ptr(dmap), _native.ptr(ext_q),
            _native.ptr(ext_k), _native.ptr(kept), _retain_on_current_stream(dev, qc, kc, qn, kn, dmap, ext_q, ext_k,
                                                                             kept),
        )
    _raise_cluster_error(status)
    if with_kept:
        return dmap, ext_q, ext_k, kept
    return dmap, ext_q, ext_k


class SelectionWork:
    """Work list of one peco_select_work launch: the kept-segment list of every map row and
    the attention items of every (batch, head) in cost order, in ``buffer`` (int32). ``rows``
    and ``cols`` are the map's dimensions (text groups included), ``sq``/``sk`` the attention's
    query/key lengths it was built for.

    Calls of ``select_work`` of one shape on one stream share a cached buffer, so a
    SelectionWork stays valid only until the next such call: ``sparse_attention_work``
    checks ``valid()`` and raises for a work list that a later call has overwritten."""

    def __init__(self, buffer, bh, sq, sk, rows, cols, ints, slot=None):
        self.buffer, self.bh, self.sq, self.sk, self.rows, self.cols, self.ints = buffer, bh, sq, sk, rows, cols, ints
        self._slot = slot
        self._generation = None if slot is None else slot.generation

    def valid(self):
        """False once a later select_work call has rewritten this work list's buffer."""
        return self._slot is None or self._slot.generation == self._generation

    def _layout(self):
        b, re, ce = self.bh, self.rows, self.cols
        cap = -(-self.sq // 128) + min(re, self.sq)
        head = 2 * b + b * re + b * cap * 3 + self.QUEUE_INTS
        head += head & 1
        return b, re, ce, cap, head

    # The attention's item queue counters (one per XCD) and exit counter after the items.
    QUEUE_INTS = 16

    def tickets(self):
        return self.buffer[:self.bh]

    def queues(self):
        """The attention's item queue counters: zero between calls."""
        b, re, _, cap, _ = self._layout()
        start = 2 * b + b * re + b * cap * 3
        return self.buffer[start:start + self.QUEUE_INTS]

    def items(self):
        """(count int32 [bh], items int32 [bh, cap, 3]) as views of the buffer."""
        b, re, _, cap, _ = self._layout()
        counts = self.buffer[b:2 * b]
        items = self.buffer[2 * b + b * re:2 * b + b * re + b * cap * 3].view(b, cap, 3)
        return counts, items

    def row_lengths(self):
        b, re, _, _, _ = self._layout()
        return self.buffer[2 * b:2 * b + b * re].view(b, re)

    def segments(self):
        """int32 [bh, rows, cols + 2, 2]: per row {count, L}, the segments, the sentinel."""
        b, re, ce, _, head = self._layout()
        return self.buffer[head:head + b * re * (ce + 2) * 2].view(b, re, ce + 2, 2)


class _WorkSlot:
    """A cached work buffer and the number of select_work launches that have written it."""

    def __init__(self, buffer):
        self.buffer = buffer
        self.generation = 0


# Work buffers by (device, stream, shape): their arrival and queue counters start at zero and
# every launch leaves them zero, and launches on one stream are ordered, so they can share a
# buffer. The least recently used entries beyond the limit are dropped (a SelectionWork keeps
# its own buffer alive).
_WORK_BUFFERS = collections.OrderedDict()
_WORK_BUFFER_LIMIT = 8


def _work_slot(device, ints, shape):
    stream = torch.cuda.current_stream(device).cuda_stream
    key = (device.index, stream, shape)
    slot = _WORK_BUFFERS.pop(key, None)
    if slot is None:
        slot = _WorkSlot(torch.zeros(ints, dtype=torch.int32, device=device))
    _WORK_BUFFERS[key] = slot
    while len(_WORK_BUFFERS) > _WORK_BUFFER_LIMIT:
        _WORK_BUFFERS.popitem(last=False)
    slot.generation += 1
    return slot


def select_work(query_centroids, key_centroids, q_counts, k_counts, p, minimum, text, sq, sk):
    """Selection (as ``select_connections``) and the attention's work list in one launch.

    Same inputs as ``select_connections`` with ``text=(valid_text, text_length)`` or None;
    sq/sk are the attention's query/key lengths (video + text). No map is written: the
    attention reads each query cluster's kept-segment list instead. Returns a
    ``SelectionWork`` for ``attention_cuda.sparse_attention_work``, valid until the next
    ``select_work`` call of the same shape on the same stream (which reuses its buffer).
    """
    library = _library()
    lead = query_centroids.shape[:-2]
    cq, dims = query_centroids.shape[-2:]
    ck = key_centroids.shape[-2]
    bh = 1
    for n in lead:
        bh *= n
    dev = query_centroids.device
    qc = query_centroids.float().reshape(bh, cq, dims).contiguous()
    kc = key_centroids.float().reshape(bh, ck, dims).contiguous()
    qn = q_counts.to(torch.int32).reshape(bh, cq).contiguous()
    kn = k_counts.to(torch.int32).reshape(bh, ck).contiguous()
    extend = text is not None
    valid_text, text_length = text if extend else (0, 0)
    re, ce = (cq + 2, ck + 2) if extend else (cq, ck)
    ints = library.peco_select_work_size(bh, int(sq), cq, ck, int(extend))
    if ints == 0:
        raise ValueError("invalid selection work shape")
    with torch.cuda.device(dev):
        slot = _work_slot(dev, ints, (bh, int(sq), re, ce))
        work = slot.buffer
        status = library.peco_select_work(
            _native.ptr(qc), _native.ptr(kc), _native.ptr(qn), _native.ptr(kn), bh, cq, ck, dims, float(p),
            int(minimum), int(extend), int(valid_text), int(text_length), int(sq), int(sk), None, None, None,
            _native.ptr(work), ints, _retain_on_current_stream(dev, qc, kc, qn, kn, work))
    _raise_cluster_error(status)
    return SelectionWork(work, bh, int(sq), int(sk), re, ce, ints, slot)


def pack_clustered(tensors, indices, labels, centroids, bits, video):
    """Gather up to three [B,H,S,D] tensors into cluster order in one launch.

    Rows [0, video) of tensor i are taken in the order of indices[i] [B*H, video]; when
    bits[i] is 4 or 8 they are Base-Offset fake-quantized against (labels[i], centroids[i])
    on the way. Rows [video, S) (text) are copied unchanged. Returns new tensors.
    """
    library = _library()
    ref = tensors[0]
    b, h, s, d = ref.shape
    outs = [torch.empty_like(t) for t in tensors]
    n = len(tensors)
    clusters = [0 if c is None else c.shape[1] for c in centroids]
    with torch.cuda.device(ref.device):
        status = library.peco_pack_clustered(
            _native.ptr_array(tensors), _native.ptr_array(outs), _native.ptr_array(indices),
            _native.ptr_array(labels), _native.ptr_array(centroids), _native.int_array(clusters),
            _native.int_array(bits), n, b * h, s, video, d, _DTYPES[ref.dtype],
            _retain_on_current_stream(ref.device, *tensors, *outs, *[t for t in indices + labels + centroids]),
        )
    _raise_cluster_error(status)
    return outs


if __name__ == "__main__":
    print(build_cluster_library())
