"""ctypes wrapper over the C oracle (oracle/peco_oracle.c). Test infrastructure only.

All functions take and return numpy arrays (float32 / int32 / uint8, C-contiguous).
"""
from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np

from . import build as _build

_LIB = None


def _lib():
    global _LIB
    if _LIB is None:
        path = _build.OUTPUT
        if not path.exists():
            path = _build.build()
        lib = ctypes.CDLL(str(path))
        P, I = ctypes.c_void_p, ctypes.c_int
        lib.oracle_center_norms.argtypes = [P, I, I, I, P]
        lib.oracle_assign.argtypes = [P, P, P, I, I, I, I, P, P, P]
        lib.oracle_update.argtypes = [P, P, P, I, I, I, I, P, P, P]
        lib.oracle_stable_sort.argtypes = [P, I, I, I, P, P]
        lib.oracle_kmeans_fit.argtypes = [P, P, I, I, I, I, I, P, P, P, P, P]
        lib.oracle_base_offset.argtypes = [P, P, P, I, I, I, I, I, P, P, P, P]
        lib.oracle_sparse_attention.argtypes = [P, P, P, P, P, P, I, I, I, I, I, I, P]
        lib.oracle_num_threads.restype = I
        for name in ("oracle_center_norms", "oracle_assign", "oracle_update", "oracle_stable_sort",
                     "oracle_kmeans_fit", "oracle_base_offset", "oracle_sparse_attention"):
            getattr(lib, name).restype = None
        _LIB = lib
    return _LIB


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _i32(a):
    return np.ascontiguousarray(a, dtype=np.int32)


def _ptr(a):
    return ctypes.c_void_p(a.ctypes.data) if a is not None else None


def num_threads() -> int:
    return _lib().oracle_num_threads()


def center_norms(centers):
    c = _f32(centers)
    b, k, d = c.shape
    out = np.empty((b, k), np.float32)
    _lib().oracle_center_norms(_ptr(c), b, k, d, _ptr(out))
    return out


def assign(x, centers, norms=None, *, margins=False):
    """labels [B,N] (and best/second canonical distances when ``margins``)."""
    x, c = _f32(x), _f32(centers)
    b, n, d = x.shape
    k = c.shape[1]
    norms = center_norms(c) if norms is None else _f32(norms)
    labels = np.empty((b, n), np.int32)
    best = np.empty((b, n), np.float32) if margins else None
    second = np.empty((b, n), np.float32) if margins else None
    _lib().oracle_assign(_ptr(x), _ptr(c), _ptr(norms), b, n, d, k, _ptr(labels), _ptr(best), _ptr(second))
    return (labels, best, second) if margins else labels


def update(x, labels, previous):
    """(sums, counts, means) from labels, sums accumulated in token order."""
    x, lab, prev = _f32(x), _i32(labels), _f32(previous)
    b, n, d = x.shape
    k = prev.shape[1]
    sums = np.empty_like(prev)
    counts = np.empty((b, k), np.int32)
    means = np.empty_like(prev)
    _lib().oracle_update(_ptr(x), _ptr(lab), _ptr(prev), b, n, d, k, _ptr(sums), _ptr(counts), _ptr(means))
    return sums, counts, means


def stable_sort(labels, clusters):
    """(indices [B,N], offsets [B,K+1]) of the stable argsort by label."""
    lab = _i32(labels)
    b, n = lab.shape
    idx = np.empty((b, n), np.int32)
    off = np.empty((b, clusters + 1), np.int32)
    _lib().oracle_stable_sort(_ptr(lab), b, n, clusters, _ptr(idx), _ptr(off))
    return idx, off


def kmeans_fit(x, init, iterations):
    """(labels, centers, counts, indices, offsets) after ``iterations`` Lloyd steps."""
    x, c0 = _f32(x), _f32(init)
    b, n, d = x.shape
    k = c0.shape[1]
    labels = np.empty((b, n), np.int32)
    centers = np.empty_like(c0)
    counts = np.empty((b, k), np.int32)
    idx = np.empty((b, n), np.int32)
    off = np.empty((b, k + 1), np.int32)
    _lib().oracle_kmeans_fit(_ptr(x), _ptr(c0), b, n, d, k, int(iterations), _ptr(labels), _ptr(centers),
                             _ptr(counts), _ptr(idx), _ptr(off))
    return labels, centers, counts, idx, off


def base_offset(x, labels, centroids, bits):
    """(codes uint8 [B,N,D], low [B,N], scale [B,N], xhat fp32 [B,N,D])."""
    x, lab, c = _f32(x), _i32(labels), _f32(centroids)
    b, n, d = x.shape
    k = c.shape[1]
    codes = np.empty((b, n, d), np.uint8)
    low = np.empty((b, n), np.float32)
    scale = np.empty((b, n), np.float32)
    xhat = np.empty((b, n, d), np.float32)
    _lib().oracle_base_offset(_ptr(x), _ptr(lab), _ptr(c), b, n, k, d, int(bits), _ptr(codes), _ptr(low),
                              _ptr(scale), _ptr(xhat))
    return codes, low, scale, xhat


def sparse_attention(q, k, v, dynamic_map, q_sizes, k_sizes):
    """Cluster-masked attention, float64 internally, float32 result [BH,SQ,D]."""
    q, k, v = _f32(q), _f32(k), _f32(v)
    bh, sq, d = q.shape
    sk = k.shape[1]
    m = np.ascontiguousarray(dynamic_map, dtype=np.uint8).reshape(bh, -1)
    qs = _i32(q_sizes).reshape(bh, -1)
    ks = _i32(k_sizes).reshape(bh, -1)
    cq, ck = qs.shape[1], ks.shape[1]
    out = np.empty_like(q)
    _lib().oracle_sparse_attention(_ptr(q), _ptr(k), _ptr(v), _ptr(m), _ptr(qs), _ptr(ks), bh, sq, sk, d, cq, ck,
                                   _ptr(out))
    return out
