"""peco_sparse_attention_noalloc, the allocation-free variant of peco_sparse_attention.

It takes no workspace: its work list lives in a static per-device array. Called through the
C-ABI twice in a row (the second call smaller, so the array still holds the first call's
larger work list) and compared bit for bit with peco_sparse_attention on the same inputs,
which runs the same kernels on a caller workspace.
"""
import ctypes

import pytest
import torch

from peco_amd import _native

DEV = "cuda:0"


def _partition(g, n, c, empty):
    cuts = torch.sort(torch.randint(n + 1, (c - 1,), generator=g)).values
    sizes = torch.diff(torch.cat([torch.tensor([0]), cuts, torch.tensor([n])]))
    sizes[:empty] = 0
    sizes[-1] += n - sizes.sum()
    return sizes.to(torch.int32)


def _case(seed, heads, sq, sk, cq, ck, dims, dtype):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(1, heads, sq, dims, generator=g).to(dtype)
    k = torch.randn(1, heads, sk, dims, generator=g).to(dtype)
    v = torch.randn(1, heads, sk, dims, generator=g).to(dtype)
    qs = torch.stack([_partition(g, sq, cq, 1) for _ in range(heads)])[None]
    ks = torch.stack([_partition(g, sk, ck, 2) for _ in range(heads)])[None]
    m = torch.rand(1, heads, cq, ck, generator=g) < 0.4
    return [t.to(DEV).contiguous() for t in (q, k, v, m, qs, ks)]


def _p(t):
    return ctypes.c_void_p(t.data_ptr())


def _both(lib, tensors):
    q, k, v, m, qs, ks = tensors
    _, heads, sq, dims = q.shape
    sk = k.shape[2]
    cq, ck = qs.shape[-1], ks.shape[-1]
    dtype = 1 if q.dtype == torch.bfloat16 else 0
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    ws = torch.empty(heads * (ck + 2 + 3 * ((sq + 15) // 16 + cq)), dtype=torch.int32, device=DEV)
    with_ws = torch.empty_like(q)
    status = lib.peco_sparse_attention(_p(q), _p(k), _p(v), _p(m), _p(qs), _p(ks), _p(with_ws), _p(ws), heads, sq,
                                       sk, dims, cq, ck, dtype, stream)
    assert status == 0, lib.peco_attention_error_string(status)
    static = torch.full_like(q, float("nan"))
    status = lib.peco_sparse_attention_noalloc(_p(q), _p(k), _p(v), _p(m), _p(qs), _p(ks), _p(static), heads, sq,
                                               sk, dims, cq, ck, dtype, stream)
    assert status == 0, lib.peco_attention_error_string(status)
    torch.cuda.synchronize()
    return with_ws, static


@pytest.mark.gpu
def test_noalloc_attention_matches_workspace_entry_twice(announce):
    lib = _native.library()
    cases = [(1, 6, 3000, 3400, 24, 70, 128, torch.bfloat16), (2, 2, 900, 700, 7, 13, 64, torch.float16)]
    for seed, heads, sq, sk, cq, ck, dims, dtype in cases:
        announce(f"noalloc seed={seed} heads={heads} sq={sq} sk={sk} cq={cq} ck={ck} D={dims} {dtype}")
        with_ws, static = _both(lib, _case(seed, heads, sq, sk, cq, ck, dims, dtype))
        assert torch.equal(static, with_ws), f"seed {seed}: outputs differ"


@pytest.mark.gpu
def test_noalloc_attention_rejects_problems_beyond_its_scratch(announce):
    """A work list larger than the static array returns status 20004 before any launch."""
    lib = _native.library()
    null = ctypes.c_void_p(0)
    announce("oversized problem")
    # 512 heads of 119056 rows with 258/1026 clusters: about 2.35 M int32 of work list.
    assert lib.peco_sparse_attention_workspace_size(512, 119056, 119056, 258, 1026) > (1 << 20)
    status = lib.peco_sparse_attention_noalloc(null, null, null, null, null, null, null, 512, 119056, 119056, 128,
                                               258, 1026, 1, null)
    assert status == 20004
    assert b"static scratch" in lib.peco_attention_error_string(status)
