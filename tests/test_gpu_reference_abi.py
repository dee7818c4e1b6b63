"""The reference's own ctypes bindings against libpeco_hip.so, on the GPU.

The library is opened with a fresh ctypes handle whose argtypes are exactly those of the
reference's Python wrappers (peco/clustering_cuda.py:65-71, peco/attention_cuda.py:57-60),
and every call passes the buffers those wrappers allocate: the assign scratch
[chunk_size, C] and center_norms [B, C] (peco/clustering.py:59-61), the recompute sums
[B, C, D] (clustering.py:55), and the attention workspace of BH*(CK+2+3*(ceil(SQ/16)+CQ))
int32 (peco/attention_cuda.py:112-113,128). Results are compared with the oracle.
"""
import ctypes

import numpy as np
import pytest
import torch

from oracle import canonical, reference_path
from peco_amd import _native, workloads

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _reference_bound_library():
    lib = ctypes.CDLL(str(_native.LIB_PATH))
    pointer, integer = ctypes.c_void_p, ctypes.c_int
    lib.peco_assign_tokens_to_centers.argtypes = [pointer] * 5 + [integer] * 5 + [pointer]
    lib.peco_recompute_cluster_centers.argtypes = [pointer] * 6 + [integer] * 4 + [pointer]
    lib.peco_reorder_token_features.argtypes = [pointer] * 3 + [integer] * 5 + [pointer]
    for name in ("peco_assign_tokens_to_centers", "peco_recompute_cluster_centers", "peco_reorder_token_features"):
        getattr(lib, name).restype = integer
    lib.peco_cluster_error_message.argtypes = [integer]
    lib.peco_cluster_error_message.restype = ctypes.c_char_p
    lib.peco_sparse_attention.argtypes = [pointer] * 8 + [integer] * 7 + [pointer]
    lib.peco_sparse_attention.restype = integer
    lib.peco_attention_error_string.argtypes = [integer]
    lib.peco_attention_error_string.restype = ctypes.c_char_p
    return lib


def _p(t):
    return ctypes.c_void_p(t.data_ptr())


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def test_reference_bindings_assign_and_recompute(announce):
    """One Lloyd iteration through the two reference k-means symbols at the 480p Q shape
    (2 heads, 6750 tokens, 64 centres)."""
    lib = _reference_bound_library()
    wl = workloads.make_workload("hunyuan_480p", heads=2)
    n = wl.shape.video
    x = wl.query[0, :, :n].float().contiguous()
    c = wl.q_init.contiguous()
    b, k, d = c.shape
    chunk = min(1024, n)
    announce(f"assign/recompute B={b} N={n} K={k} D={d}")
    xg, cg = x.to(DEV), c.to(DEV)
    labels = torch.empty(b, n, dtype=torch.int32, device=DEV)
    scratch = torch.empty(chunk, k, device=DEV)
    norms = torch.empty(b, k, device=DEV)
    status = lib.peco_assign_tokens_to_centers(_p(xg), _p(cg), _p(labels), _p(scratch), _p(norms), b, n, d, k,
                                               chunk, _stream())
    assert status == 0, lib.peco_cluster_error_message(status)
    sums = torch.empty(b, k, d, device=DEV)
    counts = torch.empty(b, k, dtype=torch.int32, device=DEV)
    means = torch.empty(b, k, d, device=DEV)
    status = lib.peco_recompute_cluster_centers(_p(xg), _p(labels), _p(cg), _p(sums), _p(counts), _p(means), b, n,
                                                d, k, _stream())
    assert status == 0, lib.peco_cluster_error_message(status)
    torch.cuda.synchronize()
    ref_norms = canonical.center_norms(c.numpy())
    ref_labels = canonical.assign(x.numpy(), c.numpy(), ref_norms)
    rs, rc, rm = canonical.update(x.numpy(), ref_labels, c.numpy())
    assert np.array_equal(norms.cpu().numpy().view(np.int32), ref_norms.view(np.int32))
    assert np.array_equal(labels.cpu().numpy(), ref_labels)
    assert np.array_equal(counts.cpu().numpy(), rc)
    assert np.array_equal(sums.cpu().numpy().view(np.int32), rs.view(np.int32))
    assert np.array_equal(means.cpu().numpy().view(np.int32), rm.view(np.int32))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_reference_binding_sparse_attention(announce, dtype):
    """peco_sparse_attention, the reference's attention symbol, on the packed inputs of the
    480p layer (2 heads; Q/K/V in cluster order with the text rows appended, the extended
    map and sizes), with the reference-sized workspace, against the float64 oracle."""
    lib = _reference_bound_library()
    wl = workloads.make_workload("hunyuan_480p", heads=2)
    shape = wl.shape
    q, k, v = (t.to(dtype) for t in (wl.query, wl.key, wl.value))

    def fit(x, clusters, iterations, init):
        labels, centers, counts, _, _ = canonical.kmeans_fit(x.float().numpy(), init.numpy(), iterations)
        return torch.from_numpy(labels), torch.from_numpy(centers), torch.from_numpy(counts), iterations

    st = {}
    reference_path.peco_layer(q, k, v, num_q_centroids=shape.num_q_centroids, num_k_centroids=shape.num_k_centroids,
                              iterations=2, q_init=wl.q_init, k_init=wl.k_init, top_p=wl.top_p,
                              min_kc_ratio=wl.min_kc_ratio, bits=0, text_length=shape.text, valid_text=shape.text,
                              fit=fit, attention=lambda *a: a[0], stages=st)
    qp, kp, vp = (st[n].contiguous() for n in ("q_perm", "k_perm", "v_perm"))
    m, qs, ks = st["ext_map"].contiguous(), st["ext_q_sizes"].contiguous(), st["ext_k_sizes"].contiguous()
    batch, heads, sq, dim = qp.shape
    sk = kp.shape[2]
    cq, ck = qs.shape[-1], ks.shape[-1]
    stride = ck + 2 + 3 * ((sq + 15) // 16 + cq)
    announce(f"peco_sparse_attention {dtype} BH={batch * heads} S={sq} CQ={cq} CK={ck} workspace={stride}")
    tensors = [t.to(DEV) for t in (qp, kp, vp, m, qs, ks)]
    out = torch.empty_like(tensors[0])
    workspace = torch.empty(batch * heads * stride, dtype=torch.int32, device=DEV)
    status = lib.peco_sparse_attention(*(_p(t) for t in tensors), _p(out), _p(workspace), batch * heads, sq, sk, dim,
                                       cq, ck, 0 if dtype == torch.float16 else 1, _stream())
    assert status == 0, lib.peco_attention_error_string(status)
    torch.cuda.synchronize()
    ref = canonical.sparse_attention(qp[0].float().numpy(), kp[0].float().numpy(), vp[0].float().numpy(),
                                     m[0].numpy(), qs[0].numpy(), ks[0].numpy())
    err = np.abs(out[0].float().cpu().numpy() - ref)
    print(f"[reference ABI] {dtype}: max {err.max():.3e} mean {err.mean():.3e}", flush=True)
    assert err.max() <= 2e-2 and err.mean() <= 2e-3


def test_reference_binding_reorder_roundtrip(announce):
    lib = _reference_bound_library()
    g = torch.Generator().manual_seed(5)
    x = torch.randn(1, 3, 1000, 128, generator=g).bfloat16().to(DEV)
    idx = torch.stack([torch.randperm(1000, generator=g) for _ in range(3)]).to(torch.int32).to(DEV)
    announce("reorder forward + inverse")
    fwd = torch.empty_like(x)
    back = torch.empty_like(x)
    assert lib.peco_reorder_token_features(_p(x), _p(idx), _p(fwd), 3, 1000, 128, 2, 0, _stream()) == 0
    assert lib.peco_reorder_token_features(_p(fwd), _p(idx), _p(back), 3, 1000, 128, 2, 1, _stream()) == 0
    torch.cuda.synchronize()
    assert torch.equal(fwd[0].cpu(), x[0].cpu().gather(1, idx.long().cpu()[..., None].expand(-1, -1, 128)))
    assert torch.equal(back, x)
