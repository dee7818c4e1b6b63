"""The fused selection + work list (peco_select_work) and the attention over it.

The selection launch writes, per map row, the kept-segment list of its key stream and, per
head, the attention items in cost order. Checked here against what the map defines:
- expanding a row's segments gives exactly the physical key rows of its kept clusters in
  cluster order (clamped cluster offsets, as the attention's own builder computes them), and
  segments are maximal (physically adjacent kept clusters share one);
- the items are every query cluster cut into chunks of at most 128 rows (256 when the query
  length is at least 65536: 8-wavefront attention workgroups), ordered by
  descending cost rows x stream length (cluster order beyond 2048 items), the builder's rule;
- the attention over this work list equals, bit for bit, the map-driven attention on the
  same inputs (indexed and packed inputs);
- the arrival counters are zero after every call, so the buffer serves the next call.
"""
import numpy as np
import pytest
import torch

from peco_amd import attention_cuda, clustering_cuda

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
INT_MAX = 2**31 - 1


def _gen(seed):
    g = torch.Generator()
    g.manual_seed(seed)
    return g


def _clamped_offsets(sizes, limit):
    pre = np.concatenate([[0], np.cumsum(np.maximum(sizes.astype(np.int64), 0))])
    return np.minimum(pre, limit)


def _expected_rows(map_row, koff):
    rows = []
    for j in np.nonzero(map_row)[0]:
        rows.extend(range(int(koff[j]), int(koff[j + 1])))
    return rows


def _segment_rows(seg_row):
    n, length = int(seg_row[0, 0]), int(seg_row[0, 1])
    segs = seg_row[1:1 + n]
    assert tuple(seg_row[1 + n]) == (0, INT_MAX)
    rows = []
    for i in range(n):
        delta, off = int(segs[i, 0]), int(segs[i, 1])
        end = int(segs[i + 1, 1]) if i + 1 < n else length
        assert end > off
        rows.extend(range(off + delta, end + delta))
    # Maximal: consecutive segments are never physically adjacent.
    deltas = segs[:, 0].astype(np.int64)
    assert np.all(np.diff(deltas) > 0)
    return rows, length


def _expected_items(qsizes, lengths, sq):
    qoff = _clamped_offsets(qsizes, sq)
    tile = 256 if sq >= 65536 else 128
    entries = []
    for c in range(len(qsizes)):
        rows = int(qoff[c + 1] - qoff[c])
        for ri, r in enumerate(range(0, rows, tile)):
            n = min(tile, rows - r)
            entries.append((min(n * int(lengths[c]), INT_MAX), c, ri, int(qoff[c]) + r, n))
    if len(entries) <= 2048:
        entries.sort(key=lambda e: (-e[0], e[1], e[2]))
    return [(e[3], e[1], e[4]) for e in entries]


def _selection_inputs(seed, h, cq, ck, dims, qmax, kmax, empty=True):
    g = _gen(seed)
    qc = torch.randn(1, h, cq, dims, generator=g) * 0.5
    kc = torch.randn(1, h, ck, dims, generator=g) * 0.5
    qs = torch.randint(0, qmax, (1, h, cq), generator=g, dtype=torch.int32)
    ks = torch.randint(0, kmax, (1, h, ck), generator=g, dtype=torch.int32)
    if empty:
        qs[0, 0, :3] = 0
        ks[0, -1, :5] = 0
    return qc, kc, qs, ks


def _check_work(work, emap, eqs, eks, sq, sk):
    m = emap.cpu().numpy().reshape(work.bh, work.rows, work.cols)
    qsz = eqs.cpu().numpy().reshape(work.bh, work.rows)
    ksz = eks.cpu().numpy().reshape(work.bh, work.cols)
    segs = work.segments().cpu().numpy()
    lengths = work.row_lengths().cpu().numpy()
    counts, items = (t.cpu().numpy() for t in work.items())
    assert not work.tickets().cpu().any(), "arrival counters must be left at zero"
    assert not work.queues().cpu().any(), "queue counters must be left at zero"
    for b in range(work.bh):
        koff = _clamped_offsets(ksz[b], sk)
        for r in range(work.rows):
            rows, length = _segment_rows(segs[b, r])
            assert rows == _expected_rows(m[b, r], koff), (b, r)
            assert length == len(rows) == lengths[b, r]
        want = _expected_items(qsz[b], lengths[b], sq)
        assert counts[b] == len(want)
        assert [tuple(int(x) for x in it) for it in items[b, :counts[b]]] == want


@pytest.mark.parametrize("p,ratio", [(1e-9, 0.25), (0.9, 0.0), (1.0, 0.0)])
@pytest.mark.parametrize("cq,ck,dims", [(20, 70, 128), (64, 256, 128), (9, 1000, 64)])
def test_select_work_matches_map(announce, p, ratio, cq, ck, dims):
    qc, kc, qs, ks = _selection_inputs(cq * 7 + ck + int(p * 10), 3, cq, ck, dims, 300, 40)
    video_q, video_k = qs.sum(-1).max().item(), ks.sum(-1).max().item()
    valid, text = 7, 9
    sq, sk = video_q + text, video_k + text
    minimum = int(np.ceil(ratio * ck))
    announce(f"p={p} ratio={ratio} CQ={cq} CK={ck} D={dims} sq={sq} sk={sk}")
    args = (qc.to(DEV), kc.to(DEV), qs.to(DEV), ks.to(DEV), p, minimum)
    emap, eqs, eks = clustering_cuda.select_connections(*args, text=(valid, text))
    work = clustering_cuda.select_work(*args, (valid, text), sq, sk)
    torch.cuda.synchronize()
    _check_work(work, emap, eqs, eks, sq, sk)


def test_select_work_without_text_and_clamped_sizes(announce):
    """No text partition, and key sizes whose sum exceeds sk (rows clamp as in the builder)."""
    qc, kc, qs, ks = _selection_inputs(5, 2, 12, 50, 128, 50, 30)
    sq = int(qs.sum(-1).max())
    sk = int(ks.sum(-1).min()) - 17
    announce(f"sq={sq} sk={sk}")
    args = (qc.to(DEV), kc.to(DEV), qs.to(DEV), ks.to(DEV), 0.7, 3)
    emap, _, _ = clustering_cuda.select_connections(*args)
    work = clustering_cuda.select_work(*args, None, sq, sk)
    torch.cuda.synchronize()
    _check_work(work, emap, qs.to(DEV), ks.to(DEV), sq, sk)


@pytest.mark.parametrize("cq,qmax", [(258, 1000), (4, 200000)])
def test_select_work_item_order_paths(announce, cq, qmax):
    """Many items: the bitonic sort (more than 512 items) and the cluster-order list (more than
    2048 items)."""
    qc, kc, qs, ks = _selection_inputs(cq, 1, cq, 64, 64, qmax, 50, empty=False)
    sq = int(qs.sum()) + 3
    sk = int(ks.sum()) + 3
    announce(f"CQ={cq} sq={sq}")
    args = (qc.to(DEV), kc.to(DEV), qs.to(DEV), ks.to(DEV), 0.5, 0)
    emap, eqs, eks = clustering_cuda.select_connections(*args, text=(3, 3))
    work = clustering_cuda.select_work(*args, (3, 3), sq, sk)
    torch.cuda.synchronize()
    count = int(work.items()[0][0])
    assert count > 512
    _check_work(work, emap, eqs, eks, sq, sk)


def _clustered_inputs(seed, h, cq, ck, video, text, d, dtype):
    g = _gen(seed)
    length = video + text
    q = torch.randn(1, h, length, d, generator=g).to(dtype)
    k = torch.randn(1, h, length, d, generator=g).to(dtype)
    v = torch.randn(1, h, length, d, generator=g).to(dtype)
    qs = torch.stack([torch.bincount(torch.randint(cq, (video,), generator=g), minlength=cq) for _ in range(h)])
    ks = torch.stack([torch.bincount(torch.randint(ck, (video,), generator=g), minlength=ck) for _ in range(h)])
    qidx = torch.stack([torch.randperm(video, generator=g) for _ in range(h)]).to(torch.int32)
    kidx = torch.stack([torch.randperm(video, generator=g) for _ in range(h)]).to(torch.int32)
    qc = torch.randn(1, h, cq, 64, generator=g)
    kc = torch.randn(1, h, ck, 64, generator=g)
    return q, k, v, qs.to(torch.int32)[None], ks.to(torch.int32)[None], qidx, kidx, qc, kc


@pytest.mark.parametrize("dtype,d", [(torch.bfloat16, 128), (torch.float16, 64)])
@pytest.mark.parametrize("indexed", [True, False])
def test_attention_over_work_equals_map_attention(announce, dtype, d, indexed):
    h, cq, ck, video, text, valid = 4, 24, 96, 3000, 40, 29
    q, k, v, qs, ks, qidx, kidx, qc, kc = _clustered_inputs(d + indexed, h, cq, ck, video, text, d, dtype)
    length = video + text
    announce(f"{dtype} D={d} indexed={indexed}")
    q, k, v, qidx, kidx = (t.to(DEV) for t in (q, k, v, qidx, kidx))
    args = (qc.to(DEV), kc.to(DEV), qs.to(DEV), ks.to(DEV), 0.6, 10)
    emap, eqs, eks, kept = clustering_cuda.select_connections(*args, text=(valid, text), with_kept=True)
    work = clustering_cuda.select_work(*args, (valid, text), length, length)
    if indexed:
        ref = attention_cuda.sparse_attention_indexed(q, k, v, emap, eqs, eks, qidx, kidx, video,
                                                      validate_sizes=False, kept_keys=kept)
        out = attention_cuda.sparse_attention_work(q, k, v, work, out_index=qidx, out_index_rows=video,
                                                   k_index=kidx)
    else:
        ref = attention_cuda.sparse_attention(q, k, v, emap, eqs, eks, validate_sizes=False, out_index=qidx,
                                              out_index_rows=video, kept_keys=kept)
        out = attention_cuda.sparse_attention_work(q, k, v, work, out_index=qidx, out_index_rows=video)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)
    # A second call on the same work list (its item queues reset by the first) gives the same.
    again = attention_cuda.sparse_attention_work(q, k, v, work, out_index=qidx, out_index_rows=video,
                                                 k_index=kidx if indexed else None)
    torch.cuda.synchronize()
    assert torch.equal(again, out)
    assert not work.tickets().cpu().any()
    assert not work.queues().cpu().any(), "the attention leaves its queue counters at zero"


def test_work_buffer_serves_consecutive_calls(announce):
    """The same shape twice with other selections (one buffer), then another query-cluster
    count (a second buffer); every list is checked."""
    for seed, cq in ((1, 20), (2, 20), (3, 33)):
        qc, kc, qs, ks = _selection_inputs(seed, 2, cq, 80, 128, 100, 40)
        sq, sk = 4000, 4000
        announce(f"seed={seed} CQ={cq}")
        args = (qc.to(DEV), kc.to(DEV), qs.to(DEV), ks.to(DEV), 0.5 + 0.1 * seed, 2)
        emap, eqs, eks = clustering_cuda.select_connections(*args, text=(5, 8))
        work = clustering_cuda.select_work(*args, (5, 8), sq, sk)
        torch.cuda.synchronize()
        _check_work(work, emap, eqs, eks, sq, sk)


def test_overwritten_work_list_is_rejected(announce):
    """A later select_work of the same shape on the same stream reuses the buffer: the
    earlier SelectionWork reports itself invalid and the attention refuses it, while the
    latest one (and one of another shape, with its own buffer) still runs."""
    h, cq, ck, video, text, valid, d = 2, 16, 48, 2000, 24, 24, 64
    q, k, v, qs, ks, qidx, kidx, qc, kc = _clustered_inputs(11, h, cq, ck, video, text, d, torch.bfloat16)
    length = video + text
    announce(f"H={h} N={video} CQ={cq} CK={ck}")
    q, k, v, qidx, kidx = (t.to(DEV) for t in (q, k, v, qidx, kidx))
    args = (qc.to(DEV), kc.to(DEV), qs.to(DEV), ks.to(DEV))
    first = clustering_cuda.select_work(*args, 0.6, 4, (valid, text), length, length)
    assert first.valid()
    second = clustering_cuda.select_work(*args, 0.8, 4, (valid, text), length, length)
    assert not first.valid() and second.valid()
    kw = dict(out_index=qidx, out_index_rows=video, k_index=kidx)
    with pytest.raises(RuntimeError, match="overwritten"):
        attention_cuda.sparse_attention_work(q, k, v, first, **kw)
    out = attention_cuda.sparse_attention_work(q, k, v, second, **kw)
    emap, eqs, eks, kept = clustering_cuda.select_connections(*args, 0.8, 4, text=(valid, text), with_kept=True)
    ref = attention_cuda.sparse_attention_indexed(q, k, v, emap, eqs, eks, qidx, kidx, video, validate_sizes=False,
                                                  kept_keys=kept)
    torch.cuda.synchronize()
    assert torch.equal(out, ref)


def _persistent_case(announce, seed, h, cq, ck, video, text, valid, d, indexed, check_items):
    q, k, v, qs, ks, qidx, kidx, qc, kc = _clustered_inputs(seed, h, cq, ck, video, text, d, torch.bfloat16)
    length = video + text
    announce(f"H={h} N={video} CQ={cq} CK={ck} D={d} indexed={indexed}")
    q, k, v, qidx, kidx = (t.to(DEV) for t in (q, k, v, qidx, kidx))
    args = (qc.to(DEV), kc.to(DEV), qs.to(DEV), ks.to(DEV), 1e-9, 100)
    emap, eqs, eks, kept = clustering_cuda.select_connections(*args, text=(valid, text), with_kept=True)
    work = clustering_cuda.select_work(*args, (valid, text), length, length)
    if check_items:
        # The items against the map (the segment lists are checked on smaller shapes above).
        counts, items = (t.cpu().numpy() for t in work.items())
        lengths = work.row_lengths().cpu().numpy()
        qsz = eqs.cpu().numpy().reshape(work.bh, work.rows)
        for b in range(work.bh):
            want = _expected_items(qsz[b], lengths[b], length)
            assert [tuple(int(x) for x in it) for it in items[b, :counts[b]]] == want
    kw = dict(out_index=qidx, out_index_rows=video)
    if indexed:
        ref = attention_cuda.sparse_attention_indexed(q, k, v, emap, eqs, eks, qidx, kidx, video,
                                                      validate_sizes=False, kept_keys=kept)
        kw["k_index"] = kidx
    else:
        ref = attention_cuda.sparse_attention(q, k, v, emap, eqs, eks, validate_sizes=False, kept_keys=kept, **kw)
    for _ in range(2):
        out = attention_cuda.sparse_attention_work(q, k, v, work, **kw)
        torch.cuda.synchronize()
        assert torch.equal(out, ref)
        assert not work.queues().cpu().any()
    return work


@pytest.mark.parametrize("indexed", [True, False])
def test_persistent_grid_equals_map_attention(announce, indexed):
    """A launch with at least 8 item slots per resident workgroup (16 heads x 32896 rows, 130 x
    514 extended map: 387 slots per head) runs the persistent grid, whose workgroups take items
    from one queue per XCD; it must equal the map-driven attention (one workgroup per item) bit
    for bit, twice on one work list (the first call resets the queues for the second)."""
    _persistent_case(announce, 7 + indexed, 16, 128, 512, 32640, 256, 200, 64, indexed, False)


@pytest.mark.parametrize("indexed,d", [(True, 128), (False, 128), (True, 64)])
def test_long_sequence_items_on_eight_wave_workgroups(announce, indexed, d):
    """At 65536 query rows and more, query clusters are cut into items of 256 rows, run by
    8-wavefront workgroups (4 heads x 65856 rows, 130 x 514 extended map): the items follow the
    map, and the persistent grid over them equals the one-workgroup-per-item grid of the
    map-driven attention bit for bit (items of up to 128 rows pair their waves over the two key
    halves of every tile, longer ones give each wave its own 32-row block)."""
    work = _persistent_case(announce, 11 + indexed + d, 4, 128, 512, 65600, 256, 200, d, indexed, True)
    counts, items = (t.cpu().numpy() for t in work.items())
    rows = np.concatenate([items[b, :counts[b], 2] for b in range(work.bh)])
    assert rows.max() == 256 and (rows <= 128).any() and ((rows > 128) & (rows < 256)).any()
