"""The search entry points queue their work and return without waiting on the host.

Overflowed queries are finished on the device (a fallback of five passes that recompute keys
with the scan's own arithmetic), so a search never reads a counter back: several searches can
be queued back to back on one context and synchronised once.  The fallback must give the same
bits as the scan's own path, including when whole databases tie."""
from __future__ import annotations

import time

import numpy as np
import pytest

from tests.helpers import COSINE, DOT, L2, L2SQ, check_topk, check_topk_exact

pytestmark = pytest.mark.gpu


def _dev(ctx, a):
    return ctx.buffer(np.ascontiguousarray(a))


def _out(ctx, Q, k, dtype):
    import torch

    return ctx.empty((Q, k), dtype)


def _fused(ctx, metric, qd, xd, Q, N, D, k):
    import torch

    idx, dist = _out(ctx, Q, k, torch.int32), _out(ctx, Q, k, torch.float32)
    ctx.order_after_torch()
    ctx.check(ctx.lib.va_fused_topk(ctx.handle, metric, qd.data_ptr(), xd.data_ptr(), Q, N, D, k, idx.data_ptr(),
                                    dist.data_ptr()), "va_fused_topk")
    return idx, dist


def _host(t, view=None):
    a = t.cpu().numpy()
    return a.view(view) if view else a


def test_search_returns_before_the_gpu_finishes(ctx):
    """A headline-shaped screened search (GPU time in milliseconds) returns long before its
    work is done: an event recorded on the context stream right after the call is pending."""
    import torch

    g = torch.Generator(device="cuda").manual_seed(3)
    Q, N, D, k = 1024, 1_000_000, 768, 100
    x = torch.randn(N, D, device="cuda", generator=g)
    q = torch.randn(Q, D, device="cuda", generator=g)
    torch.cuda.synchronize()
    _fused(ctx, L2SQ, q, x, Q, N, D, k)  # grows the scratch arena (a call may wait for that)
    ctx.synchronize()
    stream = ctx.torch_stream()
    pending = 0
    for _ in range(3):
        t0 = time.perf_counter()
        _fused(ctx, L2SQ, q, x, Q, N, D, k)
        host_ms = (time.perf_counter() - t0) * 1e3
        ev = torch.cuda.Event()
        ev.record(stream)
        pending += int(not ev.query())
        t1 = time.perf_counter()
        ctx.synchronize()
        total_ms = host_ms + (time.perf_counter() - t1) * 1e3
        print(f"fused top-k: call returned after {host_ms:.3f} ms, work done after {total_ms:.3f} ms", flush=True)
    assert pending == 3


def test_back_to_back_searches_match_oracle(ctx, oracle):
    """Five different searches queued on one context with no synchronisation between them (a
    screened fp32 search, a plain fp32 search with a forced overflow, int8, Hamming, PQ), then
    one synchronisation: each result equals the oracle's."""
    import torch

    from vectoraccelerate_amd import _lib

    rng = np.random.default_rng(8)
    # fp32, screened (Q >= 192) and plain (small Q, candidate cap forced small: overflow fallback)
    x = rng.standard_normal((30000, 96), dtype=np.float32)
    q1 = rng.standard_normal((256, 96), dtype=np.float32)
    q2 = rng.standard_normal((40, 96), dtype=np.float32)
    # int8 and binary codes
    xc = rng.integers(-128, 128, (20000, 64)).astype(np.int8)
    qc = rng.integers(-128, 128, (50, 64)).astype(np.int8)
    xb = rng.integers(0, 2**32, (25000, 8), dtype=np.uint64).astype(np.uint32)
    qb = rng.integers(0, 2**32, (30, 8), dtype=np.uint64).astype(np.uint32)
    # PQ: random codebooks, the oracle's codes
    M, K, Dp = 8, 64, 64
    xp = rng.standard_normal((15000, Dp), dtype=np.float32)
    qp = rng.standard_normal((20, Dp), dtype=np.float32)
    cb = rng.standard_normal((M, K, Dp // M), dtype=np.float32)
    codes = oracle.pq_encode(xp, cb, M, K)

    xd, q1d, q2d = _dev(ctx, x), _dev(ctx, q1), _dev(ctx, q2)
    xcd, qcd = _dev(ctx, xc), _dev(ctx, qc)
    xbd, qbd = _dev(ctx, xb.view(np.int32)), _dev(ctx, qb.view(np.int32))
    xpd, qpd, cbd, cd = _dev(ctx, xp), _dev(ctx, qp), _dev(ctx, cb), _dev(ctx, codes)
    i32, f32 = torch.int32, torch.float32
    o1 = (_out(ctx, 256, 20, i32), _out(ctx, 256, 20, f32))
    o2 = (_out(ctx, 40, 15, i32), _out(ctx, 40, 15, f32))
    o3 = (_out(ctx, 50, 10, i32), _out(ctx, 50, 10, i32))
    o4 = (_out(ctx, 30, 25, i32), _out(ctx, 30, 25, i32))
    o5 = (_out(ctx, 20, 12, i32), _out(ctx, 20, 12, f32))
    ctx.order_after_torch()
    L, p = ctx.lib, lambda t: t.data_ptr()  # noqa: E731
    try:
        ctx.check(L.va_fused_topk(ctx.handle, COSINE, p(q1d), p(xd), 256, 30000, 96, 20, p(o1[0]), p(o1[1])), "fused")
        ctx.set_option(_lib.VA_OPT_CANDIDATE_CAP, 64)
        ctx.set_option(_lib.VA_OPT_SAMPLE_ROWS, 2000)
        ctx.check(L.va_fused_topk(ctx.handle, L2, p(q2d), p(xd), 40, 30000, 96, 15, p(o2[0]), p(o2[1])), "fused")
        ctx.check(L.va_i8_scan_topk(ctx.handle, p(qcd), p(xcd), 50, 20000, 64, 10, p(o3[0]), p(o3[1])), "i8")
        ctx.set_option(_lib.VA_OPT_CANDIDATE_CAP, 0)
        ctx.set_option(_lib.VA_OPT_SAMPLE_ROWS, 0)
        ctx.check(L.va_hamming_topk(ctx.handle, p(qbd), p(xbd), 30, 25000, 8, 25, p(o4[0]), p(o4[1])), "hamming")
        ctx.check(L.va_pq_search(ctx.handle, p(qpd), 20, Dp, M, K, p(cbd), p(cd), 15000, 12, p(o5[0]), p(o5[1])), "pq")
    finally:
        ctx.set_option(_lib.VA_OPT_CANDIDATE_CAP, 0)
        ctx.set_option(_lib.VA_OPT_SAMPLE_ROWS, 0)
    ctx.synchronize()

    oi, od = oracle.flat_topk(COSINE, q1, x, 20)
    check_topk(COSINE, q1, x, 20, _host(o1[0], np.uint32), _host(o1[1]), oi, od)
    oi, od = oracle.flat_topk(L2, q2, x, 15)
    check_topk(L2, q2, x, 15, _host(o2[0], np.uint32), _host(o2[1]), oi, od)
    oi, od = oracle.i8_topk(qc, xc, 10)
    check_topk_exact(_host(o3[0], np.uint32), _host(o3[1]), oi, od)
    oi, od = oracle.hamming_topk(qb, xb, 25)
    check_topk_exact(_host(o4[0], np.uint32), _host(o4[1], np.uint32), oi, od)
    oi, od = oracle.pq_search(qp, cb, codes, M, K, 12)
    np.testing.assert_array_equal(_host(o5[0], np.uint32), oi)
    np.testing.assert_array_equal(_host(o5[1]).view(np.uint32), od.view(np.uint32))


def _with_cap(ctx, fn, cap, sample):
    """Run fn with a forced candidate cap and sample size; a forced cap also pins the threshold
    to the sample's k-th key (the rank that overflows a small cap most)."""
    from vectoraccelerate_amd import _lib

    ctx.set_option(_lib.VA_OPT_CANDIDATE_CAP, cap)
    ctx.set_option(_lib.VA_OPT_SAMPLE_ROWS, sample)
    ctx.set_option(_lib.VA_OPT_SAMPLE_RANK, 2**32 if cap else 0)
    ctx.set_profiling(True)
    try:
        r = fn()
        t = ctx.last_scan_timings()
    finally:
        ctx.set_option(_lib.VA_OPT_CANDIDATE_CAP, 0)
        ctx.set_option(_lib.VA_OPT_SAMPLE_ROWS, 0)
        ctx.set_option(_lib.VA_OPT_SAMPLE_RANK, 0)
        ctx.set_profiling(False)
    return r, t


@pytest.mark.parametrize("metric", [L2SQ, COSINE, DOT, L2])
@pytest.mark.parametrize("Q,N,D,k", [(37, 20011, 100, 10), (300, 9000, 36, 50), (8, 40000, 17, 130)])
def test_fallback_bit_identical_to_scan(ctx, metric, Q, N, D, k):
    """Every query overflows a tiny candidate list: the device fallback's ids and distances equal
    the unforced search's bit for bit (its keys replay the distance GEMM's MFMA sequence), on
    both the plain fp32 scan and the screened scan (Q >= 192)."""
    rng = np.random.default_rng(Q + N + D + metric)
    x = rng.standard_normal((N, D), dtype=np.float32)
    q = rng.standard_normal((Q, D), dtype=np.float32)
    qd, xd = _dev(ctx, q), _dev(ctx, x)

    def run():
        i, d = _fused(ctx, metric, qd, xd, Q, N, D, k)
        ctx.synchronize()
        return _host(i, np.uint32), _host(d)

    (ri, rd), rt = _with_cap(ctx, run, 0, 0)
    (fi, fd), ft = _with_cap(ctx, run, 64, 1500)
    assert rt["overflow_rows"] == 0 and ft["overflow_rows"] >= 0.9 * Q, (rt, ft)
    np.testing.assert_array_equal(fi, ri)
    np.testing.assert_array_equal(fd.view(np.uint32), rd.view(np.uint32))


def test_fallback_whole_database_ties(ctx, oracle):
    """Every row identical: every key ties, the tie list overflows and the id-edge pass keeps the
    k lowest ids (fp32, int8 and Hamming)."""
    import torch

    from vectoraccelerate_amd import _lib

    rng = np.random.default_rng(4)
    N, Q = 30000, 12
    x = np.repeat(rng.standard_normal((1, 48), dtype=np.float32), N, axis=0)
    q = rng.standard_normal((Q, 48), dtype=np.float32)
    qd, xd = _dev(ctx, q), _dev(ctx, x)

    def run():
        i, d = _fused(ctx, L2SQ, qd, xd, Q, N, 48, 40)
        ctx.synchronize()
        return _host(i, np.uint32)

    gi, t = _with_cap(ctx, run, 64, 2000)
    assert t["overflow_rows"] == Q
    np.testing.assert_array_equal(gi, np.tile(np.arange(40, dtype=np.uint32), (Q, 1)))

    xc = np.repeat(rng.integers(-128, 128, (1, 32)).astype(np.int8), N, axis=0)
    qc = rng.integers(-128, 128, (Q, 32)).astype(np.int8)
    qcd, xcd = _dev(ctx, qc), _dev(ctx, xc)

    def run8():
        i, d = _out(ctx, Q, 9, torch.int32), _out(ctx, Q, 9, torch.int32)
        ctx.order_after_torch()
        ctx.check(ctx.lib.va_i8_scan_topk(ctx.handle, qcd.data_ptr(), xcd.data_ptr(), Q, N, 32, 9, i.data_ptr(),
                                          d.data_ptr()), "i8")
        ctx.synchronize()
        return _host(i, np.uint32), _host(d)

    (gi, gd), t = _with_cap(ctx, run8, 64, 2000)
    assert t["overflow_rows"] == Q
    oi, od = oracle.i8_topk(qc, xc, 9)
    check_topk_exact(gi, gd, oi, od)

    xb = np.repeat(rng.integers(0, 2**32, (1, 4), dtype=np.uint64).astype(np.uint32), N, axis=0)
    qb = rng.integers(0, 2**32, (Q, 4), dtype=np.uint64).astype(np.uint32)
    qbd, xbd = _dev(ctx, qb.view(np.int32)), _dev(ctx, xb.view(np.int32))

    def runh():
        i, d = _out(ctx, Q, 33, torch.int32), _out(ctx, Q, 33, torch.int32)
        ctx.order_after_torch()
        ctx.check(ctx.lib.va_hamming_topk(ctx.handle, qbd.data_ptr(), xbd.data_ptr(), Q, N, 4, 33, i.data_ptr(),
                                          d.data_ptr()), "hamming")
        ctx.synchronize()
        return _host(i, np.uint32), _host(d, np.uint32)

    (gi, gd), t = _with_cap(ctx, runh, 64, 2000)
    assert t["overflow_rows"] == Q
    oi, od = oracle.hamming_topk(qb, xb, 33)
    check_topk_exact(gi, gd, oi, od)


def _ivf(ctx, C, D, N, Q, seed, zipf, add_first_id=None):
    from tests.test_gpu_ivf import clustered
    from vectoraccelerate_amd import IVFSearchConfiguration, IVFSearchPipeline

    c, x, q = clustered(C, D, N, Q, seed, zipf)
    pipe = IVFSearchPipeline(ctx, IVFSearchConfiguration(C, 8, D))
    xd = ctx.buffer(x)
    if add_first_id is None:
        st = pipe.prepareIndexStructure(c, xd)
        ids = np.arange(N, dtype=np.int64)
    else:  # the second half added with caller ids far above N
        h = N // 2
        st = pipe.prepareIndexStructure(c, xd[:h])
        st.add(xd[h:], add_first_id)
        ids = np.concatenate([np.arange(h), add_first_id + np.arange(N - h)]).astype(np.int64)
    return pipe, st, c, x, q, ids


@pytest.mark.parametrize("screen", [0, 1])
@pytest.mark.parametrize("added", [False, True])
def test_ivf_fallback_bit_identical_to_scan(ctx, added, screen):
    """IVF queries forced to overflow a tiny candidate list: the device fallback (which walks each
    overflowed query's probed lists with the arithmetic of the kernel that scanned each list,
    the 16-query tiles for lists few queries probe and the distance GEMM for the others) gives the
    unforced search's ids and distances bit for bit, also with row ids far above N, after the
    screened list scan (screen 0) and after the fp32 one (screen 1)."""
    from vectoraccelerate_amd import _lib

    pipe, st, c, x, q, ids = _ivf(ctx, 64, 96, 30000, 300, 5, 1.1, 3_000_000_000 if added else None)
    ctx.set_option(_lib.VA_OPT_SCREEN, screen)
    try:
        ref = pipe.search(q, st, 20)
        ctx.set_option(_lib.VA_OPT_CANDIDATE_CAP, 24)
        forced = pipe.search(q, st, 20)
    finally:
        ctx.set_option(_lib.VA_OPT_CANDIDATE_CAP, 0)
        ctx.set_option(_lib.VA_OPT_SCREEN, 0)
    ri, fi = ref.indices.cpu().numpy().view(np.uint32), forced.indices.cpu().numpy().view(np.uint32)
    np.testing.assert_array_equal(fi, ri)
    np.testing.assert_array_equal(forced.distances.cpu().numpy().view(np.uint32),
                                  ref.distances.cpu().numpy().view(np.uint32))
    assert np.isin(ri.astype(np.int64), ids).all()
    st.close()


def test_ivf_fallback_whole_list_ties(ctx, oracle):
    """Every row of a list equal to its centroid: all keys of a list tie, the tie lists overflow
    and the id-edge pass keeps the lowest ids, as the oracle's list scan does."""
    from tests.test_gpu_ivf import clustered
    from vectoraccelerate_amd import IVFSearchConfiguration, IVFSearchPipeline, _lib

    c, x, q = clustered(16, 32, 20000, 24, 11, 1.1)
    lab = oracle.ivf_assign(x, c)
    x = np.ascontiguousarray(c[lab])  # rows = their centroids (every list's keys tie)
    pipe = IVFSearchPipeline(ctx, IVFSearchConfiguration(16, 3, 32))
    st = pipe.prepareIndexStructure(c, x)
    off, ids = st.lists()
    probes = pipe.findNearestCentroids(q, st).cpu().numpy().view(np.uint32)
    ctx.set_option(_lib.VA_OPT_CANDIDATE_CAP, 16)
    try:
        res = pipe.searchLists(q, st, probes, 30)
    finally:
        ctx.set_option(_lib.VA_OPT_CANDIDATE_CAP, 0)
    oi, od = oracle.ivf_scan(q, x, off, ids, probes, 30)
    check_topk(L2SQ, q, x, 30, res.indices.cpu().numpy().view(np.uint32), res.distances.cpu().numpy(), oi, od)
    st.close()


def test_ivf_search_queues_behind_other_searches(ctx, oracle):
    """An IVF search between two flat searches on one context, one synchronisation at the end."""
    import torch

    from tests.test_gpu_ivf import clustered
    from vectoraccelerate_amd import IVFSearchConfiguration, IVFSearchPipeline

    c, x, q = clustered(64, 64, 20000, 200, 3, 1.1)
    pipe = IVFSearchPipeline(ctx, IVFSearchConfiguration(64, 8, 64))
    st = pipe.prepareIndexStructure(c, x)
    off, ids = st.lists()
    qd, xd = _dev(ctx, q), _dev(ctx, x)
    i1, d1 = _fused(ctx, L2SQ, qd, xd, 200, 20000, 64, 10)
    ii, di = _out(ctx, 200, 10, torch.int32), _out(ctx, 200, 10, torch.float32)
    pipe.encodeSearch(qd, st, ii, di, 10)
    i2, d2 = _fused(ctx, COSINE, qd, xd, 200, 20000, 64, 5)
    ctx.synchronize()
    oi, od = oracle.flat_topk(L2SQ, q, x, 10)
    check_topk(L2SQ, q, x, 10, _host(i1, np.uint32), _host(d1), oi, od)
    oi, od = oracle.flat_topk(COSINE, q, x, 5)
    check_topk(COSINE, q, x, 5, _host(i2, np.uint32), _host(d2), oi, od)
    probes = oracle.ivf_probe(q, c, 8)
    oi, od = oracle.ivf_scan(q, x, off, ids, probes, 10)
    check_topk(L2SQ, q, x, 10, _host(ii, np.uint32), _host(di), oi, od)
    st.close()


def test_profiling_levels(ctx):
    """Profiling level 2 records the scan phase alone (its two events): scan_ms of a screened
    search is set and equals its level-1 value within the run-to-run spread, while the other
    phases and the counts read 0; levels outside 0..2 are rejected.  The results are the same at
    every level."""
    from vectoraccelerate_amd import FusedL2TopKKernel, FusedL2TopKParameters, _lib

    rng = np.random.default_rng(11)
    N, D, Q, k = 60000, 256, 512, 20
    x = ctx.buffer(rng.standard_normal((N, D), dtype=np.float32))
    q = ctx.buffer(rng.standard_normal((Q, D), dtype=np.float32))
    kern = FusedL2TopKKernel(ctx)
    params = FusedL2TopKParameters(Q, N, D, k)
    out = {}
    for level in (1, 2, 0):
        ctx.set_profiling(level)
        try:
            r = kern.execute(q, x, params)
            ctx.synchronize()
            out[level] = (r.indices.cpu().numpy(), r.distances.cpu().numpy(),
                          ctx.last_scan_timings() if level else None)
        finally:
            ctx.set_profiling(False)
    t1, t2 = out[1][2], out[2][2]
    assert t1["sample_ms"] > 0 and t1["select_ms"] > 0 and t1["scan_ms"] > 0 and t1["rerank_rows"] > 0
    assert t2["scan_ms"] > 0 and t2["sample_ms"] == 0 and t2["select_ms"] == 0 and t2["rerank_rows"] == 0
    assert t2["total_ms"] == t2["scan_ms"]
    assert 0.2 < t2["scan_ms"] / t1["scan_ms"] < 5.0
    for level in (2, 0):
        np.testing.assert_array_equal(out[level][0], out[1][0])
        np.testing.assert_array_equal(out[level][1].view(np.uint32), out[1][1].view(np.uint32))
    assert ctx.lib.va_context_set_profiling(ctx.handle, 3) == _lib.VA_ERR_INVALID_ARG
    assert ctx.lib.va_context_set_profiling(ctx.handle, -1) == _lib.VA_ERR_INVALID_ARG
