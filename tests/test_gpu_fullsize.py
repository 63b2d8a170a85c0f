"""Parity at the BASELINE configs' full sizes.

Each test builds the config's data on the GPU (torch generators; data plumbing only), runs the
search through the C ABI, and checks (a) size-independent properties over every query and (b) a
query subset against the CPU oracle over the full database (the oracle finishes it in seconds on
the box's cores).  Integer paths bit-exact; fp32 within the tolerance of tests/helpers.py.
"""
from __future__ import annotations

import sys

import numpy as np
import pytest

from tests.helpers import COSINE, L2SQ, SENT, check_topk, check_topk_exact

pytestmark = pytest.mark.gpu


def note(msg):
    print(f"[fullsize] {msg}", file=sys.stderr, flush=True)


def test_configs1_cosine_top100_full(ctx, oracle):
    """1,000,000 x 1536 normalised rows, Q=1024 noisy copies of rows, cosine top-100."""
    import torch
    from vectoraccelerate_amd import FusedL2TopKKernel, FusedL2TopKParameters, Metric

    N, D, Q, k = 1_000_000, 1536, 1024, 100
    g = torch.Generator(device="cuda").manual_seed(0)
    x = torch.randn(N, D, device="cuda", generator=g)
    x /= x.norm(dim=1, keepdim=True)
    gq = torch.Generator(device="cuda").manual_seed(1)
    src = torch.randint(0, N, (Q,), device="cuda", generator=gq)
    q = x[src] + 0.05 * torch.randn(Q, D, device="cuda", generator=gq)
    q = (q / q.norm(dim=1, keepdim=True)).contiguous()
    res = FusedL2TopKKernel(ctx).execute(q, x, FusedL2TopKParameters(Q, N, D, k), metric=Metric.cosine)
    gi = res.indices.cpu().numpy().view(np.uint32)
    gd = res.distances.cpu().numpy()
    note("configs[1] searched")
    # properties over all queries: the source row ranks first, rows sorted, no sentinel, unique
    np.testing.assert_array_equal(gi[:, 0], src.cpu().numpy())
    assert np.all(np.diff(gd, axis=1) >= 0)
    assert np.all(gi != SENT)
    assert all(len(set(r)) == k for r in gi)
    # batch == sequential for one query
    one = FusedL2TopKKernel(ctx).execute(q[7:8].contiguous(), x, FusedL2TopKParameters(1, N, D, k),
                                         metric=Metric.cosine)
    np.testing.assert_array_equal(one.indices.cpu().numpy().view(np.uint32)[0], gi[7])
    # the headline route: AcceleratedVectorIndex.search over the index's fp16 shadow (screen16_kernel),
    # bit for bit equal to va_fused_topk over the fp32 rows for all 1024 queries
    hi, hd, t = _index_search_full(ctx, x, q, COSINE, k)
    note(f"configs[1] index searched: {t}")
    assert t["screened"] == 2, t
    np.testing.assert_array_equal(hi, gi)
    np.testing.assert_array_equal(hd.view(np.uint32), gd.view(np.uint32))
    # oracle on 64 queries against the full database
    xh = x.cpu().numpy()
    qh = q.cpu().numpy()
    sub = np.arange(0, Q, Q // 64)
    oi, od = oracle.flat_topk(COSINE, qh[sub], xh, k)
    note("configs[1] oracle subset done")
    check_topk(COSINE, qh[sub], xh, k, hi[sub], hd[sub], oi, od)


def test_configs1_metric_wording_l2_top10_full(ctx, oracle):
    """The metric's own wording at configs[1]'s shape: flat L2^2 top-10 over 1,000,000 x 1536
    N(0,1) rows, Q=1024, through the index (screen16_kernel), bit for bit equal to the fp32-only
    scan, 64 queries against the oracle."""
    import torch
    from vectoraccelerate_amd import _lib

    N, D, Q, k = 1_000_000, 1536, 1024, 10
    g = torch.Generator(device="cuda").manual_seed(10)
    x = torch.randn(N, D, device="cuda", generator=g)
    gq = torch.Generator(device="cuda").manual_seed(11)
    src = torch.randint(0, N, (Q,), device="cuda", generator=gq)
    q = (x[src] + 0.3 * torch.randn(Q, D, device="cuda", generator=gq)).contiguous()
    hi, hd, t = _index_search_full(ctx, x, q, L2SQ, k)
    assert t["screened"] == 2, t
    np.testing.assert_array_equal(hi[:, 0], src.cpu().numpy())
    # the fp32-only scan of the same search
    from vectoraccelerate_amd.context import dptr

    fi = ctx.empty((Q, k), torch.int32)
    fd = ctx.empty((Q, k), torch.float32)
    ctx.set_option(_lib.VA_OPT_SCREEN, 1)
    try:
        ctx.order_after_torch()
        ctx.check(ctx.lib.va_fused_topk(ctx.handle, L2SQ, dptr(q), dptr(x), Q, N, D, k, dptr(fi), dptr(fd)),
                  "va_fused_topk")
        ctx.synchronize()
    finally:
        ctx.set_option(_lib.VA_OPT_SCREEN, 0)
    note("configs[1] L2 top-10: fp32 scan done")
    np.testing.assert_array_equal(hi, fi.cpu().numpy().view(np.uint32))
    np.testing.assert_array_equal(hd.view(np.uint32), fd.cpu().numpy().view(np.uint32))
    xh = x.cpu().numpy()
    qh = q.cpu().numpy()
    sub = np.arange(0, Q, Q // 64)
    oi, od = oracle.flat_topk(L2SQ, qh[sub], xh, k)
    check_topk(L2SQ, qh[sub], xh, k, hi[sub], hd[sub], oi, od)


def _index_search_full(ctx, x, q, metric, k):
    """Insert device rows x into a native index and search it once with profiling on:
    (handles, distances, profiling record)."""
    import ctypes as C

    import torch
    from vectoraccelerate_amd.context import dptr

    N, D = x.shape
    Q = q.shape[0]
    h = C.c_void_p()
    ctx.check(ctx.lib.va_index_create(ctx.handle, D, N, C.byref(h)), "va_index_create")
    try:
        ctx.order_after_torch()
        ctx.check(ctx.lib.va_index_insert(ctx.handle, h, dptr(x), N, None), "va_index_insert")
        hi = ctx.empty((Q, k), torch.int32)
        hd = ctx.empty((Q, k), torch.float32)
        ctx.set_profiling(True)
        try:
            ctx.check(ctx.lib.va_index_search(ctx.handle, h, metric, dptr(q), Q, k, dptr(hi), dptr(hd)),
                      "va_index_search")
            ctx.synchronize()
            t = ctx.last_scan_timings()
        finally:
            ctx.set_profiling(False)
    finally:
        ctx.lib.va_index_destroy(h)
    return hi.cpu().numpy().view(np.uint32), hd.cpu().numpy(), t


def test_configs2_int8_top10_full(ctx, oracle):
    """10,000,000 x 512 U(-1,1)*s_d, per-dimension affine int8, Q=4096, top-10, bit-exact."""
    import torch
    from vectoraccelerate_amd import ScalarQuantizationKernel

    N, D, Q, k = 10_000_000, 512, 4096, 10
    g = torch.Generator(device="cuda").manual_seed(2)
    s = torch.rand(D, device="cuda", generator=g) * 1.5 + 0.5
    x = (torch.rand(N, D, device="cuda", generator=g) * 2 - 1).mul_(s)
    qf = ((torch.rand(Q, D, device="cuda", generator=g) * 2 - 1) * s).contiguous()
    sq = ScalarQuantizationKernel(ctx)
    p = sq.computePerDimensionParameters(x)
    xc = sq.quantizePerDimension(x, p)
    qc = sq.quantizePerDimension(qf, p)
    note("configs[2] quantised")
    xh = x.cpu().numpy()
    mn, mx, sc, zp = oracle.sq_params_per_dim(xh)
    np.testing.assert_array_equal(p.min, mn)
    np.testing.assert_array_equal(p.max, mx)
    np.testing.assert_array_equal(p.scale, sc)
    np.testing.assert_array_equal(p.zeroPoint, zp)
    xch = xc.cpu().numpy()
    rows = np.r_[0:20000, N - 20000:N]
    np.testing.assert_array_equal(xch[rows], oracle.sq_quantize(xh[rows], sc, zp))
    np.testing.assert_array_equal(qc.cpu().numpy(), oracle.sq_quantize(qf.cpu().numpy(), sc, zp))
    del xh
    assert xch.min() == -128 and xch.max() >= 126
    gi, gd = sq.searchTopK(qc, xc, k)
    note("configs[2] searched")
    assert np.all(np.diff(gd, axis=1) >= 0)
    sub = np.arange(0, Q, Q // 64)
    oi, od = oracle.i8_topk(qc.cpu().numpy()[sub], xch, k)
    check_topk_exact(gi[sub], gd[sub], oi, od)


def test_configs3_binary_top100_full(ctx, oracle):
    """50,000,000 x 768-bit codes, Q=256, top-100 with ties to the lower id, bit-exact."""
    import torch
    from vectoraccelerate_amd import BinaryQuantizationKernel, HammingDistanceKernel

    N, W, Q, k = 50_000_000, 24, 256, 100
    # pack path at scale: sign bits of N(0,1) floats for the first 1M rows, checked bit-exactly
    g = torch.Generator(device="cuda").manual_seed(3)
    xf = torch.randn(1_000_000, 768, device="cuda", generator=g)
    packed = BinaryQuantizationKernel(ctx).pack(xf)
    np.testing.assert_array_equal(packed.cpu().numpy().view(np.uint32), oracle.bq_pack(xf.cpu().numpy()))
    del xf
    x = torch.empty(N, W, device="cuda", dtype=torch.int32)
    x[:1_000_000] = packed
    x[1_000_000:] = torch.randint(-2**31, 2**31 - 1, (N - 1_000_000, W), device="cuda", generator=g,
                                  dtype=torch.int32)
    q = torch.randint(-2**31, 2**31 - 1, (Q, W), device="cuda", generator=g, dtype=torch.int32)
    q[:4] = x[torch.tensor([5, 123456, 30_000_000, N - 1], device="cuda")]  # exact matches
    gi, gd = HammingDistanceKernel(ctx).nearestNeighbors(q, x, k)
    note("configs[3] searched")
    np.testing.assert_array_equal(gi[:4, 0], [5, 123456, 30_000_000, N - 1])
    assert np.all(gd[:4, 0] == 0)
    assert np.all(np.diff(gd.astype(np.int64), axis=1) >= 0)
    sub = np.r_[0:4, 4:Q:4][:64]
    xh = x.cpu().numpy().view(np.uint32)
    oi, od = oracle.hamming_topk(q.cpu().numpy().view(np.uint32)[sub], xh, k)
    check_topk_exact(gi[sub], gd[sub], oi, od)


def test_configs4_ivf_top10_full(ctx, oracle):
    """4096 centroids N(0,4^2), 4,000,000 points with Zipf(1.1) cluster sizes, Q=1024, nprobe 32."""
    import torch
    from tests.test_gpu_ivf import _assignment_matches
    from vectoraccelerate_amd import IVFSearchConfiguration, IVFSearchPipeline

    C, D, N, Q, nprobe, k = 4096, 768, 4_000_000, 1024, 32, 10
    g = torch.Generator(device="cuda").manual_seed(4)
    cen = torch.randn(C, D, device="cuda", generator=g) * 4.0
    p = 1.0 / torch.arange(1, C + 1, device="cuda", dtype=torch.float64) ** 1.1
    p = (p / p.sum()).float()
    x = cen[torch.multinomial(p, N, replacement=True, generator=g)] + torch.randn(N, D, device="cuda", generator=g)
    q = (cen[torch.multinomial(p, Q, replacement=True, generator=g)]
         + torch.randn(Q, D, device="cuda", generator=g)).contiguous()
    pipe = IVFSearchPipeline(ctx, IVFSearchConfiguration(C, nprobe, D))
    st = pipe.prepareIndexStructure(cen, x)
    off, ids = st.lists()
    note("configs[4] built")
    assert off[-1] == N and np.all(np.diff(off.astype(np.int64)) >= 0)
    assert np.array_equal(np.sort(ids), np.arange(N, dtype=np.uint32))
    # assignment of a row sample against the oracle (near-ties allowed)
    xh = x.cpu().numpy()
    ch = cen.cpu().numpy()
    lists = np.empty(N, np.int64)
    for l in range(C):
        lists[ids[off[l]:off[l + 1]]] = l
    rows = np.random.default_rng(0).choice(N, 20000, replace=False)
    _assignment_matches(oracle, xh[rows], ch, lists[rows])
    probes = pipe.findNearestCentroids(q, st).cpu().numpy().view(np.uint32)
    res = pipe.search(q, st, k)
    gi = res.indices.cpu().numpy().view(np.uint32)
    gd = res.distances.cpu().numpy()
    note("configs[4] searched")
    assert np.all(np.diff(gd, axis=1) >= 0)
    qh = q.cpu().numpy()
    sub = np.arange(0, Q, 64)
    op = oracle.ivf_probe(qh[sub], ch, nprobe)
    check_topk(L2SQ, qh[sub], ch, nprobe, probes[sub], None, op, None)
    oi, od = oracle.ivf_scan(qh[sub], xh, off, ids, probes[sub], k)
    check_topk(L2SQ, qh[sub], xh, k, gi[sub], gd[sub], oi, od)
    st.close()
    # End to end against the oracle alone, nothing taken from the device: the oracle's assignment
    # of every row, its lists, its probes and its scan, for 128 queries.
    olists = _oracle_assignment(oracle, x, cen, xh, ch)
    note("configs[4] oracle assignment")
    moved = np.nonzero(olists != lists)[0]
    if moved.size:  # rows the device placed in another list: near-ties only
        _assignment_matches(oracle, xh[moved], ch, lists[moved])
    ooff, oids = oracle.ivf_csr(olists, C)
    sub = np.arange(0, Q, Q // 128)
    op = oracle.ivf_probe(qh[sub], ch, nprobe)
    oi, od = oracle.ivf_scan(qh[sub], xh, ooff, oids, op, k)
    note("configs[4] oracle scan")
    # a query is comparable when the device probed the oracle's lists and none of their rows moved
    moved_lists = set(olists[moved].tolist()) | set(lists[moved].tolist())
    same = np.array([set(op[i].tolist()) == set(probes[s].tolist()) and not moved_lists & set(op[i].tolist())
                     for i, s in enumerate(sub)])
    note(f"configs[4] end to end: {moved.size} rows in another list, {same.sum()}/{len(sub)} queries compared")
    assert same.sum() >= len(sub) - 2, f"only {same.sum()} of {len(sub)} queries probe the oracle's lists"
    check_topk(L2SQ, qh[sub[same]], xh, k, gi[sub[same]], gd[sub[same]], oi[same], od[same])


def _oracle_assignment(oracle, x, cen, xh, ch, chunk=1 << 16):
    """vo_ivf_assign's list for every row of x (the nearest centroid in double precision, the lower
    index on ties), without its 4M x 4096 scalar pass: a float64 expanded-form pass on the device
    (torch's own GEMM, none of this library's kernels) settles every row whose two nearest
    centroids are more than 1e-9 (|x|^2 + |c|^2) apart, far beyond both computations' rounding
    (under 1e-12 of that scale at D = 768); vo_ivf_assign itself decides the rest."""
    import torch

    c64 = cen.double()
    ct = c64.t().contiguous()
    cn = (c64 * c64).sum(1)
    out = np.empty(x.shape[0], np.int64)
    unsure = []
    for s in range(0, x.shape[0], chunk):
        xb = x[s:s + chunk].double()
        xn = (xb * xb).sum(1)
        d = xn[:, None] + cn[None] - 2.0 * (xb @ ct)
        val, idx = torch.topk(d, 2, dim=1, largest=False)
        close = (val[:, 1] - val[:, 0]) <= 1e-9 * (xn + cn[idx[:, 0]])
        out[s:s + xb.shape[0]] = idx[:, 0].cpu().numpy()
        unsure.append(np.nonzero(close.cpu().numpy())[0] + s)
    unsure = np.concatenate(unsure)
    if unsure.size:
        out[unsure] = oracle.ivf_assign(xh[unsure], ch)
    return out
