"""GPU parity of IVF-Flat: list assignment, CSR layout, coarse probes and the list scan against
the CPU oracle (fp32 distances: 1e-4 relative, ids equal up to near-ties)."""
from __future__ import annotations

import numpy as np
import pytest

from tests.helpers import L2SQ, SENT, check_topk

pytestmark = pytest.mark.gpu


def rng(seed):
    return np.random.default_rng(seed)


def clustered(C, D, N, Q, seed, zipf=None):
    """configs[4] generator at reduced size: centroids N(0, 4^2), points = centroid + N(0,1),
    cluster sizes Zipf(s) over centroid ranks (uniform when zipf is None)."""
    g = rng(seed)
    c = (g.standard_normal((C, D)) * 4).astype(np.float32)
    if zipf is None:
        p = np.full(C, 1.0 / C)
    else:
        p = 1.0 / np.arange(1, C + 1) ** zipf
        p /= p.sum()
    lab = g.choice(C, N, p=p)
    x = (c[lab] + g.standard_normal((N, D))).astype(np.float32)
    ql = g.choice(C, Q, p=p)
    q = (c[ql] + g.standard_normal((Q, D))).astype(np.float32)
    return c, x, q


def _assignment_matches(oracle, x, c, gpu_lists):
    """GPU list ids equal the oracle's nearest centroid except for near-ties (1e-4 relative)."""
    ref = oracle.ivf_assign(x, c)
    bad = np.nonzero(ref != gpu_lists)[0]
    for i in bad:
        d_ref = oracle.distance(0, x[i], c[ref[i]])
        d_gpu = oracle.distance(0, x[i], c[gpu_lists[i]])
        scale = float((x[i].astype(np.float64) ** 2).sum() + (c[ref[i]].astype(np.float64) ** 2).sum())
        assert abs(d_gpu - d_ref) <= 1e-4 * scale, f"row {i}: gpu list {gpu_lists[i]} vs {ref[i]}"
    return len(bad)


def _lists_from_csr(off, ids, N):
    lists = np.empty(N, np.int64)
    for l in range(len(off) - 1):
        lists[ids[off[l]:off[l + 1]]] = l
    return lists


@pytest.mark.parametrize("C,D,N,Q,nprobe,k,zipf", [(16, 12, 800, 20, 4, 10, 1.1), (64, 96, 20000, 50, 8, 10, 1.1),
                                                    (256, 768, 30000, 64, 32, 10, 1.1),
                                                    (32, 40, 5000, 30, 32, 100, None)])
def test_ivf_build_probe_scan_match_oracle(ctx, oracle, C, D, N, Q, nprobe, k, zipf):
    from vectoraccelerate_amd import IVFSearchConfiguration, IVFSearchPipeline

    c, x, q = clustered(C, D, N, Q, C + N, zipf)
    pipe = IVFSearchPipeline(ctx, IVFSearchConfiguration(C, nprobe, D))
    st = pipe.prepareIndexStructure(c, x)
    off, ids = st.lists()
    lists = _lists_from_csr(off, ids, N)
    _assignment_matches(oracle, x, c, lists)
    # CSR: centroid order, insertion order inside each list (IVFStructure.swift:370-381)
    ooff, oids = oracle.ivf_csr(lists.astype(np.int32), C)
    np.testing.assert_array_equal(off, ooff)
    np.testing.assert_array_equal(ids, oids)
    # coarse probes: the nprobe nearest centroids by (L2^2, id) -- compared as a top-k
    probes = pipe.findNearestCentroids(q, st).cpu().numpy().view(np.uint32)
    op = oracle.ivf_probe(q, c, nprobe)
    check_topk(L2SQ, q, c, nprobe, probes, None, op, None)
    # list scan over the GPU's probes vs the oracle scan over the same probes and lists
    res = pipe.searchLists(q, st, probes, k)
    gi = res.indices.cpu().numpy().view(np.uint32)
    gd = res.distances.cpu().numpy()
    oi, od = oracle.ivf_scan(q, x, off, ids, probes, k)
    check_topk(L2SQ, q, x, k, gi, gd, oi, od)
    # the full search equals probe + scan
    full = pipe.search(q, st, k)
    np.testing.assert_array_equal(full.indices.cpu().numpy().view(np.uint32), gi)
    st.close()


def test_ivf_scan_overflow_path(ctx, oracle):
    from vectoraccelerate_amd import IVFSearchConfiguration, IVFSearchPipeline, _lib

    c, x, q = clustered(16, 32, 8000, 25, 7, 1.1)
    pipe = IVFSearchPipeline(ctx, IVFSearchConfiguration(16, 6, 32))
    st = pipe.prepareIndexStructure(c, x)
    off, ids = st.lists()
    probes = pipe.findNearestCentroids(q, st).cpu().numpy().view(np.uint32)
    try:
        ctx.set_option(_lib.VA_OPT_CANDIDATE_CAP, 16)
        res = pipe.searchLists(q, st, probes, 10)
    finally:
        ctx.set_option(_lib.VA_OPT_CANDIDATE_CAP, 0)
    oi, od = oracle.ivf_scan(q, x, off, ids, probes, 10)
    check_topk(L2SQ, q, x, 10, res.indices.cpu().numpy().view(np.uint32), res.distances.cpu().numpy(), oi, od)
    st.close()


def test_ivf_probe_edge_cases(ctx, oracle):
    """Sentinel / duplicate probes are skipped; too few candidates pad with sentinels."""
    from vectoraccelerate_amd import IVFSearchConfiguration, IVFSearchPipeline

    c, x, q = clustered(8, 16, 60, 4, 9)
    pipe = IVFSearchPipeline(ctx, IVFSearchConfiguration(8, 2, 16))
    st = pipe.prepareIndexStructure(c, x)
    off, ids = st.lists()
    probes = np.array([[0, 0], [1, SENT], [SENT, SENT], [7, 3]], np.uint32)
    res = pipe.searchLists(q, st, probes, 50)
    gi = res.indices.cpu().numpy().view(np.uint32)
    oi, od = oracle.ivf_scan(q, x, off, ids, np.array([[0, SENT], [1, SENT], [SENT, SENT], [7, 3]], np.uint32), 50)
    check_topk(L2SQ, q, x, 50, gi, res.distances.cpu().numpy(), oi, od)
    assert np.all(gi[2] == SENT)
    st.close()


def test_ivf_recall_vs_flat(ctx, oracle):
    """IVFValidationTests: recall against flat search grows with nprobe; nprobe = C is exact."""
    from vectoraccelerate_amd import FusedL2TopKKernel, IVFSearchConfiguration, IVFSearchPipeline

    c, x, q = clustered(32, 64, 10000, 40, 11)
    flat = FusedL2TopKKernel(ctx).findNearestNeighbors(q, x, 10)
    truth = [set(i for i, _ in r) for r in flat]
    recalls = []
    for nprobe in (1, 4, 32):
        pipe = IVFSearchPipeline(ctx, IVFSearchConfiguration(32, nprobe, 64))
        st = pipe.prepareIndexStructure(c, x)
        res = pipe.search(q, st, 10).allResults()
        recalls.append(np.mean([len(truth[i] & set(j for j, _ in res[i])) / 10 for i in range(len(res))]))
        st.close()
    assert recalls[0] <= recalls[1] <= recalls[2]
    assert recalls[2] == 1.0


@pytest.mark.parametrize("C,D,N0,adds", [(64, 48, 3000, [500, 1, 2500]), (7, 30, 1, [10, 1000]), (256, 96, 20000, [30000])])
def test_ivf_add_matches_rebuild(ctx, oracle, C, D, N0, adds):
    """va_ivf_add appends rows to their nearest lists: the CSR equals a build over all rows and
    searches agree with the rebuilt index."""
    import torch

    from vectoraccelerate_amd import IVFSearchConfiguration, IVFSearchPipeline

    N = N0 + sum(adds)
    print(f"ivf add C={C} D={D} N0={N0} adds={adds}", flush=True)
    c, x, q = clustered(C, D, N, 40, seed=C + D)[:3]
    pipe = IVFSearchPipeline(ctx, IVFSearchConfiguration(C, min(8, C), D))
    xd = ctx.buffer(x)
    st = pipe.prepareIndexStructure(c, xd[:N0])
    r0 = N0
    for n in adds:
        st.add(xd[r0:r0 + n], r0)
        r0 += n
    off, ids = st.lists()
    lists = oracle.ivf_assign(x, c)
    ooff, oids = oracle.ivf_csr(lists, C)
    np.testing.assert_array_equal(off, ooff)
    np.testing.assert_array_equal(ids, oids)
    full = pipe.prepareIndexStructure(c, xd)
    a = pipe.search(q, st, 10)
    b = pipe.search(q, full, 10)
    np.testing.assert_array_equal(a.indices.cpu().numpy(), b.indices.cpu().numpy())
    np.testing.assert_array_equal(a.distances.cpu().numpy(), b.distances.cpu().numpy())
    st.close()
    full.close()


def _search_mode(ctx, pipe, q, st, k, screen):
    """One search with VA_OPT_SCREEN = screen (0 automatic, 1 fp32 list scan only); returns the
    result and whether the list scan ran screened."""
    from vectoraccelerate_amd import _lib

    ctx.set_option(_lib.VA_OPT_SCREEN, screen)
    ctx.set_profiling(True)
    try:
        res = pipe.search(q, st, k)
        screened = ctx.last_scan_timings()["screened"]
    finally:
        ctx.set_profiling(False)
        ctx.set_option(_lib.VA_OPT_SCREEN, 0)
    return res, screened


# Shapes that reach every tile group of the screened scan: lists probed by a few queries (16-query
# tiles), by 17-32 (32-query tiles) and by many (64-query tiles, several query blocks per list);
# D not a multiple of 64 (zero-padded shadow rows) and a single 64-value chunk.  The full pass
# over lists probed by more than 32 queries runs on resident-query tiles (96 queries x 512 rows up
# to padded D = 768, 64 x 1024 above) with a ring of 1, 2, 3, 4 or 6 slots of 128 bytes per row
# (padded D = 64, 128, 192, 256, 768, 1024): lists of several row tiles, ragged last tiles and
# sub-tiles.
@pytest.mark.parametrize("C,D,N,Q,nprobe,k,zipf", [(256, 64, 40000, 64, 8, 10, 1.1),
                                                    (64, 96, 30000, 600, 4, 20, None),
                                                    (16, 128, 20000, 600, 4, 10, None),
                                                    (128, 100, 30000, 300, 8, 10, 1.1),
                                                    (48, 36, 12000, 200, 6, 50, 1.1),
                                                    (32, 768, 20000, 96, 32, 100, None),
                                                    (8, 256, 40000, 400, 4, 10, None),
                                                    (12, 180, 30000, 300, 3, 10, 1.1),
                                                    (16, 1000, 20000, 300, 4, 10, None)])
def test_ivf_screened_bit_identical_to_fp32(ctx, oracle, C, D, N, Q, nprobe, k, zipf):
    """The screened list scan (fp16 shadow rows on the fp16 MFMA, exact rerank with each list's
    fp32 arithmetic) returns the fp32 list scan's ids and distances bit for bit, and both match
    the oracle."""
    from vectoraccelerate_amd import IVFSearchConfiguration, IVFSearchPipeline

    c, x, q = clustered(C, D, N, Q, 7 * C + D, zipf)
    pipe = IVFSearchPipeline(ctx, IVFSearchConfiguration(C, nprobe, D))
    st = pipe.prepareIndexStructure(c, x)
    scr, on = _search_mode(ctx, pipe, q, st, k, 0)
    ref, off_ = _search_mode(ctx, pipe, q, st, k, 1)
    assert (on, off_) == (1, 0)
    si, ri = scr.indices.cpu().numpy().view(np.uint32), ref.indices.cpu().numpy().view(np.uint32)
    np.testing.assert_array_equal(si, ri)
    np.testing.assert_array_equal(scr.distances.cpu().numpy().view(np.uint32),
                                  ref.distances.cpu().numpy().view(np.uint32))
    off, ids = st.lists()
    probes = pipe.findNearestCentroids(q, st).cpu().numpy().view(np.uint32)
    oi, od = oracle.ivf_scan(q, x, off, ids, probes, k)
    check_topk(L2SQ, q, x, k, si, scr.distances.cpu().numpy(), oi, od)
    st.close()


def test_ivf_screened_after_add(ctx, oracle):
    """va_ivf_add rebuilds the fp16 shadow of the merged lists: the screened search still equals
    the fp32 list scan after rows are added."""
    from vectoraccelerate_amd import IVFSearchConfiguration, IVFSearchPipeline

    c, x, q = clustered(64, 64, 24000, 200, 17, 1.1)
    pipe = IVFSearchPipeline(ctx, IVFSearchConfiguration(64, 6, 64))
    xd = ctx.buffer(x)
    st = pipe.prepareIndexStructure(c, xd[:10000])
    st.add(xd[10000:], 10000)
    scr, on = _search_mode(ctx, pipe, q, st, 15, 0)
    ref, _ = _search_mode(ctx, pipe, q, st, 15, 1)
    assert on == 1
    np.testing.assert_array_equal(scr.indices.cpu().numpy(), ref.indices.cpu().numpy())
    np.testing.assert_array_equal(scr.distances.cpu().numpy().view(np.uint32),
                                  ref.distances.cpu().numpy().view(np.uint32))
    st.close()


def test_ivf_screened_large_entries_always_reranked(ctx):
    """Rows with entries beyond the fp16 range cannot be bounded: they are always candidates and
    their exact keys decide, so the screened search still equals the fp32 list scan."""
    from vectoraccelerate_amd import IVFSearchConfiguration, IVFSearchPipeline

    c, x, q = clustered(32, 64, 8000, 64, 23, None)
    g = rng(5)
    big = g.choice(8000, 200, replace=False)
    x[big] *= np.float32(3e4)  # some entries far beyond 65504
    q[:8] = x[big[:8]] * np.float32(1.0001)  # queries next to those rows
    pipe = IVFSearchPipeline(ctx, IVFSearchConfiguration(32, 4, 64))
    st = pipe.prepareIndexStructure(c, x)
    scr, on = _search_mode(ctx, pipe, q, st, 10, 0)
    ref, _ = _search_mode(ctx, pipe, q, st, 10, 1)
    assert on == 1
    np.testing.assert_array_equal(scr.indices.cpu().numpy(), ref.indices.cpu().numpy())
    np.testing.assert_array_equal(scr.distances.cpu().numpy().view(np.uint32),
                                  ref.distances.cpu().numpy().view(np.uint32))
    st.close()
