"""The native IVF index (va_index_create_ivf / va_index_train / va_index_search) against the oracle.

Reference: AcceleratedVectorIndex.train (Index/AcceleratedVectorIndex.swift:406-446), routing
(:911-926), searchIVF / searchIVFBatch (:1378-1481).  The reference over-fetches k + deleted rows
(or 3k with a filter) and drops them on the host; here deleted slots are excluded inside the list
scan (its threshold samples and device fallback included), so the result is the exact top-k over
the live rows of each query's nprobe nearest lists however many rows are deleted.  The oracle side
of every check: vo_ivf_scan over the index's own lists with the deleted slots taken out.
"""
from __future__ import annotations

import numpy as np
import pytest

from tests.helpers import L2SQ, SENT, check_topk

pytestmark = pytest.mark.gpu


def _live_csr(off, ids, dead):
    """The CSR lists without the dead slots (order kept)."""
    keep = ~np.isin(ids, np.asarray(sorted(dead), np.uint32))
    lens = np.diff(off.astype(np.int64))
    list_of = np.repeat(np.arange(len(lens)), lens)
    new_lens = np.bincount(list_of[keep], minlength=len(lens))
    noff = np.concatenate([[0], np.cumsum(new_lens)]).astype(np.uint32)
    return noff, ids[keep]


def _search(idx, q, k):
    res = idx.search(queries=q, k=k)
    gi = np.full((q.shape[0], k), SENT, np.uint32)
    gd = np.full((q.shape[0], k), np.inf, np.float32)
    for r, rr in enumerate(res):
        gi[r, :rr.count] = [x.id.stableID for x in rr.results]
        gd[r, :rr.count] = [x.distance for x in rr.results]
    return gi, gd


def _check_against_lists(oracle, idx, x, q, k, dead=()):
    """Index results == vo_ivf_scan over the live rows of the index's own lists and probes."""
    off, ids = idx.lists()
    probes = idx.probes(q)
    noff, nids = _live_csr(off, ids, set(dead))
    gi, gd = _search(idx, q, k)
    oi, od = oracle.ivf_scan(q, x, noff, nids, probes, k)
    check_topk(L2SQ, q, x, k, gi, gd, oi, od)
    assert not set(gi.ravel().tolist()) & set(dead)
    return gi, gd


@pytest.fixture
def clustered():
    from tests.test_gpu_ivf import clustered as gen

    return gen


@pytest.mark.parametrize("screen", [0, 1])
def test_removing_more_than_max_k_nearest_rows_of_a_trained_ivf_index(ctx, oracle, clustered, screen):
    """More than 1024 of a query's nearest rows removed from a trained IVF index, no compaction:
    the search still returns k results equal to the oracle's over the live rows of the probed
    lists, through the screened list scan (screen 0) and the fp32 list scan (screen 1)."""
    from vectoraccelerate_amd import AcceleratedVectorIndex, IndexConfiguration, _lib

    c, x, q = clustered(16, 64, 40000, 8, 31)
    # every query sits in cluster 0's neighbourhood: its nearest rows are that cluster's
    q = (c[0] + 0.5 * np.random.default_rng(5).standard_normal((8, 64))).astype(np.float32)
    x[:6000] = (c[0] + np.random.default_rng(6).standard_normal((6000, 64))).astype(np.float32)
    idx = AcceleratedVectorIndex(IndexConfiguration.ivf(dimension=64, nlist=16, nprobe=3, capacity=1000), ctx)
    hs = idx.insert(vectors=x)
    idx.train(c)
    assert idx.isTrained and idx._use_ivf()
    d0 = ((x.astype(np.float64) - q[0]) ** 2).sum(1)
    near = np.argsort(d0, kind="stable")[:3000]
    assert idx.remove([hs[i] for i in near]) == 3000
    ctx.set_option(_lib.VA_OPT_SCREEN, screen)
    try:
        gi, _ = _check_against_lists(oracle, idx, x, q, 50, dead=near.tolist())
    finally:
        ctx.set_option(_lib.VA_OPT_SCREEN, 0)
    assert (gi != SENT).all()
    assert idx.count == 37000  # nothing was compacted
    idx.close()


def test_deletions_with_forced_overflow_take_the_masked_fallback(ctx, oracle, clustered):
    """A candidate cap of 64 sends every query to the device fallback, which must skip the deleted
    rows too (both list scans)."""
    from vectoraccelerate_amd import AcceleratedVectorIndex, IndexConfiguration, _lib

    c, x, q = clustered(24, 48, 20000, 40, 32, 1.1)
    idx = AcceleratedVectorIndex(IndexConfiguration.ivf(dimension=48, nlist=24, nprobe=5), ctx)
    hs = idx.insert(vectors=x)
    idx.train(c)
    dead = np.random.default_rng(7).choice(20000, 4000, replace=False)
    idx.remove([hs[i] for i in dead])
    ctx.set_option(_lib.VA_OPT_CANDIDATE_CAP, 64)
    try:
        for screen in (0, 1):
            ctx.set_option(_lib.VA_OPT_SCREEN, screen)
            _check_against_lists(oracle, idx, x, q, 30, dead=dead.tolist())
    finally:
        ctx.set_option(_lib.VA_OPT_CANDIDATE_CAP, 0)
        ctx.set_option(_lib.VA_OPT_SCREEN, 0)
    idx.close()


def test_insert_after_training_joins_nearest_lists_and_compact_rebuilds(ctx, oracle, clustered):
    """Rows inserted after training land at the end of their nearest lists (the lists equal the
    oracle's assignment + CSR over all rows); compact() drops the removed slots, rebuilds the lists
    from the trained centroids and keeps every handle."""
    from vectoraccelerate_amd import AcceleratedVectorIndex, IndexConfiguration

    c, x, q = clustered(20, 32, 9000, 25, 33, 1.1)
    idx = AcceleratedVectorIndex(IndexConfiguration.ivf(dimension=32, nlist=20, nprobe=4, capacity=100), ctx)
    hs = idx.insert(vectors=x[:5000])
    idx.train(c)
    hs += idx.insert(vectors=x[5000:])
    off, ids = idx.lists()
    ooff, oids = oracle.ivf_csr(oracle.ivf_assign(x, c), 20)
    np.testing.assert_array_equal(off, ooff)
    np.testing.assert_array_equal(ids, oids)
    _check_against_lists(oracle, idx, x, q, 10)
    dead = np.arange(0, 9000, 3)
    idx.remove([hs[i] for i in dead])
    before = _check_against_lists(oracle, idx, x, q, 10, dead=dead.tolist())
    idx.compact()
    live = np.setdiff1d(np.arange(9000), dead)
    off2, ids2 = idx.lists()  # slots of the compacted index: the live rows in order
    ooff2, oids2 = oracle.ivf_csr(oracle.ivf_assign(x[live], c), 20)
    np.testing.assert_array_equal(off2, ooff2)
    np.testing.assert_array_equal(ids2, oids2)
    after = _search(idx, q, 10)
    np.testing.assert_array_equal(after[0], before[0])  # the same handles, in the same order
    np.testing.assert_array_equal(after[1].view(np.uint32), before[1].view(np.uint32))
    idx.close()


def test_filtered_ivf_search_is_exact_over_the_probed_lists(ctx, oracle, clustered):
    """A filter on a trained IVF index: the k nearest rows of the probed lists that pass it (the
    reference over-fetches 3k and may return fewer); a filter that rejects every row of the probed
    lists returns what passes, after examining exactly the probed lists' live rows."""
    from vectoraccelerate_amd import AcceleratedVectorIndex, IndexConfiguration

    c, x, q = clustered(16, 32, 12000, 6, 34)
    idx = AcceleratedVectorIndex(IndexConfiguration.ivf(dimension=32, nlist=16, nprobe=2), ctx)
    hs = idx.insert(vectors=x)
    idx.train(c)
    idx.remove(hs[:100])
    off, ids = idx.lists()
    probes = idx.probes(q)
    for r in range(q.shape[0]):
        keep = lambda h, m: h.stableID % 7 == 0  # noqa: E731
        res = idx.search(q[r], k=40, filter=keep)
        assert not res.isExhaustive
        rows = np.concatenate([ids[off[p]:off[p + 1]] for p in probes[r]])
        rows = np.sort(rows[(rows % 7 == 0) & (rows >= 100)])
        noff = np.array([0, len(rows)], np.uint32)
        oi, od = oracle.ivf_scan(q[r:r + 1], x, noff, rows.astype(np.uint32), np.zeros((1, 1), np.uint32), 40)
        gi = np.array([[h.id.stableID for h in res.results]], np.uint32)
        gd = np.array([[h.distance for h in res.results]], np.float32)
        check_topk(L2SQ, q[r:r + 1], x, 40, gi, gd, oi, od)
    # nothing in the probed lists passes: every live row of them is examined, none returned
    res = idx.search(q[0], k=5, filter=lambda h, m: False)
    rows0 = np.concatenate([ids[off[p]:off[p + 1]] for p in probes[0]])
    assert res.count == 0 and res.candidatesSearched == int((rows0 >= 100).sum())
    idx.close()


def test_routing_threshold_and_training_on_the_device(ctx, oracle, clustered):
    """Below routingThreshold live vectors the index answers flat (exact over every row); above it
    the trained lists answer.  train() without centroids runs device k-means over the live rows."""
    from vectoraccelerate_amd import AcceleratedVectorIndex, IndexConfiguration

    c, x, q = clustered(8, 16, 4000, 10, 35)
    idx = AcceleratedVectorIndex(IndexConfiguration.ivf(dimension=16, nlist=8, nprobe=2, routingThreshold=3000), ctx)
    idx.insert(vectors=x[:2500])
    idx.train(seed=3)
    assert idx.isTrained and not idx._use_ivf()
    gi, gd = _search(idx, q, 10)
    oi, od = oracle.flat_topk(L2SQ, q, x[:2500], 10)
    check_topk(L2SQ, q, x[:2500], 10, gi, gd, oi, od)
    assert all(r.isExhaustive for r in idx.search(queries=q, k=3))
    idx.insert(vectors=x[2500:])
    assert idx._use_ivf()
    _check_against_lists(oracle, idx, x, q, 10)
    assert not any(r.isExhaustive for r in idx.search(queries=q, k=3))
    idx.close()


def test_k_above_max_k_is_rejected(ctx):
    """k > VA_MAX_K with more live rows than that: invalidInput (FusedL2TopKParameters rejects
    k > maxK, FusedL2TopKKernel.swift:57-79); k above the live count is clamped to it."""
    from vectoraccelerate_amd import AcceleratedVectorIndex, IndexConfiguration, VectorError

    g = np.random.default_rng(36)
    idx = AcceleratedVectorIndex(IndexConfiguration.flat(8, 2000), ctx)
    idx.insert(vectors=g.standard_normal((1100, 8)).astype(np.float32))
    with pytest.raises(VectorError) as e:
        idx.search(np.zeros(8, np.float32), k=1025)
    assert e.value.kind == "invalidInput"
    with pytest.raises(VectorError):
        idx.search(queries=np.zeros((2, 8), np.float32), k=1025)
    assert idx.search(np.zeros(8, np.float32), k=1024).count == 1024
    small = AcceleratedVectorIndex(IndexConfiguration.flat(8, 10), ctx)
    small.insert(vectors=g.standard_normal((5, 8)).astype(np.float32))
    assert small.search(np.zeros(8, np.float32), k=5000).count == 5
    idx.close()
    small.close()


def test_flat_filter_accepting_only_far_rows_uses_the_sorted_pass(ctx, oracle):
    """A filter that accepts only the 3 farthest of 60,000 rows: after rounds up to VA_MAX_K rows the
    rest are taken in one sorted pass, exact, examining each row at most once."""
    from vectoraccelerate_amd import AcceleratedVectorIndex, IndexConfiguration

    g = np.random.default_rng(37)
    x = g.standard_normal((60000, 24)).astype(np.float32)
    q = g.standard_normal(24).astype(np.float32)
    idx = AcceleratedVectorIndex(IndexConfiguration.flat(24, 60000), ctx)
    hs = idx.insert(vectors=x)
    idx.remove(hs[:10])
    d = ((x.astype(np.float64) - q) ** 2).sum(1)
    d[:10] = -1.0  # the removed rows are not candidates
    far = set(np.argsort(d, kind="stable")[-3:].tolist())
    res = idx.search(q, k=3, filter=lambda h, m: h.stableID in far)
    ok = np.array(sorted(far))
    oi, od = oracle.flat_topk(L2SQ, q[None], x[ok], 3)
    assert [h.id.stableID for h in res.results] == ok[oi[0]].tolist()
    np.testing.assert_allclose([h.distance for h in res.results], od[0], rtol=1e-4)
    assert res.candidatesSearched <= 59990
    idx.close()
