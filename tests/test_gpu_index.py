"""AcceleratedVectorIndex semantics on the GPU — restated from the reference's
FlatIndexSearchTests.swift, ValidationEdgeCaseTests.swift and IVF tests."""
from __future__ import annotations

import numpy as np
import pytest

from tests.helpers import L2SQ, check_topk

pytestmark = pytest.mark.gpu


@pytest.fixture
def flat4(ctx):
    from vectoraccelerate_amd import AcceleratedVectorIndex, IndexConfiguration

    return AcceleratedVectorIndex(IndexConfiguration.flat(dimension=4, capacity=100), ctx)


def test_results_are_ordered(flat4):
    """FlatIndexSearchTests.swift:101-138."""
    for v in ([3, 0, 0, 0], [1, 0, 0, 0], [2, 0, 0, 0], [0.5, 0, 0, 0], [4, 0, 0, 0]):
        flat4.insert(v)
    r = flat4.search([0, 0, 0, 0], k=5)
    assert r.count == 5
    np.testing.assert_allclose([x.distance for x in r.results], [0.25, 1, 4, 9, 16], atol=1e-3)


def test_ordering_with_negative_values_and_ties(flat4):
    """FlatIndexSearchTests.swift:141-170."""
    hs = [flat4.insert(v) for v in ([-2, 0, 0, 0], [1, 0, 0, 0], [-1, 0, 0, 0], [0, 0, 0, 0])]
    r = flat4.search([0, 0, 0, 0], k=4)
    np.testing.assert_allclose([x.distance for x in r.results], [0, 1, 1, 4], atol=1e-3)
    assert [x.id for x in r.results] == [hs[3], hs[1], hs[2], hs[0]]


def test_distance_is_l2_squared(flat4):
    """FlatIndexSearchTests.swift:577-672."""
    flat4.insert([3, 4, 0, 0])
    r = flat4.search([0, 0, 0, 0], k=1)
    assert r.results[0].distance == pytest.approx(25.0, abs=1e-3)
    assert r.results[0].euclideanDistance == pytest.approx(5.0, abs=1e-3)


def test_k_exceeding_count_and_empty_index(ctx, flat4):
    """ValidationEdgeCaseTests: k > count returns count; empty index returns nothing."""
    assert flat4.search([0, 0, 0, 0], k=3).count == 0
    for v in ([1, 0, 0, 0], [2, 0, 0, 0], [3, 0, 0, 0]):
        flat4.insert(v)
    assert flat4.search([0, 0, 0, 0], k=10).count == 3


def test_dimension_mismatch_throws(flat4):
    from vectoraccelerate_amd import VectorError

    with pytest.raises(VectorError) as e:
        flat4.insert([1, 2, 3])
    assert e.value.kind == "dimensionMismatch"
    flat4.insert([1, 2, 3, 4])
    with pytest.raises(VectorError):
        flat4.search([1, 2, 3], k=1)


def test_deleted_vectors_are_excluded_and_compaction_keeps_handles(ctx):
    from vectoraccelerate_amd import AcceleratedVectorIndex, IndexConfiguration

    g = np.random.default_rng(5)
    idx = AcceleratedVectorIndex(IndexConfiguration.flat(dimension=16, capacity=8), ctx)  # grows
    data = g.standard_normal((300, 16)).astype(np.float32)
    hs = idx.insert(vectors=data)
    q = data[10] + 0.01
    first = idx.search(q, k=5)
    assert first.results[0].id == hs[10]
    idx.remove([first.results[0].id, first.results[1].id])
    after = idx.search(q, k=5)
    assert hs[10] not in [r.id for r in after.results]
    assert [r.id for r in after.results][:3] == [r.id for r in first.results][2:5]
    assert idx.count == 298
    idx.compact()
    again = idx.search(q, k=3)
    assert [r.id for r in again.results] == [r.id for r in after.results][:3]
    assert idx.vector(hs[299]) == pytest.approx(data[299].tolist())


def test_batch_equals_sequential(ctx):
    from vectoraccelerate_amd import AcceleratedVectorIndex, IndexConfiguration

    g = np.random.default_rng(6)
    idx = AcceleratedVectorIndex(IndexConfiguration.flat(dimension=32, capacity=2000), ctx)
    idx.insert(vectors=g.standard_normal((2000, 32)).astype(np.float32))
    qs = g.standard_normal((9, 32)).astype(np.float32)
    batch = idx.search(queries=qs, k=7)
    for i, q in enumerate(qs):
        assert [r.id for r in idx.search(q, k=7).results] == [r.id for r in batch[i].results]


def test_filtered_search_iterative_fetch(ctx):
    """searchFiltered (AcceleratedVectorIndex.swift:1188-1265): doubling fetch until k pass."""
    from vectoraccelerate_amd import AcceleratedVectorIndex, IndexConfiguration

    g = np.random.default_rng(7)
    idx = AcceleratedVectorIndex(IndexConfiguration.flat(dimension=8, capacity=500), ctx)
    data = g.standard_normal((500, 8)).astype(np.float32)
    hs = [idx.insert(v, metadata={"even": i % 10 == 0}) for i, v in enumerate(data)]
    q = g.standard_normal(8).astype(np.float32)
    r = idx.search(q, k=5, filter=lambda h, m: m is not None and m["even"])
    assert r.count == 5
    want = np.argsort(((data[::10] - q) ** 2).sum(1), kind="stable")[:5] * 10
    assert [x.id for x in r.results] == [hs[i] for i in want]


def test_ivf_index_matches_oracle_and_routes(ctx, oracle):
    from tests.test_gpu_ivf import clustered
    from vectoraccelerate_amd import AcceleratedVectorIndex, IndexConfiguration

    c, x, q = clustered(32, 48, 6000, 20, 8, 1.1)
    idx = AcceleratedVectorIndex(IndexConfiguration.ivf(dimension=48, nlist=32, nprobe=4, capacity=1000), ctx)
    hs = idx.insert(vectors=x)
    assert [h.stableID for h in hs] == list(range(6000))
    idx.train(c)
    res = idx.search(queries=q, k=10)
    gi = np.array([[r.id.stableID for r in rr.results] for rr in res], np.uint32)
    gd = np.array([[r.distance for r in rr.results] for rr in res], np.float32)
    off, ids = idx.lists()
    probes = idx.probes(q)
    np.testing.assert_array_equal(probes, oracle.ivf_probe(q, c, 4))
    oi, od = oracle.ivf_scan(q, x, off, ids, probes, 10)
    check_topk(L2SQ, q, x, 10, gi, gd, oi, od)
    # routing threshold: below it the index answers exactly (flat)
    flat_ix = AcceleratedVectorIndex(IndexConfiguration.ivf(dimension=48, nlist=32, nprobe=4, capacity=1000,
                                                            routingThreshold=10**9), ctx)
    flat_ix.insert(vectors=x)
    flat_ix.train(c)
    flat = flat_ix.search(q[0], k=10)
    fi, fd = oracle.flat_topk(L2SQ, q[:1], x, 10)
    check_topk(L2SQ, q[:1], x, 10, np.array([[r.id.stableID for r in flat.results]], np.uint32),
               np.array([[r.distance for r in flat.results]], np.float32), fi, fd)
    flat_ix.close()
    idx.close()
