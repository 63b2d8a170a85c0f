"""MetalComputeProvider (Integration/MetalComputeProvider.swift:119-269) against the oracle.

batchDistance: euclidean = sqrt(L2^2), cosine = 1 - similarity, dotProduct = raw dot (VectorCore's
DotProductDistance through the BatchKernelProvider conformance: -dot).  findNearest: the
min(k, count) nearest as (index, distance), nearest first; dotProduct = largest dot first.
fp32 tolerance as everywhere (tests/helpers.py).
"""
from __future__ import annotations

import numpy as np
import pytest

from tests.helpers import COSINE, DOT, L2, check_topk

pytestmark = pytest.mark.gpu


@pytest.fixture
def data():
    g = np.random.default_rng(41)
    x = g.standard_normal((3000, 48)).astype(np.float32)
    q = g.standard_normal((5, 48)).astype(np.float32)
    return q, x


def test_batch_distance_semantics(ctx, oracle, data):
    from vectoraccelerate_amd import DotProductDistance, MetalComputeProvider

    q, x = data
    p = MetalComputeProvider(ctx)
    l2 = np.array(p.batchDistance(q[0], x, "euclidean"))
    np.testing.assert_allclose(l2, oracle.distance_matrix("l2sq", q[:1], x)[0] ** 0.5, rtol=1e-4)
    cs = np.array(p.batchDistance(q[0], x, "cosine"))
    np.testing.assert_allclose(cs, oracle.distance_matrix("cos_dist", q[:1], x)[0], atol=1e-4)
    dot = np.array(p.batchDistance(q[0], x, "dotProduct"))
    ref = x.astype(np.float64) @ q[0].astype(np.float64)
    scale = np.linalg.norm(x, axis=1) * np.linalg.norm(q[0])
    assert np.all(np.abs(dot - ref) <= 1e-4 * scale)
    np.testing.assert_array_equal(np.array(p.batchDistance(q[0], x, DotProductDistance())), -dot)
    m = np.array(p.distanceMatrix(q, x, "cosine"))
    assert m.shape == (5, 3000)
    np.testing.assert_array_equal(m[0], cs)
    assert p.batchDistance(q[0], x[:0], "euclidean") == []


@pytest.mark.parametrize("metric,va", [("euclidean", L2), ("cosine", COSINE), ("dotProduct", DOT)])
def test_find_nearest_matches_oracle(ctx, oracle, data, metric, va):
    from vectoraccelerate_amd import MetalComputeProvider

    q, x = data
    p = MetalComputeProvider(ctx)
    k = 12
    rows = p.findNearestBatch(q, x, k, metric)
    gi = np.array([[i for i, _ in r] for r in rows], np.uint32)
    gd = np.array([[d for _, d in r] for r in rows], np.float32)
    oi, od = oracle.flat_topk(va, q, x, k)
    check_topk(va, q, x, k, gi, -gd if metric == "dotProduct" else gd, oi, od)
    one = p.findNearest(q[2], x, k, metric)
    assert [i for i, _ in one] == gi[2].tolist()
    if metric == "dotProduct":
        assert all(a >= b for (_, a), (_, b) in zip(one, one[1:]))  # largest dot first


def test_find_nearest_edges_and_errors(ctx, data):
    from vectoraccelerate_amd import DotProductDistance, MetalComputeProvider, VectorError

    q, x = data
    p = MetalComputeProvider(ctx)
    assert len(p.findNearest(q[0], x[:7], 50, "euclidean")) == 7  # min(k, count)
    assert p.findNearest(q[0], x, 0, "euclidean") == []
    assert p.findNearest(q[0], x[:0], 3, "euclidean") == []
    vc = p.findNearest(q[0], x, 5, DotProductDistance())  # -dot, ascending
    assert all(a <= b for (_, a), (_, b) in zip(vc, vc[1:]))
    assert [i for i, _ in vc] == [i for i, _ in p.findNearest(q[0], x, 5, "dotProduct")]
    with pytest.raises(VectorError) as e:
        p.findNearest(q[0], x[:, :10], 3, "euclidean")
    assert e.value.kind == "invalidInput"
    for m in ("manhattan", "chebyshev"):
        with pytest.raises(VectorError) as e:
            p.batchDistance(q[0], x, m)
        assert e.value.kind == "unsupported"
