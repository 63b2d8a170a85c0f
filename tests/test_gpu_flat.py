"""GPU parity of the fp32 path (distances, fused top-k, selection) against the CPU oracle.

All calls go through libva_hip.so's C ABI (via the host mirror classes).  Tolerances: fp32
distances within 1e-4 relative (per-pair scale, tests/helpers.py); top-k ids equal except
for ties within that tolerance; integer-valued selections bit-exact.
"""
from __future__ import annotations

import numpy as np
import pytest

from tests.helpers import COSINE, DOT, L2, L2SQ, SENT, check_topk, exact_distances

pytestmark = pytest.mark.gpu


def rng(seed):
    return np.random.default_rng(seed)


def _fused(ctx, metric, q, x, k):
    import torch
    from vectoraccelerate_amd import FusedL2TopKKernel, FusedL2TopKParameters, Metric

    kern = FusedL2TopKKernel(ctx)
    res = kern.execute(ctx.buffer(q), ctx.buffer(x), FusedL2TopKParameters(q.shape[0], x.shape[0], q.shape[1], k),
                       metric=Metric(metric))
    return res.indices.cpu().numpy().view(np.uint32), res.distances.cpu().numpy()


# ---------------------------------------------------------------------------------------
# distances
# ---------------------------------------------------------------------------------------
SHAPES = [(1, 1, 1), (3, 5, 7), (5, 129, 13), (33, 200, 64), (65, 300, 100), (130, 257, 768), (7, 1000, 1536)]


@pytest.mark.parametrize("Q,N,D", SHAPES)
def test_dot_all_pairs_matches_numpy(ctx, Q, N, D):
    from vectoraccelerate_amd import DotProductKernel

    g = rng(Q * 1000 + N + D)
    q = g.standard_normal((Q, D)).astype(np.float32)
    x = g.standard_normal((N, D)).astype(np.float32)
    got = DotProductKernel(ctx).compute(q, x)
    ref = q.astype(np.float64) @ x.T.astype(np.float64)
    scale = np.sqrt((q.astype(np.float64) ** 2).sum(1))[:, None] * np.sqrt((x.astype(np.float64) ** 2).sum(1))[None]
    assert np.all(np.abs(got - ref) <= 1e-5 * np.maximum(scale, 1e-30) + 1e-30), np.abs(got - ref).max()
    got_abs = DotProductKernel(ctx).compute(q, x, absoluteValue=True)
    np.testing.assert_array_equal(got_abs, np.abs(got))


@pytest.mark.parametrize("Q,N,D", SHAPES)
def test_l2_and_cosine_all_pairs_match_oracle(ctx, oracle, Q, N, D):
    from vectoraccelerate_amd import CosineSimilarityKernel, L2DistanceKernel

    g = rng(Q + N * 7 + D)
    q = g.standard_normal((Q, D)).astype(np.float32)
    x = g.standard_normal((N, D)).astype(np.float32)
    l2 = L2DistanceKernel(ctx).allPairs(q, x, computeSqrt=False)
    ref = oracle.distance_matrix("l2sq", q, x).astype(np.float64)
    scale = (q.astype(np.float64) ** 2).sum(1)[:, None] + (x.astype(np.float64) ** 2).sum(1)[None]
    assert np.all(np.abs(l2 - ref) <= 1e-4 * np.maximum(ref, scale)), np.abs(l2 - ref).max()
    cs = CosineSimilarityKernel(ctx).allPairs(q, x, outputDistance=True)
    ref_c = oracle.distance_matrix("cos_dist", q, x)
    assert np.all(np.abs(cs - ref_c) <= 1e-4), np.abs(cs - ref_c).max()


def test_pairs_match_oracle(ctx, oracle):
    from vectoraccelerate_amd import CosineSimilarityKernel, L2DistanceKernel

    for P, D in [(1, 1), (17, 3), (100, 768), (9, 1537)]:
        g = rng(P + D)
        q = g.standard_normal((P, D)).astype(np.float32)
        t = g.standard_normal((P, D)).astype(np.float32)
        for sq in (False, True):
            got = L2DistanceKernel(ctx).compute(q, t, computeSqrt=sq)
            np.testing.assert_allclose(got, oracle.l2_pairs(q, t, sq), rtol=1e-5)
        for od in (False, True):
            got = CosineSimilarityKernel(ctx).compute(q, t, outputDistance=od)
            np.testing.assert_allclose(got, oracle.cosine_pairs(q, t, od), rtol=1e-5, atol=1e-6)


def test_distance_known_answers(ctx):
    """NumericalStabilityTests.swift:354-420 on the GPU."""
    from vectoraccelerate_amd import CosineSimilarityKernel, DotProductKernel, L2DistanceKernel

    z = np.zeros((1, 128), np.float32)
    ones = np.ones((1, 128), np.float32)
    assert L2DistanceKernel(ctx).allPairs(z, z)[0, 0] == 0.0
    assert abs(L2DistanceKernel(ctx).allPairs(z, ones)[0, 0] - np.sqrt(128)) < 1e-4
    assert CosineSimilarityKernel(ctx).allPairs(z, z)[0, 0] == 0.0
    assert CosineSimilarityKernel(ctx).allPairs(z, ones / np.sqrt(128))[0, 0] == 0.0
    assert CosineSimilarityKernel(ctx).compute(z, z)[0] == 0.0
    assert DotProductKernel(ctx).compute(z, rng(0).standard_normal((1, 128)).astype(np.float32))[0, 0] == 0.0
    a = np.array([[1, 2, 3]], np.float32)
    assert abs(CosineSimilarityKernel(ctx).allPairs(a, a)[0, 0] - 1.0) < 1e-6
    assert abs(CosineSimilarityKernel(ctx).allPairs(a, -a)[0, 0] + 1.0) < 1e-6


def test_nan_propagates(ctx):
    """NumericalStabilityTests.swift:968-1035."""
    from vectoraccelerate_amd import CosineSimilarityKernel, DotProductKernel, L2DistanceKernel

    a = np.array([[1.0, np.nan, 3.0]], np.float32)
    b = np.array([[1.0, 2.0, 3.0]], np.float32)
    assert np.isnan(L2DistanceKernel(ctx).compute(a, b)[0])
    assert np.isnan(CosineSimilarityKernel(ctx).compute(a, b)[0])
    assert np.isnan(L2DistanceKernel(ctx).allPairs(a, b)[0, 0])
    assert np.isnan(CosineSimilarityKernel(ctx).allPairs(a, b)[0, 0])
    assert np.isnan(DotProductKernel(ctx).compute(a, b)[0, 0])


# ---------------------------------------------------------------------------------------
# fused top-k
# ---------------------------------------------------------------------------------------
def test_fused_topk_known_answers(ctx):
    """KernelTests.swift:806-835 and FlatIndexSearchTests.swift:101-172, 577-646."""
    from vectoraccelerate_amd import FusedTopKKernel

    k = FusedTopKKernel(ctx)
    res = k.findNearestNeighbors([[0, 0, 0, 0]], [[1, 0, 0, 0], [2, 0, 0, 0], [0.5, 0, 0, 0], [3, 0, 0, 0]], 2)
    assert [i for i, _ in res[0]] == [2, 0]
    np.testing.assert_allclose([d for _, d in res[0]], [0.25, 1.0], atol=1e-4)
    res = k.findNearestNeighbors([[0, 0, 0, 0]], [[-2, 0, 0, 0], [1, 0, 0, 0], [-1, 0, 0, 0], [0, 0, 0, 0]], 4)
    assert [i for i, _ in res[0]] == [3, 1, 2, 0]
    np.testing.assert_allclose([d for _, d in res[0]], [0, 1, 1, 4], atol=1e-4)
    assert abs(k.findNearestNeighbors([[0, 0, 0, 0]], [[3, 4, 0, 0]], 1)[0][0][1] - 25.0) < 1e-3
    assert abs(k.findNearestNeighbors([[0, 0, 0, 0]], [[1, 2, 3, 4]], 1)[0][0][1] - 30.0) < 1e-3
    assert abs(k.findNearestNeighbors([[4, 6, 8]], [[1, 2, 3]], 1)[0][0][1] - 50.0) < 1e-3
    v = [1.5, 2.5, 3.5, 4.5]
    assert k.findNearestNeighbors([v], [v], 1)[0][0][1] == pytest.approx(0.0, abs=1e-4)


def test_fused_topk_k_exceeds_n_pads_with_sentinels(ctx):
    from vectoraccelerate_amd import FusedTopKKernel

    res = FusedTopKKernel(ctx).findNearestNeighbors([[0.0, 0.0]], [[1.0, 0.0], [0.0, 2.0], [3.0, 0.0]], 5)
    assert [i for i, _ in res[0]] == [0, 1, 2]  # ValidationEdgeCaseTests: k > count returns count


def test_fused_topk_rejects_bad_parameters(ctx):
    from vectoraccelerate_amd import FusedL2TopKParameters, VectorError

    with pytest.raises(VectorError):
        FusedL2TopKParameters(1, 10, 4, 0)
    with pytest.raises(VectorError):
        FusedL2TopKParameters(0, 10, 4, 1)
    with pytest.raises(VectorError):
        FusedL2TopKParameters(1, 10, 4, 5000)


def test_config1_flat_l2_top10_matches_oracle(ctx, oracle):
    """BASELINE config 1 in full: 10,000 x 768 N(0,1) seed 0, Q=100 seed 1, L2^2, top-10."""
    x = np.random.default_rng(0).standard_normal((10000, 768), dtype=np.float32)
    q = np.random.default_rng(1).standard_normal((100, 768), dtype=np.float32)
    gi, gd = _fused(ctx, L2SQ, q, x, 10)
    oi, od = oracle.flat_topk(L2SQ, q, x, 10)
    check_topk(L2SQ, q, x, 10, gi, gd, oi, od)


@pytest.mark.parametrize("metric", [L2SQ, COSINE, DOT, L2])
@pytest.mark.parametrize("Q,N,D,k", [(1, 50, 16, 5), (40, 3000, 96, 10), (130, 20000, 64, 100), (7, 40000, 33, 1)])
def test_fused_topk_matches_oracle(ctx, oracle, metric, Q, N, D, k):
    g = rng(Q * 31 + N + D + metric)
    q = g.standard_normal((Q, D)).astype(np.float32)
    x = g.standard_normal((N, D)).astype(np.float32)
    gi, gd = _fused(ctx, metric, q, x, k)
    oi, od = oracle.flat_topk(metric, q, x, k)
    check_topk(metric, q, x, k, gi, gd, oi, od)


def _with_options(ctx, cap, sample):
    from vectoraccelerate_amd import _lib

    ctx.set_option(_lib.VA_OPT_CANDIDATE_CAP, cap)
    ctx.set_option(_lib.VA_OPT_SAMPLE_ROWS, sample)


@pytest.mark.parametrize("metric", [L2SQ, COSINE])
def test_sampled_threshold_path(ctx, oracle, metric):
    """Force the sample -> filter -> select path at a size the oracle finishes quickly."""
    g = rng(77 + metric)
    q = g.standard_normal((70, 48)).astype(np.float32)
    x = g.standard_normal((30000, 48)).astype(np.float32)
    try:
        _with_options(ctx, 0, 1000)
        gi, gd = _fused(ctx, metric, q, x, 20)
    finally:
        _with_options(ctx, 0, 0)
    oi, od = oracle.flat_topk(metric, q, x, 20)
    check_topk(metric, q, x, 20, gi, gd, oi, od)


@pytest.mark.parametrize("rank", [1, 2, 0])
def test_speculative_threshold_rank(ctx, oracle, rank):
    """A threshold below the sample's k-th key (rank 1 or 2, or the automatic rank) leaves some
    queries short of k candidates; the select lists them for the exact fallback."""
    from vectoraccelerate_amd import _lib

    g = rng(80 + rank)
    q = g.standard_normal((70, 48)).astype(np.float32)
    x = g.standard_normal((30000, 48)).astype(np.float32)
    x[::30][:35] = q[:35]  # exact matches at sampled rows (1000 rows: stride 30) for half the queries
    try:
        _with_options(ctx, 0, 1000)
        ctx.set_option(_lib.VA_OPT_SAMPLE_RANK, rank)
        gi, gd = _fused(ctx, L2SQ, q, x, 20)
    finally:
        _with_options(ctx, 0, 0)
        ctx.set_option(_lib.VA_OPT_SAMPLE_RANK, 0)
    oi, od = oracle.flat_topk(L2SQ, q, x, 20)
    check_topk(L2SQ, q, x, 20, gi, gd, oi, od)


def test_overflow_fallback_is_exact(ctx, oracle):
    """A tiny candidate capacity makes every query overflow: the chunked exact path must agree."""
    g = rng(78)
    q = g.standard_normal((9, 40)).astype(np.float32)
    x = g.standard_normal((25000, 40)).astype(np.float32)
    try:
        _with_options(ctx, 64, 2000)
        gi, gd = _fused(ctx, L2SQ, q, x, 30)
    finally:
        _with_options(ctx, 0, 0)
    oi, od = oracle.flat_topk(L2SQ, q, x, 30)
    check_topk(L2SQ, q, x, 30, gi, gd, oi, od)


def test_ties_go_to_lower_index(ctx):
    """Duplicate database rows: equal distances must come back in index order."""
    g = rng(79)
    base = g.standard_normal((50, 32)).astype(np.float32)
    x = np.concatenate([base] * 40)  # 2000 rows, every row repeated 40 times
    q = base[:3].copy()
    gi, gd = _fused(ctx, L2SQ, q, x, 40)
    for r in range(3):
        np.testing.assert_array_equal(gi[r], r + 50 * np.arange(40))


def test_nan_rows_rank_last(ctx):
    x = np.array([[np.nan, 0.0], [1.0, 0.0], [2.0, 0.0]], np.float32)
    gi, gd = _fused(ctx, L2SQ, np.zeros((1, 2), np.float32), x, 3)
    np.testing.assert_array_equal(gi[0], [1, 2, 0])


def test_batch_equals_sequential(ctx):
    """FlatIndexSearchTests: batch search equals per-query search."""
    g = rng(80)
    q = g.standard_normal((20, 64)).astype(np.float32)
    x = g.standard_normal((5000, 64)).astype(np.float32)
    bi, bd = _fused(ctx, L2SQ, q, x, 10)
    for r in (0, 7, 19):
        si, sd = _fused(ctx, L2SQ, q[r:r + 1], x, 10)
        np.testing.assert_array_equal(si[0], bi[r])
        np.testing.assert_array_equal(sd[0], bd[r])


# ---------------------------------------------------------------------------------------
# selection and merge
# ---------------------------------------------------------------------------------------
def test_topk_select_known_answers(ctx):
    """KernelTests.swift:621-671."""
    from vectoraccelerate_amd import Metal4SelectionMode, TopKSelectionKernel

    k = TopKSelectionKernel(ctx)
    r = k.select([[5, 2, 8, 1, 9, 3], [7, 4, 0.5, 6, 2.5, 1.5]], 3, Metal4SelectionMode.minimum)
    assert r == [[(3, 1.0), (1, 2.0), (5, 3.0)], [(2, 0.5), (5, 1.5), (4, 2.5)]]
    r = k.select([[5, 2, 8, 1, 9, 3]], 3, Metal4SelectionMode.maximum)
    assert r == [[(4, 9.0), (2, 8.0), (0, 5.0)]]
    r = k.selectSingle(list(range(100)), 5)
    assert [i for i, _ in r] == [0, 1, 2, 3, 4]


@pytest.mark.parametrize("rows,n,k", [(3, 10, 3), (13, 300, 17), (4, 100000, 100), (2, 5000, 1024), (5, 7, 9)])
def test_topk_select_matches_oracle_with_ties(ctx, oracle, rows, n, k):
    from vectoraccelerate_amd import Metal4SelectionMode, TopKSelectionKernel

    g = rng(rows * n + k)
    vals = g.integers(0, 50, size=(rows, n)).astype(np.float32)  # heavy ties
    vals[0, :3] = [np.nan, -np.inf, np.inf]
    for mode in (Metal4SelectionMode.minimum, Metal4SelectionMode.maximum):
        got = TopKSelectionKernel(ctx).select(vals, k, mode)
        oi, ov = oracle.topk_rows(vals, k, mode == Metal4SelectionMode.maximum)
        for r in range(rows):
            want = [(int(i), float(v)) for i, v in zip(oi[r], ov[r]) if i != SENT]
            gi = [i for i, _ in got[r]]
            assert gi == [i for i, _ in want], f"row {r} mode {mode}"
            np.testing.assert_array_equal([v for _, v in got[r]], [v for _, v in want])


def test_topk_merge_matches_oracle(ctx, oracle):
    import torch
    from vectoraccelerate_amd import TopKMergeKernel

    g = rng(81)
    Q, k = 6, 16
    a_d = np.sort(g.integers(0, 30, (Q, k)).astype(np.float32), axis=1)
    b_d = np.sort(g.integers(0, 30, (Q, k)).astype(np.float32), axis=1)
    a_i = np.tile(np.arange(k, dtype=np.uint32), (Q, 1))
    b_i = np.tile(np.arange(k, dtype=np.uint32), (Q, 1))
    a_i[0, -3:] = SENT
    a_d[0, -3:] = np.inf
    oi, od = oracle.topk_merge(a_i, a_d, b_i, b_d, 1000)
    dev = lambda a, dt: ctx.buffer(a.view(np.int32) if a.dtype == np.uint32 else a)
    out_i = ctx.empty((Q, k), torch.int32)
    out_d = ctx.empty((Q, k), torch.float32)
    ctx.order_after_torch()
    TopKMergeKernel(ctx).encode(dev(a_i, 0), dev(a_d, 0), dev(b_i, 0), dev(b_d, 0), out_i, out_d, Q, k, 1000)
    ctx.synchronize()
    np.testing.assert_array_equal(out_i.cpu().numpy().view(np.uint32), oi)
    np.testing.assert_array_equal(out_d.cpu().numpy(), od)


# ---------------------------------------------------------------------------------------
# streamed search over a host-resident database (chunked upload + running merge)
# ---------------------------------------------------------------------------------------
@pytest.mark.parametrize("metric", [L2SQ, COSINE, DOT, L2])
@pytest.mark.parametrize("Q,N,D,k,chunk", [(300, 50000, 128, 10, 7000), (64, 20011, 96, 50, 4096),
                                           (5, 3000, 40, 20, 7), (257, 40000, 768, 100, 0)])
def test_streamed_equals_resident(ctx, metric, Q, N, D, k, chunk):
    """The host-streamed search returns the resident search's ids and distances bit for bit,
    for chunk sizes that do not divide N and chunks smaller than k."""
    import torch
    from vectoraccelerate_amd import FusedL2TopKKernel, FusedL2TopKParameters, Metric

    g = rng(Q + N + D + metric)
    x = g.standard_normal((N, D)).astype(np.float32)
    q = g.standard_normal((Q, D)).astype(np.float32)
    kern = FusedL2TopKKernel(ctx)
    p = FusedL2TopKParameters(Q, N, D, k)
    ri, rd = _fused(ctx, metric, q, x, k)
    host = torch.from_numpy(x).pin_memory()
    res = kern.executeStreamed(ctx.buffer(q), host, p, Metric(metric), chunkRows=chunk)
    si = res.indices.cpu().numpy().view(np.uint32)
    sd = res.distances.cpu().numpy()
    np.testing.assert_array_equal(si, ri)
    np.testing.assert_array_equal(sd.view(np.uint32), rd.view(np.uint32))


def test_streamed_pageable_and_errors(ctx):
    import torch
    from vectoraccelerate_amd import FusedL2TopKKernel, FusedL2TopKParameters, Metric, VectorError

    g = rng(91)
    x = g.standard_normal((9000, 32)).astype(np.float32)
    q = g.standard_normal((10, 32)).astype(np.float32)
    kern = FusedL2TopKKernel(ctx)
    p = FusedL2TopKParameters(10, 9000, 32, 5)
    ri, rd = _fused(ctx, L2SQ, q, x, 5)
    res = kern.executeStreamed(ctx.buffer(q), torch.from_numpy(x), p, Metric(L2SQ), chunkRows=2500)  # pageable
    np.testing.assert_array_equal(res.indices.cpu().numpy().view(np.uint32), ri)
    with pytest.raises(VectorError):
        kern.executeStreamed(ctx.buffer(q), ctx.buffer(x), p, Metric(L2SQ))  # a device tensor is refused
