"""GPU parity of the screened fp32 top-k (fp16 screening scan + exact fp32 rerank).

The screened search must return exactly what the fp32 filtering scan returns: the same ids
and the same fp32 distances, bit for bit, for every metric and for data that defeats the
screen (entries beyond the fp16 range, NaN rows, zero rows, tiny magnitudes, dense ties).
VA_OPT_SCREEN = 1 runs the fp32 scan only, 2 forces the screen wherever it applies.  One
shape per metric is also checked against the CPU oracle (1e-4 relative, ties within it).
"""
from __future__ import annotations

import numpy as np
import pytest

from tests.helpers import COSINE, DOT, L2, L2SQ, check_topk

pytestmark = pytest.mark.gpu


def _search(ctx, metric, q, x, k, screen):
    from vectoraccelerate_amd import FusedL2TopKKernel, FusedL2TopKParameters, Metric, _lib

    ctx.set_option(_lib.VA_OPT_SCREEN, screen)
    ctx.set_profiling(True)
    try:
        res = FusedL2TopKKernel(ctx).execute(ctx.buffer(q), ctx.buffer(x),
                                             FusedL2TopKParameters(q.shape[0], x.shape[0], q.shape[1], k),
                                             metric=Metric(metric))
        t = ctx.last_scan_timings()
    finally:
        ctx.set_option(_lib.VA_OPT_SCREEN, 0)
        ctx.set_profiling(False)
    return res.indices.cpu().numpy().view(np.uint32), res.distances.cpu().numpy(), t


def _same(ctx, metric, q, x, k, expect_screen=True):
    fi, fd, ft = _search(ctx, metric, q, x, k, 1)
    si, sd, st = _search(ctx, metric, q, x, k, 2)
    assert ft["screened"] == 0
    if expect_screen:
        assert st["screened"] == 1, st
    np.testing.assert_array_equal(si, fi)
    np.testing.assert_array_equal(sd.view(np.uint32), fd.view(np.uint32))
    return si, sd, st


def _unit(a):
    return (a / np.linalg.norm(a, axis=1, keepdims=True)).astype(np.float32)


@pytest.mark.parametrize("metric", [L2SQ, COSINE, DOT, L2])
@pytest.mark.parametrize("Q,N,D,k", [(300, 40000, 128, 10), (257, 20000, 1536, 100), (64, 50000, 100, 7),
                                     (5, 30000, 36, 1), (520, 33000, 768, 64)])
def test_screened_equals_fp32_scan(ctx, metric, Q, N, D, k):
    g = np.random.default_rng(Q * 7 + N + D + metric)
    x = g.standard_normal((N, D), dtype=np.float32)
    q = g.standard_normal((Q, D), dtype=np.float32)
    _, _, st = _same(ctx, metric, q, x, k)
    # the rerank is a thin band around the k-th distance, not a rescan
    assert st["rerank_rows"] <= Q * max(4 * k, k + 512), st


@pytest.mark.parametrize("metric", [L2SQ, COSINE, DOT, L2])
def test_screened_matches_oracle(ctx, oracle, metric):
    g = np.random.default_rng(11 + metric)
    x = g.standard_normal((30000, 96), dtype=np.float32)
    q = g.standard_normal((200, 96), dtype=np.float32)
    si, sd, _ = _same(ctx, metric, q, x, 20)
    oi, od = oracle.flat_topk(metric, q, x, 20)
    check_topk(metric, q, x, 20, si, sd, oi, od)


def test_cosine_headline_shape_small(ctx):
    """configs[1]'s data model (unit rows, queries = rows + N(0, 0.05) noise) at 1/10 scale."""
    g = np.random.default_rng(1)
    x = _unit(g.standard_normal((100000, 1536), dtype=np.float32))
    src = g.integers(0, x.shape[0], 256)
    q = _unit(x[src] + 0.05 * g.standard_normal((256, 1536), dtype=np.float32))
    si, sd, st = _same(ctx, COSINE, q, x, 100)
    np.testing.assert_array_equal(si[:, 0], src.astype(np.uint32))
    assert st["overflow_rows"] == 0 and st["rerank_rows"] < 256 * 400, st


@pytest.mark.parametrize("metric", [L2SQ, COSINE, DOT, L2])
def test_unscreenable_rows(ctx, metric):
    """Entries beyond fp16's range, NaN rows and zero rows must reach the exact rerank."""
    g = np.random.default_rng(5 + metric)
    x = g.standard_normal((40000, 64), dtype=np.float32)
    q = g.standard_normal((256, 64), dtype=np.float32)
    x[::997] *= 1e5            # |x| ~ 1e5 > 65504: fp16 overflow
    x[3::1999, 7] = np.nan     # NaN rows
    x[11::2999] = 0.0          # zero rows (cosine: FLT_MIN floor)
    x[17::3001] *= 1e-30       # tiny rows: fp16 underflow
    q[5] *= 1e5
    q[6] = 0.0
    _same(ctx, metric, q, x, 15)


@pytest.mark.parametrize("metric", [L2SQ, COSINE])
def test_dense_ties_and_near_ties(ctx, metric):
    """Many rows at nearly the same distance overflow the rerank band: exact fallback."""
    g = np.random.default_rng(9)
    base = g.standard_normal((1, 128), dtype=np.float32)
    x = np.repeat(base, 30000, axis=0) + 1e-4 * g.standard_normal((30000, 128), dtype=np.float32)
    x[::50] = base                     # exact duplicates: ties broken by index
    q = np.repeat(base, 200, axis=0) + 1e-3 * g.standard_normal((200, 128), dtype=np.float32)
    _same(ctx, metric, q.astype(np.float32), x.astype(np.float32), 40)


def test_screen_overflow_falls_back(ctx):
    """A tiny candidate capacity makes every screened list overflow: the chunked exact path."""
    from vectoraccelerate_amd import _lib

    g = np.random.default_rng(12)
    x = g.standard_normal((30000, 64), dtype=np.float32)
    q = g.standard_normal((200, 64), dtype=np.float32)
    ctx.set_option(_lib.VA_OPT_CANDIDATE_CAP, 64)
    try:
        _, _, st = _same(ctx, L2SQ, q, x, 30)
    finally:
        ctx.set_option(_lib.VA_OPT_CANDIDATE_CAP, 0)
    assert st["overflow_rows"] > 0, st


@pytest.mark.parametrize("rank", [1, 3, 0])
def test_screen_speculative_rank_checks(ctx, rank):
    """A threshold below the sample's k-th upper bound (rank 1 or 3, or the automatic rank): a
    query whose list holds fewer than k candidates, or whose k-th candidate upper bound exceeds
    the threshold, takes the exact fallback.  Half the queries have an exact copy on a sampled
    row (16,384 rows sampled of 60,000: stride 3), which puts their threshold at that row."""
    from vectoraccelerate_amd import _lib

    g = np.random.default_rng(40 + rank)
    x = g.standard_normal((60000, 64), dtype=np.float32)
    q = g.standard_normal((200, 64), dtype=np.float32)
    x[::3][:100] = q[:100]
    ctx.set_option(_lib.VA_OPT_SAMPLE_RANK, rank)
    try:
        _, _, st = _same(ctx, L2SQ, q, x, 30)
    finally:
        ctx.set_option(_lib.VA_OPT_SAMPLE_RANK, 0)
    if rank:
        assert st["overflow_rows"] > 0, st


def test_large_magnitudes_scale_exactly(ctx):
    """Query scaling is a power of two: large and small but finite data give the fp32 result."""
    g = np.random.default_rng(13)
    x = (g.standard_normal((30000, 256)) * 3e3).astype(np.float32)
    q = (g.standard_normal((300, 256)) * 1e-3).astype(np.float32)
    for metric in (L2SQ, DOT):
        _same(ctx, metric, q, x, 25)


@pytest.mark.parametrize("metric", [L2SQ, COSINE, DOT, L2])
def test_mixed_norms_and_large_k(ctx, metric):
    """Rows whose norms span twelve decades and a k of 1000: the bound's relative and absolute
    terms all matter, and the k-th distance sits deep in the distribution."""
    g = np.random.default_rng(21 + metric)
    x = g.standard_normal((40000, 96), dtype=np.float32)
    x *= (10.0 ** g.uniform(-6, 6, size=(40000, 1))).astype(np.float32)
    q = g.standard_normal((260, 96), dtype=np.float32)
    q *= (10.0 ** g.uniform(-3, 3, size=(260, 1))).astype(np.float32)
    _same(ctx, metric, q, x, 1000)


def test_cosine_anticorrelated_queries(ctx):
    """Queries pointing away from every row: the k-th cosine distance is near 2, where the
    pre-test's linear form does not hold and every row must pass."""
    g = np.random.default_rng(22)
    x = np.abs(g.standard_normal((30000, 64), dtype=np.float32)) + 0.1
    q = -np.abs(g.standard_normal((200, 64), dtype=np.float32)) - 0.1
    _same(ctx, COSINE, q, x, 50)
    # half the queries correlated, half anti-correlated, in one launch
    q[::2] *= -1.0
    _same(ctx, COSINE, q, x, 50)


@pytest.mark.parametrize("metric", [L2SQ, COSINE])
def test_duplicate_queries_and_rows_at_scale(ctx, metric):
    """Repeated queries and exact duplicate rows across the sample and the scan."""
    g = np.random.default_rng(23)
    base = g.standard_normal((3000, 128), dtype=np.float32)
    x = np.concatenate([base] * 12)  # 36,000 rows, every row 12 times
    q = np.repeat(base[:40], 7, axis=0) + 0.0  # 280 queries, each repeated 7 times
    si, sd, _ = _same(ctx, metric, q, x, 36)
    # the exact duplicates of the query's source row come first, in index order
    for r in range(0, 280, 7):
        np.testing.assert_array_equal(si[r, :12], (r // 7) + 3000 * np.arange(12))
