"""The headline kernel, screen16_kernel, pinned to the oracle through va_index_search.

va_index_search with Q >= 192 over an index whose dimension is a multiple of 4 screens the
fp16 shadow written at insert (screen16_kernel; smaller batches screen16_small_kernel), reranks
a proven band exactly in fp32 and selects by (distance, slot).  Every family below runs through that route (asserted from the
profiling record: screened == 2) and is checked twice:
  * against the CPU oracle (vo_flat_topk, float64): distances within 1e-4 of the per-pair scale,
    ids equal rank by rank except for ties within that tolerance (tests/helpers.py);
  * bit for bit against the fp32-only scan (va_fused_topk with VA_OPT_SCREEN = 1) over the same
    rows, which is the result the screen must reproduce exactly.
The families are those that defeat an fp16 screen: entries beyond fp16's range, NaN, zero and
1e-30 rows, dense ties and near-ties, 1e5-scaled data, norms over twelve decades with k = 1000,
anti-correlated cosine queries and duplicate rows (reference: NumericalStabilityTests.swift:968-1035
for NaN / Inf propagation; AcceleratedVectorIndex.swift:1278-1374, searchBatchGPU, for the route).
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from tests.helpers import COSINE, DOT, L2, L2SQ, check_topk

pytestmark = pytest.mark.gpu


class _Index:
    """A native index over rows x, searched through the C ABI with any metric."""

    def __init__(self, ctx, x):
        from vectoraccelerate_amd.context import dptr

        self.ctx = ctx
        self.h = C.c_void_p()
        ctx.check(ctx.lib.va_index_create(ctx.handle, x.shape[1], x.shape[0], C.byref(self.h)), "va_index_create")
        xd = ctx.buffer(x)
        ctx.order_after_torch()
        ctx.check(ctx.lib.va_index_insert(ctx.handle, self.h, dptr(xd), x.shape[0], None), "va_index_insert")
        ctx.synchronize()

    def search(self, metric, q, k):
        """(handles, distances, profiling record) of one va_index_search."""
        import torch
        from vectoraccelerate_amd.context import dptr

        c = self.ctx
        qd = c.buffer(q)
        hi = c.empty((q.shape[0], k), torch.int32)
        hd = c.empty((q.shape[0], k), torch.float32)
        c.order_after_torch()
        c.set_profiling(True)
        try:
            c.check(c.lib.va_index_search(c.handle, self.h, metric, dptr(qd), q.shape[0], k, dptr(hi), dptr(hd)),
                    "va_index_search")
            c.synchronize()
            t = c.last_scan_timings()
        finally:
            c.set_profiling(False)
        return hi.cpu().numpy().view(np.uint32), hd.cpu().numpy(), t

    def close(self):
        self.ctx.lib.va_index_destroy(self.h)


def _fp32_scan(ctx, metric, q, x, k):
    from tests.test_gpu_native_index import _fused

    return _fused(ctx, metric, q, x, k, screen=1)


def _pinned(ctx, oracle, metric, q, x, k, oracle_rows=None, accum_double=True):
    """Index search (screen16) == fp32 scan bit for bit, and == the oracle within tolerance."""
    ix = _Index(ctx, x)
    try:
        gi, gd, t = ix.search(metric, q, k)
    finally:
        ix.close()
    assert t["screened"] == 2, t
    fi, fd = _fp32_scan(ctx, metric, q, x, k)
    np.testing.assert_array_equal(gi, fi)
    np.testing.assert_array_equal(gd.view(np.uint32), fd.view(np.uint32))
    sub = np.arange(q.shape[0]) if oracle_rows is None else oracle_rows
    oi, od = oracle.flat_topk(metric, q[sub], x, k, accum_double=accum_double)
    check_topk(metric, q[sub], x, k, gi[sub], gd[sub], oi, od)
    return gi, gd, t


def _unit(a):
    return (a / np.linalg.norm(a, axis=1, keepdims=True)).astype(np.float32)


# ---- small batches (Q < 192): screen16_small_kernel over the same shadow -----------------------
@pytest.mark.parametrize("Q", [1, 7, 32, 33, 64, 65, 100, 128, 129, 191])
@pytest.mark.parametrize("metric", [L2SQ, COSINE, DOT, L2])
def test_small_batches(ctx, oracle, metric, Q):
    """Every query-tile configuration of the small-batch screen and its partial last query block,
    over 40,003 rows (a partial last row tile) of a dimension that is not a multiple of the chunk."""
    g = np.random.default_rng(200 + Q + 7 * metric)
    x = g.standard_normal((40003, 200), dtype=np.float32)
    q = g.standard_normal((Q, 200), dtype=np.float32)
    _pinned(ctx, oracle, metric, q, x, 17)


@pytest.mark.parametrize("Q", [1, 50, 150])
@pytest.mark.parametrize("metric", [L2SQ, COSINE, DOT, L2])
def test_small_batches_unscreenable_rows(ctx, oracle, metric, Q):
    """The adversarial rows of test_unscreenable_rows through the small-batch screen."""
    g = np.random.default_rng(300 + Q + metric)
    x = g.standard_normal((40000, 64), dtype=np.float32)
    q = g.standard_normal((Q, 64), dtype=np.float32)
    x[::997] *= 1e5
    x[3::1999, 7] = np.nan
    x[11::2999] = 0.0
    x[17::3001] *= 1e-30
    q[0] *= 1e5
    if Q > 1:
        q[1] = 0.0
    _pinned(ctx, oracle, metric, q, x, 15, accum_double=metric != COSINE)


@pytest.mark.parametrize("Q", [1, 20, 100])
@pytest.mark.parametrize("metric", [L2SQ, COSINE])
def test_small_batches_mixed_norms_and_ties(ctx, oracle, metric, Q):
    """Norms over twelve decades with k = 1000, then dense near-ties, at small batch sizes."""
    g = np.random.default_rng(400 + Q + metric)
    x = g.standard_normal((40000, 96), dtype=np.float32)
    x *= (10.0 ** g.uniform(-6, 6, size=(40000, 1))).astype(np.float32)
    q = g.standard_normal((Q, 96), dtype=np.float32)
    _pinned(ctx, oracle, metric, q, x, 1000, oracle_rows=np.arange(0, Q, max(1, Q // 10)))
    base = g.standard_normal((1, 128), dtype=np.float32)
    x = (np.repeat(base, 30000, axis=0) + 1e-4 * g.standard_normal((30000, 128), dtype=np.float32)).astype(np.float32)
    x[::50] = base
    q = (np.repeat(base, Q, axis=0) + 1e-3 * g.standard_normal((Q, 128), dtype=np.float32)).astype(np.float32)
    _pinned(ctx, oracle, metric, q, x, 40)


@pytest.mark.parametrize("metric", [L2SQ, COSINE, DOT, L2])
def test_gaussian_rows(ctx, oracle, metric):
    g = np.random.default_rng(100 + metric)
    x = g.standard_normal((40000, 128), dtype=np.float32)
    q = g.standard_normal((256, 128), dtype=np.float32)
    _pinned(ctx, oracle, metric, q, x, 25)


@pytest.mark.parametrize("metric", [L2SQ, COSINE, DOT, L2])
def test_unscreenable_rows(ctx, oracle, metric):
    """fp16-overflow rows (|x| ~ 1e5 > 65504), NaN rows, zero rows, 1e-30 rows (fp16 underflow),
    a 1e5-scaled query and a zero query: each must reach the exact rerank."""
    g = np.random.default_rng(110 + metric)
    x = g.standard_normal((40000, 64), dtype=np.float32)
    q = g.standard_normal((256, 64), dtype=np.float32)
    x[::997] *= 1e5
    x[3::1999, 7] = np.nan
    x[11::2999] = 0.0
    x[17::3001] *= 1e-30
    q[5] *= 1e5
    q[6] = 0.0
    # Cosine of a 1e-30 row: its squared norm (~1e-59) underflows in fp32, so the reference's fp32
    # CPU path (AccelerateFallback.batchCosineSimilarity, Operations/AccelerateFallback.swift:209-237)
    # floors the denominator and reports distance 1, as the GPU does, while float64 sees the true
    # angle.  For cosine the oracle's fp32 port of that path is the reference here.
    gi, gd, _ = _pinned(ctx, oracle, metric, q, x, 15, accum_double=metric != COSINE)
    nan_rows = set(range(3, 40000, 1999))
    assert not nan_rows & set(gi.ravel().tolist())  # NaN keys order after every finite key


@pytest.mark.parametrize("metric", [L2SQ, COSINE])
def test_dense_ties_and_near_ties(ctx, oracle, metric):
    """30,000 rows within 1e-4 of one point (every 50th an exact duplicate of it): the rerank band
    overflows and the device fallback decides, ties by the lower slot."""
    g = np.random.default_rng(120)
    base = g.standard_normal((1, 128), dtype=np.float32)
    x = (np.repeat(base, 30000, axis=0) + 1e-4 * g.standard_normal((30000, 128), dtype=np.float32)).astype(np.float32)
    x[::50] = base
    q = (np.repeat(base, 200, axis=0) + 1e-3 * g.standard_normal((200, 128), dtype=np.float32)).astype(np.float32)
    _pinned(ctx, oracle, metric, q, x, 40)


@pytest.mark.parametrize("metric", [L2SQ, DOT])
def test_large_magnitudes(ctx, oracle, metric):
    """Rows of magnitude ~1e5 per entry, queries ~1e-3: the power-of-two query scale and the flagged
    rows (fp16 image beyond 65504) keep the result exact."""
    g = np.random.default_rng(130 + metric)
    x = (g.standard_normal((30000, 256)) * 1e5).astype(np.float32)
    q = (g.standard_normal((300, 256)) * 1e-3).astype(np.float32)
    _pinned(ctx, oracle, metric, q, x, 25)


@pytest.mark.parametrize("metric", [L2SQ, COSINE, DOT, L2])
def test_mixed_norms_large_k(ctx, oracle, metric):
    """Row norms over twelve decades, query norms over six, k = 1000."""
    g = np.random.default_rng(140 + metric)
    x = g.standard_normal((40000, 96), dtype=np.float32)
    x *= (10.0 ** g.uniform(-6, 6, size=(40000, 1))).astype(np.float32)
    q = g.standard_normal((260, 96), dtype=np.float32)
    q *= (10.0 ** g.uniform(-3, 3, size=(260, 1))).astype(np.float32)
    _pinned(ctx, oracle, metric, q, x, 1000, oracle_rows=np.arange(0, 260, 5))


def test_cosine_anticorrelated_queries(ctx, oracle):
    """Queries pointing away from every row (k-th cosine distance near 2), then half correlated
    and half anti-correlated in one launch."""
    g = np.random.default_rng(150)
    x = np.abs(g.standard_normal((30000, 64), dtype=np.float32)) + 0.1
    q = -np.abs(g.standard_normal((200, 64), dtype=np.float32)) - 0.1
    _pinned(ctx, oracle, COSINE, q, x, 50)
    q[::2] *= -1.0
    _pinned(ctx, oracle, COSINE, q, x, 50)


@pytest.mark.parametrize("metric", [L2SQ, COSINE])
def test_duplicate_rows_and_queries(ctx, oracle, metric):
    """Every row 12 times and every query 7 times: the duplicates of a query's source row come
    first, in slot order."""
    g = np.random.default_rng(160)
    base = g.standard_normal((3000, 128), dtype=np.float32)
    x = np.concatenate([base] * 12)
    q = np.repeat(base[:40], 7, axis=0) + 0.0
    gi, _, _ = _pinned(ctx, oracle, metric, q, x, 36)
    for r in range(0, 280, 7):
        np.testing.assert_array_equal(gi[r, :12], (r // 7) + 3000 * np.arange(12))


def test_headline_data_model_small(ctx, oracle):
    """configs[1]'s data model (unit rows, queries = rows + N(0, 0.05) noise, renormalised) at
    100,000 x 1536 with 256 queries, cosine top-100: the source row ranks first."""
    g = np.random.default_rng(170)
    x = _unit(g.standard_normal((100000, 1536), dtype=np.float32))
    src = g.integers(0, x.shape[0], 256)
    q = _unit(x[src] + 0.05 * g.standard_normal((256, 1536), dtype=np.float32))
    gi, _, t = _pinned(ctx, oracle, COSINE, q, x, 100, oracle_rows=np.arange(0, 256, 4))
    np.testing.assert_array_equal(gi[:, 0], src.astype(np.uint32))
    assert t["overflow_rows"] == 0, t
