"""The native index (va_index_*) through the C ABI and its Python mirror.

Exactness: a search over an index with removed vectors returns what the fp32 scan returns over
the live vectors alone (same distances bit for bit, same order), whether or not the fp16 shadow
screens the scan; removals and filter rejections beyond VA_MAX_K never shorten a result
(reference: AcceleratedVectorIndex.swift:1103-1265 over-fetches k + deletedCount).
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

L2SQ, COSINE, DOT, L2 = 0, 1, 2, 3


def _fused(ctx, metric, q, x, k, screen):
    """va_fused_topk over x (fp32 scan when screen == 1)."""
    import torch
    from vectoraccelerate_amd import _lib
    from vectoraccelerate_amd.context import dptr

    ctx.set_option(_lib.VA_OPT_SCREEN, screen)
    try:
        qd, xd = ctx.buffer(q), ctx.buffer(x)
        idx = ctx.empty((q.shape[0], k), torch.int32)
        dist = ctx.empty((q.shape[0], k), torch.float32)
        ctx.order_after_torch()
        ctx.check(ctx.lib.va_fused_topk(ctx.handle, metric, dptr(qd), dptr(xd), q.shape[0], x.shape[0], q.shape[1], k,
                                        dptr(idx), dptr(dist)), "va_fused_topk")
        ctx.synchronize()
        return idx.cpu().numpy().view(np.uint32), dist.cpu().numpy()
    finally:
        ctx.set_option(_lib.VA_OPT_SCREEN, 0)


def _index_search(ix, q, k):
    import torch

    c = ix.context
    hd = c.empty((q.shape[0], k), torch.int32)
    dd = c.empty((q.shape[0], k), torch.float32)
    ix.searchDevice(c.buffer(q), k, hd, dd)
    c.synchronize()
    return hd.cpu().numpy().view(np.uint32), dd.cpu().numpy()


def _data(seed, n, d, q, normalise=False):
    g = np.random.default_rng(seed)
    x = g.standard_normal((n, d)).astype(np.float32)
    qs = (x[g.integers(0, n, q)] + 0.05 * g.standard_normal((q, d))).astype(np.float32)
    if normalise:
        x /= np.linalg.norm(x, axis=1, keepdims=True)
        qs /= np.linalg.norm(qs, axis=1, keepdims=True)
    return x, qs


@pytest.mark.parametrize("metric,name", [(L2SQ, "euclidean"), (COSINE, "cosine"), (DOT, "dotProduct")])
def test_index_search_equals_fp32_scan_over_live_rows(ctx, metric, name):
    """Shadow-screened index search (Q >= 192, sampled path) with 10 % of the rows removed."""
    from vectoraccelerate_amd import AcceleratedVectorIndex, IndexConfiguration

    x, q = _data(3 + metric, 50_000, 128, 256, normalise=metric == COSINE)
    ix = AcceleratedVectorIndex(IndexConfiguration.flat(128, 1000, metric=name), ctx)
    hs = ix.insert(vectors=x)
    k = 50
    # no removals: equal to the fp32 scan over all rows, and to the screened raw search
    gi, gd = _index_search(ix, q, k)
    fi, fd = _fused(ctx, metric, q, x, k, screen=1)
    np.testing.assert_array_equal(gi, fi)
    np.testing.assert_array_equal(gd.view(np.uint32), fd.view(np.uint32))
    g = np.random.default_rng(9)
    dead = np.sort(g.choice(x.shape[0], 5000, replace=False))
    assert ix.remove([hs[i] for i in dead]) == 5000
    live = np.setdiff1d(np.arange(x.shape[0]), dead)
    gi, gd = _index_search(ix, q, k)
    fi, fd = _fused(ctx, metric, q, x[live], k, screen=1)
    np.testing.assert_array_equal(gi, live[fi].astype(np.uint32))
    np.testing.assert_array_equal(gd.view(np.uint32), fd.view(np.uint32))
    # compaction keeps handles and results
    ix.compact()
    ci, cd = _index_search(ix, q, k)
    np.testing.assert_array_equal(ci, gi)
    np.testing.assert_array_equal(cd.view(np.uint32), gd.view(np.uint32))
    ix.close()


@pytest.mark.parametrize("metric,name", [(L2SQ, "euclidean"), (COSINE, "cosine"), (DOT, "dotProduct")])
def test_index_search_many_tiles_per_workgroup(ctx, metric, name):
    """More fp16-shadow tiles than workgroups (300 queries x 70,001 rows: 2 x 280 tiles of 256 x 256,
    partial in both directions, padding tiles included) and a dimension that is not a multiple of
    the 64-value stage: every workgroup of the persistent screen walks several tiles."""
    from vectoraccelerate_amd import AcceleratedVectorIndex, IndexConfiguration

    x, q = _data(40 + metric, 70_001, 136, 300, normalise=metric == COSINE)
    ix = AcceleratedVectorIndex(IndexConfiguration.flat(136, 1000, metric=name), ctx)
    ix.insert(vectors=x)
    k = 37
    gi, gd = _index_search(ix, q, k)
    fi, fd = _fused(ctx, metric, q, x, k, screen=1)
    np.testing.assert_array_equal(gi, fi)
    np.testing.assert_array_equal(gd.view(np.uint32), fd.view(np.uint32))
    # a second search on the same index and context (the workgroups' tile walk starts afresh)
    gi2, gd2 = _index_search(ix, q[:211], k)
    np.testing.assert_array_equal(gi2, fi[:211])
    np.testing.assert_array_equal(gd2.view(np.uint32), fd[:211].view(np.uint32))
    ix.close()


@pytest.mark.parametrize("k", [1, 1024])
@pytest.mark.parametrize("metric,name", [(L2SQ, "euclidean"), (COSINE, "cosine")])
def test_index_search_k_extremes(ctx, metric, name, k):
    """k = 1 and the largest k (1024) through the shadow screen, 520 queries (three query blocks,
    the last partial) over 40,000 rows: the sample rank, the candidate capacity and the rerank band
    at both ends."""
    from vectoraccelerate_amd import AcceleratedVectorIndex, IndexConfiguration

    x, q = _data(60 + metric, 40_000, 64, 520, normalise=metric == COSINE)
    ix = AcceleratedVectorIndex(IndexConfiguration.flat(64, 1000, metric=name), ctx)
    ix.insert(vectors=x)
    gi, gd = _index_search(ix, q, k)
    fi, fd = _fused(ctx, metric, q, x, k, screen=1)
    np.testing.assert_array_equal(gi, fi)
    np.testing.assert_array_equal(gd.view(np.uint32), fd.view(np.uint32))
    ix.close()


@pytest.mark.parametrize("metric,name", [(L2SQ, "euclidean"), (COSINE, "cosine")])
def test_index_search_overflow_through_the_shadow_screen(ctx, metric, name):
    """A forced candidate cap of 64 (and the sample's k-th key as the threshold) overflows the
    screen's lists: the appends stop at the cap, the overflowed queries finish in the device
    fallback, and the result still equals the fp32 scan's."""
    from vectoraccelerate_amd import AcceleratedVectorIndex, IndexConfiguration, _lib

    x, q = _data(70 + metric, 30_000, 64, 300, normalise=metric == COSINE)
    ix = AcceleratedVectorIndex(IndexConfiguration.flat(64, 1000, metric=name), ctx)
    ix.insert(vectors=x)
    k = 40
    ctx.set_option(_lib.VA_OPT_CANDIDATE_CAP, 64)
    ctx.set_option(_lib.VA_OPT_SAMPLE_RANK, 2**32)
    ctx.set_profiling(True)
    try:
        gi, gd = _index_search(ix, q, k)
        t = ctx.last_scan_timings()
    finally:
        ctx.set_option(_lib.VA_OPT_CANDIDATE_CAP, 0)
        ctx.set_option(_lib.VA_OPT_SAMPLE_RANK, 0)
        ctx.set_profiling(False)
    assert t["screened"] == 2 and t["overflow_rows"] > 0, t
    fi, fd = _fused(ctx, metric, q, x, k, screen=1)
    np.testing.assert_array_equal(gi, fi)
    np.testing.assert_array_equal(gd.view(np.uint32), fd.view(np.uint32))
    ix.close()


def test_removing_more_than_max_k_nearest_rows_keeps_k_results(ctx, oracle):
    """ADVICE: k + deletedCount > VA_MAX_K must not shorten the result."""
    from vectoraccelerate_amd import AcceleratedVectorIndex, IndexConfiguration

    g = np.random.default_rng(21)
    q = g.standard_normal(24).astype(np.float32)
    # rows at growing distance from q: the first 3000 are the nearest
    x = (q + np.linspace(0.01, 3.0, 5000)[:, None] * g.standard_normal((5000, 24)) / np.sqrt(24)).astype(np.float32)
    ix = AcceleratedVectorIndex(IndexConfiguration.flat(24, 64), ctx)
    hs = ix.insert(vectors=x)
    near = np.argsort(((x - q) ** 2).sum(1), kind="stable")[:3000]
    assert ix.remove([hs[i] for i in near]) == 3000
    r = ix.search(q, k=10)
    assert r.count == 10 and r.isExhaustive
    live = np.setdiff1d(np.arange(5000), near)
    oi, od = oracle.flat_topk(L2SQ, q[None], x[live], 10)
    assert [h.id.stableID for h in r.results] == live[oi[0]].tolist()
    np.testing.assert_allclose([h.distance for h in r.results], od[0], rtol=1e-4)
    ix.close()


def test_filter_rejecting_more_than_max_k_rows(ctx, oracle):
    """A filter that rejects the 2000 nearest vectors still yields the k nearest that pass."""
    from vectoraccelerate_amd import AcceleratedVectorIndex, IndexConfiguration

    g = np.random.default_rng(22)
    x = g.standard_normal((6000, 16)).astype(np.float32)
    q = g.standard_normal(16).astype(np.float32)
    ix = AcceleratedVectorIndex(IndexConfiguration.flat(16, 6000), ctx)
    hs = ix.insert(vectors=x)
    order = np.argsort(((x - q) ** 2).sum(1), kind="stable")
    banned = {hs[i].stableID for i in order[:2000]}
    ix.remove([hs[int(order[2500])]])
    r = ix.search(q, k=7, filter=lambda h, m: h.stableID not in banned)
    ok = np.array([i for i in range(6000) if i not in {int(order[j]) for j in range(2000)} and i != int(order[2500])])
    oi, od = oracle.flat_topk(L2SQ, q[None], x[ok], 7)
    assert [h.id.stableID for h in r.results] == ok[oi[0]].tolist()
    np.testing.assert_allclose([h.distance for h in r.results], od[0], rtol=1e-4)
    assert r.candidatesSearched >= 2007
    ix.close()


def test_unaligned_dimension_and_sentinels(ctx, oracle):
    """dim % 4 != 0 (no shadow), k above the live count, everything removed."""
    from vectoraccelerate_amd import AcceleratedVectorIndex, IndexConfiguration, VectorError

    g = np.random.default_rng(23)
    x = g.standard_normal((40, 7)).astype(np.float32)
    q = g.standard_normal((3, 7)).astype(np.float32)
    ix = AcceleratedVectorIndex(IndexConfiguration.flat(7, 4), ctx)
    hs = ix.insert(vectors=x)
    ix.remove(hs[5:])
    hi, hd = _index_search(ix, q, 8)
    oi, od = oracle.flat_topk(L2SQ, q, x[:5], 5)
    np.testing.assert_array_equal(hi[:, :5], oi)
    assert (hi[:, 5:] == 0xFFFFFFFF).all() and np.isinf(hd[:, 5:]).all()
    ix.remove(hs[:5])
    assert ix.count == 0 and ix.search(q[0], k=3).count == 0
    hi, hd = _index_search(ix, q, 2)
    assert (hi == 0xFFFFFFFF).all()
    with pytest.raises(VectorError):
        ix.remove(hs[0])  # already removed
    assert not ix.contains(hs[0]) and ix.vector(hs[0]) is None
    ix.close()


def test_native_index_through_the_c_abi(ctx):
    """va_index_* called directly: handles in insertion order, info counters, contains."""
    import torch
    from vectoraccelerate_amd import _lib
    from vectoraccelerate_amd.context import dptr

    lib = ctx.lib
    h = C.c_void_p()
    ctx.check(lib.va_index_create(ctx.handle, 12, 2, C.byref(h)), "va_index_create")
    x = np.arange(10 * 12, dtype=np.float32).reshape(10, 12)
    xd = ctx.buffer(x)
    out = np.zeros(10, np.uint32)
    ctx.order_after_torch()
    ctx.check(lib.va_index_insert(ctx.handle, h, dptr(xd), 10, out.ctypes.data), "va_index_insert")
    ctx.synchronize()
    assert out.tolist() == list(range(10))
    rm = C.c_uint32()
    ctx.check(lib.va_index_remove(ctx.handle, h, np.array([3, 3, 77], np.uint32).ctypes.data, 3, C.byref(rm)),
              "va_index_remove")
    assert rm.value == 1
    info = _lib.IndexInfo()
    ctx.check(lib.va_index_get_info(h, C.byref(info)), "va_index_get_info")
    assert (info.count, info.deleted, info.slots, info.dimension, info.next_handle) == (9, 1, 10, 12, 10)
    assert info.capacity >= 10 and info.rows
    assert lib.va_index_contains(h, 2) == 1 and lib.va_index_contains(h, 3) == 0
    v = np.zeros(12, np.float32)
    ctx.check(lib.va_index_get_vector(ctx.handle, h, 9, v.ctypes.data), "va_index_get_vector")
    np.testing.assert_array_equal(v, x[9])
    ctx.check(lib.va_index_compact(ctx.handle, h), "va_index_compact")
    ctx.check(lib.va_index_get_info(h, C.byref(info)), "va_index_get_info")
    assert (info.count, info.deleted, info.slots) == (9, 0, 9)
    qd = ctx.buffer(x[3:4] + 0.1)
    hi = ctx.empty((1, 3), torch.int32)
    hd = ctx.empty((1, 3), torch.float32)
    ctx.order_after_torch()
    ctx.check(lib.va_index_search(ctx.handle, h, L2SQ, dptr(qd), 1, 3, dptr(hi), dptr(hd)), "va_index_search")
    ctx.synchronize()
    assert hi.cpu().numpy().view(np.uint32)[0].tolist() == [4, 2, 5]
    assert lib.va_index_destroy(h) == 0
