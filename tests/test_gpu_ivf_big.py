"""The screened IVF scan's tiles for lists probed by many queries (ivf16_big_kernel: 192 queries x
256 rows, both operands staged in LDS by direct loads, queries gathered through the plan).

Every search here runs the screened list scan with that group in its full pass and is compared bit
for bit with the fp32 list scan (VA_OPT_SCREEN = 1) and with the oracle's scan over the same lists
and probes (IVFListSearch.metal:199-339 is the reference's list scan; its results are exact per
list, as are these).
"""
from __future__ import annotations

import numpy as np
import pytest

from tests.helpers import L2SQ, SENT, check_topk
from tests.test_gpu_ivf import clustered

pytestmark = pytest.mark.gpu


def _search(ctx, pipe, q, st, k, screen):
    """(result, scan timings) of one search with VA_OPT_SCREEN = screen."""
    from vectoraccelerate_amd import _lib

    ctx.set_option(_lib.VA_OPT_SCREEN, screen)
    ctx.set_profiling(True)
    try:
        res = pipe.search(q, st, k)
        t = ctx.last_scan_timings()
    finally:
        ctx.set_profiling(False)
        ctx.set_option(_lib.VA_OPT_SCREEN, 0)
    return res, t


def _probe_counts(pipe, q, st, C):
    probes = pipe.findNearestCentroids(q, st).cpu().numpy().view(np.uint32)
    cnt = np.zeros(C, np.int64)
    for row in probes:
        for l in set(int(v) for v in row if v < C):
            cnt[l] += 1
    return probes, cnt


def _compare(ctx, oracle, C, D, x, q, c, nprobe, k):
    from vectoraccelerate_amd import IVFSearchConfiguration, IVFSearchPipeline

    pipe = IVFSearchPipeline(ctx, IVFSearchConfiguration(C, nprobe, D))
    st = pipe.prepareIndexStructure(c, x)
    probes, cnt = _probe_counts(pipe, q, st, C)
    scr, ts = _search(ctx, pipe, q, st, k, 0)
    ref, tr = _search(ctx, pipe, q, st, k, 1)
    assert ts["screened"] == 1 and tr["screened"] == 0
    big = int((cnt > 96).sum())
    # the big group is launched beside the three tile groups when Q > 96
    assert ts["scan_launches"] == (4 if q.shape[0] > 96 else 3)
    si = scr.indices.cpu().numpy().view(np.uint32)
    np.testing.assert_array_equal(si, ref.indices.cpu().numpy().view(np.uint32))
    np.testing.assert_array_equal(scr.distances.cpu().numpy().view(np.uint32),
                                  ref.distances.cpu().numpy().view(np.uint32))
    off, ids = st.lists()
    oi, od = oracle.ivf_scan(q, x, off, ids, probes, k)
    check_topk(L2SQ, q, x, k, si, scr.distances.cpu().numpy(), oi, od)
    st.close()
    return cnt, big


# Lists probed by 97-192 queries (one query block, most of a 192-query tile used), by more than 192
# (several query blocks per list: tiles alternate blocks inside a row block), ragged last row tiles;
# padded D = 64, 128, 192, 768 and 1024 (zero-padded shadow rows), k from 1 to 100.
@pytest.mark.parametrize("C,D,N,Q,nprobe,k,zipf", [(8, 64, 20000, 400, 2, 10, None),
                                                    (16, 100, 30000, 500, 4, 1, 1.1),
                                                    (6, 180, 9000, 700, 3, 25, None),
                                                    (32, 768, 40000, 256, 8, 100, 1.1),
                                                    (12, 1000, 12000, 300, 6, 10, None),
                                                    (4, 128, 1500, 420, 4, 10, None)])
def test_big_list_tiles_equal_fp32_list_scan_and_oracle(ctx, oracle, C, D, N, Q, nprobe, k, zipf):
    c, x, q = clustered(C, D, N, Q, 11 * C + D, zipf)
    cnt, big = _compare(ctx, oracle, C, D, x, q, c, nprobe, k)
    assert big >= 1, f"no list is probed by more than 96 queries: {cnt.max()}"


def test_big_list_tiles_several_query_blocks(ctx, oracle):
    """Every query probes every one of 4 lists (420 probing queries each: three query blocks of a
    192-query tile, the last one ragged)."""
    c, x, q = clustered(4, 96, 6000, 420, 3, None)
    cnt, big = _compare(ctx, oracle, 4, 96, x, q, c, 4, 20)
    assert big == 4 and cnt.min() == 420


def test_big_list_tiles_flagged_rows(ctx, oracle):
    """Rows with entries beyond the fp16 range in a list probed by many queries: flagged rows pass
    the pre-test (their NaN inputs make every comparison pass) and their exact keys decide."""
    c, x, q = clustered(8, 64, 16000, 300, 29, None)
    g = np.random.default_rng(9)
    far = g.choice(16000, 300, replace=False)
    x[far] *= np.float32(3e4)
    q[:6] = x[far[:6]] * np.float32(1.0001)
    _compare(ctx, oracle, 8, 64, x, q, c, 3, 10)


def test_big_list_tiles_not_used_at_96_queries(ctx, oracle):
    """Q <= 96: no list can be probed by more than 96 queries; three tile groups run."""
    c, x, q = clustered(8, 64, 8000, 96, 5, None)
    _compare(ctx, oracle, 8, 64, x, q, c, 8, 10)


def test_big_list_tiles_with_index_deletions(ctx, oracle):
    """A trained native IVF index with many queries per list and a third of its rows removed: the
    deletion mask reaches the big tiles' candidates (through their CSR positions), and the result
    equals the oracle over the live rows of the probed lists."""
    from tests.test_gpu_ivf_index import _live_csr, _search as index_search
    from vectoraccelerate_amd import AcceleratedVectorIndex, IndexConfiguration

    c, x, q = clustered(8, 64, 24000, 300, 41, 1.1)
    idx = AcceleratedVectorIndex(IndexConfiguration.ivf(dimension=64, nlist=8, nprobe=3), ctx)
    hs = idx.insert(vectors=x)
    idx.train(c)
    dead = np.random.default_rng(3).choice(24000, 8000, replace=False)
    idx.remove([hs[i] for i in dead])
    off, ids = idx.lists()
    probes = idx.probes(q)
    noff, nids = _live_csr(off, ids, set(dead.tolist()))
    gi, gd = index_search(idx, q, 30)
    oi, od = oracle.ivf_scan(q, x, noff, nids, probes, 30)
    check_topk(L2SQ, q, x, 30, gi, gd, oi, od)
    assert not set(gi.ravel().tolist()) & set(dead.tolist())
    assert (gi != SENT).all()
    idx.close()
