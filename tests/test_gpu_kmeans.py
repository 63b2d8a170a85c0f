"""k-means on the device (va_kmeans_fit / va_kmeans_plusplus) against the CPU oracle.

The oracle restates KMeansPipeline.fit (KMeansPipeline.swift:102-270) with the reference's
float difference-form assignment; the device assigns with the fp32 MFMA distance kernel
(|x|^2 + |c|^2 - 2 x.c).  On data whose nearest centroid is unambiguous both give the same
assignments, and then the same centroid bits: both sum a cluster's points in chunks of 256 in
point order, then the chunk sums in order, in fp32, times 1/count.  The device recomputes each
point's distance to its centroid in difference form (other summation order than the oracle's),
so distances agree within
2 (D + 4) 2^-24 relative: each side's sum of D squares is within (D + 1) 2^-24 of the exact one.
"""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _blobs(C_, D, per, seed, spread=0.05, sep=10.0):
    r = np.random.default_rng(seed)
    centers = (r.standard_normal((C_, D)) * sep).astype(np.float32)
    lab = np.repeat(np.arange(C_), per)
    r.shuffle(lab)
    x = (centers[lab] + r.standard_normal((lab.size, D)).astype(np.float32) * spread).astype(np.float32)
    return x, lab, centers


def _fit(ctx, x, init, iters, thr):
    from vectoraccelerate_amd import KMeansConfiguration, KMeansPipeline

    cfg = KMeansConfiguration(numClusters=init.shape[0], dimension=x.shape[1], maxIterations=iters,
                              convergenceThreshold=thr)
    r = KMeansPipeline(ctx, cfg).fit(x, init)
    return (r.centroids.cpu().numpy(), r.assignments.cpu().numpy().view(np.uint32),
            r.distances.cpu().numpy(), r.clusterCounts.cpu().numpy().view(np.uint32), r)


def _check_dist(dist, ref, D):
    np.testing.assert_allclose(dist, ref, rtol=2 * (D + 4) * 2.0**-24, atol=0)


def _margins(x, cen):
    """Relative gap between each point's two smallest float64 squared distances to cen (1 with a
    single centroid: no tie is possible)."""
    if cen.shape[0] < 2:
        return np.ones(x.shape[0])
    x64, c64 = x.astype(np.float64), cen.astype(np.float64)
    d = (x64 * x64).sum(1)[:, None] + (c64 * c64).sum(1)[None] - 2 * x64 @ c64.T
    two = np.sort(np.maximum(d, 0), axis=1)[:, :2]
    return (two[:, 1] - two[:, 0]) / np.maximum(two[:, 1], 1e-30)


def _compare(ctx, oracle, x, init, iters, thr):
    cen, assign, dist, counts, r = _fit(ctx, x, init, iters, thr)
    ocen, oassign, odist, ocounts, oit, oconv, oinertia, omm = oracle.kmeans_fit(x, init, iters, thr)
    # Bit equality with the oracle holds only where no point is nearly equidistant from two
    # centroids: the device assigns in the expanded form, the oracle in the difference form.
    # These data sets are built tie-free; check that against the oracle's final centroids (the
    # planted-tie test below covers the other case).
    assert _margins(x, ocen).min() > 1e-4, "data set has near-ties: use the near-tie comparison"
    print(f"kmeans N={x.shape[0]} D={x.shape[1]} C={init.shape[0]} iters={r.iterations}/{oit}", flush=True)
    assert r.iterations == oit and r.converged == oconv
    np.testing.assert_array_equal(assign, oassign)
    np.testing.assert_array_equal(counts, ocounts)
    np.testing.assert_array_equal(cen, ocen)  # same members, same order, same fp32 sums
    _check_dist(dist, odist, x.shape[1])
    assert abs(r.inertia - float(dist.astype(np.float64).sum())) <= 1e-6 * max(1.0, r.inertia)
    assert abs(r.maxMovement - omm) <= 1e-4 * max(1.0, omm) + 1e-6  # same bits, other sum order
    return r


@pytest.mark.parametrize("C_,D,per,iters", [(8, 3, 300, 20), (17, 100, 250, 20), (50, 64, 400, 20),
                                            (256, 128, 120, 5), (40, 768, 100, 10)])
def test_kmeans_fit_matches_oracle(ctx, oracle, C_, D, per, iters):
    x, lab, centers = _blobs(C_, D, per, seed=C_ * 7 + D)
    init = (centers + 0.3 * np.random.default_rng(1).standard_normal(centers.shape)).astype(np.float32)
    r = _compare(ctx, oracle, x, init, iters, 1e-4)
    assert r.converged


def test_kmeans_empty_clusters_gpu(ctx, oracle):
    # the reference's small case: three seeds far away get no points and take the farthest ones
    x = np.array([[0, 0], [1, 0], [0, 1], [10, 0], [13, 0], [10, 4]], np.float32)
    init = np.array([[100, 100], [0.3, 0.3], [-100, -100], [11, 1], [200, 0]], np.float32)
    _compare(ctx, oracle, x, init, 1, 0.0)
    _compare(ctx, oracle, x, init, 10, 1e-4)
    # blobs plus 30 seeds nobody is near: repair in the first iteration, then Lloyd
    xb, lab, centers = _blobs(20, 32, 150, seed=3)
    far = (np.random.default_rng(4).standard_normal((30, 32)) * 1000).astype(np.float32)
    init = np.concatenate([centers[:10] + 0.2, far, centers[10:] + 0.2]).astype(np.float32)
    _compare(ctx, oracle, xb, init, 1, 0.0)


def test_kmeans_zero_iterations_and_single_cluster(ctx, oracle):
    x, lab, centers = _blobs(5, 24, 100, seed=9)
    _compare(ctx, oracle, x, centers.copy(), 0, 1e-4)
    _compare(ctx, oracle, x, x[:1].copy(), 5, 1e-4)
    # every point its own cluster
    _compare(ctx, oracle, x[:64].copy(), x[:64].copy(), 3, 1e-4)


def test_kmeans_deterministic_and_self_consistent(ctx):
    """Seeds inside the same blob make ties between nearby centroids: no oracle comparison, but
    two runs give the same bits and every centroid is the mean of the points assigned to it."""
    x, lab, centers = _blobs(16, 48, 500, seed=11, spread=1.0, sep=3.0)
    init = x[np.random.default_rng(2).choice(x.shape[0], 64, replace=False)].copy()
    a = _fit(ctx, x, init, 4, 0.0)
    b = _fit(ctx, x, init, 4, 0.0)
    for u, v in zip(a[:4], b[:4]):
        np.testing.assert_array_equal(u, v)
    cen, assign, dist, counts, r = a
    assert r.iterations == 4 and counts.sum() == x.shape[0]
    np.testing.assert_array_equal(counts, np.bincount(assign, minlength=64))
    for c in range(64):
        if counts[c]:
            np.testing.assert_allclose(cen[c], x[assign == c].astype(np.float64).mean(0), rtol=1e-5, atol=1e-5)
    seen = init_before_last(ctx, x, init, 4)
    _check_dist(dist, np.sqrt(((x.astype(np.float64) - seen.astype(np.float64)[assign]) ** 2).sum(1)), x.shape[1])


def init_before_last(ctx, x, init, iters):
    return init if iters == 1 else _fit(ctx, x, init, iters - 1, 0.0)[0]


def test_kmeans_errors(ctx):
    from vectoraccelerate_amd import KMeansConfiguration, KMeansPipeline, VectorError

    x = np.zeros((4, 3), np.float32)
    with pytest.raises(VectorError):
        KMeansPipeline(ctx, KMeansConfiguration(numClusters=5, dimension=3)).fit(x, np.zeros((5, 3), np.float32))
    with pytest.raises(VectorError):
        KMeansPipeline(ctx, KMeansConfiguration(numClusters=2, dimension=3)).fit(x, np.zeros((3, 3), np.float32))
    with pytest.raises(VectorError):
        KMeansPipeline(ctx, KMeansConfiguration(numClusters=2, dimension=4)).fit(x, np.zeros((2, 4), np.float32))
    with pytest.raises(VectorError):
        KMeansPipeline(ctx, KMeansConfiguration(numClusters=2, dimension=3)).fit([])


@pytest.mark.parametrize("N,D,k", [(2000, 32, 64), (500, 7, 500), (10000, 128, 16)])
def test_kmeans_plusplus_matches_oracle(ctx, oracle, N, D, k):
    from vectoraccelerate_amd import KMeansPlusPlusKernel

    x = np.random.default_rng(N + D).standard_normal((N, D)).astype(np.float32)
    for seed in (0, 7):
        cen, idx = KMeansPlusPlusKernel(ctx).selectCentroidsBuffer(x, k, seed)
        np.testing.assert_array_equal(idx, oracle.kmeans_plusplus(x, k, seed))
        np.testing.assert_array_equal(cen.cpu().numpy(), x[idx])


def test_kmeans_plusplus_duplicates_and_full_pipeline(ctx, oracle):
    from vectoraccelerate_amd import KMeansConfiguration, KMeansPipeline, KMeansPlusPlusKernel

    locs = np.random.default_rng(3).standard_normal((9, 6)).astype(np.float32) * 5
    dup = np.repeat(locs, 11, axis=0)
    _, idx = KMeansPlusPlusKernel(ctx).selectCentroidsBuffer(dup, 9, 5)
    assert sorted(set((idx // 11).tolist())) == list(range(9))
    np.testing.assert_array_equal(idx, oracle.kmeans_plusplus(dup, 9, 5))
    # fit() without initial centroids seeds with k-means++ (configuration seed)
    x, lab, centers = _blobs(12, 40, 200, seed=21)
    cfg = KMeansConfiguration(numClusters=12, dimension=40, maxIterations=50, seed=123)
    r = KMeansPipeline(ctx, cfg).fit(x)
    init = x[oracle.kmeans_plusplus(x, 12, 123)]
    ocen, oassign, *_rest = oracle.kmeans_fit(x, init, 50, 1e-4)
    np.testing.assert_array_equal(r.assignments.cpu().numpy().view(np.uint32), oassign)
    np.testing.assert_array_equal(r.centroids.cpu().numpy(), ocen)


def test_kmeans_planted_near_ties(ctx, oracle):
    """Points planted equidistant (to ~1e-7 relative) from two centroids.  The device's
    expanded-form assignment may differ from the oracle's difference form there; every device
    choice must be a nearest centroid within the fp32 tolerance, every point with a clear margin
    must match the oracle, and the update must equal the oracle's update of the device's own
    assignment bit for bit.  The divergence is recorded (printed), not hidden."""
    g = np.random.default_rng(93)
    C_, D = 6, 32
    cen0 = (g.standard_normal((C_, D)) * 4).astype(np.float32)
    pts = []
    for a, b in [(0, 1), (2, 3), (4, 5), (1, 4)]:
        u = (cen0[b] - cen0[a]).astype(np.float64)
        u /= np.linalg.norm(u)
        for _ in range(120):
            v = g.standard_normal(D)
            v -= (v @ u) * u  # orthogonal to the pair's axis: equidistant in exact arithmetic
            p = (cen0[a] + cen0[b]) / 2 + 0.5 * v + u * g.uniform(-1e-6, 1e-6)
            pts.append(p)
    pts += list(cen0[g.integers(0, C_, 600)] + 0.3 * g.standard_normal((600, D)))
    x = np.asarray(pts, np.float32)
    cen, assign, dist, counts, r = _fit(ctx, x, cen0, 1, 0.0)
    ocen, oassign, odist, ocounts, *_ = oracle.kmeans_fit(x, cen0, 1, 0.0)
    x64, c64 = x.astype(np.float64), cen0.astype(np.float64)
    d = ((x64[:, None, :] - c64[None]) ** 2).sum(2)
    best = d.min(1)
    chosen = d[np.arange(x.shape[0]), assign]
    scale = (x64 * x64).sum(1) + (c64[assign] ** 2).sum(1)
    assert np.all(chosen - best <= 1e-5 * scale), "device picked a centroid that is not nearest"
    clear = _margins(x, cen0) > 1e-4
    np.testing.assert_array_equal(assign[clear], oassign[clear])
    diverged = int((assign != oassign).sum())
    print(f"planted near-ties: {int((~clear).sum())} ambiguous points, {diverged} assigned differently "
          f"from the difference-form oracle", flush=True)
    uc, ucnt = oracle.kmeans_update(x, assign, dist, cen0)
    np.testing.assert_array_equal(cen, uc)
    np.testing.assert_array_equal(counts, ucnt)


def test_index_train_without_centroids(ctx, oracle):
    """AcceleratedVectorIndex.train() with no centroids: device k-means (k-means++ seed, 25
    iterations, threshold 0.001) over the live vectors, then the IVF lists from them
    (AcceleratedVectorIndex.swift:406-446, IVFStructure.swift:202-259)."""
    from vectoraccelerate_amd import AcceleratedVectorIndex, IndexConfiguration, VectorError

    x, lab, centers = _blobs(16, 32, 60, seed=31)
    idx = AcceleratedVectorIndex(IndexConfiguration.ivf(dimension=32, nlist=16, nprobe=4, capacity=2000), ctx)
    with pytest.raises(VectorError):
        idx.train()  # no vectors
    hs = idx.insert(vectors=x)
    idx.remove(hs[0])
    idx.train(seed=77)
    live = x[1:]
    init = live[oracle.kmeans_plusplus(live, 16, 77)]
    ocen, oassign, *_ = oracle.kmeans_fit(live, init, 25, 0.001)
    np.testing.assert_array_equal(idx.centroids(), ocen)
    # the lists: every stored row under its nearest trained centroid, in row order
    off, ids = idx.lists()
    # train() compacts first: the stored rows are the live rows, in insertion order
    assert idx.count == live.shape[0]
    stored = np.array([idx.vector(h) for h in hs[1:]], np.float32)
    np.testing.assert_array_equal(stored, live)
    lists = oracle.ivf_assign(stored, ocen)
    ooff, oids = oracle.ivf_csr(lists, 16)
    np.testing.assert_array_equal(off, ooff)
    np.testing.assert_array_equal(ids, oids)
    res = idx.search(queries=centers, k=5)
    assert all(len(r.results) == 5 for r in res)


def test_kmeans_tiny_and_ivf_add_nothing(ctx, oracle):
    """One point and one cluster; a zero-row add leaves the lists unchanged."""
    from vectoraccelerate_amd import IVFSearchConfiguration, IVFSearchPipeline

    x = np.array([[1.5, -2.0, 3.0]], np.float32)
    _compare(ctx, oracle, x, x.copy(), 3, 1e-4)
    xb, lab, centers = _blobs(4, 8, 20, seed=5)
    pipe = IVFSearchPipeline(ctx, IVFSearchConfiguration(4, 2, 8))
    st = pipe.prepareIndexStructure(centers, xb)
    before = st.lists()
    st.add(ctx.buffer(xb)[:0], xb.shape[0])
    after = st.lists()
    np.testing.assert_array_equal(before[0], after[0])
    np.testing.assert_array_equal(before[1], after[1])
    st.close()


def test_kmeans_zipf_sized_clusters(ctx, oracle):
    """configs[4]-like cluster sizes (Zipf 1.1) at 120,000 points: the largest clusters span
    hundreds of 256-point chunks; centroids must still equal the oracle's bit for bit."""
    r = np.random.default_rng(17)
    C_, D, N = 128, 48, 120_000
    centers = (r.standard_normal((C_, D)) * 10).astype(np.float32)
    p = 1.0 / np.arange(1, C_ + 1) ** 1.1
    lab = r.choice(C_, N, p=p / p.sum())
    x = (centers[lab] + 0.05 * r.standard_normal((N, D))).astype(np.float32)
    init = (centers + 0.3 * r.standard_normal(centers.shape)).astype(np.float32)
    res = _compare(ctx, oracle, x, init, 4, 1e-4)
    counts = res.clusterCounts.cpu().numpy().view(np.uint32)
    assert counts.max() > 100 * 256
