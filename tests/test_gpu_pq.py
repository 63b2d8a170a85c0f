"""Product quantization on the device (va_pq_*) against the CPU oracle.

Codes, tables and ADC sums use the reference shader's summation orders on both sides, so they
are compared bit for bit; training sums members in the same fixed order, so codebooks are
bit-identical too.  ADC top-k ids are exact (ties by row id); distances are sqrt of the sums.
"""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

SHAPES = [(2000, 32, 8, 256), (1500, 30, 5, 64), (3000, 96, 16, 256), (500, 7, 7, 3), (4000, 768, 64, 256)]


def _data(N, D, seed):
    r = np.random.default_rng(seed)
    return (r.standard_normal((N, D)) * 2).astype(np.float32)


def _init(x, M, K, seed):
    r = np.random.default_rng(seed)
    ds = x.shape[1] // M
    rows = r.integers(0, x.shape[0], size=(M, K))
    return np.stack([x[rows[m], m * ds:(m + 1) * ds] for m in range(M)]).astype(np.float32)


@pytest.mark.parametrize("N,D,M,K", SHAPES)
def test_pq_train_encode_tables_adc_match_oracle(ctx, oracle, N, D, M, K):
    from vectoraccelerate_amd import Metal4PQConfig, ProductQuantizationKernel

    print(f"pq N={N} D={D} M={M} K={K}", flush=True)
    x = _data(N, D, N + D)
    init = _init(x, M, K, 3)
    cfg = Metal4PQConfig(D, M, K, trainIterations=6, convergenceThreshold=0.0)
    pq = ProductQuantizationKernel(ctx)
    model = pq.train(x, cfg, initialCodebooks=init)
    ocb, oit = oracle.pq_train(x, init, M, K, 6, 0.0)
    assert model.iterations == oit == 6
    np.testing.assert_array_equal(model.codebooks.cpu().numpy(), ocb)
    enc = pq.encode(x, model)
    ocodes = oracle.pq_encode(x, ocb, M, K)
    np.testing.assert_array_equal(enc.codes.cpu().numpy(), ocodes)
    q = _data(37, D, 99)
    t = pq.computeDistanceTables(q, model).cpu().numpy()
    np.testing.assert_array_equal(t, oracle.pq_tables(q, ocb, M, K))
    d = pq.computeDistances(q, enc, model).cpu().numpy()
    np.testing.assert_array_equal(d, oracle.pq_adc(t, ocodes))


@pytest.mark.parametrize("N,D,M,K,k,Q", [(20000, 64, 8, 256, 10, 64), (70000, 32, 16, 256, 100, 200),
                                          (5000, 48, 6, 32, 1, 5), (300, 16, 4, 16, 300, 3),
                                          (150000, 128, 32, 256, 1024, 8)])
def test_pq_search_matches_oracle(ctx, oracle, N, D, M, K, k, Q):
    """Covers the dense path (small N), the sampled path and a k at the maximum."""
    from vectoraccelerate_amd import Metal4PQConfig, Metal4PQModel, ProductQuantizationKernel

    print(f"pq search N={N} D={D} M={M} K={K} k={k} Q={Q}", flush=True)
    x = _data(N, D, 5)
    cb = _init(x, M, K, 4)
    cfg = Metal4PQConfig(D, M, K)
    pq = ProductQuantizationKernel(ctx)
    model = Metal4PQModel(ctx.buffer(cb), cfg)
    enc = pq.encode(x, model)
    codes = enc.codes.cpu().numpy()
    q = _data(Q, D, 6)
    idx, dist = pq.search(q, enc, model, k)
    oi, od = oracle.pq_search(q, cb, codes, M, K, k)
    np.testing.assert_array_equal(idx.cpu().numpy().view(np.uint32), oi)
    np.testing.assert_array_equal(dist.cpu().numpy(), od)


@pytest.mark.parametrize("M,scale,Q", [(64, 1.0e4, 37), (16, 1.0e-4, 21), (8, 1.0, 9), (32, 3.0e17, 5)])
def test_pq_screened_filter_scales_and_odd_queries(ctx, oracle, M, scale, Q):
    """The fp16-screened filter (K = 256): tables far above fp16's range (each query's scale
    brings them down; at 3e17 the squared entries overflow float and the screen passes every row),
    far below it, an odd query count (a pair with one query) and a NaN query, whose keys all tie
    (ids ascending).  Ids and distances equal the oracle's bit for bit."""
    from vectoraccelerate_amd import Metal4PQConfig, Metal4PQModel, ProductQuantizationKernel

    N, D, K, k = 30000, 128, 256, 20
    print(f"pq screened M={M} scale={scale} Q={Q}", flush=True)
    x = _data(N, D, 11) * np.float32(scale)
    cb = _init(x, M, K, 12)
    cfg = Metal4PQConfig(D, M, K)
    pq = ProductQuantizationKernel(ctx)
    model = Metal4PQModel(ctx.buffer(cb), cfg)
    enc = pq.encode(x, model)
    codes = enc.codes.cpu().numpy()
    q = _data(Q, D, 13) * np.float32(scale)
    q[Q // 2, 3] = np.nan
    idx, dist = pq.search(q, enc, model, k)
    oi, od = oracle.pq_search(q, cb, codes, M, K, k)
    np.testing.assert_array_equal(idx.cpu().numpy().view(np.uint32), oi)
    np.testing.assert_array_equal(dist.cpu().numpy(), od)  # NaN rows: NaN at the same places
    assert np.isnan(od[Q // 2]).all() and not np.isnan(np.delete(od, Q // 2, axis=0)).any()


def test_pq_duplicate_codes_tie_by_row(ctx, oracle):
    """Many rows share a code, so ADC sums tie: the lower row id comes first."""
    from vectoraccelerate_amd import Metal4PQConfig, Metal4PQModel, ProductQuantizationKernel

    r = np.random.default_rng(8)
    D, M, K = 16, 4, 4
    cb = r.standard_normal((M, K, D // M)).astype(np.float32)
    x = np.concatenate([cb[np.arange(M), r.integers(0, K, M)].reshape(1, D) for _ in range(50)] * 40)
    pq = ProductQuantizationKernel(ctx)
    model = Metal4PQModel(ctx.buffer(cb), Metal4PQConfig(D, M, K))
    enc = pq.encode(x, model)
    q = x[:4] + 0.01
    idx, dist = pq.search(q, enc, model, 64)
    oi, od = oracle.pq_search(q, cb, enc.codes.cpu().numpy(), M, K, 64)
    np.testing.assert_array_equal(idx.cpu().numpy().view(np.uint32), oi)
    np.testing.assert_array_equal(dist.cpu().numpy(), od)


def test_pq_seeded_training_and_errors(ctx, oracle):
    from vectoraccelerate_amd import Metal4PQConfig, ProductQuantizationKernel, VectorError

    x = _data(3000, 64, 12)
    pq = ProductQuantizationKernel(ctx)
    cfg = Metal4PQConfig(64, 8, 256)
    a = pq.train(x, cfg, seed=5)
    b = pq.train(x, cfg, seed=5)
    np.testing.assert_array_equal(a.codebooks.cpu().numpy(), b.codebooks.cpu().numpy())
    assert 1 <= a.iterations <= 25
    model, enc = pq.trainAndEncode(x, cfg, seed=5)
    np.testing.assert_array_equal(enc.codes.cpu().numpy(), oracle.pq_encode(x, model.codebooks.cpu().numpy(), 8, 256))
    nn = pq.findNearestNeighbors(x[7], enc, model, 5)
    assert len(nn) == 5 and nn[0][1] <= nn[-1][1]
    with pytest.raises(VectorError):
        Metal4PQConfig(65, 8)
    with pytest.raises(VectorError):
        Metal4PQConfig(64, 8, 300)
    with pytest.raises(VectorError):
        pq.encode(_data(10, 32, 1), model)


def test_pq_edge_cases(ctx, oracle):
    """k above N (sentinel slots), one row, one query, and a code array whose rows are not
    16-byte aligned (the runtime-M kernel instead of the specialised one)."""
    from vectoraccelerate_amd import Metal4EncodedVectors, Metal4PQConfig, Metal4PQModel, ProductQuantizationKernel

    D, M, K = 32, 8, 256
    x = _data(300, D, 41)
    cb = _init(x, M, K, 42)
    cfg = Metal4PQConfig(D, M, K)
    pq = ProductQuantizationKernel(ctx)
    model = Metal4PQModel(ctx.buffer(cb), cfg)
    enc = pq.encode(x, model)
    codes = enc.codes.cpu().numpy()
    q = _data(3, D, 43)
    for n, k in ((300, 400), (1, 5), (300, 1)):
        e = Metal4EncodedVectors(enc.codes[:n], n, cfg)
        idx, dist = pq.search(q[:1] if n == 1 else q, e, model, k)
        oi, od = oracle.pq_search(q[:1] if n == 1 else q, cb, codes[:n], M, K, k)
        np.testing.assert_array_equal(idx.cpu().numpy().view(np.uint32), oi)
        np.testing.assert_array_equal(dist.cpu().numpy(), od)
    # rows start 8 bytes into a 16-byte block: the generic kernel
    e = Metal4EncodedVectors(enc.codes[1:], 299, cfg)
    assert e.codes.data_ptr() % 16 == 8
    idx, dist = pq.search(q, e, model, 10)
    oi, od = oracle.pq_search(q, cb, codes[1:], M, K, 10)
    np.testing.assert_array_equal(idx.cpu().numpy().view(np.uint32), oi)
    np.testing.assert_array_equal(dist.cpu().numpy(), od)


def test_pq_train_multi_chunk(ctx, oracle):
    """200,000 training rows over 16 centroids per subspace: each centroid's mean sums dozens
    of 256-row chunks; codebooks must equal the oracle's bit for bit."""
    from vectoraccelerate_amd import Metal4PQConfig, ProductQuantizationKernel

    N, D, M, K = 200_000, 32, 4, 16
    x = _data(N, D, 51)
    init = _init(x, M, K, 52)
    cfg = Metal4PQConfig(D, M, K, trainIterations=3, convergenceThreshold=0.0)
    model = ProductQuantizationKernel(ctx).train(x, cfg, initialCodebooks=init)
    ocb, oit = oracle.pq_train(x, init, M, K, 3, 0.0)
    assert model.iterations == oit == 3
    np.testing.assert_array_equal(model.codebooks.cpu().numpy(), ocb)
