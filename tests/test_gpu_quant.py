"""GPU parity of the scalar-int8 and binary paths: codes, integer distances and top-k ids are
bit-exact against the CPU oracle (the oracle is pinned in tests/test_oracle.py)."""
from __future__ import annotations

import numpy as np
import pytest

from tests.helpers import SENT, check_topk_exact

pytestmark = pytest.mark.gpu


def rng(seed):
    return np.random.default_rng(seed)


def c3_like(n, d, seed):
    """configs[2] generator at a reduced size: U(-1,1) scaled per dimension by U(0.5, 2)."""
    g = rng(seed)
    s = g.uniform(0.5, 2.0, d).astype(np.float32)
    return (g.uniform(-1, 1, (n, d)) * s).astype(np.float32), s


# ---------------------------------------------------------------------------------------
# scalar int8
# ---------------------------------------------------------------------------------------
@pytest.mark.parametrize("N,D", [(1, 1), (7, 3), (1000, 512), (3001, 100), (20000, 64), (513, 1024), (300, 1028),
                                 (40001, 8)])
def test_sq_params_and_codes_bit_exact(ctx, oracle, N, D):
    from vectoraccelerate_amd import ScalarQuantizationKernel

    x, _ = c3_like(N, D, N + D)
    k = ScalarQuantizationKernel(ctx)
    p = k.computePerDimensionParameters(x)
    mn, mx, sc, zp = oracle.sq_params_per_dim(x)
    np.testing.assert_array_equal(p.min, mn)
    np.testing.assert_array_equal(p.max, mx)
    np.testing.assert_array_equal(p.scale, sc)
    np.testing.assert_array_equal(p.zeroPoint, zp)
    codes = k.quantizePerDimension(x, p).cpu().numpy()
    np.testing.assert_array_equal(codes, oracle.sq_quantize(x, sc, zp))
    deq = k.dequantizePerDimension(ctx.buffer(codes), p).cpu().numpy()
    np.testing.assert_array_equal(deq, oracle.sq_dequantize(codes, sc, zp))


def test_sq_golden_and_edge_values(ctx, oracle):
    from vectoraccelerate_amd import PerDimensionParameters, ScalarQuantizationKernel

    k = ScalarQuantizationKernel(ctx)
    x = np.array([[-1, 0], [1, 255], [0, 100]], np.float32)
    p = k.computePerDimensionParameters(x)
    np.testing.assert_array_equal(p.zeroPoint, [-1, -128])  # tests/golden/sq_per_dim.json
    np.testing.assert_array_equal(k.quantizePerDimension(x, p).cpu().numpy(), [[-128, -128], [126, 127], [-1, -28]])
    # half-even rounding, clamping, NaN, and the near-zero scale guard
    v = np.array([[0.5, 1.5, 2.5, -0.5, -1.5, 200.0, -300.0, np.nan, 3.0]], np.float32)
    sc = np.array([1, 1, 1, 1, 1, 1, 1, 1, 1e-10], np.float32)
    zp = np.array([0, 0, 0, 0, 0, 0, 0, 0, 300], np.int32)
    p = PerDimensionParameters(sc, sc, sc, zp)
    got = k.quantizePerDimension(v, p).cpu().numpy()
    np.testing.assert_array_equal(got, oracle.sq_quantize(v, sc, zp))
    np.testing.assert_array_equal(got, [[0, 2, 2, 0, -2, 127, -128, 0, 127]])


def test_sq_params_with_nan_and_signed_zero(ctx, oracle):
    """NaN never wins a min/max comparison (a column of only NaN gets min = max = 0), and -0/+0
    compare equal; checked on the vectorised (D % 4 == 0) and the scalar paths."""
    from vectoraccelerate_amd import ScalarQuantizationKernel

    g = rng(23)
    for d in (16, 7):
        x = g.standard_normal((2000, d)).astype(np.float32)
        x[g.random(x.shape) < 0.01] = np.nan
        x[:, 1] = np.nan
        x[:, 2] = -0.0
        x[5, 2] = 0.0
        k = ScalarQuantizationKernel(ctx)
        p = k.computePerDimensionParameters(x)
        mn, mx, sc, zp = oracle.sq_params_per_dim(x)
        np.testing.assert_array_equal(p.min, mn)
        np.testing.assert_array_equal(p.max, mx)
        np.testing.assert_array_equal(p.scale, sc)
        np.testing.assert_array_equal(p.zeroPoint, zp)
        np.testing.assert_array_equal(k.quantizePerDimension(x, p).cpu().numpy(), oracle.sq_quantize(x, sc, zp))


def test_sq_constant_columns(ctx, oracle):
    """NumericalStabilityTests.swift:1295-1370: zero / constant data quantises to finite values."""
    from vectoraccelerate_amd import ScalarQuantizationKernel

    x = np.zeros((50, 8), np.float32)
    x[:, 3] = 2.5
    k = ScalarQuantizationKernel(ctx)
    p = k.computePerDimensionParameters(x)
    mn, mx, sc, zp = oracle.sq_params_per_dim(x)
    np.testing.assert_array_equal(p.scale, sc)
    np.testing.assert_array_equal(p.zeroPoint, zp)
    codes = k.quantizePerDimension(x, p)
    assert np.all(np.isfinite(k.dequantizePerDimension(codes, p).cpu().numpy()))


def test_global_quantize_roundtrip(ctx):
    """ScalarQuantizationKernel.quantize/dequantize with global symmetric parameters."""
    from vectoraccelerate_amd import Metal4QuantizationType, ScalarQuantizationKernel

    data = rng(3).uniform(-2, 2, 1000).astype(np.float32)
    k = ScalarQuantizationKernel(ctx)
    r = k.quantize(data)
    assert r.zeroPoint is None and r.compressionRatio == pytest.approx(4.0)
    back = k.dequantize(r, data.size)
    assert np.max(np.abs(back - data)) <= r.scale * 0.5 + 1e-6
    r2 = k.quantize(data, type=Metal4QuantizationType.asymmetric)
    assert r2.zeroPoint is not None


def test_global_quantize_matches_oracle_and_fixture(ctx, oracle):
    """ScalarQuantizationKernel.quantize with global parameters (computeQuantizationParams,
    ScalarQuantizationKernel.swift:496-520): scale, the saturating Int8 zero point and the codes
    are bit-exact against the oracle, on the golden closed-form cases and on random data whose
    asymmetric zero point saturates."""
    import json
    from pathlib import Path

    from vectoraccelerate_amd import Metal4QuantizationType, ScalarQuantizationKernel

    k = ScalarQuantizationKernel(ctx)
    fx = json.loads((Path(__file__).resolve().parent / "golden" / "sq_global.json").read_text())
    g = rng(11)
    randoms = [(g.uniform(-3, 5, 5000).astype(np.float32), a) for a in (False, True)]
    randoms += [(g.uniform(400, 410, 3000).astype(np.float32), True),   # zero point saturates at -128
                (g.uniform(-90, -80, 3000).astype(np.float32), True)]    # ... and at 127
    cases = [(np.array(c["data"], np.float32), c["asymmetric"]) for c in fx["cases"]] + randoms
    for data, asym in cases:
        qt = Metal4QuantizationType.asymmetric if asym else Metal4QuantizationType.symmetric
        r = k.quantize(data, type=qt)
        codes, scale, zp = oracle.sq_global_quantize(data, asym)
        assert np.float32(r.scale) == scale
        assert (r.zeroPoint if asym else 0) == zp
        if not asym:
            assert r.zeroPoint is None
        np.testing.assert_array_equal(np.frombuffer(r.quantizedData, np.int8), codes)


@pytest.mark.parametrize("Q,N,D,k", [(1, 50, 16, 5), (40, 3000, 512, 10), (130, 20000, 64, 100), (9, 40000, 100, 7),
                                     (300, 5000, 48, 1),
                                     # large-Q tiles (256 queries x 128 rows): ragged Q and N,
                                     # several 64-byte stages, a partial last stage, one-stage D
                                     (257, 3001, 512, 10), (450, 20000, 160, 50), (1000, 7000, 1024, 5),
                                     (513, 129, 16, 3),
                                     # resident query blocks on the 16x16x64 MFMA (256 queries at
                                     # d = 256 and 512, 128 at 768 and 1024): ragged blocks, rows past
                                     # N inside a wave's rows, ranges of several tiles
                                     (600, 7001, 768, 10), (193, 50000, 256, 3), (2000, 12011, 512, 10)])
def test_i8_scan_topk_bit_exact(ctx, oracle, Q, N, D, k):
    from vectoraccelerate_amd import ScalarQuantizationKernel

    g = rng(Q + N + D)
    qc = g.integers(-128, 128, (Q, D)).astype(np.int8)
    xc = g.integers(-128, 128, (N, D)).astype(np.int8)
    xc[N // 2] = xc[N // 3]  # a tie
    gi, gd = ScalarQuantizationKernel(ctx).searchTopK(qc, xc, k)
    oi, od = oracle.i8_topk(qc, xc, k)
    check_topk_exact(gi, gd, oi, od)


@pytest.mark.parametrize("Q,N,D,k", [(300, 6000, 96, 20), (260, 4000, 512, 10), (700, 3000, 256, 40),
                                     (300, 5000, 768, 30), (1100, 2500, 1024, 64)])
def test_i8_large_q_many_passes(ctx, oracle, Q, N, D, k):
    """Large-Q filter scan where every query has hundreds of tied passes (the database is 40
    distinct rows repeated): each wave stages and flushes many batches of passes, and ties are
    broken by the smaller id.  D=96 also has a zero-padding k-step."""
    from vectoraccelerate_amd import ScalarQuantizationKernel

    g = rng(Q * 7 + D)
    base = g.integers(-128, 128, (40, D)).astype(np.int8)
    xc = base[g.integers(0, 40, N)]
    qc = g.integers(-128, 128, (Q, D)).astype(np.int8)
    gi, gd = ScalarQuantizationKernel(ctx).searchTopK(qc, xc, k)
    oi, od = oracle.i8_topk(qc, xc, k)
    check_topk_exact(gi, gd, oi, od)


def test_i8_scan_rejects_dimensions_beyond_int32_range(ctx):
    """dim 131071 keeps every dot inside int32 (16384 * 131071 < 2^31); one more could wrap, so the
    call is refused before any memory is touched (the 1-byte buffers are never read)."""
    import torch

    from vectoraccelerate_amd import VectorError, _lib

    assert _lib.VA_I8_MAX_DIM == 131071 and 16384 * 131071 < 2**31 <= 16384 * 131072
    b = torch.zeros(1, dtype=torch.int8, device="cuda")
    out = torch.zeros(1, dtype=torch.int32, device="cuda")
    with pytest.raises(VectorError) as e:
        ctx.check(ctx.lib.va_i8_scan_topk(ctx.handle, b.data_ptr(), b.data_ptr(), 1, 1, 131072, 1, out.data_ptr(),
                                          None), "va_i8_scan_topk")
    assert e.value.kind == "invalidInput" and "131071" in str(e.value)


def test_i8_sampled_and_overflow_paths(ctx, oracle):
    from vectoraccelerate_amd import ScalarQuantizationKernel, _lib

    g = rng(21)
    qc = g.integers(-128, 128, (70, 64)).astype(np.int8)
    xc = g.integers(-128, 128, (30000, 64)).astype(np.int8)
    oi, od = oracle.i8_topk(qc, xc, 10)
    for cap, sample in [(0, 1000), (64, 2000)]:
        try:
            ctx.set_option(_lib.VA_OPT_CANDIDATE_CAP, cap)
            ctx.set_option(_lib.VA_OPT_SAMPLE_ROWS, sample)
            gi, gd = ScalarQuantizationKernel(ctx).searchTopK(qc, xc, 10)
        finally:
            ctx.set_option(_lib.VA_OPT_CANDIDATE_CAP, 0)
            ctx.set_option(_lib.VA_OPT_SAMPLE_ROWS, 0)
        check_topk_exact(gi, gd, oi, od)


def test_i8_large_q_overflow_rescan(ctx, oracle):
    """Large-Q tiles on the overflow path: a tiny candidate cap sends most queries (more than
    six 32-query slot groups) to the device-side exact fallback."""
    from vectoraccelerate_amd import ScalarQuantizationKernel, _lib

    g = rng(22)
    qc = g.integers(-128, 128, (600, 128)).astype(np.int8)
    xc = g.integers(-128, 128, (40000, 128)).astype(np.int8)
    qc[5] = xc[17]
    oi, od = oracle.i8_topk(qc, xc, 20)
    try:
        ctx.set_option(_lib.VA_OPT_CANDIDATE_CAP, 24)
        ctx.set_option(_lib.VA_OPT_SAMPLE_ROWS, 3000)
        ctx.set_option(_lib.VA_OPT_SAMPLE_RANK, 2**32)  # the sample's 20th key: most lists overflow
        ctx.set_profiling(True)  # the overflow count is read back only when profiling
        gi, gd = ScalarQuantizationKernel(ctx).searchTopK(qc, xc, 20)
        t = ctx.last_scan_timings()
    finally:
        ctx.set_option(_lib.VA_OPT_CANDIDATE_CAP, 0)
        ctx.set_option(_lib.VA_OPT_SAMPLE_ROWS, 0)
        ctx.set_option(_lib.VA_OPT_SAMPLE_RANK, 0)
        ctx.set_profiling(False)
    check_topk_exact(gi, gd, oi, od)
    assert gi[5, 0] == 17
    assert t["overflow_rows"] > 192


@pytest.mark.parametrize("D", [128, 512])
def test_i8_large_q_overflow_rescan_resident_blocks(ctx, oracle, D):
    """The overflow path behind both resident-query scans (d = 128: 256-query blocks on the
    32x32x32 MFMA; d = 512: 256-query blocks on the 16x16x64 MFMA): a tiny candidate cap sends
    most queries to the device-side exact fallback."""
    from vectoraccelerate_amd import ScalarQuantizationKernel, _lib

    g = rng(23 + D)
    qc = g.integers(-128, 128, (450, D)).astype(np.int8)
    xc = g.integers(-128, 128, (30000, D)).astype(np.int8)
    qc[7] = xc[29999]
    oi, od = oracle.i8_topk(qc, xc, 16)
    try:
        ctx.set_option(_lib.VA_OPT_CANDIDATE_CAP, 20)
        ctx.set_option(_lib.VA_OPT_SAMPLE_ROWS, 2500)
        ctx.set_option(_lib.VA_OPT_SAMPLE_RANK, 2**32)
        ctx.set_profiling(True)
        gi, gd = ScalarQuantizationKernel(ctx).searchTopK(qc, xc, 16)
        t = ctx.last_scan_timings()
    finally:
        ctx.set_option(_lib.VA_OPT_CANDIDATE_CAP, 0)
        ctx.set_option(_lib.VA_OPT_SAMPLE_ROWS, 0)
        ctx.set_option(_lib.VA_OPT_SAMPLE_RANK, 0)
        ctx.set_profiling(False)
    check_topk_exact(gi, gd, oi, od)
    assert gi[7, 0] == 29999
    assert t["overflow_rows"] > 128


def test_c3_pipeline_small(ctx, oracle):
    """configs[2] pipeline at reduced size: per-dim params from the database, queries quantised
    with the database parameters, int32 dot scan, top-10 — codes and ids bit-exact."""
    from vectoraccelerate_amd import ScalarQuantizationKernel

    x, s = c3_like(50000, 512, 5)
    g = rng(6)
    q = (g.uniform(-1, 1, (64, 512)) * s).astype(np.float32)
    k = ScalarQuantizationKernel(ctx)
    p = k.computePerDimensionParameters(x)
    xc = k.quantizePerDimension(x, p)
    qc = k.quantizePerDimension(q, p)
    mn, mx, sc, zp = oracle.sq_params_per_dim(x)
    oxc = oracle.sq_quantize(x, sc, zp)
    oqc = oracle.sq_quantize(q, sc, zp)
    np.testing.assert_array_equal(xc.cpu().numpy(), oxc)
    np.testing.assert_array_equal(qc.cpu().numpy(), oqc)
    gi, gd = k.searchTopK(qc, xc, 10)
    oi, od = oracle.i8_topk(oqc, oxc, 10)
    check_topk_exact(gi, gd, oi, od)


# ---------------------------------------------------------------------------------------
# binary
# ---------------------------------------------------------------------------------------
@pytest.mark.parametrize("N,D", [(1, 1), (5, 31), (7, 32), (9, 33), (100, 768), (1000, 100), (3, 2049)])
def test_bq_pack_bit_exact(ctx, oracle, N, D):
    from vectoraccelerate_amd import BinaryQuantizationKernel

    x = rng(N * D).standard_normal((N, D)).astype(np.float32)
    x[0, 0] = 0.0
    if D > 1:
        x[0, 1] = -0.0
    got = BinaryQuantizationKernel(ctx).pack(x).cpu().numpy().view(np.uint32)
    np.testing.assert_array_equal(got, oracle.bq_pack(x))


def test_binary_known_answers(ctx):
    """KernelTests.swift:1891-2004 and :3440-3505."""
    from vectoraccelerate_amd import BinaryQuantizationKernel, HammingDistanceKernel

    b = BinaryQuantizationKernel(ctx)
    r = b.quantize([[1.0, -1.0, 1.0, -1.0], [-1.0, 1.0, -1.0, 1.0]])
    assert r.binaryVectors.count == 2 and r.binaryVectors.dimension == 4
    assert r.compressionRatio == pytest.approx(4.0, abs=0.1)
    v = b.quantize([[1.0, -1.0, 1.0, -1.0, 1.0, -1.0, 1.0, -1.0]]).binaryVectors.vector(0)
    assert v.asBoolArray() == [True, False] * 4
    for vecs, j, want in [([[1.0] * 4, [1.0] * 4], 0, 0.0), ([[1.0] * 4, [-1.0] * 4], 1, 4.0),
                          ([[1, 1, -1, -1], [1, -1, 1, -1]], 1, 2.0)]:
        res = b.quantize(vecs)
        d = b.computeHammingDistances(res.binaryVectors.vectors[0], res.binaryVectors)
        assert d.distances[j] == want
    h = HammingDistanceKernel(ctx)
    assert h.distance([True, False, True, False], [True, False, True, False]) == 0
    assert h.distance([True] * 4, [False] * 4) == 4
    assert h.distance([True, False, True, False], [True, True, False, False]) == 2
    m = h.distanceMatrix([[True, False], [False, True]], [[True, False], [False, False], [True, True]])
    np.testing.assert_array_equal(m[0], [0, 1, 1])
    assert h.packBinary([True, False, True, False, False, False, False, False]) == [0b101]
    assert h.packBinary([True] * 64) == [0xFFFFFFFF, 0xFFFFFFFF]


def test_cpu_hamming_matches_gpu(ctx):
    """KernelTests.swift:1988-2004 (testCPUHammingMatch)."""
    from vectoraccelerate_amd import BinaryQuantizationKernel

    b = BinaryQuantizationKernel(ctx)
    res = b.quantize(rng(4).uniform(-1, 1, (10, 32)).astype(np.float32))
    q = res.binaryVectors.vectors[0]
    d = b.computeHammingDistances(q, res.binaryVectors)
    for i in range(10):
        assert int(d.distances[i]) == q.hammingDistance(res.binaryVectors.vectors[i])


@pytest.mark.parametrize("Q,N,W", [(2, 3, 1), (17, 1000, 24), (5, 300, 3), (3, 500, 40)])
def test_hamming_matrix_bit_exact(ctx, oracle, Q, N, W):
    from vectoraccelerate_amd import HammingDistanceKernel

    g = rng(Q * N + W)
    q = g.integers(0, 2**32, (Q, W), dtype=np.uint64).astype(np.uint32)
    x = g.integers(0, 2**32, (N, W), dtype=np.uint64).astype(np.uint32)
    np.testing.assert_array_equal(HammingDistanceKernel(ctx).computeBitPacked(q, x), oracle.hamming_matrix(q, x))


@pytest.mark.parametrize("Q,N,W,k", [(1, 10, 1, 3), (32, 20000, 24, 100), (256, 5000, 24, 100), (7, 40000, 24, 10),
                                     (3, 2000, 40, 5), (4, 100, 3, 200),
                                     # large Q (fp4 MFMA filter scan): ragged Q and N, every row width
                                     # it takes, a database shorter than one 256-row tile
                                     (300, 20000, 8, 10), (257, 3001, 16, 50), (513, 70000, 24, 100),
                                     (450, 100, 24, 7)])
def test_hamming_topk_bit_exact(ctx, oracle, Q, N, W, k):
    from vectoraccelerate_amd import HammingDistanceKernel

    g = rng(Q + N + W + k)
    q = g.integers(0, 2**32, (Q, W), dtype=np.uint64).astype(np.uint32)
    x = g.integers(0, 2**32, (N, W), dtype=np.uint64).astype(np.uint32)
    gi, gd = HammingDistanceKernel(ctx).nearestNeighbors(q, x, k)
    oi, od = oracle.hamming_topk(q, x, k)
    check_topk_exact(gi, gd, oi, od)


def test_hamming_large_q_many_ties_and_overflow(ctx, oracle):
    """fp4 MFMA filter scan with hundreds of tied passes per query (40 distinct rows repeated),
    repeated staging flushes, and a tiny candidate cap that sends queries to the rescan."""
    from vectoraccelerate_amd import HammingDistanceKernel, _lib

    g = rng(32)
    base = g.integers(0, 2**32, (40, 24), dtype=np.uint64).astype(np.uint32)
    x = base[g.integers(0, 40, 9000)]
    q = g.integers(0, 2**32, (300, 24), dtype=np.uint64).astype(np.uint32)
    q[7] = x[123]
    oi, od = oracle.hamming_topk(q, x, 20)
    for cap, sample in [(0, 0), (32, 1000)]:
        try:
            ctx.set_option(_lib.VA_OPT_CANDIDATE_CAP, cap)
            ctx.set_option(_lib.VA_OPT_SAMPLE_ROWS, sample)
            gi, gd = HammingDistanceKernel(ctx).nearestNeighbors(q, x, 20)
        finally:
            ctx.set_option(_lib.VA_OPT_CANDIDATE_CAP, 0)
            ctx.set_option(_lib.VA_OPT_SAMPLE_ROWS, 0)
        check_topk_exact(gi, gd, oi, od)
        assert gd[7, 0] == 0


@pytest.mark.parametrize("rank", [1, 3, 0])
def test_hamming_speculative_threshold_rank(ctx, oracle, rank):
    """fp4 MFMA filter with a threshold below the sample's k-th key: queries whose exact copy
    sits on a sampled row get threshold 0 at rank 1 (one candidate) and take the fallback."""
    from vectoraccelerate_amd import HammingDistanceKernel, _lib

    g = rng(33 + rank)
    q = g.integers(0, 2**32, (260, 24), dtype=np.uint64).astype(np.uint32)
    x = g.integers(0, 2**32, (30000, 24), dtype=np.uint64).astype(np.uint32)
    x[::30][:100] = q[:100]  # 1000 sampled rows: stride 30
    oi, od = oracle.hamming_topk(q, x, 50)
    try:
        ctx.set_option(_lib.VA_OPT_SAMPLE_ROWS, 1000)
        ctx.set_option(_lib.VA_OPT_SAMPLE_RANK, rank)
        gi, gd = HammingDistanceKernel(ctx).nearestNeighbors(q, x, 50)
    finally:
        ctx.set_option(_lib.VA_OPT_SAMPLE_ROWS, 0)
        ctx.set_option(_lib.VA_OPT_SAMPLE_RANK, 0)
    check_topk_exact(gi, gd, oi, od)
    assert np.all(gd[:100, 0] == 0)


def test_hamming_sampled_and_overflow_paths(ctx, oracle):
    from vectoraccelerate_amd import HammingDistanceKernel, _lib

    g = rng(31)
    q = g.integers(0, 2**32, (20, 24), dtype=np.uint64).astype(np.uint32)
    x = g.integers(0, 2**32, (60000, 24), dtype=np.uint64).astype(np.uint32)
    oi, od = oracle.hamming_topk(q, x, 100)
    for cap, sample in [(0, 3000), (256, 3000)]:
        try:
            ctx.set_option(_lib.VA_OPT_CANDIDATE_CAP, cap)
            ctx.set_option(_lib.VA_OPT_SAMPLE_ROWS, sample)
            gi, gd = HammingDistanceKernel(ctx).nearestNeighbors(q, x, 100)
        finally:
            ctx.set_option(_lib.VA_OPT_CANDIDATE_CAP, 0)
            ctx.set_option(_lib.VA_OPT_SAMPLE_ROWS, 0)
        check_topk_exact(gi, gd, oi, od)


def test_c4_pipeline_small(ctx, oracle):
    """configs[3] at reduced size: sign bits of N(0,1) floats (768-d -> 24 words), top-100."""
    from vectoraccelerate_amd import BinaryQuantizationKernel, HammingDistanceKernel

    g = rng(41)
    xf = g.standard_normal((30000, 768)).astype(np.float32)
    qf = g.standard_normal((64, 768)).astype(np.float32)
    b = BinaryQuantizationKernel(ctx)
    xc, qc = b.pack(xf), b.pack(qf)
    np.testing.assert_array_equal(xc.cpu().numpy().view(np.uint32), oracle.bq_pack(xf))
    gi, gd = HammingDistanceKernel(ctx).nearestNeighbors(qc, xc, 100)
    oi, od = oracle.hamming_topk(oracle.bq_pack(qf), oracle.bq_pack(xf), 100)
    check_topk_exact(gi, gd, oi, od)
