"""CPU tests that pin the oracle (oracle/va_oracle.c) before it is trusted as the checker.

Each oracle function is checked against something that does not share its code:
  * the reference's own known-answer tests (restated as fixtures, file:line cited);
  * numpy / scipy float64 re-derivations and brute force on small inputs;
  * closed forms and invariants (a planted mistake in any of these fails one check).
"""
from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest
import scipy.spatial.distance as ssd

from tests.helpers import COSINE, DOT, L2, L2SQ, SENT, exact_distances

GOLDEN = Path(__file__).resolve().parent / "golden"


def rng(seed):
    return np.random.default_rng(seed)


# ---------------------------------------------------------------------------------------
# distances
# ---------------------------------------------------------------------------------------
def test_l2_pairs_matches_numpy(oracle):
    g = rng(1)
    q = g.standard_normal((37, 77)).astype(np.float32)
    t = g.standard_normal((37, 77)).astype(np.float32)
    ref = ((q.astype(np.float64) - t) ** 2).sum(1)
    np.testing.assert_allclose(oracle.l2_pairs(q, t, False), ref, rtol=1e-6)
    np.testing.assert_allclose(oracle.l2_pairs(q, t, True), np.sqrt(ref), rtol=1e-6)


def test_cosine_pairs_matches_scipy(oracle):
    g = rng(2)
    q = g.standard_normal((25, 33)).astype(np.float32)
    t = g.standard_normal((25, 33)).astype(np.float32)
    ref = np.array([1.0 - ssd.cosine(q[i], t[i]) for i in range(25)])
    np.testing.assert_allclose(oracle.cosine_pairs(q, t, False), ref, rtol=1e-6, atol=1e-7)
    np.testing.assert_allclose(oracle.cosine_pairs(q, t, True), 1 - ref, rtol=1e-6, atol=1e-7)


def test_distance_matrix_matches_scipy_cdist(oracle):
    g = rng(3)
    q = g.standard_normal((9, 20)).astype(np.float32)
    x = g.standard_normal((31, 20)).astype(np.float32)
    np.testing.assert_allclose(oracle.distance_matrix("l2sq", q, x), ssd.cdist(q, x, "sqeuclidean"), rtol=1e-6)
    np.testing.assert_allclose(oracle.distance_matrix("l2", q, x), ssd.cdist(q, x, "euclidean"), rtol=1e-6)
    np.testing.assert_allclose(oracle.distance_matrix("cos_dist", q, x), ssd.cdist(q, x, "cosine"), rtol=1e-6,
                               atol=1e-7)
    dots = q.astype(np.float64) @ x.T.astype(np.float64)
    np.testing.assert_allclose(oracle.distance_matrix("dot", q, x), dots, rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(oracle.distance_matrix("abs_dot", q, x), np.abs(dots), rtol=1e-6, atol=1e-6)


def test_distance_known_answers(oracle):
    """NumericalStabilityTests.swift:354-420 and FlatIndexSearchTests.swift:577-650."""
    z = np.zeros((1, 128), np.float32)
    ones = np.ones((1, 128), np.float32)
    assert oracle.l2_pairs(z, z)[0] == 0.0
    assert abs(oracle.l2_pairs(z, ones, True)[0] - np.sqrt(128)) < 1e-4
    # cosine(0, .) = 0 by convention (FLT_MIN floor), not NaN
    assert oracle.cosine_pairs(z, z)[0] == 0.0
    assert oracle.cosine_pairs(z, ones / np.sqrt(128))[0] == 0.0
    # L2^2 known answers: [3,4,0,0] -> 25, [1,2,3,4] -> 30, [4,6,8] vs [1,2,3] -> 50, self -> 0
    assert oracle.l2_pairs(np.zeros((1, 4), np.float32), np.array([[3, 4, 0, 0]], np.float32))[0] == 25.0
    assert oracle.l2_pairs(np.zeros((1, 4), np.float32), np.array([[1, 2, 3, 4]], np.float32))[0] == 30.0
    assert oracle.l2_pairs(np.array([[4, 6, 8]], np.float32), np.array([[1, 2, 3]], np.float32))[0] == 50.0
    v = np.array([[1.5, 2.5, 3.5, 4.5]], np.float32)
    assert oracle.l2_pairs(v, v)[0] == 0.0
    # cosine +1, -1, 0 (NumericalStabilityTests.swift:1216-1270)
    a = np.array([[1, 2, 3]], np.float32)
    assert abs(oracle.cosine_pairs(a, a)[0] - 1.0) < 1e-6
    assert abs(oracle.cosine_pairs(a, -a)[0] + 1.0) < 1e-6
    assert abs(oracle.cosine_pairs(np.array([[1, 0]], np.float32), np.array([[0, 1]], np.float32))[0]) < 1e-7


def test_nan_inf_propagate(oracle):
    """NumericalStabilityTests.swift:968-1035: NaN propagates through L2, cosine and dot; Inf through L2."""
    a = np.array([[1.0, np.nan, 3.0]], np.float32)
    b = np.array([[1.0, 2.0, 3.0]], np.float32)
    assert np.isnan(oracle.l2_pairs(a, b)[0])
    assert np.isnan(oracle.cosine_pairs(a, b)[0])
    assert np.isnan(oracle.distance_matrix("dot", a, b)[0, 0])
    c = np.array([[np.inf, 0.0, 0.0]], np.float32)
    assert np.isinf(oracle.l2_pairs(c, b)[0])


# ---------------------------------------------------------------------------------------
# top-k
# ---------------------------------------------------------------------------------------
def test_topk_rows_known_answers(oracle):
    """KernelTests.swift:621-671 (TopKSelectionKernel)."""
    vals = np.array([[5, 2, 8, 1, 9, 3], [7, 4, 0.5, 6, 2.5, 1.5]], np.float32)
    idx, v = oracle.topk_rows(vals, 3)
    np.testing.assert_array_equal(idx, [[3, 1, 5], [2, 5, 4]])
    np.testing.assert_array_equal(v, [[1, 2, 3], [0.5, 1.5, 2.5]])
    idx, v = oracle.topk_rows(vals[:1], 3, mode_max=True)
    np.testing.assert_array_equal(idx, [[4, 2, 0]])
    np.testing.assert_array_equal(v, [[9, 8, 5]])
    idx, v = oracle.topk_rows(np.arange(100, dtype=np.float32)[None], 5)
    np.testing.assert_array_equal(idx, [[0, 1, 2, 3, 4]])


def test_topk_rows_matches_lexsort_with_ties(oracle):
    g = rng(4)
    vals = g.integers(0, 20, size=(13, 300)).astype(np.float32)  # many ties
    for mode_max in (False, True):
        idx, v = oracle.topk_rows(vals, 17, mode_max)
        for r in range(vals.shape[0]):
            key = -vals[r] if mode_max else vals[r]
            order = np.lexsort((np.arange(vals.shape[1]), key))[:17]
            np.testing.assert_array_equal(idx[r], order)
            np.testing.assert_array_equal(v[r], vals[r][order])


def test_topk_rows_pads_when_k_exceeds_n(oracle):
    idx, v = oracle.topk_rows(np.array([[3.0, 1.0]], np.float32), 4)
    np.testing.assert_array_equal(idx, [[1, 0, SENT, SENT]])
    assert np.isinf(v[0, 2]) and np.isinf(v[0, 3])


def test_topk_rows_nan_orders_last(oracle):
    idx, _ = oracle.topk_rows(np.array([[np.nan, 2.0, np.inf, 1.0]], np.float32), 4)
    np.testing.assert_array_equal(idx, [[3, 1, 2, 0]])


def test_flat_topk_known_answers(oracle):
    """KernelTests.swift:806-835 (query 0 over x in {1,2,0.5,3} -> idx [2,0], dist [0.25,1]) and
    FlatIndexSearchTests.swift:101-172 (ordering 0.25,1,4,9,16; tie case 0,1,1,4)."""
    ds = np.array([[1, 0, 0, 0], [2, 0, 0, 0], [0.5, 0, 0, 0], [3, 0, 0, 0]], np.float32)
    idx, d = oracle.flat_topk(L2SQ, np.zeros((1, 4), np.float32), ds, 2)
    np.testing.assert_array_equal(idx, [[2, 0]])
    np.testing.assert_allclose(d, [[0.25, 1.0]])
    ds = np.array([[3, 0, 0, 0], [1, 0, 0, 0], [2, 0, 0, 0], [0.5, 0, 0, 0], [4, 0, 0, 0]], np.float32)
    idx, d = oracle.flat_topk(L2SQ, np.zeros((1, 4), np.float32), ds, 5)
    np.testing.assert_array_equal(idx, [[3, 1, 2, 0, 4]])
    np.testing.assert_allclose(d, [[0.25, 1, 4, 9, 16]])
    ds = np.array([[-2, 0, 0, 0], [1, 0, 0, 0], [-1, 0, 0, 0], [0, 0, 0, 0]], np.float32)
    idx, d = oracle.flat_topk(L2SQ, np.zeros((1, 4), np.float32), ds, 4)
    np.testing.assert_array_equal(idx, [[3, 1, 2, 0]])
    np.testing.assert_allclose(d, [[0, 1, 1, 4]])


@pytest.mark.parametrize("metric", [L2SQ, COSINE, DOT, L2])
def test_flat_topk_matches_brute_force(oracle, metric):
    g = rng(5 + metric)
    q = g.standard_normal((7, 24)).astype(np.float32)
    x = g.standard_normal((500, 24)).astype(np.float32)
    k = 11
    for accum_double in (True, False):
        idx, d = oracle.flat_topk(metric, q, x, k, accum_double)
        for r in range(q.shape[0]):
            dd = exact_distances(metric, q[r], x)
            order = np.lexsort((np.arange(len(dd)), dd))[:k]
            np.testing.assert_array_equal(idx[r], order)
            np.testing.assert_allclose(d[r], dd[order], rtol=1e-5, atol=1e-6)


def test_flat_topk_float_port_close_to_double(oracle):
    g = rng(9)
    q = g.standard_normal((4, 768)).astype(np.float32)
    x = g.standard_normal((2000, 768)).astype(np.float32)
    i1, d1 = oracle.flat_topk(L2SQ, q, x, 10, True)
    i2, d2 = oracle.flat_topk(L2SQ, q, x, 10, False)
    np.testing.assert_allclose(d1, d2, rtol=1e-5)


def test_topk_merge(oracle):
    """merge_topk_sorted_kernel semantics (SearchAndRetrieval.metal:320-385): b ids offset by chunk_base."""
    a_i = np.array([[0, 5, SENT]], np.uint32)
    a_d = np.array([[0.1, 0.4, np.inf]], np.float32)
    b_i = np.array([[1, 2, 3]], np.uint32)
    b_d = np.array([[0.2, 0.4, 0.5]], np.float32)
    oi, od = oracle.topk_merge(a_i, a_d, b_i, b_d, 100)
    np.testing.assert_array_equal(oi, [[0, 101, 5]])
    np.testing.assert_allclose(od, [[0.1, 0.2, 0.4]])


# ---------------------------------------------------------------------------------------
# scalar int8
# ---------------------------------------------------------------------------------------
def test_sq_params_closed_form(oracle):
    x = np.array([[-1.0, 0.0, 5.0], [1.0, 0.0, 7.0], [0.5, 0.0, 6.0]], np.float32)
    mn, mx, sc, zp = oracle.sq_params_per_dim(x)
    np.testing.assert_array_equal(mn, [-1, 0, 5])
    np.testing.assert_array_equal(mx, [1, 0, 7])
    np.testing.assert_array_equal(sc, np.array([2 / 255, 1e-8, 2 / 255], np.float32))
    # zp = -128 - round_half_away(min/scale), evaluated in fp32: float32(2/255) rounds up, so
    # -1/scale = -127.49999 -> -127 -> zp = -1, and 5/scale = 637.49994 -> 637 -> zp = -765
    assert zp[0] == -1
    assert zp[1] == -128  # constant dimension: scale floors at 1e-8, min 0
    assert zp[2] == -765
    codes = oracle.sq_quantize(x, sc, zp)
    # -128.49999 -> -128; 127.49999 - 1 -> 126; 0.5/scale = 63.749996, - 1 -> 63
    np.testing.assert_array_equal(codes[:, 0], [-128, 126, 63])
    np.testing.assert_array_equal(codes[:, 1], [-128, -128, -128])


def test_sq_quantize_spans_int8_and_rounds_half_even(oracle):
    # min 0, max 255: scale 1, zp -128 -> the full int8 range
    x = np.array([[0.0], [255.0], [100.0]], np.float32)
    mn, mx, sc, zp = oracle.sq_params_per_dim(x)
    codes = oracle.sq_quantize(x, sc, zp)
    assert codes[0, 0] == -128 and codes[1, 0] == 127 and codes[2, 0] == -28
    # direct half-even cases with scale 1, zp 0
    v = np.array([[0.5, 1.5, 2.5, -0.5, -1.5, 200.0, -300.0]], np.float32)
    c = oracle.sq_quantize(v, np.ones(7, np.float32), np.zeros(7, np.int32))
    np.testing.assert_array_equal(c, [[0, 2, 2, 0, -2, 127, -128]])


def test_sq_quantize_matches_numpy_rederivation(oracle):
    g = rng(11)
    s = g.uniform(0.5, 2.0, 64).astype(np.float32)
    x = (g.uniform(-1, 1, (500, 64)) * s).astype(np.float32)
    mn, mx, sc, zp = oracle.sq_params_per_dim(x)
    np.testing.assert_array_equal(mn, x.min(0))
    np.testing.assert_array_equal(mx, x.max(0))
    sc_np = np.maximum((mx - mn) / np.float32(255), np.float32(1e-8)).astype(np.float32)
    np.testing.assert_array_equal(sc, sc_np)
    r = mn / sc_np
    zp_np = (-128 - (np.sign(r) * np.floor(np.abs(r) + 0.5))).astype(np.int32)
    np.testing.assert_array_equal(zp, zp_np)
    codes = oracle.sq_quantize(x, sc, zp)
    ref = np.clip(np.rint((x / sc_np).astype(np.float32) + zp_np.astype(np.float32)), -128, 127).astype(np.int8)
    np.testing.assert_array_equal(codes, ref)
    assert codes.min() == -128 and codes.max() == 127
    # dequantize error bounded by half a step (plus clamp at the top)
    deq = oracle.sq_dequantize(codes, sc, zp)
    assert np.all(np.abs(deq - x) <= sc * 1.01)


def test_sq_constant_and_zero_inputs_are_finite(oracle):
    """NumericalStabilityTests.swift:1295-1370: quantising zero / constant data stays finite."""
    for x in (np.zeros((4, 3), np.float32), np.full((4, 3), 2.5, np.float32)):
        mn, mx, sc, zp = oracle.sq_params_per_dim(x)
        codes = oracle.sq_quantize(x, sc, zp)
        deq = oracle.sq_dequantize(codes, sc, zp)
        assert np.all(np.isfinite(deq))


def test_i8_topk_matches_numpy(oracle):
    g = rng(12)
    qc = g.integers(-128, 128, (9, 64)).astype(np.int8)
    xc = g.integers(-128, 128, (700, 64)).astype(np.int8)
    xc[5] = xc[6]  # exact duplicate rows -> ties broken by lower id
    dots = qc.astype(np.int64) @ xc.T.astype(np.int64)
    np.testing.assert_array_equal(oracle.i8_dot_matrix(qc, xc), dots)
    idx, dist = oracle.i8_topk(qc, xc, 10)
    for r in range(9):
        order = np.lexsort((np.arange(700), -dots[r]))[:10]
        np.testing.assert_array_equal(idx[r], order)
        np.testing.assert_array_equal(dist[r], -dots[r][order])


# ---------------------------------------------------------------------------------------
# binary
# ---------------------------------------------------------------------------------------
def test_bq_pack_known_answers(oracle):
    """KernelTests.swift:3490-3500 (packBinary) and :1891-1930 (signs)."""
    x = np.array([[1, -1, 1, -1, -1, -1, -1, -1]], np.float32)
    np.testing.assert_array_equal(oracle.bq_pack(x), [[0b101]])
    np.testing.assert_array_equal(oracle.bq_pack(np.ones((1, 64), np.float32)), [[0xFFFFFFFF, 0xFFFFFFFF]])
    # > 0.0 rule: zero and -0.0 give 0 bits
    np.testing.assert_array_equal(oracle.bq_pack(np.array([[0.0, -0.0, 1e-30, -1e-30]], np.float32)), [[0b100]])


def test_bq_pack_matches_numpy_packbits(oracle):
    g = rng(13)
    x = g.standard_normal((50, 100)).astype(np.float32)
    codes = oracle.bq_pack(x)
    bits = (x > 0).astype(np.uint8)
    padded = np.zeros((50, 128), np.uint8)
    padded[:, :100] = bits
    ref = np.packbits(padded, axis=1, bitorder="little").view(np.uint32)
    np.testing.assert_array_equal(codes, ref)


def test_hamming_known_answers(oracle):
    """KernelTests.swift:1933-1985: identical 0, opposite 4, partial 2; :3463-3480 matrix."""
    codes = oracle.bq_pack(np.array([[1, 1, 1, 1], [-1, -1, -1, -1], [1, 1, -1, -1], [1, -1, 1, -1]], np.float32))
    h = oracle.hamming_matrix(codes, codes)
    assert h[0, 0] == 0 and h[0, 1] == 4 and h[2, 3] == 2
    q = oracle.bq_pack(np.array([[1, -1], [-1, 1]], np.float32))
    x = oracle.bq_pack(np.array([[1, -1], [-1, -1], [1, 1]], np.float32))
    np.testing.assert_array_equal(oracle.hamming_matrix(q, x)[0], [0, 1, 1])


def test_hamming_topk_matches_numpy(oracle):
    g = rng(14)
    q = g.integers(0, 2**32, (6, 24), dtype=np.uint64).astype(np.uint32)
    x = g.integers(0, 2**32, (3000, 24), dtype=np.uint64).astype(np.uint32)
    ref = np.unpackbits((q[:, None, :] ^ x[None]).view(np.uint8), axis=-1).sum(-1)
    np.testing.assert_array_equal(oracle.hamming_matrix(q, x), ref)
    idx, dist = oracle.hamming_topk(q, x, 100)
    for r in range(6):
        order = np.lexsort((np.arange(3000), ref[r]))[:100]  # stable: ties -> lower index
        np.testing.assert_array_equal(idx[r], order)
        np.testing.assert_array_equal(dist[r], ref[r][order])


# ---------------------------------------------------------------------------------------
# IVF
# ---------------------------------------------------------------------------------------
def test_ivf_assign_csr_probe_scan_brute_force(oracle):
    g = rng(15)
    C_, D = 16, 12
    c = (g.standard_normal((C_, D)) * 4).astype(np.float32)
    lab = g.integers(0, C_, 800)
    x = (c[lab] + g.standard_normal((800, D))).astype(np.float32)
    q = (c[g.integers(0, C_, 20)] + g.standard_normal((20, D))).astype(np.float32)
    lists = oracle.ivf_assign(x, c)
    d_xc = ssd.cdist(x, c, "sqeuclidean")
    np.testing.assert_array_equal(lists, d_xc.argmin(1))  # argmin takes the first (lowest) on ties
    off, ids = oracle.ivf_csr(lists, C_)
    assert off[0] == 0 and off[-1] == 800
    for j in range(C_):
        members = ids[off[j]:off[j + 1]]
        np.testing.assert_array_equal(members, np.nonzero(lists == j)[0])  # insertion order
    nprobe, k = 4, 10
    probes = oracle.ivf_probe(q, c, nprobe)
    d_qc = ssd.cdist(q, c, "sqeuclidean")
    for r in range(20):
        np.testing.assert_array_equal(probes[r], np.lexsort((np.arange(C_), d_qc[r]))[:nprobe])
    idx, dist = oracle.ivf_scan(q, x, off, ids, probes, k)
    for r in range(20):
        cand = np.nonzero(np.isin(lists, probes[r]))[0]
        dd = ((x[cand].astype(np.float64) - q[r]) ** 2).sum(1)
        order = np.lexsort((cand, dd))[:k]
        np.testing.assert_array_equal(idx[r], cand[order])
        np.testing.assert_allclose(dist[r], dd[order], rtol=1e-6)


def test_ivf_tie_goes_to_lowest_centroid(oracle):
    c = np.array([[1.0, 0.0], [-1.0, 0.0]], np.float32)
    x = np.array([[0.0, 0.0], [0.0, 5.0]], np.float32)
    np.testing.assert_array_equal(oracle.ivf_assign(x, c), [0, 0])


# ---------------------------------------------------------------------------------------
# committed golden vectors
# ---------------------------------------------------------------------------------------
def test_golden_fixtures_reproduce(oracle):
    """tests/golden/*.json hold reference known answers restated as data (gen script beside them)."""
    files = sorted(GOLDEN.glob("*.json"))
    assert files, "no golden fixtures"
    for f in files:
        fx = json.loads(f.read_text())
        kind = fx["kind"]
        if kind == "flat_topk":
            idx, d = oracle.flat_topk(fx["metric"], np.array(fx["queries"], np.float32),
                                      np.array(fx["dataset"], np.float32), fx["k"])
            np.testing.assert_array_equal(idx, fx["expected_idx"], err_msg=f.name)
            np.testing.assert_allclose(d, fx["expected_dist"], rtol=1e-4, atol=1e-4, err_msg=f.name)
        elif kind == "topk_rows":
            idx, v = oracle.topk_rows(np.array(fx["values"], np.float32), fx["k"], fx["mode"] == "maximum")
            np.testing.assert_array_equal(idx, fx["expected_idx"], err_msg=f.name)
            np.testing.assert_allclose(v, fx["expected_values"], rtol=1e-5, err_msg=f.name)
        elif kind == "bq_pack":
            np.testing.assert_array_equal(oracle.bq_pack(np.array(fx["vectors"], np.float32)), fx["expected_codes"],
                                          err_msg=f.name)
        elif kind == "hamming":
            q = oracle.bq_pack(np.array(fx["queries"], np.float32))
            x = oracle.bq_pack(np.array(fx["dataset"], np.float32))
            np.testing.assert_array_equal(oracle.hamming_matrix(q, x), fx["expected"], err_msg=f.name)
        elif kind == "sq":
            x = np.array(fx["vectors"], np.float32)
            mn, mx, sc, zp = oracle.sq_params_per_dim(x)
            np.testing.assert_array_equal(zp, fx["expected_zero_point"], err_msg=f.name)
            np.testing.assert_array_equal(oracle.sq_quantize(x, sc, zp), fx["expected_codes"], err_msg=f.name)
        elif kind == "sq_global":
            for case in fx["cases"]:
                codes, scale, zp = oracle.sq_global_quantize(np.array(case["data"], np.float32), case["asymmetric"])
                assert scale == np.float32(case["scale"]), (f.name, case)
                assert zp == case["zero_point"], (f.name, case)
                np.testing.assert_array_equal(codes, case["codes"], err_msg=f"{f.name} {case}")
        else:
            raise AssertionError(f"unknown fixture kind {kind} in {f.name}")


def test_sq_global_reference_properties(oracle):
    """The properties the reference's ScalarQuantizationKernel tests assert on the global int8
    path: round trip within 0.02 (KernelTests.swift:1775-1787) and order preserved over a wide
    range (:1850-1862)."""
    data = np.array([0.0, 0.25, 0.5, 0.75, 1.0, -0.25, -0.5, -0.75, -1.0], np.float32)
    codes, scale, zp = oracle.sq_global_quantize(data, False)
    back = oracle.sq_dequantize(codes.reshape(-1, 1), [scale], [zp]).reshape(-1)
    assert np.max(np.abs(back - data)) <= 0.02
    wide = np.array([-1000, -100, 0, 100, 1000], np.float32)
    c2, s2, z2 = oracle.sq_global_quantize(wide, False)
    assert np.all(np.diff(oracle.sq_dequantize(c2.reshape(-1, 1), [s2], [z2]).reshape(-1)) > 0)


def test_config1_oracle_is_self_consistent(oracle):
    """BASELINE config 1 (10,000 x 768, Q=100, L2^2 top-10): double and float oracles agree up to ties."""
    from tests.helpers import check_topk

    x = np.random.default_rng(0).standard_normal((10000, 768), dtype=np.float32)
    q = np.random.default_rng(1).standard_normal((100, 768), dtype=np.float32)
    i1, d1 = oracle.flat_topk(L2SQ, q, x, 10, True)
    i2, d2 = oracle.flat_topk(L2SQ, q, x, 10, False)
    check_topk(L2SQ, q, x, 10, i2, d2, i1, d1)
    # the nearest neighbour distance of i.i.d. N(0,1) in 768-d is ~2*768 minus a few sigma
    assert np.all(d1[:, 0] > 1000) and np.all(d1[:, 0] < 1536)


# ---------------------------------------------------------------------------
# k-means (IVF centroid training)
# ---------------------------------------------------------------------------

def _blobs(C_, D, per, seed, spread=0.05, sep=10.0):
    r = np.random.default_rng(seed)
    centers = (r.standard_normal((C_, D)) * sep).astype(np.float32)
    lab = np.repeat(np.arange(C_), per)
    r.shuffle(lab)
    x = (centers[lab] + r.standard_normal((lab.size, D)).astype(np.float32) * spread).astype(np.float32)
    return x, lab, centers


def test_kmeans_matches_sklearn_lloyd(oracle):
    """A textbook Lloyd (scikit-learn, given init, tol=0) reaches the same centroids after the
    same number of iterations; a dropped 1/count, a wrong argmin or an off-by-one iteration fails."""
    from sklearn.cluster import KMeans

    r = np.random.default_rng(5)
    x = r.standard_normal((600, 8)).astype(np.float32)
    init = x[r.choice(600, 12, replace=False)].copy()
    for iters in (1, 2, 5):
        cen, assign, dist, counts, it, conv, inertia, mm = oracle.kmeans_fit(x, init, iters, 0.0)
        assert it == iters and not conv
        km = KMeans(12, init=init.astype(np.float64), n_init=1, max_iter=iters, tol=0.0, algorithm="lloyd")
        km.fit(x.astype(np.float64))
        np.testing.assert_allclose(cen, km.cluster_centers_, rtol=1e-5, atol=1e-5)
    # the last assignment is the nearest centroid by brute force (float64), distances are L2
    d2 = ((x[:, None, :].astype(np.float64) - init_prev(oracle, x, init, 5)[None]) ** 2).sum(-1)
    np.testing.assert_array_equal(assign, d2.argmin(1))
    np.testing.assert_allclose(dist, np.sqrt(d2.min(1)), rtol=1e-5, atol=1e-6)
    np.testing.assert_array_equal(counts, np.bincount(assign, minlength=12))
    assert abs(inertia - float(np.sqrt(d2.min(1)).sum())) <= 1e-4 * inertia


def init_prev(oracle, x, init, iters):
    """Centroids the iters-th assignment saw (those after iters-1 iterations)."""
    if iters == 1:
        return init.astype(np.float64)
    return oracle.kmeans_fit(x, init, iters - 1, 0.0)[0].astype(np.float64)


def test_kmeans_blobs_converge_to_blob_means(oracle):
    x, lab, centers = _blobs(6, 16, 200, 1)
    init = centers + 0.5  # one seed near each blob
    cen, assign, dist, counts, it, conv, inertia, mm = oracle.kmeans_fit(x, init, 50, 1e-4)
    assert conv and it >= 2 and mm < 1e-4
    np.testing.assert_array_equal(assign, lab)
    means = np.stack([x[lab == c].astype(np.float64).mean(0) for c in range(6)])
    np.testing.assert_allclose(cen, means, rtol=1e-5, atol=1e-5)
    np.testing.assert_array_equal(counts, np.full(6, 200))
    # a second fit from the converged centroids stops after one iteration
    cen2, *_, it2, conv2, _, mm2 = oracle.kmeans_fit(x, cen, 50, 1e-4)
    assert it2 == 1 and conv2 and mm2 < 1e-4


def test_kmeans_empty_clusters_take_farthest_points(oracle):
    """Clusters that receive no point take, in index order, the points farthest from their
    assigned centroid (first index on ties), each point once, with count 1."""
    x = np.array([[0, 0], [1, 0], [0, 1], [10, 0], [13, 0], [10, 4]], np.float32)
    init = np.array([[100, 100], [0.3, 0.3], [-100, -100], [11, 1], [200, 0]], np.float32)
    cen, assign, dist, counts, it, conv, inertia, mm = oracle.kmeans_fit(x, init, 1, 0.0)
    np.testing.assert_array_equal(assign, [1, 1, 1, 3, 3, 3])
    d = np.sqrt(((x - init[assign]) ** 2).sum(1))
    np.testing.assert_allclose(dist, d, rtol=1e-6)
    order = sorted(range(6), key=lambda i: (-d[i], i))
    np.testing.assert_array_equal(cen[0], x[order[0]])
    np.testing.assert_array_equal(cen[2], x[order[1]])
    np.testing.assert_array_equal(cen[4], x[order[2]])
    np.testing.assert_allclose(cen[1], x[:3].mean(0), rtol=1e-6)
    np.testing.assert_allclose(cen[3], x[3:].mean(0), rtol=1e-6)
    np.testing.assert_array_equal(counts, [1, 3, 1, 3, 1])
    # ties: equal distances go to the lower point
    x2 = np.array([[1, 0], [-1, 0], [0, 1], [0, -1]], np.float32)
    init2 = np.array([[0, 0], [50, 50]], np.float32)
    cen2, assign2, *_ = oracle.kmeans_fit(x2, init2, 1, 0.0)
    np.testing.assert_array_equal(assign2, [0, 0, 0, 0])
    np.testing.assert_array_equal(cen2[1], x2[0])


def test_kmeans_zero_iterations_and_ties(oracle):
    x = np.array([[0, 0], [2, 0], [1, 0]], np.float32)
    init = np.array([[0, 0], [2, 0]], np.float32)
    cen, assign, dist, counts, it, conv, inertia, mm = oracle.kmeans_fit(x, init, 0, 1e-4)
    assert it == 0 and not conv
    np.testing.assert_array_equal(cen, init)
    np.testing.assert_array_equal(assign, [0, 1, 0])  # the midpoint ties: lower centroid
    np.testing.assert_array_equal(counts, [2, 1])
    np.testing.assert_allclose(dist, [0, 0, 1])


def test_kmeans_update_given_assignment(oracle):
    """vo_kmeans_update: cluster means (float64 reference within fp32 rounding), empty clusters
    (index order) take the unused points of largest distance, first index on ties; and one
    iteration of vo_kmeans_fit is exactly its own assignment followed by this update."""
    g = np.random.default_rng(17)
    x = g.standard_normal((900, 12)).astype(np.float32)
    old = g.standard_normal((9, 12)).astype(np.float32)
    assign = g.integers(0, 6, 900).astype(np.uint32)  # clusters 6, 7, 8 empty
    dist = g.random(900).astype(np.float32)
    dist[[5, 77]] = 2.0  # a tie: index 5 first
    cen, counts = oracle.kmeans_update(x, assign, dist, old)
    for c in range(6):
        m = x[assign == c].astype(np.float64).mean(0)
        np.testing.assert_allclose(cen[c], m, rtol=1e-5, atol=1e-6)
        assert counts[c] == (assign == c).sum()
    order = sorted(range(900), key=lambda i: (-dist[i], i))[:3]
    assert order[:2] == [5, 77]
    for j, c in enumerate((6, 7, 8)):
        np.testing.assert_array_equal(cen[c], x[order[j]])
        assert counts[c] == 1
    init = x[:9].copy()
    fc, fa, fd, fcnt, *_ = oracle.kmeans_fit(x, init, 1, 0.0)
    uc, ucnt = oracle.kmeans_update(x, fa, fd, init)
    np.testing.assert_array_equal(fc, uc)
    np.testing.assert_array_equal(fcnt, ucnt)


def test_kmeans_plusplus_properties(oracle):
    """D^2 seeding: distinct rows; with k distinct locations (each repeated) it picks one of each;
    the first row is floor(u0 * N) of the splitmix64 stream."""
    r = np.random.default_rng(2)
    x = r.standard_normal((300, 5)).astype(np.float32)
    for seed in (0, 1, 99):
        idx = oracle.kmeans_plusplus(x, 40, seed)
        assert len(set(idx.tolist())) == 40
        s = (seed + 0x9E3779B97F4A7C15) & (2**64 - 1)
        z = s
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & (2**64 - 1)
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & (2**64 - 1)
        z ^= z >> 31
        assert idx[0] == int((z >> 11) * 2.0**-53 * 300)
    locs = r.standard_normal((7, 5)).astype(np.float32) * 5
    dup = np.repeat(locs, 9, axis=0)
    for seed in range(5):
        idx = oracle.kmeans_plusplus(dup, 7, seed)
        assert sorted(set((idx // 9).tolist())) == list(range(7))


def test_kmeans_plusplus_samples_proportional_to_squared_distance(oracle):
    """Three points on a line: with the first pick fixed by the draw, the second is taken with
    probability d^2 / sum d^2 over many seeds (a d-weighted or uniform draw fails)."""
    x = np.array([[0.0], [1.0], [3.0]], np.float32)
    seen = {0: {}, 1: {}, 2: {}}
    for seed in range(3000):
        a, b = oracle.kmeans_plusplus(x, 2, seed).tolist()
        seen[a][b] = seen[a].get(b, 0) + 1
    for first, hist in seen.items():
        n = sum(hist.values())
        if n < 300:
            continue
        w = {j: float((x[j, 0] - x[first, 0]) ** 2) for j in range(3) if j != first}
        tot = sum(w.values())
        for j, wj in w.items():
            p = wj / tot
            assert abs(hist.get(j, 0) / n - p) < 4 * np.sqrt(p * (1 - p) / n) + 1e-9


# ---------------------------------------------------------------------------
# product quantization
# ---------------------------------------------------------------------------

def test_pq_sub_distance_order_and_value(oracle):
    """The four-lane fmaf order agrees with float64 to fp32 rounding, and its lane structure is
    visible: a sum that the lanes split exactly differs from a sequential one."""
    r = np.random.default_rng(0)
    for n in (1, 3, 4, 7, 12, 48, 97):
        v = r.standard_normal(n).astype(np.float32)
        c = r.standard_normal(n).astype(np.float32)
        exact = float(((v.astype(np.float64) - c) ** 2).sum())
        assert abs(oracle.pq_sub_l2sq(v, c) - exact) <= (n + 2) * 2.0**-24 * exact + 1e-30
    # squares [1, e, e, e, 0, e, e, e], e = 2^-24: the lanes hold 1, 2e, 2e, 2e and add to 1 + 6e
    # exactly; a sequential sum loses every e (1 + e rounds back to 1)
    e = 2.0**-12
    v = np.array([1.0, e, e, e, 0.0, e, e, e], np.float32)
    assert oracle.pq_sub_l2sq(v, np.zeros(8, np.float32)) == np.float32(1.0 + 6 * 2.0**-24)


def test_pq_encode_tables_adc_brute_force(oracle):
    r = np.random.default_rng(1)
    N, D, M, K = 300, 24, 6, 16
    x = r.standard_normal((N, D)).astype(np.float32)
    cb = r.standard_normal((M, K, D // M)).astype(np.float32)
    codes = oracle.pq_encode(x, cb, M, K)
    sub = x.reshape(N, M, 1, D // M).astype(np.float64) - cb[None].astype(np.float64)
    d2 = (sub ** 2).sum(-1)  # [N, M, K]
    np.testing.assert_array_equal(codes, d2.argmin(-1))
    q = r.standard_normal((5, D)).astype(np.float32)
    t = oracle.pq_tables(q, cb, M, K)
    tq = ((q.reshape(5, M, 1, D // M).astype(np.float64) - cb[None]) ** 2).sum(-1)
    np.testing.assert_allclose(t, tq, rtol=1e-5, atol=1e-6)
    adc = oracle.pq_adc(t, codes)
    ref = np.stack([t[i][np.arange(M)[None, :], codes].sum(1, dtype=np.float64) for i in range(5)])
    np.testing.assert_allclose(adc, ref, rtol=1e-5)
    # ADC of a row equals |q - decode(row)|^2 (the sub-spaces are orthogonal)
    dec = cb[np.arange(M)[None, :], codes].reshape(N, D)
    np.testing.assert_allclose(adc, ((q[:, None, :].astype(np.float64) - dec[None]) ** 2).sum(-1), rtol=1e-4)
    idx, dist = oracle.pq_search(q, cb, codes, M, K, 7)
    for i in range(5):
        order = sorted(range(N), key=lambda n: (adc[i, n], n))[:7]
        np.testing.assert_array_equal(idx[i], order)
        np.testing.assert_allclose(dist[i], np.sqrt(adc[i, order]), rtol=1e-6)


def test_pq_train_is_lloyd_per_subspace(oracle):
    """Each subspace's training equals k-means on that sub-vector slice (the k-means oracle is
    pinned against scikit-learn); the movement rule stops early on converged codebooks."""
    r = np.random.default_rng(2)
    N, D, M, K = 500, 12, 3, 8
    x = r.standard_normal((N, D)).astype(np.float32)
    init = x[r.choice(N, K, replace=False)].reshape(K, M, D // M).transpose(1, 0, 2).copy()
    cb, it = oracle.pq_train(x, init, M, K, 4, 0.0)
    assert it == 4
    from sklearn.cluster import KMeans

    for m in range(M):
        xs = x[:, m * 4:(m + 1) * 4].astype(np.float64)
        km = KMeans(K, init=init[m].astype(np.float64), n_init=1, max_iter=4, tol=0.0, algorithm="lloyd").fit(xs)
        np.testing.assert_allclose(cb[m], km.cluster_centers_, rtol=1e-4, atol=1e-5)
    cb2, it2 = oracle.pq_train(x, cb, M, K, 50, 1e-3)
    cb3, it3 = oracle.pq_train(x, cb2, M, K, 50, 1e-3)
    assert it3 == 1
