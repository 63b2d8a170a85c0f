"""The screening scan's error bound, checked on the CPU (no GPU needed).

The fp16 screen returns the fp32 scan's result exactly only if, for every pair, the fp32 key lies
in the interval [lo, hi] that va_screen_bound.hpp derives from the fp16 dot, and the scan's
linear pre-test never drops a pair whose lo is at or below the threshold.  This test builds the
bound's own source (the header the kernels compile) for the host, twice (with and without fma
contraction), and checks both properties on adversarial inputs: mixed magnitudes down to fp16
subnormals, rows whose fp16 image underflows, near-FLT_MIN norms, entries at and beyond the fp16
range, anti-correlated and near-duplicate pairs, queries spanning 16 decades.  The fp32 key is
computed in several summation orders (sequential, reversed, pairwise, fused, paired as the fp32
MFMA adds two products per step) and the screened accumulator in several orders as well (the
bound claims any order); each accumulator is checked against its own interval and pre-test.

Inputs built to reach the bound (entries just above an fp16 rounding midpoint, rows of fp16
subnormals) use at least 0.7 of the interval, so dropping or halving the fp16 term c1, the row
floor c0x (also inside the L2 bound), or a term of the pre-test's A, B, C makes these tests fail.
The norm-order term cn and the final rounding room are each below the 1/16 slack on the fp16
term, so no input separates them; they are kept because the proof needs them.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
SRC = ROOT / "tests" / "cpp" / "screen_bound_host.cpp"
L2SQ, L2, COS, NEG_DOT = 0, 1, 3, 6
F32 = np.float32


@pytest.fixture(scope="module", params=["plain", "contracted"])
def sb(request, tmp_path_factory):
    out = tmp_path_factory.mktemp("sb") / f"sb_{request.param}.so"
    flags = ["-ffp-contract=off"] if request.param == "plain" else ["-mfma", "-ffp-contract=fast"]
    if os.environ.get("VA_SANITIZE"):  # oracle/run_sanitized.sh: the harness under ASan + UBSan too
        flags += ["-g", "-fsanitize=address,undefined", "-fno-sanitize-recover=undefined"]
    proc = subprocess.run(["g++", "-std=c++17", "-O2", "-shared", "-fPIC", *flags, str(SRC), "-o", str(out)],
                          capture_output=True, text=True)
    assert proc.returncode == 0, proc.stderr
    lib = C.CDLL(str(out))
    fp = C.POINTER(C.c_float)
    lib.sb_make_bound.argtypes = [C.c_uint32, fp]
    lib.sb_query_scale.argtypes = [C.c_float, C.c_int]
    lib.sb_query_scale.restype = C.c_int
    lib.sb_bounds.argtypes = [C.c_int, fp] + [C.c_float] * 6 + [fp]
    lib.sb_bounds.restype = C.c_int
    lib.sb_pretest.argtypes = [C.c_int, fp] + [C.c_float] * 4 + [C.c_uint32, fp]
    lib.sb_key.argtypes = [C.c_float]
    lib.sb_key.restype = C.c_uint32
    lib.sb_make_bound_v.argtypes = [C.c_uint32, fp]
    lib.sb_err_norm_up.argtypes = [C.c_float, C.c_uint32]
    lib.sb_err_norm_up.restype = C.c_float
    lib.sb_bounds_v.argtypes = [fp] + [C.c_float] * 7 + [fp]
    lib.sb_bounds_v.restype = C.c_int
    lib.sb_pretest_v.argtypes = [fp] + [C.c_float] * 4 + [C.c_uint32, fp]
    lib.sb_bounds_m.argtypes = [fp, C.c_int] + [C.c_float] * 7 + [fp]
    lib.sb_bounds_m.restype = C.c_int
    return lib


def _fp(a):
    return a.ctypes.data_as(C.POINTER(C.c_float))


def _fma(a, b, c):
    # float32 fma: the exact product of two floats fits a double, one more rounding of the sum
    return F32(np.float64(a) * np.float64(b) + np.float64(c))


def _sums(p):
    """A float32 sum of the float32 terms p in several orders."""
    p = p.astype(F32)
    out = [np.cumsum(p, dtype=F32)[-1], np.cumsum(p[::-1], dtype=F32)[-1], p.sum(dtype=F32)]
    if p.size >= 2:
        pairs = (p[0::2][: p.size // 2] + p[1::2][: p.size // 2]).astype(F32)
        tail = p[-1:] if p.size % 2 else p[:0]
        out.append(np.cumsum(np.concatenate([pairs, tail]), dtype=F32)[-1])
    return [F32(v) for v in out]


def _dots(a, b):
    """float32 dot products of a and b in several orders (separate multiply-add and fused)."""
    a, b = a.astype(F32), b.astype(F32)
    out = _sums((a * b).astype(F32))
    s = F32(0)
    for x, y in zip(a, b):
        s = _fma(x, y, s)
    out.append(s)
    return out


def _key(op, dot, qq, xx):
    with np.errstate(all="ignore"):
        if op in (L2SQ, L2):
            v = F32(qq + xx - F32(2) * dot)
            v = F32(0) if v < 0 else v
            return F32(np.sqrt(v)) if op == L2 else v
        if op == NEG_DOT:
            return F32(-dot)
        den = F32(np.sqrt(qq) * np.sqrt(xx))
        raw = F32(0) if den < np.finfo(F32).tiny else F32(dot / den)
        s = raw if raw != raw else F32(min(max(raw, F32(-1)), F32(1)))
        return F32(F32(1) - s)


def _cases(rng, D):
    """(query, row) pairs of the adversarial families."""
    g = lambda *s: rng.standard_normal(s).astype(F32)  # noqa: E731
    out = []
    for _ in range(6):
        q = g(D)
        out.append((q, g(D)))                                          # plain Gaussian
        out.append((q, (g(D) * 10.0 ** rng.uniform(-7, 3, D)).astype(F32)))  # mixed magnitudes, fp16 subnormals
        out.append((q, (g(D) * F32(1e-22)).astype(F32)))               # fp16 image underflows to zero
        out.append((q, (g(D) * F32(1e-39)).astype(F32)))               # fp32 subnormal entries, near-FLT_MIN norm
        out.append((q, (-q + F32(1e-3) * g(D)).astype(F32)))           # anti-correlated
        out.append((q, (q + F32(1e-4) * g(D)).astype(F32)))            # near duplicate (cancellation)
        big = g(D)
        big[0] = F32(65000.0)
        out.append((q, big))                                           # near the fp16 maximum
        over = g(D)
        over[D // 2] = F32(7.0e4)
        out.append((q, over))                                          # beyond the fp16 range
        out.append(((g(D) * 10.0 ** rng.uniform(-8, 8, D)).astype(F32), g(D)))  # query over 16 decades
        out.append(((g(D) * F32(1e-30)).astype(F32), g(D)))            # tiny query
    return out


def _worst_cases(D):
    """Inputs that reach the bound's dominant terms.  (a) every query and row entry sits just above
    the midpoint of two fp16 values, so each rounds up by almost a unit roundoff u and the fp16
    dot exceeds the fp32 one by nearly 2u |q||x| (the fp16 part of c1); the row is (a, ..., 2a,
    ...) so that the cosine stays below its clamp and the L2 distance away from 0.  (b) the row's
    entries sit just above the midpoint of two fp16 subnormals: each product is off by almost
    2^-25 |q_i|, about c0x |q| in all (the row-side floor); with a tiny query the L2 key's own
    scale |q|^2 + |x|^2 falls below that floor, which then dominates its bound too."""
    mid = F32(1 + 2.0**-11 + 2.0**-20)
    half = D // 2
    q = np.full(D, mid, F32)
    row = np.concatenate([np.full(half, mid, F32), np.full(D - half, 2 * mid, F32)])
    sub = np.full(D, F32((1.5 + 2.0**-8) * 2.0**-24), F32)
    return [("fp16 relative", q, row, (NEG_DOT, COS, L2SQ)), ("fp16 subnormal floor", np.ones(D, F32), sub, (NEG_DOT,)),
            ("subnormal floor, tiny query", np.full(D, F32(2.0**-20), F32), sub, (L2SQ,))]


def _prep(sb, q, c0):
    sc = sb.sb_query_scale(F32(np.abs(q).max()), int(not np.all(np.isfinite(q))))
    inv = F32(2.0 ** -sc)
    q16 = (q * F32(2.0 ** sc)).astype(np.float16).astype(F32)  # the prep's RNE rounding
    qq = _sums(q * q)[0]
    return inv, q16, qq, F32(np.sqrt(qq)), F32(c0 * F32(2.0 ** -25) * inv)


@pytest.mark.parametrize("D", [4, 96, 1536])
def test_screen_interval_is_nearly_reached(sb, D):
    """The worst-case inputs stay inside [lo, hi]; where the fp16 terms dominate the bound (D up to
    96; at larger D the fp32 accumulation terms, which no simple input reaches, take over) the
    farthest fp32 key is at least 0.7 of the half-width away from the screened value, so a bound
    that drops or halves its fp16 term or its row floor fails the containment check."""
    bound = np.zeros(4, F32)
    sb.sb_make_bound(D, _fp(bound))
    for name, q, x, ops in _worst_cases(D):
        inv, q16, qq, nq, c0q = _prep(sb, q, bound[2])
        acc = _sums((q16 * x.astype(np.float16).astype(F32)).astype(F32))[0]
        for op in ops:
            reach = 0.0
            for xx in _sums(x * x):
                nx = F32(np.sqrt(xx))
                lohi = np.zeros(2, F32)
                assert sb.sb_bounds(op, _fp(bound), F32(acc * inv), qq, nq, xx, nx, c0q, _fp(lohi))
                lo, hi = (float(v) for v in lohi)
                keys = [float(_key(op, d, q2, x2)) for d in _dots(q, x) for q2 in _sums(q * q) for x2 in _sums(x * x)]
                assert all(lo <= k <= hi for k in keys), (name, op, lo, min(keys), max(keys), hi)
                s = (lo + hi) / 2
                reach = max(reach, max(abs(k - s) for k in keys) / ((hi - lo) / 2))
            if D <= 96:
                assert reach >= 0.7, (name, op, D, reach)


@pytest.mark.parametrize("D", [4, 96, 1536])
def test_screen_interval_contains_fp32_key_and_pretest_keeps_it(sb, D):
    rng = np.random.default_rng(1000 + D)
    bound = np.zeros(4, F32)
    sb.sb_make_bound(D, _fp(bound))
    c0, c0x = bound[2], F32(bound[2] * F32(2.0**-25))
    checked = passed = 0
    for q, x in _cases(rng, D):
        inv, q16, qq, nq, c0q = _prep(sb, q, c0)
        with np.errstate(over="ignore"):
            x16 = x.astype(np.float16).astype(F32)
        with np.errstate(all="ignore"):  # entries beyond the fp16 range become inf (flagged rows)
            prods = (q16 * x16).astype(F32)  # exact: two 11-bit significands
            accs = _sums(prods)  # the scan's accumulator, in several orders
        for op in (L2SQ, L2, COS, NEG_DOT):
            for xx in _sums(x * x):
                nx = F32(np.sqrt(xx))
                flagged = not (xx < F32(4.29e9)) or (op == COS and nx < F32(8) * c0x)
                xxp, nxp = (F32(np.nan), F32(np.nan)) if flagged else (xx, nx)
                keys = [_key(op, d, q2, x2) for d in _dots(q, x) for q2 in _sums(q * q)[:2] for x2 in _sums(x * x)[:2]]
                for acc in accs:
                    # the bound and the pre-test see the same accumulator (the kernel's dot = acc * 2^-sc)
                    lohi = np.zeros(2, F32)
                    ok = sb.sb_bounds(op, _fp(bound), F32(acc * inv), qq, nq, xx, nx, c0q, _fp(lohi))
                    lo, hi = lohi
                    if ok:
                        for k in keys:
                            if k == k:  # a NaN key is the largest key; nothing to contain
                                assert lo <= k <= hi, (op, D, float(lo), float(k), float(hi))
                                checked += 1
                    # the pre-test at thresholds around the interval: a pair with lo <= tau passes
                    taus = [lo, np.nextafter(lo, F32(np.inf)), hi, max(keys)] if ok else [F32(0), F32(1), F32(-1e30)]
                    for tau in taus:
                        abc = np.zeros(3, F32)
                        sb.sb_pretest(op, _fp(bound), qq, nq, inv, c0q, sb.sb_key(F32(tau)), _fp(abc))
                        if ok and not (lo <= tau):
                            continue
                        rhs = _fma(abc[0], xxp, _fma(abc[1], nxp, abc[2]))
                        assert not (acc < rhs), ("pre-test dropped a pair", op, D, float(tau), float(lo))
                        passed += 1
    assert checked > 1000 and passed > 1000


# ---- the L2^2 bound with measured rounding errors (the IVF list scan's screen) -------------------
def _err_norm(sb, v, D):
    """The kernels' error bound of a vector's fp16 image: the fp32 sum of the squared differences
    (exact in fp32) through err_norm_up.  Entries beyond the fp16 range give inf."""
    with np.errstate(all="ignore"):
        d = (v.astype(np.float16).astype(F32) - v).astype(F32)
        ss = F32(0)
        for e in d:
            ss = _fma(e, e, ss)
    return F32(sb.sb_err_norm_up(ss, D))


def _prep_v(sb, q, D):
    """inv, the scaled fp16 query as floats, |q|^2, |q| and the unscaled error bound eq."""
    sc = sb.sb_query_scale(F32(np.abs(q).max()), int(not np.all(np.isfinite(q))))
    inv = F32(2.0 ** -sc)
    qs = (q * F32(2.0 ** sc)).astype(F32)
    q16 = qs.astype(np.float16).astype(F32)
    qq = _sums(q * q)[0]
    return inv, q16, qq, F32(np.sqrt(qq)), F32(_err_norm(sb, qs, D) * inv)


@pytest.mark.parametrize("D", [4, 96, 1536])
def test_screen_v_interval_is_nearly_reached(sb, D):
    """Every entry of the query and the row just above an fp16 rounding midpoint: both round up by
    almost u of themselves, so the fp16 dot exceeds the fp32 one by nearly eq|x| + |q|ex.  The fp32
    keys stay inside [lo, hi], and where the measured-error terms dominate (D up to 96) the farthest
    reaches 0.7 of the half-width, so dropping or halving either term fails the containment."""
    b3 = np.zeros(3, F32)
    sb.sb_make_bound_v(D, _fp(b3))
    mid = F32(1 + 2.0**-11 + 2.0**-20)
    half = D // 2
    q = np.full(D, mid, F32)
    x = np.concatenate([np.full(half, mid, F32), np.full(D - half, 2 * mid, F32)])
    inv, q16, qq, nq, eq = _prep_v(sb, q, D)
    ex = _err_norm(sb, x, D)
    acc = _sums((q16 * x.astype(np.float16).astype(F32)).astype(F32))[0]
    reach = 0.0
    for xx in _sums(x * x):
        nx = F32(np.sqrt(xx))
        lohi = np.zeros(2, F32)
        assert sb.sb_bounds_v(_fp(b3), F32(acc * inv), qq, nq, eq, xx, nx, ex, _fp(lohi))
        lo, hi = (float(v) for v in lohi)
        keys = [float(_key(L2SQ, d, q2, x2)) for d in _dots(q, x) for q2 in _sums(q * q) for x2 in _sums(x * x)]
        assert all(lo <= k <= hi for k in keys), (lo, min(keys), max(keys), hi)
        s = (lo + hi) / 2
        reach = max(reach, max(abs(k - s) for k in keys) / ((hi - lo) / 2))
    if D <= 96:
        assert reach >= 0.7, (D, reach)


@pytest.mark.parametrize("D", [4, 96, 1536])
def test_screen_v_contains_fp32_key_and_pretest_keeps_it(sb, D):
    """The adversarial families of the fp16 screen (mixed magnitudes, fp16 subnormals and underflow,
    fp32 subnormals, anti-correlated and near-duplicate pairs, entries at and beyond the fp16 range,
    queries over 16 decades): with the measured error norms every fp32 L2^2 key (several summation
    orders) lies in [lo, hi] for every order of the screened accumulator, and the pre-test never
    drops a pair whose lower bound is at or below the threshold."""
    rng = np.random.default_rng(2000 + D)
    b3 = np.zeros(3, F32)
    sb.sb_make_bound_v(D, _fp(b3))
    checked = passed = 0
    for q, x in _cases(rng, D):
        inv, q16, qq, nq, eq = _prep_v(sb, q, D)
        ex = _err_norm(sb, x, D)
        with np.errstate(over="ignore"):
            x16 = x.astype(np.float16).astype(F32)
        with np.errstate(all="ignore"):
            accs = _sums((q16 * x16).astype(F32))
        for xx in _sums(x * x):
            nx = F32(np.sqrt(xx))
            flagged = not (xx < F32(4.29e9))
            xxp, nxp, exp = (F32(np.nan),) * 3 if flagged else (xx, nx, ex)
            keys = [_key(L2SQ, d, q2, x2) for d in _dots(q, x) for q2 in _sums(q * q)[:2] for x2 in _sums(x * x)[:2]]
            for acc in accs:
                lohi = np.zeros(2, F32)
                ok = sb.sb_bounds_v(_fp(b3), F32(acc * inv), qq, nq, eq, xx, nx, ex, _fp(lohi))
                lo, hi = lohi
                if ok:
                    for k in keys:
                        if k == k:
                            assert lo <= k <= hi, (D, float(lo), float(k), float(hi))
                            checked += 1
                taus = [lo, np.nextafter(lo, F32(np.inf)), hi, max(keys)] if ok else [F32(0), F32(1), F32(-1e30)]
                for tau in taus:
                    abce = np.zeros(4, F32)
                    sb.sb_pretest_v(_fp(b3), qq, nq, eq, inv, sb.sb_key(F32(tau)), _fp(abce))
                    if ok and not (lo <= tau):
                        continue
                    rhs = _fma(abce[0], xxp, _fma(abce[1], nxp, _fma(abce[2], exp, abce[3])))
                    assert not (acc < rhs), ("pre-test dropped a pair", D, float(tau), float(lo))
                    passed += 1
    assert checked > 200 and passed > 200


def test_screen_v_is_tighter_on_typical_rows(sb):
    """On Gaussian data the measured-error interval is narrower than the worst-case one (the point
    of measuring): at D = 768 at most 0.65 of its width (about 0.6)."""
    D = 768
    rng = np.random.default_rng(7)
    b4, b3 = np.zeros(4, F32), np.zeros(3, F32)
    sb.sb_make_bound(D, _fp(b4))
    sb.sb_make_bound_v(D, _fp(b3))
    ratios = []
    for _ in range(20):
        q = (rng.standard_normal(D) + 4 * rng.standard_normal(D)).astype(F32)
        x = (q + rng.standard_normal(D)).astype(F32)
        inv, q16, qq, nq, c0q = _prep(sb, q, b4[2])
        eq = _prep_v(sb, q, D)[4]
        ex = _err_norm(sb, x, D)
        acc = _sums((q16 * x.astype(np.float16).astype(F32)).astype(F32))[0]
        xx = _sums(x * x)[0]
        nx = F32(np.sqrt(xx))
        w0, w1 = np.zeros(2, F32), np.zeros(2, F32)
        assert sb.sb_bounds(L2SQ, _fp(b4), F32(acc * inv), qq, nq, xx, nx, c0q, _fp(w0))
        assert sb.sb_bounds_v(_fp(b3), F32(acc * inv), qq, nq, eq, xx, nx, ex, _fp(w1))
        ratios.append(float(w1[1] - w1[0]) / float(w0[1] - w0[0]))
    assert max(ratios) <= 0.65, ratios


# ---- every distance family with measured rounding errors (the flat screen's candidate intervals) --
@pytest.mark.parametrize("D", [4, 96, 1536])
def test_screen_m_interval_is_nearly_reached(sb, D):
    """The midpoint inputs of the measured-error test for every family: the fp32 keys stay inside
    [lo, hi], and for cosine and -dot (whose error is the dot's alone) the farthest reaches 0.7 of
    the half-width where the measured terms dominate (D up to 96), so dropping or halving the
    query's or the row's measured term fails the containment."""
    b3 = np.zeros(3, F32)
    sb.sb_make_bound_v(D, _fp(b3))
    mid = F32(1 + 2.0**-11 + 2.0**-20)
    half = D // 2
    q = np.full(D, mid, F32)
    x = np.concatenate([np.full(half, mid, F32), np.full(D - half, 2 * mid, F32)])
    inv, q16, qq, nq, eq = _prep_v(sb, q, D)
    ex = _err_norm(sb, x, D)
    acc = _sums((q16 * x.astype(np.float16).astype(F32)).astype(F32))[0]
    for op in (L2SQ, L2, COS, NEG_DOT):
        reach = 0.0
        for xx in _sums(x * x):
            nx = F32(np.sqrt(xx))
            lohi = np.zeros(2, F32)
            assert sb.sb_bounds_m(_fp(b3), op, F32(acc * inv), qq, nq, eq, xx, nx, ex, _fp(lohi))
            lo, hi = (float(v) for v in lohi)
            keys = [float(_key(op, d, q2, x2)) for d in _dots(q, x) for q2 in _sums(q * q) for x2 in _sums(x * x)]
            assert all(lo <= k <= hi for k in keys), (op, lo, min(keys), max(keys), hi)
            s = (lo + hi) / 2
            reach = max(reach, max(abs(k - s) for k in keys) / ((hi - lo) / 2))
        if D <= 96 and op in (COS, NEG_DOT):
            assert reach >= 0.7, (op, D, reach)


@pytest.mark.parametrize("D", [4, 96, 1536])
def test_screen_m_contains_fp32_key(sb, D):
    """The adversarial families: with the measured error norms every fp32 key of every family
    (several summation orders of the dot and of both norms) lies in [lo, hi] for every order of
    the screened accumulator, and the interval lies inside the worst-case one's reach (a pair the
    worst-case bound cannot bound is not bounded here either, or its interval still holds)."""
    rng = np.random.default_rng(3000 + D)
    b3 = np.zeros(3, F32)
    sb.sb_make_bound_v(D, _fp(b3))
    checked = 0
    for q, x in _cases(rng, D):
        inv, q16, qq, nq, eq = _prep_v(sb, q, D)
        ex = _err_norm(sb, x, D)
        with np.errstate(over="ignore"):
            x16 = x.astype(np.float16).astype(F32)
        with np.errstate(all="ignore"):
            accs = _sums((q16 * x16).astype(F32))
        for op in (L2SQ, L2, COS, NEG_DOT):
            for xx in _sums(x * x):
                nx = F32(np.sqrt(xx))
                keys = [_key(op, d, q2, x2) for d in _dots(q, x) for q2 in _sums(q * q)[:2] for x2 in _sums(x * x)[:2]]
                for acc in accs:
                    lohi = np.zeros(2, F32)
                    if not sb.sb_bounds_m(_fp(b3), op, F32(acc * inv), qq, nq, eq, xx, nx, ex, _fp(lohi)):
                        continue
                    lo, hi = lohi
                    for k in keys:
                        if k == k:
                            assert lo <= k <= hi, (op, D, float(lo), float(k), float(hi))
                            checked += 1
    assert checked > 1000


def test_screen_m_cosine_is_tighter_on_typical_rows(sb):
    """The point of measuring: on Gaussian rows at D = 1536 the cosine interval with measured
    errors is at most 0.8 of the worst-case width (about 0.65: the fp32 accumulation terms, which
    both share, dominate at this D)."""
    D = 1536
    rng = np.random.default_rng(11)
    b4, b3 = np.zeros(4, F32), np.zeros(3, F32)
    sb.sb_make_bound(D, _fp(b4))
    sb.sb_make_bound_v(D, _fp(b3))
    ratios = []
    for _ in range(20):
        q = rng.standard_normal(D).astype(F32)
        x = (q + 3 * rng.standard_normal(D)).astype(F32)
        inv, q16, qq, nq, c0q = _prep(sb, q, b4[2])
        eq = _prep_v(sb, q, D)[4]
        ex = _err_norm(sb, x, D)
        acc = _sums((q16 * x.astype(np.float16).astype(F32)).astype(F32))[0]
        xx = _sums(x * x)[0]
        nx = F32(np.sqrt(xx))
        w0, w1 = np.zeros(2, F32), np.zeros(2, F32)
        assert sb.sb_bounds(COS, _fp(b4), F32(acc * inv), qq, nq, xx, nx, c0q, _fp(w0))
        assert sb.sb_bounds_m(_fp(b3), COS, F32(acc * inv), qq, nq, eq, xx, nx, ex, _fp(w1))
        ratios.append(float(w1[1] - w1[0]) / float(w0[1] - w0[0]))
    assert max(ratios) <= 0.8, ratios
