"""Shared checks for the parity tests.

Tolerance rule for fp32 paths (north-star: fp32 distances within 1e-4 relative, top-k ids
equal except for ties within that tolerance).  The error of a distance computed as
|q|^2 + |x|^2 - 2 q.x scales with the magnitudes involved, so the relative tolerance is
taken against a per-pair scale:
    L2^2        : |q|^2 + |x|^2
    cosine dist : 1          (distances live in [0, 2])
    -dot        : |q| |x|
"""
from __future__ import annotations

import numpy as np

SENT = 0xFFFFFFFF
RTOL = 1e-4
# fp32's smallest normal number: below it a float has no relative precision to speak of (products
# of 1e-30 entries underflow to zero in any fp32 computation, the oracle's own fp32 output
# included), so distances closer than this to the float64 value count as equal.
ABS_FLOOR = float(np.finfo(np.float32).tiny)

L2SQ, COSINE, DOT, L2 = 0, 1, 2, 3


def exact_distances(metric: int, q: np.ndarray, x: np.ndarray) -> np.ndarray:
    """float64 distances of one query to rows x (independent of the oracle's C code)."""
    q64 = q.astype(np.float64)
    x64 = x.astype(np.float64)
    if metric in (L2SQ, L2):
        d = ((x64 - q64) ** 2).sum(axis=1)
        return np.sqrt(d) if metric == L2 else d
    dots = x64 @ q64
    if metric == DOT:
        return -dots
    nq = np.sqrt((q64 * q64).sum())
    nx = np.sqrt((x64 * x64).sum(axis=1))
    den = nq * nx
    with np.errstate(invalid="ignore", divide="ignore"):
        s = np.where(den < np.finfo(np.float32).tiny, 0.0, dots / np.where(den == 0, 1, den))
    s = np.where(np.isnan(s), s, np.clip(s, -1.0, 1.0))
    return 1.0 - s


def pair_scale(metric: int, q: np.ndarray, x: np.ndarray) -> np.ndarray:
    q64 = q.astype(np.float64)
    x64 = x.astype(np.float64)
    qq = (q64 * q64).sum()
    xx = (x64 * x64).sum(axis=1)
    if metric in (L2SQ, L2):
        return qq + xx
    if metric == DOT:
        return np.sqrt(qq * xx)
    return np.ones_like(xx)


def check_topk(metric: int, q: np.ndarray, x: np.ndarray, k: int, gi: np.ndarray, gd: np.ndarray | None,
               oi: np.ndarray, od: np.ndarray, rtol: float = RTOL) -> int:
    """Assert a GPU fp32 top-k equals the oracle's up to near-ties; returns #id mismatches.

    Checks per query: the GPU list has no duplicates and the same number of valid slots;
    every reported distance matches the float64 distance of its id; rank by rank the true
    distance of the GPU's id equals the oracle's distance at that rank within tolerance
    (so any id difference is a tie within tolerance); the padding matches.
    """
    gi = np.asarray(gi).astype(np.uint32)
    oi = np.asarray(oi).astype(np.uint32)
    mism = 0
    for r in range(q.shape[0]):
        gv = gi[r] != SENT
        ov = oi[r] != SENT
        assert gv.sum() == ov.sum(), f"query {r}: {gv.sum()} valid ids vs oracle {ov.sum()}"
        assert np.all(gv[: gv.sum()]), f"query {r}: sentinels must trail"
        ids = gi[r][gv].astype(np.int64)
        assert len(set(ids.tolist())) == len(ids), f"query {r}: duplicate ids {ids}"
        if len(ids) == 0:
            continue
        m = metric if metric != L2 else L2SQ
        true_d = exact_distances(m, q[r], x[ids])
        scale = pair_scale(m, q[r], x[ids])
        tol = np.maximum(rtol * np.maximum(np.abs(true_d), scale), ABS_FLOOR)
        if gd is not None:
            rep = gd[r][gv].astype(np.float64)
            if metric == L2:
                rep = rep ** 2
            bad = np.abs(rep - true_d) > tol
            assert not bad.any(), (
                f"query {r}: reported distances off at ranks {np.nonzero(bad)[0][:5]}: "
                f"{rep[bad][:5]} vs {true_d[bad][:5]}"
            )
        ref_ids = oi[r][ov].astype(np.int64)
        ref_d = exact_distances(m, q[r], x[ref_ids])
        ref_scale = pair_scale(m, q[r], x[ref_ids])
        tol2 = np.maximum(rtol * np.maximum(np.maximum(np.abs(ref_d), ref_scale), np.maximum(np.abs(true_d), scale)),
                          ABS_FLOOR)
        bad = np.abs(true_d - ref_d) > tol2
        assert not bad.any(), (
            f"query {r}: rank distances differ at {np.nonzero(bad)[0][:5]}: gpu ids {ids[bad][:5]} "
            f"({true_d[bad][:5]}) vs oracle ids {ref_ids[bad][:5]} ({ref_d[bad][:5]})"
        )
        mism += int((ids != ref_ids).sum())
    return mism


def check_topk_exact(gi, gd, oi, od):
    """Integer paths: ids and distances must be bit-identical."""
    np.testing.assert_array_equal(np.asarray(gi).astype(np.uint32), np.asarray(oi).astype(np.uint32))
    if gd is not None:
        np.testing.assert_array_equal(np.asarray(gd), np.asarray(od))
