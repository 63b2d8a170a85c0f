"""The board-ceiling probe (va_probe_mfma, no reference counterpart): every kind runs and reports a
positive rate and engine clock; the HBM kind's buffer size is range-checked before any launch."""
from __future__ import annotations

import ctypes as C

import pytest

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("kind,iters,ops_per_iter", [(0, 50, None), (1, 50, None), (2, 50, None), (3, 50, None),
                                                      (4, 200, None), (5, 256, 1 << 20)])
def test_probe_kinds_report_rates(ctx, kind, iters, ops_per_iter):
    from vectoraccelerate_amd import _lib

    r = _lib.ProbeResult()
    ctx.check(ctx.lib.va_probe_mfma(ctx.handle, kind, 1, iters, C.byref(r)), "va_probe_mfma")
    assert r.ms > 0 and r.ops > 0 and r.ops_per_second > 0
    assert 100.0 < r.engine_mhz < 4000.0
    if ops_per_iter:
        assert r.ops == iters * ops_per_iter  # the HBM kind counts the bytes read


def test_probe_rejects_bad_arguments(ctx):
    from vectoraccelerate_amd import _lib

    r = _lib.ProbeResult()
    assert ctx.lib.va_probe_mfma(ctx.handle, 6, 1, 10, C.byref(r)) == _lib.VA_ERR_INVALID_ARG
    assert ctx.lib.va_probe_mfma(ctx.handle, _lib.VA_PROBE_HBM, 1, 64, C.byref(r)) == _lib.VA_ERR_INVALID_ARG
    assert ctx.lib.va_probe_mfma(ctx.handle, _lib.VA_PROBE_FP16, 1, 0, C.byref(r)) == _lib.VA_ERR_INVALID_ARG
