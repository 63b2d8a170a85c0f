"""va_fused_topk_noalloc (the allocation-free entry point) against va_fused_topk, through the C ABI.

Both entry points run the same search; the allocation-free one takes every scratch buffer from
the library's fixed per-GPU block instead of the context's arena, so its ids and distances must
equal va_fused_topk's bit for bit.  Each case runs two calls in a row on one context, the second
on a smaller input, so the second call also checks that nothing left in the shared block by the
first one leaks into its result.
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

L2SQ, COSINE, DOT, L2 = 0, 1, 2, 3


def _run(ctx, fn, metric, q, x, k):
    import torch
    from vectoraccelerate_amd import _lib
    from vectoraccelerate_amd.context import dptr

    qd, xd = ctx.buffer(q), ctx.buffer(x)
    idx = ctx.empty((q.shape[0], k), torch.int32)
    dist = ctx.empty((q.shape[0], k), torch.float32)
    idx.fill_(-7)
    dist.fill_(-7.0)
    ctx.order_after_torch()
    st = getattr(ctx.lib, fn)(ctx.handle, metric, C.c_void_p(dptr(qd)), C.c_void_p(dptr(xd)), q.shape[0], x.shape[0],
                              q.shape[1], k, C.c_void_p(dptr(idx)), C.c_void_p(dptr(dist)))
    msg = (ctx.lib.va_last_error_message(ctx.handle) or b"").decode()
    if st != _lib.VA_OK:
        return st, msg, None, None
    ctx.synchronize()
    return st, msg, idx.cpu().numpy().view(np.uint32), dist.cpu().numpy()


def _data(seed, Q, N, D):
    g = np.random.default_rng(seed)
    return g.standard_normal((Q, D)).astype(np.float32), g.standard_normal((N, D)).astype(np.float32)


def _same(ctx, metric, q, x, k, label):
    print(f"[no_alloc] {label}: metric {metric} Q={q.shape[0]} N={x.shape[0]} D={q.shape[1]} k={k}", flush=True)
    st_a, msg_a, ia, da = _run(ctx, "va_fused_topk", metric, q, x, k)
    st_b, msg_b, ib, db = _run(ctx, "va_fused_topk_noalloc", metric, q, x, k)
    assert st_a == 0, msg_a
    assert st_b == 0, msg_b
    np.testing.assert_array_equal(ib, ia)
    np.testing.assert_array_equal(db.view(np.uint32), da.view(np.uint32))


@pytest.mark.parametrize("screen", [0, 1, 2])
def test_noalloc_equals_fused_topk_two_calls(ctx, screen):
    from vectoraccelerate_amd import _lib

    ctx.set_option(_lib.VA_OPT_SCREEN, screen)
    try:
        # first call: the sampled path (screened when screen != 1); second: smaller, dense path
        q, x = _data(11 + screen, 128, 120_000, 256)
        _same(ctx, COSINE if screen != 1 else L2SQ, q, x, 100, f"screen {screen} first call")
        q2, x2 = _data(29 + screen, 37, 5_000, 100)
        _same(ctx, L2SQ if screen != 1 else DOT, q2, x2, 10, f"screen {screen} second call")
    finally:
        ctx.set_option(_lib.VA_OPT_SCREEN, 0)


def test_noalloc_overflow_path_two_calls(ctx):
    """Tiny candidate lists force the exact chunked recomputation, whose scratch must also fit."""
    from vectoraccelerate_amd import _lib

    ctx.set_option(_lib.VA_OPT_CANDIDATE_CAP, 64)
    try:
        q, x = _data(5, 70, 60_000, 64)
        _same(ctx, L2SQ, q, x, 50, "overflow first call")
        q2, x2 = _data(6, 9, 40_000, 48)
        _same(ctx, L2, q2, x2, 20, "overflow second call")
    finally:
        ctx.set_option(_lib.VA_OPT_CANDIDATE_CAP, 0)


def test_noalloc_rejects_searches_beyond_its_block(ctx):
    from vectoraccelerate_amd import _lib

    q, x = _data(7, 1024, 300_000, 8)
    print("[no_alloc] oversize: Q=1024 N=300000 D=8 k=1000", flush=True)
    st, msg, _, _ = _run(ctx, "va_fused_topk_noalloc", L2SQ, q, x, 1000)
    assert st == _lib.VA_ERR_INVALID_ARG
    assert "scratch" in msg and str(_lib.VA_NOALLOC_SCRATCH_BYTES) in msg
    # the context stays usable: a search that fits still matches
    q2, x2 = _data(8, 16, 2_000, 8)
    _same(ctx, L2SQ, q2, x2, 5, "after the rejected call")
