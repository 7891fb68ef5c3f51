"""qa_linear_noalloc (the allocation-free linear) against qa_linear through
the C ABI: two calls in a row, the second with a smaller input, each with
split-K forced so the partials go through the fixed device scratch, must give
outputs identical to qa_linear's (same kernels, same split order).  The
allocation-free call runs first, on a fresh context that has never sized a
workspace, under stream capture, so a call that allocated would fail.  A forced
split whose partials exceed the scratch is refused with QA_EINVAL; without a
forced split the planner keeps within the scratch on its own.  Runs alone in a
fresh process and after the other tests (the scratch keeps the previous
call's contents, which nothing may read)."""
from __future__ import annotations

import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _h16(orc, x, dtype):
    return orc.h16_from_f32(np.asarray(x, np.float32), dtype)


def _run(c, fn, pkg, dtype, a, w, c0, flags, bias, splits, capture=False):
    da, dw, dc = c.to_device(a), c.to_device(w), c.to_device(c0)
    db = c.to_device(bias) if bias is not None else None
    m, k = a.shape
    n = w.shape[0]
    desc = pkg.linear_desc(dtype, m, n, k, da, dw, dc, flags=flags, bias=db, ldc=c0.shape[1])
    os.environ["QA_SPLITS"] = str(splits)
    try:
        if capture:
            # recorded into a graph: a call that allocated (or grew the
            # context's workspace, which refuses to under capture) would fail
            from hipgraph import Capture
            with Capture(c.stream) as cap:
                fn(desc)
            try:
                cap.replay()
            finally:
                cap.close()
        else:
            fn(desc)
    finally:
        del os.environ["QA_SPLITS"]
    out = c.download(dc, c0.shape)
    for b in (da, dw, dc, db):
        if b is not None:
            b.free()
    return out


def _both(ctx, pkg, dtype, a, w, c0, flags, bias, splits):
    """qa_linear on the session context, and qa_linear_noalloc FIRST on a fresh
    context that has never sized a workspace, under stream capture."""
    with pkg.Context(0) as fresh:
        got = _run(fresh, fresh.linear_noalloc, pkg, dtype, a, w, c0, flags, bias, splits,
                   capture=True)
    want = _run(ctx, ctx.linear, pkg, dtype, a, w, c0, flags, bias, splits)
    return want, got


@pytest.mark.parametrize("dtype", [0, 1], ids=["f16", "bf16"])
def test_noalloc_matches_linear_twice_second_smaller(ctx, pkg, orc, dtype):
    rng = np.random.default_rng(31 + dtype)
    cases = [(1024, 1024, 3072, 3, "acc"), (300, 512, 1216, 2, "silu")]  # second one smaller
    for m, n, k, splits, kind in cases:
        a = _h16(orc, rng.standard_normal((m, k)), dtype)
        w = _h16(orc, 0.02 * rng.standard_normal((n, k)), dtype)
        if kind == "acc":
            c0 = _h16(orc, rng.standard_normal((m, n)), dtype)
            bias = _h16(orc, 0.1 * rng.standard_normal(n), dtype)
            flags = pkg.ACCUMULATE
        else:
            c0 = np.zeros((m, n // 2), np.uint16)
            bias, flags = None, pkg.EPI_SILU_MUL
        want, got = _both(ctx, pkg, dtype, a, w, c0, flags, bias, splits)
        assert np.array_equal(got, want), (m, n, k, splits)
        exact = orc.linear(dtype, a, w, c0.copy(), flags=flags | orc.EXACT, bias=bias)
        g, r = orc.h16_to_f32(got, dtype), orc.h16_to_f32(exact, dtype)
        assert np.isfinite(g).all() and np.abs(g - r).mean() <= 1e-3 * (1 if dtype == 0 else 8)


def test_noalloc_refuses_partials_beyond_the_scratch(ctx, pkg, orc):
    cap = pkg.lib().qa_linear_noalloc_scratch_floats()
    assert cap == 4 << 20
    m, n, k = 1024, 2048, 1024  # 3 splits: 6 M partial floats > 4 M
    a, w = ctx.alloc(m * k * 2), ctx.alloc(n * k * 2)
    c = ctx.alloc(m * n * 2)
    d = pkg.linear_desc(0, m, n, k, a, w, c)
    os.environ["QA_SPLITS"] = "3"
    try:
        with pytest.raises(pkg.QAError) as e:
            ctx.linear_noalloc(d)
        assert e.value.code == pkg.QA_EINVAL and "scratch" in e.value.message
    finally:
        del os.environ["QA_SPLITS"]
    # unforced, the same shape runs (the planner keeps within the scratch)
    ctx.linear_noalloc(d)
    ctx.sync()
    for b in (a, w, c):
        b.free()
