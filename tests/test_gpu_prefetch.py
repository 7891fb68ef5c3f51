"""qa_prefetch_hint: the projection launch that takes a hint over also loads
the named bytes (one dword per 128-byte line) so the NEXT launch finds them in
the memory-side cache.  The hint must never change a result: every tile
shape, with and without split-K, with a ring deeper and shallower than K
(the MMA waves that also issue the DMA then prefetch, or skip it), and every
epilogue, must give the same bits with a hint as without, and those bits
stay within 1 ulp of the f64-exact oracle.  Also: the hint is consumed by one
launch, and a null pointer with a byte count is refused.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np
import pytest

from conftest import assert_parity

pytestmark = pytest.mark.gpu

HINT_BYTES = 40 << 20  # more than any launch below can touch (16-32 MB)


def _h16(orc, x, dtype):
    return orc.h16_from_f32(np.asarray(x, np.float32), dtype)


@pytest.fixture(scope="module")
def hint_buf(ctx):
    b = ctx.alloc(HINT_BYTES)
    yield b
    b.free()


def _linear(ctx, pkg, dtype, da, dw, dc, m, n, k, ldc, flags, db, hint):
    if hint is not None:
        ctx.prefetch_hint(hint)
    ctx.linear(pkg.linear_desc(dtype, m, n, k, da, dw, dc, flags=flags, bias=db, ldc=ldc))


# TILE_256x192 (9) has a 2-stage ring whose MMA waves issue their own DMA:
# the prefetch loads share their vmcnt stream; k = 64 is shorter than its ring.
@pytest.mark.parametrize("dtype", [0, 1], ids=["f16", "bf16"])
@pytest.mark.parametrize("k", [128, 1216])
@pytest.mark.parametrize("tile,splits", [(t, 1) for t in range(8)] + [(5, 3), (7, 2), (9, 1), (9, 2)])
def test_hint_leaves_results_unchanged(ctx, pkg, orc, hint_buf, tile, splits, k, dtype):
    _hint_case(ctx, pkg, orc, hint_buf, tile, splits, k, dtype)


@pytest.mark.parametrize("dtype", [0, 1], ids=["f16", "bf16"])
def test_hint_with_k_shorter_than_the_ring(ctx, pkg, orc, hint_buf, dtype):
    _hint_case(ctx, pkg, orc, hint_buf, 9, 1, 64, dtype)


def _hint_case(ctx, pkg, orc, hint_buf, tile, splits, k, dtype):
    rng = np.random.default_rng(7000 + 10 * tile + splits + k + dtype)
    m, n = 300, 512
    a = _h16(orc, rng.standard_normal((m, k)), dtype)
    w = _h16(orc, 0.02 * rng.standard_normal((n, k)), dtype)
    gw = _h16(orc, 0.05 * rng.standard_normal((512, k)), dtype)
    c0 = _h16(orc, rng.standard_normal((m, n)), dtype)
    bias = _h16(orc, 0.1 * rng.standard_normal(n), dtype)
    da, dw, dg, db = ctx.to_device(a), ctx.to_device(w), ctx.to_device(gw), ctx.to_device(bias)
    os.environ["QA_TILE"], os.environ["QA_SPLITS"] = str(tile), str(splits)
    out = {}
    try:
        for hinted in (False, True):
            hint = hint_buf if hinted else None
            dc = ctx.to_device(c0)
            _linear(ctx, pkg, dtype, da, dw, dc, m, n, k, n, pkg.ACCUMULATE, db, hint)
            dgel = ctx.to_device(np.zeros_like(c0))
            _linear(ctx, pkg, dtype, da, dw, dgel, m, n, k, n, pkg.EPI_GELU, db, hint)
            dact = ctx.to_device(np.zeros((m, 256), np.uint16))
            _linear(ctx, pkg, dtype, da, dg, dact, m, 512, k, 256, pkg.EPI_SILU_MUL, None, hint)
            out[hinted] = [ctx.download(dc, c0.shape), ctx.download(dgel, c0.shape),
                           ctx.download(dact, (m, 256))]
            for b in (dc, dgel, dact):
                b.free()
    finally:
        del os.environ["QA_TILE"], os.environ["QA_SPLITS"]
        for b in (da, dw, dg, db):
            b.free()
    for x, y in zip(out[False], out[True]):
        assert np.array_equal(x, y), "a prefetch hint changed a result"
    exact = orc.linear(dtype, a, w, c0.copy(), flags=orc.ACCUMULATE | orc.EXACT, bias=bias)
    assert_parity(out[True][0], exact, orc, dtype, ulp_tol=1)


def test_hint_arguments(ctx, pkg, hint_buf):
    lib = pkg.lib()
    assert lib.qa_prefetch_hint(ctx.handle, None, 5) == pkg.QA_EINVAL
    assert "null pointer" in pkg.last_error()
    assert lib.qa_prefetch_hint(ctx.handle, None, 0) == pkg.QA_OK  # clears
    assert lib.qa_prefetch_hint(ctx.handle, hint_buf.ptr, 0) == pkg.QA_OK
    # a hint a projection never takes over (no launch follows) is harmless
    ctx.prefetch_hint(hint_buf, 100)
    ctx.sync()
    assert lib.qa_prefetch_hint(ctx.handle, None, 0) == pkg.QA_OK  # leave none behind


def _events(n):
    import ctypes
    from hipgraph import hip
    L = hip()
    L.hipEventCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
    L.hipEventDestroy.argtypes = [ctypes.c_void_p]
    ev = [ctypes.c_void_p() for _ in range(n)]
    for e in ev:
        assert L.hipEventCreate(ctypes.byref(e)) == 0
    return ev


def test_calls_that_launch_nothing_drop_the_hint_and_events(pkg, orc):
    """A hint and timing events set before a call that launches nothing (m = 0,
    a refused descriptor, a fused MLP of zero rows) end with that call: the
    hinted buffer is freed afterwards, and the next projection is captured
    into a graph (which refuses leftover timing events) and replays to the
    same bits as an eager launch."""
    from hipgraph import Capture, hip
    rng = np.random.default_rng(78)
    m, n, k = 256, 512, 1024
    a = _h16(orc, rng.standard_normal((m, k)), 0)
    w = _h16(orc, 0.02 * rng.standard_normal((n, k)), 0)
    with pkg.Context(0) as fresh:
        lib = pkg.lib()
        da, dw = fresh.to_device(a), fresh.to_device(w)
        dc, want_buf = fresh.alloc(m * n * 2), fresh.alloc(m * n * 2)
        fresh.linear(pkg.linear_desc(0, m, n, k, da, dw, want_buf))
        want = fresh.download(want_buf, (m, n))
        ev = _events(2)
        try:
            bad = pkg.linear_desc(0, m, n, 12, da, dw, dc)  # k not a multiple of 8
            zero = pkg.linear_desc(0, 0, n, k, da, dw, dc)
            mlp0 = pkg.MlpDesc(dtype=0, flags=0, m=0, hidden=k, inter=n, x=da.ptr, w_gu=dw.ptr,
                               w_down=dw.ptr, act=dc.ptr, h=want_buf.ptr)
            calls = [lambda: fresh.linear(zero), lambda: fresh.linear_noalloc(zero),
                     lambda: fresh.mlp_fused(mlp0)]
            for call in calls + ["bad"]:
                doomed = fresh.alloc(8 << 20)
                fresh.prefetch_hint(doomed)
                pkg.check(lib.qa_time_next_launch(fresh.handle, ev[0], ev[1]))
                if call == "bad":
                    with pytest.raises(pkg.QAError):
                        fresh.linear(bad)
                else:
                    call()
                doomed.free()
                fresh.sync()
                with Capture(fresh.stream) as cap:
                    fresh.linear(pkg.linear_desc(0, m, n, k, da, dw, dc))
                try:
                    for _ in range(3):
                        fresh.upload(dc, np.zeros((m, n), np.uint16))
                        cap.replay()
                        assert np.array_equal(fresh.download(dc, (m, n)), want)
                finally:
                    cap.close()
        finally:
            for e in ev:
                hip().hipEventDestroy(e)


def test_fused_mlp_with_and_without_a_caller_hint(ctx, pkg, orc, hint_buf):
    """qa_mlp_fused prefetches its down weights during gate|up, or keeps a
    caller's hint for the gate|up launch: same bits either way."""
    rng = np.random.default_rng(77)
    m, hid, inter = 256, 1024, 3072
    x = _h16(orc, rng.standard_normal((m, hid)), 0)
    wgu = _h16(orc, 0.02 * rng.standard_normal((2 * inter, hid)), 0)
    wd = _h16(orc, 0.02 * rng.standard_normal((hid, inter)), 0)
    dx, dgu, dd = ctx.to_device(x), ctx.to_device(wgu), ctx.to_device(wd)
    res = []
    for hinted in (False, True):
        dact = ctx.alloc(m * inter * 2)
        dh = ctx.to_device(x)
        if hinted:
            ctx.prefetch_hint(hint_buf)
        ctx.mlp_fused(pkg.MlpDesc(dtype=0, flags=0, m=m, hidden=hid, inter=inter, x=dx.ptr,
                                  w_gu=dgu.ptr, w_down=dd.ptr, act=dact.ptr, h=dh.ptr))
        res.append(ctx.download(dh, x.shape))
        dact.free()
        dh.free()
    for b in (dx, dgu, dd):
        b.free()
    assert np.array_equal(res[0], res[1])


@pytest.mark.parametrize("tile", [0, 5, 6, 7])
def test_hint_with_a_batched_call(ctx, pkg, orc, hint_buf, tile):
    """Batched problems (only the first problem's blocks prefetch): same bits
    with and without a hint, each problem equal to its own single call."""
    rng = np.random.default_rng(7100 + tile)
    b, m, n, k = 3, 200, 256, 640
    a = _h16(orc, rng.standard_normal((b, m, k)), 0)
    w = _h16(orc, 0.02 * rng.standard_normal((b, n, k)), 0)
    da, dw = ctx.to_device(a), ctx.to_device(w)
    os.environ["QA_TILE"] = str(tile)
    outs = []
    try:
        for hinted in (False, True):
            dc = ctx.alloc(b * m * n * 2)
            if hinted:
                ctx.prefetch_hint(hint_buf)
            ctx.linear(pkg.linear_desc(0, m, n, k, da, dw, dc, batch=b, bsa=m * k, bsb=n * k,
                                       bsc=m * n))
            outs.append(ctx.download(dc, (b, m, n)))
            dc.free()
    finally:
        del os.environ["QA_TILE"]
        da.free()
        dw.free()
    assert np.array_equal(outs[0], outs[1])
    for i in range(b):
        want = orc.linear(0, a[i], w[i], np.zeros((m, n), np.uint16), flags=orc.EXACT)
        assert_parity(outs[1][i], want, orc, 0, ulp_tol=1)
