"""Seeded random sweep of qa_linear against the f64-exact oracle: shapes with
ragged m, n and k, padded row strides on every operand (lda, ldb, ldc > the
row length, the padding left untouched), random epilogues (bias, residual,
GELU, SiLU.up), both 16-bit formats, and the planner's choice or a forced
tile and split count.  The same tolerance as tests/test_gpu_linear.py: within
1 ulp of the exact result (SiLU.up within its derived elementwise bound).
"""
from __future__ import annotations

import os

import numpy as np
import pytest

from conftest import assert_parity, assert_silu_mul

pytestmark = pytest.mark.gpu

SILU_REL = {0: 1e-2, 1: 0.03}
CASES = int(os.environ.get("QA_RANDOM_CASES", "40"))  # more for a longer sweep


def _h16(orc, x, dtype):
    return orc.h16_from_f32(np.asarray(x, np.float32), dtype)


def _draw(seed):
    rng = np.random.default_rng(9000 + seed)
    dtype = int(rng.integers(0, 2))
    m = int(rng.integers(1, 700))
    k = 8 * int(rng.integers(1, 300))
    kind = rng.choice(["plain", "bias", "acc", "bias_acc", "gelu", "bias_gelu", "silu"])
    nout = 4 * int(rng.integers(1, 280))
    n = 2 * nout if kind == "silu" else nout
    if kind == "silu" and n % 8:
        nout += 2
        n = 2 * nout
    pads = (8 * int(rng.integers(0, 3)), 8 * int(rng.integers(0, 3)), 4 * int(rng.integers(0, 3)))
    # -1: the planner's choice (8, TILE_256x160, is the conv loader's alone)
    tile = int(rng.choice([-1, 0, 1, 2, 3, 4, 5, 6, 7, 9]))
    splits = int(rng.integers(1, 4)) if tile >= 0 else 0
    return rng, dtype, m, n, k, nout, kind, pads, tile, splits


@pytest.mark.parametrize("seed", range(CASES))
def test_random_linear(ctx, pkg, orc, seed):
    rng, dtype, m, n, k, nout, kind, (pa, pb, pc), tile, splits = _draw(seed)
    lda, ldb, ldc = k + pa, k + pb, nout + pc
    a = _h16(orc, rng.standard_normal((m, k)), dtype)
    w = _h16(orc, 0.05 * rng.standard_normal((n, k)), dtype)
    flags = {"plain": 0, "bias": 0, "acc": pkg.ACCUMULATE, "bias_acc": pkg.ACCUMULATE,
             "gelu": pkg.EPI_GELU, "bias_gelu": pkg.EPI_GELU, "silu": pkg.EPI_SILU_MUL}[kind]
    bias = _h16(orc, 0.1 * rng.standard_normal(n), dtype) if "bias" in kind else None
    c0 = _h16(orc, rng.standard_normal((m, nout)), dtype) if "acc" in kind else \
        np.zeros((m, nout), np.uint16)
    # padded device images; the padding holds a marker that must survive
    marker = np.uint16(0x7E00)
    a_pad = np.full((m, lda), marker, np.uint16)
    a_pad[:, :k] = a
    w_pad = np.full((n, ldb), marker, np.uint16)
    w_pad[:, :k] = w
    c_pad = np.full((m, ldc), marker, np.uint16)
    c_pad[:, :nout] = c0
    if tile >= 0:
        os.environ["QA_TILE"], os.environ["QA_SPLITS"] = str(tile), str(splits)
    try:
        da, dw, dc = ctx.to_device(a_pad), ctx.to_device(w_pad), ctx.to_device(c_pad)
        db = ctx.to_device(bias) if bias is not None else None
        ctx.linear(pkg.linear_desc(dtype, m, n, k, da, dw, dc, flags=flags, bias=db,
                                   lda=lda, ldb=ldb, ldc=ldc))
        out = ctx.download(dc, c_pad.shape)
        for b in (da, dw, dc, db):
            if b is not None:
                b.free()
    finally:
        if tile >= 0:
            del os.environ["QA_TILE"], os.environ["QA_SPLITS"]
    assert (out[:, nout:] == marker).all(), "the output row padding was written"
    got = np.ascontiguousarray(out[:, :nout])
    if kind == "silu":
        exact = orc.linear(dtype, a, w, c0.copy(), flags=orc.EPI_SILU_MUL | orc.EXACT)
        gu_exact = orc.linear(dtype, a, w, np.zeros((m, n), np.uint16), flags=orc.EXACT)
        assert_silu_mul(got, exact, a, w, gu_exact, orc, dtype, k, rel_tol=SILU_REL[dtype])
    else:
        oflags = (orc.ACCUMULATE if "acc" in kind else 0) | \
                 (orc.EPI_GELU if "gelu" in kind else 0) | orc.EXACT
        exact = orc.linear(dtype, a, w, c0.copy(), flags=oflags, bias=bias)
        assert_parity(got, exact, orc, dtype, ulp_tol=1)
