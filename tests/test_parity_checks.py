"""Pins the parity checks the GPU tests rely on (CPU only).

A check that cannot fail pins nothing, so each one is shown to accept a
correct result computed in another f32 summation order and to reject the
plausible mistakes of a fused SiLU.up epilogue: gate and up swapped, the up
half paired one column off, and the intermediate 16-bit roundings of g and u
skipped (one rounding of silu(g) * u instead of three).  The mistakes are
planted in CPU-side results built from the oracle's pieces.
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import assert_silu_mul, ulp16


def _case(orc, dtype, m=64, inter=256, hidden=512, seed=3):
    rng = np.random.default_rng(seed)
    a = orc.h16_from_f32(rng.standard_normal((m, hidden)).astype(np.float32), dtype)
    w = orc.h16_from_f32((0.05 * rng.standard_normal((2 * inter, hidden))).astype(np.float32),
                         dtype)
    exact = orc.linear(dtype, a, w, np.zeros((m, inter), np.uint16),
                       flags=orc.EPI_SILU_MUL | orc.EXACT)
    gu_exact = orc.linear(dtype, a, w, np.zeros((m, 2 * inter), np.uint16), flags=orc.EXACT)
    return a, w, exact, gu_exact, hidden, inter


def _silu_mul16(orc, dtype, g, u):
    g = np.asarray(g, np.float64)
    act = g / (1.0 + np.exp(-g)) * np.asarray(u, np.float64)
    return orc.h16_from_f32(act.astype(np.float32), dtype)


@pytest.mark.parametrize("dtype", [0, 1], ids=["f16", "bf16"])
def test_ulp16_spacing(orc, dtype):
    mant = 10 if dtype == 0 else 7
    for x in (1.0, 1.5, -3.0, 1024.0, 2.0 ** -5):
        e = np.floor(np.log2(abs(x)))
        assert ulp16(np.array([x]), dtype)[0] == 2.0 ** (e - mant)
    # the next representable value above x is x + ulp16(x)
    x = orc.h16_from_f32(np.array([1.7, 300.0, 0.013], np.float32), dtype)
    nxt = orc.h16_to_f32(x + 1, dtype).astype(np.float64)
    cur = orc.h16_to_f32(x, dtype).astype(np.float64)
    assert np.array_equal(nxt - cur, ulp16(cur, dtype))


@pytest.mark.parametrize("dtype", [0, 1], ids=["f16", "bf16"])
def test_silu_check_accepts_other_summation_order(orc, dtype):
    """The oracle's blocked f32 GEMM (a summation order unlike the f64-exact
    one) passes: its g and u differ only by rounding ties."""
    a, w, exact, gu_exact, k, _ = _case(orc, dtype)
    f32_order = orc.linear(dtype, a, w, np.zeros_like(exact), flags=orc.EPI_SILU_MUL)
    rel = 1e-2 if dtype == 0 else 0.03
    assert_silu_mul(f32_order, exact, a, w, gu_exact, orc, dtype, k, rel_tol=rel)


@pytest.mark.parametrize("dtype", [0, 1], ids=["f16", "bf16"])
@pytest.mark.parametrize("mistake", ["swap_gate_up", "up_off_by_one", "single_rounding"])
def test_silu_check_rejects_mistakes(orc, dtype, mistake):
    a, w, exact, gu_exact, k, inter = _case(orc, dtype)
    gu = orc.h16_to_f32(gu_exact, dtype).astype(np.float64)
    g, u = gu[:, :inter], gu[:, inter:]
    if mistake == "swap_gate_up":
        bad = _silu_mul16(orc, dtype, u, g)
    elif mistake == "up_off_by_one":
        bad = _silu_mul16(orc, dtype, g, np.roll(u, 1, axis=1))
    else:
        af = orc.h16_to_f32(a, dtype).astype(np.float64)
        wf = orc.h16_to_f32(w, dtype).astype(np.float64)
        s = af @ wf.T  # unrounded g | u
        bad = _silu_mul16(orc, dtype, s[:, :inter], s[:, inter:])
    rel = 1e-2 if dtype == 0 else 0.03
    with pytest.raises(AssertionError):
        assert_silu_mul(bad, exact, a, w, gu_exact, orc, dtype, k, rel_tol=rel)
