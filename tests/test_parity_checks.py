"""Pins the parity checks the GPU tests rely on (CPU only).

A check that cannot fail pins nothing, so each one is shown to accept a
correct result computed in another f32 summation order and to reject the
plausible mistakes of a fused SiLU.up epilogue: gate and up swapped, the up
half paired one column off, and the intermediate 16-bit roundings of g and u
skipped (one rounding of silu(g) * u instead of three).  The mistakes are
planted in CPU-side results built from the oracle's pieces.

The attention check is pinned the same way: it accepts the GPU kernel's
arithmetic in both modes (unnormalised probabilities, scaled by 2^7 for f16,
entering the P.V product as two 16-bit terms or rounded once) and the
reference GPU path's (normalised, then rounded), each emulated here in f64
with the probabilities rounded as that arithmetic rounds them, and rejects a
causal bound one key too far, a missing 1/sqrt(hd), a wrong q-head -> kv-head
map and an unpermuted V cache.
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import REL_TOL, assert_attention, assert_silu_mul, parity_stats, ulp16


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


def _attn_inputs(orc, dtype, rows=40, q0=24, nqh=4, nkvh=2, hd=128, cap=80, seed=5):
    rng = np.random.default_rng(seed)
    h16 = lambda x: orc.h16_from_f32(x.astype(np.float32), dtype)  # noqa: E731
    q = h16(1.5 * rng.standard_normal((nqh, rows, hd)))
    kc = h16(rng.standard_normal((nkvh, cap, hd)))
    vc = h16(rng.standard_normal((nkvh, hd, cap)))
    return q, kc, vc, q0


def _attn_emulate(orc, dtype, q, kc, vc, q0, *, mode="split", causal_shift=0,
                  scale=None, kv_of=None, permute=True):
    """f64 attention with the probabilities rounded to the 16-bit format as
    `mode` says (conftest.P_ROUNDING)."""
    f = lambda b: orc.h16_to_f32(b, dtype).astype(np.float64)  # noqa: E731
    qf, kf, vf = f(q), f(kc), f(vc)
    nqh, rows, hd = qf.shape
    nkvh, cap, _ = kf.shape
    cols = orc.vperm(cap) if permute else np.arange(cap)
    vf = vf[:, :, cols]
    scale = 1.0 / np.sqrt(hd) if scale is None else scale
    kv_of = (lambda h: h // (nqh // nkvh)) if kv_of is None else kv_of
    vis = np.arange(cap)[None, :] <= (q0 + np.arange(rows) + causal_shift)[:, None]
    out = np.zeros((rows, nqh * hd))
    r16 = lambda x: f(orc.h16_from_f32(x.astype(np.float32), dtype))  # noqa: E731
    for h in range(nqh):
        kh = kv_of(h)
        s = np.where(vis, qf[h] @ kf[kh].T * scale, -np.inf)
        p = np.exp(s - s.max(axis=1, keepdims=True))
        z = p.sum(axis=1, keepdims=True)
        if mode == "p16_unscaled":
            o = r16(p / z) @ vf[kh].T
        else:
            ps = (p * (2.0 ** 7 if dtype == 0 else 1.0)).astype(np.float32)
            pr = r16(ps)
            if mode == "split":
                pr = pr + r16((ps - pr.astype(np.float32)).astype(np.float64))
            o = (pr @ vf[kh].T) / (z * (2.0 ** 7 if dtype == 0 else 1.0))
        out[:, h * hd:(h + 1) * hd] = o
    return orc.h16_from_f32(out.astype(np.float32), dtype)


@pytest.mark.parametrize("dtype", [0, 1], ids=["f16", "bf16"])
@pytest.mark.parametrize("mode", ["split", "p16", "p16_unscaled"])
def test_attention_check_accepts_rounded_probabilities(orc, dtype, mode):
    q, kc, vc, q0 = _attn_inputs(orc, dtype)
    want = orc.attention(dtype, q, kc, vc, q0)
    got = _attn_emulate(orc, dtype, q, kc, vc, q0, mode=mode)
    assert_attention(got, want, q, kc, vc, q0, orc, dtype, mode=mode)


@pytest.mark.parametrize("dtype", [0, 1], ids=["f16", "bf16"])
def test_attention_single_rounding_misses_the_north_star(orc, dtype):
    """Why the split is the default: one 16-bit rounding of the probabilities
    already exceeds the north star's max relative error on outputs near the
    relative-error floor, while the split stays within one 16-bit ulp."""
    q, kc, vc, q0 = _attn_inputs(orc, dtype, rows=120, q0=200, cap=320)
    want = orc.attention(dtype, q, kc, vc, q0)
    single = parity_stats(_attn_emulate(orc, dtype, q, kc, vc, q0, mode="p16"), want, orc, dtype)
    split = parity_stats(_attn_emulate(orc, dtype, q, kc, vc, q0, mode="split"), want, orc, dtype)
    assert single["max_rel"] > REL_TOL and split["max_rel"] <= REL_TOL, (single, split)
    assert split["max_ulp"] <= 1 and split["identical"] >= 0.99, split


@pytest.mark.parametrize("dtype", [0, 1], ids=["f16", "bf16"])
@pytest.mark.parametrize("mode", ["split", "p16"])
@pytest.mark.parametrize("mistake", ["causal_plus_one", "no_scale", "kv_head_map", "v_unpermuted"])
def test_attention_check_rejects_mistakes(orc, dtype, mode, mistake):
    q, kc, vc, q0 = _attn_inputs(orc, dtype)
    want = orc.attention(dtype, q, kc, vc, q0)
    kw = {"causal_plus_one": dict(causal_shift=1), "no_scale": dict(scale=1.0),
          "kv_head_map": dict(kv_of=lambda h: h % 2), "v_unpermuted": dict(permute=False)}[mistake]
    bad = _attn_emulate(orc, dtype, q, kc, vc, q0, mode=mode, **kw)
    with pytest.raises(AssertionError):
        assert_attention(bad, want, q, kc, vc, q0, orc, dtype, mode=mode)


def _window_emulate(orc, dtype, qkv, nh, hd, wlen, *, shift=0, scale=None):
    """f64 windowed attention with two-term 16-bit probabilities (the kernel's
    arithmetic); `shift` moves the window boundaries, `scale` replaces 1/sqrt(hd)."""
    f = lambda b: orc.h16_to_f32(b, dtype).astype(np.float64)  # noqa: E731
    r16 = lambda x: f(orc.h16_from_f32(x.astype(np.float32), dtype))  # noqa: E731
    x = f(qkv)
    s, dm = x.shape[0], nh * hd
    scale = 1.0 / np.sqrt(hd) if scale is None else scale
    out = np.zeros((s, dm))
    starts = sorted(set([0] + list(range(wlen + shift, s, wlen))))
    for i, st in enumerate(starts):
        en = starts[i + 1] if i + 1 < len(starts) else s
        for h in range(nh):
            q = x[st:en, h * hd:(h + 1) * hd]
            k = x[st:en, dm + h * hd:dm + (h + 1) * hd]
            v = x[st:en, 2 * dm + h * hd:2 * dm + (h + 1) * hd]
            sc = q @ k.T * scale
            p = np.exp(sc - sc.max(axis=1, keepdims=True))
            ps = (p * (2.0 ** 15 if dtype == 0 else 1.0)).astype(np.float32)
            pr = r16(ps)
            pr = pr + r16((ps - pr.astype(np.float32)).astype(np.float64))
            out[st:en, h * hd:(h + 1) * hd] = (pr @ v) / (p.sum(axis=1, keepdims=True)
                                                          * (2.0 ** 15 if dtype == 0 else 1.0))
    return orc.h16_from_f32(out.astype(np.float32), dtype)


@pytest.mark.parametrize("dtype", [0, 1], ids=["f16", "bf16"])
def test_window_attention_check_accepts_kernel_and_rejects_mistakes(orc, dtype):
    from conftest import assert_window_attention
    rng = np.random.default_rng(11)
    nh, hd, wlen, s = 2, 64, 24, 70
    qkv = orc.h16_from_f32((1.5 * rng.standard_normal((s, 3 * nh * hd))).astype(np.float32), dtype)
    want = orc.window_attention(dtype, qkv, nh, hd, wlen)
    assert_window_attention(_window_emulate(orc, dtype, qkv, nh, hd, wlen), want, qkv, nh, hd,
                            wlen, orc, dtype)
    for kw in (dict(shift=1), dict(scale=1.0)):
        with pytest.raises(AssertionError):
            assert_window_attention(_window_emulate(orc, dtype, qkv, nh, hd, wlen, **kw), want,
                                    qkv, nh, hd, wlen, orc, dtype)
