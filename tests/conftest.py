"""Shared fixtures.

`-m gpu` tests need an MI355X and call the product through the C ABI
(csrc/libqa.so); everything else runs on the CPU.  The oracle
(oracle/liboracle.so) is the checker in both.
"""
from __future__ import annotations

import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

import __graft_entry__ as entry  # noqa: E402


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def _ensure_built() -> None:
    pkg_lib = os.path.join(entry.PKG_DIR, "csrc", "libqa.so")
    host_lib = os.path.join(entry.PKG_DIR, "csrc", "libqa_host.so")
    orc_lib = os.path.join(ROOT, "oracle", "liboracle.so")
    if not (os.path.exists(pkg_lib) and os.path.exists(host_lib) and os.path.exists(orc_lib)):
        entry.build()


@pytest.fixture(scope="session")
def pkg():
    _ensure_built()
    return entry.load_package()


@pytest.fixture(scope="session")
def orc():
    _ensure_built()
    return entry.load_oracle()


@pytest.fixture(scope="session")
def ctx(pkg):
    c = pkg.Context(0)
    yield c
    c.close()


def parity_stats(got_bits: np.ndarray, want_bits: np.ndarray, orc, dtype: int) -> dict:
    """The north star's statistics: max relative error with the
    max(|r|, 1e-3 max|r|) floor, mean absolute error, share of bit-identical
    16-bit outputs and the largest distance in units in the last place."""
    g = orc.h16_to_f32(got_bits, dtype).astype(np.float64)
    r = orc.h16_to_f32(want_bits, dtype).astype(np.float64)
    err = np.abs(g - r)
    floor = 1e-3 * max(np.abs(r).max(), 1e-30)
    rel = err / np.maximum(np.abs(r), floor)

    def ordinal(bits):
        b = bits.astype(np.int64)
        return np.where(b & 0x8000, -(b & 0x7FFF), b)

    # ulp distance where |r| is above the floor: near zero, the f32
    # accumulation error of any summation order spans several subnormal ulps.
    ulp = np.abs(ordinal(got_bits) - ordinal(want_bits))[np.abs(r) >= floor]
    return {
        "max_rel": float(rel.max()) if rel.size else 0.0,
        "mae": float(err.mean()) if err.size else 0.0,
        "identical": float((got_bits == want_bits).mean()) if err.size else 1.0,
        "max_ulp": int(ulp.max()) if ulp.size else 0,
        "finite": bool(np.isfinite(g).all()),
    }


# North-star gate for 16-bit outputs: max relative error <= 1e-2 and mean
# absolute error <= 1e-3 against the reference CPU path on identical inputs.
REL_TOL = 1e-2
MAE_TOL = 1e-3


def assert_parity(got_bits, want_bits, orc, dtype, rel_tol=REL_TOL, mae_tol=MAE_TOL, ulp_tol=None):
    s = parity_stats(got_bits, want_bits, orc, dtype)
    assert s["finite"], s
    assert s["max_rel"] <= rel_tol and s["mae"] <= mae_tol, s
    if ulp_tol is not None:
        assert s["max_ulp"] <= ulp_tol, s
    return s


def ulp16(x: np.ndarray, dtype: int) -> np.ndarray:
    """Spacing of the 16-bit format (f16 or bf16) at |x|, in float64."""
    mant, emin = (10, -14) if dtype == 0 else (7, -126)
    ax = np.abs(np.asarray(x, np.float64))
    e = np.floor(np.log2(np.where(ax > 0, ax, 1.0)))
    e = np.maximum(np.where(ax > 0, e, emin), emin)
    return np.exp2(e - mant)


def silu_mul_bound(a_bits, w_bits, gu_exact_bits, want_bits, orc, dtype, k):
    """Elementwise bound on |act_gpu - act_exact| for act = r(silu(r(g)) * r(u)).

    The GPU's rounded g and u (r = 16-bit RNE) are each within one ulp of the
    exactly rounded value plus the f32 accumulation error of its sum, at most
    (K/16 + 2) * 2^-24 * sum_k |a_k w_k|: each 32x32x16 MFMA adds 16 exact
    f16/bf16 products into the f32 accumulator (K/16 accumulations along a
    k chain, counting the k-group merge), the classic gamma_n bound.  That
    perturbation propagates through silu(g) * u with the first-order terms
    |silu'(g) u| dg and |silu(g)| du, the cross term max|silu'| dg du
    (silu' <= 1.1) and the curvature term max|silu''| dg^2 |u| / 2
    (silu'' <= 0.5); the final rounding adds one ulp of the result, and the
    f32 evaluation of silu a few f32 ulps (1e-6 relative)."""
    n = gu_exact_bits.shape[1] // 2
    gu = orc.h16_to_f32(gu_exact_bits, dtype).astype(np.float64)
    g, u = gu[:, :n], gu[:, n:]
    af = np.abs(orc.h16_to_f32(a_bits, dtype).astype(np.float64))
    wf = np.abs(orc.h16_to_f32(w_bits, dtype).astype(np.float64))
    sabs = af @ wf.T
    eps = (k / 16.0 + 2.0) * 2.0 ** -24 * sabs
    dg = ulp16(g, dtype) + eps[:, :n]
    du = ulp16(u, dtype) + eps[:, n:]
    sig = 1.0 / (1.0 + np.exp(-g))
    silu = g * sig
    dsilu = sig * (1.0 + g * (1.0 - sig))
    want = orc.h16_to_f32(want_bits, dtype).astype(np.float64)
    return (np.abs(dsilu * u) * dg + (np.abs(silu) + 1.1 * dg) * du + 0.25 * dg * dg * np.abs(u)
            + ulp16(want, dtype) + 1e-6 * np.abs(silu * u))


def assert_silu_mul(got_bits, want_bits, a_bits, w_bits, gu_exact_bits, orc, dtype, k,
                    rel_tol=REL_TOL, min_identical=0.97):
    """SiLU.up output against the exactly rounded reference: the north-star
    statistics, the propagated-rounding bound elementwise, and a floor on the
    share of bit-identical outputs (differences come only from rounding ties
    the f32 summation order moves, a small share)."""
    s = assert_parity(got_bits, want_bits, orc, dtype, rel_tol=rel_tol)
    bound = silu_mul_bound(a_bits, w_bits, gu_exact_bits, want_bits, orc, dtype, k)
    got = orc.h16_to_f32(got_bits, dtype).astype(np.float64)
    want = orc.h16_to_f32(want_bits, dtype).astype(np.float64)
    excess = np.abs(got - want) - bound
    worst = np.unravel_index(np.argmax(excess), excess.shape)
    assert excess.max() <= 0, (s, worst, got[worst], want[worst], bound[worst])
    assert s["identical"] >= min_identical, s
    return s


# Rounding of the probabilities before the P.V product, per attention mode:
# (relative, absolute) error per weight, for (f16, bf16).
#   split: p (scaled by 2^7 for f16) enters as two 16-bit terms, value and
#          rounding residue: the residue's own rounding, 2^-11 * 2^-11 (f16) or
#          2^-8 * 2^-8 (bf16) relative; subnormal residues cost 2^-25 * 2^-7.
#   p16:   p (scaled by 2^7 for f16) rounded once: 2^-11 / 2^-8 relative,
#          and 2^-25 * 2^-7 absolute below the f16 normal range.
# (The kernel's running max may lag the row max by up to 2^8, so its p reach
# 2^8 before scaling; relative rounding errors are the same at any scale.)
#   p16_unscaled: p in [0, 1] rounded once (the reference GPU path's
#          normalised 16-bit probabilities): f16 subnormals below 2^-14 add
#          2^-25 absolute.
P_ROUNDING = {
    "split": ((2.0 ** -22, 2.0 ** -32), (2.0 ** -16, 0.0)),
    "p16": ((2.0 ** -11, 2.0 ** -32), (2.0 ** -8, 0.0)),
    "p16_unscaled": ((2.0 ** -11, 2.0 ** -25), (2.0 ** -8, 0.0)),
}


def _attention_bound_rows(q, k, v, vis, dtype, mode):
    """Bound rows [rows, hd] for one head: q [rows, hd], k, v [keys, hd] (f64),
    vis [rows, keys] the keys each row attends to (see attention_bound)."""
    hd = q.shape[1]
    kend = k.shape[0]
    scale = 1.0 / np.sqrt(hd)
    u_p, u_abs = P_ROUNDING[mode][dtype]
    gam = (hd + 16) * 2.0 ** -24
    acc = (2 * kend + 16) * 2.0 ** -24 + 2.0 ** -20
    s = q @ k.T * scale
    sabs = np.abs(q) @ np.abs(k).T * scale
    s = np.where(vis, s, -np.inf)
    p = np.exp(s - s.max(axis=1, keepdims=True))
    z = p.sum(axis=1, keepdims=True)
    smax = np.where(vis, np.abs(s), 0.0).max(axis=1, keepdims=True)
    d = gam * np.where(vis, sabs, 0.0).max(axis=1, keepdims=True) + 6 * 2.0 ** -24 * smax
    va = np.abs(v)
    wabs = (p @ va) / z
    return (u_p + np.expm1(2 * d) + acc) * wabs + u_abs * (vis.astype(np.float64) @ va) / z


def attention_bound(q_bits, kc_bits, vc_bits, q0, want_bits, orc, dtype, mode="split"):
    """Elementwise bound on |out_gpu - out_ref| for causal GQA attention.

    Both sides compute s = q.k / sqrt(hd) in f32, p = exp(s - max) and
    out = r(sum_t p_t v_t / sum_t p_t) with one 16-bit rounding r.  They may
    differ by
      * the f32 score error: each side's dot product is within
        (hd + 16) 2^-24 sum_i |q_i k_i| / sqrt(hd) of the exact score (a
        gamma_n bound covering both the 4-way partial sums and the MFMA
        chain), and the exp argument's roundings (4 2^-24 |s| log2 e); a
        score perturbation d moves every normalised weight by a factor
        within exp(+-2d), so the weighted mean by expm1(2d) sum_t w_t |v_t|;
      * P rounded to the 16-bit format before the P.V product, as `mode`
        says (P_ROUNDING): relative u_p times sum_t w_t |v_t|, absolute
        u_abs times sum_t |v_t| / sum_t p_t;
      * the f32 accumulation over the kend visible keys on each side,
        (2 kend + 16) 2^-24 sum_t w_t |v_t|, and the exp / merge roundings,
        2^-20 relative;
      * the final rounding of each side: one ulp of the result.
    q [nqh, rows, hd], k cache [nkvh, cap, hd], transposed V cache
    [nkvh, hd, cap] (key t at column vperm(t)), bits of the 16-bit format."""
    q = orc.h16_to_f32(q_bits, dtype).astype(np.float64)
    kf = orc.h16_to_f32(kc_bits, dtype).astype(np.float64)
    vf = orc.h16_to_f32(vc_bits, dtype).astype(np.float64)
    nqh, rows, hd = q.shape
    nkvh, cap, _ = kf.shape
    rep = nqh // nkvh
    kend = q0 + rows
    vf = vf[:, :, orc.vperm(cap)[:kend]]  # [nkvh, hd, key]
    vis = np.arange(kend)[None, :] <= (q0 + np.arange(rows))[:, None]
    bound = np.zeros((rows, nqh * hd))
    for h in range(nqh):
        kh = h // rep
        bound[:, h * hd:(h + 1) * hd] = _attention_bound_rows(q[h], kf[kh, :kend], vf[kh].T, vis,
                                                              dtype, mode)
    want = orc.h16_to_f32(want_bits, dtype).astype(np.float64)
    return bound + ulp16(np.abs(want) + bound, dtype)


def window_attention_bound(qkv_bits, nh, hd, wlen, want_bits, orc, dtype, mode="split"):
    """attention_bound's error model for the audio tower's windowed attention:
    qkv [s, 3 nh hd] (q | k | v), every token of a window attends to every
    token of it."""
    x = orc.h16_to_f32(qkv_bits, dtype).astype(np.float64)
    s = x.shape[0]
    dm = nh * hd
    bound = np.zeros((s, dm))
    for st in range(0, s, wlen):
        en = min(s, st + wlen)
        vis = np.ones((en - st, en - st), bool)
        for h in range(nh):
            c = slice(h * hd, (h + 1) * hd)
            bound[st:en, c] = _attention_bound_rows(
                x[st:en, c], x[st:en, dm + h * hd:dm + (h + 1) * hd],
                x[st:en, 2 * dm + h * hd:2 * dm + (h + 1) * hd], vis, dtype, mode)
    want = orc.h16_to_f32(want_bits, dtype).astype(np.float64)
    return bound + ulp16(np.abs(want) + bound, dtype)


def assert_attention(got_bits, want_bits, q_bits, kc_bits, vc_bits, q0, orc, dtype, mode="split"):
    """Attention output against the oracle: finite, the north star's mean
    absolute error (and, in the default split mode, its max relative error),
    and the derived elementwise bound (attention_bound)."""
    s = parity_stats(got_bits, want_bits, orc, dtype)
    assert s["finite"], s
    assert s["mae"] <= MAE_TOL, s
    if mode == "split":
        assert s["max_rel"] <= REL_TOL, s
    bound = attention_bound(q_bits, kc_bits, vc_bits, q0, want_bits, orc, dtype, mode)
    return _assert_within(got_bits, want_bits, bound, orc, dtype, s)


def assert_window_attention(got_bits, want_bits, qkv_bits, nh, hd, wlen, orc, dtype):
    """Windowed attention against the oracle: finite, the north star (max
    relative error and MAE) and window_attention_bound elementwise."""
    s = parity_stats(got_bits, want_bits, orc, dtype)
    assert s["finite"], s
    assert s["mae"] <= MAE_TOL and s["max_rel"] <= REL_TOL, s
    bound = window_attention_bound(qkv_bits, nh, hd, wlen, want_bits, orc, dtype)
    return _assert_within(got_bits, want_bits, bound, orc, dtype, s)


def _assert_within(got_bits, want_bits, bound, orc, dtype, s):
    got = orc.h16_to_f32(got_bits, dtype).astype(np.float64)
    want = orc.h16_to_f32(want_bits, dtype).astype(np.float64)
    excess = np.abs(got - want) - bound
    worst = np.unravel_index(np.argmax(excess), excess.shape)
    assert excess.max() <= 0, (s, worst, got[worst], want[worst], bound[worst])
    s["bound_use"] = float((np.abs(got - want) / bound).max())
    return s


def round16(x, dtype):
    """f32 values rounded to the 16-bit format and widened back: numpy's IEEE
    cast for f16; (u + 0x7FFF + ((u >> 16) & 1)) >> 16 for bf16
    (src/shaders.rs:169-179)."""
    x = np.asarray(x, np.float32)
    if dtype == 0:
        return x.astype(np.float16).astype(np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    return (((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16).astype(np.uint32).view(np.float32)


def rope_tables(rows, hd, pos0, theta=1e6, dtype=0):
    """cos/sin [pos][hd] as src/mrope.rs:55-82 builds them for text positions:
    angle(pos, j) = pos * theta^(-2j/hd) in f64, the second half repeating the
    first, rounded to f32 and then to the run's 16-bit format, as the reference
    narrows both tables before the decoder reads them
    (src/align_inference.rs:371-372,394-395; src/cpu_decoder.rs:247)."""
    half = hd // 2
    inv = 1.0 / theta ** (2.0 * np.arange(half) / hd)
    pos = np.arange(pos0 + rows, dtype=np.float64)[:, None]
    ang = pos * inv[None, :]
    c = np.concatenate([np.cos(ang), np.cos(ang)], axis=1).astype(np.float32)
    s = np.concatenate([np.sin(ang), np.sin(ang)], axis=1).astype(np.float32)
    return round16(c, dtype), round16(s, dtype)
