"""Pins the decoder-op restatements in oracle/qa_oracle_decoder.c before they
are trusted as the checker for qa_rms_norm / qa_qk_norm_rope /
qa_attention_prefill.

The reference ships no known-answer test for these ops (its golds are absent,
tools/gold/), so each function is checked against what the mathematics fixes:
  * f64 closed forms evaluated on the same 16-bit inputs: RMSNorm
    (src/cpu_decoder.rs:288-300), per-head norm + rotate-half RoPE
    (src/cpu_decoder.rs:302-322), softmax attention (src/cpu_decoder.rs:324-411);
  * special cases: RoPE at angle 0 is the plain head norm; a rotation keeps
    each (j, j + hd/2) pair's length; identical keys average V over the
    visible rows; a row ignores every later key (causality); q heads 2h, 2h+1
    read kv head h (GQA);
  * layout invariants: K lands at cache rows start.., V is copied verbatim,
    transposed, key t at column vperm(t) (bits 2 and 3 of t swapped).
A dropped norm weight, a sign flip in the rotation, a missing 1/sqrt(hd),
an off-by-one in the causal bound or a wrong kv-head mapping fails one of them.
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import rope_tables

F16, BF16 = 0, 1


def _h16(orc, x, dtype):
    return orc.h16_from_f32(np.asarray(x, np.float32), dtype)


def _f(orc, bits, dtype):
    return orc.h16_to_f32(bits, dtype).astype(np.float64)


def _ulps(orc, got, want_f64, dtype):
    """Distance of 16-bit results from the f64 value, in units of the 16-bit
    spacing at that value."""
    from conftest import ulp16
    return np.abs(_f(orc, got, dtype) - want_f64) / ulp16(want_f64, dtype)


@pytest.mark.parametrize("dtype", [F16, BF16], ids=["f16", "bf16"])
def test_rms_norm_closed_form(orc, dtype):
    rng = np.random.default_rng(1)
    rows, n, eps = 37, 1024, 1e-6
    x = _h16(orc, 3.0 * rng.standard_normal((rows, n)), dtype)
    w = (1.0 + 0.1 * rng.standard_normal(n)).astype(np.float32)
    y = orc.rms_norm(dtype, x, w, eps)
    xf = _f(orc, x, dtype)
    ref = xf / np.sqrt((xf * xf).mean(axis=1, keepdims=True) + eps) * w.astype(np.float64)
    assert _ulps(orc, y, ref, dtype).max() <= 1.0


def _norm_rope_f64(xf, nw, c, s, eps):
    """f64 closed form of one head row set: xf [..., hd]."""
    hd = xf.shape[-1]
    half = hd // 2
    inv = 1.0 / np.sqrt((xf * xf).mean(axis=-1, keepdims=True) + eps)
    x = xf * inv * nw
    partner = np.concatenate([-x[..., half:], x[..., :half]], axis=-1)
    return x * c + partner * s


def _qkv_case(orc, dtype, rows, nqh, nkvh, hd, seed):
    rng = np.random.default_rng(seed)
    qkv = _h16(orc, 2.0 * rng.standard_normal((rows, (nqh + 2 * nkvh) * hd)), dtype)
    qn = (1.0 + 0.2 * rng.standard_normal(hd)).astype(np.float32)
    kn = (1.0 + 0.2 * rng.standard_normal(hd)).astype(np.float32)
    return qkv, qn, kn


@pytest.mark.parametrize("dtype", [F16, BF16], ids=["f16", "bf16"])
def test_qk_norm_rope_closed_form_and_layouts(orc, dtype):
    rows, nqh, nkvh, hd, pos0, start, cap, eps = 23, 4, 2, 128, 40, 40, 96, 1e-6
    qkv, qn, kn = _qkv_case(orc, dtype, rows, nqh, nkvh, hd, 2)
    c, s = rope_tables(rows, hd, pos0, dtype=dtype)
    kc = np.full((nkvh, cap, hd), 0x1234, np.uint16)
    vc = np.full((nkvh, hd, cap), 0x4321, np.uint16)
    q = orc.qk_norm_rope(dtype, qkv, nqh, nkvh, hd, qn, kn, c, s, pos0, eps, kc, vc, start)
    cols = orc.vperm(cap)  # V-cache column of each key
    xf = _f(orc, qkv, dtype)
    cs, sn = c[pos0:pos0 + rows].astype(np.float64), s[pos0:pos0 + rows].astype(np.float64)
    for h in range(nqh):
        ref = _norm_rope_f64(xf[:, h * hd:(h + 1) * hd], qn.astype(np.float64), cs, sn, eps)
        assert _ulps(orc, q[h], ref, dtype).max() <= 1.0, h
    q_dim, kv_dim = nqh * hd, nkvh * hd
    for h in range(nkvh):
        ref = _norm_rope_f64(xf[:, q_dim + h * hd:q_dim + (h + 1) * hd], kn.astype(np.float64),
                             cs, sn, eps)
        assert _ulps(orc, kc[h, start:start + rows], ref, dtype).max() <= 1.0, h
        v = qkv[:, q_dim + kv_dim + h * hd:q_dim + kv_dim + (h + 1) * hd]
        assert np.array_equal(vc[h][:, cols[start:start + rows]], v.T)
    # untouched cache rows / columns stay as they were
    assert (kc[:, :start] == 0x1234).all() and (kc[:, start + rows:] == 0x1234).all()
    other = np.setdiff1d(np.arange(cap), cols[start:start + rows])
    assert (vc[:, :, other] == 0x4321).all()


def test_rope_at_angle_zero_is_the_head_norm_and_rotation_keeps_pair_length(orc):
    rows, nqh, nkvh, hd, eps = 9, 2, 1, 64, 1e-6
    qkv, qn, kn = _qkv_case(orc, F16, rows, nqh, nkvh, hd, 3)
    ones, zeros = np.ones((rows, hd), np.float32), np.zeros((rows, hd), np.float32)
    kc = np.zeros((nkvh, 16, hd), np.uint16)
    vc = np.zeros((nkvh, hd, 16), np.uint16)
    q0 = orc.qk_norm_rope(F16, qkv, nqh, nkvh, hd, qn, kn, ones, zeros, 0, eps, kc, vc, 0)
    xf = _f(orc, qkv, F16)
    for h in range(nqh):
        x = xf[:, h * hd:(h + 1) * hd]
        plain = x / np.sqrt((x * x).mean(axis=1, keepdims=True) + eps) * qn
        assert _ulps(orc, q0[h], plain, F16).max() <= 1.0
    c, s = rope_tables(rows, hd, 0, theta=10.0)
    q1 = orc.qk_norm_rope(F16, qkv, nqh, nkvh, hd, qn, kn, c, s, 0, eps, kc, vc, 0)
    half = hd // 2
    for h in range(nqh):
        a, b = _f(orc, q0[h], F16), _f(orc, q1[h], F16)
        la = a[:, :half] ** 2 + a[:, half:] ** 2
        lb = b[:, :half] ** 2 + b[:, half:] ** 2
        np.testing.assert_allclose(lb, la, rtol=4e-3, atol=1e-4)


def _attention_f64(orc, q, kc, vc, q0, dtype):
    """Brute-force f64 causal GQA attention on the same 16-bit inputs."""
    nqh, rows, hd = q.shape
    nkvh, cap, _ = kc.shape
    rep = nqh // nkvh
    qf, kf, vf = _f(orc, q, dtype), _f(orc, kc, dtype), _f(orc, vc, dtype)
    vf = vf[:, :, orc.vperm(cap)]  # [nkvh, hd, key]
    out = np.zeros((rows, nqh * hd))
    for h in range(nqh):
        kh = h // rep
        s = qf[h] @ kf[kh].T / np.sqrt(hd)          # [rows, cap]
        pos = q0 + np.arange(rows)[:, None]
        s = np.where(np.arange(cap)[None, :] <= pos, s, -np.inf)
        p = np.exp(s - s.max(axis=1, keepdims=True))
        p /= p.sum(axis=1, keepdims=True)
        out[:, h * hd:(h + 1) * hd] = p @ vf[kh].T  # vf[kh] is [hd, cap]
    return out


def _attn_case(orc, dtype, rows, nqh, nkvh, hd, cap, seed, qscale=0.6):
    rng = np.random.default_rng(seed)
    q = _h16(orc, qscale * rng.standard_normal((nqh, rows, hd)), dtype)
    kc = _h16(orc, rng.standard_normal((nkvh, cap, hd)), dtype)
    vc = _h16(orc, rng.standard_normal((nkvh, hd, cap)), dtype)
    return q, kc, vc


@pytest.mark.parametrize("dtype", [F16, BF16], ids=["f16", "bf16"])
@pytest.mark.parametrize("rows,q0,cap", [(1, 0, 16), (33, 0, 48), (20, 50, 80)])
def test_attention_matches_f64_softmax(orc, dtype, rows, q0, cap):
    nqh, nkvh, hd = 4, 2, 64
    q, kc, vc = _attn_case(orc, dtype, rows, nqh, nkvh, hd, cap, rows + q0)
    got = orc.attention(dtype, q, kc, vc, q0)
    ref = _attention_f64(orc, q, kc, vc, q0, dtype)
    # f32 scores / softmax / accumulation, one 16-bit rounding: within one
    # 16-bit ulp of the exact value (plus a hair for near-zero outputs).
    from conftest import ulp16
    err = np.abs(_f(orc, got, dtype) - ref)
    assert (err <= ulp16(ref, dtype) + 1e-6).all(), err.max()


def test_attention_is_causal_and_averages_identical_keys(orc):
    rows, nqh, nkvh, hd, cap = 16, 2, 1, 64, 16
    q, kc, vc = _attn_case(orc, F16, rows, nqh, nkvh, hd, cap, 7)
    base = orc.attention(F16, q, kc, vc, 0)
    # changing keys / values at position 10 leaves rows 0..9 alone
    kc2, vc2 = kc.copy(), vc.copy()
    kc2[:, 10] = _h16(orc, np.full(hd, 3.0), F16)
    vc2[:, :, orc.vperm(cap)[10]] = _h16(orc, np.full(hd, -5.0), F16)
    moved = orc.attention(F16, q, kc2, vc2, 0)
    assert np.array_equal(moved[:10], base[:10])
    assert not np.array_equal(moved[10:], base[10:])
    # identical keys: every visible row weighs 1/(r+1), output = mean of V[0..r]
    same = np.repeat(kc[:, :1], cap, axis=1)
    out = _f(orc, orc.attention(F16, q, same, vc, 0), F16)
    vf = _f(orc, vc, F16)[0][:, orc.vperm(cap)]      # [hd, key]
    for r in range(rows):
        mean = vf[:, :r + 1].mean(axis=1)
        from conftest import ulp16
        for h in range(nqh):
            assert (np.abs(out[r, h * hd:(h + 1) * hd] - mean) <= ulp16(mean, F16) + 1e-6).all()


def test_attention_gqa_head_sharing(orc):
    """q heads 2h and 2h+1 read kv head h: with equal queries they agree, and
    swapping the two kv heads swaps the output head pairs."""
    rows, nqh, nkvh, hd, cap = 8, 4, 2, 64, 16
    q, kc, vc = _attn_case(orc, F16, rows, nqh, nkvh, hd, cap, 9)
    q[1], q[3] = q[0], q[2]
    out = orc.attention(F16, q, kc, vc, 0)
    assert np.array_equal(out[:, 0:hd], out[:, hd:2 * hd])
    assert np.array_equal(out[:, 2 * hd:3 * hd], out[:, 3 * hd:4 * hd])
    qs = q[[2, 3, 0, 1]].copy()
    swapped = orc.attention(F16, qs, kc[::-1].copy(), vc[::-1].copy(), 0)
    assert np.array_equal(swapped[:, :2 * hd], out[:, 2 * hd:])
    assert np.array_equal(swapped[:, 2 * hd:], out[:, :2 * hd])
