"""Pins the audio-tower op restatements in oracle/qa_oracle_audio.c before they
are trusted as the checker for qa_layer_norm / qa_window_attention /
qa_add_position_table.

The reference ships no known-answer vectors for these ops, so each is checked
against what the mathematics fixes:
  * LayerNorm (src/audio_encoder.rs:147-171): the f64 closed form on the same
    16-bit inputs (<= 1 ulp); a constant row maps to the bias; with unit
    weight and zero bias every row has mean ~0 and variance ~1.
  * windowed attention (src/audio_encoder.rs:517-616): brute-force f64
    softmax per window (<= 1 ulp); a window ignores every other window;
    identical keys average V over the window; the last window holds the
    remainder; a sequence shorter than one window is one window.
  * the position add (src/audio_encoder.rs:331-343): f64 add then one
    rounding; row r takes table row r % period.
  * the sinusoid table (src/audio_encoder.rs:270-283): its definition in f64,
    position 0 = [0 ... 0 | 1 ... 1].
A dropped mean, a variance without the square, a missing 1/sqrt(hd), a window
boundary off by one or a table row off by one fails one of them.
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import ulp16

F16, BF16 = 0, 1


def _h16(orc, x, dtype):
    return orc.h16_from_f32(np.asarray(x, np.float32), dtype)


def _f(orc, bits, dtype):
    return orc.h16_to_f32(bits, dtype).astype(np.float64)


@pytest.mark.parametrize("dtype", [F16, BF16], ids=["f16", "bf16"])
def test_layer_norm_closed_form(orc, dtype):
    rng = np.random.default_rng(3)
    rows, n, eps = 29, 896, 1e-5
    x = _h16(orc, 2.0 * rng.standard_normal((rows, n)) + 0.5, dtype)
    w = (1.0 + 0.2 * rng.standard_normal(n)).astype(np.float32)
    b = (0.1 * rng.standard_normal(n)).astype(np.float32)
    y = orc.layer_norm(dtype, x, w, b, eps)
    xf = _f(orc, x, dtype)
    mu = xf.mean(axis=1, keepdims=True)
    var = ((xf - mu) ** 2).mean(axis=1, keepdims=True)
    ref = (xf - mu) / np.sqrt(var + eps) * w + b
    err = np.abs(_f(orc, y, dtype) - ref)
    assert (err <= ulp16(ref, dtype) + 1e-6).all(), err.max()


def test_layer_norm_constant_row_and_standardisation(orc):
    n = 256
    x = np.stack([np.full(n, 3.25, np.float32), np.linspace(-2, 5, n, dtype=np.float32)])
    xb = _h16(orc, x, F16)
    b = np.linspace(-1, 1, n).astype(np.float32)
    y = _f(orc, orc.layer_norm(F16, xb, np.ones(n, np.float32), b, 1e-5), F16)
    assert np.allclose(y[0], _f(orc, _h16(orc, b, F16), F16))  # constant row -> bias
    z = _f(orc, orc.layer_norm(F16, xb, np.ones(n, np.float32), np.zeros(n, np.float32), 1e-5),
           F16)[1]
    assert abs(z.mean()) < 2e-3 and abs(z.var() - 1.0) < 5e-3


def _window_attention_f64(orc, qkv, nh, hd, wlen, dtype):
    xf = _f(orc, qkv, dtype)
    s = xf.shape[0]
    dm = nh * hd
    out = np.zeros((s, dm))
    for st in range(0, s, wlen):
        en = min(s, st + wlen)
        for h in range(nh):
            q = xf[st:en, h * hd:(h + 1) * hd]
            k = xf[st:en, dm + h * hd:dm + (h + 1) * hd]
            v = xf[st:en, 2 * dm + h * hd:2 * dm + (h + 1) * hd]
            sc = q @ k.T / np.sqrt(hd)
            p = np.exp(sc - sc.max(axis=1, keepdims=True))
            out[st:en, h * hd:(h + 1) * hd] = (p / p.sum(axis=1, keepdims=True)) @ v
    return out


@pytest.mark.parametrize("dtype", [F16, BF16], ids=["f16", "bf16"])
@pytest.mark.parametrize("s,wlen", [(30, 104), (104, 104), (250, 104), (77, 13)])
def test_window_attention_matches_f64(orc, dtype, s, wlen):
    rng = np.random.default_rng(s + wlen)
    nh, hd = 3, 64
    qkv = _h16(orc, rng.standard_normal((s, 3 * nh * hd)), dtype)
    got = orc.window_attention(dtype, qkv, nh, hd, wlen)
    ref = _window_attention_f64(orc, qkv, nh, hd, wlen, dtype)
    err = np.abs(_f(orc, got, dtype) - ref)
    assert (err <= ulp16(ref, dtype) + 1e-6).all(), err.max()


def test_window_attention_windows_are_independent_and_average_identical_keys(orc):
    rng = np.random.default_rng(5)
    s, nh, hd, wlen = 40, 2, 64, 16
    dm = nh * hd
    qkv = _h16(orc, rng.standard_normal((s, 3 * dm)), F16)
    base = orc.window_attention(F16, qkv, nh, hd, wlen)
    moved = qkv.copy()
    moved[20] = _h16(orc, rng.standard_normal(3 * dm) * 3, F16)  # a token of window 1
    out = orc.window_attention(F16, moved, nh, hd, wlen)
    assert np.array_equal(out[:16], base[:16]) and np.array_equal(out[32:], base[32:])
    assert not np.array_equal(out[16:32], base[16:32])
    same = qkv.copy()
    same[:, dm:2 * dm] = same[0, dm:2 * dm]  # every key identical
    o = _f(orc, orc.window_attention(F16, same, nh, hd, wlen), F16)
    v = _f(orc, same, F16)[:, 2 * dm:]
    for st in range(0, s, wlen):
        mean = v[st:min(s, st + wlen)].mean(axis=0)
        assert (np.abs(o[st:min(s, st + wlen)] - mean) <= ulp16(mean, F16) + 1e-6).all()


@pytest.mark.parametrize("dtype", [F16, BF16], ids=["f16", "bf16"])
def test_add_position_table(orc, dtype):
    rng = np.random.default_rng(8)
    rows, n, period = 40, 96, 13
    y = _h16(orc, rng.standard_normal((rows, n)), dtype)
    table = rng.standard_normal((period, n)).astype(np.float32)
    got = orc.add_position_table(dtype, y, table)
    ref = _f(orc, y, dtype) + table[np.arange(rows) % period].astype(np.float64)
    want = orc.h16_from_f32(ref.astype(np.float32), dtype)
    # f32 sum then one rounding: identical to rounding the f64 sum except at
    # double-rounding ties, which these random values never hit
    assert np.array_equal(got, want)


def test_sinusoid_table_definition(orc):
    pos, dm = 13, 896
    t = orc.sinusoid_table(pos, dm).astype(np.float64)
    half = dm // 2
    assert np.array_equal(t[0, :half], np.zeros(half)) and np.array_equal(t[0, half:], np.ones(half))
    inv = np.exp(-np.arange(half) * np.log(10000.0) / (half - 1))
    ang = np.arange(pos)[:, None] * inv[None, :]
    assert np.abs(t[:, :half] - np.sin(ang)).max() < 1e-7
    assert np.abs(t[:, half:] - np.cos(ang)).max() < 1e-7
