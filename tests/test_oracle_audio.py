"""Pins the audio-tower op restatements in oracle/qa_oracle_audio.c before they
are trusted as the checker for qa_layer_norm / qa_window_attention /
qa_add_position_table / qa_conv2d_3x3s2.

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
  * the conv level (src/audio_encoder.rs:204-236,376-447): torch's float64
    conv2d (stride 2, padding 1, NCHW, the checkpoint's weight layout) plus
    GELU, and a restatement of the reference's own im2col times its weight
    matrix; both output row orders.
A dropped mean, a variance without the square, a missing 1/sqrt(hd), a window
boundary off by one, a table row off by one, a transposed tap, a wrong stride
or padding fails one of them.
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


def _conv_case(orc, dtype, b, h, w, c_in, c_out, seed):
    """Random NHWC input, checkpoint-layout weight [c_out][c_in][3][3] and its
    (kh, kw, ic) permutation padded to ldw = 9 c_in rounded up to 8."""
    rng = np.random.default_rng(seed)
    x = _h16(orc, rng.standard_normal((b, h, w, c_in)), dtype)
    wck = _h16(orc, 0.2 * rng.standard_normal((c_out, c_in, 3, 3)), dtype)
    ldw = (9 * c_in + 7) // 8 * 8
    wperm = np.zeros((c_out, ldw), np.uint16)
    wperm[:, :9 * c_in] = wck.transpose(0, 2, 3, 1).reshape(c_out, 9 * c_in)
    bias = _h16(orc, 0.1 * rng.standard_normal(c_out), dtype)
    return x, wck, wperm, bias


@pytest.mark.parametrize("dtype", [F16, BF16], ids=["f16", "bf16"])
@pytest.mark.parametrize("b,h,w,c_in,c_out", [(2, 9, 7, 1, 16), (1, 8, 10, 16, 24),
                                              (2, 5, 6, 64, 8)])
def test_conv_matches_torch_conv2d(orc, dtype, b, h, w, c_in, c_out):
    """The conv definition (stride 2, padding 1, the (kh, kw, ic) weight
    permutation, both output row orders, bias, erf GELU) against torch's float64
    conv2d on the same values in NCHW with the checkpoint's weight layout."""
    import torch
    x, wck, wperm, bias = _conv_case(orc, dtype, b, h, w, c_in, c_out, b * h + c_in)
    xt = torch.from_numpy(_f(orc, x, dtype)).permute(0, 3, 1, 2)
    wt = torch.from_numpy(_f(orc, wck, dtype))
    bt = torch.from_numpy(_f(orc, bias, dtype))
    ref = torch.nn.functional.gelu(torch.nn.functional.conv2d(xt, wt, bt, stride=2, padding=1))
    ho, wo = ref.shape[2], ref.shape[3]
    assert (ho, wo) == ((h - 1) // 2 + 1, (w - 1) // 2 + 1)
    for tmajor in (False, True):
        got = _f(orc, orc.conv3x3s2(dtype, x, wperm, bias, token_major=tmajor), dtype)
        r = ref.permute(0, 3, 2, 1) if tmajor else ref.permute(0, 2, 3, 1)  # rows (b,wo,ho)/(b,ho,wo)
        r = r.reshape(-1, c_out).numpy()
        assert (np.abs(got - r) <= ulp16(r, dtype) + 1e-6).all(), np.abs(got - r).max()


def test_conv_matches_the_reference_im2col(orc):
    """A restatement of the reference's own im2col (src/audio_encoder.rs:
    204-236: NCHW input, col[ic*9 + kh*3 + kw], ih = 2 ho + kh - 1) times the
    checkpoint weight [c_out][c_in*9], row order (b, ho, wo)."""
    b, h, w, c_in, c_out = 2, 7, 6, 3, 8
    x, wck, wperm, bias = _conv_case(orc, F16, b, h, w, c_in, c_out, 4)
    xn = _f(orc, x, F16).transpose(0, 3, 1, 2)  # NCHW
    ho, wo = (h - 1) // 2 + 1, (w - 1) // 2 + 1
    cols = np.zeros((b * ho * wo, c_in * 9))
    for i in range(b * ho * wo):
        ib, rem = divmod(i, ho * wo)
        oh, ow = divmod(rem, wo)
        for ic in range(c_in):
            for kh in range(3):
                for kw in range(3):
                    ih, iw = oh * 2 + kh - 1, ow * 2 + kw - 1
                    if 0 <= ih < h and 0 <= iw < w:
                        cols[i, ic * 9 + kh * 3 + kw] = xn[ib, ic, ih, iw]
    pre = cols @ _f(orc, wck, F16).reshape(c_out, c_in * 9).T + _f(orc, bias, F16)
    got = _f(orc, orc.conv3x3s2(F16, x, wperm, bias, gelu=False), F16)
    assert (np.abs(got - pre) <= ulp16(pre, F16) + 1e-6).all()
