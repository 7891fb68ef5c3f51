"""Direct pins of the oracle's f32 audio-tower functions
(oracle/qa_oracle_audio.c: or_linear_f32, or_layer_norm_f32, or_gelu_f32_n,
or_window_attention_f32, or_conv3x3s2_f32, or_head_fold, and the head built
on it, oracle.timestamp_head_f32), the restatement of the reference's CPU
tower, which keeps every value in f32 (CpuAudioEncoder::forward,
src/audio_encoder.rs:754-832; CpuAudioLinear::forward :134-143; LayerNorm
:147-171; gelu :194-202; attention_window :493-616; conv_block :376-447) and
the host head (src/align_inference.rs:766-790).

Each function is checked against what the mathematics fixes, in f64, with an
error bound derived from its f32 evaluation, and each test also computes a
plausible mistake in f64 and shows that it falls OUTSIDE the same bound, so
the bound is tight enough to catch it:
  * linear: x W^T + b.  Mistakes: the output narrowed to 16 bits (the tower
    keeps f32), the bias narrowed to 16 bits, the bias dropped.
  * LayerNorm: (x - mean) / sqrt(var + eps) w + b.  Mistakes: eps outside the
    root, the unbiased variance (/(n-1)), no centring, no bias.
  * GELU: 0.5 x (1 + erf(x / sqrt 2)) against math.erf.  Mistakes: the tanh
    approximation, erf(x) without the 1/sqrt 2.
  * windowed attention: brute-force f64 softmax per window.  Mistakes: no
    1/sqrt(hd), a causal mask, one window over the whole sequence, a ragged
    last window padded to full length.
  * conv level: torch float64 conv2d (stride 2, padding 1) + bias + GELU.
    Mistakes: padding 0, kh and kw transposed.
  * head fold: x w / sqrt(mean((x w)^2) + eps) and its logits.  Mistakes: the
    weight outside the variance, eps dropped.
"""
from __future__ import annotations

import math

import numpy as np
import pytest

F16, BF16 = 0, 1
U = 2.0 ** -24  # f32 unit roundoff


def _within(got, want, bound):
    return bool((np.abs(np.asarray(got, np.float64) - want) <= bound).all())


def _h16(orc, x, dtype):
    return orc.h16_from_f32(np.asarray(x, np.float32), dtype)


# ---- linear ----------------------------------------------------------------

@pytest.mark.parametrize("dtype", [F16, BF16])
def test_linear_f32_closed_form(orc, dtype):
    rng = np.random.default_rng(100 + dtype)
    m, n, k = 37, 96, 448
    x = rng.standard_normal((m, k)).astype(np.float32)
    w = _h16(orc, 0.05 * rng.standard_normal((n, k)), dtype)
    # a bias large enough that its 16-bit rounding (a mistake) exceeds the
    # bound's f32 summation term
    b = (20.0 * rng.standard_normal(n)).astype(np.float32)
    got = orc.linear_f32(x, w, dtype, b)
    assert got.dtype == np.float32
    wf = orc.h16_to_f32(w, dtype).astype(np.float64)
    want = x.astype(np.float64) @ wf.T + b
    # f32 sum of k products (any blocked order, with or without FMA), then
    # one f32 add of the bias: gamma_{k+2} on the absolute sums
    bound = (k + 4) * U * (np.abs(x).astype(np.float64) @ np.abs(wf).T + np.abs(b))
    assert _within(got, want, bound)
    nob = orc.linear_f32(x, w, dtype)
    assert _within(nob, want - b, (k + 4) * U * (np.abs(x).astype(np.float64) @ np.abs(wf).T))
    # the mistakes this bound catches
    narrowed_out = orc.h16_to_f32(_h16(orc, want, dtype), dtype)
    assert not _within(narrowed_out, want, bound)
    narrowed_bias = want - b + orc.h16_to_f32(_h16(orc, b, dtype), dtype)
    assert not _within(narrowed_bias, want, bound)
    assert not _within(want - b, want, bound)


def test_linear_f32_rows_are_independent(orc):
    rng = np.random.default_rng(101)
    x = rng.standard_normal((9, 64)).astype(np.float32)
    w = _h16(orc, 0.1 * rng.standard_normal((32, 64)), F16)
    full = orc.linear_f32(x, w, F16)
    for r in (0, 4, 8):
        assert np.array_equal(orc.linear_f32(x[r:r + 1], w, F16)[0], full[r])


# ---- LayerNorm -------------------------------------------------------------

def _ln64(x, w, b, eps, ddof=0, centre=True):
    x = x.astype(np.float64)
    mean = x.mean(axis=1, keepdims=True) if centre else 0.0
    var = ((x - x.mean(axis=1, keepdims=True)) ** 2).sum(axis=1, keepdims=True) / (x.shape[1] - ddof)
    return (x - mean) / np.sqrt(var + eps) * w + b


def _ln_bound(x, w, b, eps):
    n = x.shape[1]
    x = x.astype(np.float64)
    mean = x.mean(axis=1, keepdims=True)
    d = x - mean
    var = (d ** 2).mean(axis=1, keepdims=True)
    inv = 1.0 / np.sqrt(var + eps)
    # mean: n U sum|x| / n; var: its own sum's (n + 2) U relative error plus the
    # mean error's effect 2 |d| dmean; the root and reciprocal a few ulps
    dmean = (n + 2) * U * np.abs(x).mean(axis=1, keepdims=True)
    dvar = (n + 4) * U * var + 2 * np.abs(d).mean(axis=1, keepdims=True) * dmean
    rel_inv = 0.5 * dvar / (var + eps) + 4 * U
    y = d * inv * w
    return np.abs(y) * (rel_inv + 4 * U) + dmean * inv * np.abs(w) + U * np.abs(y + b) + 1e-30


def test_layer_norm_f32_closed_form(orc):
    rng = np.random.default_rng(102)
    rows, n, eps = 12, 64, 0.25
    # a nonzero mean and a variance comparable with eps, so each term matters
    x = (3.0 + 0.6 * rng.standard_normal((rows, n))).astype(np.float32)
    w = (1.0 + 0.5 * rng.standard_normal(n)).astype(np.float32)
    b = (0.2 * rng.standard_normal(n)).astype(np.float32)
    got = orc.layer_norm_f32(x, w, b, eps)
    want = _ln64(x, w, b, eps)
    bound = _ln_bound(x, w, b, eps)
    assert _within(got, want, bound)
    xd = x.astype(np.float64)
    var = ((xd - xd.mean(axis=1, keepdims=True)) ** 2).mean(axis=1, keepdims=True)
    eps_outside = (xd - xd.mean(axis=1, keepdims=True)) / (np.sqrt(var) + eps) * w + b
    assert not _within(eps_outside, want, bound)
    assert not _within(_ln64(x, w, b, eps, ddof=1), want, bound)
    assert not _within(_ln64(x, w, b, eps, centre=False), want, bound)
    assert not _within(want - b, want, bound)


def test_layer_norm_f32_tower_width(orc):
    """At the tower's width (d_model 896, eps 1e-5) the unbiased-variance
    mistake still leaves the bound."""
    rng = np.random.default_rng(103)
    x = rng.standard_normal((6, 896)).astype(np.float32)
    w = np.ones(896, np.float32)
    b = np.zeros(896, np.float32)
    got = orc.layer_norm_f32(x, w, b, 1e-5)
    want = _ln64(x, w, b, 1e-5)
    bound = _ln_bound(x, w, b, 1e-5)
    assert _within(got, want, bound)
    assert not _within(_ln64(x, w, b, 1e-5, ddof=1), want, bound)


# ---- GELU ------------------------------------------------------------------

def test_gelu_f32_against_math_erf(orc):
    x = np.concatenate([np.linspace(-8, 8, 4001), [0.0, -0.0, 1e-30, -1e-30, 20.0, -20.0]])
    x = x.astype(np.float32)
    got = orc.gelu_f32(x)
    xd = x.astype(np.float64)
    want = np.array([0.5 * v * (1.0 + math.erf(v / math.sqrt(2.0))) for v in xd])
    # erff within a few ulps of erf (|erf| <= 1: absolute 4 U), the argument's
    # rounding (|x| / sqrt 2 * U, times erf' <= 1.13), then 3 f32 operations
    bound = 0.5 * np.abs(xd) * (4 * U + 1.2 * np.abs(xd) * U) + 4 * U * np.abs(want) + 1e-45
    assert _within(got, want, bound)
    assert got[np.argmin(np.abs(xd))] == 0.0
    tanh_form = 0.5 * xd * (1 + np.tanh(math.sqrt(2 / math.pi) * (xd + 0.044715 * xd ** 3)))
    assert not _within(tanh_form, want, bound)
    no_sqrt2 = np.array([0.5 * v * (1.0 + math.erf(v)) for v in xd])
    assert not _within(no_sqrt2, want, bound)


# ---- windowed attention ----------------------------------------------------

def _win_attn64(q, k, v, nh, hd, wlen, scale=True, causal=False, pad_last=False):
    s = q.shape[0]
    out = np.zeros((s, nh * hd))
    wabs = np.zeros((s, nh * hd))
    smax = np.zeros((s, nh))
    for st in range(0, s, wlen):
        en = min(s, st + wlen)
        for h in range(nh):
            cs = slice(h * hd, (h + 1) * hd)
            qq, kk, vv = (a[st:en, cs].astype(np.float64) for a in (q, k, v))
            if pad_last and en - st < wlen:  # a mistake: zero keys to a full window
                pad = wlen - (en - st)
                kk = np.vstack([kk, np.zeros((pad, hd))])
                vv = np.vstack([vv, np.zeros((pad, hd))])
            sc = qq @ kk.T * (1 / math.sqrt(hd) if scale else 1.0)
            if causal:
                sc = np.where(np.tril(np.ones_like(sc)) > 0, sc, -np.inf)
            p = np.exp(sc - sc.max(axis=1, keepdims=True))
            p /= p.sum(axis=1, keepdims=True)
            out[st:en, cs] = p @ vv
            wabs[st:en, cs] = p @ np.abs(vv)
            smax[st:en, h] = (np.abs(qq) @ np.abs(kk).T).max(axis=1) / math.sqrt(hd)
    return out, wabs, smax


def test_window_attention_f32_brute_force(orc):
    rng = np.random.default_rng(104)
    nh, hd, wlen, s = 2, 64, 24, 61  # 3 windows, the last one ragged (13 rows)
    q, k, v = (rng.standard_normal((s, nh * hd)).astype(np.float32) for _ in range(3))
    got = orc.window_attention_f32(q, k, v, nh, hd, wlen)
    want, wabs, smax = _win_attn64(q, k, v, nh, hd, wlen)
    # each score within (hd + 2) U of its absolute sum; a score error d moves
    # a normalised weight by at most a factor e^(2d); the exp, the sum over
    # <= wlen keys and the weighted sum of V add (wlen + 8) U relative
    d = np.repeat((hd + 4) * U * smax, hd, axis=1)
    bound = (np.expm1(2 * d) + (2 * wlen + 16) * U) * wabs + 1e-30
    assert _within(got, want, bound)
    for mistake in (dict(scale=False), dict(causal=True), dict(pad_last=True)):
        bad, _, _ = _win_attn64(q, k, v, nh, hd, wlen, **mistake)
        assert not _within(bad, want, bound), mistake
    one_window, _, _ = _win_attn64(q, k, v, nh, hd, s)
    assert not _within(one_window, want, bound)


# ---- conv level ------------------------------------------------------------

def _conv_torch(x, weight, bias, c_in, transpose_taps=False):
    import torch
    b, h, w, _ = x.shape
    c_out = weight.shape[0]
    wt = weight[:, :9 * c_in].reshape(c_out, 3, 3, c_in).astype(np.float64)
    wt = wt.transpose(0, 3, 2, 1) if transpose_taps else wt.transpose(0, 3, 1, 2)
    xt = torch.from_numpy(x.astype(np.float64)).permute(0, 3, 1, 2)
    y = torch.nn.functional.conv2d(xt, torch.from_numpy(np.ascontiguousarray(wt)),
                                   torch.from_numpy(bias.astype(np.float64)), stride=2, padding=1)
    z = 0.5 * y * (1 + torch.erf(y / math.sqrt(2.0)))
    # rows (b, ho, wo)
    return z.permute(0, 2, 3, 1).reshape(-1, c_out).numpy(), y.permute(0, 2, 3, 1).reshape(-1, c_out).numpy()


@pytest.mark.parametrize("tmajor", [False, True])
def test_conv3x3s2_f32_matches_torch_conv2d(orc, tmajor):
    rng = np.random.default_rng(105 + tmajor)
    b, h, w, c_in, c_out = 2, 9, 7, 8, 12
    x = rng.standard_normal((b, h, w, c_in)).astype(np.float32)
    ldw = 9 * c_in + 8  # a padded row stride
    weight = np.zeros((c_out, ldw), np.float32)
    weight[:, :9 * c_in] = (rng.standard_normal((c_out, 9 * c_in)) / math.sqrt(9 * c_in)).astype(np.float32)
    bias = (0.1 * rng.standard_normal(c_out)).astype(np.float32)
    got = orc.conv3x3s2_f32(x, weight, bias, gelu=True, token_major=tmajor)
    want, pre = _conv_torch(x, weight, bias, c_in)
    ho, wo = (h - 1) // 2 + 1, (w - 1) // 2 + 1
    if tmajor:  # the oracle's rows are (b, wo, ho): reorder the reference to match
        want = want.reshape(b, ho, wo, c_out).transpose(0, 2, 1, 3).reshape(-1, c_out)
        pre = pre.reshape(b, ho, wo, c_out).transpose(0, 2, 1, 3).reshape(-1, c_out)
    # an f64 sum rounded to f32 once, one f32 bias add, then GELU in f32: the
    # pre-activation within 2 ulps, GELU's slope <= 1.13, erff and 3 ops
    bound = 1.13 * 2 * U * (np.abs(pre) + 0.1) + 4 * U * np.abs(want) + 0.5 * np.abs(pre) * 5 * U + 1e-30
    assert _within(got, want, bound)
    swapped, _ = _conv_torch(x, weight, bias, c_in, transpose_taps=True)
    if tmajor:
        swapped = swapped.reshape(b, ho, wo, c_out).transpose(0, 2, 1, 3).reshape(-1, c_out)
    assert not _within(swapped, want, bound)
    nogelu = orc.conv3x3s2_f32(x, weight, bias, gelu=False, token_major=tmajor)
    assert _within(nogelu, pre, 2 * U * (np.abs(pre) + 0.1) + 1e-30)


def test_conv3x3s2_f32_padding_mistake_is_caught(orc):
    """Padding 1 against padding 0 on an even input, where both give the
    same output size (ho = h / 2)."""
    rng = np.random.default_rng(107)
    b, h, w, c_in, c_out = 1, 8, 6, 8, 4
    x = rng.standard_normal((b, h, w, c_in)).astype(np.float32)
    weight = (rng.standard_normal((c_out, 9 * c_in)) / 8).astype(np.float32)
    bias = np.zeros(c_out, np.float32)
    got = orc.conv3x3s2_f32(x, weight, bias, gelu=False)
    _, pre = _conv_torch(x, weight, bias, c_in)
    assert _within(got, pre, 2 * U * (np.abs(pre) + 0.1))
    import torch
    wt = weight.reshape(c_out, 3, 3, c_in).transpose(0, 3, 1, 2).astype(np.float64)
    xt = torch.from_numpy(np.pad(x.astype(np.float64), ((0, 0), (0, 1), (0, 1), (0, 0)))).permute(0, 3, 1, 2)
    pad0 = torch.nn.functional.conv2d(xt, torch.from_numpy(np.ascontiguousarray(wt)), stride=2)
    pad0 = pad0.permute(0, 2, 3, 1).reshape(-1, c_out).numpy()
    assert pad0.shape == pre.shape
    assert not _within(pad0, pre, 2 * U * (np.abs(pre) + 0.1))


# ---- head fold and logits --------------------------------------------------

@pytest.mark.parametrize("dtype", [F16, BF16])
def test_head_fold_closed_form(orc, dtype):
    rng = np.random.default_rng(108 + dtype)
    rows, n, labels, eps = 24, 1024, 200, 0.5
    h = _h16(orc, 2.0 * rng.standard_normal((rows + 5, n)), dtype)
    w = (1.0 + 0.5 * rng.standard_normal(n)).astype(np.float32)
    pos = rng.permutation(rows + 5)[:rows].astype(np.int32)
    got = orc.head_fold(dtype, h, pos, w, eps)
    x = orc.h16_to_f32(h, dtype).astype(np.float64)[pos]
    xw = x * w.astype(np.float64)
    inv = 1.0 / np.sqrt((xw ** 2).mean(axis=1, keepdims=True) + eps)
    want = xw * inv
    # the sum of n squares in f32 (n + 2) U relative, the root and reciprocal
    # a few ulps, the two products 2 ulps
    bound = np.abs(want) * ((n + 8) * U) + 1e-30
    assert _within(got, want, bound)
    unfolded = x / np.sqrt((x ** 2).mean(axis=1, keepdims=True) + eps) * w
    assert not _within(unfolded, want, bound)
    no_eps = xw / np.sqrt((xw ** 2).mean(axis=1, keepdims=True))
    assert not _within(no_eps, want, bound)
    # the logits: the folded rows times the score matrix with the f32 GEMM
    score = (0.05 * rng.standard_normal((labels, n))).astype(np.float32)
    logits, cls = orc.timestamp_head_f32(dtype, h, pos, w, eps, score)
    want_l = want @ score.astype(np.float64).T
    lb = (np.abs(want) * (n + 8) * U + np.abs(want) * (n + 4) * U) @ np.abs(score.astype(np.float64)).T
    assert _within(logits, want_l, lb + 1e-30)
    assert np.array_equal(cls, np.argmax(logits, axis=1))
    assert not _within(unfolded @ score.T, want_l, lb)
