"""GPU parity of the audio tower's non-GEMM ops: qa_layer_norm,
qa_window_attention and qa_add_position_table against the oracle
(oracle/qa_oracle_audio.c: the CPU twin's arithmetic, src/audio_encoder.rs:
147-171 LayerNorm, 517-616 windowed attention, 331-343 position add).

Every case calls the product through the C ABI (csrc/libqa.so) on an MI355X.

Tolerances:
  * LayerNorm: one 16-bit rounding of an f32 value whose summation order
    differs from the CPU's: within 1 ulp, at least 99% bit-identical.
  * position add: one f32 add and one rounding on both sides: bit-exact.
  * windowed attention: the north star (max relative error <= 1e-2 with the
    1e-3 max|r| floor, MAE <= 1e-3) and the derived elementwise bound
    (conftest.window_attention_bound: f32 score error, the two-term
    probabilities' residue rounding, f32 accumulation, final rounding).
The audio tower's shapes: d_model 896 = 14 heads x 64, windows of 104 tokens
(13 tokens per 100-frame chunk x 8 chunks, src/audio_encoder.rs:819-822),
3900 tokens for 300 s of audio.
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

from conftest import assert_parity, assert_window_attention

pytestmark = pytest.mark.gpu

F16, BF16 = 0, 1
DTYPES = pytest.mark.parametrize("dtype", [F16, BF16], ids=["f16", "bf16"])


def _h16(orc, x, dtype):
    return orc.h16_from_f32(np.asarray(x, np.float32), dtype)


@DTYPES
@pytest.mark.parametrize("rows,n,pad", [(1, 896, 0), (37, 896, 16), (3900, 896, 0), (5, 8, 8),
                                        (300, 1280, 64)])
def test_layer_norm(ctx, pkg, orc, dtype, rows, n, pad):
    rng = np.random.default_rng(rows + n)
    ld = n + pad
    x = _h16(orc, 2.0 * rng.standard_normal((rows, ld)) + 0.3, dtype)
    w = (1.0 + 0.2 * rng.standard_normal(n)).astype(np.float32)
    b = (0.1 * rng.standard_normal(n)).astype(np.float32)
    y0 = np.full((rows, ld), 0x3C01, np.uint16)
    dx, dw, db, dy = (ctx.to_device(a) for a in (x, w, b, y0))
    ctx.layer_norm(pkg.LayerNormDesc(dtype=dtype, flags=0, rows=rows, n=n, x=int(dx), ldx=ld,
                                     w=int(dw), b=int(db), y=int(dy), ldy=ld, eps=1e-5))
    y = ctx.download(dy, (rows, ld))
    want = orc.layer_norm(dtype, np.ascontiguousarray(x[:, :n]), w, b, 1e-5)
    s = assert_parity(y[:, :n], want, orc, dtype, ulp_tol=1)
    assert s["identical"] >= 0.99, s
    assert (y[:, n:] == 0x3C01).all()
    for buf in (dx, dw, db, dy):
        buf.free()


@DTYPES
@pytest.mark.parametrize("rows,n,period", [(3900, 896, 13), (20, 64, 13), (7, 896, 1)])
def test_add_position_table(ctx, pkg, orc, dtype, rows, n, period):
    rng = np.random.default_rng(rows)
    y = _h16(orc, rng.standard_normal((rows, n)), dtype)
    table = orc.sinusoid_table(period, n) if n % 2 == 0 else rng.standard_normal((period, n))
    table = np.ascontiguousarray(table, np.float32)
    dy, dt = ctx.to_device(y), ctx.to_device(table)
    ctx.add_position_table(pkg.PositionAddDesc(dtype=dtype, flags=0, rows=rows, n=n, y=int(dy),
                                               ldy=n, table=int(dt), period=period))
    got = ctx.download(dy, (rows, n))
    assert np.array_equal(got, orc.add_position_table(dtype, y, table))
    dy.free()
    dt.free()


def _win_gpu(ctx, pkg, dtype, qkv, nh, hd, wlen, ld_pad=8):
    s = qkv.shape[0]
    ldo = nh * hd + ld_pad
    dq = ctx.to_device(qkv)
    do = ctx.to_device(np.full((s, ldo), 0x7E00, np.uint16))
    ctx.window_attention(pkg.WindowAttentionDesc(dtype=dtype, flags=0, s=s, nh=nh, hd=hd,
                                                 wlen=wlen, qkv=int(dq), ldqkv=qkv.shape[1],
                                                 out=int(do), ldo=ldo))
    out = ctx.download(do, (s, ldo))
    dq.free()
    do.free()
    assert (out[:, nh * hd:] == 0x7E00).all()  # the stride padding is not written
    return np.ascontiguousarray(out[:, :nh * hd])


@DTYPES
@pytest.mark.parametrize("s,wlen,nh", [(30, 104, 14), (104, 104, 14), (250, 104, 14),
                                       (3900, 104, 14), (77, 13, 3), (300, 128, 2),
                                       (129, 128, 1)])
def test_window_attention(ctx, pkg, orc, dtype, s, wlen, nh):
    rng = np.random.default_rng(s + wlen + nh)
    hd = 64
    qkv = _h16(orc, 1.5 * rng.standard_normal((s, 3 * nh * hd + 16)), dtype)
    got = _win_gpu(ctx, pkg, dtype, qkv, nh, hd, wlen)
    want = orc.window_attention(dtype, qkv, nh, hd, wlen)
    assert_window_attention(got, want, np.ascontiguousarray(qkv[:, :3 * nh * hd]), nh, hd, wlen,
                            orc, dtype)


def test_window_of_one_token_copies_v(ctx, pkg, orc):
    """wlen = 1: every token attends only to itself, so the output is its V
    bit for bit (weight exactly 1, one product, one rounding of an exact value)."""
    rng = np.random.default_rng(2)
    s, nh, hd = 50, 4, 64
    qkv = _h16(orc, 3.0 * rng.standard_normal((s, 3 * nh * hd)), F16)
    got = _win_gpu(ctx, pkg, F16, qkv, nh, hd, 1)
    assert np.array_equal(got, qkv[:, 2 * nh * hd:])


def test_audio_ops_validate(ctx, pkg):
    lib = pkg.lib()
    h = ctx.handle
    ok = dict(dtype=F16, flags=0, s=104, nh=14, hd=64, wlen=104, qkv=0x100000, ldqkv=2688,
              out=0x200000, ldo=896)
    for kw, code, needle in [(dict(hd=32), pkg.QA_EUNSUPPORTED, "hd=32"),
                             (dict(wlen=129), pkg.QA_EUNSUPPORTED, "wlen=129"),
                             (dict(ldqkv=2680), pkg.QA_EINVAL, "ldqkv"),
                             (dict(out=0x200008), pkg.QA_EINVAL, "aligned"),
                             (dict(flags=1), pkg.QA_EINVAL, "flags")]:
        d = pkg.WindowAttentionDesc(**{**ok, **kw})
        assert lib.qa_window_attention(h, ctypes.byref(d)) == code, kw
        assert needle in pkg.last_error(), (kw, pkg.last_error())
    ln = dict(dtype=F16, flags=0, rows=4, n=896, x=0x100000, ldx=896, w=0x200000, b=0x200400,
              y=0x300000, ldy=896, eps=1e-5)
    for kw, needle in [(dict(n=890), "multiple of 8"), (dict(ldx=800), "strides"),
                       (dict(b=None), "null pointer"), (dict(eps=-1.0), "eps")]:
        d = pkg.LayerNormDesc(**{**ln, **kw})
        assert lib.qa_layer_norm(h, ctypes.byref(d)) == pkg.QA_EINVAL, kw
        assert needle in pkg.last_error(), (kw, pkg.last_error())
    pa = dict(dtype=F16, flags=0, rows=4, n=896, y=0x100000, ldy=896, table=0x200000, period=13)
    for kw, needle in [(dict(period=0), "period"), (dict(ldy=880), "ldy")]:
        d = pkg.PositionAddDesc(**{**pa, **kw})
        assert lib.qa_add_position_table(h, ctypes.byref(d)) == pkg.QA_EINVAL, kw
        assert needle in pkg.last_error(), (kw, pkg.last_error())
