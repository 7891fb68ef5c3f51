"""GPU parity of qa_conv2d_3x3s2, one conv level of the audio tower's stem
(3x3, stride 2, pad 1, + bias, erf GELU; src/audio_encoder.rs:204-236,
376-447), against the oracle (oracle/qa_oracle_audio.c or_conv3x3s2: f64
accumulation, f32 GELU, one rounding; pinned to torch's conv2d).

Every case calls the product through the C ABI on an MI355X: c_in = 1 takes
the direct kernel (qa_conv.hip), c_in a multiple of 8 >= 64 the implicit GEMM
(qa_gemm.hip with the convolution loader, both tile shapes).

Tolerance: one rounding of an f32 sum (and the f32 GELU): the north star
(max relative error <= 1e-2 with the 1e-3 max|r| floor, MAE <= 1e-3) and
every output above the floor within 1 ulp of the f64-exact oracle.  The stem's
shapes per 100-frame mel chunk: conv1 [128 x 100 x 1] -> [64 x 50 x 480],
conv2 -> [32 x 25 x 480], conv3 -> [16 x 13 x 480] (rows (b, t, f) for
conv_out).  At 300 s (300 chunks) the oracle checks sampled row blocks.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np
import pytest

from conftest import assert_parity

pytestmark = pytest.mark.gpu

F16, BF16 = 0, 1


def _h16(orc, x, dtype):
    return orc.h16_from_f32(np.asarray(x, np.float32), dtype)


def _case(orc, dtype, b, h, w, c_in, c_out, seed, w_std=None):
    rng = np.random.default_rng(seed)
    x = _h16(orc, rng.standard_normal((b, h, w, c_in)), dtype)
    ldw = (9 * c_in + 7) // 8 * 8
    std = w_std if w_std is not None else 1.0 / np.sqrt(9 * c_in)
    wt = np.zeros((c_out, ldw), np.uint16)
    wt[:, :9 * c_in] = _h16(orc, std * rng.standard_normal((c_out, 9 * c_in)), dtype)
    bias = _h16(orc, 0.05 * rng.standard_normal(c_out), dtype)
    return x, wt, bias


def _conv_gpu(ctx, pkg, dtype, x, wt, bias, c_out, flags):
    b, h, w, c_in = x.shape
    ho, wo = (h - 1) // 2 + 1, (w - 1) // 2 + 1
    dx, dw = ctx.to_device(x), ctx.to_device(wt)
    db = ctx.to_device(bias) if bias is not None else None
    dy = ctx.alloc(b * ho * wo * c_out * 2)
    ctx.conv2d_3x3s2(pkg.ConvDesc(dtype=dtype, flags=flags, batch=b, h=h, w=w, c_in=c_in,
                                  c_out=c_out, x=int(dx), weight=int(dw),
                                  bias=int(db) if db is not None else None, y=int(dy)))
    y = ctx.download(dy, (b * ho * wo, c_out))
    for buf in (dx, dw, db, dy):
        if buf is not None:
            buf.free()
    return y


CASES = [
    # b, h, w, c_in, c_out
    (2, 128, 100, 1, 480),   # conv1 of two mel chunks
    (1, 9, 7, 1, 16),        # odd sizes, direct
    (1, 64, 50, 480, 480),   # conv2 of one chunk
    (2, 32, 25, 480, 480),   # conv3 of two chunks
    (1, 13, 11, 64, 40),     # odd sizes, ragged N, implicit
    (3, 6, 5, 128, 136),
]


@pytest.mark.parametrize("dtype", [F16, BF16], ids=["f16", "bf16"])
@pytest.mark.parametrize("b,h,w,c_in,c_out", CASES)
@pytest.mark.parametrize("tmajor", [False, True], ids=["rows_hw", "rows_wh"])
def test_conv(ctx, pkg, orc, dtype, b, h, w, c_in, c_out, tmajor):
    x, wt, bias = _case(orc, dtype, b, h, w, c_in, c_out, b * h * w + c_in)
    flags = pkg.QA_CONV_GELU | (pkg.QA_CONV_TOKEN_MAJOR if tmajor else 0)
    got = _conv_gpu(ctx, pkg, dtype, x, wt, bias, c_out, flags)
    want = orc.conv3x3s2(dtype, x, wt, bias, gelu=True, token_major=tmajor)
    assert_parity(got, want, orc, dtype, ulp_tol=1)


@pytest.mark.parametrize("tile", ["0", "1", "2", "6", "8"],
                         ids=["128x128", "256x128", "128x256", "256x256", "256x160"])
def test_conv_tiles_and_no_activation(ctx, pkg, orc, monkeypatch, tile):
    """Every implicit-GEMM tile shape, without bias and GELU (the plain sum)."""
    monkeypatch.setenv("QA_TILE", tile)
    x, wt, _ = _case(orc, F16, 2, 20, 18, 96, 200, 7)
    got = _conv_gpu(ctx, pkg, F16, x, wt, None, 200, 0)
    want = orc.conv3x3s2(F16, x, wt, None, gelu=False)
    assert_parity(got, want, orc, F16, ulp_tol=1)


def test_conv_stem_at_300_s(ctx, pkg, orc):
    """conv2 over the 300 chunks of 300 s of audio (240 000 output pixels,
    995 GFLOP): the oracle checks the first, a middle and the last block of 64
    output rows."""
    from qwen3_aligner_wgpu_amd import host
    b, h, w, c = 300, 64, 50, 480
    _, wt, bias = _case(orc, F16, 1, 1, 1, c, c, 3)
    x = host.synth_normal(3, 1, (b, h, w, c))  # 921.6 MB, generated in parallel C
    got = _conv_gpu(ctx, pkg, F16, x, wt, bias, c, pkg.QA_CONV_GELU)
    m = got.shape[0]
    for m0 in (0, m // 2 + 17, m - 64):
        want = orc.conv3x3s2(F16, x, wt, bias, gelu=True, rows=(m0, m0 + 64))
        assert_parity(got[m0:m0 + 64], want, orc, F16, ulp_tol=1)


def test_conv_validate(ctx, pkg):
    lib = pkg.lib()
    ok = dict(dtype=F16, flags=pkg.QA_CONV_GELU, batch=1, h=64, w=50, c_in=480, c_out=480,
              x=0x100000, weight=0x200000, bias=None, y=0x300000)
    for kw, code, needle in [(dict(c_in=40), pkg.QA_EUNSUPPORTED, "c_in=40"),
                             (dict(c_in=100), pkg.QA_EUNSUPPORTED, "c_in=100"),
                             (dict(c_out=20), pkg.QA_EINVAL, "multiple of 8"),
                             (dict(flags=8), pkg.QA_EINVAL, "unknown flags"),
                             (dict(x=0x100008), pkg.QA_EINVAL, "aligned"),
                             (dict(h=0), pkg.QA_EINVAL, "bad shape"),
                             (dict(c_in=1, c_out=2048), pkg.QA_EUNSUPPORTED, "c_out=2048"),
                             (dict(batch=1 << 20), pkg.QA_EINVAL, "2 GiB")]:
        d = pkg.ConvDesc(**{**ok, **kw})
        assert lib.qa_conv2d_3x3s2(ctx.handle, ctypes.byref(d)) == code, kw
        assert needle in pkg.last_error(), (kw, pkg.last_error())
