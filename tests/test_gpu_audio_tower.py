"""GPU parity of the whole audio tower (the host mirror of
GpuAudioEncoder::encode, csrc/host/audio_encoder.cpp) against the oracle ops
chained the way the tower chains them (src/audio_encoder.rs:754-832 for the
op order; a 16-bit rounding after every op, as the reference's GPU tower
stores every intermediate).

Qwen3-ASR tower shapes (128 mel bins in chunks of 100 frames, conv stem of
480 channels, d_model 896 = 14 x 64, FFN 3584, output 1024, windows of 104
tokens), random weights (conv weights ~ N(0, 1/fan_in), linears ~ N(0, 0.02),
LayerNorm ~ 1 + N(0, 0.1)), mel ~ N(0, 1); the last chunk is a tail of 37
frames, zero-padded, whose feo(37) = 5 tokens are kept.

Two gates:
  * per stage (no transformer layers): each conv level on the GPU's own input
    of that level, conv_out + position add on the GPU's conv3 output, and
    ln_post / proj1 + GELU / proj2 on the GPU's residual stream, each within
    1 ulp of the oracle (the conv_out + position add: one ulp of the GEMM's
    rounded output plus one of the sum);
  * chained (two layers): the tower output against the oracle chain; a
    one-ulp difference moves every later op's inputs, so the gate is
    statistical: the north star's mean absolute error and a relative RMS
    difference below one ulp at 1.0.
"""
from __future__ import annotations

import numpy as np
import pytest

from chains import oracle_tower as _oracle_tower, perm_co as _perm_co, perm_conv as _perm_conv
from conftest import assert_parity, ulp16

pytestmark = pytest.mark.gpu

F16, BF16 = 0, 1
NM, CS, CC, DM, NH, FFN, OD, WLEN = 128, 100, 480, 896, 14, 3584, 1024, 104


def _weights(orc, dtype, layers, seed):
    rng = np.random.default_rng(seed)
    h16 = lambda shape, std: orc.h16_from_f32((std * rng.standard_normal(shape)).astype(np.float32), dtype)  # noqa: E731
    f32 = lambda shape, mean, std: (mean + std * rng.standard_normal(shape)).astype(np.float32)  # noqa: E731
    w = dict(
        conv=[(h16((CC, 1, 3, 3), 1 / 3.0), h16(CC, 0.05)),
              (h16((CC, CC, 3, 3), 1 / np.sqrt(9 * CC)), h16(CC, 0.05)),
              (h16((CC, CC, 3, 3), 1 / np.sqrt(9 * CC)), h16(CC, 0.05))],
        co=(h16((DM, CC * 16), 1 / np.sqrt(CC * 16)), h16(DM, 0.02)),
        layers=[dict(ln1=(f32(DM, 1, 0.1), f32(DM, 0, 0.1)), qkv=(h16((3 * DM, DM), 0.02), h16(3 * DM, 0.02)),
                     o=(h16((DM, DM), 0.02), h16(DM, 0.02)), ln2=(f32(DM, 1, 0.1), f32(DM, 0, 0.1)),
                     fc1=(h16((FFN, DM), 0.02), h16(FFN, 0.02)), fc2=(h16((DM, FFN), 0.02), h16(DM, 0.02)))
                for _ in range(layers)],
        post=((f32(DM, 1, 0.1), f32(DM, 0, 0.1)), (h16((DM, DM), 0.02), h16(DM, 0.02)),
              (h16((OD, DM), 0.02), h16(OD, 0.02))),
    )
    return w


def _mel(orc, dtype, n_chunks, tail, seed):
    rng = np.random.default_rng(seed)
    mel = orc.h16_from_f32(rng.standard_normal((n_chunks, NM, CS)).astype(np.float32), dtype)
    if tail:
        mel[-1, :, tail:] = 0  # the zero-padded tail chunk
    return mel


def _build(ctx, dtype, w, n_chunks):
    from qwen3_aligner_wgpu_amd import host
    enc = host.AudioEncoder(ctx, dtype, len(w["layers"]), n_chunks)
    for lv, (cw, cb) in enumerate(w["conv"]):
        enc.load_conv(lv, cw, cb)
    enc.load_conv_out(*w["co"])
    for li, l in enumerate(w["layers"]):
        enc.load_layer(li, *l["ln1"], *l["qkv"], *l["o"], *l["ln2"], *l["fc1"], *l["fc2"])
    (lw, lb), (p1w, p1b), (p2w, p2b) = w["post"]
    enc.load_post(lw, lb, p1w, p1b, p2w, p2b)
    return enc


@pytest.mark.parametrize("dtype", [F16, BF16], ids=["f16", "bf16"])
def test_audio_tower_stages(ctx, pkg, orc, dtype):
    n_chunks, tail = 3, 37
    w = _weights(orc, dtype, 0, 1 + dtype)
    mel = _mel(orc, dtype, n_chunks, tail, 2)
    enc = _build(ctx, dtype, w, n_chunks)
    try:
        n = enc.tokens(n_chunks, tail)
        assert n == 2 * 13 + 5
        enc.set_mel(mel)
        enc.forward(n_chunks, tail)
        g = {k: enc.read(k, rows) for k, rows in (("conv1", n_chunks * 64 * 50),
                                                  ("conv2", n_chunks * 32 * 25),
                                                  ("conv3", n_chunks * 13), ("h", n),
                                                  ("normed", n), ("pact", n), ("out", n))}
    finally:
        enc.close()
    b = n_chunks
    want1 = orc.conv3x3s2(dtype, mel.reshape(b, NM, CS, 1), _perm_conv(w["conv"][0][0]), w["conv"][0][1])
    assert_parity(g["conv1"], want1, orc, dtype, ulp_tol=1)
    want2 = orc.conv3x3s2(dtype, g["conv1"].reshape(b, 64, 50, CC), _perm_conv(w["conv"][1][0]),
                          w["conv"][1][1])
    assert_parity(g["conv2"], want2, orc, dtype, ulp_tol=1)
    want3 = orc.conv3x3s2(dtype, g["conv2"].reshape(b, 32, 25, CC), _perm_conv(w["conv"][2][0]),
                          w["conv"][2][1], token_major=True).reshape(b * 13, CC * 16)
    assert_parity(g["conv3"], want3, orc, dtype, ulp_tol=1)
    # conv_out + position add on the GPU's conv3 rows (the n kept tokens)
    hco = orc.linear(dtype, np.ascontiguousarray(g["conv3"][:n]), _perm_co(w["co"][0]),
                     np.zeros((n, DM), np.uint16), bias=w["co"][1])
    want_h = orc.add_position_table(dtype, hco, orc.sinusoid_table(13, DM))
    f = lambda x: orc.h16_to_f32(x, dtype).astype(np.float64)  # noqa: E731
    assert (np.abs(f(g["h"]) - f(want_h)) <= ulp16(f(hco), dtype) + ulp16(f(want_h), dtype)).all()
    # the projector on the GPU's residual stream
    (lw, lb), (p1w, p1b), (p2w, p2b) = w["post"]
    assert_parity(g["normed"], orc.layer_norm(dtype, g["h"], lw, lb, 1e-5), orc, dtype, ulp_tol=1)
    assert_parity(g["pact"], orc.linear(dtype, g["normed"], p1w, np.zeros((n, DM), np.uint16),
                                        flags=orc.EPI_GELU, bias=p1b), orc, dtype, ulp_tol=1)
    assert_parity(g["out"], orc.linear(dtype, g["pact"], p2w, np.zeros((n, OD), np.uint16),
                                       bias=p2b), orc, dtype, ulp_tol=1)


@pytest.mark.parametrize("dtype,n_chunks,tail", [(F16, 20, 61), (BF16, 9, 0)],
                         ids=["f16-20c", "bf16-9c"])
def test_audio_tower_chain(ctx, pkg, orc, dtype, n_chunks, tail):
    w = _weights(orc, dtype, 2, 5 + dtype)
    mel = _mel(orc, dtype, n_chunks, tail, 6)
    enc = _build(ctx, dtype, w, n_chunks)
    try:
        n = enc.tokens(n_chunks, tail)
        enc.set_mel(mel)
        enc.forward(n_chunks, tail)
        got = enc.read("out", n)
    finally:
        enc.close()
    want, _ = _oracle_tower(orc, dtype, w, mel, n)
    g = orc.h16_to_f32(got, dtype).astype(np.float64)
    r = orc.h16_to_f32(want, dtype).astype(np.float64)
    assert np.isfinite(g).all()
    ulp = 2.0 ** -10 if dtype == F16 else 2.0 ** -7
    mae = np.abs(g - r).mean()
    rel_rms = np.sqrt(((g - r) ** 2).mean() / (r ** 2).mean())
    assert mae <= 1e-3 * (1 if dtype == F16 else 8), mae
    assert rel_rms <= ulp, rel_rms
