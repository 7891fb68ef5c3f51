"""GPU parity of BASELINE config 4 at its size: the audio tower's linear stack
in bf16 at M = 3750 tokens (host.EncoderLinears, the mirror of
GpuAudioEncoder::layer's linears, src/audio_encoder_gpu.rs:1414-1419,
1579-1581, 1594-1605, and the conv-downsampler GEMM [3750, 1152] -> 896 with
bias and GELU, src/audio_encoder.rs:416-447), through the planner's own
tile choices at that size (none forced).

Each stage is checked on rows sampled across the whole M range (every 7th
row plus the ragged last tile's rows; a linear's rows are independent, so a
sample is exact) against the f64-exact oracle (or_linear with EXACT):
  * the conv GEMM + bias + GELU, the last layer's qkv + bias and fc1 + bias +
    GELU outputs, each one rounding of the exact value: within 1 ulp;
  * the residual stream after 2 layers (o + bias and fc2 + bias accumulated
    onto it, four roundings): the oracle chain run step by step on the same
    inputs.  Each step rounds h_i = r(h_{i-1} + y_i) once, so a difference
    of at most half an ulp of |h_i| (plus the f32 accumulation error, far
    smaller) enters per step and is carried into the next: elementwise
    |got - want| <= sum_i ulp(|h_i|) <= 4 ulp(max_i |h_i|).  Where the chain
    cancels (|h| small after adding y), that is many ulps of the result,
    which is why the single-op relative metric does not apply here; the
    north star's MAE does, and >= 99% of the outputs are bit-identical.
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import assert_parity, parity_stats, ulp16

pytestmark = pytest.mark.gpu

BF16 = 1
M, D, F, CK, LAYERS = 3750, 896, 3584, 1152, 2


def test_config4_encoder_linear_stack_bf16(ctx, pkg, orc):
    from qwen3_aligner_wgpu_amd import host
    dt = BF16
    g = lambda tid, shape, std: host.synth_normal(3, tid, shape, 0.0, std, dt)  # noqa: E731
    layers = []
    for li in range(LAYERS):
        b = 100 + 16 * li
        layers.append(dict(qkv=(g(b, (3 * D, D), 0.02), g(b + 1, (3 * D,), 0.01)),
                           o=(g(b + 2, (D, D), 0.02), g(b + 3, (D,), 0.01)),
                           fc1=(g(b + 4, (F, D), 0.02), g(b + 5, (F,), 0.01)),
                           fc2=(g(b + 6, (D, F), 0.02), g(b + 7, (D,), 0.01))))
    conv_w, conv_b = g(1, (D, CK), 0.02), g(2, (D,), 0.01)
    col = g(3, (M, CK), 1.0)
    normed, attn, norm2 = g(4, (M, D), 1.0), g(5, (M, D), 1.0), g(6, (M, D), 1.0)
    h0 = g(7, (M, D), 1.0)
    enc = host.EncoderLinears(ctx, dt, LAYERS, M, D, F, CK)
    try:
        for li, l in enumerate(layers):
            enc.load_layer(li, *l["qkv"], *l["o"], *l["fc1"], *l["fc2"])
        enc.load_conv(conv_w, conv_b)
        enc.set_inputs(M, col, normed, attn, norm2, h0)
        enc.forward_linears(M)
        got = {k: enc.read(k, M) for k in ("conv", "qkv", "act", "h")}
    finally:
        enc.close()
    rows = np.union1d(np.arange(0, M, 7), np.arange(M - 10, M))
    ex = orc.EXACT
    z = lambda n: np.zeros((rows.size, n), np.uint16)  # noqa: E731
    want_conv = orc.linear(dt, col[rows], conv_w, z(D), flags=orc.EPI_GELU | ex, bias=conv_b)
    assert_parity(got["conv"][rows], want_conv, orc, dt, ulp_tol=1)
    last = layers[-1]
    want_qkv = orc.linear(dt, normed[rows], last["qkv"][0], z(3 * D), flags=ex, bias=last["qkv"][1])
    assert_parity(got["qkv"][rows], want_qkv, orc, dt, ulp_tol=1)
    want_act = orc.linear(dt, norm2[rows], last["fc1"][0], z(F), flags=orc.EPI_GELU | ex,
                          bias=last["fc1"][1])
    assert_parity(got["act"][rows], want_act, orc, dt, ulp_tol=1)
    h = h0[rows].copy()
    f = lambda bits: orc.h16_to_f32(bits, dt).astype(np.float64)  # noqa: E731
    big = np.abs(f(h))
    for l in layers:
        h = orc.linear(dt, attn[rows], l["o"][0], h, flags=orc.ACCUMULATE | ex, bias=l["o"][1])
        big = np.maximum(big, np.abs(f(h)))
        act = orc.linear(dt, norm2[rows], l["fc1"][0], z(F), flags=orc.EPI_GELU | ex,
                         bias=l["fc1"][1])
        h = orc.linear(dt, act, l["fc2"][0], h, flags=orc.ACCUMULATE | ex, bias=l["fc2"][1])
        big = np.maximum(big, np.abs(f(h)))
    err = np.abs(f(got["h"][rows]) - f(h))
    bound = 2 * LAYERS * ulp16(big, dt)
    worst = np.unravel_index(np.argmax(err - bound), err.shape)
    assert (err <= bound).all(), (worst, err[worst], bound[worst])
    s = parity_stats(got["h"][rows], h, orc, dt)
    assert s["finite"] and s["mae"] <= 8e-3 and s["identical"] >= 0.99, s
