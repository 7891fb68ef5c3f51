"""GPU parity of the object the headline benchmark times, and of the unfused
config-3 projections.

`host.DecoderLinears` (the C++ mirror TextDecoderLinears of the four
projection sites of WgpuTextDecoder::prefill, src/decoder.rs:1321-1327,
1602-1608, 1628-1650, 1652-1657) is set up exactly as bench.py's
bench_decoder sets it up: f16, M = 1024 tokens, the same seeded weights and
activations, every projection launched with the prefetch hint of the next
one (the last down of a layer pulls the next layer's qkv weights).

  * Layer by layer (each layer enqueued alone, then read back): the layer's
    qkv within 1 ulp of the f64-exact oracle; act = SiLU.up within the
    propagated-rounding bound of conftest.silu_mul_bound; the residual stream
    after the layer against the oracle run on the GPU's own inputs (the h
    the GPU held before the layer and the act it produced): two roundings,
    h_mid = r(h + attn.o^T) and h_out = r(h_mid + act.down^T), each within
    one ulp of the exact value given the same inputs, so
    |got - want| <= ulp(h_mid) + ulp(h_out) elementwise.
  * The whole pass enqueued back to back (hints crossing layers, no wait in
    between) gives the same bits as the layer-by-layer run; and the timed
    path, one captured hipGraph per step (qah_decoder_time: one eager step,
    the graph's upload launch, then `steps` replays), gives the same bits as
    that many eager passes.  The kernels sum in a fixed order, so any
    difference is a bug in the sequence, not rounding.

The unfused shapes are the reference CPU path's (q, k, v and gate, up as
separate GEMMs, src/cpu_decoder.rs:494-505): q 1024->2048, k and v
1024->1024, gate and up 1024->3072 at M = 1024, in both 16-bit formats, each
within 1 ulp of or_linear with EXACT.

Rows are sampled (every 4th row plus the last 8): a linear's rows are
independent, so the sample is exact for the rows it holds.
"""
from __future__ import annotations

import numpy as np
import pytest

import bench
from conftest import assert_parity, assert_silu_mul, ulp16

pytestmark = pytest.mark.gpu

M = 1024
LAYERS = 3
F16 = 0
ROWS = np.union1d(np.arange(0, M, 4), np.arange(M - 8, M))


def _setup(pkg, host, ctx, layers):
    D = bench.DEC
    dec = host.DecoderLinears(ctx, pkg.F16, layers, M, D["hidden"], D["q_dim"], D["kv_dim"],
                              D["inter"])
    ws = []
    for li in range(layers):
        w = bench.decoder_weights(host, li)
        dec.load_layer(li, w["q"], w["k"], w["v"], w["o"], w["gate"], w["up"], w["down"])
        ws.append(w)
    inputs = dict(normed=bench.rmsnormed(host, 0, 1, (M, D["hidden"]), 0),
                  attn=bench.rmsnormed(host, 0, 2, (M, D["q_dim"]), 0),
                  norm2=bench.rmsnormed(host, 0, 3, (M, D["hidden"]), 0),
                  h=host.synth_normal(0, 4, (M, D["hidden"])))
    dec.set_inputs(M, **inputs)
    return dec, ws, inputs


def test_decoder_linears_layer_by_layer_against_the_oracle(pkg, orc, ctx):
    from qwen3_aligner_wgpu_amd import host
    dec, ws, x = _setup(pkg, host, ctx, LAYERS)
    ex = orc.EXACT
    f = lambda bits: orc.h16_to_f32(bits, F16).astype(np.float64)  # noqa: E731
    normed, attn, norm2 = (np.ascontiguousarray(x[k][ROWS]) for k in ("normed", "attn", "norm2"))
    try:
        h_before = x["h"][ROWS].copy()
        per_layer = []
        for li, w in enumerate(ws):
            dec.layer(li, M)
            qkv, act, h = (dec.read(k, M)[ROWS] for k in ("qkv", "act", "h"))
            per_layer.append(h)
            wqkv = np.concatenate([w["q"], w["k"], w["v"]])
            want = orc.linear(F16, normed, wqkv, np.zeros_like(qkv), flags=ex)
            assert_parity(qkv, want, orc, F16, ulp_tol=1)
            wgu = np.concatenate([w["gate"], w["up"]])
            gu_exact = orc.linear(F16, norm2, wgu, np.zeros((ROWS.size, wgu.shape[0]), np.uint16),
                                  flags=ex)
            want_act = orc.linear(F16, norm2, wgu, np.zeros_like(act), flags=orc.EPI_SILU_MUL | ex)
            assert_silu_mul(act, want_act, norm2, wgu, gu_exact, orc, F16, norm2.shape[1])
            h_mid = orc.linear(F16, attn, w["o"], h_before.copy(), flags=orc.ACCUMULATE | ex)
            h_out = orc.linear(F16, np.ascontiguousarray(act), w["down"], h_mid.copy(),
                               flags=orc.ACCUMULATE | ex)
            err = np.abs(f(h) - f(h_out))
            bound = ulp16(f(h_mid), F16) + ulp16(f(h_out), F16)
            worst = np.unravel_index(np.argmax(err - bound), err.shape)
            assert (err <= bound).all(), (li, worst, err[worst], bound[worst])
            assert (h == h_out).mean() >= 0.99, (li, (h == h_out).mean())
            h_before = h
        # the whole pass back to back: same bits as layer by layer
        dec.set_inputs(M, h=x["h"])
        dec.prefill_linears(M)
        assert np.array_equal(dec.read("h", M)[ROWS], per_layer[-1])
    finally:
        dec.close()


def test_decoder_linears_graph_replay_matches_eager_passes(pkg, orc, ctx):
    """qah_decoder_time with a graph runs 1 eager step, the graph's upload
    launch and `steps` replays: h after it equals that many eager passes."""
    from qwen3_aligner_wgpu_amd import host
    dec, ws, x = _setup(pkg, host, ctx, LAYERS)
    try:
        steps = 2
        dec.time(M, 0, steps, use_graph=True)
        got = {k: dec.read(k, M) for k in ("h", "qkv", "act")}
        dec.set_inputs(M, h=x["h"])
        for _ in range(1 + 1 + steps):
            dec.prefill_linears(M)
        want = {k: dec.read(k, M) for k in ("h", "qkv", "act")}
    finally:
        dec.close()
    for k in got:
        assert np.array_equal(got[k], want[k]), k
    assert np.isfinite(orc.h16_to_f32(got["h"], F16)).all()


@pytest.mark.parametrize("dtype", [0, 1], ids=["f16", "bf16"])
def test_unfused_config3_projections(pkg, orc, ctx, dtype):
    """q, k, v, gate and up as the reference CPU path runs them (separate
    GEMMs, src/cpu_decoder.rs:494-505) at M = 1024, planner's own tiles."""
    from qwen3_aligner_wgpu_amd import host
    D = bench.DEC
    h = D["hidden"]
    x = bench.rmsnormed(host, 0, 1, (M, h), dtype)
    w = bench.decoder_weights(host, 0, dtype)
    dx = ctx.to_device(x)
    xs = np.ascontiguousarray(x[ROWS])
    try:
        for name in ("q", "k", "v", "gate", "up"):
            n = w[name].shape[0]
            dw, dc = ctx.to_device(w[name]), ctx.alloc(M * n * 2)
            ctx.linear(pkg.linear_desc(dtype, M, n, h, dx, dw, dc))
            got = ctx.download(dc, (M, n))[ROWS]
            dw.free()
            dc.free()
            want = orc.linear(dtype, xs, w[name], np.zeros((ROWS.size, n), np.uint16),
                              flags=orc.EXACT)
            s = assert_parity(got, want, orc, dtype, ulp_tol=1,
                              mae_tol=1e-3 if dtype == 0 else 8e-3)
            assert s["identical"] >= 0.97, (name, s)
    finally:
        dx.free()
