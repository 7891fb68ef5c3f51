"""GPU parity of whole decoder layers (the host mirror of
WgpuTextDecoder::prefill's layer loop, csrc/host/decoder_prefill.cpp) against
the oracle chain of the CPU twin (src/cpu_decoder.rs:416-512: rms_norm ->
q|k|v -> head norm + RoPE -> attention -> o + residual -> rms_norm ->
SiLU(gate) * up -> down + residual, a 16-bit rounding after every op).

Config-3 layer shapes (hidden 1024, 16 q heads over 8 kv heads of 128, MLP
3072), random weights ~ N(0, 0.02), norm weights ~ 1 + N(0, 0.1), the residual
stream ~ N(0, 1).

Two gates:
  * per stage, one layer: every op the mirror launches is compared with the
    oracle op run on the GPU's own inputs of that op (read back from the
    device), to that op's bar: RMSNorm, the projections and the residual adds
    within 1 ulp (where the input is the oracle's recomputation of a residual
    the GPU also rounded: 2 ulps after the norm, one ulp of that residual plus
    one of the output after the add), head norm + RoPE within 1 ulp and the V
    copy bit-exact, attention by the north star plus the derived bound
    (conftest.attention_bound), SiLU.up by its propagated bound.
  * chained, two layers: the residual stream after two layers of each chain.
    A one-ulp difference anywhere moves every later op's inputs (attention
    mixes rows, the projections mix columns), so after two layers about half
    of the outputs differ in their last bit: the gate is statistical, the
    north star's mean absolute error <= 1e-3 and a relative RMS difference
    below one f16 ulp at 1.0 (2^-10); for bf16 both scale by its 8x larger
    ulp (2^-7).
"""
from __future__ import annotations

import numpy as np
import pytest

from chains import oracle_dec_layer as _oracle_layer
from conftest import assert_attention, assert_parity, rope_tables, ulp16

pytestmark = pytest.mark.gpu

HID, NQH, NKVH, HD, INTER, EPS = 1024, 16, 8, 128, 3072, 1e-6


def _weights(rng, orc, dtype, layers):
    def h16(shape, std):
        return orc.h16_from_f32((std * rng.standard_normal(shape)).astype(np.float32), dtype)
    out = []
    for _ in range(layers):
        out.append(dict(
            q=h16((NQH * HD, HID), 0.02), k=h16((NKVH * HD, HID), 0.02),
            v=h16((NKVH * HD, HID), 0.02), o=h16((HID, NQH * HD), 0.02),
            gate=h16((INTER, HID), 0.02), up=h16((INTER, HID), 0.02),
            down=h16((HID, INTER), 0.02),
            iln=(1.0 + 0.1 * rng.standard_normal(HID)).astype(np.float32),
            pln=(1.0 + 0.1 * rng.standard_normal(HID)).astype(np.float32),
            qn=(1.0 + 0.1 * rng.standard_normal(HD)).astype(np.float32),
            kn=(1.0 + 0.1 * rng.standard_normal(HD)).astype(np.float32)))
    return out


def _run_gpu(ctx, dtype, ws, h0, cos, sin, attn_flags, reads):
    from qwen3_aligner_wgpu_amd import host
    rows = h0.shape[0]
    dec = host.TextDecoder(ctx, dtype, len(ws), rows)
    try:
        for li, w in enumerate(ws):
            dec.load_layer(li, w["q"], w["k"], w["v"], w["o"], w["gate"], w["up"], w["down"],
                           w["iln"], w["pln"], w["qn"], w["kn"])
        dec.set_rope(cos, sin)
        dec.set_attention_flags(attn_flags)
        dec.set_hidden(h0)
        dec.prefill(rows)
        return {k: dec.read(k, rows) for k in reads}, dec.cap
    finally:
        dec.close()


@pytest.mark.parametrize("dtype,rows,attn_flags", [(0, 96, 0), (0, 200, 1), (1, 130, 0),
                                                   (0, 1024, 0)],
                         ids=["f16-96", "f16-200-p16", "bf16-130", "f16-1024"])
def test_decoder_layer_per_stage(ctx, pkg, orc, dtype, rows, attn_flags):
    rng = np.random.default_rng(rows + dtype)
    ws = _weights(rng, orc, dtype, 1)
    w = ws[0]
    h0 = orc.h16_from_f32(rng.standard_normal((rows, HID)).astype(np.float32), dtype)
    cos, sin = rope_tables(rows, HD, 0, dtype=dtype)
    g, cap = _run_gpu(ctx, dtype, ws, h0, cos, sin, attn_flags,
                      ("normed", "qkv", "q", "k_cache", "v_cache", "attn", "norm2", "act", "h"))
    # 1. input RMSNorm
    assert_parity(g["normed"], orc.rms_norm(dtype, h0, w["iln"], EPS), orc, dtype, ulp_tol=1)
    # 2. fused qkv projection on the GPU's normed rows
    qkv_w = np.ascontiguousarray(np.concatenate([w["q"], w["k"], w["v"]]))
    assert_parity(g["qkv"], orc.linear(dtype, g["normed"], qkv_w,
                                       np.zeros((rows, qkv_w.shape[0]), np.uint16)),
                  orc, dtype, ulp_tol=1)
    # 3. head norm + RoPE and the cache writes on the GPU's qkv
    kc = np.zeros((NKVH, cap, HD), np.uint16)
    vc = np.zeros((NKVH, HD, cap), np.uint16)
    q = orc.qk_norm_rope(dtype, g["qkv"], NQH, NKVH, HD, w["qn"], w["kn"], cos, sin, 0, EPS,
                         kc, vc, 0)
    assert_parity(g["q"], q, orc, dtype, ulp_tol=1)
    assert_parity(g["k_cache"][:, :rows], kc[:, :rows], orc, dtype, ulp_tol=1)
    assert np.array_equal(g["v_cache"], vc)
    # 4. attention on the GPU's q and caches
    mode = "p16" if attn_flags else "split"
    want = orc.attention(dtype, g["q"], g["k_cache"], g["v_cache"], 0)
    assert_attention(g["attn"], want, g["q"], g["k_cache"], g["v_cache"], 0, orc, dtype, mode=mode)
    # 5-6. o + residual (recomputed by the oracle on the GPU's attn), then RMSNorm
    hmid = orc.linear(dtype, g["attn"], w["o"], h0.copy(), flags=orc.ACCUMULATE)
    assert_parity(g["norm2"], orc.rms_norm(dtype, hmid, w["pln"], EPS), orc, dtype, ulp_tol=2)
    # 7. gate|up + SiLU.up on the GPU's norm2
    from conftest import assert_silu_mul
    gu_w = np.ascontiguousarray(np.concatenate([w["gate"], w["up"]]))
    want_act = orc.linear(dtype, g["norm2"], gu_w, np.zeros((rows, INTER), np.uint16),
                          flags=orc.EPI_SILU_MUL | orc.EXACT)
    gu_exact = orc.linear(dtype, g["norm2"], gu_w, np.zeros((rows, 2 * INTER), np.uint16),
                          flags=orc.EXACT)
    assert_silu_mul(g["act"], want_act, g["norm2"], gu_w, gu_exact, orc, dtype, HID,
                    rel_tol=1e-2 if dtype == 0 else 0.03)
    # 8. down + residual on the GPU's act, over the oracle's recomputed hmid: the
    # GPU's own hmid may differ from it by one ulp of hmid, which a cancelling
    # residual add carries over unchanged, so the bound is absolute: one ulp of
    # the residual input plus one of the output
    want_h = orc.linear(dtype, g["act"], w["down"], hmid.copy(), flags=orc.ACCUMULATE)
    f = lambda b: orc.h16_to_f32(b, dtype).astype(np.float64)  # noqa: E731
    err = np.abs(f(g["h"]) - f(want_h))
    assert (err <= ulp16(f(hmid), dtype) + ulp16(f(want_h), dtype)).all(), err.max()
    assert err.mean() <= 1e-3


@pytest.mark.parametrize("dtype,rows", [(0, 96), (1, 160)], ids=["f16-96", "bf16-160"])
def test_decoder_two_layers_chain(ctx, pkg, orc, dtype, rows):
    rng = np.random.default_rng(7 * rows + dtype)
    ws = _weights(rng, orc, dtype, 2)
    h0 = orc.h16_from_f32(rng.standard_normal((rows, HID)).astype(np.float32), dtype)
    cos, sin = rope_tables(rows, HD, 0, dtype=dtype)
    g, cap = _run_gpu(ctx, dtype, ws, h0, cos, sin, 0, ("h",))
    h = h0
    for w in ws:
        h = _oracle_layer(orc, dtype, h, w, cos, sin, cap)
    got = orc.h16_to_f32(g["h"], dtype).astype(np.float64)
    want = orc.h16_to_f32(h, dtype).astype(np.float64)
    assert np.isfinite(got).all()
    mae = np.abs(got - want).mean()
    rel_rms = np.sqrt(((got - want) ** 2).mean() / (want ** 2).mean())
    ulp = 2.0 ** -10 if dtype == 0 else 2.0 ** -7
    assert mae <= 1e-3 * (1 if dtype == 0 else 8), mae
    assert rel_rms <= ulp, rel_rms


def test_graph_timing_without_warmup(pkg, orc):
    """The host's step timer captures one step into a hipGraph after at least
    one eager step even with warmup = 0: the first call of a step sizes the
    context's workspace, which cannot grow under capture (a fresh context, so
    nothing is sized yet)."""
    from qwen3_aligner_wgpu_amd import host
    rng = np.random.default_rng(11)
    rows = 96
    ws = _weights(rng, orc, 0, 1)
    h0 = orc.h16_from_f32(rng.standard_normal((rows, HID)).astype(np.float32), 0)
    cos, sin = rope_tables(rows, HD, 0, dtype=0)
    with pkg.Context(0) as fresh:
        dec = host.TextDecoder(fresh, 0, 1, rows)
        try:
            w = ws[0]
            dec.load_layer(0, w["q"], w["k"], w["v"], w["o"], w["gate"], w["up"], w["down"],
                           w["iln"], w["pln"], w["qn"], w["kn"])
            dec.set_rope(cos, sin)
            dec.set_hidden(h0)
            ms, wall = dec.time(rows, 0, 2, use_graph=True)
        finally:
            dec.close()
    assert 0 < ms < 1e3 and 0 < wall < 1e3, (ms, wall)
