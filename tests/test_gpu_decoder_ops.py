"""GPU parity of the decoder prefill ops around the projections:
qa_rms_norm, qa_qk_norm_rope and qa_attention_prefill against the oracle
(oracle/qa_oracle_decoder.c: the CPU twin's arithmetic, src/cpu_decoder.rs:
288-322 for the norms and RoPE, :324-411 for the attention).

Every case calls the product through the C ABI (csrc/libqa.so) on an MI355X.

Tolerances:
  * RMSNorm and q/k norm + RoPE: one 16-bit rounding of an f32 value whose
    summation order differs from the CPU's: within 1 ulp of the oracle, with
    at least 99% of the outputs bit-identical.  The V-cache copy is verbatim:
    bit-exact, and every cache entry the call must not write is untouched.
  * attention, default mode: the north star (max relative error <= 1e-2 with
    the 1e-3 max|r| floor, mean absolute error <= 1e-3) and the derived
    elementwise bound of conftest.attention_bound (f32 score error, the
    two-term probabilities' residue rounding, f32 accumulation, final
    rounding).  QA_ATTN_P16 mode (probabilities rounded once, as the
    reference's GPU path rounds them) is gated by the same bound with the
    single rounding's 2^-11 / 2^-8 relative term and the north star's mean
    absolute error; its max relative error exceeds 1e-2 on outputs near the
    floor by construction (tests/test_parity_checks.py shows this on the CPU).
At BASELINE's full prefill length (s ~ 4.3 k keys) the oracle checks sampled
row blocks: attention rows are independent, so the oracle run over rows
i..i+n with q0 = i is exactly rows i..i+n of the full result.
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

from conftest import assert_attention, assert_parity, rope_tables

pytestmark = pytest.mark.gpu

F16, BF16 = 0, 1
DTYPES = pytest.mark.parametrize("dtype", [F16, BF16], ids=["f16", "bf16"])


def _h16(orc, x, dtype):
    return orc.h16_from_f32(np.asarray(x, np.float32), dtype)


def _assert_1ulp(got, want, orc, dtype):
    s = assert_parity(got, want, orc, dtype, ulp_tol=1)
    assert s["identical"] >= 0.99, s
    return s


# ---------------------------------------------------------------- RMSNorm

@DTYPES
@pytest.mark.parametrize("rows,n,pad", [(1, 1024, 0), (37, 1024, 16), (1024, 1024, 0),
                                        (5, 8, 8), (3, 2056, 0), (300, 2048, 64)])
def test_rms_norm(ctx, pkg, orc, dtype, rows, n, pad):
    rng = np.random.default_rng(rows + n)
    ld = n + pad
    x = _h16(orc, 3.0 * rng.standard_normal((rows, ld)), dtype)
    w = (1.0 + 0.1 * rng.standard_normal(n)).astype(np.float32)
    y0 = np.full((rows, ld), 0x3C01, np.uint16)
    dx, dw, dy = ctx.to_device(x), ctx.to_device(w), ctx.to_device(y0)
    ctx.rms_norm(pkg.RmsNormDesc(dtype=dtype, flags=0, rows=rows, n=n, x=int(dx), ldx=ld,
                                 w=int(dw), y=int(dy), ldy=ld, eps=1e-6))
    y = ctx.download(dy, (rows, ld))
    want = orc.rms_norm(dtype, np.ascontiguousarray(x[:, :n]), w, 1e-6)
    _assert_1ulp(y[:, :n], want, orc, dtype)
    assert (y[:, n:] == 0x3C01).all()  # the stride padding is not written
    for b in (dx, dw, dy):
        b.free()


# ------------------------------------------------- q/k norm + RoPE + KV write

def _rope_case(ctx, pkg, orc, dtype, rows, nqh, nkvh, hd, pos0, start, cap, seed, ld_pad=8):
    rng = np.random.default_rng(seed)
    width = (nqh + 2 * nkvh) * hd
    ld = width + ld_pad
    qkv = _h16(orc, 2.0 * rng.standard_normal((rows, ld)), dtype)
    qn = (1.0 + 0.2 * rng.standard_normal(hd)).astype(np.float32)
    kn = (1.0 + 0.2 * rng.standard_normal(hd)).astype(np.float32)
    c, s = rope_tables(rows, hd, pos0, dtype=dtype)
    kc0 = np.full((nkvh, cap, hd), 0x1234, np.uint16)
    vc0 = np.full((nkvh, hd, cap), 0x4321, np.uint16)
    bufs = [ctx.to_device(a) for a in (qkv, qn, kn, c, s, kc0, vc0)]
    dq = ctx.alloc(nqh * rows * hd * 2)
    bufs.append(dq)
    d_qkv, d_qn, d_kn, d_c, d_s, d_kc, d_vc = bufs[:7]
    ctx.qk_norm_rope(pkg.QkRopeDesc(
        dtype=dtype, flags=0, rows=rows, nqh=nqh, nkvh=nkvh, hd=hd, eps=1e-6, qkv=int(d_qkv),
        ldqkv=ld, qn_w=int(d_qn), kn_w=int(d_kn), cos=int(d_c), sin=int(d_s), pos0=pos0,
        q_out=int(dq), k_cache=int(d_kc), v_cache=int(d_vc), cap=cap, start=start))
    got = (ctx.download(dq, (nqh, rows, hd)), ctx.download(d_kc, kc0.shape),
           ctx.download(d_vc, vc0.shape))
    kc, vc = kc0.copy(), vc0.copy()
    q = orc.qk_norm_rope(dtype, np.ascontiguousarray(qkv[:, :width]), nqh, nkvh, hd, qn, kn, c, s,
                         pos0, 1e-6, kc, vc, start)
    for b in bufs:
        b.free()
    return got, (q, kc, vc)


@DTYPES
@pytest.mark.parametrize("rows,nqh,nkvh,hd,pos0,start,cap", [
    (1, 16, 8, 128, 0, 0, 16),
    (33, 16, 8, 128, 5, 7, 64),
    (300, 16, 8, 128, 100, 100, 512),
    (70, 4, 2, 64, 3, 10, 96),
    (9, 2, 1, 256, 0, 0, 16),
])
def test_qk_norm_rope(ctx, pkg, orc, dtype, rows, nqh, nkvh, hd, pos0, start, cap):
    (q, kc, vc), (wq, wkc, wvc) = _rope_case(ctx, pkg, orc, dtype, rows, nqh, nkvh, hd, pos0,
                                             start, cap, rows + hd)
    _assert_1ulp(q, wq, orc, dtype)
    _assert_1ulp(kc[:, start:start + rows], wkc[:, start:start + rows], orc, dtype)
    assert (kc[:, :start] == 0x1234).all() and (kc[:, start + rows:] == 0x1234).all()
    assert np.array_equal(vc, wvc)  # verbatim, permuted, untouched elsewhere


@DTYPES
def test_qk_norm_rope_unaligned_rows(ctx, pkg, orc, dtype):
    """A row stride that is not a multiple of 8 elements takes the
    element-wise kernel (the 16-byte one needs aligned rows); same bar."""
    rows, nqh, nkvh, hd, start, cap = 45, 16, 8, 128, 3, 64
    (q, kc, vc), (wq, wkc, wvc) = _rope_case(ctx, pkg, orc, dtype, rows, nqh, nkvh, hd, 2, start,
                                             cap, 77, ld_pad=3)
    _assert_1ulp(q, wq, orc, dtype)
    _assert_1ulp(kc[:, start:start + rows], wkc[:, start:start + rows], orc, dtype)
    assert np.array_equal(vc, wvc)


# ------------------------------------------------------------- attention

def _attn_inputs(orc, dtype, rows, q0, cap, nqh, nkvh, seed, qscale=1.0):
    """q/k ~ N(0, 1) (score std ~ qscale), V ~ N(0, 1); cache entries past the
    visible keys hold large finite values, which the causal mask must ignore."""
    rng = np.random.default_rng(seed)
    hd = 128
    q = _h16(orc, qscale * rng.standard_normal((nqh, rows, hd)), dtype)
    kc = _h16(orc, rng.standard_normal((nkvh, cap, hd)), dtype)
    vc = _h16(orc, rng.standard_normal((nkvh, hd, cap)), dtype)
    kend = q0 + rows
    kc[:, kend:] = _h16(orc, 50.0 * rng.standard_normal((nkvh, cap - kend, hd)), dtype)
    cols = orc.vperm(cap)[kend:]
    vc[:, :, cols] = _h16(orc, 300.0 * rng.standard_normal((nkvh, hd, cap - kend)), dtype)
    return q, kc, vc


def _attn_gpu(ctx, pkg, dtype, q, kc, vc, q0, flags=0, ld_pad=0):
    nqh, rows, hd = q.shape
    nkvh, cap, _ = kc.shape
    ldo = nqh * hd + ld_pad
    dq, dk, dv = ctx.to_device(q), ctx.to_device(kc), ctx.to_device(vc)
    do = ctx.to_device(np.full((rows, ldo), 0x7E00, np.uint16))
    ctx.attention_prefill(pkg.AttentionDesc(dtype=dtype, flags=flags, rows=rows, nqh=nqh,
                                            nkvh=nkvh, hd=hd, q=int(dq), k_cache=int(dk),
                                            v_cache=int(dv), cap=cap, q0=q0, out=int(do),
                                            ldo=ldo))
    out = ctx.download(do, (rows, ldo))
    for b in (dq, dk, dv, do):
        b.free()
    if ld_pad:
        assert (out[:, nqh * hd:] == 0x7E00).all()  # the stride padding is not written
    return np.ascontiguousarray(out[:, :nqh * hd])


ATTN_CASES = [
    # rows, q0, cap, nqh, nkvh
    (1, 0, 16, 16, 8),
    (33, 0, 64, 16, 8),
    (64, 0, 64, 16, 8),
    (100, 0, 128, 16, 8),
    (20, 50, 80, 16, 8),      # cache offset; key block 64..127 straddles cap
    (130, 3, 144, 8, 8),      # MHA (one q head per kv head)
    (1, 700, 704, 16, 8),     # a single row deep in the cache
    (257, 0, 272, 16, 8),
]


@DTYPES
@pytest.mark.parametrize("mode", ["split", "p16"])
@pytest.mark.parametrize("rows,q0,cap,nqh,nkvh", ATTN_CASES)
def test_attention(ctx, pkg, orc, dtype, mode, rows, q0, cap, nqh, nkvh):
    q, kc, vc = _attn_inputs(orc, dtype, rows, q0, cap, nqh, nkvh, rows * 7 + q0)
    flags = pkg.QA_ATTN_P16 if mode == "p16" else 0
    got = _attn_gpu(ctx, pkg, dtype, q, kc, vc, q0, flags=flags, ld_pad=8)
    want = orc.attention(dtype, q, kc, vc, q0)
    assert_attention(got, want, q, kc, vc, q0, orc, dtype, mode=mode)


@DTYPES
def test_attention_peaked_scores(ctx, pkg, orc, dtype):
    """Score std ~ 6: the running max moves often and most weights are tiny."""
    rows, q0, cap, nqh, nkvh = 192, 64, 256, 16, 8
    q, kc, vc = _attn_inputs(orc, dtype, rows, q0, cap, nqh, nkvh, 11, qscale=6.0)
    got = _attn_gpu(ctx, pkg, dtype, q, kc, vc, q0)
    want = orc.attention(dtype, q, kc, vc, q0)
    assert_attention(got, want, q, kc, vc, q0, orc, dtype)


@pytest.mark.parametrize("dtype,rows", [(F16, 1024), (BF16, 1024), (F16, 4352)])
def test_attention_prefill_length(ctx, pkg, orc, dtype, rows):
    """BASELINE's decoder shapes: 1024 tokens (config 3) and the ~4.3 k-token
    300 s prefill (config 5), 16 q heads over 8 kv heads, hd 128.  The oracle
    checks the first, the last and a middle block of 64 rows (each oracle run
    over rows i..i+64 with q0 = i is exactly those rows of the full result)."""
    nqh, nkvh = 16, 8
    q, kc, vc = _attn_inputs(orc, dtype, rows, 0, rows, nqh, nkvh, rows + dtype)
    got = _attn_gpu(ctx, pkg, dtype, q, kc, vc, 0)
    for i in (0, (rows // 2 // 64) * 64 + 5, rows - 64):
        qs = np.ascontiguousarray(q[:, i:i + 64])
        want = orc.attention(dtype, qs, kc, vc, i)
        assert_attention(got[i:i + 64], want, qs, kc, vc, i, orc, dtype)


def test_attention_is_deterministic_and_causal(ctx, pkg, orc):
    rows, nqh, nkvh = 200, 16, 8
    q, kc, vc = _attn_inputs(orc, F16, rows, 0, 208, nqh, nkvh, 5)
    a = _attn_gpu(ctx, pkg, F16, q, kc, vc, 0)
    b = _attn_gpu(ctx, pkg, F16, q, kc, vc, 0)
    assert np.array_equal(a, b)
    # new keys / values at position 150 leave rows 0..149 bit-identical
    kc2, vc2 = kc.copy(), vc.copy()
    kc2[:, 150] = _h16(orc, np.full(128, 2.0), F16)
    vc2[:, :, orc.vperm(208)[150]] = _h16(orc, np.full(128, -4.0), F16)
    c = _attn_gpu(ctx, pkg, F16, q, kc2, vc2, 0)
    assert np.array_equal(c[:150], a[:150]) and not np.array_equal(c[150:], a[150:])


def test_prefill_chain_rope_then_attention(ctx, pkg, orc):
    """qa_qk_norm_rope writes the caches qa_attention_prefill reads: the GPU
    chain over a 2-chunk prefill (rows 0..95, then 96..159 at start = 96)
    matches the oracle attention on the GPU-written caches and q."""
    nqh, nkvh, hd, cap, eps = 16, 8, 128, 160, 1e-6
    rng = np.random.default_rng(21)
    width = (nqh + 2 * nkvh) * hd
    qkv = _h16(orc, 2.0 * rng.standard_normal((cap, width)), F16)
    qn = (1.0 + 0.2 * rng.standard_normal(hd)).astype(np.float32)
    kn = (1.0 + 0.2 * rng.standard_normal(hd)).astype(np.float32)
    c, s = rope_tables(cap, hd, 0)
    d_qkv, d_qn, d_kn, d_c, d_s = (ctx.to_device(a) for a in (qkv, qn, kn, c, s))
    d_kc, d_vc = ctx.alloc(nkvh * cap * hd * 2), ctx.alloc(nkvh * hd * cap * 2)
    outs = []
    for start, rows in ((0, 96), (96, 64)):
        dq = ctx.alloc(nqh * rows * hd * 2)
        do = ctx.alloc(rows * nqh * hd * 2)
        ctx.qk_norm_rope(pkg.QkRopeDesc(
            dtype=F16, flags=0, rows=rows, nqh=nqh, nkvh=nkvh, hd=hd, eps=eps,
            qkv=int(d_qkv) + start * width * 2, ldqkv=width, qn_w=int(d_qn), kn_w=int(d_kn),
            cos=int(d_c), sin=int(d_s), pos0=start, q_out=int(dq), k_cache=int(d_kc),
            v_cache=int(d_vc), cap=cap, start=start))
        ctx.attention_prefill(pkg.AttentionDesc(
            dtype=F16, flags=0, rows=rows, nqh=nqh, nkvh=nkvh, hd=hd, q=int(dq),
            k_cache=int(d_kc), v_cache=int(d_vc), cap=cap, q0=start, out=int(do),
            ldo=nqh * hd))
        outs.append((start, ctx.download(dq, (nqh, rows, hd)), ctx.download(do, (rows, nqh * hd))))
        dq.free()
        do.free()
    kc = ctx.download(d_kc, (nkvh, cap, hd))
    vc = ctx.download(d_vc, (nkvh, hd, cap))
    wkc = np.zeros_like(kc)
    wvc = np.zeros_like(vc)
    orc.qk_norm_rope(F16, qkv, nqh, nkvh, hd, qn, kn, c, s, 0, eps, wkc, wvc, 0)
    _assert_1ulp(kc, wkc, orc, F16)
    assert np.array_equal(vc, wvc)
    for start, q, out in outs:
        want = orc.attention(F16, q, kc, vc, start)
        assert_attention(out, want, q, kc, vc, start, orc, F16)
    for b in (d_qkv, d_qn, d_kn, d_c, d_s, d_kc, d_vc):
        b.free()


# ------------------------------------------------------------- validation

def test_decoder_ops_validate(ctx, pkg):
    lib = pkg.lib()
    h = ctx.handle
    ok_attn = dict(dtype=F16, flags=0, rows=64, nqh=16, nkvh=8, hd=128, q=0x100000,
                   k_cache=0x200000, v_cache=0x300000, cap=64, q0=0, out=0x400000, ldo=2048)
    for kw, code, needle in [
        (dict(hd=64), pkg.QA_EUNSUPPORTED, "hd=64"),
        (dict(nqh=32), pkg.QA_EUNSUPPORTED, "nqh / nkvh = 4"),
        (dict(nqh=12), pkg.QA_EINVAL, "multiple of nkvh"),
        (dict(cap=72, rows=72), pkg.QA_EINVAL, "multiple of 16"),
        (dict(q0=8), pkg.QA_EINVAL, "q0 + rows <= cap"),
        (dict(flags=2), pkg.QA_EINVAL, "unknown flags"),
        (dict(ldo=2040), pkg.QA_EINVAL, "ldo"),
        (dict(q=0x100008), pkg.QA_EINVAL, "aligned"),
        (dict(out=None), pkg.QA_EINVAL, "null pointer"),
    ]:
        d = pkg.AttentionDesc(**{**ok_attn, **kw})
        assert lib.qa_attention_prefill(h, ctypes.byref(d)) == code, kw
        assert needle in pkg.last_error(), (kw, pkg.last_error())
    ok_rope = dict(dtype=F16, flags=0, rows=4, nqh=16, nkvh=8, hd=128, eps=1e-6, qkv=0x100000,
                   ldqkv=4096, qn_w=0x200000, kn_w=0x200400, cos=0x300000, sin=0x380000, pos0=0,
                   q_out=0x400000, k_cache=0x500000, v_cache=0x600000, cap=16, start=0)
    for kw, needle in [(dict(hd=96), "multiple of 64"), (dict(ldqkv=4000), "ldqkv"),
                       (dict(start=14), "start + rows <= cap"), (dict(eps=-1.0), "eps"),
                       (dict(cap=20), "multiple of 16")]:
        d = pkg.QkRopeDesc(**{**ok_rope, **kw})
        assert lib.qa_qk_norm_rope(h, ctypes.byref(d)) == pkg.QA_EINVAL, kw
        assert needle in pkg.last_error(), (kw, pkg.last_error())
    ok_rms = dict(dtype=F16, flags=0, rows=4, n=1024, x=0x100000, ldx=1024, w=0x200000,
                  y=0x300000, ldy=1024, eps=1e-6)
    for kw, needle in [(dict(n=1020), "multiple of 8"), (dict(ldy=1000), "strides"),
                       (dict(x=0x100004), "aligned"), (dict(dtype=3), "dtype")]:
        d = pkg.RmsNormDesc(**{**ok_rms, **kw})
        assert lib.qa_rms_norm(h, ctypes.byref(d)) == pkg.QA_EINVAL, kw
        assert needle in pkg.last_error(), (kw, pkg.last_error())
    # rows == 0 is a no-op that touches nothing
    d = pkg.AttentionDesc(**{**ok_attn, "rows": 0})
    assert lib.qa_attention_prefill(h, ctypes.byref(d)) == pkg.QA_OK
