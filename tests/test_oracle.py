"""Pins the CPU oracle (oracle/qa_oracle.c) before it is trusted as the checker.

Each function is checked against what fixes it independently:
  * the reference's own known-answer tests (src/half16.rs:95-157,
    src/shaders.rs:191-254, src/cpu_decoder.rs:620-646), whose inputs and
    bounds are in tests/golden/reference_kats.json;
  * library routines that implement the same standard: numpy's float16 cast
    (IEEE round-to-nearest-even) and torch's bfloat16 cast (RNE, the rule
    half::bf16::from_f32 follows), numpy float64 matmul, math.erf;
  * invariants of the linear op (zero operand, transposed layout, batching,
    fused-row splits) and f64 closed forms.
A mistake such as a transposed operand, a dropped bias or residual term, a
swapped gate/up half or a truncating (not rounding) conversion fails one of
these.
"""
from __future__ import annotations

import json
import math
import os

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
KATS = json.load(open(os.path.join(HERE, "golden", "reference_kats.json")))


def _lcg_sweep(seed: int, n: int) -> np.ndarray:
    """The reference's sweep generator, s = s*1664525 + 1013904223 (u32)."""
    out = np.empty(n, np.uint32)
    s = seed
    for i in range(n):
        s = (s * 1664525 + 1013904223) & 0xFFFFFFFF
        out[i] = s
    return out


def _halfway_grid() -> np.ndarray:
    g = KATS["bf16_halfway_grid"]
    vals = []
    for e in g["exponents"]:
        for mt in g["mantissa_top"]:
            for low in g["low_bits"]:
                for sign in (0, 1 << 31):
                    vals.append(sign | (e << 23) | (mt << 16) | low)
    return np.array(vals, np.uint32)


@pytest.fixture(scope="module")
def sweep_bits():
    kat = KATS["bf16_sweep"]
    bits = np.concatenate([_halfway_grid(), _lcg_sweep(kat["seed"], kat["count"])])
    f = bits.view(np.float32)
    return bits[np.isfinite(f)]


def test_bf16_known_answer(orc):
    """src/half16.rs:113-119: 0.1f32 = 0x3DCCCCCD rounds (not truncates) to 0x3DCD."""
    kat = KATS["bf16_known_answer"]
    x = np.float32(kat["input"])
    assert orc.lib().or_bf16_from_f32(float(x)) == kat["bits"]
    assert kat["bits"] != (x.view(np.uint32) >> 16)
    assert orc.lib().or_bf16_to_f32(kat["bits"]) == np.uint32(kat["bits"] << 16).view(np.float32)
    assert orc.lib().or_f16_from_f32(float(x)) != kat["bits"]


def test_round_trip_values(orc):
    """src/half16.rs:95-110: narrowing a widened 16-bit value is the identity."""
    for v in KATS["round_trip_values"]:
        for dt in (orc.F16, orc.BF16):
            b = orc.h16_from_f32(np.array([v], np.float32), dt)
            again = orc.h16_from_f32(orc.h16_to_f32(b, dt), dt)
            assert again[0] == b[0], (v, dt)
    for dt in (orc.F16, orc.BF16):
        assert orc.h16_to_f32(orc.h16_from_f32(np.array([-0.0], np.float32), dt), dt)[0] == 0.0


def test_bf16_rounding_matches_torch(orc, sweep_bits):
    """The halfway grid + LCG sweep of src/shaders.rs:191-243, against torch's RNE cast."""
    torch = pytest.importorskip("torch")
    f = sweep_bits.view(np.float32)
    ours = orc.h16_from_f32(f, orc.BF16)
    want = torch.from_numpy(f.copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    bad = np.nonzero(ours != want)[0]
    assert bad.size == 0, [(hex(sweep_bits[i]), hex(ours[i]), hex(want[i])) for i in bad[:8]]
    assert f.size > 400_000


def test_f16_rounding_matches_numpy(orc, sweep_bits):
    """f16 RNE (half::f16::from_f32) against numpy's IEEE cast, same inputs
    plus every f16 halfway point and the overflow/underflow edges."""
    f = sweep_bits.view(np.float32)
    edges = []
    for h in range(0, 0x7C00):  # every finite positive f16 and the midpoint above it
        lo = np.float32(np.uint16(h).view(np.float16))
        hi = np.float32(np.uint16(h + 1).view(np.float16))
        mid = np.float32((np.float64(lo) + np.float64(hi)) / 2)
        edges += [lo, mid, np.nextafter(mid, np.float32(0)), np.nextafter(mid, np.float32(np.inf))]
    edges = np.array(edges, np.float32)
    allv = np.concatenate([f, edges, -edges, np.array([65504, 65519.99, 65520, 1e-8, 2.0**-25, 2.0**-24], np.float32)])
    with np.errstate(over="ignore"):
        want = allv.astype(np.float16).view(np.uint16)
    ours = orc.h16_from_f32(allv, orc.F16)
    bad = np.nonzero(ours != want)[0]
    assert bad.size == 0, [(float(allv[i]), hex(ours[i]), hex(want[i])) for i in bad[:8]]


def test_widening_is_exact(orc):
    """Every 16-bit pattern widens to the value numpy/IEEE gives (NaNs stay NaN)."""
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    f16 = orc.h16_to_f32(bits, orc.F16)
    want = bits.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(f16), nan)
    assert np.array_equal(f16[~nan].view(np.uint32), want[~nan].view(np.uint32))
    bf = orc.h16_to_f32(bits, orc.BF16)
    assert np.array_equal(bf.view(np.uint32), bits.astype(np.uint32) << 16)


@pytest.mark.parametrize("shape", [tuple(s) for s in KATS["gemm_row_major_matches_naive"]["shapes"]])
def test_gemm_reference_kat(orc, shape):
    """src/cpu_decoder.rs:620-646 verbatim: closed-form inputs, worst |d| < 1e-3
    against a naive f32 triple loop, at the toy and the production shapes."""
    kat = KATS["gemm_row_major_matches_naive"]
    m, n, k = shape
    xi, wi = kat["x"], kat["w"]
    x = ((np.arange(m * k) * xi["mul"] % xi["mod"]).astype(np.float32) * np.float32(xi["scale"])
         - np.float32(xi["offset"])).reshape(m, k)
    w = ((np.arange(n * k) * wi["mul"] % wi["mod"]).astype(np.float32) * np.float32(wi["scale"])
         - np.float32(wi["offset"])).reshape(n, k)
    got = orc.gemm_f32(x, w)
    naive = orc.gemm_f32_naive(x, w)
    assert np.abs(got - naive).max() < kat["bound"]
    exact = x.astype(np.float64) @ w.astype(np.float64).T
    assert np.abs(got - exact).max() < kat["bound"]
    assert np.abs(naive - exact).max() < kat["bound"]


def test_gemm_f64_and_beta(orc):
    rng = np.random.default_rng(1)
    x = rng.standard_normal((37, 129)).astype(np.float32)
    w = rng.standard_normal((53, 129)).astype(np.float32)
    exact = x.astype(np.float64) @ w.astype(np.float64).T
    np.testing.assert_allclose(orc.gemm_f64(x, w), exact, rtol=1e-12, atol=1e-12)
    # beta: out = beta*out + x.w^T (the gemm crate's (beta, alpha) order,
    # src/cpu_decoder.rs:576-610)
    base = rng.standard_normal((37, 53)).astype(np.float32)
    got = orc.gemm_f32(x, w, base.copy(), beta=0.5)
    np.testing.assert_allclose(got, 0.5 * base + exact, rtol=1e-5, atol=1e-4)
    # a transposed operand would not match: W is [n, k], not [k, n]
    assert not np.allclose(orc.gemm_f32(x, w), x @ w.T[:, ::-1], atol=1e-3)


def _rand16(orc, rng, shape, dt, std=1.0):
    return orc.h16_from_f32((std * rng.standard_normal(shape)).astype(np.float32), dt)


def _ulp_dist(a, b):
    a = a.astype(np.int64)
    b = b.astype(np.int64)
    oa = np.where(a & 0x8000, -(a & 0x7FFF), a)
    ob = np.where(b & 0x8000, -(b & 0x7FFF), b)
    return np.abs(oa - ob)


@pytest.mark.parametrize("dt", [0, 1], ids=["f16", "bf16"])
def test_linear_matches_f64_rounding(orc, dt):
    """Plain linear: one rounding of the f32 accumulator, so within 1 ulp of the
    exactly rounded f64 result and mostly identical to it."""
    rng = np.random.default_rng(2)
    a, w = _rand16(orc, rng, (48, 256), dt), _rand16(orc, rng, (96, 256), dt, 0.05)
    c = orc.linear(dt, a, w, np.zeros((48, 96), np.uint16))
    exact = orc.h16_to_f32(a, dt).astype(np.float64) @ orc.h16_to_f32(w, dt).astype(np.float64).T
    want = orc.h16_from_f32(exact.astype(np.float32), dt)
    assert _ulp_dist(c, want).max() <= 1
    assert (c == want).mean() > 0.95
    ex = orc.linear(dt, a, w, np.zeros((48, 96), np.uint16), flags=orc.EXACT)
    assert _ulp_dist(ex, want).max() <= 1


@pytest.mark.parametrize("dt", [0, 1], ids=["f16", "bf16"])
def test_linear_epilogue_terms(orc, dt):
    """bias, residual and GELU each enter the single rounding: f64 closed form."""
    rng = np.random.default_rng(3)
    m, n, k = 32, 64, 128
    a, w = _rand16(orc, rng, (m, k), dt), _rand16(orc, rng, (n, k), dt, 0.05)
    bias, c0 = _rand16(orc, rng, (n,), dt, 0.5), _rand16(orc, rng, (m, n), dt)
    A = orc.h16_to_f32(a, dt).astype(np.float64)
    W = orc.h16_to_f32(w, dt).astype(np.float64)
    B = orc.h16_to_f32(bias, dt).astype(np.float64)
    C0 = orc.h16_to_f32(c0, dt).astype(np.float64)
    acc = A @ W.T
    cases = {
        "bias": (orc.linear(dt, a, w, np.zeros((m, n), np.uint16), bias=bias, flags=orc.EXACT), acc + B),
        "acc": (orc.linear(dt, a, w, c0.copy(), flags=orc.ACCUMULATE | orc.EXACT), acc + C0),
        "bias_acc": (orc.linear(dt, a, w, c0.copy(), bias=bias, flags=orc.ACCUMULATE | orc.EXACT),
                     acc + B + C0),
    }
    gelu = np.vectorize(lambda v: 0.5 * v * (1.0 + math.erf(v / math.sqrt(2.0))))
    cases["gelu"] = (orc.linear(dt, a, w, np.zeros((m, n), np.uint16), bias=bias,
                                flags=orc.EPI_GELU | orc.EXACT), gelu(acc + B))
    for name, (got, ref) in cases.items():
        want = orc.h16_from_f32(ref.astype(np.float32), dt)
        assert _ulp_dist(got, want).max() <= 1, name
        # dropping the term would not pass
    dropped = orc.h16_from_f32(acc.astype(np.float32), dt)
    assert _ulp_dist(cases["bias"][0], dropped).max() > 1


def test_bias_rows_and_invariants(orc):
    rng = np.random.default_rng(4)
    dt = orc.F16
    m, n, k = 16, 40, 64
    a, w = _rand16(orc, rng, (m, k), dt), _rand16(orc, rng, (n, k), dt, 0.05)
    brow = _rand16(orc, rng, (m,), dt)
    got = orc.linear(dt, a, w, np.zeros((m, n), np.uint16), bias=brow, flags=orc.BIAS_ROWS | orc.EXACT)
    ref = (orc.h16_to_f32(a, dt).astype(np.float64) @ orc.h16_to_f32(w, dt).astype(np.float64).T
           + orc.h16_to_f32(brow, dt)[:, None])
    assert _ulp_dist(got, orc.h16_from_f32(ref.astype(np.float32), dt)).max() <= 1
    # zero A with ACCUMULATE leaves C unchanged (bit-exact)
    c0 = _rand16(orc, rng, (m, n), dt)
    z = np.zeros((m, k), np.uint16)
    assert np.array_equal(orc.linear(dt, z, w, c0.copy(), flags=orc.ACCUMULATE), c0)
    # zero W with a bias gives the bias
    bias = _rand16(orc, rng, (n,), dt)
    got = orc.linear(dt, a, np.zeros((n, k), np.uint16), np.zeros((m, n), np.uint16), bias=bias)
    assert np.array_equal(got, np.broadcast_to(bias, (m, n)))


def test_transb_and_batch_are_layouts(orc):
    """W as [k, n] (TRANSB) and batching change layout only: bit-identical."""
    rng = np.random.default_rng(5)
    dt = orc.BF16
    m, n, k, b = 24, 32, 48, 3
    a, w = _rand16(orc, rng, (b, m, k), dt), _rand16(orc, rng, (b, n, k), dt, 0.1)
    plain = np.stack([orc.linear(dt, a[i].copy(), w[i].copy(), np.zeros((m, n), np.uint16))
                      for i in range(b)])
    wt = np.ascontiguousarray(np.transpose(w, (0, 2, 1)))
    tb = np.stack([orc.linear(dt, a[i].copy(), wt[i].copy(), np.zeros((m, n), np.uint16),
                              flags=orc.TRANSB, n=n) for i in range(b)])
    assert np.array_equal(plain, tb)
    batched = orc.linear(dt, a, w, np.zeros((b, m, n), np.uint16), m=m, n=n, k=k, batch=b,
                         bsa=m * k, bsb=n * k, bsc=m * n)
    assert np.array_equal(plain, batched)


@pytest.mark.parametrize("dt", [0, 1], ids=["f16", "bf16"])
def test_silu_mul_rounding_points(orc, dt):
    """src/cpu_decoder.rs:496-505: gate and up rounded to 16 bits, then
    f16(silu(g)*u) with silu(g) = g/(1+exp(-g)); the [gate|up] halves of W
    (src/decoder.rs:840-871) must not be swapped."""
    rng = np.random.default_rng(6)
    m, inter, k = 20, 48, 96
    a = _rand16(orc, rng, (m, k), dt)
    w = _rand16(orc, rng, (2 * inter, k), dt, 0.1)
    got = orc.linear(dt, a, w, np.zeros((m, inter), np.uint16), flags=orc.EPI_SILU_MUL | orc.EXACT)
    acc = orc.h16_to_f32(a, dt).astype(np.float64) @ orc.h16_to_f32(w, dt).astype(np.float64).T
    g = orc.h16_to_f32(orc.h16_from_f32(acc[:, :inter].astype(np.float32), dt), dt).astype(np.float64)
    u = orc.h16_to_f32(orc.h16_from_f32(acc[:, inter:].astype(np.float32), dt), dt).astype(np.float64)
    want = orc.h16_from_f32((g / (1 + np.exp(-g)) * u).astype(np.float32), dt)
    assert _ulp_dist(got, want).max() <= 1
    swapped = orc.h16_from_f32((u / (1 + np.exp(-u)) * g).astype(np.float32), dt)
    assert _ulp_dist(got, swapped).max() > 1


def test_silu_brute_force_all_f16_gates(orc):
    """or_silu_mul over every finite f16 gate value at fixed up values, against
    the f64 formula: relative error within a few f32 ulps."""
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    g = bits.view(np.float16).astype(np.float32)
    g = g[np.isfinite(g)]
    for u in (1.0, -0.37, 2.5e-3):
        got = np.array([orc.silu_mul(float(x), u) for x in g[::7]], np.float64)
        gg = g[::7].astype(np.float64)
        with np.errstate(over="ignore"):
            ref = gg / (1.0 + np.exp(-gg)) * u
        err = np.abs(got - ref) / np.maximum(np.abs(ref), 1e-30)
        assert err[np.abs(ref) > 1e-30].max() < 4e-7, u
    assert orc.silu_mul(0.0, 5.0) == 0.0


def test_gelu_against_erf(orc):
    xs = np.linspace(-8, 8, 4001, dtype=np.float32)
    got = np.array([orc.gelu(float(x)) for x in xs], np.float64)
    ref = np.array([0.5 * x * (1 + math.erf(x / math.sqrt(2))) for x in xs.astype(np.float64)])
    assert np.abs(got - ref).max() < 2e-6


def test_fused_rows_split_back(orc):
    """[q|k|v] fused rows (src/decoder.rs:840-871): column blocks of the fused
    output equal the separate projections (src/cpu_decoder.rs:456-458)."""
    rng = np.random.default_rng(7)
    dt = orc.F16
    a = _rand16(orc, rng, (16, 64), dt)
    parts = [_rand16(orc, rng, (r, 64), dt, 0.05) for r in (32, 16, 16)]
    fused = orc.linear(dt, a, np.concatenate(parts), np.zeros((16, 64), np.uint16), flags=orc.EXACT)
    lo = 0
    for p in parts:
        sep = orc.linear(dt, a, p, np.zeros((16, p.shape[0]), np.uint16), flags=orc.EXACT)
        assert np.array_equal(fused[:, lo:lo + p.shape[0]], sep)
        lo += p.shape[0]


def test_linear_rejects_bad_descriptors(orc):
    a = np.zeros((4, 16), np.uint16)
    w = np.zeros((8, 16), np.uint16)
    c = np.zeros((4, 8), np.uint16)
    with pytest.raises(ValueError):
        orc.linear(orc.F16, a, w, c, flags=orc.EPI_GELU | orc.ACCUMULATE)
    with pytest.raises(ValueError):
        orc.linear(orc.F16, a, w, c, flags=orc.EPI_SILU_MUL, bias=np.zeros(8, np.uint16))
    with pytest.raises(ValueError):
        orc.linear(7, a, w, c)


def test_linear_fixtures_regression(orc, pkg):
    """The oracle's linear outputs (f64-exact and f32 modes, every epilogue,
    f16 and bf16, M in {1, 7, 64}, K in {16, 1024}) on seeded inputs match the
    digests committed in tests/golden/linear_fixtures.json (written by
    tests/golden/make_linear_fixtures.py): a change to the oracle's arithmetic
    or rounding points shows here."""
    import importlib.util
    import json
    import os
    here = os.path.dirname(os.path.abspath(__file__))
    spec = importlib.util.spec_from_file_location(
        "make_linear_fixtures", os.path.join(here, "golden", "make_linear_fixtures.py"))
    mk = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mk)
    from qwen3_aligner_wgpu_amd import host
    fx = json.load(open(os.path.join(here, "golden", "linear_fixtures.json")))["cases"]
    assert len(fx) == len(list(mk.cases()))
    for c in fx:
        case = {k: c[k] for k in ("dtype", "m", "n", "k", "epi")}
        exact, f32 = mk.run(orc, host, case)
        assert mk.digest(exact) == c["exact"], case
        assert mk.digest(f32) == c["f32"], case
