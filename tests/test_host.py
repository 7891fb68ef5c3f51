"""Host-side logic of the C++ mirror, on the CPU: the seeded synthetic-input
generator, 16-bit narrowing (src/weights.rs:57-89 narrow_h16_into; its
rounding must equal the oracle's, i.e. the reference's) and the fused-row
concatenation of src/decoder.rs:840-871 / src/weights.rs:345-360."""
from __future__ import annotations

import numpy as np
import pytest


@pytest.fixture(scope="module")
def host(pkg):
    from qwen3_aligner_wgpu_amd import host as h

    return h


def test_synth_is_deterministic_and_salted(host):
    a = host.synth_normal(0, 11, (1000,))
    b = host.synth_normal(0, 11, (1000,))
    c = host.synth_normal(0, 12, (1000,))
    d = host.synth_normal(1, 11, (1000,))
    assert np.array_equal(a, b)
    assert not np.array_equal(a, c) and not np.array_equal(a, d)
    # thread count does not change the stream: a large draw's prefix is the small draw
    big = host.synth_normal(0, 11, (1 << 18,))
    assert np.array_equal(big[:1000], a)


def test_synth_moments(host):
    x = host.synth_normal_f32(0, 3, (1 << 20,), 0.0, 0.02)
    assert abs(x.mean()) < 1e-4 and abs(x.std() - 0.02) < 2e-4
    y = host.synth_normal_f32(0, 4, (1 << 20,), 1.5, 1.0)
    assert abs(y.mean() - 1.5) < 5e-3 and abs(y.std() - 1.0) < 5e-3
    # tails of a Gaussian, not of a uniform
    assert 0.002 < (np.abs(y - 1.5) > 3).mean() < 0.0035


@pytest.mark.parametrize("dt", [0, 1], ids=["f16", "bf16"])
def test_narrowing_matches_oracle(host, orc, dt):
    x = host.synth_normal_f32(5, 1, (200_000,), 0.0, 3.0)
    x[:6] = [0.1, -0.0, 65504.0, 1e-8, 3.0e38, -65520.0]
    assert np.array_equal(host.narrow(x, dt), orc.h16_from_f32(x, dt))
    h = host.synth_normal(5, 1, (200_000,), 0.0, 3.0, dt)
    assert np.array_equal(h, orc.h16_from_f32(host.synth_normal_f32(5, 1, (200_000,), 0.0, 3.0), dt))


def test_concat_rows(host):
    rng = np.random.default_rng(0)
    parts = [rng.integers(0, 65535, (r, 24), dtype=np.uint16) for r in (16, 8, 8)]
    assert np.array_equal(host.concat_rows(parts), np.concatenate(parts))
