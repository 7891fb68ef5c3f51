"""Shared fixtures.

`-m gpu` tests need an MI355X and call the product through the C ABI
(csrc/libqa.so); everything else runs on the CPU.  The oracle
(oracle/liboracle.so) is the checker in both.
"""
from __future__ import annotations

import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

import __graft_entry__ as entry  # noqa: E402


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def _ensure_built() -> None:
    pkg_lib = os.path.join(entry.PKG_DIR, "csrc", "libqa.so")
    host_lib = os.path.join(entry.PKG_DIR, "csrc", "libqa_host.so")
    orc_lib = os.path.join(ROOT, "oracle", "liboracle.so")
    if not (os.path.exists(pkg_lib) and os.path.exists(host_lib) and os.path.exists(orc_lib)):
        entry.build()


@pytest.fixture(scope="session")
def pkg():
    _ensure_built()
    return entry.load_package()


@pytest.fixture(scope="session")
def orc():
    _ensure_built()
    return entry.load_oracle()


@pytest.fixture(scope="session")
def ctx(pkg):
    c = pkg.Context(0)
    yield c
    c.close()


def parity_stats(got_bits: np.ndarray, want_bits: np.ndarray, orc, dtype: int) -> dict:
    """The north star's statistics: max relative error with the
    max(|r|, 1e-3 max|r|) floor, mean absolute error, share of bit-identical
    16-bit outputs and the largest distance in units in the last place."""
    g = orc.h16_to_f32(got_bits, dtype).astype(np.float64)
    r = orc.h16_to_f32(want_bits, dtype).astype(np.float64)
    err = np.abs(g - r)
    floor = 1e-3 * max(np.abs(r).max(), 1e-30)
    rel = err / np.maximum(np.abs(r), floor)

    def ordinal(bits):
        b = bits.astype(np.int64)
        return np.where(b & 0x8000, -(b & 0x7FFF), b)

    # ulp distance where |r| is above the floor: near zero, the f32
    # accumulation error of any summation order spans several subnormal ulps.
    ulp = np.abs(ordinal(got_bits) - ordinal(want_bits))[np.abs(r) >= floor]
    return {
        "max_rel": float(rel.max()) if rel.size else 0.0,
        "mae": float(err.mean()) if err.size else 0.0,
        "identical": float((got_bits == want_bits).mean()) if err.size else 1.0,
        "max_ulp": int(ulp.max()) if ulp.size else 0,
        "finite": bool(np.isfinite(g).all()),
    }


# North-star gate for 16-bit outputs: max relative error <= 1e-2 and mean
# absolute error <= 1e-3 against the reference CPU path on identical inputs.
REL_TOL = 1e-2
MAE_TOL = 1e-3


def assert_parity(got_bits, want_bits, orc, dtype, rel_tol=REL_TOL, mae_tol=MAE_TOL, ulp_tol=None):
    s = parity_stats(got_bits, want_bits, orc, dtype)
    assert s["finite"], s
    assert s["max_rel"] <= rel_tol and s["mae"] <= mae_tol, s
    if ulp_tol is not None:
        assert s["max_ulp"] <= ulp_tol, s
    return s
