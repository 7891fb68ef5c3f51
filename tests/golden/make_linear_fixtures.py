#!/usr/bin/env python3
"""Writes tests/golden/linear_fixtures.json: digests of the oracle's linear
outputs (oracle/qa_oracle.c or_linear, f64-exact and f32 modes) on seeded
inputs from the host library's counter-based generator, for M in {1, 7, 64},
N = 384, K in {16, 1024}, f16 and bf16, each epilogue.  tests/test_oracle.py
recomputes them, so a change to the oracle's arithmetic or rounding shows as
a digest mismatch.

    python tests/golden/make_linear_fixtures.py
"""
from __future__ import annotations

import hashlib
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))


def cases():
    for dtype in (0, 1):
        for m in (1, 7, 64):
            for k in (16, 1024):
                for epi in ("plain", "bias", "acc", "bias_gelu", "silu"):
                    yield dict(dtype=dtype, m=m, n=384, k=k, epi=epi)


def run(orc, host, c):
    """The oracle's exact and f32 outputs for case c (inputs from seed 3, tensor
    ids derived from the case)."""
    dt, m, n, k, epi = c["dtype"], c["m"], c["n"], c["k"], c["epi"]
    tid = 1000 * dt + 100 * m + k
    a = host.synth_normal(3, tid, (m, k), 0.0, 1.0, dt)
    w = host.synth_normal(3, tid + 1, (n, k), 0.0, 0.05, dt)
    bias = host.synth_normal(3, tid + 2, (n,), 0.0, 0.1, dt) if "bias" in epi else None
    c0 = host.synth_normal(3, tid + 3, (m, n // 2 if epi == "silu" else n), 0.0, 1.0, dt)
    flags = {"plain": 0, "bias": 0, "acc": orc.ACCUMULATE, "bias_gelu": orc.EPI_GELU,
             "silu": orc.EPI_SILU_MUL}[epi]
    out = []
    for extra in (orc.EXACT, 0):
        cc = c0.copy() if epi == "acc" else np.zeros_like(c0)
        out.append(orc.linear(dt, a, w, cc, flags=flags | extra, bias=bias))
    return out


def digest(x: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(x).tobytes()).hexdigest()[:20]


def main():
    import __graft_entry__ as entry
    entry.load_package()
    orc = entry.load_oracle()
    from qwen3_aligner_wgpu_amd import host
    out = []
    for c in cases():
        exact, f32 = run(orc, host, c)
        out.append(dict(c, exact=digest(exact), f32=digest(f32),
                        exact_head=[int(v) for v in exact.reshape(-1)[:4]]))
    json.dump({"note": "digests of oracle/qa_oracle.c or_linear outputs on seeded inputs; "
                       "written by tests/golden/make_linear_fixtures.py", "cases": out},
              open(os.path.join(HERE, "linear_fixtures.json"), "w"), indent=0)
    print(f"{len(out)} cases")


if __name__ == "__main__":
    main()
