"""The timestamp repair: the host library's qah_fix_timestamps
(csrc/host/aligner.cpp) and the oracle's restatement (oracle/oracle.py),
both against the reference's own known-answer vectors
(tests/golden/fix_timestamps.json, from src/postprocess.rs:156-222), then
against each other on random class sequences, with the invariants the
repair promises: a non-decreasing output, the kept subsequence unchanged,
every value within the input's range, and an already non-decreasing input
returned as is.
"""
from __future__ import annotations

import json
import os

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
CASES = json.load(open(os.path.join(HERE, "golden", "fix_timestamps.json")))["cases"]


@pytest.fixture(scope="module")
def host(pkg):
    from qwen3_aligner_wgpu_amd import host
    return host


@pytest.mark.parametrize("case", CASES, ids=[c["name"] for c in CASES])
def test_known_answers(orc, host, case):
    for got in (orc.fix_timestamps(case["data"]), list(host.fix_timestamps(case["data"]))):
        if case["want"] is not None:
            assert got == case["want"]
        assert all(a <= b for a, b in zip(got, got[1:]))


def _lis_len(x):
    best = []
    for i, v in enumerate(x):
        best.append(1 + max([best[j] for j in range(i) if x[j] <= v], default=0))
    return max(best, default=0)


def test_random_sequences_match_and_hold_the_invariants(orc, host):
    rng = np.random.default_rng(3)
    for trial in range(400):
        n = int(rng.integers(0, 60))
        # a drifting sequence of 80 ms classes with outliers, as the head emits
        base = np.cumsum(rng.integers(0, 4, n)) * 80
        noise = rng.random(n) < rng.uniform(0, 0.4)
        data = np.where(noise, rng.integers(0, 5000, n) * 80, base).astype(np.int64)
        got = host.fix_timestamps(data)
        want = orc.fix_timestamps(data)
        assert list(got) == want, (trial, list(data))
        if n:
            assert (np.diff(got) >= 0).all()
            assert got.min() >= data.min() and got.max() <= data.max()
            # a longest non-decreasing subsequence is kept as it is
            assert (got == data).sum() >= _lis_len(list(data))
    mono = np.sort(rng.integers(0, 10 ** 6, 50))
    assert list(host.fix_timestamps(mono)) == list(mono)


def test_known_answers_pin_the_rounding_and_the_distance_rule():
    """The vectors separate the reference's choices from two plausible slips:
    rounding the interpolation instead of truncating, and snapping a short
    run to the neighbour nearer in value instead of in index."""
    case = next(c for c in CASES if c["name"] == "interpolation_truncates_toward_zero")
    step = (101 - 4) / 4
    assert [round(4 + step * k) for k in (1, 2, 3)] != case["want"][2:5]
    case = next(c for c in CASES
                if c["name"] == "short_block_snaps_to_the_nearer_neighbour_by_index_distance")
    by_value = [100 if abs(v - 100) <= abs(200 - v) else 200 for v in case["data"][2:4]]
    assert by_value != case["want"][2:4]
