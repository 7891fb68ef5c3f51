"""The end-to-end gates (tests/chains.py rows_gate, logits_gate) on the CPU:
the oracle's forward of a small seeded config (tests/golden/e2e_tiny.json /
.npz, made by tests/golden/make_e2e_golden.py --tag tiny) is recomputed here
and must pass against its own fixture, the reference CPU path's forward
(f32 tower) must pass against the 16-bit chain's fixture (a different but
correct arithmetic), and plausible mistakes planted in the oracle's forward
must fail: layer 0's attention output zeroed, the tower's position add left
out, the head's logits taken from the neighbouring slot's row.
"""
from __future__ import annotations

import json
import os

import numpy as np
import pytest

from chains import logits_gate, oracle_aligner, rows_gate

HERE = os.path.dirname(os.path.abspath(__file__))
TINY = os.path.join(HERE, "golden", "e2e_tiny")


@pytest.fixture(scope="module")
def tiny(pkg, orc):
    from qwen3_aligner_wgpu_amd import synthetic as syn
    gold = json.load(open(TINY + ".json"))
    arr = np.load(TINY + ".npz")
    c = gold["config"]
    w = syn.aligner_weights(c["dtype"], c["enc_layers"], c["dec_layers"], c["seed"])
    x = syn.synthetic_audio(c["seconds"], c["seed"])
    words = [syn.word_token_ids(t) for t in syn.synthetic_words(c["words"], c["seed"])]
    run = lambda **kw: oracle_aligner(  # noqa: E731
        orc, c["dtype"], w, x, words, pkg.mel_filterbank(),
        lambda n: pkg.rope_tables(n, 128, 1e6, c["dtype"]), **kw)
    return gold, arr, w, run


def _gates(orc, r, gold, arr, w, prefix):
    rows = r["h"][r["ts"]]
    ok_rows, st = rows_gate(orc, gold["config"]["dtype"], rows, arr[f"{prefix}_rows"])
    ok_lg, use = logits_gate(orc, gold["config"]["dtype"], rows, r["logits32"],
                             arr[f"{prefix}_rows"], arr[f"{prefix}_top_idx"],
                             arr[f"{prefix}_top_logits"], w["norm_w"], w["score"])
    return ok_rows, st, ok_lg, use


def test_oracle_forward_passes_its_fixture(orc, tiny):
    gold, arr, w, run = tiny
    r = run()
    ok_rows, st, ok_lg, use = _gates(orc, r, gold, arr, w, "chain16")
    assert ok_rows and st["identical"] == 1.0, st
    assert ok_lg and use <= 1.0
    assert [int(v) for v in r["classes"]] == gold["classes"]


def test_cpu_reference_path_passes_the_chain_gate(orc, tiny):
    """The reference CPU path's forward (f32 tower, one f16 narrowing) is a
    correct forward with different rounding points: it passes the gates that
    the GPU forward must pass against the 16-bit chain's fixture."""
    gold, arr, w, run = tiny
    r = run(tower="f32")
    ok_rows, st, ok_lg, use = _gates(orc, r, gold, arr, w, "chain16")
    assert ok_rows, st
    assert st["identical"] < 1.0  # it really is a different arithmetic
    assert ok_lg, use
    ok_rows, st, ok_lg, use = _gates(orc, r, gold, arr, w, "cpu_ref")
    assert ok_rows and st["identical"] == 1.0 and ok_lg


@pytest.mark.parametrize("tower,skip,prefix", [("16", ("attention",), "chain16"),
                                               ("f32", ("position",), "cpu_ref"),
                                               ("f32", ("attention",), "cpu_ref")],
                         ids=["no-attention", "no-position-add", "f32-no-attention"])
def test_gates_reject_a_planted_mistake(orc, tiny, tower, skip, prefix):
    gold, arr, w, run = tiny
    r = run(tower=tower, skip=skip)
    ok_rows, st, _, _ = _gates(orc, r, gold, arr, w, prefix)
    assert not ok_rows, st
    # far outside the looser bound the 300 s test derives from two correct
    # forwards (twice their 1.3e-3 relative RMS distance)
    assert st["rel_rms"] > 50 * 2 * 1.3e-3, st


def test_logits_gate_rejects_a_shifted_row(orc, tiny):
    """Logits computed from each slot's neighbour (a wrong timestamp position)
    fall outside the bound even where the rows themselves are right."""
    gold, arr, w, run = tiny
    rows = arr["chain16_rows"]
    logits, _ = orc.timestamp_head_f32(0, np.roll(rows, 1, axis=0), np.arange(rows.shape[0]),
                                       w["norm_w"], 1e-6, w["score"])
    ok, use = logits_gate(orc, 0, rows, logits, rows, arr["chain16_top_idx"],
                          arr["chain16_top_logits"], w["norm_w"], w["score"])
    assert not ok and use > 1.0
    # and the unshifted head passes
    logits, _ = orc.timestamp_head_f32(0, rows, np.arange(rows.shape[0]), w["norm_w"], 1e-6,
                                       w["score"])
    ok, use = logits_gate(orc, 0, rows, logits, rows, arr["chain16_top_idx"],
                          arr["chain16_top_logits"], w["norm_w"], w["score"])
    assert ok, use


def test_discriminating_head_makes_the_classes_decide(pkg, orc):
    """On the 300 s fixture's rows (tests/golden/e2e_300s.npz) the random
    head gives every slot the same class, so classes read from each slot's
    neighbour (a wrong timestamp position) equal the right ones and a class
    comparison cannot see the mistake.  Under chains.discriminating_head the
    classes differ across slots and the same mistake changes most of them
    (82% of the 240; a word's two slots sit side by side and often agree)."""
    from chains import EPS, discriminating_head
    from qwen3_aligner_wgpu_amd import synthetic as syn
    path = os.path.join(HERE, "golden", "e2e_300s")
    c = json.load(open(path + ".json"))["config"]
    rows = np.load(path + ".npz")["chain16_rows"]
    dt = c["dtype"]
    w = syn.aligner_weights(dt, 0, 0, c["seed"])  # embed / norm / head only
    pos = np.arange(rows.shape[0])

    def classes(score, r):
        return orc.timestamp_head(dt, r, pos, w["norm_w"], EPS, score)[1]

    shifted = np.roll(rows, 1, axis=0)
    plain = classes(w["score"], rows)
    assert np.unique(plain).size == 1
    assert np.array_equal(classes(w["score"], shifted), plain)  # the mistake is invisible
    head2 = discriminating_head(orc, dt, rows, w["norm_w"], w["score"])
    good = classes(head2, rows)
    assert np.unique(good).size >= rows.shape[0] // 2
    assert (classes(head2, shifted) != good).mean() > 0.5  # neighbours often share a class
