"""GPU parity of the aligner's forward pass (the host mirror of
Aligner::align_raw_rows, csrc/host/aligner.cpp: samples -> log-mel ->
audio tower -> embedding gather + audio scatter -> decoder prefill ->
timestamp head -> fix_timestamps) against the oracle chain (tests/chains.py
oracle_aligner: the same steps from the oracle's ops, a 16-bit rounding
after every op).

Inputs are the benchmark's (synthetic.py): seeded synthetic audio (noise at
-30 dBFS plus tone bursts), synthetic words through the tokenizer stand-in,
seeded random-init weights.

Gates:
  * the assembled input (ids, audio-row sources, timestamp positions) equals
    the oracle's assembly (src/align_input.rs) exactly;
  * the head stage: the classes equal the oracle head's on the GPU's own
    final hidden state, except where that head's best two logits are within
    its f32 error bound (as in test_gpu_head);
  * the chain: the final hidden state within the north star's mean absolute
    error and a relative RMS of one 16-bit ulp; the classes identical at
    every slot whose oracle margin (best minus second logit) exceeds 2^-8 of
    the slot's logit RMS (a margin below that is a near-tie, which a 16-bit
    forward can answer either way -- the reference notes the same of its own
    GPU path); the repaired times equal the oracle's repair of the GPU's
    classes;
  * at the benchmark's end-to-end config (300 s, 120 words, 18 + 28 layers)
    against the committed oracle fixture (tests/golden/e2e_300s.json / .npz,
    written by tests/golden/make_e2e_golden.py on the same seeded inputs):
    the final hidden rows at the 240 <timestamp> slots and the logits at each
    slot's 8 best labels (the gates of tests/chains.py, which
    tests/test_e2e_gate.py shows reject planted mistakes), the classes with
    the same near-tie rule, and the distance to the reference CPU path's
    forward (its f32 tower).  With random-init weights the <timestamp>
    embedding dominates those rows, so every slot picks the same class: the
    classes alone would not tell a correct forward from a wrong one, the rows
    and logits do;
  * the head stage again with a head whose classes differ by slot
    (chains.discriminating_head: the random head with the rows' shared
    directions projected out), rerun on the same aligner: logits within the
    f32 bound, every class a maximum within it, classes varied.
"""
from __future__ import annotations

import json
import os

import numpy as np
import pytest

from chains import EPS, assemble, oracle_aligner

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
F16, BF16 = 0, 1
NEAR_TIE = 2.0 ** -8


def _inputs(seconds, n_words, seed):
    from qwen3_aligner_wgpu_amd import synthetic as syn
    x = syn.synthetic_audio(seconds, seed)
    words = [syn.word_token_ids(t) for t in syn.synthetic_words(n_words, seed)]
    return x, words


def _run(pkg, ctx, dtype, w, x, words, max_rows, heads=()):
    """The forward with w's head, then once more per extra score head in
    `heads` (loaded into the same aligner): out["extra"][i] holds that
    forward's classes, logits and final rows."""
    from qwen3_aligner_wgpu_amd import synthetic as syn
    al, enc, dec = syn.build_aligner(pkg, ctx, dtype, w, x.size / 16000 + 0.01, max_rows)
    try:
        info = al.prepare(x, words)
        al.forward()
        raw, fixed = al.result()
        out = dict(info=info, raw=raw, fixed=fixed, classes=al.read("classes"),
                   logits=al.read("logits"), ids=al.read("ids"), src=al.read("src"),
                   ts=al.read("ts_pos"), h=dec.read("h", info["seq"]), extra=[])
        for score in heads:
            al.load_head(w["norm_w"], score)
            al.forward()
            out["extra"].append(dict(classes=al.read("classes"), logits=al.read("logits"),
                                     h=dec.read("h", info["seq"])))
    finally:
        al.close()
        enc.close()
        dec.close()
    return out


def _clear(gap, rms):
    return np.asarray(gap) > NEAR_TIE * np.asarray(rms)


def _discriminating_gate(orc, dtype, g, e, ts, norm_w, score, min_distinct):
    """The forward `e`, run with a discriminating head (chains.discriminating_head)
    loaded into the same aligner: its final rows equal the first forward's
    (only the head changed); its logits are within the f32 head's error bound
    of the oracle head's (f64) on those rows; at every slot its class is a
    maximum of the exact logits to within that bound (the chosen label's
    exact logit at least the best one's less both labels' bounds), and equals
    the oracle's class wherever the best two logits are apart by more than
    twice the bound; and the classes differ across slots (at least
    min_distinct), so this head-stage gate decides something, which the
    random head, with one class at every slot, does not.  The head's classes
    are not compared across two forwards: with the shared directions
    projected out they follow the rows' smallest differences, and two correct
    oracle forwards of the 300 s config (16-bit and f32 tower, 1.3e-3
    relative RMS apart) agree at fewer than half of the slots under it."""
    rows = e["h"][ts]
    assert np.array_equal(e["h"], g["h"])
    hl, hc = orc.timestamp_head(dtype, rows, np.arange(ts.size), norm_w, EPS, score)
    y = orc.head_fold(dtype, rows, np.arange(ts.size), norm_w, EPS).astype(np.float64)
    bound = (2 * y.shape[1] + 64) * 2.0 ** -24 * (np.abs(y) @ np.abs(score.astype(np.float64)).T)
    assert (np.abs(e["logits"] - hl) <= bound).all()
    r = np.arange(ts.size)
    cls = e["classes"]
    assert (hl[r, cls] >= hl[r, hc] - bound[r, cls] - bound[r, hc]).all()
    top2 = np.sort(hl, axis=1)[:, -2:]
    sure = top2[:, 1] - top2[:, 0] > 2 * bound.max(axis=1)
    assert np.array_equal(cls[sure], hc[sure])
    distinct = np.unique(cls).size
    print(f"discriminating head: {distinct} distinct classes over {ts.size} slots, equal to the "
          f"oracle head's at {(cls == hc).sum()} ({sure.sum()} outside twice the f32 bound)")
    assert distinct >= min_distinct, distinct


@pytest.mark.parametrize("dtype,seconds,n_words,layers", [(F16, 7.37, 16, (2, 3)),
                                                          (BF16, 4.0, 9, (1, 2))],
                         ids=["f16-7s", "bf16-4s"])
def test_aligner_against_oracle_chain(ctx, pkg, orc, dtype, seconds, n_words, layers):
    from qwen3_aligner_wgpu_amd import synthetic as syn
    from chains import discriminating_head
    w = syn.aligner_weights(dtype, *layers, seed=7)
    x, words = _inputs(seconds, n_words, 11)
    r = oracle_aligner(orc, dtype, w, x, words, pkg.mel_filterbank(),
                       lambda n: pkg.rope_tables(n, 128, 1e6, dtype))
    _, _, ts0 = assemble(r["n_audio"], words)
    head2 = discriminating_head(orc, dtype, r["h"][ts0], w["norm_w"], w["score"])
    g = _run(pkg, ctx, dtype, w, x, words, 512, heads=[head2])
    # the assembled input
    assert g["info"]["n_audio"] == r["n_audio"] and g["info"]["seq"] == r["ids"].size
    ids, src, ts = assemble(r["n_audio"], words)
    assert np.array_equal(g["ids"], ids) and np.array_equal(g["src"], src)
    assert np.array_equal(g["ts"], ts)
    # the head on the GPU's own final hidden state
    hl, hc = orc.timestamp_head(dtype, g["h"], ts, w["norm_w"], EPS, w["score"])
    top2 = np.sort(hl, axis=1)[:, -2:]
    xw = orc.h16_to_f32(g["h"][ts], dtype).astype(np.float64) * w["norm_w"]
    y = xw / np.sqrt((xw ** 2).mean(axis=1, keepdims=True) + EPS)
    bound = (2 * 1024 + 64) * 2.0 ** -24 * (np.abs(y) @ np.abs(w["score"].astype(np.float64)).T)
    assert (np.abs(g["logits"] - hl) <= bound).all()
    sure = top2[:, 1] - top2[:, 0] > 2 * bound.max(axis=1)
    assert np.array_equal(g["classes"][sure], hc[sure])
    # the chain
    gh = orc.h16_to_f32(g["h"], dtype).astype(np.float64)
    rh = orc.h16_to_f32(r["h"], dtype).astype(np.float64)
    ulp = 2.0 ** -10 if dtype == F16 else 2.0 ** -7
    assert np.abs(gh - rh).mean() <= 1e-3 * (1 if dtype == F16 else 8)
    assert np.sqrt(((gh - rh) ** 2).mean() / (rh ** 2).mean()) <= ulp
    lg = r["logits"]
    srt = np.sort(lg, axis=1)
    clear = _clear(srt[:, -1] - srt[:, -2], np.sqrt((lg ** 2).mean(axis=1)))
    assert np.array_equal(g["classes"][clear], r["classes"][clear]), (g["classes"], r["classes"])
    print(f"classes identical at {(g['classes'] == r['classes']).sum()}/{ts.size} slots "
          f"({clear.sum()} with a clear margin)")
    assert np.array_equal(g["raw"], (g["classes"] * 80).astype(np.int64))
    assert list(g["fixed"]) == orc.fix_timestamps(list(g["raw"]))
    # a head whose classes differ by slot
    _discriminating_gate(orc, dtype, g, g["extra"][0], ts, w["norm_w"], head2,
                         min_distinct=ts.size // 4)


def test_aligner_e2e_300s_against_fixture(ctx, pkg, orc):
    """BASELINE config 5 against the oracle's forward of the same seeded
    inputs (tests/golden/e2e_300s.json / .npz):
      * the final hidden rows at the 240 <timestamp> slots against the 16-bit
        chain's (rows_gate).  After 18 + 28 layers of 16-bit arithmetic two
        correct forwards drift apart by more than an ulp: the oracle's own
        16-bit-tower and f32-tower forwards are 1.3e-3 relative RMS apart
        (rows16_vs_cpu_ref in the fixture).  The GPU, which rounds where the
        16-bit chain does, may differ from it by at most twice that distance
        in relative RMS and MAE; a wiring mistake moves the rows by orders of
        magnitude more (tests/test_e2e_gate.py);
      * the logits at each slot's 8 best labels within what the two sets of
        rows allow (logits_gate);
      * the classes identical at every slot with a clear oracle margin;
      * against the reference CPU path's forward (f32 tower, cpu_ref): the
        rows within twice the oracle chains' distance, and the classes
        identical at clear slots;
      * the head stage once more under a discriminating head built from the
        fixture's rows (_discriminating_gate): the random head gives every
        slot one class, this one about 180 over the 240 slots."""
    from qwen3_aligner_wgpu_amd import synthetic as syn
    from chains import logits_gate, rows_gate
    path = os.path.join(HERE, "golden", "e2e_300s")
    gold = json.load(open(path + ".json"))
    arr = np.load(path + ".npz")
    c = gold["config"]
    w = syn.aligner_weights(c["dtype"], c["enc_layers"], c["dec_layers"], c["seed"])
    x = syn.synthetic_audio(c["seconds"], c["seed"])
    words = [syn.word_token_ids(t) for t in syn.synthetic_words(c["words"], c["seed"])]
    import hashlib
    dg = lambda a: hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()[:16]  # noqa: E731
    assert dg(w["embed"]) == gold["digests"]["embed"] and dg(w["score"]) == gold["digests"]["score"]
    same_audio = dg(x) == gold["digests"]["samples"]
    from chains import discriminating_head
    head2 = discriminating_head(orc, c["dtype"], arr["chain16_rows"], w["norm_w"], w["score"])
    g = _run(pkg, ctx, c["dtype"], w, x, words, 4352, heads=[head2])
    assert g["info"]["seq"] == gold["seq"] and g["info"]["n_audio"] == gold["n_audio"]
    assert dg(g["ids"]) == gold["digests"]["ids"]
    assert list(g["ts"]) == gold["ts"]
    rows = g["h"][g["ts"]]
    drift = gold["rows16_vs_cpu_ref"]
    ok, st = rows_gate(orc, c["dtype"], rows, arr["chain16_rows"],
                       rel_rms_bound=2 * drift["rel_rms"], mae_bound=2 * drift["mae"])
    ok_lg, use = logits_gate(orc, c["dtype"], rows, g["logits"], arr["chain16_rows"],
                             arr["chain16_top_idx"], arr["chain16_top_logits"], w["norm_w"],
                             w["score"])
    want = np.array(gold["classes"])
    clear = _clear(gold["gap"], gold["logit_rms"])
    same = g["classes"] == want
    print(f"e2e 300 s vs the 16-bit chain: rows {st}; logits bound use {use:.3f}; classes "
          f"identical at {same.sum()}/{want.size} slots, {clear.sum()} with a clear margin; "
          f"samples bit-identical: {same_audio}")
    assert ok, st
    assert ok_lg, use
    assert same[clear].all(), np.nonzero(~same & clear)
    # the reference CPU path (f32 tower)
    ref = gold["cpu_ref"]
    _, st_ref = rows_gate(orc, c["dtype"], rows, arr["cpu_ref_rows"])
    want_ref = np.array(ref["classes_f32_head"])
    clear_ref = _clear(ref["gap"], ref["logit_rms"])
    same_ref = g["classes"] == want_ref
    print(f"e2e 300 s vs the reference CPU path (f32 tower): rows {st_ref}; classes identical at "
          f"{same_ref.sum()}/{want_ref.size} slots ({clear_ref.sum()} clear)")
    assert st_ref["rel_rms"] <= 2 * drift["rel_rms"], (st_ref, drift)
    assert same_ref[clear_ref].all(), np.nonzero(~same_ref & clear_ref)
    # every slot's class above is the same one (random init): the head stage
    # again under a head whose classes differ by slot
    _discriminating_gate(orc, c["dtype"], g, g["extra"][0], g["ts"], w["norm_w"], head2,
                         min_distinct=g["ts"].size // 4)


def test_failed_prepare_forgets_the_previous_clip(ctx, pkg):
    """A prepare that fails (here: an audio placeholder id among the words)
    leaves nothing prepared: forward() refuses with QA_EINVAL instead of
    aligning the previous clip, and the host arrays describe nothing."""
    from qwen3_aligner_wgpu_amd import synthetic as syn
    w = syn.aligner_weights(F16, 1, 1, seed=3)
    x, words = _inputs(2.0, 3, 4)
    al, enc, dec = syn.build_aligner(pkg, ctx, F16, w, 2.1, 256)
    try:
        al.prepare(x, words)
        al.forward()
        with pytest.raises(pkg.QAError) as e:
            al.prepare(x, words + [[151676]])  # audio_pad among the word ids
        assert e.value.code == pkg.QA_EINVAL
        with pytest.raises(pkg.QAError) as e:
            al.forward()
        assert e.value.code == pkg.QA_EINVAL
        # a good prepare afterwards works again
        al.prepare(x, words)
        al.forward()
        assert al.result()[0].size == 2 * len(words)
    finally:
        al.close()
        enc.close()
        dec.close()
