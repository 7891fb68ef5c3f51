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
    the classes against the committed oracle fixture
    (tests/golden/e2e_300s.json, written by tests/golden/make_e2e_golden.py
    on the same seeded inputs), with the same near-tie rule.
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


def _run(pkg, ctx, dtype, w, x, words, max_rows):
    from qwen3_aligner_wgpu_amd import synthetic as syn
    al, enc, dec = syn.build_aligner(pkg, ctx, dtype, w, x.size / 16000 + 0.01, max_rows)
    try:
        info = al.prepare(x, words)
        al.forward()
        raw, fixed = al.result()
        out = dict(info=info, raw=raw, fixed=fixed, classes=al.read("classes"),
                   logits=al.read("logits"), ids=al.read("ids"), src=al.read("src"),
                   ts=al.read("ts_pos"), h=dec.read("h", info["seq"]))
    finally:
        al.close()
        enc.close()
        dec.close()
    return out


def _clear(gap, rms):
    return np.asarray(gap) > NEAR_TIE * np.asarray(rms)


@pytest.mark.parametrize("dtype,seconds,n_words,layers", [(F16, 7.37, 16, (2, 3)),
                                                          (BF16, 4.0, 9, (1, 2))],
                         ids=["f16-7s", "bf16-4s"])
def test_aligner_against_oracle_chain(ctx, pkg, orc, dtype, seconds, n_words, layers):
    from qwen3_aligner_wgpu_amd import synthetic as syn
    w = syn.aligner_weights(dtype, *layers, seed=7)
    x, words = _inputs(seconds, n_words, 11)
    g = _run(pkg, ctx, dtype, w, x, words, 512)
    r = oracle_aligner(orc, dtype, w, x, words, pkg.mel_filterbank(),
                       lambda n: pkg.rope_tables(n, 128, 1e6))
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


def test_aligner_e2e_300s_against_fixture(ctx, pkg):
    from qwen3_aligner_wgpu_amd import synthetic as syn
    path = os.path.join(HERE, "golden", "e2e_300s.json")
    gold = json.load(open(path))
    c = gold["config"]
    w = syn.aligner_weights(c["dtype"], c["enc_layers"], c["dec_layers"], c["seed"])
    x = syn.synthetic_audio(c["seconds"], c["seed"])
    words = [syn.word_token_ids(t) for t in syn.synthetic_words(c["words"], c["seed"])]
    import hashlib
    dg = lambda a: hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()[:16]  # noqa: E731
    assert dg(w["embed"]) == gold["digests"]["embed"] and dg(w["score"]) == gold["digests"]["score"]
    same_audio = dg(x) == gold["digests"]["samples"]
    g = _run(pkg, ctx, c["dtype"], w, x, words, 4352)
    assert g["info"]["seq"] == gold["seq"] and g["info"]["n_audio"] == gold["n_audio"]
    assert dg(g["ids"]) == gold["digests"]["ids"]
    want = np.array(gold["classes"])
    clear = _clear(gold["gap"], gold["logit_rms"])
    same = g["classes"] == want
    print(f"e2e 300 s: classes identical at {same.sum()}/{want.size} slots, "
          f"{clear.sum()} with a clear oracle margin; samples bit-identical: {same_audio}")
    assert same[clear].all(), np.nonzero(~same & clear)
