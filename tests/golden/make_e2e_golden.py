#!/usr/bin/env python3
"""Computes the oracle's results for the aligner's end-to-end config
(300 s of synthetic 16 kHz audio, 120 synthetic words,
the 18-layer audio tower and the 28-layer decoder with seeded random-init
weights, f16) and writes them to tests/golden/e2e_<tag>.json (+ .npz).

Two CPU forwards run on the same seeded inputs (synthetic.py):
  * "chain16": the tower with the reference GPU tower's rounding points (every
    op rounded to 16 bits), as this build's GPU tower computes it; then the
    decoder with the CPU decoder's rounding points and the head;
  * "cpu_ref": the reference's CPU path, CpuAudioEncoder::forward in f32
    throughout with one f16 narrowing (src/audio_encoder.rs:754-832,
    src/align_inference.rs:124-131), then the same decoder and head.
For each the files keep, per <timestamp> slot: the class from the f64 logits
and from the reference's f32 head (src/align_inference.rs:766-805), the gap
between the best two logits (a slot whose gap is below the accumulated
difference of two correct 16-bit forwards is a near-tie), the logit RMS, the
final hidden row (f16 bits, .npz) and the 8 largest logits with their label
ids (.npz); plus digests of the inputs so a consumer can tell whether it
rebuilt the same ones.  CPU only (the oracle plus the host library's seeded
generator); about half an hour on 8 cores at full size.

    python tests/golden/make_e2e_golden.py                     # config 5
    python tests/golden/make_e2e_golden.py --seconds 12 --words 20 --enc-layers 2 --dec-layers 3 --tag small
"""
from __future__ import annotations

import argparse
import hashlib
import json
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.dirname(HERE))

TOPK = 8


def digest(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()[:16]


def rows_distance(a_bits, b_bits):
    """MAE and relative RMS between two sets of f16 rows (b the reference)."""
    a = a_bits.view(np.float16).astype(np.float64)
    b = b_bits.view(np.float16).astype(np.float64)
    d = a - b
    return dict(mae=float(np.abs(d).mean()), rel_rms=float(np.sqrt((d ** 2).mean() / (b ** 2).mean())))


def summary(r, topk=TOPK):
    """Per-slot results of one oracle forward: json-able lists + arrays."""
    lg = r["logits"]
    order = np.argsort(-lg, axis=1, kind="stable")
    top = order[:, :topk]
    best = lg[np.arange(lg.shape[0]), order[:, 0]]
    second = lg[np.arange(lg.shape[0]), order[:, 1]]
    js = dict(classes=[int(c) for c in r["classes"]],
              classes_f32_head=[int(c) for c in r["classes32"]],
              gap=[float(v) for v in best - second],
              logit_rms=[float(v) for v in np.sqrt((lg ** 2).mean(axis=1))])
    arrays = dict(rows=np.ascontiguousarray(r["h"][r["ts"]]),
                  top_idx=top.astype(np.int32),
                  top_logits=np.take_along_axis(lg, top, axis=1))
    return js, arrays


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--seconds", type=float, default=300.0)
    ap.add_argument("--words", type=int, default=120)
    ap.add_argument("--enc-layers", type=int, default=18)
    ap.add_argument("--dec-layers", type=int, default=28)
    ap.add_argument("--dtype", type=int, default=0)
    ap.add_argument("--seed", type=int, default=5)
    ap.add_argument("--tag", default="300s")
    args = ap.parse_args()

    import __graft_entry__ as entry
    from chains import oracle_aligner
    pkg = entry.load_package()
    orc = entry.load_oracle()
    from qwen3_aligner_wgpu_amd import synthetic as syn

    t0 = time.time()
    log = lambda *a: print(f"[{time.time() - t0:7.1f}s]", *a, flush=True)  # noqa: E731
    w = syn.aligner_weights(args.dtype, args.enc_layers, args.dec_layers, args.seed)
    x = syn.synthetic_audio(args.seconds, args.seed)
    words = syn.synthetic_words(args.words, args.seed)
    ids = [syn.word_token_ids(t) for t in words]
    fb = pkg.mel_filterbank()
    rope = lambda n: pkg.rope_tables(n, 128, 1e6, args.dtype)  # noqa: E731
    log("inputs ready")
    r = oracle_aligner(orc, args.dtype, w, x, ids, fb, rope, log)
    js16, ar16 = summary(r)
    raw = [int(c * syn.SEGMENT_MS) for c in r["classes"]]
    out = dict(
        note="oracle results of the aligner forward; written by tests/golden/make_e2e_golden.py",
        config=dict(seconds=args.seconds, words=args.words, enc_layers=args.enc_layers,
                    dec_layers=args.dec_layers, dtype=args.dtype, seed=args.seed),
        digests=dict(samples=digest(x), ids=digest(r["ids"]), embed=digest(w["embed"]),
                     score=digest(w["score"]), dec0_q=digest(w["dec"][0]["q"]) if w["dec"] else None,
                     mel=digest(r["mel"]), h0=digest(r["h0"]), h=digest(r["h"])),
        seq=int(r["ids"].size), n_audio=int(r["n_audio"]), frames=int(r["frames"]),
        ts=[int(v) for v in r["ts"]],
        raw_ms=raw, fixed_ms=[int(v) for v in orc.fix_timestamps(raw)],
        **js16,
    )
    arrays = {f"chain16_{k}": v for k, v in ar16.items()}
    log(f"chain16 done: min gap {min(out['gap']):.3g}")
    if args.dtype == 0:
        c = oracle_aligner(orc, args.dtype, w, x, ids, fb, rope, log, tower="f32")
        jsc, arc = summary(c)
        out["cpu_ref"] = dict(digests=dict(audio=digest(c["audio"]), h=digest(c["h"])), **jsc)
        arrays.update({f"cpu_ref_{k}": v for k, v in arc.items()})
        a16 = orc.h16_to_f32(r["audio"], 0).astype(np.float64)
        a32 = orc.h16_to_f32(c["audio"], 0).astype(np.float64)
        d = a16 - a32
        out["tower16_vs_cpu_ref"] = dict(mae=float(np.abs(d).mean()),
                                         rel_rms=float(np.sqrt((d ** 2).mean() / (a32 ** 2).mean())))
        out["rows16_vs_cpu_ref"] = rows_distance(ar16["rows"], arc["rows"])
        log(f"cpu_ref done: tower distance {out['tower16_vs_cpu_ref']}")
    out["seconds_cpu"] = round(time.time() - t0, 1)
    path = os.path.join(HERE, f"e2e_{args.tag}.json")
    json.dump(out, open(path, "w"))
    np.savez_compressed(os.path.join(HERE, f"e2e_{args.tag}.npz"), **arrays)
    log(f"wrote {path} (+ .npz): {len(out['classes'])} slots")


if __name__ == "__main__":
    main()
