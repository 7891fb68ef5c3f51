#!/usr/bin/env python3
"""Computes the oracle's timestamp classes for the aligner's end-to-end
config (300 s of synthetic 16 kHz audio, 120 synthetic
words, the 18-layer audio tower and the 28-layer decoder with seeded
random-init weights, f16) and writes them to tests/golden/e2e_<tag>.json.

The GPU test and the benchmark rebuild the same inputs (synthetic.py:
seeded audio, words and weights) and compare their classes with the ones
stored here.  Besides the classes, the file keeps per slot the oracle's gap
between its best and second-best logit (a slot whose gap is below the
accumulated difference of two correct 16-bit forward passes is a near-tie),
and digests of the inputs so a consumer can tell whether it rebuilt the same
ones.  Runs on the CPU only (the oracle plus the host library's seeded
generator); about ten minutes on 8 cores at full size.

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


def digest(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()[:16]


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
    log("inputs ready")
    r = oracle_aligner(orc, args.dtype, w, x, ids, pkg.mel_filterbank(),
                       lambda n: pkg.rope_tables(n, 128, 1e6), log)
    lg = r["logits"]
    order = np.argsort(-lg, axis=1, kind="stable")[:, :2]
    top = lg[np.arange(lg.shape[0]), order[:, 0]]
    second = lg[np.arange(lg.shape[0]), order[:, 1]]
    raw = [int(c * syn.SEGMENT_MS) for c in r["classes"]]
    out = dict(
        note="oracle classes of the aligner forward; written by tests/golden/make_e2e_golden.py",
        config=dict(seconds=args.seconds, words=args.words, enc_layers=args.enc_layers,
                    dec_layers=args.dec_layers, dtype=args.dtype, seed=args.seed),
        digests=dict(samples=digest(x), ids=digest(r["ids"]), embed=digest(w["embed"]),
                     score=digest(w["score"]), dec0_q=digest(w["dec"][0]["q"]) if w["dec"] else None,
                     mel=digest(r["mel"]), h0=digest(r["h0"]), h=digest(r["h"])),
        seq=int(r["ids"].size), n_audio=int(r["n_audio"]), frames=int(r["frames"]),
        classes=[int(c) for c in r["classes"]],
        gap=[float(v) for v in top - second],
        logit_rms=[float(v) for v in np.sqrt((lg ** 2).mean(axis=1))],
        raw_ms=raw, fixed_ms=[int(v) for v in orc.fix_timestamps(raw)],
        seconds_cpu=round(time.time() - t0, 1),
    )
    path = os.path.join(HERE, f"e2e_{args.tag}.json")
    json.dump(out, open(path, "w"))
    log(f"wrote {path}: {len(out['classes'])} slots, min gap {min(out['gap']):.3g}")


if __name__ == "__main__":
    main()
