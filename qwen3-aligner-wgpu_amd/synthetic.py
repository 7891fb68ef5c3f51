"""Seeded synthetic inputs and random-init weights for the aligner's forward
pass (the shapes of the Qwen3-ForcedAligner-0.6B checkpoint, which is not
available here), and the builder that loads them into the host mirror.

Weights come from qah_synth_normal (a counter-based SplitMix64 / Box-Muller
stream per tensor id), so every process that asks for the same (seed,
tensor id, shape) gets the same bits: the benchmark, the GPU tests and the
script that computes the oracle's classes for the end-to-end fixture all
see the same model.
"""
from __future__ import annotations

import numpy as np

from . import host

AUDIO = dict(n_mels=128, cs=100, c_conv=480, d_model=896, nh=14, ffn=3584, out_dim=1024, wlen=104)
TEXT = dict(hidden=1024, nqh=16, nkvh=8, hd=128, inter=3072, eps=1e-6)
VOCAB, LABELS, SEGMENT_MS = 151936, 5000, 80.0
TEXT_VOCAB = 151643  # ids below the special tokens
SAMPLE_RATE = 16000


def synthetic_audio(seconds: float, seed: int, sr: int = SAMPLE_RATE) -> np.ndarray:
    """White noise at -30 dBFS plus 200-800 Hz tones of amplitude 0.2 in
    0.3-0.8 s bursts with 0.1-0.5 s gaps, f32."""
    rng = np.random.default_rng(seed)
    n = int(seconds * sr)
    x = rng.standard_normal(n) * 10 ** (-30 / 20)
    t = 0.0
    while t < seconds:
        dur = rng.uniform(0.3, 0.8)
        f0 = rng.uniform(200, 800)
        a, b = int(t * sr), min(n, int((t + dur) * sr))
        x[a:b] += 0.2 * np.sin(2 * np.pi * f0 * np.arange(b - a) / sr)
        t += dur + rng.uniform(0.1, 0.5)
    return x.astype(np.float32)


def synthetic_words(n: int, seed: int) -> list[str]:
    """n words of 2-8 lowercase ASCII letters."""
    rng = np.random.default_rng(seed)
    return ["".join(chr(97 + int(c)) for c in rng.integers(0, 26, int(rng.integers(2, 9))))
            for _ in range(n)]


def word_token_ids(word: str, vocab: int = TEXT_VOCAB) -> list[int]:
    """Stand-in for the checkpoint's BPE tokenizer (absent here): the word in
    pieces of up to 4 letters (ceil(len / 4) ids), each piece an id in
    [0, vocab) from its FNV-1a hash, so a 2-8 letter word costs 1-2 ids (the
    reference's 15 s clip spends 48 BPE ids on 39 words).  The ids stay below
    the special tokens."""
    ids = []
    for i in range(0, len(word), 4):
        h = 0xcbf29ce484222325
        for ch in word[i:i + 4].encode():
            h = ((h ^ ch) * 0x100000001b3) & 0xFFFFFFFFFFFFFFFF
        ids.append(int(h % vocab))
    return ids


def aligner_weights(dtype: int, enc_layers: int, dec_layers: int, seed: int = 5) -> dict:
    """Random-init weights: linears ~ N(0, 0.02) with biases ~ N(0, 0.01)
    (the tower's), conv weights ~ N(0, 1/fan_in) with biases ~ N(0, 0.05),
    every norm weight 1 and every LayerNorm bias 0, the token embedding
    ~ N(0, 0.02), the score head ~ N(0, 0.02) in f32.

    Returns {"enc": {conv, co, layers, post}, "dec": [layer dicts],
    "embed", "norm_w", "score"} in the checkpoint's layouts ([out][in]
    linears, [c_out][c_in][3][3] convs)."""
    g = lambda tid, shape, std: host.synth_normal(seed, tid, shape, 0.0, std, dtype)  # noqa: E731
    f = lambda tid, shape, mean, std: host.synth_normal_f32(seed, tid, shape, mean, std)  # noqa: E731
    cc, dm, ff, od = AUDIO["c_conv"], AUDIO["d_model"], AUDIO["ffn"], AUDIO["out_dim"]
    enc = dict(
        conv=[(g(1, (cc, 1, 3, 3), 1 / 3.0), g(2, (cc,), 0.05)),
              (g(3, (cc, cc, 3, 3), (9 * cc) ** -0.5), g(4, (cc,), 0.05)),
              (g(5, (cc, cc, 3, 3), (9 * cc) ** -0.5), g(6, (cc,), 0.05))],
        co=(g(7, (dm, cc * 16), (cc * 16) ** -0.5), g(8, (dm,), 0.01)),
        layers=[], post=None)
    for li in range(enc_layers):
        b = 1000 + 16 * li
        enc["layers"].append(dict(
            ln1=(f(b, (dm,), 1.0, 0.0), f(b + 1, (dm,), 0.0, 0.0)),
            qkv=(g(b + 2, (3 * dm, dm), 0.02), g(b + 3, (3 * dm,), 0.01)),
            o=(g(b + 4, (dm, dm), 0.02), g(b + 5, (dm,), 0.01)),
            ln2=(f(b + 6, (dm,), 1.0, 0.0), f(b + 7, (dm,), 0.0, 0.0)),
            fc1=(g(b + 8, (ff, dm), 0.02), g(b + 9, (ff,), 0.01)),
            fc2=(g(b + 10, (dm, ff), 0.02), g(b + 11, (dm,), 0.01))))
    enc["post"] = ((f(20, (dm,), 1.0, 0.0), f(21, (dm,), 0.0, 0.0)),
                   (g(22, (dm, dm), 0.02), g(23, (dm,), 0.01)),
                   (g(24, (od, dm), 0.02), g(25, (od,), 0.01)))
    hs, hd, nq, nk, it = TEXT["hidden"], TEXT["hd"], TEXT["nqh"], TEXT["nkvh"], TEXT["inter"]
    dec = []
    for li in range(dec_layers):
        b = 5000 + 16 * li
        dec.append(dict(
            q=g(b, (nq * hd, hs), 0.02), k=g(b + 1, (nk * hd, hs), 0.02),
            v=g(b + 2, (nk * hd, hs), 0.02), o=g(b + 3, (hs, nq * hd), 0.02),
            gate=g(b + 4, (it, hs), 0.02), up=g(b + 5, (it, hs), 0.02),
            down=g(b + 6, (hs, it), 0.02),
            iln=f(b + 7, (hs,), 1.0, 0.0), pln=f(b + 8, (hs,), 1.0, 0.0),
            qn=f(b + 9, (hd,), 1.0, 0.0), kn=f(b + 10, (hd,), 1.0, 0.0)))
    return dict(enc=enc, dec=dec, embed=g(30, (VOCAB, hs), 0.02),
                norm_w=f(31, (hs,), 1.0, 0.0), score=f(32, (LABELS, hs), 0.0, 0.02))


def build_aligner(pkg, ctx, dtype: int, w: dict, max_seconds: float, max_rows: int):
    """An AudioEncoder, a TextDecoder (RoPE tables for max_rows positions) and
    the Aligner over them, loaded with `w`.  Returns (aligner, encoder, decoder);
    close the aligner before the other two."""
    max_samples = int(max_seconds * SAMPLE_RATE)
    max_chunks = (max_samples // 160 + AUDIO["cs"] - 1) // AUDIO["cs"]
    A, T = AUDIO, TEXT
    enc = host.AudioEncoder(ctx, dtype, len(w["enc"]["layers"]), max_chunks, A["n_mels"], A["cs"],
                            A["c_conv"], A["d_model"], A["nh"], A["ffn"], A["out_dim"], A["wlen"])
    dec = host.TextDecoder(ctx, dtype, len(w["dec"]), max_rows, T["hidden"], T["nqh"], T["nkvh"],
                           T["hd"], T["inter"], T["eps"])
    try:
        for lv, (cw, cb) in enumerate(w["enc"]["conv"]):
            enc.load_conv(lv, cw, cb)
        enc.load_conv_out(*w["enc"]["co"])
        for li, l in enumerate(w["enc"]["layers"]):
            enc.load_layer(li, *l["ln1"], *l["qkv"], *l["o"], *l["ln2"], *l["fc1"], *l["fc2"])
        (lw, lb), (p1w, p1b), (p2w, p2b) = w["enc"]["post"]
        enc.load_post(lw, lb, p1w, p1b, p2w, p2b)
        for li, l in enumerate(w["dec"]):
            dec.load_layer(li, l["q"], l["k"], l["v"], l["o"], l["gate"], l["up"], l["down"],
                           l["iln"], l["pln"], l["qn"], l["kn"])
        dec.set_rope(*pkg.rope_tables(max_rows, T["hd"], 1e6, dtype))
        al = host.Aligner(ctx, enc, dec, VOCAB, LABELS, SEGMENT_MS, max_samples)
    except Exception:
        enc.close()
        dec.close()
        raise
    try:
        al.load_embed(w["embed"])
        al.load_head(w["norm_w"], w["score"])
    except Exception:
        al.close()
        enc.close()
        dec.close()
        raise
    return al, enc, dec
