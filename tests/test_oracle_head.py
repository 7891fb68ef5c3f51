"""Pins of the oracle's timestamp head (oracle/qa_oracle_audio.c
or_timestamp_head, following src/align_inference.rs:760-805).

  * the f64 closed form: normed = x w / sqrt(mean((x w)^2) + eps) computed in
    numpy f64, logits = normed . score^T; the oracle's f32 norm sits within
    (n + 8) f32 ulps (relative) of it, so its logits within that times
    sum |normed| |score|.  A norm without the weight inside the variance, a
    dropped eps or a transposed score fails it (the weights here are far from
    1 and eps is large enough to matter);
  * a constructed case with a known argmax: score row L is the normalised
    row of position L's hidden state, so row L scores |normed|^2 and any other
    unit row scores less (Cauchy-Schwarz);
  * ties: two identical score rows give the first index (`v > best_v`).
"""
from __future__ import annotations

import numpy as np

F16, BF16 = 0, 1


def _case(orc, dtype, rows, n, labels, seed):
    rng = np.random.default_rng(seed)
    h = orc.h16_from_f32(rng.standard_normal((rows + 3, n)).astype(np.float32) * 2.0, dtype)
    w = (1.0 + 0.5 * rng.standard_normal(n)).astype(np.float32)
    score = (0.05 * rng.standard_normal((labels, n))).astype(np.float32)
    pos = rng.permutation(rows + 3)[:rows].astype(np.int32)
    return h, w, score, pos


def _closed_form(orc, dtype, h, pos, w, eps, score):
    x = orc.h16_to_f32(h, dtype).astype(np.float64)[pos]
    xw = x * w.astype(np.float64)
    y = xw / np.sqrt((xw ** 2).mean(axis=1, keepdims=True) + eps)
    return y, y @ score.astype(np.float64).T


def test_head_matches_closed_form(orc):
    for dtype in (F16, BF16):
        n, eps = 1024, 0.5
        h, w, score, pos = _case(orc, dtype, 40, n, 300, 3 + dtype)
        logits, cls = orc.timestamp_head(dtype, h, pos, w, eps, score)
        y, want = _closed_form(orc, dtype, h, pos, w, eps, score)
        bound = (n + 8) * 2.0 ** -24 * (np.abs(y) @ np.abs(score.astype(np.float64)).T) + 1e-300
        assert (np.abs(logits - want) <= bound).all()
        assert np.array_equal(cls, np.argmax(logits, axis=1))
        # the planted mistakes this bound catches
        x = orc.h16_to_f32(h, dtype).astype(np.float64)[pos]
        unfolded = x / np.sqrt((x ** 2).mean(axis=1, keepdims=True) + eps) * w
        assert not (np.abs(unfolded @ score.T - want) <= bound).all()
        no_eps = x * w / np.sqrt(((x * w) ** 2).mean(axis=1, keepdims=True))
        assert not (np.abs(no_eps @ score.T - want) <= bound).all()


def test_head_known_argmax_and_ties(orc):
    dtype, n, rows = F16, 256, 16
    h, w, _, pos = _case(orc, dtype, rows, n, 1, 7)
    pos = np.arange(rows, dtype=np.int32)
    y, _ = _closed_form(orc, dtype, h, pos, w, 1e-6, np.zeros((1, n), np.float32))
    unit = y / np.linalg.norm(y, axis=1, keepdims=True)
    labels = 2 * rows
    score = np.zeros((labels, n), np.float32)
    score[rows:] = unit.astype(np.float32)          # row r's own direction at label rows + r
    score[3] = score[rows + 3]                      # a tie with an earlier label
    _, cls = orc.timestamp_head(dtype, h, pos, w, 1e-6, score)
    want = np.arange(rows) + rows
    want[3] = 3
    assert np.array_equal(cls, want)
