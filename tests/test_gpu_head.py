"""GPU parity of the aligner's ends around the towers:

  * qa_embed_scatter, the decoder's input rows (align_raw_rows,
    src/align_inference.rs:688-714): bit-exact against a numpy gather, with
    token rows, audio rows, and out-of-range indices (zero rows);
  * qa_timestamp_head (src/align_inference.rs:760-805) against the oracle's
    head (or_timestamp_head: f32 folded norm, f64 logits).  The GPU sums the
    norm's squares in another order and the logits in f32, so each logit is
    within (2n + 64) f32 ulps of sum |normed| |score| of the oracle's, and the
    class equals the oracle's wherever the oracle's best logit leads the
    runner-up by more than twice that bound (a near-tie can go either way, in
    the reference as well: its GEMM's accumulation order decides it).

Shapes: the decoder's hidden 1024 and the 5000 labels of the checkpoint's
score head, rows up to 512 (a 300 s transcript holds a few hundred words,
two timestamps each); position rows are picked from a longer hidden state
with a row stride larger than n.
"""
from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

F16, BF16 = 0, 1


@pytest.mark.parametrize("dtype", [F16, BF16], ids=["f16", "bf16"])
def test_embed_scatter(ctx, pkg, dtype):
    rng = np.random.default_rng(11 + dtype)
    vocab, hidden, n_audio, rows = 3000, 1024, 77, 400
    table = rng.integers(0, 2 ** 16, (vocab, hidden), dtype=np.uint16)
    audio = rng.integers(0, 2 ** 16, (n_audio, hidden), dtype=np.uint16)
    src = rng.integers(0, vocab, rows).astype(np.int32)
    src[20:20 + n_audio] = -1 - np.arange(n_audio)            # the audio span
    src[5], src[6], src[7] = vocab, -1 - n_audio, 2 ** 31 - 1  # out of range -> zero rows
    src[8] = -(2 ** 31)
    want = np.zeros((rows, hidden), np.uint16)
    tok = (src >= 0) & (src < vocab)
    want[tok] = table[src[tok]]
    aud = (src < 0) & (-(src.astype(np.int64)) - 1 < n_audio)
    want[aud] = audio[-(src[aud].astype(np.int64)) - 1]
    dt, da, ds = ctx.to_device(table), ctx.to_device(audio), ctx.to_device(src)
    do = ctx.alloc(rows * hidden * 2)
    try:
        ctx.embed_scatter(pkg.EmbedDesc(dtype=dtype, flags=0, rows=rows, hidden=hidden, src=int(ds),
                                        table=int(dt), vocab=vocab, audio=int(da), n_audio=n_audio,
                                        out=int(do)))
        got = ctx.download(do, (rows, hidden))
    finally:
        for b in (dt, da, ds, do):
            b.free()
    assert np.array_equal(got, want)


def _gpu_head(ctx, pkg, dtype, h, pos, w, eps, score):
    rows, labels = pos.size, score.shape[0]
    bufs = [ctx.to_device(a) for a in (h, pos, w, score)]
    dl, dc = ctx.alloc(rows * labels * 4), ctx.alloc(rows * 4)
    try:
        ctx.timestamp_head(pkg.HeadDesc(dtype=dtype, flags=0, rows=rows, positions=int(bufs[1]),
                                        h=int(bufs[0]), h_rows=h.shape[0], ldh=h.shape[1],
                                        n=w.size, norm_w=int(bufs[2]), eps=eps,
                                        score=int(bufs[3]), labels=labels, logits=int(dl),
                                        classes=int(dc)))
        return ctx.download(dl, (rows, labels), np.float32), ctx.download(dc, rows, np.int32)
    finally:
        for b in bufs + [dl, dc]:
            b.free()


@pytest.mark.parametrize("dtype,rows", [(F16, 512), (BF16, 97), (F16, 1)],
                         ids=["f16-512", "bf16-97", "f16-1"])
def test_timestamp_head(ctx, pkg, orc, dtype, rows):
    rng = np.random.default_rng(21 + rows)
    n, labels, h_rows, ldh = 1024, 5000, 2 * rows + 5, 1040
    h = np.zeros((h_rows, ldh), np.uint16)
    h[:, :n] = orc.h16_from_f32(rng.standard_normal((h_rows, n)).astype(np.float32) * 3.0, dtype)
    w = (1.0 + 0.3 * rng.standard_normal(n)).astype(np.float32)
    score = (0.03 * rng.standard_normal((labels, n))).astype(np.float32)
    pos = np.sort(rng.permutation(h_rows)[:rows]).astype(np.int32)
    logits, cls = _gpu_head(ctx, pkg, dtype, h, pos, w, 1e-6, score)
    want_l, want_c = orc.timestamp_head(dtype, h, pos, w, 1e-6, score)
    x = orc.h16_to_f32(h[pos, :n], dtype).astype(np.float64) * w
    y = x / np.sqrt((x ** 2).mean(axis=1, keepdims=True) + 1e-6)
    bound = (2 * n + 64) * 2.0 ** -24 * (np.abs(y) @ np.abs(score.astype(np.float64)).T)
    assert (np.abs(logits - want_l) <= bound).all(), np.abs(logits - want_l).max()
    top2 = np.sort(want_l, axis=1)[:, -2:]
    clear = top2[:, 1] - top2[:, 0] > 2 * bound.max(axis=1)
    assert clear.mean() > 0.5
    assert np.array_equal(cls[clear], want_c[clear])
    # wherever the GPU disagrees, it picked a near-tie of the oracle's best
    best = want_l[np.arange(rows), want_c]
    assert (best - want_l[np.arange(rows), cls] <= 2 * bound.max(axis=1)).all()


def test_timestamp_head_out_of_range_position(ctx, pkg, orc):
    rng = np.random.default_rng(5)
    n, labels = 256, 300
    h = orc.h16_from_f32(rng.standard_normal((4, n)).astype(np.float32), F16)
    w = np.ones(n, np.float32)
    score = rng.standard_normal((labels, n)).astype(np.float32)
    pos = np.array([1, 4, -1, 2], np.int32)
    logits, cls = _gpu_head(ctx, pkg, F16, h, pos, w, 1e-6, score)
    assert (logits[1:3] == 0).all() and cls[1] == 0 and cls[2] == 0
    _, want_c = orc.timestamp_head(F16, h, pos[[0, 3]], w, 1e-6, score)
    assert cls[0] == want_c[0] and cls[3] == want_c[1]


def test_timestamp_head_ragged_width(ctx, pkg, orc):
    """A hidden width that is not a multiple of 4 takes the head's scalar
    loader (the vector one needs 16-byte rows); same bound."""
    rng = np.random.default_rng(9)
    n, labels, rows = 254, 70, 5
    h = orc.h16_from_f32(rng.standard_normal((9, n)).astype(np.float32), F16)
    w = (1.0 + 0.3 * rng.standard_normal(n)).astype(np.float32)
    score = (0.05 * rng.standard_normal((labels, n))).astype(np.float32)
    pos = np.array([0, 3, 8, 2, 5], np.int32)
    logits, cls = _gpu_head(ctx, pkg, F16, h, pos, w, 1e-6, score)
    want_l, want_c = orc.timestamp_head(F16, h, pos, w, 1e-6, score)
    x = orc.h16_to_f32(h[pos], F16).astype(np.float64) * w
    y = x / np.sqrt((x ** 2).mean(axis=1, keepdims=True) + 1e-6)
    bound = (2 * n + 64) * 2.0 ** -24 * (np.abs(y) @ np.abs(score.astype(np.float64)).T)
    assert (np.abs(logits - want_l) <= bound).all()
    top2 = np.sort(want_l, axis=1)[:, -2:]
    sure = top2[:, 1] - top2[:, 0] > 2 * bound.max(axis=1)
    assert np.array_equal(cls[sure], want_c[sure])
