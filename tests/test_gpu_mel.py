"""GPU parity of qa_log_mel (the log-mel front end, src/mel.rs:203-243, plus
the chunking of encode, src/audio_encoder_gpu.rs:1079-1091) against the
oracle (oracle/qa_oracle_audio.c or_log_mel: f64 STFT pinned to numpy's rfft,
the slaney filterbank, log10 / clamp / affine in f64).

The GPU accumulates the DFT in f64 and runs the filterbank, log10 and clamp
in f32, so each output is within one 16-bit ulp of the oracle's value (the
f32 log10 and filterbank sum differ from f64 by a few f32 ulps, which moves
only rounding ties); frames past the last valid one are exactly 0.

Inputs: BASELINE config 5's synthetic audio (white noise at -30 dBFS plus
200-800 Hz tones in 0.3-0.8 s bursts, seeded), at lengths from one frame to
300 s, including a partial last chunk.
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import assert_parity

pytestmark = pytest.mark.gpu

F16, BF16 = 0, 1


def synth_audio(seconds, seed, sr=16000):
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


def _gpu_mel(ctx, pkg, dtype, x, fb):
    frames = x.size // 160
    n_chunks = (frames + 99) // 100
    dx, df = ctx.to_device(x), ctx.to_device(fb)
    do = ctx.alloc(n_chunks * 128 * 100 * 2)
    ctx.log_mel(pkg.MelDesc(dtype=dtype, flags=0, n_samples=x.size, samples=int(dx),
                            filterbank=int(df), n_mels=128, cs=100, out=int(do)))
    out = ctx.download(do, (n_chunks, 128, 100))
    for b in (dx, df, do):
        b.free()
    return out


@pytest.mark.parametrize("dtype", [F16, BF16], ids=["f16", "bf16"])
@pytest.mark.parametrize("seconds", [0.01, 1.0, 2.37, 30.0, 300.0])
def test_log_mel(ctx, pkg, orc, dtype, seconds):
    x = synth_audio(seconds, int(seconds * 100))
    fb = pkg.mel_filterbank()
    got = _gpu_mel(ctx, pkg, dtype, x, fb)
    lm = orc.log_mel(x, fb)  # [128, frames] f32
    frames = lm.shape[1]
    n_chunks = got.shape[0]
    want = np.zeros((n_chunks, 128, 100), np.float32)
    for c in range(n_chunks):
        seg = lm[:, c * 100:min(frames, (c + 1) * 100)]
        want[c, :, :seg.shape[1]] = seg
    want16 = orc.h16_from_f32(want, dtype)
    s = assert_parity(got, want16, orc, dtype, ulp_tol=1)
    assert s["identical"] >= 0.99, s
    tail = frames - (n_chunks - 1) * 100
    assert (got[-1, :, tail:] == 0).all()
