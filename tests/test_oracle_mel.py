"""Pins the log-mel restatement (oracle/qa_oracle_audio.c: or_mel_filterbank,
or_stft_power, or_log_mel; the reference's src/mel.rs) before it checks
qa_log_mel.  The reference's FFT is the rustfft crate (absent here), so the
STFT is pinned to numpy's rfft of the same frames, and the rest to what the
definitions fix:
  * the power spectrum: numpy.fft.rfft of numpy.pad(mode="reflect") frames
    times the periodic Hann window, last frame dropped (src/mel.rs:47-98,203-214);
  * the slaney filterbank (src/mel.rs:100-154): 1 kHz is mel 15 (the linear /
    log junction), each filter is zero outside its two neighbours' centres and
    has unit area (the slaney normalisation), peaks at its centre frequency;
  * the log-mel: a pure tone's energy peaks in the mel bin whose centre is
    nearest the tone; scaling the signal by c shifts every output by
    log10(c^2) / 4 (log10 shifts every value and the clip max, hence the
    floor, alike); silence maps every value to (log10(1e-10) + 4) / 4.
"""
from __future__ import annotations

import numpy as np
import pytest


def _numpy_power(x, n_fft=400, hop=160):
    xp = np.pad(x.astype(np.float64), n_fft // 2, mode="reflect")
    frames = x.size // hop
    win = 0.5 * (1 - np.cos(2 * np.pi * np.arange(n_fft) / n_fft))
    fr = np.stack([xp[f * hop:f * hop + n_fft] * win for f in range(frames)])
    return np.abs(np.fft.rfft(fr, axis=1)) ** 2


def test_stft_power_matches_numpy_rfft(orc):
    rng = np.random.default_rng(0)
    for n in (160, 401, 4000, 16000 + 77):
        x = rng.standard_normal(n).astype(np.float32)
        got = orc.stft_power(x)
        want = _numpy_power(x)
        assert got.shape == want.shape
        assert np.allclose(got, want, rtol=1e-9, atol=1e-9 * want.max())


def test_slaney_filterbank_shape(orc):
    fb = orc.mel_filterbank(128, 400, 16000).astype(np.float64)
    nf, df = 201, 16000 / 400
    f_sp, logstep = 200.0 / 3.0, np.log(6.4) / 27.0
    hz2mel = lambda f: np.where(f < 1000, f / f_sp, 15.0 + np.log(np.maximum(f, 1e-9) / 1000) / logstep)  # noqa: E731
    assert abs(hz2mel(np.array(1000.0)) - 15.0) < 1e-12
    mel_pts = np.linspace(0, hz2mel(np.array(8000.0)), 130)
    hz_pts = np.where(mel_pts < 15, f_sp * mel_pts, 1000 * np.exp(logstep * (mel_pts - 15)))
    freqs = np.arange(nf) * df
    for i in range(128):
        outside = (freqs <= hz_pts[i]) | (freqs >= hz_pts[i + 2])
        assert (fb[i][outside] == 0).all(), i
        if hz_pts[i + 2] - hz_pts[i] > 8 * df:  # wide enough for the bin sum to be an area
            assert abs(fb[i].sum() * df - 1.0) < 0.03, (i, fb[i].sum() * df)
            assert abs(freqs[np.argmax(fb[i])] - hz_pts[i + 1]) <= df


def test_log_mel_tone_scale_and_silence(orc):
    sr, n = 16000, 16000
    t = np.arange(n) / sr
    fb = orc.mel_filterbank()
    for f0 in (300.0, 1000.0, 2500.0):
        x = (0.3 * np.sin(2 * np.pi * f0 * t)).astype(np.float32)
        lm = orc.log_mel(x, fb)
        mid = lm[:, 20:80].mean(axis=1)
        centres = (np.arange(201) * 40.0)[np.argmax(fb, axis=1)]
        assert abs(centres[np.argmax(mid)] - f0) < 0.08 * f0 + 40, (f0, centres[np.argmax(mid)])
        lm2 = orc.log_mel((x * 7.5).astype(np.float32), fb)
        assert np.abs(lm2 - lm - 2 * np.log10(7.5) / 4).max() < 1e-4  # power scales by c^2
    silent = orc.log_mel(np.zeros(3200, np.float32), fb)
    assert np.allclose(silent, (-10.0 + 4.0) / 4.0)
