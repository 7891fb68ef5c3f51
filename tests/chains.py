"""Oracle chains shared by the GPU parity tests and the end-to-end fixture
script: the audio tower, a decoder layer, the log-mel chunking, the input
assembly and the whole aligner forward, each composed from the oracle's ops
with a 16-bit rounding after every op (the reference's GPU path stores every
intermediate in the 16-bit format; src/audio_encoder.rs:754-832 and
src/cpu_decoder.rs:416-512 give the op order).
"""
from __future__ import annotations

import numpy as np

NM, CS, CC, DM, NH, FFN, OD, WLEN = 128, 100, 480, 896, 14, 3584, 1024, 104
HID, NQH, NKVH, HD, INTER, EPS = 1024, 16, 8, 128, 3072, 1e-6
AUDIO_START, AUDIO_END, AUDIO_PAD, TIMESTAMP = 151669, 151670, 151676, 151705


def perm_conv(w):
    """[c_out][c_in][3][3] -> [c_out][ldw] in (kh, kw, ic) order (zero-padded)."""
    c_out, c_in = w.shape[:2]
    ldw = (9 * c_in + 7) // 8 * 8
    out = np.zeros((c_out, ldw), np.uint16)
    out[:, :9 * c_in] = w.transpose(0, 2, 3, 1).reshape(c_out, 9 * c_in)
    return out


def perm_co(w):
    """conv_out columns (c, f) -> (f, c)."""
    return np.ascontiguousarray(w.reshape(DM, CC, 16).transpose(0, 2, 1).reshape(DM, CC * 16))


def feo(n):
    """Tokens after the three stride-2 convs, (l - 1) / 2 + 1 three times."""
    for _ in range(3):
        n = (n - 1) // 2 + 1 if n > 0 else 0
    return n


def oracle_tower(orc, dtype, w, mel, n_tok, start="mel", h0=None):
    """The tower from mel chunks [b][NM][CS] (or from the residual stream h0)
    -> (output rows [n_tok][OD], residual stream after the last layer)."""
    if start == "mel":
        b = mel.shape[0]
        x = mel.reshape(b, NM, CS, 1)
        y1 = orc.conv3x3s2(dtype, x, perm_conv(w["conv"][0][0]), w["conv"][0][1])
        y2 = orc.conv3x3s2(dtype, y1.reshape(b, 64, 50, CC), perm_conv(w["conv"][1][0]), w["conv"][1][1])
        y3 = orc.conv3x3s2(dtype, y2.reshape(b, 32, 25, CC), perm_conv(w["conv"][2][0]), w["conv"][2][1],
                           token_major=True).reshape(b * 13, CC * 16)[:n_tok]
        h = orc.linear(dtype, np.ascontiguousarray(y3), perm_co(w["co"][0]),
                       np.zeros((n_tok, DM), np.uint16), bias=w["co"][1])
        h = orc.add_position_table(dtype, h, orc.sinusoid_table(13, DM))
    else:
        h = h0
    for l in w["layers"]:
        x = orc.layer_norm(dtype, h, *l["ln1"], 1e-5)
        qkv = orc.linear(dtype, x, l["qkv"][0], np.zeros((n_tok, 3 * DM), np.uint16), bias=l["qkv"][1])
        a = orc.window_attention(dtype, qkv, NH, 64, WLEN)
        h = orc.linear(dtype, a, l["o"][0], h.copy(), flags=orc.ACCUMULATE, bias=l["o"][1])
        x = orc.layer_norm(dtype, h, *l["ln2"], 1e-5)
        act = orc.linear(dtype, x, l["fc1"][0], np.zeros((n_tok, FFN), np.uint16),
                         flags=orc.EPI_GELU, bias=l["fc1"][1])
        h = orc.linear(dtype, act, l["fc2"][0], h.copy(), flags=orc.ACCUMULATE, bias=l["fc2"][1])
    (lw, lb), (p1w, p1b), (p2w, p2b) = w["post"]
    x = orc.layer_norm(dtype, h, lw, lb, 1e-5)
    pa = orc.linear(dtype, x, p1w, np.zeros((n_tok, DM), np.uint16), flags=orc.EPI_GELU, bias=p1b)
    return orc.linear(dtype, pa, p2w, np.zeros((n_tok, OD), np.uint16), bias=p2b), h


def oracle_dec_layer(orc, dtype, h, w, cos, sin, cap):
    """One decoder layer over the residual stream h [rows][HID]."""
    rows = h.shape[0]
    normed = orc.rms_norm(dtype, h, w["iln"], EPS)
    qkv_w = np.ascontiguousarray(np.concatenate([w["q"], w["k"], w["v"]]))
    qkv = orc.linear(dtype, normed, qkv_w, np.zeros((rows, qkv_w.shape[0]), np.uint16))
    kc = np.zeros((NKVH, cap, HD), np.uint16)
    vc = np.zeros((NKVH, HD, cap), np.uint16)
    q = orc.qk_norm_rope(dtype, qkv, NQH, NKVH, HD, w["qn"], w["kn"], cos, sin, 0, EPS, kc, vc, 0)
    attn = orc.attention(dtype, q, kc, vc, 0)
    h = orc.linear(dtype, attn, w["o"], h.copy(), flags=orc.ACCUMULATE)
    norm2 = orc.rms_norm(dtype, h, w["pln"], EPS)
    gu_w = np.ascontiguousarray(np.concatenate([w["gate"], w["up"]]))
    act = orc.linear(dtype, norm2, gu_w, np.zeros((rows, INTER), np.uint16),
                     flags=orc.EPI_SILU_MUL)
    return orc.linear(dtype, act, w["down"], h, flags=orc.ACCUMULATE)


def oracle_mel_chunks(orc, dtype, x, fb):
    """Log-mel of the samples as the tower's chunks [n_chunks][NM][CS], 16-bit,
    zero past the last valid frame; also the valid frame count."""
    lm = orc.log_mel(x, fb)
    frames = lm.shape[1]
    n_chunks = (frames + CS - 1) // CS
    out = np.zeros((n_chunks, NM, CS), np.float32)
    for c in range(n_chunks):
        seg = lm[:, c * CS:min(frames, (c + 1) * CS)]
        out[c, :, :seg.shape[1]] = seg
    return orc.h16_from_f32(out, dtype), frames


def assemble(n_audio, words):
    """The input sequence (src/align_input.rs:1-20): audio_start, audio_pad x
    n_audio, audio_end, then each word's ids and two timestamp tokens.
    Returns (ids, row sources: id or -1 - audio row, timestamp positions)."""
    ids = [AUDIO_START] + [AUDIO_PAD] * n_audio + [AUDIO_END]
    ts = []
    for word in words:
        ids += list(word)
        ts += [len(ids), len(ids) + 1]
        ids += [TIMESTAMP, TIMESTAMP]
    src = [-1 - (i - 1) if AUDIO_PAD == t else t for i, t in enumerate(ids)]
    return np.array(ids, np.int32), np.array(src, np.int32), np.array(ts, np.int32)


def oracle_aligner(orc, dtype, w, samples, words, fb, rope, log=None):
    """The whole forward on the CPU: samples -> mel chunks -> tower -> rows
    -> decoder layers -> head.  rope(rows) -> (cos, sin).  Returns a dict of
    the intermediate results and the head's logits and classes."""
    say = log or (lambda *a: None)
    mel, frames = oracle_mel_chunks(orc, dtype, samples, fb)
    n_audio = (frames // CS) * 13 + feo(frames % CS)
    say(f"mel: {frames} frames, {mel.shape[0]} chunks, {n_audio} audio tokens")
    audio, _ = oracle_tower(orc, dtype, w["enc"], mel, n_audio)
    say("tower done")
    ids, src, ts = assemble(n_audio, words)
    rows = ids.size
    h = np.where((src >= 0)[:, None], w["embed"][np.maximum(src, 0)], 0).astype(np.uint16)
    h[src < 0] = audio[-1 - src[src < 0]]
    h0 = h.copy()
    cap = (rows + 63) // 64 * 64
    cos, sin = rope(rows)
    for li, lw in enumerate(w["dec"]):
        h = oracle_dec_layer(orc, dtype, h, lw, cos, sin, cap)
        say(f"decoder layer {li} done")
    logits, classes = orc.timestamp_head(dtype, h, ts, w["norm_w"], EPS, w["score"])
    return dict(mel=mel, frames=frames, n_audio=n_audio, audio=audio, ids=ids, src=src, ts=ts,
                h0=h0, h=h, logits=logits, classes=classes)
