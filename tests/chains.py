"""Oracle chains shared by the GPU parity tests and the end-to-end fixture
script: the audio tower, a decoder layer, the log-mel chunking, the input
assembly and the whole aligner forward, each composed from the oracle's ops
(src/audio_encoder.rs:754-832 and src/cpu_decoder.rs:416-512 give the op
order).  The decoder chain has the CPU decoder's rounding points (16 bits
after every op, src/cpu_decoder.rs:416-512).  The tower comes in two forms:
oracle_tower rounds after every op, as the reference's GPU tower stores every
intermediate in the 16-bit format (and as this build's GPU tower does);
oracle_tower_f32 is the reference's CPU tower, f32 throughout with one f16
narrowing of its output (src/audio_encoder.rs:754-832,
src/align_inference.rs:124-131).
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


def oracle_tower_f32(orc, w, mel_f32, n_tok, skip=()):
    """The reference's CPU tower, CpuAudioEncoder::forward
    (src/audio_encoder.rs:754-832): f32 mel chunks [b][NM][CS] in, every
    value f32 (linears with an f32 bias, LayerNorm, GELU, residual adds), the
    output rows [n_tok][OD] narrowed once to f16 (src/align_inference.rs:124-131;
    the CPU path's format is f16 whatever the run's, :103-108).  Weights are
    the f16 checkpoint values widened (CpuWeightF16::to_f32).  `skip` names
    steps to leave out ("position"), for the tests that show the gates catch
    such a mistake."""
    F = lambda bits: orc.h16_to_f32(bits, 0)  # noqa: E731
    b = mel_f32.shape[0]
    x = np.ascontiguousarray(mel_f32, np.float32).reshape(b, NM, CS, 1)
    (c1w, c1b), (c2w, c2b), (c3w, c3b) = w["conv"]
    y1 = orc.conv3x3s2_f32(x, F(perm_conv(c1w)), F(c1b))
    y2 = orc.conv3x3s2_f32(y1.reshape(b, 64, 50, CC), F(perm_conv(c2w)), F(c2b))
    y3 = orc.conv3x3s2_f32(y2.reshape(b, 32, 25, CC), F(perm_conv(c3w)), F(c3b),
                           token_major=True).reshape(b * 13, CC * 16)[:n_tok]
    h = orc.linear_f32(y3, perm_co(w["co"][0]), 0, F(w["co"][1]))
    if "position" not in skip:  # pe[t], t the token's place in its chunk (:331-343)
        h = h + orc.sinusoid_table(13, DM)[np.arange(n_tok) % 13]
    for l in w["layers"]:
        x = orc.layer_norm_f32(h, *l["ln1"], 1e-5)
        qkv = orc.linear_f32(x, l["qkv"][0], 0, F(l["qkv"][1]))
        a = orc.window_attention_f32(qkv[:, :DM], qkv[:, DM:2 * DM], qkv[:, 2 * DM:], NH, 64, WLEN)
        h = h + orc.linear_f32(a, l["o"][0], 0, F(l["o"][1]))
        x = orc.layer_norm_f32(h, *l["ln2"], 1e-5)
        act = orc.gelu_f32(orc.linear_f32(x, l["fc1"][0], 0, F(l["fc1"][1])))
        h = h + orc.linear_f32(act, l["fc2"][0], 0, F(l["fc2"][1]))
    (lw, lb), (p1w, p1b), (p2w, p2b) = w["post"]
    x = orc.layer_norm_f32(h, lw, lb, 1e-5)
    pa = orc.gelu_f32(orc.linear_f32(x, p1w, 0, F(p1b)))
    out = orc.linear_f32(pa, p2w, 0, F(p2b))
    return orc.h16_from_f32(out, 0), h


def oracle_dec_layer(orc, dtype, h, w, cos, sin, cap, zero_attention=False):
    """One decoder layer over the residual stream h [rows][HID]
    (`zero_attention`: the attention output replaced by zeros, a planted
    mistake for the tests of the gates)."""
    rows = h.shape[0]
    normed = orc.rms_norm(dtype, h, w["iln"], EPS)
    qkv_w = np.ascontiguousarray(np.concatenate([w["q"], w["k"], w["v"]]))
    qkv = orc.linear(dtype, normed, qkv_w, np.zeros((rows, qkv_w.shape[0]), np.uint16))
    kc = np.zeros((NKVH, cap, HD), np.uint16)
    vc = np.zeros((NKVH, HD, cap), np.uint16)
    q = orc.qk_norm_rope(dtype, qkv, NQH, NKVH, HD, w["qn"], w["kn"], cos, sin, 0, EPS, kc, vc, 0)
    attn = orc.attention(dtype, q, kc, vc, 0)
    if zero_attention:
        attn = np.zeros_like(attn)
    h = orc.linear(dtype, attn, w["o"], h.copy(), flags=orc.ACCUMULATE)
    norm2 = orc.rms_norm(dtype, h, w["pln"], EPS)
    gu_w = np.ascontiguousarray(np.concatenate([w["gate"], w["up"]]))
    act = orc.linear(dtype, norm2, gu_w, np.zeros((rows, INTER), np.uint16),
                     flags=orc.EPI_SILU_MUL)
    return orc.linear(dtype, act, w["down"], h, flags=orc.ACCUMULATE)


def oracle_mel_chunks(orc, dtype, x, fb, f32=False):
    """Log-mel of the samples as the tower's chunks [n_chunks][NM][CS], 16-bit
    (or f32, the CPU tower's input, with `f32`), zero past the last valid
    frame; also the valid frame count."""
    lm = orc.log_mel(x, fb)
    frames = lm.shape[1]
    n_chunks = (frames + CS - 1) // CS
    out = np.zeros((n_chunks, NM, CS), np.float32)
    for c in range(n_chunks):
        seg = lm[:, c * CS:min(frames, (c + 1) * CS)]
        out[c, :, :seg.shape[1]] = seg
    return (out if f32 else orc.h16_from_f32(out, dtype)), frames


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


def oracle_aligner(orc, dtype, w, samples, words, fb, rope, log=None, tower="16", skip=(),
                   audio=None):
    """The whole forward on the CPU: samples -> mel chunks -> tower -> rows
    -> decoder layers -> head.  rope(rows) -> (cos, sin).  tower = "16": the
    reference GPU tower's rounding points (every op rounded to 16 bits);
    "f32": the reference CPU tower (f32 throughout, one f16 narrowing;
    oracle_tower_f32, f16 runs only).  `audio` reuses tower output rows from
    an earlier call.  `skip` names steps to leave out (tests of the gates:
    "position" in the tower, "attention" = layer 0's attention output zeroed).
    Returns a dict of the intermediate results, the head's logits and classes
    (f64 logits) and the reference head's (f32 GEMM, logits32 / classes32)."""
    say = log or (lambda *a: None)
    mel, frames = oracle_mel_chunks(orc, dtype, samples, fb, f32=tower == "f32")
    n_audio = (frames // CS) * 13 + feo(frames % CS)
    say(f"mel: {frames} frames, {mel.shape[0]} chunks, {n_audio} audio tokens")
    if audio is None:
        if tower == "f32":
            assert dtype == 0, "the CPU tower's output format is f16"
            audio, _ = oracle_tower_f32(orc, w["enc"], mel, n_audio, skip=skip)
        else:
            assert "position" not in skip
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
        h = oracle_dec_layer(orc, dtype, h, lw, cos, sin, cap,
                             zero_attention=li == 0 and "attention" in skip)
        say(f"decoder layer {li} done")
    logits, classes = orc.timestamp_head(dtype, h, ts, w["norm_w"], EPS, w["score"])
    logits32, classes32 = orc.timestamp_head_f32(dtype, h, ts, w["norm_w"], EPS, w["score"])
    return dict(mel=mel, frames=frames, n_audio=n_audio, audio=audio, ids=ids, src=src, ts=ts,
                h0=h0, h=h, logits=logits, classes=classes, logits32=logits32,
                classes32=classes32)


# ---- gates of the end-to-end comparison (shared by the GPU test and the CPU
# tests that show they reject a planted mistake) ----

def rows_gate(orc, dtype, got_bits, want_bits, rel_rms_bound=None, mae_bound=None):
    """Final hidden rows: the north star's MAE (<= 1e-3; 8e-3 for bf16, whose
    ulp is 8x f16's), stated for unit-scale outputs and so scaled by the rows'
    mean magnitude where that exceeds 1 (the rows at the 300 s config's
    <timestamp> slots average |x| ~ 2.7 after 28 layers), and a relative RMS
    difference of at most one 16-bit ulp at 1.0 (2^-10 f16, 2^-7 bf16).  One
    ulp anywhere early in the forward moves every later op's inputs, so two
    correct forwards differ in the last bit of many outputs, but not by more
    than that on average; deeper forwards drift further, and the caller then
    passes bounds derived from two correct oracle forwards (rel_rms_bound,
    mae_bound).  Returns (ok, stats)."""
    g = orc.h16_to_f32(got_bits, dtype).astype(np.float64)
    w = orc.h16_to_f32(want_bits, dtype).astype(np.float64)
    d = g - w
    ulp = 2.0 ** -10 if dtype == 0 else 2.0 ** -7
    scale = max(1.0, float(np.abs(w).mean()))
    st = dict(mae=float(np.abs(d).mean()), rel_rms=float(np.sqrt((d ** 2).mean() / (w ** 2).mean())),
              max_abs=float(np.abs(d).max()), identical=float((got_bits == want_bits).mean()),
              mae_bound=mae_bound or 1e-3 * (1 if dtype == 0 else 8) * scale,
              rel_rms_bound=rel_rms_bound or ulp)
    ok = (np.isfinite(g).all() and st["mae"] <= st["mae_bound"]
          and st["rel_rms"] <= st["rel_rms_bound"])
    return bool(ok), st


def logits_gate(orc, dtype, got_rows, got_logits, want_rows, top_idx, top_logits, norm_w, score):
    """The head's logits at the oracle's 8 best labels of each slot, against
    what the two sets of final rows allow: the folded norm y of a row enters a
    logit as y . score_l, so |L_got - L_want| <= sum_j |y_got_j - y_want_j|
    |score_lj| plus each side's f32 / f64 accumulation error ((2n + 64) and
    (n + 8) f32 ulps of sum |y||score|).  A logit from another row or another
    label, or a head that skipped the norm, falls outside.  Returns (ok,
    largest share of the bound used)."""
    pos = np.arange(got_rows.shape[0])
    yg = orc.head_fold(dtype, got_rows, pos, norm_w, EPS).astype(np.float64)
    yw = orc.head_fold(dtype, want_rows, pos, norm_w, EPS).astype(np.float64)
    n = yg.shape[1]
    s = np.abs(score.astype(np.float64))[top_idx]            # [slots, 8, n]
    bound = (np.einsum("rn,rkn->rk", np.abs(yg - yw), s)
             + (2 * n + 64) * 2.0 ** -24 * np.einsum("rn,rkn->rk", np.abs(yg), s)
             + (n + 8) * 2.0 ** -24 * np.einsum("rn,rkn->rk", np.abs(yw), s))
    got = np.take_along_axis(np.asarray(got_logits, np.float64), top_idx, axis=1)
    use = np.abs(got - top_logits) / bound
    return bool(np.isfinite(got).all() and (use <= 1.0).all()), float(use.max())


def discriminating_head(orc, dtype, rows_bits, norm_w, score, k=4):
    """A score head under which the slots' classes differ: `score` with the k
    leading principal directions of the slots' folded rows (head_fold of
    rows_bits) projected out of every label's row.  At random init those
    directions carry what every <timestamp> row shares (its embedding and
    what the layers make of it), which gives every slot the same class under
    the random head; what is left follows how the slots differ.  It gives the
    class gates something to decide.  f32, like the checkpoint's head."""
    pos = np.arange(rows_bits.shape[0])
    y = orc.head_fold(dtype, rows_bits, pos, norm_w, EPS).astype(np.float64)
    _, _, vt = np.linalg.svd(y, full_matrices=False)
    s = np.asarray(score, np.float64)
    return (s - (s @ vt[:k].T) @ vt[:k]).astype(np.float32)

