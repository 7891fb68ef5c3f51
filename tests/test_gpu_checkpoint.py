"""The aligner built from a checkpoint directory (qah_ckpt_load_aligner,
csrc/host/checkpoint.cpp) against the same model uploaded directly through
the host loaders: on the same input the two forwards must give identical
logits and classes.  The checkpoint is a reduced-size model (2 + 1 layers,
narrow widths, the real vocabulary and token ids) written here with the
original or the `-hf` tensor names, its tensors stored in f16, bf16 and f32
so every narrowing path runs; no real checkpoint is available offline."""
from __future__ import annotations

import numpy as np
import pytest

from ckpt_util import aligner_config, bf16_bits, bf16_to_f32, write_checkpoint

pytestmark = pytest.mark.gpu

F16, BF16 = 0, 1
DIMS = dict(d_model=128, enc_layers=1, ffn=256, c_conv=64, hidden=256, vocab=151936, inter=512,
            layers=2, nqh=2, nkvh=1, hd=128, labels=50)


def _model(seed):
    """Original-name tensors as f32 values, and how each is stored."""
    rng = np.random.default_rng(seed)
    D = DIMS
    dm, ff, cc, hs, hd = D["d_model"], D["ffn"], D["c_conv"], D["hidden"], D["hd"]
    t, store = {}, {}

    def put(name, arr, how):
        t[name] = np.asarray(arr, np.float32)
        store[name] = how

    A, T = "thinker.audio_tower", "thinker.model"
    for lv in range(3):
        cin = 1 if lv == 0 else cc
        put(f"{A}.conv2d{lv + 1}.weight", rng.standard_normal((cc, cin, 3, 3)) / np.sqrt(9 * cin), "bf16")
        put(f"{A}.conv2d{lv + 1}.bias", 0.05 * rng.standard_normal(cc), "f32")
    put(f"{A}.conv_out.weight", rng.standard_normal((dm, cc * 16)) / np.sqrt(cc * 16), "f16")
    for li in range(D["enc_layers"]):
        p = f"{A}.layers.{li}"
        for n in ("q_proj", "k_proj", "v_proj", "out_proj"):
            put(f"{p}.self_attn.{n}.weight", 0.05 * rng.standard_normal((dm, dm)), "f16")
            if n != "k_proj":  # an absent bias reads as zero
                put(f"{p}.self_attn.{n}.bias", 0.01 * rng.standard_normal(dm), "f16")
        for n in ("self_attn_layer_norm", "final_layer_norm"):
            put(f"{p}.{n}.weight", 1 + 0.1 * rng.standard_normal(dm), "f32")
            put(f"{p}.{n}.bias", 0.1 * rng.standard_normal(dm), "f32")
        put(f"{p}.fc1.weight", 0.05 * rng.standard_normal((ff, dm)), "bf16")
        put(f"{p}.fc1.bias", 0.01 * rng.standard_normal(ff), "f16")
        put(f"{p}.fc2.weight", 0.05 * rng.standard_normal((dm, ff)), "f16")
        put(f"{p}.fc2.bias", 0.01 * rng.standard_normal(dm), "f16")
    put(f"{A}.ln_post.weight", 1 + 0.1 * rng.standard_normal(dm), "f32")
    put(f"{A}.ln_post.bias", 0.1 * rng.standard_normal(dm), "f32")
    put(f"{A}.proj1.weight", 0.05 * rng.standard_normal((dm, dm)), "f16")
    put(f"{A}.proj1.bias", 0.01 * rng.standard_normal(dm), "f16")
    put(f"{A}.proj2.weight", 0.05 * rng.standard_normal((hs, dm)), "f32")
    put(f"{A}.proj2.bias", 0.01 * rng.standard_normal(hs), "f16")
    qd, kd, it = D["nqh"] * hd, D["nkvh"] * hd, D["inter"]
    for li in range(D["layers"]):
        p = f"{T}.layers.{li}"
        put(f"{p}.self_attn.q_proj.weight", 0.05 * rng.standard_normal((qd, hs)), "bf16")
        put(f"{p}.self_attn.k_proj.weight", 0.05 * rng.standard_normal((kd, hs)), "f16")
        put(f"{p}.self_attn.v_proj.weight", 0.05 * rng.standard_normal((kd, hs)), "f16")
        put(f"{p}.self_attn.o_proj.weight", 0.05 * rng.standard_normal((hs, qd)), "f16")
        put(f"{p}.mlp.gate_proj.weight", 0.05 * rng.standard_normal((it, hs)), "f16")
        put(f"{p}.mlp.up_proj.weight", 0.05 * rng.standard_normal((it, hs)), "f32")
        put(f"{p}.mlp.down_proj.weight", 0.05 * rng.standard_normal((hs, it)), "f16")
        put(f"{p}.input_layernorm.weight", 1 + 0.1 * rng.standard_normal(hs), "f32")
        put(f"{p}.post_attention_layernorm.weight", 1 + 0.1 * rng.standard_normal(hs), "bf16")
        put(f"{p}.self_attn.q_norm.weight", 1 + 0.1 * rng.standard_normal(hd), "f32")
        put(f"{p}.self_attn.k_norm.weight", 1 + 0.1 * rng.standard_normal(hd), "f32")
    put(f"{T}.embed_tokens.weight", 0.05 * rng.standard_normal((D["vocab"], hs)), "f16")
    put(f"{T}.norm.weight", 1 + 0.1 * rng.standard_normal(hs), "f32")
    put("score.weight", 0.05 * rng.standard_normal((D["labels"], hs)), "f32")
    return t, store


def _stored(arr, how):
    if how == "f16":
        return arr.astype(np.float16)
    if how == "bf16":
        return ("BF16", bf16_bits(arr))
    return arr.astype(np.float32)


def _as_stored_f32(arr, how):
    """The value the file holds, widened to f32."""
    if how == "f16":
        return arr.astype(np.float16).astype(np.float32)
    if how == "bf16":
        return bf16_to_f32(bf16_bits(arr)).reshape(arr.shape)
    return arr.astype(np.float32)


def _direct(pkg, ctx, t, store, max_seconds, max_rows):
    """The same model through the host loaders, converted here: 16-bit
    weights rounded from the stored values, norm weights rounded to f16 and
    widened, the final norm and score in f32."""
    from qwen3_aligner_wgpu_amd import host
    D = DIMS
    v = {k: _as_stored_f32(a, store[k]) for k, a in t.items()}
    h16 = lambda k: v[k].astype(np.float16).view(np.uint16)  # noqa: E731
    n16 = lambda k: v[k].astype(np.float16).astype(np.float32)  # noqa: E731
    zero16 = lambda n: np.zeros(n, np.uint16)  # noqa: E731
    A, T = "thinker.audio_tower", "thinker.model"
    dm = D["d_model"]
    max_samples = int(max_seconds * 16000)
    enc = host.AudioEncoder(ctx, F16, D["enc_layers"], (max_samples // 160 + 99) // 100, 128, 100,
                            D["c_conv"], dm, dm // 64, D["ffn"], D["hidden"], 104)
    dec = host.TextDecoder(ctx, F16, D["layers"], max_rows, D["hidden"], D["nqh"], D["nkvh"],
                           D["hd"], D["inter"], 1e-6)
    for lv in range(3):
        enc.load_conv(lv, h16(f"{A}.conv2d{lv + 1}.weight"), h16(f"{A}.conv2d{lv + 1}.bias"))
    enc.load_conv_out(h16(f"{A}.conv_out.weight"), zero16(dm))
    for li in range(D["enc_layers"]):
        p = f"{A}.layers.{li}.self_attn"
        qkv = np.concatenate([h16(f"{p}.{n}_proj.weight") for n in ("q", "k", "v")])
        qkvb = np.concatenate([h16(f"{p}.q_proj.bias"), zero16(dm), h16(f"{p}.v_proj.bias")])
        q = f"{A}.layers.{li}"
        enc.load_layer(li, n16(f"{q}.self_attn_layer_norm.weight"), n16(f"{q}.self_attn_layer_norm.bias"),
                       qkv, qkvb, h16(f"{p}.out_proj.weight"), h16(f"{p}.out_proj.bias"),
                       n16(f"{q}.final_layer_norm.weight"), n16(f"{q}.final_layer_norm.bias"),
                       h16(f"{q}.fc1.weight"), h16(f"{q}.fc1.bias"), h16(f"{q}.fc2.weight"),
                       h16(f"{q}.fc2.bias"))
    enc.load_post(n16(f"{A}.ln_post.weight"), n16(f"{A}.ln_post.bias"), h16(f"{A}.proj1.weight"),
                  h16(f"{A}.proj1.bias"), h16(f"{A}.proj2.weight"), h16(f"{A}.proj2.bias"))
    for li in range(D["layers"]):
        p = f"{T}.layers.{li}"
        dec.load_layer(li, *[h16(f"{p}.{n}.weight") for n in (
            "self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj", "self_attn.o_proj",
            "mlp.gate_proj", "mlp.up_proj", "mlp.down_proj")],
            *[n16(f"{p}.{n}.weight") for n in ("input_layernorm", "post_attention_layernorm",
                                               "self_attn.q_norm", "self_attn.k_norm")])
    dec.set_rope(*pkg.rope_tables(max_rows, D["hd"], 1e6, F16))
    al = host.Aligner(ctx, enc, dec, D["vocab"], D["labels"], 80.0, max_samples)
    al.load_embed(h16(f"{T}.embed_tokens.weight"))
    al.load_head(v[f"{T}.norm.weight"], v["score.weight"])
    return al, enc, dec


def _forward(al, x, words):
    al.prepare(x, words)
    al.forward()
    raw, fixed = al.result()
    return al.read("logits"), al.read("classes"), raw, fixed


@pytest.mark.parametrize("hf", [False, True], ids=["original_names", "hf_names"])
def test_checkpoint_aligner_matches_direct_upload(tmp_path, pkg, ctx, hf):
    from qwen3_aligner_wgpu_amd import host, synthetic as syn
    t, store = _model(11)
    write_checkpoint(str(tmp_path), {k: _stored(a, store[k]) for k, a in t.items()},
                     aligner_config(DIMS, hf), hf=hf, shards=2 if hf else 1)
    x = syn.synthetic_audio(3.0, 2)
    words = [syn.word_token_ids(w) for w in syn.synthetic_words(6, 2)]
    max_seconds, max_rows = 3.1, 128
    with host.Checkpoint(str(tmp_path)) as ck:
        al, enc, dec = ck.load_aligner(ctx, F16, max_seconds, max_rows)
    try:
        got = _forward(al, x, words)
    finally:
        al.close(), enc.close(), dec.close()
    al, enc, dec = _direct(pkg, ctx, t, store, max_seconds, max_rows)
    try:
        want = _forward(al, x, words)
    finally:
        al.close(), enc.close(), dec.close()
    assert np.isfinite(got[0]).all() and got[0].shape == (12, DIMS["labels"])
    for g, w in zip(got, want):
        assert np.array_equal(g, w)


def test_checkpoint_aligner_rejects_bad_shapes(tmp_path, pkg, ctx):
    from qwen3_aligner_wgpu_amd import host
    t, store = _model(12)
    t["thinker.model.layers.1.mlp.down_proj.weight"] = t["thinker.model.layers.1.mlp.down_proj.weight"][:, :-8]
    write_checkpoint(str(tmp_path), {k: _stored(a, store[k]) for k, a in t.items()},
                     aligner_config(DIMS, False))
    with host.Checkpoint(str(tmp_path)) as ck:
        with pytest.raises(host.CheckpointError, match=r"down_proj.weight: shape \[256, 504\], expected \[256, 512\]"):
            ck.load_aligner(ctx, F16, 3.0, 128)
