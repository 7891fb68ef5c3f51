"""Test helper: writes safetensors files (the format's published layout: an
8-byte little-endian header length, a JSON header of name -> dtype / shape /
data_offsets, then the raw little-endian data) and Qwen3-ForcedAligner-style
checkpoint directories, so the checkpoint loader can be exercised without
the real checkpoint (not available offline)."""
from __future__ import annotations

import json
import os
import struct

import numpy as np


def bf16_bits(x) -> np.ndarray:
    """f32 -> bf16 bits, round to nearest even (finite values)."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def bf16_to_f32(b) -> np.ndarray:
    return (np.asarray(b, np.uint16).astype(np.uint32) << 16).view(np.float32)


def write_safetensors(path: str, tensors: dict, pad_header: bool = True) -> None:
    """tensors: name -> float16 / float32 array, or ("BF16", uint16 bits)."""
    header, blobs, off = {}, [], 0
    for name, t in tensors.items():
        if isinstance(t, tuple):
            dt, arr = t
        else:
            arr = t
            dt = {np.dtype(np.float16): "F16", np.dtype(np.float32): "F32"}[arr.dtype]
        b = np.ascontiguousarray(arr).tobytes()
        header[name] = {"dtype": dt, "shape": list(arr.shape), "data_offsets": [off, off + len(b)]}
        blobs.append(b)
        off += len(b)
    header["__metadata__"] = {"format": "pt"}
    h = json.dumps(header).encode()
    if pad_header:
        h += b" " * ((8 - len(h) % 8) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)))
        f.write(h)
        for b in blobs:
            f.write(b)


HF_PREFIXES = (("thinker.audio_tower.proj1", "model.multi_modal_projector.linear_1"),
               ("thinker.audio_tower.proj2", "model.multi_modal_projector.linear_2"),
               ("thinker.audio_tower.", "model.audio_tower."),
               ("thinker.model.", "model.language_model."),
               ("score.", "thinker.lm_head."))


def hf_name(name: str) -> str:
    """The original name as the `-hf` conversion spells it."""
    for orig, hf in HF_PREFIXES:
        if name.startswith(orig):
            return hf + name[len(orig):]
    return name


def aligner_config(dims: dict, hf: bool) -> dict:
    """config.json in the original (thinker_config) or `-hf` layout."""
    audio = {"d_model": dims["d_model"], "encoder_layers": dims["enc_layers"],
             "encoder_attention_heads": dims["d_model"] // 64, "encoder_ffn_dim": dims["ffn"],
             "num_mel_bins": 128, "downsample_hidden_size": dims["c_conv"], "n_window": 50,
             "n_window_infer": 800, "output_dim": dims["hidden"]}
    text = {"vocab_size": dims["vocab"], "hidden_size": dims["hidden"],
            "intermediate_size": dims["inter"], "num_hidden_layers": dims["layers"],
            "num_attention_heads": dims["nqh"], "num_key_value_heads": dims["nkvh"],
            "head_dim": dims["hd"], "rms_norm_eps": 1e-6, "rope_theta": 1000000.0}
    if hf:
        return {"audio_config": audio, "text_config": text, "timestamp_token_id": 151705,
                "timestamp_segment_time": 80.0,
                "id2label": {str(i): f"LABEL_{i}" for i in range(dims["labels"])}}
    return {"thinker_config": {"audio_config": audio, "text_config": text,
                               "classify_num": dims["labels"]},
            "timestamp_token_id": 151705, "timestamp_segment_time": 80.0}


def write_checkpoint(d: str, tensors: dict, config: dict, hf: bool = False, shards: int = 1) -> None:
    """A checkpoint directory: tensors under their original names (renamed
    to the `-hf` spelling with hf=True), split over `shards` files with an
    index when shards > 1, and config.json."""
    os.makedirs(d, exist_ok=True)
    named = {(hf_name(k) if hf else k): v for k, v in tensors.items()}
    if shards == 1:
        write_safetensors(os.path.join(d, "model.safetensors"), named)
    else:
        keys = sorted(named)
        weight_map = {}
        for s in range(shards):
            fn = f"model-{s + 1:05d}-of-{shards:05d}.safetensors"
            part = {k: named[k] for k in keys[s::shards]}
            write_safetensors(os.path.join(d, fn), part)
            weight_map.update({k: fn for k in part})
        with open(os.path.join(d, "model.safetensors.index.json"), "w") as f:
            json.dump({"metadata": {"total_size": 0}, "weight_map": weight_map}, f)
    with open(os.path.join(d, "config.json"), "w") as f:
        json.dump(config, f)
