"""The real-checkpoint loader (csrc/host/checkpoint.cpp) on the CPU:
safetensors parsing, the `-hf` name remap (src/weights.rs:229-264), sharded
checkpoints through the index, narrowing to f16 / bf16 (round to nearest
even, src/weights.rs:56-88) and config.json in both layouts
(src/config.rs:186-235).  The files are written here (tests/ckpt_util.py);
no real checkpoint is available offline."""
from __future__ import annotations

import json
import os
import struct

import numpy as np
import pytest

F16, BF16 = 0, 1  # QA_F16, QA_BF16 (include/qa.h)

from ckpt_util import (aligner_config, bf16_bits, bf16_to_f32, write_checkpoint,
                       write_safetensors)


@pytest.fixture(scope="module")
def host(pkg):
    from qwen3_aligner_wgpu_amd import host as h
    h.host_lib()
    return h


def _values(rng, n):
    # ordinary values, halfway cases of both 16-bit formats, tiny / huge ones
    v = rng.standard_normal(n).astype(np.float32)
    v[:4] = [1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11, 1.0 + 2.0 ** -8, 1.0 + 3 * 2.0 ** -8]
    v[4:8] = [6e-8, -3e-5, 65000.0, 1e-40]
    return v


def test_narrowing_and_metadata(tmp_path, host, pkg):
    rng = np.random.default_rng(3)
    f32 = _values(rng, 96).reshape(8, 12)
    f16 = rng.standard_normal((5, 3)).astype(np.float16)
    bf = bf16_bits(rng.standard_normal(7))
    write_safetensors(str(tmp_path / "model.safetensors"),
                      {"a.f32": f32, "b.f16": f16, "c.bf16": ("BF16", bf)})
    with host.Checkpoint(str(tmp_path)) as ck:
        assert ck.tensor("a.f32") == ("F32", (8, 12))
        assert ck.tensor("b.f16") == ("F16", (5, 3))
        assert ck.tensor("c.bf16") == ("BF16", (7,))
        # f32 -> f16 / bf16: IEEE round to nearest even / the reference's bf16 rule
        assert np.array_equal(ck.read_h16("a.f32", F16), f32.astype(np.float16).view(np.uint16))
        assert np.array_equal(ck.read_h16("a.f32", BF16), bf16_bits(f32).reshape(8, 12))
        # same format: a copy; the other format: widen (exact) and round again
        assert np.array_equal(ck.read_h16("b.f16", F16), f16.view(np.uint16))
        assert np.array_equal(ck.read_h16("b.f16", BF16), bf16_bits(f16.astype(np.float32)))
        assert np.array_equal(ck.read_h16("c.bf16", BF16), bf)
        assert np.array_equal(ck.read_h16("c.bf16", F16),
                              bf16_to_f32(bf).astype(np.float16).view(np.uint16))
        assert np.array_equal(ck.read_f32("a.f32"), f32)
        assert np.array_equal(ck.read_f32("b.f16"), f16.astype(np.float32))
        assert np.array_equal(ck.read_f32("c.bf16"), bf16_to_f32(bf))
        with pytest.raises(host.CheckpointError, match="weight not found: nope"):
            ck.tensor("nope")


def _small_tensors(rng):
    return {"thinker.model.norm.weight": rng.standard_normal(16).astype(np.float32),
            "thinker.model.layers.0.mlp.up_proj.weight": rng.standard_normal((4, 16)).astype(np.float16),
            "thinker.audio_tower.proj1.weight": rng.standard_normal((8, 8)).astype(np.float16),
            "thinker.audio_tower.proj2.bias": rng.standard_normal(8).astype(np.float32),
            "thinker.audio_tower.conv2d1.weight": rng.standard_normal((8, 1, 3, 3)).astype(np.float16),
            "score.weight": rng.standard_normal((5, 16)).astype(np.float32)}


@pytest.mark.parametrize("hf", [False, True], ids=["original_names", "hf_names"])
@pytest.mark.parametrize("shards", [1, 3])
def test_names_and_shards(tmp_path, host, hf, shards):
    """Both name spellings load under the original names, from one file or
    from shards listed in model.safetensors.index.json."""
    rng = np.random.default_rng(4)
    t = _small_tensors(rng)
    dims = dict(d_model=128, enc_layers=1, ffn=256, c_conv=64, hidden=128, vocab=151936,
                inter=256, layers=1, nqh=2, nkvh=1, hd=64, labels=5)
    write_checkpoint(str(tmp_path), t, aligner_config(dims, hf), hf=hf, shards=shards)
    with host.Checkpoint(str(tmp_path)) as ck:
        for name, arr in t.items():
            assert ck.tensor(name)[1] == arr.shape
            assert np.array_equal(ck.read_f32(name), arr.astype(np.float32))
        if hf:
            with pytest.raises(host.CheckpointError):
                ck.tensor("model.language_model.norm.weight")


@pytest.mark.parametrize("hf", [False, True], ids=["thinker_config", "hf_config"])
def test_config(tmp_path, host, hf):
    dims = dict(d_model=128, enc_layers=2, ffn=256, c_conv=64, hidden=128, vocab=151936,
                inter=384, layers=3, nqh=2, nkvh=1, hd=64, labels=7)
    cfg = aligner_config(dims, hf)
    if hf:  # rope_parameters.rope_theta overrides rope_theta (src/config.rs:205-209)
        cfg["text_config"]["rope_parameters"] = {"rope_theta": 500000.0}
    write_checkpoint(str(tmp_path), {"x": np.zeros(1, np.float32)}, cfg)
    with host.Checkpoint(str(tmp_path)) as ck:
        c = ck.config()
    assert (c["hidden"], c["layers"], c["nqh"], c["nkvh"], c["hd"], c["inter"]) == (128, 3, 2, 1, 64, 384)
    assert (c["d_model"], c["enc_layers"], c["enc_heads"], c["enc_ffn"], c["c_conv"]) == (128, 2, 2, 256, 64)
    assert (c["n_window"], c["n_window_infer"], c["out_dim"], c["num_labels"]) == (50, 800, 128, 7)
    assert (c["timestamp_token_id"], c["audio_start"], c["audio_end"], c["audio_token"]) == \
        (151705, 151669, 151670, 151676)
    assert c["rope_theta"] == (500000.0 if hf else 1e6) and c["segment_ms"] == 80.0
    assert c["rms_eps"] == 1e-6


def test_config_defaults(tmp_path, host):
    """Absent fields take the reference's defaults (src/config.rs:36-150)."""
    write_checkpoint(str(tmp_path), {"x": np.zeros(1, np.float32)},
                     {"audio_config": {}, "text_config": {}, "id2label": {"0": "a", "1": "b"}})
    with host.Checkpoint(str(tmp_path)) as ck:
        c = ck.config()
    assert (c["vocab"], c["hidden"], c["inter"], c["layers"], c["nqh"], c["nkvh"], c["hd"]) == \
        (151936, 1024, 3072, 28, 16, 8, 128)
    assert (c["d_model"], c["enc_layers"], c["enc_heads"], c["enc_ffn"], c["n_mels"], c["c_conv"]) == \
        (896, 18, 14, 3584, 128, 480)
    assert c["num_labels"] == 2 and c["timestamp_token_id"] == -1


def test_errors(tmp_path, host):
    with pytest.raises(host.CheckpointError, match="cannot open"):
        host.Checkpoint(str(tmp_path / "absent"))
    d = tmp_path / "short"
    d.mkdir()
    (d / "model.safetensors").write_bytes(b"\x05\x00")
    with pytest.raises(host.CheckpointError, match="shorter than 8 bytes"):
        host.Checkpoint(str(d))
    d = tmp_path / "hdr"
    d.mkdir()
    (d / "model.safetensors").write_bytes(struct.pack("<Q", 1000) + b"{}")
    with pytest.raises(host.CheckpointError, match="header length"):
        host.Checkpoint(str(d))
    d = tmp_path / "offsets"
    d.mkdir()
    h = json.dumps({"t": {"dtype": "F32", "shape": [4], "data_offsets": [0, 32]}}).encode()
    (d / "model.safetensors").write_bytes(struct.pack("<Q", len(h)) + h + b"\0" * 16)
    with pytest.raises(host.CheckpointError, match="out of range"):
        host.Checkpoint(str(d))
    d = tmp_path / "size"
    d.mkdir()
    h = json.dumps({"t": {"dtype": "F32", "shape": [4], "data_offsets": [0, 12]}}).encode()
    (d / "model.safetensors").write_bytes(struct.pack("<Q", len(h)) + h + b"\0" * 12)
    with pytest.raises(host.CheckpointError, match="bytes for its shape"):
        host.Checkpoint(str(d))
    d = tmp_path / "dup"
    write_checkpoint(str(d), {"a": np.zeros(2, np.float32), "b": np.zeros(2, np.float32)}, {})
    os.remove(d / "model.safetensors")
    write_safetensors(str(d / "s1.safetensors"), {"a": np.zeros(2, np.float32)})
    write_safetensors(str(d / "s2.safetensors"), {"a": np.ones(2, np.float32)})
    (d / "model.safetensors.index.json").write_text(
        json.dumps({"weight_map": {"a": "s1.safetensors", "b": "s2.safetensors"}}))
    with pytest.raises(host.CheckpointError, match="appears twice"):
        host.Checkpoint(str(d))
    d = tmp_path / "ok"
    d.mkdir()
    write_safetensors(str(d / "model.safetensors"), {"t": np.zeros((2, 3), np.float32),
                                                     "i": ("I32", np.zeros(2, np.int32))})
    with host.Checkpoint(str(d)) as ck:
        with pytest.raises(host.CheckpointError, match="6 elements, expected 5"):
            from qwen3_aligner_wgpu_amd import host as hh
            hh._ck(hh.host_lib().qah_ckpt_read_f32(ck.handle, b"t", np.zeros(5, np.float32).ctypes.data, 5))
        with pytest.raises(host.CheckpointError, match="unsupported dtype I32"):
            ck.read_f32("i")
        with pytest.raises(host.CheckpointError, match="config.json missing"):
            ck.config()


def _geometry_dir(tmp_path, hf=False, **audio_text):
    dims = dict(d_model=128, enc_layers=1, ffn=256, c_conv=64, hidden=256, vocab=151936,
                inter=384, layers=1, nqh=2, nkvh=1, hd=128, labels=7)
    cfg = aligner_config(dims, hf)
    a = cfg["audio_config"] if hf else cfg["thinker_config"]["audio_config"]
    t = cfg["text_config"] if hf else cfg["thinker_config"]["text_config"]
    for k, v in audio_text.items():
        (a if k in a else t)[k] = v
    write_checkpoint(str(tmp_path), {"x": np.zeros(1, np.float32)}, cfg, hf=hf)
    return str(tmp_path)


@pytest.mark.parametrize("n_window,n_window_infer,wlen", [(50, 800, 104), (50, 250, 26),
                                                          (30, 400, 48), (40, 250, 30)])
def test_loader_window_geometry(tmp_path, host, n_window, n_window_infer, wlen):
    """The tower's attention window is feo(cs) * (n_window_infer / cs) tokens
    with cs = 2 n_window and an integer division by cs
    (src/audio_encoder.rs:807-810, src/audio_encoder_gpu.rs:883,1103): not
    feo(cs) * n_window_infer / 100, which agrees only at cs = 100."""
    d = _geometry_dir(tmp_path, n_window=n_window, n_window_infer=n_window_infer)
    f = lambda v: (v - 1) // 2 + 1  # noqa: E731
    cs = 2 * n_window
    assert f(f(f(cs))) * (n_window_infer // cs) == wlen
    with host.Checkpoint(d) as ck:
        g = ck.geometry(10.0)
    assert g == dict(cs=cs, wlen=wlen, fdim=16, max_chunks=(10 * 16000 // 160 + cs - 1) // cs)


@pytest.mark.parametrize("field,value,code", [("n_window", 0, -1), ("num_mel_bins", 0, -1),
                                              ("n_window_infer", 60, -1), ("head_dim", 64, -4),
                                              ("num_key_value_heads", 3, -1),
                                              ("num_attention_heads", 8, -4)],
                         ids=["n_window-0", "n_mels-0", "window-below-chunk", "hd-64",
                              "heads-not-multiple", "gqa-4"])
def test_loader_refuses_unsupported_geometry(tmp_path, host, field, value, code):
    """A geometry the kernels cannot run is refused up front with QA_EINVAL
    (-1) or QA_EUNSUPPORTED (-4) and a message, before anything is sized or
    allocated (n_window = 0 would otherwise divide by zero)."""
    d = _geometry_dir(tmp_path, **{field: value})
    with host.Checkpoint(d) as ck:
        with pytest.raises(host.CheckpointError) as e:
            ck.geometry(10.0)
        assert e.value.code == code and e.value.message
