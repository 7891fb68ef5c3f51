"""ctypes view of csrc/libqa_host.so (csrc/host/qa_host.h): the C++ host
mirror of the reference's GEMM call sites, plus the synthetic-input generator.
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import check, host_lib

_vp = ctypes.c_void_p
_i = ctypes.c_int
_u64 = ctypes.c_uint64
_sz = ctypes.c_size_t
_dp = ctypes.POINTER(ctypes.c_double)


def declare(L: ctypes.CDLL) -> None:
    L.qah_synth_normal_h16.argtypes = [_u64, _u64, ctypes.c_float, ctypes.c_float, _i, _vp, _sz]
    L.qah_synth_normal_h16.restype = None
    L.qah_synth_normal_f32.argtypes = [_u64, _u64, ctypes.c_float, ctypes.c_float, _vp, _sz]
    L.qah_synth_normal_f32.restype = None
    L.qah_narrow_f32.argtypes = [_vp, _vp, _sz, _i]
    L.qah_narrow_f32.restype = None
    L.qah_concat_rows.argtypes = [ctypes.POINTER(_vp), ctypes.POINTER(ctypes.c_int64), _i,
                                  ctypes.c_int64, _vp]
    L.qah_concat_rows.restype = None
    L.qah_decoder_create.argtypes = [_vp, _i, _i, _i, _i, _i, _i, _i, ctypes.POINTER(_vp)]
    L.qah_decoder_load_layer.argtypes = [_vp, _i] + [_vp] * 7
    L.qah_decoder_set_inputs.argtypes = [_vp, _i, _vp, _vp, _vp, _vp]
    L.qah_decoder_prefill_linears.argtypes = [_vp, _i]
    L.qah_decoder_layer.argtypes = [_vp, _i, _i]
    L.qah_decoder_read.argtypes = [_vp, _i, _i, _vp]
    L.qah_decoder_time.argtypes = [_vp, _i, _i, _i, _i, _dp, _dp]
    L.qah_decoder_profile_sites.argtypes = [_vp, _i, _i, _dp]
    L.qah_decoder_destroy.argtypes = [_vp]
    L.qah_decoder_destroy.restype = None
    L.qah_encoder_create.argtypes = [_vp, _i, _i, _i, _i, _i, _i, ctypes.POINTER(_vp)]
    L.qah_encoder_load_layer.argtypes = [_vp, _i] + [_vp] * 8
    L.qah_encoder_load_conv.argtypes = [_vp, _vp, _vp]
    L.qah_encoder_set_inputs.argtypes = [_vp, _i, _vp, _vp, _vp, _vp, _vp]
    L.qah_encoder_forward_linears.argtypes = [_vp, _i]
    L.qah_encoder_read.argtypes = [_vp, _i, _i, _vp]
    L.qah_encoder_time.argtypes = [_vp, _i, _i, _i, _i, _dp, _dp]
    L.qah_encoder_profile_sites.argtypes = [_vp, _i, _i, _dp]
    L.qah_encoder_destroy.argtypes = [_vp]
    L.qah_encoder_destroy.restype = None
    _fp = ctypes.POINTER(ctypes.c_float)
    L.qah_tdec_create.argtypes = [_vp] + [_i] * 8 + [ctypes.c_float, ctypes.POINTER(_vp)]
    L.qah_tdec_load_layer.argtypes = [_vp, _i] + [_vp] * 11
    L.qah_tdec_set_rope.argtypes = [_vp, _vp, _vp, _i]
    L.qah_tdec_set_attention_flags.argtypes = [_vp, ctypes.c_uint32]
    L.qah_tdec_set_hidden.argtypes = [_vp, _i, _vp]
    L.qah_tdec_prefill.argtypes = [_vp, _i]
    L.qah_tdec_read.argtypes = [_vp, _i, _i, _vp]
    L.qah_tdec_time.argtypes = [_vp, _i, _i, _i, _i, _dp, _dp]
    L.qah_tdec_profile_ops.argtypes = [_vp, _i, _i, _dp]
    L.qah_tdec_destroy.argtypes = [_vp]
    L.qah_tdec_destroy.restype = None
    L.qah_aenc_create.argtypes = [_vp] + [_i] * 11 + [ctypes.POINTER(_vp)]
    L.qah_aenc_load_conv.argtypes = [_vp, _i, _vp, _vp]
    L.qah_aenc_load_conv_out.argtypes = [_vp, _vp, _vp]
    L.qah_aenc_load_layer.argtypes = [_vp, _i] + [_vp] * 12
    L.qah_aenc_load_post.argtypes = [_vp] + [_vp] * 6
    L.qah_aenc_set_mel.argtypes = [_vp, _i, _vp]
    L.qah_aenc_tokens.argtypes = [_vp, _i, _i]
    L.qah_aenc_tokens.restype = ctypes.c_int64
    L.qah_aenc_forward.argtypes = [_vp, _i, _i]
    L.qah_aenc_read.argtypes = [_vp, _i, ctypes.c_int64, _vp]
    L.qah_aenc_time.argtypes = [_vp, _i, _i, _i, _i, _i, _dp, _dp]
    L.qah_aenc_profile.argtypes = [_vp, _i, _i, _i, _dp]
    L.qah_aenc_destroy.argtypes = [_vp]
    L.qah_aenc_destroy.restype = None
    del _fp
    L.qah_fix_timestamps.argtypes = [_vp, ctypes.c_int64, _vp]
    L.qah_fix_timestamps.restype = None
    L.qah_aligner_create.argtypes = [_vp, _vp, _vp, ctypes.c_int64, ctypes.c_int64,
                                     ctypes.c_double, ctypes.c_int64, ctypes.POINTER(_vp)]
    L.qah_aligner_load_embed.argtypes = [_vp, _vp]
    L.qah_aligner_load_head.argtypes = [_vp, _vp, _vp]
    L.qah_aligner_prepare.argtypes = [_vp, _vp, ctypes.c_int64, _i, _vp, _vp, _vp]
    L.qah_aligner_forward.argtypes = [_vp]
    L.qah_aligner_result.argtypes = [_vp, _vp, _vp]
    L.qah_aligner_read.argtypes = [_vp, _i, _vp]
    L.qah_aligner_time.argtypes = [_vp, _i, _i, _i, _dp, _dp]
    L.qah_aligner_profile.argtypes = [_vp, _i, _dp]
    L.qah_aligner_destroy.argtypes = [_vp]
    L.qah_aligner_destroy.restype = None
    L.qah_time_linear.argtypes = [_vp, _vp, _i, _i, _dp]
    L.qah_copy_calibration.argtypes = [_vp, _sz, _i]
    L.qah_time_linears_each.argtypes = [_vp, _vp, _i, _i, _i, _vp]
    L.qah_time_linears_stamped.argtypes = [_vp, _vp, _i, _i, _i, _vp]
    L.qah_check_silu_f16x2.argtypes = [_vp, ctypes.c_int64, ctypes.c_uint64, _vp]
    for name in ("qah_decoder_create", "qah_decoder_load_layer", "qah_decoder_set_inputs",
                 "qah_decoder_prefill_linears", "qah_decoder_read", "qah_decoder_time",
                 "qah_decoder_profile_sites", "qah_encoder_create", "qah_encoder_load_layer",
                 "qah_encoder_load_conv", "qah_encoder_set_inputs", "qah_encoder_forward_linears",
                 "qah_encoder_read", "qah_encoder_time", "qah_encoder_profile_sites",
                 "qah_time_linear", "qah_copy_calibration", "qah_tdec_create",
                 "qah_tdec_load_layer", "qah_tdec_set_rope", "qah_tdec_set_attention_flags",
                 "qah_tdec_set_hidden", "qah_tdec_prefill", "qah_tdec_read", "qah_tdec_time",
                 "qah_tdec_profile_ops", "qah_aenc_create", "qah_aenc_load_conv",
                 "qah_aenc_load_conv_out", "qah_aenc_load_layer", "qah_aenc_load_post",
                 "qah_aenc_set_mel", "qah_aenc_forward", "qah_aenc_read", "qah_aenc_time",
                 "qah_aenc_profile"):
        getattr(L, name).restype = _i
    L.qah_ckpt_open.argtypes = [ctypes.c_char_p, ctypes.POINTER(_vp)]
    L.qah_ckpt_error.argtypes = []
    L.qah_ckpt_error.restype = ctypes.c_char_p
    L.qah_ckpt_tensor.argtypes = [_vp, ctypes.c_char_p, ctypes.POINTER(_i), ctypes.POINTER(_i),
                                  ctypes.POINTER(ctypes.c_int64)]
    L.qah_ckpt_read_h16.argtypes = [_vp, ctypes.c_char_p, _i, _vp, ctypes.c_int64]
    L.qah_ckpt_read_f32.argtypes = [_vp, ctypes.c_char_p, _vp, ctypes.c_int64]
    L.qah_ckpt_read_config.argtypes = [_vp, ctypes.POINTER(CkptConfig)]
    L.qah_ckpt_load_aligner.argtypes = [_vp, _vp, _i, ctypes.c_double, _i] + [ctypes.POINTER(_vp)] * 3
    L.qah_ckpt_geometry.argtypes = [_vp, ctypes.c_double, _vp]
    L.qah_ckpt_close.argtypes = [_vp]
    L.qah_ckpt_close.restype = None
    for name in ("qah_ckpt_open", "qah_ckpt_tensor", "qah_ckpt_read_h16", "qah_ckpt_read_f32",
                 "qah_ckpt_read_config", "qah_ckpt_load_aligner"):
        getattr(L, name).restype = _i


def _p(a):
    return None if a is None else a.ctypes.data


class CkptConfig(ctypes.Structure):
    """qah_ckpt_config (csrc/host/qa_host.h)."""

    _fields_ = ([(n, ctypes.c_int64) for n in ("vocab", "hidden", "inter", "layers", "nqh", "nkvh", "hd")]
                + [("rms_eps", ctypes.c_double), ("rope_theta", ctypes.c_double)]
                + [(n, ctypes.c_int64) for n in ("d_model", "enc_layers", "enc_heads", "enc_ffn",
                                                 "n_mels", "c_conv", "n_window", "n_window_infer",
                                                 "out_dim", "num_labels", "timestamp_token_id",
                                                 "audio_start", "audio_end", "audio_token")]
                + [("segment_ms", ctypes.c_double)])


class CheckpointError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(f"{message} (code {code})")
        self.code, self.message = code, message


def _ck(rc: int) -> None:
    if rc != 0:
        raise CheckpointError(rc, host_lib().qah_ckpt_error().decode())


class Checkpoint:
    """qah_ckpt: a Qwen3-ForcedAligner checkpoint directory -- safetensors
    shards mapped read-only, `-hf` names mapped onto the original ones
    (src/weights.rs:207-290) -- and the aligner built from it."""

    DTYPES = {0: "F16", 1: "BF16", 2: "F32", 3: "other"}

    def __init__(self, path: str):
        h = _vp()
        _ck(host_lib().qah_ckpt_open(str(path).encode(), ctypes.byref(h)))
        self.handle = h.value

    def close(self):
        if self.handle:
            host_lib().qah_ckpt_close(self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def tensor(self, name: str):
        """(dtype name, shape) of a tensor."""
        dt, nd, shape = _i(), _i(), (ctypes.c_int64 * 8)()
        _ck(host_lib().qah_ckpt_tensor(self.handle, name.encode(), ctypes.byref(dt),
                                       ctypes.byref(nd), shape))
        return self.DTYPES[dt.value], tuple(shape[i] for i in range(nd.value))

    def read_h16(self, name: str, dtype: int) -> np.ndarray:
        """The tensor in QA_F16 / QA_BF16 bits, in its own shape."""
        _, shape = self.tensor(name)
        out = np.empty(shape, np.uint16)
        _ck(host_lib().qah_ckpt_read_h16(self.handle, name.encode(), dtype, _p(out), out.size))
        return out

    def read_f32(self, name: str) -> np.ndarray:
        _, shape = self.tensor(name)
        out = np.empty(shape, np.float32)
        _ck(host_lib().qah_ckpt_read_f32(self.handle, name.encode(), _p(out), out.size))
        return out

    def config(self) -> dict:
        c = CkptConfig()
        _ck(host_lib().qah_ckpt_read_config(self.handle, ctypes.byref(c)))
        return {n: getattr(c, n) for n, _ in CkptConfig._fields_}

    def geometry(self, max_seconds: float) -> dict:
        """qah_ckpt_geometry: the tower geometry the loader uses."""
        out = (ctypes.c_int64 * 4)()
        _ck(host_lib().qah_ckpt_geometry(self.handle, max_seconds, out))
        return dict(zip(("cs", "wlen", "fdim", "max_chunks"), list(out)))

    def load_aligner(self, ctx, dtype: int, max_seconds: float, max_rows: int):
        """(Aligner, AudioEncoder, TextDecoder) loaded from the checkpoint;
        close the aligner before the other two."""
        c = self.config()
        geo = self.geometry(max_seconds)
        e, d, a = _vp(), _vp(), _vp()
        _ck(host_lib().qah_ckpt_load_aligner(self.handle, ctx.handle, dtype, max_seconds, max_rows,
                                             ctypes.byref(e), ctypes.byref(d), ctypes.byref(a)))
        f = lambda v: (v - 1) // 2 + 1  # noqa: E731
        cs = geo["cs"]
        enc = AudioEncoder.__new__(AudioEncoder)
        enc.ctx, enc.dtype, enc.layers = ctx, dtype, c["enc_layers"]
        enc.max_chunks = geo["max_chunks"]
        enc.n_mels, enc.cs, enc.c_conv, enc.d_model = c["n_mels"], cs, c["c_conv"], c["d_model"]
        enc.nh, enc.ffn, enc.out_dim = c["enc_heads"], c["enc_ffn"], c["out_dim"]
        enc.wlen = geo["wlen"]
        enc.h3, enc.w3 = geo["fdim"], f(f(f(cs)))
        enc.handle = e.value
        dec = TextDecoder.__new__(TextDecoder)
        dec.ctx, dec.dtype, dec.layers, dec.max_rows = ctx, dtype, c["layers"], max_rows
        dec.hidden, dec.nqh, dec.nkvh, dec.hd, dec.inter = (c["hidden"], c["nqh"], c["nkvh"],
                                                            c["hd"], c["inter"])
        dec.handle = d.value
        al = Aligner.__new__(Aligner)
        al.ctx, al.enc, al.dec, al.vocab, al.labels = ctx, enc, dec, c["vocab"], c["num_labels"]
        al.handle, al.info = a.value, None
        return al, enc, dec


def synth_normal(seed: int, tensor_id: int, shape, mean: float = 0.0, std: float = 1.0,
                 dtype: int = 0) -> np.ndarray:
    """Seeded N(mean, std^2) values as 16-bit bits (SplitMix64 + Box-Muller)."""
    out = np.empty(shape, np.uint16)
    host_lib().qah_synth_normal_h16(seed, tensor_id, mean, std, dtype, out.ctypes.data, out.size)
    return out


def synth_normal_f32(seed: int, tensor_id: int, shape, mean: float = 0.0,
                     std: float = 1.0) -> np.ndarray:
    out = np.empty(shape, np.float32)
    host_lib().qah_synth_normal_f32(seed, tensor_id, mean, std, out.ctypes.data, out.size)
    return out


def narrow(x: np.ndarray, dtype: int) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    host_lib().qah_narrow_f32(x.ctypes.data, out.ctypes.data, x.size, dtype)
    return out


def concat_rows(parts) -> np.ndarray:
    parts = [np.ascontiguousarray(p, np.uint16) for p in parts]
    cols = parts[0].shape[1]
    assert all(p.shape[1] == cols for p in parts)
    out = np.empty((sum(p.shape[0] for p in parts), cols), np.uint16)
    ptrs = (_vp * len(parts))(*[p.ctypes.data for p in parts])
    rows = (ctypes.c_int64 * len(parts))(*[p.shape[0] for p in parts])
    host_lib().qah_concat_rows(ptrs, rows, len(parts), cols, out.ctypes.data)
    return out


class DecoderLinears:
    """qah_decoder: the text decoder's per-layer projections."""

    def __init__(self, ctx, dtype: int, layers: int, max_rows: int, hidden: int = 1024,
                 q_dim: int = 2048, kv_dim: int = 1024, inter: int = 3072):
        self.ctx, self.dtype, self.layers, self.max_rows = ctx, dtype, layers, max_rows
        self.hidden, self.q_dim, self.kv_dim, self.inter = hidden, q_dim, kv_dim, inter
        h = _vp()
        check(host_lib().qah_decoder_create(ctx.handle, dtype, layers, hidden, q_dim, kv_dim,
                                            inter, max_rows, ctypes.byref(h)))
        self.handle = h.value

    def close(self):
        if self.handle:
            host_lib().qah_decoder_destroy(self.handle)
            self.handle = None

    def load_layer(self, li, q, k, v, o, gate, up, down):
        arrs = [np.ascontiguousarray(a, np.uint16) for a in (q, k, v, o, gate, up, down)]
        check(host_lib().qah_decoder_load_layer(self.handle, li, *[_p(a) for a in arrs]))

    def set_inputs(self, rows, normed=None, attn=None, norm2=None, h=None):
        check(host_lib().qah_decoder_set_inputs(self.handle, rows, _p(normed), _p(attn),
                                                _p(norm2), _p(h)))

    def prefill_linears(self, rows):
        check(host_lib().qah_decoder_prefill_linears(self.handle, rows))

    def layer(self, li, rows):
        """One layer's four projections (as prefill_linears runs them)."""
        check(host_lib().qah_decoder_layer(self.handle, li, rows))

    def read(self, which: str, rows: int) -> np.ndarray:
        idx, cols = {"h": (0, self.hidden), "qkv": (1, self.q_dim + 2 * self.kv_dim),
                     "act": (2, self.inter)}[which]
        out = np.empty((rows, cols), np.uint16)
        check(host_lib().qah_decoder_read(self.handle, idx, rows, out.ctypes.data))
        return out

    def time(self, rows, warmup, steps, use_graph=True) -> tuple[float, float]:
        """(event ms per step, host wall-clock ms per step)."""
        ms, wall = ctypes.c_double(), ctypes.c_double()
        check(host_lib().qah_decoder_time(self.handle, rows, warmup, steps, int(use_graph),
                                          ctypes.byref(ms), ctypes.byref(wall)))
        return ms.value, wall.value

    def profile_sites(self, rows, steps) -> dict:
        out = (ctypes.c_double * 4)()
        check(host_lib().qah_decoder_profile_sites(self.handle, rows, steps, out))
        return dict(zip(("qkv", "o", "gu", "down"), list(out)))


class EncoderLinears:
    """qah_encoder: the audio tower's linears + the conv block GEMM."""

    def __init__(self, ctx, dtype: int, layers: int, max_rows: int, d_model: int = 896,
                 ffn: int = 3584, conv_k: int = 1152):
        self.ctx, self.dtype, self.layers, self.max_rows = ctx, dtype, layers, max_rows
        self.d_model, self.ffn, self.conv_k = d_model, ffn, conv_k
        h = _vp()
        check(host_lib().qah_encoder_create(ctx.handle, dtype, layers, d_model, ffn, conv_k,
                                            max_rows, ctypes.byref(h)))
        self.handle = h.value

    def close(self):
        if self.handle:
            host_lib().qah_encoder_destroy(self.handle)
            self.handle = None

    def load_layer(self, li, qkv_w, qkv_b, o_w, o_b, fc1_w, fc1_b, fc2_w, fc2_b):
        arrs = [np.ascontiguousarray(a, np.uint16)
                for a in (qkv_w, qkv_b, o_w, o_b, fc1_w, fc1_b, fc2_w, fc2_b)]
        check(host_lib().qah_encoder_load_layer(self.handle, li, *[_p(a) for a in arrs]))

    def load_conv(self, w, b):
        w = np.ascontiguousarray(w, np.uint16)
        b = np.ascontiguousarray(b, np.uint16)
        check(host_lib().qah_encoder_load_conv(self.handle, _p(w), _p(b)))

    def set_inputs(self, rows, col=None, normed=None, attn=None, norm2=None, h=None):
        check(host_lib().qah_encoder_set_inputs(self.handle, rows, _p(col), _p(normed),
                                                _p(attn), _p(norm2), _p(h)))

    def forward_linears(self, rows):
        check(host_lib().qah_encoder_forward_linears(self.handle, rows))

    def read(self, which: str, rows: int) -> np.ndarray:
        idx, cols = {"h": (0, self.d_model), "conv": (1, self.d_model),
                     "qkv": (2, 3 * self.d_model), "act": (3, self.ffn)}[which]
        out = np.empty((rows, cols), np.uint16)
        check(host_lib().qah_encoder_read(self.handle, idx, rows, out.ctypes.data))
        return out

    def time(self, rows, warmup, steps, use_graph=True) -> tuple[float, float]:
        """(event ms per step, host wall-clock ms per step)."""
        ms, wall = ctypes.c_double(), ctypes.c_double()
        check(host_lib().qah_encoder_time(self.handle, rows, warmup, steps, int(use_graph),
                                          ctypes.byref(ms), ctypes.byref(wall)))
        return ms.value, wall.value

    def profile_sites(self, rows, steps) -> dict:
        out = (ctypes.c_double * 5)()
        check(host_lib().qah_encoder_profile_sites(self.handle, rows, steps, out))
        return dict(zip(("conv", "qkv", "o", "fc1", "fc2"), list(out)))


class TextDecoder:
    """qah_tdec: whole Qwen3 decoder layers (norms, qkv, RoPE + KV write,
    attention, o, gate|up + SiLU, down), WgpuTextDecoder::prefill's loop."""

    OPS = ("rms_norm", "qkv", "qk_norm_rope", "attention", "o", "rms_norm2", "gu", "down")

    def __init__(self, ctx, dtype: int, layers: int, max_rows: int, hidden: int = 1024,
                 nqh: int = 16, nkvh: int = 8, hd: int = 128, inter: int = 3072,
                 eps: float = 1e-6):
        self.ctx, self.dtype, self.layers, self.max_rows = ctx, dtype, layers, max_rows
        self.hidden, self.nqh, self.nkvh, self.hd, self.inter = hidden, nqh, nkvh, hd, inter
        h = _vp()
        check(host_lib().qah_tdec_create(ctx.handle, dtype, layers, hidden, nqh, nkvh, hd, inter,
                                         max_rows, eps, ctypes.byref(h)))
        self.handle = h.value

    def close(self):
        if self.handle:
            host_lib().qah_tdec_destroy(self.handle)
            self.handle = None

    def load_layer(self, li, q, k, v, o, gate, up, down, iln, pln, qn, kn):
        w16 = [np.ascontiguousarray(a, np.uint16) for a in (q, k, v, o, gate, up, down)]
        w32 = [np.ascontiguousarray(a, np.float32) for a in (iln, pln, qn, kn)]
        check(host_lib().qah_tdec_load_layer(self.handle, li, *[_p(a) for a in w16 + w32]))

    def set_rope(self, cos, sin):
        cos = np.ascontiguousarray(cos, np.float32)
        sin = np.ascontiguousarray(sin, np.float32)
        assert cos.shape == sin.shape and cos.shape[1] == self.hd
        check(host_lib().qah_tdec_set_rope(self.handle, _p(cos), _p(sin), cos.shape[0]))

    def set_attention_flags(self, flags: int):
        check(host_lib().qah_tdec_set_attention_flags(self.handle, flags))

    def set_hidden(self, h):
        h = np.ascontiguousarray(h, np.uint16)
        check(host_lib().qah_tdec_set_hidden(self.handle, h.shape[0], _p(h)))

    def prefill(self, rows):
        check(host_lib().qah_tdec_prefill(self.handle, rows))

    @property
    def cap(self) -> int:
        return (self.max_rows + 63) // 64 * 64

    def read(self, which: str, rows: int) -> np.ndarray:
        qd, kvd = self.nqh * self.hd, self.nkvh * self.hd
        idx, shape = {"h": (0, (rows, self.hidden)), "attn": (1, (rows, qd)),
                      "qkv": (2, (rows, qd + 2 * kvd)), "act": (3, (rows, self.inter)),
                      "normed": (4, (rows, self.hidden)), "norm2": (5, (rows, self.hidden)),
                      "q": (6, (self.nqh, rows, self.hd)),
                      "k_cache": (7, (self.nkvh, self.cap, self.hd)),
                      "v_cache": (8, (self.nkvh, self.hd, self.cap))}[which]
        out = np.empty(shape, np.uint16)
        check(host_lib().qah_tdec_read(self.handle, idx, rows, out.ctypes.data))
        return out

    def time(self, rows, warmup, steps, use_graph=True) -> tuple[float, float]:
        """(event ms per step, host wall-clock ms per step)."""
        ms, wall = ctypes.c_double(), ctypes.c_double()
        check(host_lib().qah_tdec_time(self.handle, rows, warmup, steps, int(use_graph),
                                       ctypes.byref(ms), ctypes.byref(wall)))
        return ms.value, wall.value

    def profile_ops(self, rows, steps) -> dict:
        out = (ctypes.c_double * 8)()
        check(host_lib().qah_tdec_profile_ops(self.handle, rows, steps, out))
        return dict(zip(self.OPS, list(out)))


class AudioEncoder:
    """qah_aenc: the whole audio tower (conv stem, conv_out + position add,
    windowed-attention layers, projector), GpuAudioEncoder::encode."""

    READS = {"out": 0, "h": 1, "conv1": 2, "conv2": 3, "conv3": 4, "normed": 5, "qkv": 6,
             "attn": 7, "act": 8, "pact": 9}
    PROFILE = ("conv1", "conv2", "conv3", "conv_out_pe", "ln1", "qkv", "attention", "o", "ln2",
               "fc1", "fc2", "post")

    def __init__(self, ctx, dtype: int, layers: int, max_chunks: int, n_mels: int = 128,
                 cs: int = 100, c_conv: int = 480, d_model: int = 896, nh: int = 14,
                 ffn: int = 3584, out_dim: int = 1024, wlen: int = 104):
        self.ctx, self.dtype, self.layers, self.max_chunks = ctx, dtype, layers, max_chunks
        self.n_mels, self.cs, self.c_conv, self.d_model = n_mels, cs, c_conv, d_model
        self.nh, self.ffn, self.out_dim, self.wlen = nh, ffn, out_dim, wlen
        f = lambda v: (v - 1) // 2 + 1  # noqa: E731
        self.h3, self.w3 = f(f(f(n_mels))), f(f(f(cs)))
        h = _vp()
        check(host_lib().qah_aenc_create(ctx.handle, dtype, layers, n_mels, cs, c_conv, d_model,
                                         nh, ffn, out_dim, wlen, max_chunks, ctypes.byref(h)))
        self.handle = h.value

    def close(self):
        if self.handle:
            host_lib().qah_aenc_destroy(self.handle)
            self.handle = None

    @staticmethod
    def _u16(*arrs):
        return [np.ascontiguousarray(a, np.uint16) for a in arrs]

    @staticmethod
    def _f32(*arrs):
        return [np.ascontiguousarray(a, np.float32) for a in arrs]

    def load_conv(self, level, w, b):
        w, b = self._u16(w, b)
        check(host_lib().qah_aenc_load_conv(self.handle, level, _p(w), _p(b)))

    def load_conv_out(self, w, b):
        w, b = self._u16(w, b)
        check(host_lib().qah_aenc_load_conv_out(self.handle, _p(w), _p(b)))

    def load_layer(self, li, ln1_w, ln1_b, qkv_w, qkv_b, o_w, o_b, ln2_w, ln2_b, fc1_w, fc1_b,
                   fc2_w, fc2_b):
        l1w, l1b, l2w, l2b = self._f32(ln1_w, ln1_b, ln2_w, ln2_b)
        ws = self._u16(qkv_w, qkv_b, o_w, o_b, fc1_w, fc1_b, fc2_w, fc2_b)
        check(host_lib().qah_aenc_load_layer(self.handle, li, _p(l1w), _p(l1b), _p(ws[0]),
                                             _p(ws[1]), _p(ws[2]), _p(ws[3]), _p(l2w), _p(l2b),
                                             _p(ws[4]), _p(ws[5]), _p(ws[6]), _p(ws[7])))

    def load_post(self, ln_w, ln_b, p1_w, p1_b, p2_w, p2_b):
        lw, lb = self._f32(ln_w, ln_b)
        ws = self._u16(p1_w, p1_b, p2_w, p2_b)
        check(host_lib().qah_aenc_load_post(self.handle, _p(lw), _p(lb), *[_p(a) for a in ws]))

    def set_mel(self, mel):
        mel = np.ascontiguousarray(mel, np.uint16)
        check(host_lib().qah_aenc_set_mel(self.handle, mel.shape[0], _p(mel)))

    def tokens(self, n_chunks, tail_frames=0) -> int:
        return int(host_lib().qah_aenc_tokens(self.handle, n_chunks, tail_frames))

    def forward(self, n_chunks, tail_frames=0):
        check(host_lib().qah_aenc_forward(self.handle, n_chunks, tail_frames))

    def read(self, which: str, rows: int) -> np.ndarray:
        cols = {"out": self.out_dim, "h": self.d_model, "conv1": self.c_conv,
                "conv2": self.c_conv, "conv3": self.c_conv * self.h3, "normed": self.d_model,
                "qkv": 3 * self.d_model, "attn": self.d_model, "act": self.ffn,
                "pact": self.d_model}[which]
        out = np.empty((rows, cols), np.uint16)
        check(host_lib().qah_aenc_read(self.handle, self.READS[which], rows, out.ctypes.data))
        return out

    def time(self, n_chunks, tail_frames, warmup, steps, use_graph=True) -> tuple[float, float]:
        ms, wall = ctypes.c_double(), ctypes.c_double()
        check(host_lib().qah_aenc_time(self.handle, n_chunks, tail_frames, warmup, steps,
                                       int(use_graph), ctypes.byref(ms), ctypes.byref(wall)))
        return ms.value, wall.value

    def profile(self, n_chunks, tail_frames, steps) -> dict:
        out = (ctypes.c_double * 12)()
        check(host_lib().qah_aenc_profile(self.handle, n_chunks, tail_frames, steps, out))
        return dict(zip(self.PROFILE, list(out)))


def fix_timestamps(data) -> np.ndarray:
    """qah_fix_timestamps: the timestamp repair (src/postprocess.rs:33-111)."""
    data = np.ascontiguousarray(data, np.int64)
    out = np.empty_like(data)
    host_lib().qah_fix_timestamps(_p(data), data.size, _p(out))
    return out


class Aligner:
    """qah_aligner: the aligner's forward pass over an AudioEncoder and a
    TextDecoder (Aligner::align_raw_rows, src/align_inference.rs:646-805)."""

    PHASES = ("mel", "tower", "scatter", "prefill", "head")

    def __init__(self, ctx, enc: AudioEncoder, dec: TextDecoder, vocab: int = 151936,
                 labels: int = 5000, segment_ms: float = 80.0, max_samples: int = 300 * 16000):
        self.ctx, self.enc, self.dec, self.vocab, self.labels = ctx, enc, dec, vocab, labels
        h = _vp()
        check(host_lib().qah_aligner_create(ctx.handle, enc.handle, dec.handle, vocab, labels,
                                            segment_ms, max_samples, ctypes.byref(h)))
        self.handle = h.value
        self.info = None

    def close(self):
        if self.handle:
            host_lib().qah_aligner_destroy(self.handle)
            self.handle = None

    def load_embed(self, table):
        table = np.ascontiguousarray(table, np.uint16)
        assert table.shape == (self.vocab, self.dec.hidden)
        check(host_lib().qah_aligner_load_embed(self.handle, _p(table)))

    def load_head(self, norm_w, score):
        norm_w = np.ascontiguousarray(norm_w, np.float32)
        score = np.ascontiguousarray(score, np.float32)
        assert norm_w.shape == (self.dec.hidden,) and score.shape == (self.labels, self.dec.hidden)
        check(host_lib().qah_aligner_load_head(self.handle, _p(norm_w), _p(score)))

    def prepare(self, samples, words) -> dict:
        """words: a list of token-id lists, one per word."""
        samples = np.ascontiguousarray(samples, np.float32)
        lens = np.array([len(w) for w in words], np.int32)
        ids = np.array([i for w in words for i in w] or [0], np.int32)
        info = np.zeros(5, np.int64)
        check(host_lib().qah_aligner_prepare(self.handle, _p(samples), samples.size, len(words),
                                             _p(lens), _p(ids), _p(info)))
        self.info = dict(zip(("seq", "n_audio", "slots", "chunks", "tail"), map(int, info)))
        return self.info

    def forward(self):
        check(host_lib().qah_aligner_forward(self.handle))

    def result(self) -> tuple[np.ndarray, np.ndarray]:
        raw = np.zeros(self.info["slots"], np.int64)
        fixed = np.zeros_like(raw)
        check(host_lib().qah_aligner_result(self.handle, _p(raw), _p(fixed)))
        return raw, fixed

    def read(self, which: str) -> np.ndarray:
        n, seq = self.info["slots"], self.info["seq"]
        idx, shape, dt = {"classes": (0, (n,), np.int32),
                          "logits": (1, (n, self.labels), np.float32),
                          "ids": (2, (seq,), np.int32), "ts_pos": (3, (n,), np.int32),
                          "src": (4, (seq,), np.int32)}[which]
        out = np.empty(shape, dt)
        check(host_lib().qah_aligner_read(self.handle, idx, out.ctypes.data))
        return out

    def time(self, warmup, steps, use_graph=True) -> tuple[float, float]:
        ms, wall = ctypes.c_double(), ctypes.c_double()
        check(host_lib().qah_aligner_time(self.handle, warmup, steps, int(use_graph),
                                          ctypes.byref(ms), ctypes.byref(wall)))
        return ms.value, wall.value

    def profile(self, steps) -> dict:
        out = (ctypes.c_double * 5)()
        check(host_lib().qah_aligner_profile(self.handle, steps, out))
        return dict(zip(self.PHASES, list(out)))


def time_linear(ctx, desc, warmup: int, iters: int) -> float:
    ms = ctypes.c_double()
    check(host_lib().qah_time_linear(ctx.handle, ctypes.byref(desc), warmup, iters,
                                     ctypes.byref(ms)))
    return ms.value


def time_linears_each(ctx, descs, warmup: int, iters: int) -> np.ndarray:
    """qah_time_linears_each: per-launch ms of `iters` back-to-back launches
    cycling through `descs` (a list of pkg.LinearDesc)."""
    arr = (type(descs[0]) * len(descs))(*descs)
    out = np.zeros(iters, np.float32)
    check(host_lib().qah_time_linears_each(ctx.handle, arr, len(descs), warmup, iters,
                                           out.ctypes.data))
    return out


def time_linears_stamped(ctx, descs, warmup: int, iters: int) -> np.ndarray:
    """qah_time_linears_stamped: per-launch kernel ms (dispatch-stamped events,
    no inter-launch gap) of `iters` back-to-back launches cycling through `descs`."""
    arr = (type(descs[0]) * len(descs))(*descs)
    out = np.zeros(iters, np.float32)
    check(host_lib().qah_time_linears_stamped(ctx.handle, arr, len(descs), warmup, iters,
                                              out.ctypes.data))
    return out


def check_silu_f16x2(ctx, pairs: int, seed: int = 1) -> int:
    """qah_check_silu_f16x2: outputs of the f16 SiLU.up epilogue's packed
    arithmetic that differ from silu_mul in f32 plus a separate f16 rounding,
    over 2 * pairs generated inputs."""
    bad = ctypes.c_int64()
    check(host_lib().qah_check_silu_f16x2(ctx.handle, pairs, seed, ctypes.byref(bad)))
    return bad.value


def copy_calibration(ctx, nbytes: int, reps: int = 3) -> None:
    """qah_copy_calibration: a plain copy of nbytes, reps times (counter calibration)."""
    check(host_lib().qah_copy_calibration(ctx.handle, nbytes, reps))
