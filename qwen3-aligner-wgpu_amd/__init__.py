"""MI355X-native linear-layer GEMM path of qwen3-aligner-wgpu (and the decoder
prefill ops around it).

Python binding (ctypes) of the C ABI in include/qa.h, implemented by
csrc/libqa.so (hand-written gfx950 MFMA kernels), and of the C++ host mirror of
the reference's GEMM call sites, csrc/libqa_host.so.

The directory name is not a Python identifier, so load it with
``load_package()`` from ``__graft_entry__`` or by path; it registers as
``qwen3_aligner_wgpu_amd``.

There is no CPU fallback: if libqa.so is missing, importing the binding
raises, and every op runs on the GPU through the C ABI or fails.
"""
from __future__ import annotations

import ctypes
import os
import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(_HERE, "csrc")
# QA_BUILD=stamps loads the measurement build of `make -C csrc stamps` (the
# same libraries with per-block phase stamps in the GEMM kernels and per-wave
# phase cycles in the attention kernel).
_BUILD_DIR = os.path.join(CSRC, os.environ["QA_BUILD"]) if os.environ.get("QA_BUILD") else CSRC
LIB_PATH = os.path.join(_BUILD_DIR, "libqa.so")
HOST_LIB_PATH = os.path.join(_BUILD_DIR, "libqa_host.so")
INCLUDE_DIR = os.path.join(os.path.dirname(_HERE), "include")

# include/qa.h constants
QA_OK, QA_EINVAL, QA_ENOMEM, QA_EDEVICE, QA_EUNSUPPORTED = 0, -1, -2, -3, -4
F16, BF16 = 0, 1
ACCUMULATE, EPI_GELU, EPI_SILU_MUL, TRANSB, BIAS_ROWS = 1, 2, 4, 8, 16
QA_ATTN_P16 = 1  # qa_attention_desc.flags
QA_CONV_GELU, QA_CONV_TOKEN_MAJOR = 1, 2  # qa_conv_desc.flags

_STATUS = {
    QA_EINVAL: "QA_EINVAL",
    QA_ENOMEM: "QA_ENOMEM",
    QA_EDEVICE: "QA_EDEVICE",
    QA_EUNSUPPORTED: "QA_EUNSUPPORTED",
}


class QAError(RuntimeError):
    """A negative status from the C ABI, with qa_last_error()'s message."""

    def __init__(self, code: int, message: str):
        super().__init__(f"{_STATUS.get(code, code)}: {message}")
        self.code = code
        self.message = message


class LinearDesc(ctypes.Structure):
    """qa_linear_desc (include/qa.h)."""

    _fields_ = [
        ("dtype", ctypes.c_uint32),
        ("flags", ctypes.c_uint32),
        ("m", ctypes.c_int64),
        ("n", ctypes.c_int64),
        ("k", ctypes.c_int64),
        ("lda", ctypes.c_int64),
        ("ldb", ctypes.c_int64),
        ("ldc", ctypes.c_int64),
        ("a", ctypes.c_void_p),
        ("w", ctypes.c_void_p),
        ("c", ctypes.c_void_p),
        ("bias", ctypes.c_void_p),
        ("batch", ctypes.c_int64),
        ("bsa", ctypes.c_int64),
        ("bsb", ctypes.c_int64),
        ("bsc", ctypes.c_int64),
    ]


class MlpDesc(ctypes.Structure):
    """qa_mlp_desc (include/qa.h)."""

    _fields_ = [
        ("dtype", ctypes.c_uint32),
        ("flags", ctypes.c_uint32),
        ("m", ctypes.c_int64),
        ("hidden", ctypes.c_int64),
        ("inter", ctypes.c_int64),
        ("x", ctypes.c_void_p),
        ("w_gu", ctypes.c_void_p),
        ("w_down", ctypes.c_void_p),
        ("act", ctypes.c_void_p),
        ("h", ctypes.c_void_p),
    ]


class RmsNormDesc(ctypes.Structure):
    """qa_rms_norm_desc (include/qa.h)."""

    _fields_ = [
        ("dtype", ctypes.c_uint32),
        ("flags", ctypes.c_uint32),
        ("rows", ctypes.c_int64),
        ("n", ctypes.c_int64),
        ("x", ctypes.c_void_p),
        ("ldx", ctypes.c_int64),
        ("w", ctypes.c_void_p),
        ("y", ctypes.c_void_p),
        ("ldy", ctypes.c_int64),
        ("eps", ctypes.c_float),
    ]


class QkRopeDesc(ctypes.Structure):
    """qa_qk_rope_desc (include/qa.h)."""

    _fields_ = [
        ("dtype", ctypes.c_uint32),
        ("flags", ctypes.c_uint32),
        ("rows", ctypes.c_int64),
        ("nqh", ctypes.c_int32),
        ("nkvh", ctypes.c_int32),
        ("hd", ctypes.c_int32),
        ("eps", ctypes.c_float),
        ("qkv", ctypes.c_void_p),
        ("ldqkv", ctypes.c_int64),
        ("qn_w", ctypes.c_void_p),
        ("kn_w", ctypes.c_void_p),
        ("cos", ctypes.c_void_p),
        ("sin", ctypes.c_void_p),
        ("pos0", ctypes.c_int64),
        ("q_out", ctypes.c_void_p),
        ("k_cache", ctypes.c_void_p),
        ("v_cache", ctypes.c_void_p),
        ("cap", ctypes.c_int64),
        ("start", ctypes.c_int64),
    ]


class AttentionDesc(ctypes.Structure):
    """qa_attention_desc (include/qa.h)."""

    _fields_ = [
        ("dtype", ctypes.c_uint32),
        ("flags", ctypes.c_uint32),
        ("rows", ctypes.c_int64),
        ("nqh", ctypes.c_int32),
        ("nkvh", ctypes.c_int32),
        ("hd", ctypes.c_int32),
        ("q", ctypes.c_void_p),
        ("k_cache", ctypes.c_void_p),
        ("v_cache", ctypes.c_void_p),
        ("cap", ctypes.c_int64),
        ("q0", ctypes.c_int64),
        ("out", ctypes.c_void_p),
        ("ldo", ctypes.c_int64),
    ]


class LayerNormDesc(ctypes.Structure):
    """qa_layer_norm_desc (include/qa.h)."""

    _fields_ = [
        ("dtype", ctypes.c_uint32),
        ("flags", ctypes.c_uint32),
        ("rows", ctypes.c_int64),
        ("n", ctypes.c_int64),
        ("x", ctypes.c_void_p),
        ("ldx", ctypes.c_int64),
        ("w", ctypes.c_void_p),
        ("b", ctypes.c_void_p),
        ("y", ctypes.c_void_p),
        ("ldy", ctypes.c_int64),
        ("eps", ctypes.c_float),
    ]


class WindowAttentionDesc(ctypes.Structure):
    """qa_window_attention_desc (include/qa.h)."""

    _fields_ = [
        ("dtype", ctypes.c_uint32),
        ("flags", ctypes.c_uint32),
        ("s", ctypes.c_int64),
        ("nh", ctypes.c_int32),
        ("hd", ctypes.c_int32),
        ("wlen", ctypes.c_int64),
        ("qkv", ctypes.c_void_p),
        ("ldqkv", ctypes.c_int64),
        ("out", ctypes.c_void_p),
        ("ldo", ctypes.c_int64),
    ]


class PositionAddDesc(ctypes.Structure):
    """qa_position_add_desc (include/qa.h)."""

    _fields_ = [
        ("dtype", ctypes.c_uint32),
        ("flags", ctypes.c_uint32),
        ("rows", ctypes.c_int64),
        ("n", ctypes.c_int64),
        ("y", ctypes.c_void_p),
        ("ldy", ctypes.c_int64),
        ("table", ctypes.c_void_p),
        ("period", ctypes.c_int64),
    ]


class ConvDesc(ctypes.Structure):
    """qa_conv_desc (include/qa.h)."""

    _fields_ = [
        ("dtype", ctypes.c_uint32),
        ("flags", ctypes.c_uint32),
        ("batch", ctypes.c_int64),
        ("h", ctypes.c_int64),
        ("w", ctypes.c_int64),
        ("c_in", ctypes.c_int64),
        ("c_out", ctypes.c_int64),
        ("x", ctypes.c_void_p),
        ("weight", ctypes.c_void_p),
        ("bias", ctypes.c_void_p),
        ("y", ctypes.c_void_p),
    ]


class MelDesc(ctypes.Structure):
    """qa_mel_desc (include/qa.h)."""

    _fields_ = [
        ("dtype", ctypes.c_uint32),
        ("flags", ctypes.c_uint32),
        ("n_samples", ctypes.c_int64),
        ("samples", ctypes.c_void_p),
        ("filterbank", ctypes.c_void_p),
        ("n_mels", ctypes.c_int32),
        ("cs", ctypes.c_int32),
        ("out", ctypes.c_void_p),
    ]


class EmbedDesc(ctypes.Structure):
    """qa_embed_desc (include/qa.h)."""

    _fields_ = [
        ("dtype", ctypes.c_uint32),
        ("flags", ctypes.c_uint32),
        ("rows", ctypes.c_int64),
        ("hidden", ctypes.c_int64),
        ("src", ctypes.c_void_p),
        ("table", ctypes.c_void_p),
        ("vocab", ctypes.c_int64),
        ("audio", ctypes.c_void_p),
        ("n_audio", ctypes.c_int64),
        ("out", ctypes.c_void_p),
    ]


class HeadDesc(ctypes.Structure):
    """qa_head_desc (include/qa.h)."""

    _fields_ = [
        ("dtype", ctypes.c_uint32),
        ("flags", ctypes.c_uint32),
        ("rows", ctypes.c_int64),
        ("positions", ctypes.c_void_p),
        ("h", ctypes.c_void_p),
        ("h_rows", ctypes.c_int64),
        ("ldh", ctypes.c_int64),
        ("n", ctypes.c_int64),
        ("norm_w", ctypes.c_void_p),
        ("eps", ctypes.c_float),
        ("score", ctypes.c_void_p),
        ("labels", ctypes.c_int64),
        ("logits", ctypes.c_void_p),
        ("classes", ctypes.c_void_p),
    ]


# Every symbol include/qa.h declares (checked by tests/test_abi.py).
EXPORTS = (
    "qa_ctx_create", "qa_ctx_destroy", "qa_ctx_stream", "qa_alloc", "qa_free",
    "qa_upload", "qa_download", "qa_sync", "qa_linear", "qa_linear_validate",
    "qa_linear_noalloc", "qa_linear_noalloc_scratch_floats", "qa_prefetch_hint",
    "qa_time_next_launch",
    "qa_mlp_fused", "qa_rms_norm", "qa_qk_norm_rope", "qa_attention_prefill",
    "qa_layer_norm", "qa_window_attention", "qa_add_position_table", "qa_conv2d_3x3s2",
    "qa_mel_filterbank", "qa_log_mel", "qa_rope_tables", "qa_embed_scatter", "qa_timestamp_head",
    "qa_last_error", "qa_version",
)

_lib = None


def lib() -> ctypes.CDLL:
    """Load csrc/libqa.so (raises if it is not built: there is no fallback)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} is not built; run __graft_entry__.build()")
        L = ctypes.CDLL(LIB_PATH)
        vp, i = ctypes.c_void_p, ctypes.c_int
        sz = ctypes.c_size_t
        L.qa_ctx_create.argtypes = [i, ctypes.POINTER(vp)]
        L.qa_ctx_destroy.argtypes = [vp]
        L.qa_ctx_stream.argtypes = [vp]
        L.qa_ctx_stream.restype = vp
        L.qa_linear_noalloc_scratch_floats.argtypes = []
        L.qa_linear_noalloc_scratch_floats.restype = sz
        L.qa_alloc.argtypes = [vp, sz, ctypes.POINTER(vp)]
        L.qa_free.argtypes = [vp, vp]
        L.qa_upload.argtypes = [vp, vp, sz, vp, sz]
        L.qa_download.argtypes = [vp, vp, vp, sz, sz]
        L.qa_sync.argtypes = [vp]
        L.qa_linear.argtypes = [vp, ctypes.POINTER(LinearDesc)]
        L.qa_linear_noalloc.argtypes = [vp, ctypes.POINTER(LinearDesc)]
        L.qa_prefetch_hint.argtypes = [vp, vp, sz]
        L.qa_time_next_launch.argtypes = [vp, vp, vp]
        L.qa_linear_validate.argtypes = [ctypes.POINTER(LinearDesc)]
        L.qa_mlp_fused.argtypes = [vp, ctypes.POINTER(MlpDesc)]
        L.qa_rms_norm.argtypes = [vp, ctypes.POINTER(RmsNormDesc)]
        L.qa_qk_norm_rope.argtypes = [vp, ctypes.POINTER(QkRopeDesc)]
        L.qa_attention_prefill.argtypes = [vp, ctypes.POINTER(AttentionDesc)]
        L.qa_layer_norm.argtypes = [vp, ctypes.POINTER(LayerNormDesc)]
        L.qa_window_attention.argtypes = [vp, ctypes.POINTER(WindowAttentionDesc)]
        L.qa_add_position_table.argtypes = [vp, ctypes.POINTER(PositionAddDesc)]
        L.qa_conv2d_3x3s2.argtypes = [vp, ctypes.POINTER(ConvDesc)]
        L.qa_mel_filterbank.argtypes = [i, i, i, vp]
        L.qa_log_mel.argtypes = [vp, ctypes.POINTER(MelDesc)]
        L.qa_rope_tables.argtypes = [ctypes.c_int64, i, ctypes.c_double, ctypes.c_uint32, vp, vp]
        L.qa_embed_scatter.argtypes = [vp, ctypes.POINTER(EmbedDesc)]
        L.qa_timestamp_head.argtypes = [vp, ctypes.POINTER(HeadDesc)]
        L.qa_last_error.restype = ctypes.c_char_p
        L.qa_version.restype = ctypes.c_char_p
        for name in EXPORTS:
            if name not in ("qa_ctx_stream", "qa_last_error", "qa_version"):
                getattr(L, name).restype = ctypes.c_int
        _lib = L
    return _lib


def last_error() -> str:
    return lib().qa_last_error().decode()


def version() -> str:
    return lib().qa_version().decode()


def check(rc: int) -> None:
    if rc != QA_OK:
        raise QAError(rc, last_error())


def validate(desc: LinearDesc) -> int:
    """qa_linear_validate: the status code (0 = valid), no device needed."""
    return lib().qa_linear_validate(ctypes.byref(desc))


class DeviceBuffer:
    """A qa_alloc'd device buffer, freed by free() or its context's close()."""

    def __init__(self, ctx: "Context", ptr: int, nbytes: int):
        self.ctx, self.ptr, self.nbytes = ctx, ptr, nbytes

    def free(self) -> None:
        if self.ptr:
            check(lib().qa_free(self.ctx.handle, self.ptr))
            self.ctx._bufs.discard(self)
            self.ptr = 0

    def __int__(self) -> int:
        return self.ptr


class Context:
    """qa_ctx: one device, one in-order stream (include/qa.h)."""

    def __init__(self, device: int = 0):
        h = ctypes.c_void_p()
        check(lib().qa_ctx_create(device, ctypes.byref(h)))
        self.handle = h.value
        self._bufs: set[DeviceBuffer] = set()

    def close(self) -> None:
        if self.handle:
            for b in list(self._bufs):
                b.free()
            check(lib().qa_ctx_destroy(self.handle))
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    @property
    def stream(self) -> int:
        return lib().qa_ctx_stream(self.handle) or 0

    def alloc(self, nbytes: int) -> DeviceBuffer:
        p = ctypes.c_void_p()
        check(lib().qa_alloc(self.handle, nbytes, ctypes.byref(p)))
        b = DeviceBuffer(self, p.value, nbytes)
        self._bufs.add(b)
        return b

    def upload(self, buf: DeviceBuffer, host: np.ndarray, offset: int = 0) -> None:
        host = np.ascontiguousarray(host)
        assert offset + host.nbytes <= buf.nbytes
        check(lib().qa_upload(self.handle, buf.ptr, offset, host.ctypes.data, host.nbytes))

    def to_device(self, host: np.ndarray) -> DeviceBuffer:
        host = np.ascontiguousarray(host)
        b = self.alloc(host.nbytes)
        self.upload(b, host)
        return b

    def download(self, buf: DeviceBuffer, shape, dtype=np.uint16, offset: int = 0) -> np.ndarray:
        out = np.empty(shape, dtype)
        assert offset + out.nbytes <= buf.nbytes
        check(lib().qa_download(self.handle, out.ctypes.data, buf.ptr, offset, out.nbytes))
        return out

    def sync(self) -> None:
        check(lib().qa_sync(self.handle))

    def linear(self, desc: LinearDesc) -> None:
        check(lib().qa_linear(self.handle, ctypes.byref(desc)))

    def linear_noalloc(self, desc: LinearDesc) -> None:
        """qa_linear_noalloc: qa_linear with split-K partials in the library's
        fixed device scratch (no allocation)."""
        check(lib().qa_linear_noalloc(self.handle, ctypes.byref(desc)))

    def prefetch_hint(self, buf, nbytes=None) -> None:
        """qa_prefetch_hint: the next projection launched on this context pulls
        `buf` (normally the following projection's weights) toward the caches."""
        ptr = None if buf is None else buf.ptr
        check(lib().qa_prefetch_hint(self.handle, ptr, 0 if buf is None else
                                     (buf.nbytes if nbytes is None else nbytes)))

    def mlp_fused(self, desc: MlpDesc) -> None:
        check(lib().qa_mlp_fused(self.handle, ctypes.byref(desc)))

    def rms_norm(self, desc: RmsNormDesc) -> None:
        check(lib().qa_rms_norm(self.handle, ctypes.byref(desc)))

    def qk_norm_rope(self, desc: QkRopeDesc) -> None:
        check(lib().qa_qk_norm_rope(self.handle, ctypes.byref(desc)))

    def attention_prefill(self, desc: AttentionDesc) -> None:
        check(lib().qa_attention_prefill(self.handle, ctypes.byref(desc)))

    def layer_norm(self, desc: LayerNormDesc) -> None:
        check(lib().qa_layer_norm(self.handle, ctypes.byref(desc)))

    def window_attention(self, desc: WindowAttentionDesc) -> None:
        check(lib().qa_window_attention(self.handle, ctypes.byref(desc)))

    def add_position_table(self, desc: PositionAddDesc) -> None:
        check(lib().qa_add_position_table(self.handle, ctypes.byref(desc)))

    def conv2d_3x3s2(self, desc: ConvDesc) -> None:
        check(lib().qa_conv2d_3x3s2(self.handle, ctypes.byref(desc)))

    def log_mel(self, desc: MelDesc) -> None:
        check(lib().qa_log_mel(self.handle, ctypes.byref(desc)))

    def embed_scatter(self, desc: EmbedDesc) -> None:
        check(lib().qa_embed_scatter(self.handle, ctypes.byref(desc)))

    def timestamp_head(self, desc: HeadDesc) -> None:
        check(lib().qa_timestamp_head(self.handle, ctypes.byref(desc)))


def mel_filterbank(n_mels: int = 128, n_fft: int = 400, sample_rate: int = 16000) -> np.ndarray:
    """qa_mel_filterbank (host): the slaney filterbank [n_mels, n_fft // 2 + 1] f32."""
    out = np.empty((n_mels, n_fft // 2 + 1), np.float32)
    check(lib().qa_mel_filterbank(n_mels, n_fft, sample_rate, out.ctypes.data))
    return out


def rope_tables(positions: int, hd: int = 128, theta: float = 1e6,
                dtype: int = F16) -> tuple[np.ndarray, np.ndarray]:
    """qa_rope_tables (host): cos, sin [positions, hd] for text positions,
    rounded to the run's 16-bit format `dtype` and widened back to f32."""
    c = np.empty((positions, hd), np.float32)
    s = np.empty((positions, hd), np.float32)
    check(lib().qa_rope_tables(positions, hd, theta, dtype, c.ctypes.data, s.ctypes.data))
    return c, s


def linear_desc(dtype: int, m: int, n: int, k: int, a, w, c, *, flags: int = 0, bias=None,
                lda: int | None = None, ldb: int | None = None, ldc: int | None = None,
                batch: int = 1, bsa: int = 0, bsb: int = 0, bsc: int = 0) -> LinearDesc:
    """Build a qa_linear_desc from device buffers (or raw pointers)."""
    nout = n // 2 if flags & EPI_SILU_MUL else n
    return LinearDesc(
        dtype=dtype, flags=flags, m=m, n=n, k=k,
        lda=k if lda is None else lda,
        ldb=(n if flags & TRANSB else k) if ldb is None else ldb,
        ldc=nout if ldc is None else ldc,
        a=int(a), w=int(w), c=int(c), bias=int(bias) if bias is not None else None,
        batch=batch, bsa=bsa, bsb=bsb, bsc=bsc,
    )


_host = None


def host_lib() -> ctypes.CDLL:
    """Load csrc/libqa_host.so (raises if it is not built)."""
    global _host
    if _host is None:
        lib()  # libqa.so first: libqa_host.so links against it
        if not os.path.exists(HOST_LIB_PATH):
            raise ImportError(f"{HOST_LIB_PATH} is not built; run __graft_entry__.build()")
        _host = ctypes.CDLL(HOST_LIB_PATH)
        from . import host as _h  # noqa: F401  (declares the signatures)

        _h.declare(_host)
    return _host
