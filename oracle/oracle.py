"""ctypes view of the CPU oracle (oracle/liboracle.so).

TEST INFRASTRUCTURE ONLY.  Imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, as the checker and as the timed CPU baseline.
The product (libqa.so and its Python binding) never imports this module.

Each wrapper names the C function it calls; the C file cites the reference
(eclipse005/qwen3-aligner-wgpu) file:line every function restates.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")

F16, BF16 = 0, 1
ACCUMULATE, EPI_GELU, EPI_SILU_MUL, TRANSB, BIAS_ROWS, EXACT = 1, 2, 4, 8, 16, 256


class LinearDesc(ctypes.Structure):
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


def build(force: bool = False) -> str:
    """Compile liboracle.so with its Makefile (gcc + OpenMP)."""
    import subprocess

    cmd = ["make", "-C", _HERE] + (["-B"] if force else [])
    subprocess.run(cmd, check=True, stdout=subprocess.DEVNULL)
    return _LIB_PATH


_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            raise RuntimeError(f"{_LIB_PATH} is not built; run oracle.build() or make -C oracle")
        L = ctypes.CDLL(_LIB_PATH)
        L.or_f16_from_f32.restype = ctypes.c_uint16
        L.or_f16_from_f32.argtypes = [ctypes.c_float]
        L.or_f16_to_f32.restype = ctypes.c_float
        L.or_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.or_bf16_from_f32.restype = ctypes.c_uint16
        L.or_bf16_from_f32.argtypes = [ctypes.c_float]
        L.or_bf16_to_f32.restype = ctypes.c_float
        L.or_bf16_to_f32.argtypes = [ctypes.c_uint16]
        p = ctypes.c_void_p
        i64 = ctypes.c_int64
        L.or_h16_to_f32_n.argtypes = [p, p, i64, ctypes.c_int]
        L.or_f32_to_h16_n.argtypes = [p, p, i64, ctypes.c_int]
        L.or_gemm_f32.argtypes = [i64, i64, i64, p, i64, p, i64, p, i64, ctypes.c_float]
        L.or_gemm_f32_naive.argtypes = [i64, i64, i64, p, i64, p, i64, p, i64]
        L.or_gemm_f64.argtypes = [i64, i64, i64, p, i64, p, i64, p, i64]
        L.or_silu_mul.restype = ctypes.c_float
        L.or_silu_mul.argtypes = [ctypes.c_float, ctypes.c_float]
        L.or_gelu.restype = ctypes.c_float
        L.or_gelu.argtypes = [ctypes.c_float]
        L.or_linear.restype = ctypes.c_int
        L.or_linear.argtypes = [ctypes.POINTER(LinearDesc)]
        ci, f = ctypes.c_int, ctypes.c_float
        L.or_rms_norm.argtypes = [ci, i64, i64, p, i64, p, f, p, i64]
        L.or_rms_norm.restype = None
        L.or_qk_norm_rope.argtypes = [ci, i64, ci, ci, ci, p, i64, p, p, p, p, i64, f, p, p, p,
                                      i64, i64]
        L.or_qk_norm_rope.restype = None
        L.or_attention.argtypes = [ci, i64, ci, ci, ci, p, p, p, i64, i64, p, i64]
        L.or_attention.restype = None
        L.or_vperm.argtypes = [i64]
        L.or_layer_norm.argtypes = [ci, i64, i64, p, i64, p, p, f, p, i64]
        L.or_layer_norm.restype = None
        L.or_window_attention.argtypes = [ci, i64, ci, ci, i64, p, i64, p, i64]
        L.or_window_attention.restype = None
        L.or_add_position_table.argtypes = [ci, i64, i64, p, i64, p, i64]
        L.or_add_position_table.restype = None
        L.or_sinusoid_table.argtypes = [i64, i64, p]
        L.or_sinusoid_table.restype = None
        L.or_conv3x3s2.argtypes = [ci, i64, i64, i64, i64, i64, p, p, i64, p, ci, ci, i64, i64, p]
        L.or_conv3x3s2.restype = None
        L.or_mel_filterbank.argtypes = [ci, ci, ci, p]
        L.or_mel_filterbank.restype = None
        L.or_stft_power.argtypes = [p, i64, ci, ci, p]
        L.or_stft_power.restype = None
        L.or_log_mel.argtypes = [p, i64, ci, p, p]
        L.or_log_mel.restype = None
        L.or_timestamp_head.argtypes = [ci, i64, p, p, i64, i64, p, f, p, i64, p, p]
        L.or_timestamp_head.restype = None
        L.or_linear_f32.argtypes = [i64, i64, i64, p, i64, p, ci, p, p, i64]
        L.or_linear_f32.restype = None
        L.or_layer_norm_f32.argtypes = [i64, i64, p, p, p, f, p]
        L.or_layer_norm_f32.restype = None
        L.or_gelu_f32_n.argtypes = [p, i64]
        L.or_gelu_f32_n.restype = None
        L.or_window_attention_f32.argtypes = [i64, ci, ci, i64, p, p, p, i64, p]
        L.or_window_attention_f32.restype = None
        L.or_conv3x3s2_f32.argtypes = [i64, i64, i64, i64, i64, p, p, i64, p, ci, ci, p]
        L.or_conv3x3s2_f32.restype = None
        L.or_head_fold.argtypes = [ci, i64, p, p, i64, i64, p, f, p]
        L.or_head_fold.restype = None
        L.or_vperm.restype = i64
        L.or_num_threads.restype = ctypes.c_int
        L.or_set_threads.argtypes = [ci]
        L.or_set_threads.restype = None
        _lib = L
    return _lib


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data


def _c(a: np.ndarray, dtype) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=dtype)


def h16_from_f32(x: np.ndarray, dtype: int) -> np.ndarray:
    """or_f32_to_h16_n: f32 -> 16-bit bits (uint16) in `dtype`'s format."""
    x = _c(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().or_f32_to_h16_n(_ptr(x), _ptr(out), x.size, dtype)
    return out


def h16_to_f32(h: np.ndarray, dtype: int) -> np.ndarray:
    """or_h16_to_f32_n: 16-bit bits -> f32 values (exact)."""
    h = _c(h, np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().or_h16_to_f32_n(_ptr(h), _ptr(out), h.size, dtype)
    return out


def gemm_f32(x: np.ndarray, w: np.ndarray, out: np.ndarray | None = None, beta: float = 0.0) -> np.ndarray:
    """or_gemm_f32: out = beta*out + x @ w.T (x [m,k], w [n,k], f32)."""
    x = _c(x, np.float32)
    w = _c(w, np.float32)
    m, k = x.shape
    n = w.shape[0]
    assert w.shape[1] == k
    if out is None:
        out = np.zeros((m, n), np.float32)
    assert out.dtype == np.float32 and out.flags.c_contiguous and out.shape == (m, n)
    lib().or_gemm_f32(m, n, k, _ptr(x), k, _ptr(w), k, _ptr(out), n, beta)
    return out


def gemm_f32_naive(x: np.ndarray, w: np.ndarray) -> np.ndarray:
    """or_gemm_f32_naive: sequential f32 triple loop."""
    x = _c(x, np.float32)
    w = _c(w, np.float32)
    m, k = x.shape
    n = w.shape[0]
    out = np.empty((m, n), np.float32)
    lib().or_gemm_f32_naive(m, n, k, _ptr(x), k, _ptr(w), k, _ptr(out), n)
    return out


def gemm_f64(x: np.ndarray, w: np.ndarray) -> np.ndarray:
    """or_gemm_f64: f64 triple loop over f32 inputs."""
    x = _c(x, np.float32)
    w = _c(w, np.float32)
    m, k = x.shape
    n = w.shape[0]
    out = np.empty((m, n), np.float64)
    lib().or_gemm_f64(m, n, k, _ptr(x), k, _ptr(w), k, _ptr(out), n)
    return out


def silu_mul(g: float, u: float) -> float:
    return lib().or_silu_mul(g, u)


def gelu(x: float) -> float:
    return lib().or_gelu(x)


def linear(dtype: int, a: np.ndarray, w: np.ndarray, c: np.ndarray, *, flags: int = 0,
           bias: np.ndarray | None = None, m: int | None = None, n: int | None = None,
           k: int | None = None, lda: int | None = None, ldb: int | None = None,
           ldc: int | None = None, batch: int = 1, bsa: int = 0, bsb: int = 0,
           bsc: int = 0) -> np.ndarray:
    """or_linear on uint16 bit arrays; updates and returns `c`.

    Shapes default from the arrays: a [m,k], w [n,k] ([k,n] with TRANSB),
    c [m, n] ([m, n/2] with EPI_SILU_MUL)."""
    for arr in (a, w, c):
        assert arr.dtype == np.uint16 and arr.flags.c_contiguous
    if bias is not None:
        assert bias.dtype == np.uint16 and bias.flags.c_contiguous
    if m is None:
        m = a.shape[-2]
    if k is None:
        k = a.shape[-1]
    if n is None:
        n = w.shape[-1] if flags & TRANSB else w.shape[-2]
    d = LinearDesc(
        dtype=dtype, flags=flags, m=m, n=n, k=k,
        lda=lda if lda is not None else a.shape[-1],
        ldb=ldb if ldb is not None else w.shape[-1],
        ldc=ldc if ldc is not None else c.shape[-1],
        a=_ptr(a), w=_ptr(w), c=_ptr(c), bias=_ptr(bias) if bias is not None else None,
        batch=batch, bsa=bsa, bsb=bsb, bsc=bsc,
    )
    rc = lib().or_linear(ctypes.byref(d))
    if rc != 0:
        raise ValueError(f"or_linear rejected the descriptor (rc={rc})")
    return c


def num_threads() -> int:
    return lib().or_num_threads()


def set_threads(n: int) -> None:
    lib().or_set_threads(n)


def rms_norm(dtype: int, x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    """or_rms_norm: x [rows, n] 16-bit bits, w [n] f32 -> [rows, n] bits."""
    x = _c(x, np.uint16)
    w = _c(w, np.float32)
    rows, n = x.shape
    y = np.empty_like(x)
    lib().or_rms_norm(dtype, rows, n, _ptr(x), n, _ptr(w), ctypes.c_float(eps), _ptr(y), n)
    return y


def qk_norm_rope(dtype: int, qkv: np.ndarray, nqh: int, nkvh: int, hd: int, qn: np.ndarray,
                 kn: np.ndarray, cos_t: np.ndarray, sin_t: np.ndarray, pos0: int, eps: float,
                 k_cache: np.ndarray, v_cache: np.ndarray, start: int) -> np.ndarray:
    """or_qk_norm_rope: returns q_out [nqh, rows, hd]; writes k_cache [nkvh, cap, hd]
    and the transposed v_cache [nkvh, hd, cap] in place."""
    qkv = _c(qkv, np.uint16)
    rows = qkv.shape[0]
    cap = k_cache.shape[1]
    for arr in (k_cache, v_cache):
        assert arr.dtype == np.uint16 and arr.flags.c_contiguous
    q_out = np.empty((nqh, rows, hd), np.uint16)
    lib().or_qk_norm_rope(dtype, rows, nqh, nkvh, hd, _ptr(qkv), qkv.shape[1],
                          _ptr(_c(qn, np.float32)), _ptr(_c(kn, np.float32)),
                          _ptr(_c(cos_t, np.float32)), _ptr(_c(sin_t, np.float32)), pos0,
                          ctypes.c_float(eps), _ptr(q_out), _ptr(k_cache), _ptr(v_cache), cap,
                          start)
    return q_out


def vperm(n: int) -> np.ndarray:
    """or_vperm over 0..n-1: the V-cache column of each key."""
    return np.array([lib().or_vperm(t) for t in range(n)], np.int64)


def attention(dtype: int, q: np.ndarray, k_cache: np.ndarray, v_cache: np.ndarray,
              q0: int) -> np.ndarray:
    """or_attention: q [nqh, rows, hd], k_cache [nkvh, cap, hd], v_cache [nkvh, hd, cap]
    -> out [rows, nqh * hd]."""
    q = _c(q, np.uint16)
    k_cache = _c(k_cache, np.uint16)
    v_cache = _c(v_cache, np.uint16)
    nqh, rows, hd = q.shape
    nkvh, cap, _ = k_cache.shape
    out = np.empty((rows, nqh * hd), np.uint16)
    lib().or_attention(dtype, rows, nqh, nkvh, hd, _ptr(q), _ptr(k_cache), _ptr(v_cache), cap,
                       q0, _ptr(out), nqh * hd)
    return out


def layer_norm(dtype: int, x: np.ndarray, w: np.ndarray, b: np.ndarray, eps: float) -> np.ndarray:
    """or_layer_norm: x [rows, n] 16-bit bits, w/b [n] f32 -> [rows, n] bits."""
    x = _c(x, np.uint16)
    rows, n = x.shape
    y = np.empty_like(x)
    lib().or_layer_norm(dtype, rows, n, _ptr(x), n, _ptr(_c(w, np.float32)),
                        _ptr(_c(b, np.float32)), ctypes.c_float(eps), _ptr(y), n)
    return y


def window_attention(dtype: int, qkv: np.ndarray, nh: int, hd: int, wlen: int) -> np.ndarray:
    """or_window_attention: qkv [s, 3*nh*hd] (q | k | v) -> out [s, nh*hd]."""
    qkv = _c(qkv, np.uint16)
    s = qkv.shape[0]
    out = np.empty((s, nh * hd), np.uint16)
    lib().or_window_attention(dtype, s, nh, hd, wlen, _ptr(qkv), qkv.shape[1], _ptr(out), nh * hd)
    return out


def add_position_table(dtype: int, y: np.ndarray, table: np.ndarray) -> np.ndarray:
    """or_add_position_table: returns y + table[r % period] (y [rows, n] bits)."""
    y = _c(y, np.uint16).copy()
    table = _c(table, np.float32)
    rows, n = y.shape
    lib().or_add_position_table(dtype, rows, n, _ptr(y), n, _ptr(table), table.shape[0])
    return y


def sinusoid_table(positions: int, dm: int) -> np.ndarray:
    """or_sinusoid_table: the audio tower's position table [positions, dm] f32."""
    t = np.empty((positions, dm), np.float32)
    lib().or_sinusoid_table(positions, dm, _ptr(t))
    return t


def conv3x3s2(dtype: int, x: np.ndarray, weight: np.ndarray, bias: np.ndarray | None, *,
              gelu: bool = True, token_major: bool = False, rows: tuple | None = None) -> np.ndarray:
    """or_conv3x3s2: x [b, h, w, c_in] bits, weight [c_out, ldw] bits (k = (kh*3+kw)*c_in+ic),
    bias [c_out] bits or None -> y rows [m0, m1) of [b*ho*wo, c_out]."""
    x = _c(x, np.uint16)
    weight = _c(weight, np.uint16)
    b, h, w, c_in = x.shape
    c_out, ldw = weight.shape
    ho, wo = (h - 1) // 2 + 1, (w - 1) // 2 + 1
    m0, m1 = rows if rows is not None else (0, b * ho * wo)
    y = np.empty((m1 - m0, c_out), np.uint16)
    bb = _c(bias, np.uint16) if bias is not None else None
    lib().or_conv3x3s2(dtype, b, h, w, c_in, c_out, _ptr(x), _ptr(weight), ldw,
                       _ptr(bb) if bb is not None else None, int(gelu), int(token_major), m0, m1,
                       _ptr(y))
    return y


def mel_filterbank(n_mels: int = 128, n_fft: int = 400, sr: int = 16000) -> np.ndarray:
    """or_mel_filterbank -> [n_mels, n_fft // 2 + 1] f32."""
    out = np.empty((n_mels, n_fft // 2 + 1), np.float32)
    lib().or_mel_filterbank(n_mels, n_fft, sr, _ptr(out))
    return out


def stft_power(x: np.ndarray, n_fft: int = 400, hop: int = 160) -> np.ndarray:
    """or_stft_power -> [frames, n_fft // 2 + 1] f64."""
    x = _c(x, np.float32)
    out = np.empty((x.size // hop, n_fft // 2 + 1), np.float64)
    lib().or_stft_power(_ptr(x), x.size, n_fft, hop, _ptr(out))
    return out


def log_mel(x: np.ndarray, filt: np.ndarray | None = None, n_mels: int = 128) -> np.ndarray:
    """or_log_mel -> [n_mels, frames] f32 (before the 16-bit rounding)."""
    x = _c(x, np.float32)
    filt = mel_filterbank(n_mels) if filt is None else _c(filt, np.float32)
    out = np.empty((n_mels, x.size // 160), np.float32)
    lib().or_log_mel(_ptr(x), x.size, n_mels, _ptr(filt), _ptr(out))
    return out


def timestamp_head(dtype: int, h: np.ndarray, positions, w: np.ndarray, eps: float,
                   score: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """or_timestamp_head -> (logits f64 [rows, labels], classes int32 [rows])."""
    h = _c(h, np.uint16)
    pos = _c(np.asarray(positions), np.int32)
    score = _c(score, np.float32)
    labels, n = score.shape
    logits = np.empty((pos.size, labels), np.float64)
    cls = np.empty(pos.size, np.int32)
    lib().or_timestamp_head(dtype, pos.size, _ptr(pos), _ptr(h), h.shape[1], n,
                            _ptr(_c(w, np.float32)), ctypes.c_float(eps), _ptr(score), labels,
                            _ptr(logits), _ptr(cls))
    return logits, cls


# ---- the reference's CPU audio tower in f32 (CpuAudioEncoder::forward) ----

def linear_f32(x: np.ndarray, w: np.ndarray, dtype: int, bias: np.ndarray | None = None) -> np.ndarray:
    """or_linear_f32: f32 x [m, k] . (16-bit W [n, k] widened)^T, + f32 bias -> f32 [m, n]."""
    x = _c(x, np.float32)
    w = _c(w, np.uint16)
    m, k = x.shape
    n = w.shape[0]
    y = np.empty((m, n), np.float32)
    bb = _c(bias, np.float32) if bias is not None else None
    lib().or_linear_f32(m, n, k, _ptr(x), k, _ptr(w), dtype, _ptr(bb) if bb is not None else None,
                        _ptr(y), n)
    return y


def layer_norm_f32(x: np.ndarray, w: np.ndarray, b: np.ndarray, eps: float) -> np.ndarray:
    """or_layer_norm_f32: f32 rows -> f32 rows."""
    x = _c(x, np.float32)
    y = np.empty_like(x)
    lib().or_layer_norm_f32(x.shape[0], x.shape[1], _ptr(x), _ptr(_c(w, np.float32)),
                            _ptr(_c(b, np.float32)), ctypes.c_float(eps), _ptr(y))
    return y


def gelu_f32(x: np.ndarray) -> np.ndarray:
    """or_gelu_f32_n: elementwise erf GELU in f32 (a new array)."""
    y = _c(x, np.float32).copy()
    lib().or_gelu_f32_n(_ptr(y), y.size)
    return y


def window_attention_f32(q: np.ndarray, k: np.ndarray, v: np.ndarray, nh: int, hd: int,
                         wlen: int) -> np.ndarray:
    """or_window_attention_f32: f32 q, k, v [s, nh*hd] -> out [s, nh*hd] f32."""
    q, k, v = (_c(a, np.float32) for a in (q, k, v))
    s = q.shape[0]
    out = np.empty((s, nh * hd), np.float32)
    lib().or_window_attention_f32(s, nh, hd, wlen, _ptr(q), _ptr(k), _ptr(v), q.shape[1], _ptr(out))
    return out


def conv3x3s2_f32(x: np.ndarray, weight: np.ndarray, bias: np.ndarray | None, *,
                  gelu: bool = True, token_major: bool = False) -> np.ndarray:
    """or_conv3x3s2_f32: x [b, h, w, c_in] f32, weight [c_out, ldw] f32
    (k = (kh*3+kw)*c_in+ic), bias [c_out] f32 or None -> y [b*ho*wo, c_out] f32."""
    x = _c(x, np.float32)
    weight = _c(weight, np.float32)
    b, h, w, c_in = x.shape
    c_out, ldw = weight.shape
    ho, wo = (h - 1) // 2 + 1, (w - 1) // 2 + 1
    y = np.empty((b * ho * wo, c_out), np.float32)
    bb = _c(bias, np.float32) if bias is not None else None
    lib().or_conv3x3s2_f32(b, h, w, c_in, c_out, _ptr(x), _ptr(weight), ldw,
                           _ptr(bb) if bb is not None else None, int(gelu), int(token_major),
                           _ptr(y))
    return y


def head_fold(dtype: int, h: np.ndarray, positions, w: np.ndarray, eps: float) -> np.ndarray:
    """or_head_fold: the folded final norm of rows `positions` of h -> f32 [rows, n]."""
    h = _c(h, np.uint16)
    pos = _c(np.asarray(positions), np.int32)
    n = h.shape[1]
    y = np.empty((pos.size, n), np.float32)
    lib().or_head_fold(dtype, pos.size, _ptr(pos), _ptr(h), n, n, _ptr(_c(w, np.float32)),
                       ctypes.c_float(eps), _ptr(y))
    return y


def timestamp_head_f32(dtype: int, h: np.ndarray, positions, w: np.ndarray, eps: float,
                       score: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """The head as the reference computes it on the host
    (src/align_inference.rs:766-805): the folded norm in f32, the logits with
    the f32 GEMM (cpu_tensor::linear -> or_gemm_f32), the first index of the
    maximum -> (logits f32 [rows, labels], classes int32 [rows])."""
    y = head_fold(dtype, h, positions, w, eps)
    logits = gemm_f32(y, _c(score, np.float32))
    return logits, np.argmax(logits, axis=1).astype(np.int32)


def fix_timestamps(data) -> list[int]:
    """The timestamp repair, restated from src/postprocess.rs:33-111 (test
    infrastructure: the checker of the host library's qah_fix_timestamps).

    best[i] is the longest non-decreasing subsequence ending at i, prev[i]
    the earliest predecessor reaching it; the subsequence kept ends at the
    first i of maximal length.  Every maximal run of other positions is
    rewritten from its kept neighbours: runs of 1-2 take the neighbour nearer
    by index (left when equally near), longer runs the linear interpolation
    left + (right - left) / (len + 1) * k truncated toward zero, and a run
    with a single neighbour takes that neighbour's value."""
    data = [int(v) for v in data]
    n = len(data)
    if n == 0:
        return []
    best, prev = [1] * n, [-1] * n
    for i in range(n):
        for j in range(i):
            if data[j] <= data[i] and best[j] + 1 > best[i]:
                best[i], prev[i] = best[j] + 1, j
    i = best.index(max(best))
    keep = set()
    while i != -1:
        keep.add(i)
        i = prev[i]
    out = list(data)
    i = 0
    while i < n:
        if i in keep:
            i += 1
            continue
        j = i
        while j < n and j not in keep:
            j += 1
        left = out[i - 1] if i > 0 else None
        right = out[j] if j < n else None
        run = j - i
        for p in range(i, j):
            if left is not None and right is not None:
                if run <= 2:
                    out[p] = left if p - (i - 1) <= j - p else right
                else:
                    out[p] = int(left + (right - left) / (run + 1) * (p - i + 1))
            else:
                out[p] = left if left is not None else right
        i = j
    return out
