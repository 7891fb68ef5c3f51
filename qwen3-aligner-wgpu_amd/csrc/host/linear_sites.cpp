// linear_sites.cpp -- C++ host mirror of the reference's GEMM call sites.
//
// Text decoder: WgpuTextDecoder::prefill's four projections per layer
// (src/decoder.rs:1321-1327, 1602-1608, 1628-1650, 1652-1657) over the fused
// weights of convert_layer / fused_pieces (src/decoder.rs:816-871).
// Audio tower: GpuAudioEncoder::layer's linears (src/audio_encoder_gpu.rs:
// 1414-1419, 1579-1581, 1594-1605) and a conv block as im2col GEMM + bias +
// GELU (src/audio_encoder.rs:376-447).  Only include/qa.h is used to reach the
// device; HIP is used directly for events and graph capture, as the
// reference's callers use wgpu's queue directly.
#include "linear_sites.hpp"

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstring>
#include <thread>

#include "../half_bits.h"
#include "../qa_internal.h"
#include "qa_host.h"
#include "timing.hpp"

namespace qa_host {

namespace {

int hip_status(hipError_t e) { return e == hipSuccess ? QA_OK : QA_EDEVICE; }

size_t elems_bytes(int64_t n) { return (size_t)n * 2; }

int64_t align_up(int64_t v, int64_t a) { return (v + a - 1) / a * a; }

uint16_t narrow16(float v, int dtype) {
  // by integer arithmetic (half_bits.h): src/shaders.rs:169-179 for bf16,
  // IEEE round to nearest even for f16
  return dtype == QA_BF16 ? qa_half::bf16_from_f32(v) : qa_half::f16_from_f32(v);
}

uint64_t splitmix64(uint64_t x) {
  x += 0x9E3779B97F4A7C15ull;
  x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
  x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
  return x ^ (x >> 31);
}

// Element i of the (seed, tensor) stream: two SplitMix64 outputs, Box-Muller.
double normal_at(uint64_t base, size_t i) {
  const uint64_t r1 = splitmix64(base + 2 * (uint64_t)i);
  const uint64_t r2 = splitmix64(base + 2 * (uint64_t)i + 1);
  const double u1 = ((double)(r1 >> 11) + 1.0) * 0x1.0p-53;  // (0, 1]
  const double u2 = (double)(r2 >> 11) * 0x1.0p-53;          // [0, 1)
  return std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2);
}

uint64_t stream_base(uint64_t seed, uint64_t tensor_id) {
  return splitmix64(seed ^ splitmix64(tensor_id * 0xD1B54A32D192ED03ull + 1));
}

template <class F>
void parallel_for(size_t n, F&& f) {
  const size_t hw = std::max(1u, std::min(16u, std::thread::hardware_concurrency()));
  const size_t nt = n < (1u << 16) ? 1 : hw;
  if (nt == 1) {
    f((size_t)0, n);
    return;
  }
  std::vector<std::thread> ts;
  const size_t chunk = (n + nt - 1) / nt;
  for (size_t t = 0; t < nt; ++t) {
    const size_t lo = t * chunk, hi = std::min(n, lo + chunk);
    if (lo >= hi) break;
    ts.emplace_back([&f, lo, hi] { f(lo, hi); });
  }
  for (auto& th : ts) th.join();
}

}  // namespace

int alloc(qa_ctx* ctx, size_t bytes, Buffer* b) {
  b->bytes = bytes;
  return qa_alloc(ctx, bytes, &b->ptr);
}

void release(qa_ctx* ctx, Buffer* b) {
  if (b->ptr) qa_free(ctx, b->ptr);
  b->ptr = nullptr;
  b->bytes = 0;
}

int gemm(qa_ctx* ctx, int dtype, const void* a, const void* w, void* c, int64_t m, int64_t n,
         int64_t k, int64_t ldc, int64_t bsa_words, int64_t bsb_words, int64_t bsc, int64_t batch,
         bool beta, uint32_t extra_flags, const void* bias) {
  qa_linear_desc d{};
  d.dtype = (uint32_t)dtype;
  d.flags = (beta ? QA_ACCUMULATE : 0u) | extra_flags;
  d.m = m;
  d.n = n;
  d.k = k;
  d.lda = k;
  d.ldb = (extra_flags & QA_TRANSB) ? n : k;
  d.ldc = ldc;
  d.a = a;
  d.w = w;
  d.c = c;
  d.bias = bias;
  d.batch = batch;
  d.bsa = bsa_words * 2;  // GDims words -> elements
  d.bsb = bsb_words * 2;
  d.bsc = bsc;
  return qa_linear(ctx, &d);
}

int load_linear(qa_ctx* ctx, const uint16_t* w, const uint16_t* bias, int64_t n, int64_t k,
                Linear* out) {
  out->n = n;
  out->k = k;
  out->n_pad = align_up(n, 4);
  out->k_pad = align_up(k, 8);
  std::vector<uint16_t> wp((size_t)(out->n_pad * out->k_pad), 0);
  for (int64_t r = 0; r < n; ++r) memcpy(&wp[(size_t)(r * out->k_pad)], w + r * k, elems_bytes(k));
  std::vector<uint16_t> bp((size_t)out->n_pad, 0);  // a missing bias is a zero bias (:228-229)
  if (bias) memcpy(bp.data(), bias, elems_bytes(n));
  if (int rc = alloc(ctx, wp.size() * 2, &out->w)) return rc;
  if (int rc = qa_upload(ctx, out->w.ptr, 0, wp.data(), wp.size() * 2)) return rc;
  if (int rc = alloc(ctx, bp.size() * 2, &out->b)) return rc;
  return qa_upload(ctx, out->b.ptr, 0, bp.data(), bp.size() * 2);
}

// ------------------------------------------------------------------------
TextDecoderLinears::TextDecoderLinears(qa_ctx* c, int dt, int nl, int hs, int qd, int kvd,
                                       int it, int mr)
    : ctx(c), dtype(dt), layers(nl), hidden(hs), q_dim(qd), kv_dim(kvd), inter(it),
      max_rows(mr), L((size_t)nl) {}

TextDecoderLinears::~TextDecoderLinears() {
  for (auto& l : L) {
    release(ctx, &l.qkv_w);
    release(ctx, &l.o_w);
    release(ctx, &l.gu_w);
    release(ctx, &l.dp_w);
  }
  for (Buffer* b : {&normed, &attn, &norm2, &h, &qkv, &act}) release(ctx, b);
}

int TextDecoderLinears::init() {
  const int64_t r = max_rows;
  if (int rc = alloc(ctx, elems_bytes(r * hidden), &normed)) return rc;
  if (int rc = alloc(ctx, elems_bytes(r * q_dim), &attn)) return rc;
  if (int rc = alloc(ctx, elems_bytes(r * hidden), &norm2)) return rc;
  if (int rc = alloc(ctx, elems_bytes(r * hidden), &h)) return rc;
  if (int rc = alloc(ctx, elems_bytes(r * (q_dim + 2 * kv_dim)), &qkv)) return rc;
  return alloc(ctx, elems_bytes(r * inter), &act);
}

int TextDecoderLinears::load_layer(int li, const uint16_t* q, const uint16_t* k,
                                   const uint16_t* v, const uint16_t* o, const uint16_t* gate,
                                   const uint16_t* up, const uint16_t* down) {
  if (li < 0 || li >= layers) return QA_EINVAL;
  Layer& l = L[(size_t)li];
  const int64_t hs = hidden;
  // fused [q | k | v] and [gate | up] rows (src/decoder.rs:816-871)
  const uint16_t* qkv_parts[3] = {q, k, v};
  const int64_t qkv_rows[3] = {q_dim, kv_dim, kv_dim};
  std::vector<uint16_t> fused((size_t)((q_dim + 2 * kv_dim) * hs));
  qah_concat_rows(qkv_parts, qkv_rows, 3, hs, fused.data());
  if (int rc = alloc(ctx, fused.size() * 2, &l.qkv_w)) return rc;
  if (int rc = qa_upload(ctx, l.qkv_w.ptr, 0, fused.data(), fused.size() * 2)) return rc;
  const uint16_t* gu_parts[2] = {gate, up};
  const int64_t gu_rows[2] = {inter, inter};
  fused.assign((size_t)(2 * inter * hs), 0);
  qah_concat_rows(gu_parts, gu_rows, 2, hs, fused.data());
  if (int rc = alloc(ctx, fused.size() * 2, &l.gu_w)) return rc;
  if (int rc = qa_upload(ctx, l.gu_w.ptr, 0, fused.data(), fused.size() * 2)) return rc;
  if (int rc = alloc(ctx, elems_bytes((int64_t)hs * q_dim), &l.o_w)) return rc;
  if (int rc = qa_upload(ctx, l.o_w.ptr, 0, o, elems_bytes((int64_t)hs * q_dim))) return rc;
  if (int rc = alloc(ctx, elems_bytes((int64_t)hs * inter), &l.dp_w)) return rc;
  return qa_upload(ctx, l.dp_w.ptr, 0, down, elems_bytes((int64_t)hs * inter));
}

int TextDecoderLinears::set_inputs(int rows, const uint16_t* n1, const uint16_t* at,
                                   const uint16_t* n2, const uint16_t* hh) {
  if (rows < 0 || rows > max_rows) return QA_EINVAL;
  const int64_t r = rows;
  if (n1) if (int rc = qa_upload(ctx, normed.ptr, 0, n1, elems_bytes(r * hidden))) return rc;
  if (at) if (int rc = qa_upload(ctx, attn.ptr, 0, at, elems_bytes(r * q_dim))) return rc;
  if (n2) if (int rc = qa_upload(ctx, norm2.ptr, 0, n2, elems_bytes(r * hidden))) return rc;
  if (hh) if (int rc = qa_upload(ctx, h.ptr, 0, hh, elems_bytes(r * hidden))) return rc;
  return QA_OK;
}

int TextDecoderLinears::layer(int li, int rows, hipEvent_t* ev) {
  const Layer& l = L[(size_t)li];
  const int64_t s_rows = rows, hs = hidden, qkv_n = q_dim + 2 * kv_dim;
  // per-site kernel times: the site's GEMM dispatch stamps ev[2 i], ev[2 i + 1]
  auto stamp = [&](int site) {
    return ev ? qa_time_next_launch(ctx, ev[2 * site], ev[2 * site + 1]) : QA_OK;
  };
  // Each projection pulls the next one's weights toward the caches while it
  // runs (the last down pulls the next layer's qkv weights).
  auto next_w = [&](const Buffer& b) { return qa_prefetch_hint(ctx, b.ptr, b.bytes); };
  // 3. qkv:  normed x qkv_w^T  (src/decoder.rs:1321-1327)
  if (int rc = stamp(0)) return rc;
  if (int rc = next_w(l.o_w)) return rc;
  if (int rc = gemm(ctx, dtype, normed.ptr, l.qkv_w.ptr, qkv.ptr, s_rows, qkv_n, hs, qkv_n, 0, 0,
                    0, 1, false))
    return rc;
  // 8. o + residual:  h += attn_flat x o_w^T  (src/decoder.rs:1602-1608)
  if (int rc = stamp(1)) return rc;
  if (int rc = next_w(l.gu_w)) return rc;
  if (int rc = gemm(ctx, dtype, attn.ptr, l.o_w.ptr, h.ptr, s_rows, hs, q_dim, hs, 0, 0, 0, 1,
                    true))
    return rc;
  // 10. gate|up GEMM + silu_mul_split, one kernel  (src/decoder.rs:1628-1650)
  if (int rc = stamp(2)) return rc;
  if (int rc = next_w(l.dp_w)) return rc;
  if (int rc = gemm(ctx, dtype, norm2.ptr, l.gu_w.ptr, act.ptr, s_rows, 2 * (int64_t)inter, hs,
                    inter, 0, 0, 0, 1, false, QA_EPI_SILU_MUL))
    return rc;
  // down + residual:  h += act x dp_w^T  (src/decoder.rs:1652-1657)
  if (int rc = stamp(3)) return rc;
  if (li + 1 < layers)
    if (int rc = next_w(L[(size_t)li + 1].qkv_w)) return rc;
  if (int rc = gemm(ctx, dtype, act.ptr, l.dp_w.ptr, h.ptr, s_rows, hs, inter, hs, 0, 0, 0, 1,
                    true))
    return rc;
  return QA_OK;
}

int TextDecoderLinears::prefill_linears(int rows) {
  if (rows < 0 || rows > max_rows) return QA_EINVAL;
  for (int li = 0; li < layers; ++li)
    if (int rc = layer(li, rows)) return rc;
  return QA_OK;
}

int TextDecoderLinears::read(int which, int rows, uint16_t* host) {
  if (rows < 0 || rows > max_rows) return QA_EINVAL;
  const int64_t r = rows;
  switch (which) {
    case 0: return qa_download(ctx, host, h.ptr, 0, elems_bytes(r * hidden));
    case 1: return qa_download(ctx, host, qkv.ptr, 0, elems_bytes(r * (q_dim + 2 * kv_dim)));
    case 2: return qa_download(ctx, host, act.ptr, 0, elems_bytes(r * inter));
    default: return QA_EINVAL;
  }
}

// ------------------------------------------------------------------------
AudioEncoderLinears::AudioEncoderLinears(qa_ctx* c, int dt, int nl, int dm, int ff, int ck,
                                         int mr)
    : ctx(c), dtype(dt), layers(nl), d_model(dm), ffn(ff), conv_k(ck), max_rows(mr),
      L((size_t)nl) {}

AudioEncoderLinears::~AudioEncoderLinears() {
  for (auto& l : L)
    for (Linear* x : {&l.qkv, &l.o, &l.fc1, &l.fc2}) {
      release(ctx, &x->w);
      release(ctx, &x->b);
    }
  release(ctx, &conv_w.w);
  release(ctx, &conv_w.b);
  for (Buffer* b : {&col, &normed, &attn, &norm2, &h, &conv_out, &qkv, &act}) release(ctx, b);
}

int AudioEncoderLinears::init() {
  const int64_t r = max_rows;
  if (int rc = alloc(ctx, elems_bytes(r * align_up(conv_k, 8)), &col)) return rc;
  for (Buffer* b : {&normed, &attn, &norm2, &h, &conv_out})
    if (int rc = alloc(ctx, elems_bytes(r * d_model), b)) return rc;
  if (int rc = alloc(ctx, elems_bytes(r * 3 * d_model), &qkv)) return rc;
  return alloc(ctx, elems_bytes(r * ffn), &act);
}

int AudioEncoderLinears::load_layer(int li, const uint16_t* qkv_w, const uint16_t* qkv_b,
                                    const uint16_t* o_w, const uint16_t* o_b,
                                    const uint16_t* fc1_w, const uint16_t* fc1_b,
                                    const uint16_t* fc2_w, const uint16_t* fc2_b) {
  if (li < 0 || li >= layers) return QA_EINVAL;
  Layer& l = L[(size_t)li];
  const int64_t d = d_model;
  if (int rc = load_linear(ctx, qkv_w, qkv_b, 3 * d, d, &l.qkv)) return rc;
  if (int rc = load_linear(ctx, o_w, o_b, d, d, &l.o)) return rc;
  if (int rc = load_linear(ctx, fc1_w, fc1_b, ffn, d, &l.fc1)) return rc;
  return load_linear(ctx, fc2_w, fc2_b, d, ffn, &l.fc2);
}

int AudioEncoderLinears::load_conv(const uint16_t* w, const uint16_t* b) {
  return load_linear(ctx, w, b, d_model, conv_k, &conv_w);
}

int AudioEncoderLinears::set_inputs(int rows, const uint16_t* c, const uint16_t* n1,
                                    const uint16_t* at, const uint16_t* n2, const uint16_t* hh) {
  if (rows < 0 || rows > max_rows) return QA_EINVAL;
  const int64_t r = rows, kp = align_up(conv_k, 8);
  if (c) {
    std::vector<uint16_t> cp((size_t)(r * kp), 0);
    for (int64_t i = 0; i < r; ++i)
      memcpy(&cp[(size_t)(i * kp)], c + i * conv_k, elems_bytes(conv_k));
    if (int rc = qa_upload(ctx, col.ptr, 0, cp.data(), cp.size() * 2)) return rc;
  }
  if (n1) if (int rc = qa_upload(ctx, normed.ptr, 0, n1, elems_bytes(r * d_model))) return rc;
  if (at) if (int rc = qa_upload(ctx, attn.ptr, 0, at, elems_bytes(r * d_model))) return rc;
  if (n2) if (int rc = qa_upload(ctx, norm2.ptr, 0, n2, elems_bytes(r * d_model))) return rc;
  if (hh) if (int rc = qa_upload(ctx, h.ptr, 0, hh, elems_bytes(r * d_model))) return rc;
  return QA_OK;
}

int AudioEncoderLinears::conv(int rows) {
  // im2col GEMM + bias + GELU, token-major (src/audio_encoder.rs:416-447);
  // it pulls layer 0's qkv weights toward the caches
  if (!L.empty())
    if (int rc = qa_prefetch_hint(ctx, L[0].qkv.w.ptr, L[0].qkv.w.bytes)) return rc;
  return gemm(ctx, dtype, col.ptr, conv_w.w.ptr, conv_out.ptr, rows, conv_w.n_pad,
              conv_w.k_pad, d_model, 0, 0, 0, 1, false, QA_EPI_GELU, conv_w.b.ptr);
}

int AudioEncoderLinears::layer(int li, int rows, hipEvent_t* ev) {
  const Layer& l = L[(size_t)li];
  const int64_t d = d_model;
  // per-site kernel times: the site's GEMM dispatch stamps ev[2 i], ev[2 i + 1]
  auto stamp = [&](int site) {
    return ev ? qa_time_next_launch(ctx, ev[2 * site], ev[2 * site + 1]) : QA_OK;
  };
  // each projection pulls the next one's weights toward the caches (the
  // last fc2 pulls the next layer's qkv weights)
  auto next_w = [&](const Linear& x) { return qa_prefetch_hint(ctx, x.w.ptr, x.w.bytes); };
  // qkv + bias  (src/audio_encoder_gpu.rs:1414-1419)
  if (int rc = stamp(0)) return rc;
  if (int rc = next_w(l.o)) return rc;
  if (int rc = gemm(ctx, dtype, normed.ptr, l.qkv.w.ptr, qkv.ptr, rows, l.qkv.n_pad, d,
                    3 * d, 0, 0, 0, 1, false, 0, l.qkv.b.ptr))
    return rc;
  // out_proj + bias, onto the residual  (src/audio_encoder_gpu.rs:1579-1581)
  if (int rc = stamp(1)) return rc;
  if (int rc = next_w(l.fc1)) return rc;
  if (int rc = gemm(ctx, dtype, attn.ptr, l.o.w.ptr, h.ptr, rows, l.o.n_pad, d, d, 0, 0, 0, 1,
                    true, 0, l.o.b.ptr))
    return rc;
  // fc1 + bias + GELU, one kernel  (src/audio_encoder_gpu.rs:1594-1602)
  if (int rc = stamp(2)) return rc;
  if (int rc = next_w(l.fc2)) return rc;
  if (int rc = gemm(ctx, dtype, norm2.ptr, l.fc1.w.ptr, act.ptr, rows, l.fc1.n_pad, d, ffn, 0,
                    0, 0, 1, false, QA_EPI_GELU, l.fc1.b.ptr))
    return rc;
  // fc2 + bias, onto the residual  (src/audio_encoder_gpu.rs:1603-1605)
  if (int rc = stamp(3)) return rc;
  if (li + 1 < layers)
    if (int rc = next_w(L[(size_t)li + 1].qkv)) return rc;
  if (int rc = gemm(ctx, dtype, act.ptr, l.fc2.w.ptr, h.ptr, rows, l.fc2.n_pad, ffn, d, 0, 0, 0,
                    1, true, 0, l.fc2.b.ptr))
    return rc;
  return QA_OK;
}

int AudioEncoderLinears::forward_linears(int rows) {
  if (rows < 0 || rows > max_rows) return QA_EINVAL;
  if (int rc = conv(rows)) return rc;
  for (int li = 0; li < layers; ++li)
    if (int rc = layer(li, rows)) return rc;
  return QA_OK;
}

int AudioEncoderLinears::read(int which, int rows, uint16_t* host) {
  if (rows < 0 || rows > max_rows) return QA_EINVAL;
  const int64_t r = rows;
  switch (which) {
    case 0: return qa_download(ctx, host, h.ptr, 0, elems_bytes(r * d_model));
    case 1: return qa_download(ctx, host, conv_out.ptr, 0, elems_bytes(r * d_model));
    case 2: return qa_download(ctx, host, qkv.ptr, 0, elems_bytes(r * 3 * d_model));
    case 3: return qa_download(ctx, host, act.ptr, 0, elems_bytes(r * ffn));
    default: return QA_EINVAL;
  }
}

}  // namespace qa_host

// ------------------------------------------------------------------------
// C surface
using namespace qa_host;

struct qah_decoder {
  TextDecoderLinears* d;
};
struct qah_encoder {
  AudioEncoderLinears* e;
};

namespace {

__global__ void copy_kernel(const uint4* __restrict__ src, uint4* __restrict__ dst, size_t n) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (size_t)gridDim.x * blockDim.x)
    dst[i] = src[i];
}

__device__ uint64_t mix64(uint64_t z) {  // SplitMix64's finaliser
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}

// Input i of the SiLU.up check: special values for the first 4096, then
// random f32 bit patterns (every third) and values in [-16, 16) x {1, 0.01}.
__device__ void silu_check_input(uint64_t seed, int64_t i, float* g, float* u) {
  const float sp[20] = {0.0f, -0.0f, 1e-8f, -1e-8f, 6e-8f, -6e-8f, 1e-5f, -1e-5f, 65504.f,
                        -65504.f, 70000.f, -70000.f, 1e30f, -1e30f, 88.f, -88.f, 20.f, -20.f,
                        0.5f, -0.5f};
  const uint64_t r = mix64(seed + 0x9e3779b97f4a7c15ull * (uint64_t)(i + 1));
  if (i < 4096) {
    *g = sp[i % 20];
    *u = sp[(i / 20) % 20];
  } else if (i % 3 == 0) {
    *g = __uint_as_float((uint32_t)r);
    *u = __uint_as_float((uint32_t)(r >> 32));
  } else {
    const float sg = (i % 7) ? 1.0f : 0.01f;
    *g = ((float)(r & 0xffffff) / 8388608.0f - 1.0f) * 16.0f * sg;
    *u = ((float)((r >> 24) & 0xffffff) / 8388608.0f - 1.0f) * 8.0f;
  }
}

// silu_mul_f16x2 against silu_mul in f32 followed by a separate f16 rounding
// (the empty asm keeps the compiler from fusing the two): outputs that differ,
// other than two NaNs, are counted.
__global__ void silu_check_kernel(uint64_t seed, int64_t pairs, unsigned long long* bad) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= pairs) return;
  float g[2], u[2];
  silu_check_input(seed, 2 * i, &g[0], &u[0]);
  silu_check_input(seed, 2 * i + 1, &g[1], &u[1]);
  const uint32_t got = qa::silu_mul_f16x2(g[0], g[1], u[0], u[1]);
  unsigned n = 0;
  for (int e = 0; e < 2; ++e) {
    float v = qa::silu_mul((float)(_Float16)g[e], (float)(_Float16)u[e]);
    asm volatile("" : "+v"(v));
    const uint32_t want = __builtin_bit_cast(uint16_t, (_Float16)v);
    const uint32_t have = (got >> (16 * e)) & 0xffffu;
    const bool nans = (want & 0x7c00u) == 0x7c00u && (want & 0x3ffu) &&
                      (have & 0x7c00u) == 0x7c00u && (have & 0x3ffu);
    n += want != have && !nans;
  }
  if (n) atomicAdd(bad, (unsigned long long)n);
}

}  // namespace

extern "C" {

void qah_synth_normal_h16(uint64_t seed, uint64_t tensor_id, float mean, float std_dev, int dtype,
                          uint16_t* out, size_t n) {
  const uint64_t base = stream_base(seed, tensor_id);
  parallel_for(n, [&](size_t lo, size_t hi) {
    for (size_t i = lo; i < hi; ++i)
      out[i] = narrow16((float)(mean + std_dev * normal_at(base, i)), dtype);
  });
}

void qah_synth_normal_f32(uint64_t seed, uint64_t tensor_id, float mean, float std_dev, float* out,
                          size_t n) {
  const uint64_t base = stream_base(seed, tensor_id);
  parallel_for(n, [&](size_t lo, size_t hi) {
    for (size_t i = lo; i < hi; ++i) out[i] = (float)(mean + std_dev * normal_at(base, i));
  });
}

void qah_narrow_f32(const float* src, uint16_t* dst, size_t n, int dtype) {
  parallel_for(n, [&](size_t lo, size_t hi) {
    for (size_t i = lo; i < hi; ++i) dst[i] = narrow16(src[i], dtype);
  });
}

void qah_concat_rows(const uint16_t* const* parts, const int64_t* rows, int nparts, int64_t cols,
                     uint16_t* dst) {
  size_t off = 0;
  for (int p = 0; p < nparts; ++p) {
    const size_t n = (size_t)(rows[p] * cols);
    memcpy(dst + off, parts[p], n * 2);
    off += n;
  }
}

int qah_decoder_create(qa_ctx* ctx, int dtype, int layers, int hidden, int q_dim, int kv_dim,
                       int inter, int max_rows, qah_decoder** out) {
  if (!ctx || !out || layers <= 0 || hidden <= 0 || max_rows <= 0) return QA_EINVAL;
  auto* d = new TextDecoderLinears(ctx, dtype, layers, hidden, q_dim, kv_dim, inter, max_rows);
  if (int rc = d->init()) {
    delete d;
    return rc;
  }
  *out = new qah_decoder{d};
  return QA_OK;
}

int qah_decoder_load_layer(qah_decoder* d, int li, const uint16_t* q, const uint16_t* k,
                           const uint16_t* v, const uint16_t* o, const uint16_t* gate,
                           const uint16_t* up, const uint16_t* down) {
  return d ? d->d->load_layer(li, q, k, v, o, gate, up, down) : QA_EINVAL;
}

int qah_decoder_set_inputs(qah_decoder* d, int rows, const uint16_t* normed, const uint16_t* attn,
                           const uint16_t* norm2, const uint16_t* h) {
  return d ? d->d->set_inputs(rows, normed, attn, norm2, h) : QA_EINVAL;
}

int qah_decoder_prefill_linears(qah_decoder* d, int rows) {
  return d ? d->d->prefill_linears(rows) : QA_EINVAL;
}

int qah_decoder_layer(qah_decoder* d, int li, int rows) {
  if (!d || li < 0 || li >= d->d->layers || rows < 0 || rows > d->d->max_rows) return QA_EINVAL;
  return d->d->layer(li, rows);
}

int qah_decoder_read(qah_decoder* d, int which, int rows, uint16_t* host) {
  return d ? d->d->read(which, rows, host) : QA_EINVAL;
}

int qah_decoder_time(qah_decoder* d, int rows, int warmup, int steps, int use_graph,
                     double* ms_per_step, double* wall_ms_per_step) {
  if (!d || !ms_per_step) return QA_EINVAL;
  return time_steps(d->d->ctx, warmup, steps, use_graph,
                    [&] { return d->d->prefill_linears(rows); }, ms_per_step, wall_ms_per_step);
}

int qah_decoder_profile_sites(qah_decoder* d, int rows, int steps, double* site_ms) {
  if (!d || !site_ms || steps <= 0) return QA_EINVAL;
  TextDecoderLinears& D = *d->d;
  std::vector<hipEvent_t> ev((size_t)D.layers * 8);
  for (auto& e : ev) (void)hipEventCreate(&e);
  double acc[4] = {0, 0, 0, 0};
  int rc = QA_OK;
  for (int s = 0; s < steps && rc == QA_OK; ++s) {
    for (int li = 0; li < D.layers && rc == QA_OK; ++li) rc = D.layer(li, rows, &ev[(size_t)li * 8]);
    if (rc == QA_OK) rc = qa_sync(D.ctx);
    for (int li = 0; li < D.layers && rc == QA_OK; ++li)
      for (int i = 0; i < 4; ++i) {
        float t = 0.f;
        (void)hipEventElapsedTime(&t, ev[(size_t)li * 8 + 2 * i], ev[(size_t)li * 8 + 2 * i + 1]);
        acc[i] += t;
      }
  }
  for (auto& e : ev) (void)hipEventDestroy(e);
  for (int i = 0; i < 4; ++i) site_ms[i] = acc[i] / ((double)steps * D.layers);
  return rc;
}

void qah_decoder_destroy(qah_decoder* d) {
  if (!d) return;
  delete d->d;
  delete d;
}

int qah_encoder_create(qa_ctx* ctx, int dtype, int layers, int d_model, int ffn, int conv_k,
                       int max_rows, qah_encoder** out) {
  if (!ctx || !out || layers <= 0 || d_model <= 0 || max_rows <= 0) return QA_EINVAL;
  auto* e = new AudioEncoderLinears(ctx, dtype, layers, d_model, ffn, conv_k, max_rows);
  if (int rc = e->init()) {
    delete e;
    return rc;
  }
  *out = new qah_encoder{e};
  return QA_OK;
}

int qah_encoder_load_layer(qah_encoder* e, int li, const uint16_t* qkv_w, const uint16_t* qkv_b,
                           const uint16_t* o_w, const uint16_t* o_b, const uint16_t* fc1_w,
                           const uint16_t* fc1_b, const uint16_t* fc2_w, const uint16_t* fc2_b) {
  return e ? e->e->load_layer(li, qkv_w, qkv_b, o_w, o_b, fc1_w, fc1_b, fc2_w, fc2_b)
           : QA_EINVAL;
}

int qah_encoder_load_conv(qah_encoder* e, const uint16_t* w, const uint16_t* b) {
  return e ? e->e->load_conv(w, b) : QA_EINVAL;
}

int qah_encoder_set_inputs(qah_encoder* e, int rows, const uint16_t* col, const uint16_t* normed,
                           const uint16_t* attn, const uint16_t* norm2, const uint16_t* h) {
  return e ? e->e->set_inputs(rows, col, normed, attn, norm2, h) : QA_EINVAL;
}

int qah_encoder_forward_linears(qah_encoder* e, int rows) {
  return e ? e->e->forward_linears(rows) : QA_EINVAL;
}

int qah_encoder_read(qah_encoder* e, int which, int rows, uint16_t* host) {
  return e ? e->e->read(which, rows, host) : QA_EINVAL;
}

int qah_encoder_time(qah_encoder* e, int rows, int warmup, int steps, int use_graph,
                     double* ms_per_step, double* wall_ms_per_step) {
  if (!e || !ms_per_step) return QA_EINVAL;
  return time_steps(e->e->ctx, warmup, steps, use_graph,
                    [&] { return e->e->forward_linears(rows); }, ms_per_step, wall_ms_per_step);
}

int qah_encoder_profile_sites(qah_encoder* e, int rows, int steps, double* site_ms) {
  if (!e || !site_ms || steps <= 0) return QA_EINVAL;
  AudioEncoderLinears& E = *e->e;
  std::vector<hipEvent_t> ev((size_t)E.layers * 8 + 2);
  for (auto& x : ev) (void)hipEventCreate(&x);
  double acc[5] = {0, 0, 0, 0, 0};
  int rc = QA_OK;
  for (int st = 0; st < steps && rc == QA_OK; ++st) {
    rc = qa_time_next_launch(E.ctx, ev[(size_t)E.layers * 8], ev[(size_t)E.layers * 8 + 1]);
    if (rc == QA_OK) rc = E.conv(rows);
    for (int li = 0; li < E.layers && rc == QA_OK; ++li) rc = E.layer(li, rows, &ev[(size_t)li * 8]);
    if (rc == QA_OK) rc = qa_sync(E.ctx);
    float t = 0.f;
    (void)hipEventElapsedTime(&t, ev[(size_t)E.layers * 8], ev[(size_t)E.layers * 8 + 1]);
    acc[0] += t * E.layers;  // averaged per layer below, like the others
    for (int li = 0; li < E.layers && rc == QA_OK; ++li)
      for (int i = 0; i < 4; ++i) {
        (void)hipEventElapsedTime(&t, ev[(size_t)li * 8 + 2 * i], ev[(size_t)li * 8 + 2 * i + 1]);
        acc[i + 1] += t;
      }
  }
  for (auto& x : ev) (void)hipEventDestroy(x);
  for (int i = 0; i < 5; ++i) site_ms[i] = acc[i] / ((double)steps * E.layers);
  return rc;
}

void qah_encoder_destroy(qah_encoder* e) {
  if (!e) return;
  delete e->e;
  delete e;
}

int qah_time_linear(qa_ctx* ctx, const qa_linear_desc* desc, int warmup, int iters,
                    double* ms_per_launch) {
  if (!ctx || !desc || !ms_per_launch) return QA_EINVAL;
  return time_steps(ctx, warmup, iters, 0, [&] { return qa_linear(ctx, desc); }, ms_per_launch);
}

int qah_time_linears_each(qa_ctx* ctx, const qa_linear_desc* descs, int ndesc, int warmup,
                          int iters, float* ms_each) {
  if (!ctx || !descs || ndesc <= 0 || warmup < 0 || iters <= 0 || !ms_each) return QA_EINVAL;
  hipStream_t s = (hipStream_t)qa_ctx_stream(ctx);
  for (int i = 0; i < warmup; ++i)
    if (int rc = qa_linear(ctx, &descs[i % ndesc])) return rc;
  std::vector<hipEvent_t> ev((size_t)iters + 1, nullptr);
  int rc = QA_OK;
  for (auto& e : ev)
    if (rc == QA_OK && hipEventCreate(&e) != hipSuccess) rc = QA_EDEVICE;
  if (rc == QA_OK) rc = qa_sync(ctx);
  for (int i = 0; i < iters && rc == QA_OK; ++i) {
    rc = hip_status(hipEventRecord(ev[(size_t)i], s));
    if (rc == QA_OK) rc = qa_linear(ctx, &descs[i % ndesc]);
  }
  if (rc == QA_OK) rc = hip_status(hipEventRecord(ev[(size_t)iters], s));
  if (int rs = qa_sync(ctx); rc == QA_OK) rc = rs;
  for (int i = 0; i < iters && rc == QA_OK; ++i)
    rc = hip_status(hipEventElapsedTime(&ms_each[i], ev[(size_t)i], ev[(size_t)i + 1]));
  for (auto& e : ev)
    if (e) (void)hipEventDestroy(e);
  return rc;
}

int qah_time_linears_stamped(qa_ctx* ctx, const qa_linear_desc* descs, int ndesc, int warmup,
                             int iters, float* ms_each) {
  if (!ctx || !descs || ndesc <= 0 || warmup < 0 || iters <= 0 || !ms_each) return QA_EINVAL;
  for (int i = 0; i < warmup; ++i)
    if (int rc = qa_linear(ctx, &descs[i % ndesc])) return rc;
  std::vector<hipEvent_t> ev(2 * (size_t)iters, nullptr);
  int rc = QA_OK;
  for (auto& e : ev)
    if (rc == QA_OK && hipEventCreate(&e) != hipSuccess) rc = QA_EDEVICE;
  if (rc == QA_OK) rc = qa_sync(ctx);
  for (int i = 0; i < iters && rc == QA_OK; ++i) {
    rc = qa_time_next_launch(ctx, ev[2 * (size_t)i], ev[2 * (size_t)i + 1]);
    if (rc == QA_OK) rc = qa_linear(ctx, &descs[i % ndesc]);
  }
  if (int rs = qa_sync(ctx); rc == QA_OK) rc = rs;
  for (int i = 0; i < iters && rc == QA_OK; ++i)
    rc = hip_status(hipEventElapsedTime(&ms_each[i], ev[2 * (size_t)i], ev[2 * (size_t)i + 1]));
  for (auto& e : ev)
    if (e) (void)hipEventDestroy(e);
  return rc;
}

int qah_check_silu_f16x2(qa_ctx* ctx, int64_t pairs, uint64_t seed, int64_t* mismatches) {
  if (!ctx || pairs <= 0 || pairs > ((int64_t)1 << 31) || !mismatches) return QA_EINVAL;
  Buffer cnt;
  int rc = alloc(ctx, sizeof(unsigned long long), &cnt);
  hipStream_t s = (hipStream_t)qa_ctx_stream(ctx);
  unsigned long long host = 0;
  if (rc == QA_OK) rc = qa_upload(ctx, cnt.ptr, 0, &host, sizeof host);
  if (rc == QA_OK) {
    hipLaunchKernelGGL(silu_check_kernel, dim3((unsigned)((pairs + 255) / 256)), dim3(256), 0, s,
                       seed, pairs, (unsigned long long*)cnt.ptr);
    rc = hip_status(hipGetLastError());
  }
  if (rc == QA_OK) rc = qa_sync(ctx);
  if (rc == QA_OK) rc = qa_download(ctx, &host, cnt.ptr, 0, sizeof host);
  release(ctx, &cnt);
  if (rc == QA_OK) *mismatches = (int64_t)host;
  return rc;
}

int qah_copy_calibration(qa_ctx* ctx, size_t bytes, int reps) {
  if (!ctx || bytes % 16 || reps <= 0) return QA_EINVAL;
  Buffer a, b;
  int rc = alloc(ctx, bytes, &a);
  if (rc == QA_OK) rc = alloc(ctx, bytes, &b);
  hipStream_t s = (hipStream_t)qa_ctx_stream(ctx);
  if (rc == QA_OK) rc = hip_status(hipMemsetAsync(a.ptr, 1, bytes, s));
  if (rc == QA_OK) rc = qa_sync(ctx);
  for (int i = 0; i < reps && rc == QA_OK; ++i) {
    hipLaunchKernelGGL(copy_kernel, dim3(8192), dim3(256), 0, s, (const uint4*)a.ptr, (uint4*)b.ptr,
                       bytes / 16);
    rc = hip_status(hipGetLastError());
  }
  if (rc == QA_OK) rc = qa_sync(ctx);
  release(ctx, &a);
  release(ctx, &b);
  return rc;
}

}  // extern "C"
