// decoder_prefill.cpp -- C++ host mirror of WgpuTextDecoder::prefill's layer
// loop (src/decoder.rs:1305-1657) on the C ABI: per layer
//   1. rms_norm(h, iln) -> normed            src/decoder.rs:1305-1319
//   2. qkv = normed x qkv_w^T                 :1321-1327
//   3. q/k head norm + RoPE, K/V cache write  :1329-1350
//   4. causal GQA attention -> attn           :1346-1600
//   5. h += attn x o_w^T                      :1602-1608
//   6. rms_norm(h, pln) -> norm2              :1610-1626
//   7. act = silu(gate) * up (gate|up GEMM)   :1628-1650
//   8. h += act x dp_w^T                      :1652-1657
// The reference pads rows to mp = 128 and slabs long key ranges
// (src/decoder.rs:900-950); the kernels here take exact row counts and any
// key range, so neither is needed.
#include "decoder_prefill.hpp"

#include <algorithm>
#include <cstring>

#include "handles.hpp"
#include "qa_host.h"
#include "timing.hpp"

namespace qa_host {

namespace {
int64_t round_up(int64_t v, int64_t a) { return (v + a - 1) / a * a; }
}  // namespace

TextDecoder::TextDecoder(qa_ctx* c, int dt, int nl, int hs, int nq, int nkv, int d, int it, int mr,
                         float e)
    : ctx(c), dtype(dt), layers(nl), hidden(hs), nqh(nq), nkvh(nkv), hd(d), inter(it),
      max_rows(mr), eps(e), lin(c, dt, nl, hs, nq * d, nkv * d, it, mr), L((size_t)nl) {}

TextDecoder::~TextDecoder() {
  for (auto& l : L)
    for (Buffer* b : {&l.iln, &l.pln, &l.qn, &l.kn, &l.k_cache, &l.v_cache}) release(ctx, b);
  for (Buffer* b : {&q_heads, &cos, &sin}) release(ctx, b);
}

// The KV cache holds max_rows keys rounded up to the attention's 64-key block.
static int64_t cache_cap(int max_rows) { return round_up(max_rows, 64); }

int TextDecoder::init() {
  if (int rc = lin.init()) return rc;
  const int64_t cap = cache_cap(max_rows);
  for (auto& l : L) {
    if (int rc = alloc(ctx, (size_t)hidden * 4, &l.iln)) return rc;
    if (int rc = alloc(ctx, (size_t)hidden * 4, &l.pln)) return rc;
    if (int rc = alloc(ctx, (size_t)hd * 4, &l.qn)) return rc;
    if (int rc = alloc(ctx, (size_t)hd * 4, &l.kn)) return rc;
    // qa_alloc zero-fills: cache entries past the written keys are finite
    if (int rc = alloc(ctx, (size_t)(nkvh * cap * hd) * 2, &l.k_cache)) return rc;
    if (int rc = alloc(ctx, (size_t)(nkvh * cap * hd) * 2, &l.v_cache)) return rc;
  }
  return alloc(ctx, (size_t)nqh * max_rows * hd * 2, &q_heads);
}

int TextDecoder::load_layer(int li, const uint16_t* q, const uint16_t* k, const uint16_t* v,
                            const uint16_t* o, const uint16_t* gate, const uint16_t* up,
                            const uint16_t* down, const float* iln, const float* pln,
                            const float* qn, const float* kn) {
  if (li < 0 || li >= layers || !iln || !pln || !qn || !kn) return QA_EINVAL;
  if (int rc = lin.load_layer(li, q, k, v, o, gate, up, down)) return rc;
  Layer& l = L[(size_t)li];
  if (int rc = qa_upload(ctx, l.iln.ptr, 0, iln, (size_t)hidden * 4)) return rc;
  if (int rc = qa_upload(ctx, l.pln.ptr, 0, pln, (size_t)hidden * 4)) return rc;
  if (int rc = qa_upload(ctx, l.qn.ptr, 0, qn, (size_t)hd * 4)) return rc;
  return qa_upload(ctx, l.kn.ptr, 0, kn, (size_t)hd * 4);
}

int TextDecoder::set_rope(const float* c, const float* s, int positions) {
  if (!c || !s || positions <= 0) return QA_EINVAL;
  release(ctx, &cos);
  release(ctx, &sin);
  const size_t bytes = (size_t)positions * hd * 4;
  if (int rc = alloc(ctx, bytes, &cos)) return rc;
  if (int rc = alloc(ctx, bytes, &sin)) return rc;
  if (int rc = qa_upload(ctx, cos.ptr, 0, c, bytes)) return rc;
  if (int rc = qa_upload(ctx, sin.ptr, 0, s, bytes)) return rc;
  rope_positions = positions;
  return QA_OK;
}

int TextDecoder::set_hidden(int rows, const uint16_t* h) {
  if (rows < 0 || rows > max_rows || !h) return QA_EINVAL;
  return qa_upload(ctx, lin.h.ptr, 0, h, (size_t)rows * hidden * 2);
}

int TextDecoder::layer(int li, int rows, hipEvent_t* ev) {
  if (li < 0 || li >= layers || rows < 0 || rows > max_rows) return QA_EINVAL;
  if (rows > rope_positions) return QA_EINVAL;  // the RoPE table must cover every position
  const Layer& l = L[(size_t)li];
  const TextDecoderLinears::Layer& w = lin.L[(size_t)li];
  hipStream_t st = (hipStream_t)qa_ctx_stream(ctx);
  const int64_t r = rows, hs = hidden, qd = (int64_t)nqh * hd, kvd = (int64_t)nkvh * hd;
  const int64_t qkv_n = qd + 2 * kvd, cap = cache_cap(max_rows);
  int op = 0;
  auto mark = [&](int i) {
    if (ev) (void)hipEventRecord(ev[2 * op + i], st);
  };
  auto rms = [&](const Buffer& wt, void* out) {
    qa_rms_norm_desc d{};
    d.dtype = (uint32_t)dtype;
    d.rows = r;
    d.n = hs;
    d.x = lin.h.ptr;
    d.ldx = hs;
    d.w = (const float*)wt.ptr;
    d.y = out;
    d.ldy = hs;
    d.eps = eps;
    return qa_rms_norm(ctx, &d);
  };
  int rc = QA_OK;
  auto run = [&](auto&& f) {
    if (rc) return;
    mark(0);
    rc = f();
    mark(1);
    ++op;
  };
  // 1. input RMSNorm
  run([&] { return rms(l.iln, lin.normed.ptr); });
  // Each projection pulls the next one's weights toward the caches while it
  // runs (the down projection pulls the next layer's qkv weights).
  auto next_w = [&](const Buffer& b) { return qa_prefetch_hint(ctx, b.ptr, b.bytes); };
  // 2. fused qkv projection
  run([&] {
    if (int e = next_w(w.o_w)) return e;
    return gemm(ctx, dtype, lin.normed.ptr, w.qkv_w.ptr, lin.qkv.ptr, r, qkv_n, hs, qkv_n, 0, 0, 0,
                1, false);
  });
  // 3. q/k head norm + RoPE; K and V into this layer's cache at rows 0..
  run([&] {
    qa_qk_rope_desc d{};
    d.dtype = (uint32_t)dtype;
    d.rows = r;
    d.nqh = nqh;
    d.nkvh = nkvh;
    d.hd = hd;
    d.eps = eps;
    d.qkv = lin.qkv.ptr;
    d.ldqkv = qkv_n;
    d.qn_w = (const float*)l.qn.ptr;
    d.kn_w = (const float*)l.kn.ptr;
    d.cos = (const float*)cos.ptr;
    d.sin = (const float*)sin.ptr;
    d.pos0 = 0;
    d.q_out = q_heads.ptr;
    d.k_cache = l.k_cache.ptr;
    d.v_cache = l.v_cache.ptr;
    d.cap = cap;
    d.start = 0;
    return qa_qk_norm_rope(ctx, &d);
  });
  // 4. causal GQA attention over the cache
  run([&] {
    qa_attention_desc d{};
    d.dtype = (uint32_t)dtype;
    d.flags = attn_flags;
    d.rows = r;
    d.nqh = nqh;
    d.nkvh = nkvh;
    d.hd = hd;
    d.q = q_heads.ptr;
    d.k_cache = l.k_cache.ptr;
    d.v_cache = l.v_cache.ptr;
    d.cap = cap;
    d.q0 = 0;
    d.out = lin.attn.ptr;
    d.ldo = qd;
    return qa_attention_prefill(ctx, &d);
  });
  // 5. o projection + residual
  run([&] {
    if (int e = next_w(w.gu_w)) return e;
    return gemm(ctx, dtype, lin.attn.ptr, w.o_w.ptr, lin.h.ptr, r, hs, qd, hs, 0, 0, 0, 1, true);
  });
  // 6. post-attention RMSNorm
  run([&] { return rms(l.pln, lin.norm2.ptr); });
  // 7. gate|up + SiLU.up
  run([&] {
    if (int e = next_w(w.dp_w)) return e;
    return gemm(ctx, dtype, lin.norm2.ptr, w.gu_w.ptr, lin.act.ptr, r, 2 * (int64_t)inter, hs,
                inter, 0, 0, 0, 1, false, QA_EPI_SILU_MUL);
  });
  // 8. down projection + residual
  run([&] {
    if (li + 1 < layers)
      if (int e = next_w(lin.L[(size_t)li + 1].qkv_w)) return e;
    return gemm(ctx, dtype, lin.act.ptr, w.dp_w.ptr, lin.h.ptr, r, hs, inter, hs, 0, 0, 0, 1,
                true);
  });
  return rc;
}

int TextDecoder::prefill(int rows) {
  for (int li = 0; li < layers; ++li)
    if (int rc = layer(li, rows)) return rc;
  return QA_OK;
}

int TextDecoder::read(int which, int rows, uint16_t* host) {
  if (rows < 0 || rows > max_rows || !host) return QA_EINVAL;
  const int64_t r = rows;
  switch (which) {
    case 0: return qa_download(ctx, host, lin.h.ptr, 0, (size_t)(r * hidden) * 2);
    case 1: return qa_download(ctx, host, lin.attn.ptr, 0, (size_t)(r * nqh * hd) * 2);
    case 2:
      return qa_download(ctx, host, lin.qkv.ptr, 0, (size_t)(r * (nqh + 2 * nkvh) * hd) * 2);
    case 3: return qa_download(ctx, host, lin.act.ptr, 0, (size_t)(r * inter) * 2);
    case 4: return qa_download(ctx, host, lin.normed.ptr, 0, (size_t)(r * hidden) * 2);
    case 5: return qa_download(ctx, host, lin.norm2.ptr, 0, (size_t)(r * hidden) * 2);
    case 6: return qa_download(ctx, host, q_heads.ptr, 0, (size_t)(nqh * r * hd) * 2);
    case 7:
    case 8:
      return qa_download(ctx, host, (which == 7 ? L.back().k_cache : L.back().v_cache).ptr, 0,
                         (size_t)(nkvh * cache_cap(max_rows) * hd) * 2);
    default: return QA_EINVAL;
  }
}

}  // namespace qa_host

// ------------------------------------------------------------------------
// C surface
using namespace qa_host;


extern "C" {

int qah_tdec_create(qa_ctx* ctx, int dtype, int layers, int hidden, int nqh, int nkvh, int hd,
                    int inter, int max_rows, float eps, qah_tdec** out) {
  if (!ctx || !out || layers <= 0 || hidden <= 0 || max_rows <= 0 || nqh <= 0 || nkvh <= 0 ||
      hd <= 0 || inter <= 0)
    return QA_EINVAL;
  auto* d = new TextDecoder(ctx, dtype, layers, hidden, nqh, nkvh, hd, inter, max_rows, eps);
  if (int rc = d->init()) {
    delete d;
    return rc;
  }
  *out = new qah_tdec{d};
  return QA_OK;
}

int qah_tdec_load_layer(qah_tdec* t, int li, const uint16_t* q, const uint16_t* k,
                        const uint16_t* v, const uint16_t* o, const uint16_t* gate,
                        const uint16_t* up, const uint16_t* down, const float* iln,
                        const float* pln, const float* qn, const float* kn) {
  return t ? t->d->load_layer(li, q, k, v, o, gate, up, down, iln, pln, qn, kn) : QA_EINVAL;
}

int qah_tdec_set_rope(qah_tdec* t, const float* cos, const float* sin, int positions) {
  return t ? t->d->set_rope(cos, sin, positions) : QA_EINVAL;
}

int qah_tdec_set_attention_flags(qah_tdec* t, uint32_t flags) {
  if (!t) return QA_EINVAL;
  t->d->attn_flags = flags;
  return QA_OK;
}

int qah_tdec_set_hidden(qah_tdec* t, int rows, const uint16_t* h) {
  return t ? t->d->set_hidden(rows, h) : QA_EINVAL;
}

int qah_tdec_prefill(qah_tdec* t, int rows) { return t ? t->d->prefill(rows) : QA_EINVAL; }

int qah_tdec_read(qah_tdec* t, int which, int rows, uint16_t* host) {
  return t ? t->d->read(which, rows, host) : QA_EINVAL;
}

int qah_tdec_time(qah_tdec* t, int rows, int warmup, int steps, int use_graph, double* ms_per_step,
                  double* wall_ms_per_step) {
  if (!t || !ms_per_step) return QA_EINVAL;
  return time_steps(t->d->ctx, warmup, steps, use_graph, [&] { return t->d->prefill(rows); },
                    ms_per_step, wall_ms_per_step);
}

int qah_tdec_profile_ops(qah_tdec* t, int rows, int steps, double* op_ms) {
  if (!t || !op_ms || steps <= 0) return QA_EINVAL;
  TextDecoder& D = *t->d;
  std::vector<hipEvent_t> ev((size_t)D.layers * 16);
  for (auto& e : ev) (void)hipEventCreate(&e);
  double acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  int rc = QA_OK;
  for (int s = 0; s < steps && rc == QA_OK; ++s) {
    for (int li = 0; li < D.layers && rc == QA_OK; ++li)
      rc = D.layer(li, rows, &ev[(size_t)li * 16]);
    if (rc == QA_OK) rc = qa_sync(D.ctx);
    for (int li = 0; li < D.layers && rc == QA_OK; ++li)
      for (int i = 0; i < 8; ++i) {
        float ms = 0.f;
        (void)hipEventElapsedTime(&ms, ev[(size_t)li * 16 + 2 * i], ev[(size_t)li * 16 + 2 * i + 1]);
        acc[i] += ms;
      }
  }
  for (auto& e : ev) (void)hipEventDestroy(e);
  for (int i = 0; i < 8; ++i) op_ms[i] = acc[i] / ((double)steps * D.layers);
  return rc;
}

void qah_tdec_destroy(qah_tdec* t) {
  if (!t) return;
  delete t->d;
  delete t;
}

}  // extern "C"
