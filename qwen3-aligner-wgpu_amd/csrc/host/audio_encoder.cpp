// audio_encoder.cpp -- C++ host mirror of GpuAudioEncoder::encode
// (src/audio_encoder_gpu.rs:1060-1347) on the C ABI:
//   conv stem, 3 levels of 3x3 / stride 2 + bias + GELU    :1156-1201
//   conv_out (Linear + bias) and the sinusoidal position add  :1203-1226
//   per layer: LayerNorm -> qkv + bias -> windowed attention ->
//     out_proj + bias + residual -> LayerNorm -> fc1 + bias + GELU ->
//     fc2 + bias + residual                                  :1400-1607
//   ln_post -> proj1 + bias + GELU -> proj2 + bias           :1307-1325
// Layouts: the stem runs channel-last ([chunk][h][w][c]); the last level
// writes its rows token-major so conv_out reads [token][f][c] directly, its
// weight's columns permuted from the checkpoint's (c, f) order once at load
// (the reference's permute pass, :1795-1837, becomes that permutation).
// Every op rounds its output to the 16-bit format, as the reference's GPU
// tower does.
#include "audio_encoder.hpp"

#include <cmath>
#include <cstring>

#include "handles.hpp"
#include "qa_host.h"
#include "timing.hpp"

namespace qa_host {

namespace {

int conv_out_dim(int v) { return (v - 1) / 2 + 1; }

// feo (src/audio_encoder.rs:692-696): tokens from `frames` frames
int feo(int frames) { return conv_out_dim(conv_out_dim(conv_out_dim(frames))); }

int upload_f32(qa_ctx* ctx, const float* src, size_t n, Buffer* b) {
  if (int rc = alloc(ctx, n * 4, b)) return rc;
  return qa_upload(ctx, b->ptr, 0, src, n * 4);
}

// y = x W^T + bias (+ y with `acc`, GELU with `gelu`), rows m; the launch
// pulls `next`'s weights (the projection after it) toward the caches
int linear(qa_ctx* ctx, int dtype, const void* x, const Linear& l, void* y, int64_t m,
           bool acc, bool gelu, const Linear* next = nullptr) {
  if (next)
    if (int rc = qa_prefetch_hint(ctx, next->w.ptr, next->w.bytes)) return rc;
  qa_linear_desc d{};
  d.dtype = (uint32_t)dtype;
  d.flags = (acc ? QA_ACCUMULATE : 0u) | (gelu ? QA_EPI_GELU : 0u);
  d.m = m;
  d.n = l.n_pad;
  d.k = l.k_pad;
  d.lda = l.k_pad;
  d.ldb = l.k_pad;
  d.ldc = l.n_pad;
  d.a = x;
  d.w = l.w.ptr;
  d.c = y;
  d.bias = l.b.ptr;
  d.batch = 1;
  return qa_linear(ctx, &d);
}

}  // namespace

AudioEncoder::AudioEncoder(qa_ctx* c, int dt, int nl, int nm, int chunk, int cc, int dm, int heads,
                           int ff, int od, int wl, int mc)
    : ctx(c), dtype(dt), layers(nl), n_mels(nm), cs(chunk), c_conv(cc), d_model(dm), nh(heads),
      ffn(ff), out_dim(od), wlen(wl), max_chunks(mc), L((size_t)nl) {
  h1 = conv_out_dim(n_mels);
  w1 = conv_out_dim(cs);
  h2 = conv_out_dim(h1);
  w2 = conv_out_dim(w1);
  h3 = conv_out_dim(h2);
  w3 = conv_out_dim(w2);
}

AudioEncoder::~AudioEncoder() {
  for (auto& l : L) {
    for (Buffer* b : {&l.ln1_w, &l.ln1_b, &l.ln2_w, &l.ln2_b}) release(ctx, b);
    for (Linear* x : {&l.qkv, &l.o, &l.fc1, &l.fc2}) {
      release(ctx, &x->w);
      release(ctx, &x->b);
    }
  }
  for (Conv& c : conv) {
    release(ctx, &c.w);
    release(ctx, &c.b);
  }
  for (Linear* x : {&co, &p1, &p2}) {
    release(ctx, &x->w);
    release(ctx, &x->b);
  }
  for (Buffer* b : {&post_w, &post_b, &mel, &y1, &y2, &y3, &pe, &h, &normed, &qkv, &attn, &act,
                    &pact, &out})
    release(ctx, b);
}

int AudioEncoder::init() {
  const int64_t b = max_chunks, tok = (int64_t)max_chunks * w3;
  if (int rc = alloc(ctx, (size_t)(b * n_mels * cs) * 2, &mel)) return rc;
  if (int rc = alloc(ctx, (size_t)(b * h1 * w1 * c_conv) * 2, &y1)) return rc;
  if (int rc = alloc(ctx, (size_t)(b * h2 * w2 * c_conv) * 2, &y2)) return rc;
  if (int rc = alloc(ctx, (size_t)(b * h3 * w3 * c_conv) * 2, &y3)) return rc;
  if (int rc = alloc(ctx, (size_t)(tok * d_model) * 2, &h)) return rc;
  if (int rc = alloc(ctx, (size_t)(tok * d_model) * 2, &normed)) return rc;
  if (int rc = alloc(ctx, (size_t)(tok * 3 * d_model) * 2, &qkv)) return rc;
  if (int rc = alloc(ctx, (size_t)(tok * d_model) * 2, &attn)) return rc;
  if (int rc = alloc(ctx, (size_t)(tok * ffn) * 2, &act)) return rc;
  if (int rc = alloc(ctx, (size_t)(tok * d_model) * 2, &pact)) return rc;
  if (int rc = alloc(ctx, (size_t)(tok * out_dim) * 2, &out)) return rc;
  // position table rows 0..w3-1 (CpuConvStem::load, src/audio_encoder.rs:270-283):
  // pe[p][i] = sin(p e^(-i lt)), pe[p][half + i] = cos(...), lt = ln(1e4) / (half - 1)
  std::vector<float> t((size_t)w3 * d_model);
  const int half = d_model / 2;
  const double lt = std::log(10000.0) / ((double)half - 1.0);
  for (int p = 0; p < w3; ++p)
    for (int i = 0; i < half; ++i) {
      const double a = (double)p * std::exp(-(double)i * lt);
      t[(size_t)p * d_model + i] = (float)std::sin(a);
      t[(size_t)p * d_model + half + i] = (float)std::cos(a);
    }
  return upload_f32(ctx, t.data(), t.size(), &pe);
}

int AudioEncoder::load_conv(int level, const uint16_t* w, const uint16_t* b) {
  if (level < 0 || level > 2 || !w || !b) return QA_EINVAL;
  Conv& c = conv[level];
  c.c_in = level == 0 ? 1 : c_conv;
  const int64_t ldw = (9 * (int64_t)c.c_in + 7) / 8 * 8;
  std::vector<uint16_t> wp((size_t)(c_conv * ldw), 0);
  for (int oc = 0; oc < c_conv; ++oc)  // [c_out][c_in][3][3] -> [c_out][(kh*3 + kw)*c_in + ic]
    for (int ic = 0; ic < c.c_in; ++ic)
      for (int t = 0; t < 9; ++t)
        wp[(size_t)(oc * ldw + t * c.c_in + ic)] = w[((size_t)oc * c.c_in + ic) * 9 + t];
  if (int rc = alloc(ctx, wp.size() * 2, &c.w)) return rc;
  if (int rc = qa_upload(ctx, c.w.ptr, 0, wp.data(), wp.size() * 2)) return rc;
  if (int rc = alloc(ctx, (size_t)c_conv * 2, &c.b)) return rc;
  return qa_upload(ctx, c.b.ptr, 0, b, (size_t)c_conv * 2);
}

int AudioEncoder::load_conv_out(const uint16_t* w, const uint16_t* b) {
  if (!w || !b) return QA_EINVAL;
  const int64_t k = (int64_t)c_conv * h3;
  std::vector<uint16_t> wp((size_t)(d_model * k));
  for (int o = 0; o < d_model; ++o)  // column c * f_dim + f -> f * c_conv + c
    for (int c = 0; c < c_conv; ++c)
      for (int f = 0; f < h3; ++f)
        wp[(size_t)(o * k + f * c_conv + c)] = w[(size_t)(o * k + c * h3 + f)];
  return load_linear(ctx, wp.data(), b, d_model, k, &co);
}

int AudioEncoder::load_layer(int li, const float* ln1_w, const float* ln1_b,
                             const uint16_t* qkv_w, const uint16_t* qkv_b, const uint16_t* o_w,
                             const uint16_t* o_b, const float* ln2_w, const float* ln2_b,
                             const uint16_t* fc1_w, const uint16_t* fc1_b, const uint16_t* fc2_w,
                             const uint16_t* fc2_b) {
  if (li < 0 || li >= layers) return QA_EINVAL;
  Layer& l = L[(size_t)li];
  const size_t d = (size_t)d_model;
  if (int rc = upload_f32(ctx, ln1_w, d, &l.ln1_w)) return rc;
  if (int rc = upload_f32(ctx, ln1_b, d, &l.ln1_b)) return rc;
  if (int rc = upload_f32(ctx, ln2_w, d, &l.ln2_w)) return rc;
  if (int rc = upload_f32(ctx, ln2_b, d, &l.ln2_b)) return rc;
  if (int rc = load_linear(ctx, qkv_w, qkv_b, 3 * d_model, d_model, &l.qkv)) return rc;
  if (int rc = load_linear(ctx, o_w, o_b, d_model, d_model, &l.o)) return rc;
  if (int rc = load_linear(ctx, fc1_w, fc1_b, ffn, d_model, &l.fc1)) return rc;
  return load_linear(ctx, fc2_w, fc2_b, d_model, ffn, &l.fc2);
}

int AudioEncoder::load_post(const float* ln_w, const float* ln_b, const uint16_t* p1_w,
                            const uint16_t* p1_b, const uint16_t* p2_w, const uint16_t* p2_b) {
  if (int rc = upload_f32(ctx, ln_w, (size_t)d_model, &post_w)) return rc;
  if (int rc = upload_f32(ctx, ln_b, (size_t)d_model, &post_b)) return rc;
  if (int rc = load_linear(ctx, p1_w, p1_b, d_model, d_model, &p1)) return rc;
  return load_linear(ctx, p2_w, p2_b, out_dim, d_model, &p2);
}

int AudioEncoder::set_mel(int n_chunks, const uint16_t* m) {
  if (n_chunks <= 0 || n_chunks > max_chunks || !m) return QA_EINVAL;
  return qa_upload(ctx, mel.ptr, 0, m, (size_t)n_chunks * n_mels * cs * 2);
}

int64_t AudioEncoder::tokens(int n_chunks, int tail_frames) const {
  if (n_chunks <= 0) return 0;
  return tail_frames > 0 ? (int64_t)(n_chunks - 1) * w3 + feo(tail_frames)
                         : (int64_t)n_chunks * w3;
}

int AudioEncoder::stem(int n_chunks, hipEvent_t* ev) {
  if (n_chunks <= 0 || n_chunks > max_chunks) return QA_EINVAL;
  hipStream_t st = (hipStream_t)qa_ctx_stream(ctx);
  const Buffer* in[3] = {&mel, &y1, &y2};
  Buffer* outb[3] = {&y1, &y2, &y3};
  const int hs[3] = {n_mels, h1, h2}, ws[3] = {cs, w1, w2};
  for (int lv = 0; lv < 3; ++lv) {
    if (ev) (void)hipEventRecord(ev[lv], st);
    qa_conv_desc d{};
    d.dtype = (uint32_t)dtype;
    d.flags = QA_CONV_GELU | (lv == 2 ? QA_CONV_TOKEN_MAJOR : 0u);
    d.batch = n_chunks;
    d.h = hs[lv];
    d.w = ws[lv];
    d.c_in = conv[lv].c_in;
    d.c_out = c_conv;
    d.x = in[lv]->ptr;
    d.weight = conv[lv].w.ptr;
    d.bias = conv[lv].b.ptr;
    d.y = outb[lv]->ptr;
    if (int rc = qa_conv2d_3x3s2(ctx, &d)) return rc;
  }
  if (ev) (void)hipEventRecord(ev[3], st);
  return QA_OK;
}

int AudioEncoder::conv_out(int64_t n) {
  if (int rc = linear(ctx, dtype, y3.ptr, co, h.ptr, n, false, false, layers ? &L[0].qkv : &p1))
    return rc;
  qa_position_add_desc d{};
  d.dtype = (uint32_t)dtype;
  d.rows = n;
  d.n = d_model;
  d.y = h.ptr;
  d.ldy = d_model;
  d.table = (const float*)pe.ptr;
  d.period = w3;
  return qa_add_position_table(ctx, &d);
}

int AudioEncoder::layer(int li, int64_t n, hipEvent_t* ev) {
  if (li < 0 || li >= layers) return QA_EINVAL;
  const Layer& l = L[(size_t)li];
  hipStream_t st = (hipStream_t)qa_ctx_stream(ctx);
  int op = 0, rc = QA_OK;
  auto run = [&](auto&& f) {
    if (rc) return;
    if (ev) (void)hipEventRecord(ev[2 * op], st);
    rc = f();
    if (ev) (void)hipEventRecord(ev[2 * op + 1], st);
    ++op;
  };
  auto ln = [&](const Buffer& w, const Buffer& b) {
    qa_layer_norm_desc d{};
    d.dtype = (uint32_t)dtype;
    d.rows = n;
    d.n = d_model;
    d.x = h.ptr;
    d.ldx = d_model;
    d.w = (const float*)w.ptr;
    d.b = (const float*)b.ptr;
    d.y = normed.ptr;
    d.ldy = d_model;
    d.eps = 1e-5f;
    return qa_layer_norm(ctx, &d);
  };
  run([&] { return ln(l.ln1_w, l.ln1_b); });
  const Linear* after = li + 1 < layers ? &L[(size_t)li + 1].qkv : &p1;
  run([&] { return linear(ctx, dtype, normed.ptr, l.qkv, qkv.ptr, n, false, false, &l.o); });
  run([&] {
    qa_window_attention_desc d{};
    d.dtype = (uint32_t)dtype;
    d.s = n;
    d.nh = nh;
    d.hd = d_model / nh;
    d.wlen = wlen;
    d.qkv = qkv.ptr;
    d.ldqkv = 3 * d_model;
    d.out = attn.ptr;
    d.ldo = d_model;
    return qa_window_attention(ctx, &d);
  });
  run([&] { return linear(ctx, dtype, attn.ptr, l.o, h.ptr, n, true, false, &l.fc1); });
  run([&] { return ln(l.ln2_w, l.ln2_b); });
  run([&] { return linear(ctx, dtype, normed.ptr, l.fc1, act.ptr, n, false, true, &l.fc2); });
  run([&] { return linear(ctx, dtype, act.ptr, l.fc2, h.ptr, n, true, false, after); });
  return rc;
}

int AudioEncoder::post(int64_t n) {
  qa_layer_norm_desc d{};
  d.dtype = (uint32_t)dtype;
  d.rows = n;
  d.n = d_model;
  d.x = h.ptr;
  d.ldx = d_model;
  d.w = (const float*)post_w.ptr;
  d.b = (const float*)post_b.ptr;
  d.y = normed.ptr;
  d.ldy = d_model;
  d.eps = 1e-5f;
  if (int rc = qa_layer_norm(ctx, &d)) return rc;
  if (int rc = linear(ctx, dtype, normed.ptr, p1, pact.ptr, n, false, true, &p2)) return rc;
  return linear(ctx, dtype, pact.ptr, p2, out.ptr, n, false, false);
}

int AudioEncoder::forward(int n_chunks, int tail_frames) {
  if (tail_frames < 0 || tail_frames >= cs) return QA_EINVAL;
  const int64_t n = tokens(n_chunks, tail_frames);
  if (int rc = stem(n_chunks)) return rc;
  if (int rc = conv_out(n)) return rc;
  for (int li = 0; li < layers; ++li)
    if (int rc = layer(li, n)) return rc;
  return post(n);
}

int AudioEncoder::read(int which, int64_t rows, uint16_t* host) {
  if (!host || rows < 0) return QA_EINVAL;
  const Buffer* src[] = {&out, &h, &y1, &y2, &y3, &normed, &qkv, &attn, &act, &pact};
  const int64_t cols[] = {out_dim, d_model, c_conv, c_conv, (int64_t)c_conv * h3, d_model,
                          3 * d_model, d_model, ffn, d_model};
  if (which < 0 || which >= (int)(sizeof(cols) / sizeof(cols[0]))) return QA_EINVAL;
  const size_t bytes = (size_t)(rows * cols[which]) * 2;
  if (bytes > src[which]->bytes) return QA_EINVAL;
  return qa_download(ctx, host, src[which]->ptr, 0, bytes);
}

}  // namespace qa_host

// ------------------------------------------------------------------------
// C surface
using namespace qa_host;


extern "C" {

int qah_aenc_create(qa_ctx* ctx, int dtype, int layers, int n_mels, int cs, int c_conv,
                    int d_model, int nh, int ffn, int out_dim, int wlen, int max_chunks,
                    qah_aenc** out) {
  if (!ctx || !out || layers < 0 || n_mels <= 0 || cs <= 0 || c_conv <= 0 || d_model <= 0 ||
      nh <= 0 || ffn <= 0 || out_dim <= 0 || wlen <= 0 || max_chunks <= 0)
    return QA_EINVAL;
  auto* e = new AudioEncoder(ctx, dtype, layers, n_mels, cs, c_conv, d_model, nh, ffn, out_dim,
                             wlen, max_chunks);
  if (int rc = e->init()) {
    delete e;
    return rc;
  }
  *out = new qah_aenc{e};
  return QA_OK;
}

int qah_aenc_load_conv(qah_aenc* a, int level, const uint16_t* w, const uint16_t* b) {
  return a ? a->e->load_conv(level, w, b) : QA_EINVAL;
}

int qah_aenc_load_conv_out(qah_aenc* a, const uint16_t* w, const uint16_t* b) {
  return a ? a->e->load_conv_out(w, b) : QA_EINVAL;
}

int qah_aenc_load_layer(qah_aenc* a, int li, const float* ln1_w, const float* ln1_b,
                        const uint16_t* qkv_w, const uint16_t* qkv_b, const uint16_t* o_w,
                        const uint16_t* o_b, const float* ln2_w, const float* ln2_b,
                        const uint16_t* fc1_w, const uint16_t* fc1_b, const uint16_t* fc2_w,
                        const uint16_t* fc2_b) {
  return a ? a->e->load_layer(li, ln1_w, ln1_b, qkv_w, qkv_b, o_w, o_b, ln2_w, ln2_b, fc1_w,
                              fc1_b, fc2_w, fc2_b)
           : QA_EINVAL;
}

int qah_aenc_load_post(qah_aenc* a, const float* ln_w, const float* ln_b, const uint16_t* p1_w,
                       const uint16_t* p1_b, const uint16_t* p2_w, const uint16_t* p2_b) {
  return a ? a->e->load_post(ln_w, ln_b, p1_w, p1_b, p2_w, p2_b) : QA_EINVAL;
}

int qah_aenc_set_mel(qah_aenc* a, int n_chunks, const uint16_t* mel) {
  return a ? a->e->set_mel(n_chunks, mel) : QA_EINVAL;
}

int64_t qah_aenc_tokens(qah_aenc* a, int n_chunks, int tail_frames) {
  return a ? a->e->tokens(n_chunks, tail_frames) : -1;
}

int qah_aenc_forward(qah_aenc* a, int n_chunks, int tail_frames) {
  return a ? a->e->forward(n_chunks, tail_frames) : QA_EINVAL;
}

int qah_aenc_read(qah_aenc* a, int which, int64_t rows, uint16_t* host) {
  return a ? a->e->read(which, rows, host) : QA_EINVAL;
}

int qah_aenc_time(qah_aenc* a, int n_chunks, int tail_frames, int warmup, int steps,
                  int use_graph, double* ms_per_step, double* wall_ms_per_step) {
  if (!a || !ms_per_step) return QA_EINVAL;
  return time_steps(a->e->ctx, warmup, steps, use_graph,
                    [&] { return a->e->forward(n_chunks, tail_frames); }, ms_per_step,
                    wall_ms_per_step);
}

int qah_aenc_profile(qah_aenc* a, int n_chunks, int tail_frames, int steps, double* ms) {
  if (!a || !ms || steps <= 0) return QA_EINVAL;
  AudioEncoder& E = *a->e;
  const int64_t n = E.tokens(n_chunks, tail_frames);
  hipStream_t st = (hipStream_t)qa_ctx_stream(E.ctx);
  std::vector<hipEvent_t> ev(4 + 4 + (size_t)E.layers * 14);
  for (auto& e : ev) (void)hipEventCreate(&e);
  double acc[12] = {0};
  int rc = QA_OK;
  for (int s = 0; s < steps && rc == QA_OK; ++s) {
    rc = E.stem(n_chunks, ev.data());
    if (rc == QA_OK) {
      (void)hipEventRecord(ev[4], st);
      rc = E.conv_out(n);
      (void)hipEventRecord(ev[5], st);
    }
    for (int li = 0; li < E.layers && rc == QA_OK; ++li) rc = E.layer(li, n, &ev[8 + (size_t)li * 14]);
    if (rc == QA_OK) {
      (void)hipEventRecord(ev[6], st);
      rc = E.post(n);
      (void)hipEventRecord(ev[7], st);
    }
    if (rc == QA_OK) rc = qa_sync(E.ctx);
    if (rc) break;
    float t = 0.f;
    for (int lv = 0; lv < 3; ++lv) {
      (void)hipEventElapsedTime(&t, ev[lv], ev[lv + 1]);
      acc[lv] += t;
    }
    (void)hipEventElapsedTime(&t, ev[4], ev[5]);
    acc[3] += t;
    for (int li = 0; li < E.layers; ++li)
      for (int i = 0; i < 7; ++i) {
        (void)hipEventElapsedTime(&t, ev[8 + (size_t)li * 14 + 2 * i],
                                  ev[8 + (size_t)li * 14 + 2 * i + 1]);
        acc[4 + i] += t;
      }
    (void)hipEventElapsedTime(&t, ev[6], ev[7]);
    acc[11] += t;
  }
  for (auto& e : ev) (void)hipEventDestroy(e);
  for (int i = 0; i < 12; ++i) ms[i] = acc[i] / steps;  // layer ops summed over all layers
  return rc;
}

void qah_aenc_destroy(qah_aenc* a) {
  if (!a) return;
  delete a->e;
  delete a;
}

}  // extern "C"
