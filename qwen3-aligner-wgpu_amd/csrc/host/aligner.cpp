// aligner.cpp -- the aligner's forward pass over the C ABI (see aligner.hpp).
//
// Reference call stack mirrored (src/align_inference.rs):
//   align_raw_ms (:646)  -> audio_embeds (:118, the tower)
//                        -> the host gather + scatter (:685-714)
//                        -> text_hidden (:150, the 28-layer prefill)
//                        -> the final norm + score head + argmax (:721-805)
//   decode_timestamps (src/postprocess.rs:147) -> fix_timestamps (:33).
// The reference computes the log-mel, the gather/scatter and the head on the
// host; here they are device steps, so one forward is a single stream of
// launches with no host round trip until the classes are read back.
#include "aligner.hpp"

#include <algorithm>
#include <cstring>

#include "handles.hpp"
#include "qa_host.h"
#include "timing.hpp"

namespace qa_host {

namespace {
constexpr int kHop = 160, kNfft = 400, kRate = 16000;
}

void fix_timestamps(const int64_t* d, int64_t n, int64_t* out) {
  if (n <= 0) return;
  const size_t un = (size_t)n;
  // chain[i]: length of the longest non-decreasing chain ending at i; from[i]:
  // its predecessor, the earliest j that reaches that length
  std::vector<int64_t> chain(un, 1), from(un, -1);
  for (size_t i = 1; i < un; ++i)
    for (size_t j = 0; j < i; ++j)
      if (d[j] <= d[i] && chain[j] + 1 > chain[i]) {
        chain[i] = chain[j] + 1;
        from[i] = (int64_t)j;
      }
  // the chain kept is the one ending at the first index of the maximum length
  const size_t last = (size_t)(std::max_element(chain.begin(), chain.end()) - chain.begin());
  std::vector<char> kept(un, 0);
  for (int64_t i = (int64_t)last; i >= 0; i = from[(size_t)i]) kept[(size_t)i] = 1;
  std::copy(d, d + n, out);
  for (int64_t b = 0; b < n;) {
    if (kept[(size_t)b]) {
      ++b;
      continue;
    }
    int64_t e = b;
    while (e < n && !kept[(size_t)e]) ++e;
    // the run [b, e) is maximal, so b - 1 and e (where they exist) are kept
    const bool has_l = b > 0, has_r = e < n;
    const int64_t lv = has_l ? out[b - 1] : 0, rv = has_r ? out[e] : 0;
    const int64_t count = e - b;
    for (int64_t p = b; p < e; ++p) {
      if (has_l && has_r) {
        if (count <= 2)
          out[p] = (p - (b - 1) <= e - p) ? lv : rv;  // nearer by index distance, left on ties
        else
          out[p] = (int64_t)((double)lv + (double)(rv - lv) / (double)(count + 1) * (double)(p - b + 1));
      } else {
        out[p] = has_l ? lv : rv;
      }
    }
    b = e;
  }
}

Aligner::Aligner(qa_ctx* c, AudioEncoder* e, TextDecoder* t, int64_t vocab_, int64_t labels_,
                 double segment_ms_, int64_t max_samples_)
    : ctx(c), enc(e), dec(t), vocab(vocab_), labels(labels_), segment_ms(segment_ms_),
      max_samples(max_samples_) {}

Aligner::~Aligner() {
  for (Buffer* b : {&filt, &samples, &src, &ts_pos, &logits, &classes, &embed, &norm_w, &score})
    release(ctx, b);
}

int Aligner::init() {
  if (!enc || !dec || vocab <= 0 || labels <= 0 || max_samples < kHop) return QA_EINVAL;
  if (enc->dtype != dec->dtype || enc->out_dim != dec->hidden) return QA_EINVAL;
  if (max_samples / kHop > (int64_t)enc->max_chunks * enc->cs) return QA_EINVAL;
  const int nbin = kNfft / 2 + 1;
  std::vector<float> fb((size_t)enc->n_mels * nbin);
  if (int rc = qa_mel_filterbank(enc->n_mels, kNfft, kRate, fb.data())) return rc;
  if (int rc = alloc(ctx, fb.size() * 4, &filt)) return rc;
  if (int rc = qa_upload(ctx, filt.ptr, 0, fb.data(), fb.size() * 4)) return rc;
  const size_t rows = (size_t)dec->max_rows;
  if (int rc = alloc(ctx, (size_t)max_samples * 4, &samples)) return rc;
  if (int rc = alloc(ctx, rows * 4, &src)) return rc;
  if (int rc = alloc(ctx, rows * 4, &ts_pos)) return rc;
  if (int rc = alloc(ctx, rows * (size_t)labels * 4, &logits)) return rc;
  if (int rc = alloc(ctx, rows * 4, &classes)) return rc;
  if (int rc = alloc(ctx, (size_t)vocab * dec->hidden * 2, &embed)) return rc;
  if (int rc = alloc(ctx, (size_t)dec->hidden * 4, &norm_w)) return rc;
  return alloc(ctx, (size_t)labels * dec->hidden * 4, &score);
}

int Aligner::load_embed(const uint16_t* table) {
  if (!table) return QA_EINVAL;
  return qa_upload(ctx, embed.ptr, 0, table, embed.bytes);
}

int Aligner::load_head(const float* w, const float* s) {
  if (!w || !s) return QA_EINVAL;
  if (int rc = qa_upload(ctx, norm_w.ptr, 0, w, norm_w.bytes)) return rc;
  return qa_upload(ctx, score.ptr, 0, s, score.bytes);
}

int Aligner::prepare(const float* x, int64_t n, int n_words, const int32_t* word_lens,
                     const int32_t* word_ids) {
  // Forget the previous clip first: after a failed prepare, forward() must
  // refuse (seq == 0) instead of aligning the old input, and info / the host
  // arrays must describe nothing rather than a mix of two clips.
  seq = n_audio = n_ts = 0;
  ids.clear();
  src_host.clear();
  ts_host.clear();
  if (!x || n < kHop || n > max_samples || n_words < 0 || (n_words && (!word_lens || !word_ids)))
    return QA_EINVAL;
  const int64_t frames = n / kHop;  // valid_mel_frames (src/align_input.rs:94-101)
  const int chunks = (int)((frames + enc->cs - 1) / enc->cs);
  const int tl = (int)(frames % enc->cs);
  const int64_t na = enc->tokens(chunks, tl);  // audio_token_count (src/align_input.rs:66-71)
  ids.push_back(tok.audio_start);
  for (int64_t k = 0; k < na; ++k) ids.push_back(tok.audio_pad);
  ids.push_back(tok.audio_end);
  int64_t off = 0;
  for (int w = 0; w < n_words; ++w) {
    if (word_lens[w] <= 0) return QA_EINVAL;
    for (int32_t j = 0; j < word_lens[w]; ++j) {
      const int32_t id = word_ids[off++];
      // an audio placeholder among the words would take an audio row (the
      // reference rejects the count mismatch, src/align_inference.rs:708-713)
      if (id < 0 || id >= vocab || id == tok.audio_pad) return QA_EINVAL;
      ids.push_back(id);
    }
    for (int k = 0; k < 2; ++k) {
      ts_host.push_back((int32_t)ids.size());
      ids.push_back(tok.timestamp);
    }
  }
  const int64_t s = (int64_t)ids.size();
  if (s > dec->max_rows || s > dec->rope_positions) return QA_EINVAL;
  // the row source of each position: a token id, or -1 - k for audio row k
  int64_t k = 0;
  for (int32_t id : ids) src_host.push_back(id == tok.audio_pad ? (int32_t)(-1 - k++) : id);
  auto forget = [&](int rc) {
    ids.clear();
    src_host.clear();
    ts_host.clear();
    return rc;
  };
  if (int rc = qa_upload(ctx, samples.ptr, 0, x, (size_t)n * 4)) return forget(rc);
  if (int rc = qa_upload(ctx, src.ptr, 0, src_host.data(), src_host.size() * 4)) return forget(rc);
  if (!ts_host.empty())
    if (int rc = qa_upload(ctx, ts_pos.ptr, 0, ts_host.data(), ts_host.size() * 4))
      return forget(rc);
  n_samples = n;
  seq = s;
  n_audio = na;
  n_ts = (int64_t)ts_host.size();
  n_chunks = chunks;
  tail = tl;
  return QA_OK;
}

int Aligner::forward(hipEvent_t* ev) {
  if (seq == 0) return QA_EINVAL;  // nothing prepared
  hipStream_t st = (hipStream_t)qa_ctx_stream(ctx);
  auto mark = [&](int i) {
    if (ev) (void)hipEventRecord(ev[i], st);
  };
  mark(0);
  qa_mel_desc m{};
  m.dtype = (uint32_t)enc->dtype;
  m.n_samples = n_samples;
  m.samples = (const float*)samples.ptr;
  m.filterbank = (const float*)filt.ptr;
  m.n_mels = enc->n_mels;
  m.cs = enc->cs;
  m.out = enc->mel.ptr;
  if (int rc = qa_log_mel(ctx, &m)) return rc;
  mark(1);
  if (int rc = enc->forward(n_chunks, tail)) return rc;
  mark(2);
  qa_embed_desc g{};
  g.dtype = (uint32_t)dec->dtype;
  g.rows = seq;
  g.hidden = dec->hidden;
  g.src = (const int32_t*)src.ptr;
  g.table = embed.ptr;
  g.vocab = vocab;
  g.audio = enc->out.ptr;
  g.n_audio = n_audio;
  g.out = dec->lin.h.ptr;
  if (int rc = qa_embed_scatter(ctx, &g)) return rc;
  mark(3);
  if (int rc = dec->prefill((int)seq)) return rc;
  mark(4);
  if (n_ts > 0) {
    qa_head_desc h{};
    h.dtype = (uint32_t)dec->dtype;
    h.rows = n_ts;
    h.positions = (const int32_t*)ts_pos.ptr;
    h.h = dec->lin.h.ptr;
    h.h_rows = seq;
    h.ldh = dec->hidden;
    h.n = dec->hidden;
    h.norm_w = (const float*)norm_w.ptr;
    h.eps = dec->eps;
    h.score = (const float*)score.ptr;
    h.labels = labels;
    h.logits = (float*)logits.ptr;
    h.classes = (int32_t*)classes.ptr;
    if (int rc = qa_timestamp_head(ctx, &h)) return rc;
  }
  mark(5);
  return QA_OK;
}

int Aligner::result(int64_t* raw_ms, int64_t* fixed_ms) {
  if (!raw_ms || !fixed_ms) return QA_EINVAL;
  if (n_ts == 0) return QA_OK;
  std::vector<int32_t> cls((size_t)n_ts);
  if (int rc = qa_download(ctx, cls.data(), classes.ptr, 0, cls.size() * 4)) return rc;
  for (size_t i = 0; i < cls.size(); ++i) raw_ms[i] = (int64_t)((double)cls[i] * segment_ms);
  fix_timestamps(raw_ms, n_ts, fixed_ms);
  return QA_OK;
}

}  // namespace qa_host

// ------------------------------------------------------------------------
// C surface
using namespace qa_host;

struct qah_aligner {
  Aligner* a;
};

extern "C" {

void qah_fix_timestamps(const int64_t* data, int64_t n, int64_t* out) {
  if (data && out) fix_timestamps(data, n, out);
}

int qah_aligner_create(qa_ctx* ctx, qah_aenc* enc, qah_tdec* dec, int64_t vocab, int64_t labels,
                       double segment_ms, int64_t max_samples, qah_aligner** out) {
  if (!ctx || !enc || !dec || !out) return QA_EINVAL;
  auto* a = new Aligner(ctx, enc->e, dec->d, vocab, labels, segment_ms, max_samples);
  if (int rc = a->init()) {
    delete a;
    return rc;
  }
  *out = new qah_aligner{a};
  return QA_OK;
}

int qah_aligner_load_embed(qah_aligner* h, const uint16_t* table) {
  return h ? h->a->load_embed(table) : QA_EINVAL;
}

int qah_aligner_load_head(qah_aligner* h, const float* norm_w, const float* score) {
  return h ? h->a->load_head(norm_w, score) : QA_EINVAL;
}

int qah_aligner_prepare(qah_aligner* h, const float* samples, int64_t n_samples, int n_words,
                        const int32_t* word_lens, const int32_t* word_ids, int64_t* info) {
  if (!h) return QA_EINVAL;
  if (int rc = h->a->prepare(samples, n_samples, n_words, word_lens, word_ids)) return rc;
  if (info) {
    const Aligner& A = *h->a;
    info[0] = A.seq;
    info[1] = A.n_audio;
    info[2] = A.n_ts;
    info[3] = A.n_chunks;
    info[4] = A.tail;
  }
  return QA_OK;
}

int qah_aligner_forward(qah_aligner* h) { return h ? h->a->forward() : QA_EINVAL; }

int qah_aligner_result(qah_aligner* h, int64_t* raw_ms, int64_t* fixed_ms) {
  return h ? h->a->result(raw_ms, fixed_ms) : QA_EINVAL;
}

int qah_aligner_read(qah_aligner* h, int which, void* host) {
  if (!h || !host) return QA_EINVAL;
  Aligner& A = *h->a;
  switch (which) {
    case 0: return qa_download(A.ctx, host, A.classes.ptr, 0, (size_t)A.n_ts * 4);
    case 1: return qa_download(A.ctx, host, A.logits.ptr, 0, (size_t)(A.n_ts * A.labels) * 4);
    case 2: std::memcpy(host, A.ids.data(), A.ids.size() * 4); return QA_OK;
    case 3: std::memcpy(host, A.ts_host.data(), A.ts_host.size() * 4); return QA_OK;
    case 4: std::memcpy(host, A.src_host.data(), A.src_host.size() * 4); return QA_OK;
    default: return QA_EINVAL;
  }
}

int qah_aligner_time(qah_aligner* h, int warmup, int steps, int use_graph, double* ms_per_step,
                     double* wall_ms_per_step) {
  if (!h || !ms_per_step) return QA_EINVAL;
  return time_steps(h->a->ctx, warmup, steps, use_graph, [&] { return h->a->forward(); },
                    ms_per_step, wall_ms_per_step);
}

int qah_aligner_profile(qah_aligner* h, int steps, double* ms) {
  if (!h || !ms || steps <= 0) return QA_EINVAL;
  hipEvent_t ev[6];
  for (auto& e : ev) (void)hipEventCreate(&e);
  double acc[5] = {0};
  int rc = QA_OK;
  for (int s = 0; s < steps && rc == QA_OK; ++s) {
    rc = h->a->forward(ev);
    if (rc == QA_OK) rc = qa_sync(h->a->ctx);
    for (int i = 0; i < 5 && rc == QA_OK; ++i) {
      float t = 0.f;
      (void)hipEventElapsedTime(&t, ev[i], ev[i + 1]);
      acc[i] += t;
    }
  }
  for (auto& e : ev) (void)hipEventDestroy(e);
  for (int i = 0; i < 5; ++i) ms[i] = acc[i] / steps;
  return rc;
}

void qah_aligner_destroy(qah_aligner* h) {
  if (!h) return;
  delete h->a;
  delete h;
}

}  // extern "C"
