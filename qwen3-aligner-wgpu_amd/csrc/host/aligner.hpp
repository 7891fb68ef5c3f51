// aligner.hpp -- C++ host mirror of the aligner's forward pass
// (Aligner::align_raw_rows, src/align_inference.rs:656-805, with the input
// assembly of src/align_input.rs and the repair of src/postprocess.rs):
//   16 kHz samples -> log-mel chunks (qa_log_mel) -> audio tower
//   -> token embedding gather + audio-row scatter (qa_embed_scatter)
//   -> text decoder prefill -> timestamp head (qa_timestamp_head)
//   -> classes x segment time -> fix_timestamps (host).
// Every device step runs on the context's stream with device-resident
// inputs; the host reads back only the classes.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <vector>

#include "audio_encoder.hpp"
#include "decoder_prefill.hpp"
#include "linear_sites.hpp"
#include "qa.h"

namespace qa_host {

// The timestamp repair (src/postprocess.rs:33-111): the longest
// non-decreasing subsequence (earliest index on ties) stays; each maximal run
// of other positions snaps to its nearer neighbour by index distance when it
// is at most 2 long, else is interpolated linearly between its neighbours and
// truncated toward zero; a run with one neighbour takes that neighbour.
void fix_timestamps(const int64_t* data, int64_t n, int64_t* out);

// Token ids of the input sequence (the shipped checkpoint's special tokens,
// src/align_input.rs:1-20).
struct AlignerTokens {
  int32_t audio_start = 151669, audio_end = 151670, audio_pad = 151676, timestamp = 151705;
};

class Aligner {
 public:
  // enc and dec are owned by the caller; enc's output width must equal dec's
  // hidden size and both must use the same 16-bit format.
  Aligner(qa_ctx* ctx, AudioEncoder* enc, TextDecoder* dec, int64_t vocab, int64_t labels,
          double segment_ms, int64_t max_samples);
  ~Aligner();
  int init();
  int load_embed(const uint16_t* table);                  // [vocab][hidden], 16-bit
  int load_head(const float* norm_w, const float* score);  // [hidden], [labels][hidden]
  // AlignerInput (src/align_input.rs:120-220): the sequence
  //   audio_start, audio_pad x n_audio, audio_end, then per word its token
  //   ids followed by two timestamp tokens,
  // with n_audio from the sample count (valid frames = n_samples / hop).
  // Uploads the samples, the row-source map and the timestamp positions.
  int prepare(const float* samples, int64_t n_samples, int n_words, const int32_t* word_lens,
              const int32_t* word_ids);
  // The device pass; ev (6 events) brackets mel, tower, scatter, prefill, head.
  int forward(hipEvent_t* ev = nullptr);
  // Downloads the classes: raw_ms = class * segment (truncated like the
  // reference's `as i64`), fixed_ms = fix_timestamps(raw_ms); 2 per word.
  int result(int64_t* raw_ms, int64_t* fixed_ms);

  qa_ctx* ctx;
  AudioEncoder* enc;
  TextDecoder* dec;
  int64_t vocab, labels;
  double segment_ms;
  int64_t max_samples;
  AlignerTokens tok;
  Buffer filt, samples, src, ts_pos, logits, classes, embed, norm_w, score;
  // the prepared input
  int64_t n_samples = 0, seq = 0, n_audio = 0, n_ts = 0;
  int n_chunks = 0, tail = 0;
  std::vector<int32_t> ids, src_host, ts_host;
};

}  // namespace qa_host
