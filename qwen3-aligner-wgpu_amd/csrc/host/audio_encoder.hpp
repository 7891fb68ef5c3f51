// audio_encoder.hpp -- C++ host mirror of GpuAudioEncoder::encode
// (src/audio_encoder_gpu.rs:1060-1347): the conv stem, conv_out + position
// add, the transformer layers and the projector, every op through the C ABI.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <vector>

#include "linear_sites.hpp"
#include "qa.h"

namespace qa_host {

class AudioEncoder {
 public:
  struct Layer {
    Buffer ln1_w, ln1_b, ln2_w, ln2_b;  // f32 [d_model]
    Linear qkv, o, fc1, fc2;
  };
  struct Conv {
    Buffer w, b;  // w [c_out][ldw] in (kh, kw, ic) order, b [c_out]
    int c_in = 0;
  };
  // Qwen3-ASR audio tower: n_mels bins, chunks of cs frames, conv channels
  // c_conv, d_model = nh * 64, ffn, out_dim; windows of wlen tokens.
  AudioEncoder(qa_ctx* ctx, int dtype, int layers, int n_mels, int cs, int c_conv, int d_model,
               int nh, int ffn, int out_dim, int wlen, int max_chunks);
  ~AudioEncoder();
  int init();
  // level 0..2 weight in the checkpoint's [c_out][c_in][3][3] layout, bias [c_out]
  int load_conv(int level, const uint16_t* w, const uint16_t* b);
  // conv_out weight [d_model][c_conv * f] in the checkpoint's (c, f) column order
  int load_conv_out(const uint16_t* w, const uint16_t* b);
  int load_layer(int li, const float* ln1_w, const float* ln1_b, const uint16_t* qkv_w,
                 const uint16_t* qkv_b, const uint16_t* o_w, const uint16_t* o_b,
                 const float* ln2_w, const float* ln2_b, const uint16_t* fc1_w,
                 const uint16_t* fc1_b, const uint16_t* fc2_w, const uint16_t* fc2_b);
  int load_post(const float* ln_w, const float* ln_b, const uint16_t* p1_w, const uint16_t* p1_b,
                const uint16_t* p2_w, const uint16_t* p2_b);
  // mel chunks [n_chunks][n_mels][cs], 16-bit (the reference's `chunked`
  // buffer, src/audio_encoder_gpu.rs:1079-1091)
  int set_mel(int n_chunks, const uint16_t* mel);
  // tokens of a prefill over n_chunks chunks whose last has tail_frames frames
  // (0 = full), as encode counts them (feo, src/audio_encoder.rs:692-696)
  int64_t tokens(int n_chunks, int tail_frames) const;
  int stem(int n_chunks, hipEvent_t* ev = nullptr);            // 3 conv levels (4 events)
  int conv_out(int64_t n_tokens);                              // conv_out + position add
  int layer(int li, int64_t n_tokens, hipEvent_t* ev = nullptr);  // 8 ops (16 events)
  int post(int64_t n_tokens);                                  // ln_post, proj1 + GELU, proj2
  int forward(int n_chunks, int tail_frames);
  int read(int which, int64_t rows, uint16_t* host);

  qa_ctx* ctx;
  int dtype, layers, n_mels, cs, c_conv, d_model, nh, ffn, out_dim, wlen, max_chunks;
  int h1, w1, h2, w2, h3, w3;  // conv output heights (mel) and widths (frames)
  Conv conv[3];
  Linear co, p1, p2;
  Buffer post_w, post_b;
  std::vector<Layer> L;
  Buffer mel, y1, y2, y3, pe, h, normed, qkv, attn, act, pact, out;
};

}  // namespace qa_host
