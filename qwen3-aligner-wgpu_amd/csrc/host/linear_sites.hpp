// linear_sites.hpp -- C++ host mirror of the reference's GEMM call sites,
// written against the C ABI (include/qa.h) only.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <vector>

#include "qa.h"

namespace qa_host {

// A caller-owned device buffer (Gpu::storage, src/gpu.rs:672-682).
struct Buffer {
  void* ptr = nullptr;
  size_t bytes = 0;
};

int alloc(qa_ctx* ctx, size_t bytes, Buffer* b);
void release(qa_ctx* ctx, Buffer* b);

// The decoder's `gemm!` macro (src/decoder.rs:1087-1104) as a function with
// the same argument meaning: m, n, k; ldc in elements; bsa/bsb in u32 WORDS
// and bsc in elements (GDims, src/decoder.rs:194-212); `beta` selects the
// accumulating pipeline `gemm_acc` (src/decoder.rs:524-525).  The unit
// conversion to qa_linear_desc (elements throughout) happens here.
int gemm(qa_ctx* ctx, int dtype, const void* a, const void* w, void* c, int64_t m, int64_t n,
         int64_t k, int64_t ldc, int64_t bsa_words, int64_t bsb_words, int64_t bsc, int64_t batch,
         bool beta, uint32_t extra_flags = 0, const void* bias = nullptr);

// GpuLinear (src/audio_encoder_gpu.rs:216-314): a weight [n, k] with its
// bias.  The reference pads n to its 128-wide tile and k to 16 (:235,
// :2266-2268); the MFMA kernels handle ragged edges, so only the ABI's
// alignment (k to 8, n to 4) is padded here, with zero rows/columns.
struct Linear {
  Buffer w, b;
  int64_t n = 0, n_pad = 0, k = 0, k_pad = 0;
};
int load_linear(qa_ctx* ctx, const uint16_t* w, const uint16_t* bias, int64_t n, int64_t k,
                Linear* out);

class TextDecoderLinears {
 public:
  struct Layer {
    Buffer qkv_w, o_w, gu_w, dp_w;
  };
  TextDecoderLinears(qa_ctx* ctx, int dtype, int layers, int hidden, int q_dim, int kv_dim,
                     int inter, int max_rows);
  ~TextDecoderLinears();
  int init();
  int load_layer(int li, const uint16_t* q, const uint16_t* k, const uint16_t* v,
                 const uint16_t* o, const uint16_t* gate, const uint16_t* up,
                 const uint16_t* down);
  int set_inputs(int rows, const uint16_t* normed, const uint16_t* attn, const uint16_t* norm2,
                 const uint16_t* h);
  // One layer's four projections; site_events (8 events) bracket each launch
  // when non-null.
  int layer(int li, int rows, hipEvent_t* site_events = nullptr);
  int prefill_linears(int rows);
  int read(int which, int rows, uint16_t* host);

  qa_ctx* ctx;
  int dtype, layers, hidden, q_dim, kv_dim, inter, max_rows;
  std::vector<Layer> L;
  Buffer normed, attn, norm2, h, qkv, act;
};

class AudioEncoderLinears {
 public:
  struct Layer {
    Linear qkv, o, fc1, fc2;
  };
  AudioEncoderLinears(qa_ctx* ctx, int dtype, int layers, int d_model, int ffn, int conv_k,
                      int max_rows);
  ~AudioEncoderLinears();
  int init();
  int load_layer(int li, const uint16_t* qkv_w, const uint16_t* qkv_b, const uint16_t* o_w,
                 const uint16_t* o_b, const uint16_t* fc1_w, const uint16_t* fc1_b,
                 const uint16_t* fc2_w, const uint16_t* fc2_b);
  int load_conv(const uint16_t* w, const uint16_t* b);
  int set_inputs(int rows, const uint16_t* col, const uint16_t* normed, const uint16_t* attn,
                 const uint16_t* norm2, const uint16_t* h);
  int conv(int rows);
  int layer(int li, int rows, hipEvent_t* site_events = nullptr);
  int forward_linears(int rows);
  int read(int which, int rows, uint16_t* host);

  qa_ctx* ctx;
  int dtype, layers, d_model, ffn, conv_k, max_rows;
  std::vector<Layer> L;
  Linear conv_w;
  Buffer col, normed, attn, norm2, h, conv_out, qkv, act;
};

}  // namespace qa_host
