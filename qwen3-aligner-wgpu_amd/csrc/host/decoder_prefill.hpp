// decoder_prefill.hpp -- C++ host mirror of WgpuTextDecoder::prefill's layer
// loop (src/decoder.rs:1305-1657): every op of a Qwen3 decoder layer through
// the C ABI (include/qa.h), over the projections of TextDecoderLinears.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <vector>

#include "linear_sites.hpp"
#include "qa.h"

namespace qa_host {

class TextDecoder {
 public:
  // Per-layer tensors beside the projection weights: the input and
  // post-attention RMSNorm weights [hidden], the q/k head-norm weights [hd]
  // (f32, as the CPU twin widens them, src/cpu_decoder.rs:288-322), and the
  // layer's KV cache: K [nkvh][cap][hd], V transposed [nkvh][hd][cap].
  struct Layer {
    Buffer iln, pln, qn, kn, k_cache, v_cache;
  };
  TextDecoder(qa_ctx* ctx, int dtype, int layers, int hidden, int nqh, int nkvh, int hd, int inter,
              int max_rows, float eps);
  ~TextDecoder();
  int init();
  int load_layer(int li, const uint16_t* q, const uint16_t* k, const uint16_t* v,
                 const uint16_t* o, const uint16_t* gate, const uint16_t* up,
                 const uint16_t* down, const float* iln, const float* pln, const float* qn,
                 const float* kn);
  // RoPE tables cos/sin [positions][hd] (src/mrope.rs:55-82, uploaded once
  // per prefill as the reference's scratch.cos / scratch.sin).
  int set_rope(const float* cos, const float* sin, int positions);
  int set_hidden(int rows, const uint16_t* h);
  // One layer: rms_norm -> qkv -> qk_norm_rope (KV write) -> attention ->
  // o + residual -> rms_norm -> gate|up + SiLU.up -> down + residual.
  // ev (16 events) brackets each of the 8 ops when non-null.
  int layer(int li, int rows, hipEvent_t* ev = nullptr);
  int prefill(int rows);
  int read(int which, int rows, uint16_t* host);

  qa_ctx* ctx;
  int dtype, layers, hidden, nqh, nkvh, hd, inter, max_rows;
  float eps;
  uint32_t attn_flags = 0;  // qa_attention_desc.flags
  int rope_positions = 0;
  TextDecoderLinears lin;
  std::vector<Layer> L;
  Buffer q_heads, cos, sin;
};

}  // namespace qa_host
