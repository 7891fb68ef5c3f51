// qa_internal.h -- shared between the C-ABI layer (qa_api.cpp) and the
// kernels (qa_gemm.hip).  Not installed; the public surface is include/qa.h.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "qa.h"

namespace qa {

// Epilogue kinds compiled into separate kernels.  Bias and the residual add
// are runtime switches of EPI_PLAIN (they cost one branch in the epilogue);
// GELU and SiLU-mul change the epilogue's arithmetic and its column mapping.
enum Epi : int { EPI_PLAIN = 0, EPI_GELU = 1, EPI_SILU = 2 };

// Tile shapes (block BM x BN; two k-groups of 2x2 waves each).  Chosen per
// call by plan_linear().
enum TileCfg : int {
  TILE_128x128 = 0,  // waves of 64x64
  TILE_256x128 = 1,  // waves of 128(m) x 64(n)
  TILE_128x256 = 2,  // waves of 64(m) x 128(n)
  TILE_64x128 = 3,   // waves of 32(m) x 64(n)
  TILE_64x64 = 4,    // waves of 32x32
  TILE_128x192 = 5,  // waves of 64(m) x 96(n)
  TILE_COUNT
};

struct TileShape {
  int bm, bn;
};
inline TileShape tile_shape(int cfg) {
  switch (cfg) {
    case TILE_256x128: return {256, 128};
    case TILE_128x256: return {128, 256};
    case TILE_64x128: return {64, 128};
    case TILE_64x64: return {64, 64};
    case TILE_128x192: return {128, 192};
    default: return {128, 128};
  }
}

// Kernel parameters (passed by value).  Element units throughout.
struct GemmParams {
  const uint16_t* a;
  const uint16_t* w;
  uint16_t* c;
  const uint16_t* bias;  // nullptr = no bias
  float* ws;             // split-K partials [splits][M][N] f32 (splits > 1)
  int a_bytes, w_bytes;  // byte span of one batch's A / W (buffer num_records)
  int M, N, K;           // N = rows of W (2*inter for SiLU-mul)
  int lda, ldb, ldc;
  int64_t bsa, bsb, bsc;
  int tiles_m, tiles_n;  // output tiles
  int splits;            // K splits per tile (>= 1)
  int kchunk;            // K range per split, multiple of 64
  int accumulate;        // add C_old before the rounding
  int bias_rows;         // bias indexed by output row (channel-major conv)
  int group_m;           // m-tiles per band of the tile enumeration (tile_of)
};

struct Plan {
  int tile;
  int epi;
  bool transb;
  int tiles_m, tiles_n, splits, kchunk;
  int group_m;        // see GemmParams::group_m
  size_t ws_floats;   // split-K partial floats needed
};

// Launch one planned GEMM on `stream` (grid = tiles*splits x batch).
hipError_t launch_gemm(int dtype, const Plan& plan, const GemmParams& p, int batch,
                       hipStream_t stream);

// qa_rms_norm (qa_decoder_ops.hip).
struct RmsParams {
  const uint16_t* x;
  const float* w;
  uint16_t* y;
  int64_t rows, ldx, ldy;
  int n;
  float eps;
};
hipError_t launch_rms_norm(int dtype, const RmsParams& p, hipStream_t stream);

// qa_qk_norm_rope (qa_decoder_ops.hip).
struct RopeParams {
  const uint16_t* qkv;
  const float *qn, *kn, *cos, *sin;
  uint16_t *q_out, *k_cache, *v_cache;
  int64_t rows, ldqkv, pos0, cap, start;
  int nqh, nkvh, hd;
  float eps;
};
hipError_t launch_qk_norm_rope(int dtype, const RopeParams& p, hipStream_t stream);

// qa_attention_prefill (qa_attention.hip).
struct AttnParams {
  const uint16_t *q, *k_cache, *v_cache;
  uint16_t* out;
  int64_t rows, cap, q0, ldo;
  int nqh, nkvh, hd;
  float scale;
};
// Audio tower ops (qa_audio_ops.hip).
struct LnParams {
  const uint16_t* x;
  const float* w;
  const float* b;
  uint16_t* y;
  int64_t rows, ldx, ldy;
  int n;
  float eps;
};
struct TableAddParams {
  uint16_t* y;
  const float* table;
  int64_t rows, ldy, n, period;
};
struct WinAttnParams {
  const uint16_t* qkv;
  uint16_t* out;
  int64_t s, wlen, ldqkv, ldo;
  int nh;
  float scale;
};
hipError_t launch_layer_norm(int dtype, const LnParams& p, hipStream_t stream);
hipError_t launch_add_table(int dtype, const TableAddParams& p, hipStream_t stream);
hipError_t launch_window_attention(int dtype, const WinAttnParams& p, hipStream_t stream);

// p16: probabilities rounded once to the 16-bit format (else two 16-bit terms).
hipError_t launch_attention(int dtype, const AttnParams& p, bool p16, hipStream_t stream);


}  // namespace qa
