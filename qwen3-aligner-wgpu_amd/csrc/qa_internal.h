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
  TILE_64x64 = 4,    // waves of 32(m) x 64(n)
  TILE_128x192 = 5,  // waves of 64(m) x 96(n)
  TILE_256x256 = 6,  // one k group of 2x4 waves of 128(m) x 64(n)
  TILE_64x64_P2 = 7, // 64x64 with two 64-deep planes per ring stage (one barrier per 128 k)
  TILE_256x160 = 8,  // implicit-GEMM conv only: 4 x 1 waves of 64(m) x 160(n)
  TILE_256x192 = 9,  // 4 x 2 waves of 64(m) x 96(n), two stages, MMA waves issue the DMA
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
    case TILE_64x64:
    case TILE_64x64_P2: return {64, 64};
    case TILE_128x192: return {128, 192};
    case TILE_256x256: return {256, 256};
    case TILE_256x160: return {256, 160};
    case TILE_256x192: return {256, 192};
    default: return {128, 128};
  }
}

// q = floor(n / d) for 0 <= n < 2^31 and 1 <= d < 2^31 as one 32 x 32 -> 64-bit
// multiply and a shift (Granlund & Montgomery, "Division by invariant integers
// using multiplication", PLDI 1994): with l = ceil(log2 d), p = 31 + l and
// m = ceil(2^p / d) < 2^32, m d = 2^p + e with 0 <= e < d, so
// n m / 2^p = n / d + n e / (d 2^p) where the second term is below
// 2^31 / 2^p = 2^-l <= 1 / d, too small to reach the next integer.  The
// kernels' tile enumeration divides block indices by per-launch constants;
// hipcc's generic signed division of a run-time divisor is a float reciprocal,
// a VALU -> SALU move and ~15 scalar corrections per quotient.
struct FastDiv {
  uint32_t m, p;
};
inline FastDiv fastdiv_make(uint32_t d) {
  if (d == 0) return {0, 0};  // never divided by (no tiles, nothing launched)
  uint32_t l = 0;
  while ((1ull << l) < d) ++l;
  const uint32_t p = 31 + l;
  return {(uint32_t)(((1ull << p) + d - 1) / d), p};
}
__device__ __forceinline__ int fastdiv(int n, FastDiv f) {
  return (int)(((uint64_t)(uint32_t)n * f.m) >> f.p);
}

// erf-form GELU, 0.5 x (1 + erf(x / sqrt 2)), with erf from Abramowitz &
// Stegun 7.1.26 (|error| <= 1.5e-7) on v_exp_f32 / v_rcp_f32: the form of the
// reference's `audio_bias_gelu` (src/shaders.rs:2593-2625); the CPU twin calls
// libm's erff (src/audio_encoder.rs:196-202).
//   erf(a) = 1 - P(t) e^{-a^2},  t = 1 / (1 + 0.3275911 a),  a >= 0;
// for x < 0 the factor 1 + erf(x / sqrt 2) = P(t) e^{-a^2} is formed directly,
// without cancelling against 1.  Arranged for the VALU (15 instructions, two
// of them quarter-rate transcendentals, against 17): with q = P(t) e^{-a^2} / 2
// (the coefficients halved, an exact scaling), gelu(x) = max(x, -0) - |x| q
// for either sign (x - x q for x >= 0, x q for x < 0: no cancellation on the
// negative side), one FMA that keeps a zero result's sign and propagates NaN;
// 1/sqrt 2 folds into the reciprocal's FMA and the exponent's constant.
// (+inf gives NaN through inf * 0, where 0.5 x (2 - q) gave +inf; an f32 sum
// of 16-bit products does not reach it.)
__device__ __forceinline__ float gelu_erf(float x) {
  constexpr float h = 0.5f;
  const float ax = fabsf(x);
  const float t = __builtin_amdgcn_rcpf(fmaf(ax, 0.3275911f * 0.70710678118654752f, 1.0f));
  const float e = __builtin_amdgcn_exp2f(x * x * (-0.5f * 1.44269504088896341f));  // e^{-a^2}
  const float p = (((h * 1.061405429f * t - h * 1.453152027f) * t + h * 1.421413741f) * t -
                   h * 0.284496736f) * t + h * 0.254829592f;
  // max(x, -0) as one v_max_f32: fmaxf adds a canonicalising v_max first,
  // which only matters for a NaN x, and a NaN x makes the FMA NaN anyway.
  // The instruction does not read %2 (e): that operand only orders the
  // statement after x * x, a compiler instruction reading x, ahead of which
  // the compiler puts any wait state x's producer needs (an MFMA's result,
  // in the register-staged GEMM); it puts none ahead of an asm statement.
  float mx;
  asm("v_max_f32_e64 %0, %1, neg(0)" : "=v"(mx) : "v"(x), "v"(e));
  return fmaf(-ax, p * t * e, mx);
}

// x + the f16 value in the low (hi = false) or high half of w, in f32 with
// one rounding (the sum an f32 add of the widened value gives): v_fma_mix_f32
// reads the half as an f16 operand, without a widening instruction.  x must
// not come straight from a transcendental or an MFMA (an asm statement gets
// no wait state ahead of it): the callers pass values read from LDS or
// memory, or produced by ordinary VALU instructions.
template <bool HI>
__device__ __forceinline__ float add_f16_half(uint32_t w, float x) {
  float r;
  if constexpr (HI)
    asm("v_fma_mix_f32 %0, %1, 1.0, %2 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(r) : "v"(w), "v"(x));
  else
    asm("v_fma_mix_f32 %0, %1, 1.0, %2 op_sel_hi:[1,0,0]" : "=v"(r) : "v"(w), "v"(x));
  return r;
}

// g sigmoid(g) u with sigmoid(g) = 1 / (1 + 2^(-g log2 e)), in f32 on the
// 16-bit g and u: the reference GPU kernel's form (src/shaders.rs:1411-1450).
__device__ __forceinline__ float silu_mul(float g, float u) {
  constexpr float log2e = 1.44269504088896341f;
  return g * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-g * log2e)) * u;
}

// Two f16 SiLU.up outputs packed in one word: silu_mul on the f16-rounded g
// and u, then one round-to-nearest-even to f16 of each f32 result, bit for
// bit (qah_check_silu_f16x2 compares it with that reference on 16.7 M random
// and special inputs), in 7.5 VALU instructions per output instead of 11.
// g and u are rounded in pairs (v_cvt_pk_f16_f32) and read straight as f16
// operands of v_fma_mix (no widening); each v_fma_mix_f32 rounds its product
// once to f32, as the multiply it replaces, and the addend neg(0) keeps the
// sign of a -0 product.  (v_fma_mixlo / mixhi_f16 would save the final
// conversion but round the exact product straight to f16: 1 ulp off the
// f32-then-f16 result in about 1 of 28000 outputs.)  The s_nop is the wait
// state gfx950 needs before a VALU instruction reads the result of a
// transcendental (v_rcp_f32): the compiler inserts it ahead of its own
// instructions but not ahead of an asm statement, which without it read the
// register's previous value (1 + 2^t).
// silu_mul_h2 takes g and u already rounded and packed (gw, uw: two f16
// each, element 0 in the low half); gw and uw must not come straight from a
// transcendental or an MFMA (an asm statement gets no wait state ahead of it).
__device__ __forceinline__ uint32_t silu_mul_h2(uint32_t gw, uint32_t uw) {
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  const float c = -1.44269504088896341f;
  float t0, t1, s0, s1, p0, p1;
  asm("v_fma_mix_f32 %0, %1, %2, 0 op_sel_hi:[1,0,0]" : "=v"(t0) : "v"(gw), "v"(c));
  asm("v_fma_mix_f32 %0, %1, %2, 0 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(t1) : "v"(gw), "v"(c));
  const float r0 = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(t0));
  const float r1 = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(t1));
  asm("s_nop 0\n\tv_fma_mix_f32 %0, %1, %2, neg(0) op_sel_hi:[1,0,0]" : "=v"(s0) : "v"(gw), "v"(r0));
  asm("s_nop 0\n\tv_fma_mix_f32 %0, %1, %2, neg(0) op_sel:[1,0,0] op_sel_hi:[1,0,0]"
      : "=v"(s1) : "v"(gw), "v"(r1));
  asm("v_fma_mix_f32 %0, %1, %2, neg(0) op_sel_hi:[0,1,0]" : "=v"(p0) : "v"(s0), "v"(uw));
  asm("v_fma_mix_f32 %0, %1, %2, neg(0) op_sel:[0,1,0] op_sel_hi:[0,1,0]" : "=v"(p1) : "v"(s1), "v"(uw));
  return __builtin_bit_cast(uint32_t, h2{(_Float16)p0, (_Float16)p1});
}
__device__ __forceinline__ uint32_t silu_mul_f16x2(float g0, float g1, float u0, float u1) {
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  return silu_mul_h2(__builtin_bit_cast(uint32_t, h2{(_Float16)g0, (_Float16)g1}),
                     __builtin_bit_cast(uint32_t, h2{(_Float16)u0, (_Float16)u1}));
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
  // divisions of tile_of by splits, band size group_m * tiles_n, a full band's
  // height group_m and the last band's (launch_gemm fills them)
  FastDiv fd_split, fd_band, fd_rows, fd_last;
  // implicit 3x3 / stride-2 / pad-1 convolution A operand (Plan::conv)
  int cv_c, cv_h, cv_w;  // input channels (multiple of 8, >= 64), height, width
  int cv_ho, cv_wo;      // output height, width
  int cv_tmajor;         // output rows ordered (b, wo, ho) instead of (b, ho, wo)
  // Bytes the NEXT kernel will read (its weights), pulled into the memory-side
  // cache while this one runs; pf_bytes = 0 for none (qa_prefetch_hint).
  const uint16_t* pf;
  int pf_bytes;
#ifdef QA_PHASE_STAMPS
  int stamp_slot;  // record slot of this launch's phase stamps (qa_gemm.hip)
#endif
};

struct Plan {
  int tile;
  int epi;
  bool transb;
  int tiles_m, tiles_n, splits, kchunk;
  int group_m;        // see GemmParams::group_m
  size_t ws_floats;   // split-K partial floats needed
  bool conv = false;  // A is an implicit convolution operand (GemmParams::cv_*)
};

// Launch one planned GEMM on `stream` (grid = tiles*splits x batch).  With
// t0 / t1 set, the GEMM kernel's dispatch records its start / end into them
// (hipExtLaunchKernel).
hipError_t launch_gemm(int dtype, const Plan& plan, const GemmParams& p, int batch,
                       hipStream_t stream, hipEvent_t t0 = nullptr, hipEvent_t t1 = nullptr);

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

// Direct 3x3 / stride-2 / pad-1 convolution of a single-channel input
// (qa_conv.hip): the first conv level, where the implicit GEMM's 8-channel
// chunks do not apply.
struct Conv1Params {
  const uint16_t* x;     // [b][h][w]
  const uint16_t* w;     // [c_out][ldw], taps kh * 3 + kw
  const uint16_t* bias;  // [c_out] or nullptr
  uint16_t* y;           // [M][c_out]
  int64_t M;
  int h, w_in, ho, wo, c_out, ldw, tmajor, gelu;
};
hipError_t launch_conv1(int dtype, const Conv1Params& p, hipStream_t stream);

// Log-mel front end (qa_mel.hip).
constexpr int kMelFramesPerBlock = 9;  // frames per block of mel_log_kernel
struct MelParams {
  const float* x;      // samples [n]
  const float* filt;   // [n_mels][201]
  float* logmel;       // workspace [n_mels][frames]
  float* bmax;         // workspace [nblocks]
  double* tw;          // workspace [400][2]: cos, sin of 2 pi j / 400
  int32_t* sup;        // workspace [n_mels][2]: each filter's nonzero bins [lo, hi)
  uint16_t* out;       // [n_chunks][n_mels][cs]
  int64_t n, frames;
  int n_mels, cs, n_chunks, nblocks;
};
hipError_t launch_log_mel(int dtype, const MelParams& p, hipStream_t stream);

// The aligner's input rows and timestamp head (qa_head.hip).
struct EmbedParams {
  const int32_t* src;
  const uint16_t* table;
  const uint16_t* audio;
  uint16_t* out;
  int64_t rows, vocab, n_audio;
  int hidden;
};
hipError_t launch_embed_scatter(const EmbedParams& p, hipStream_t stream);
struct HeadParams {
  const int32_t* pos;
  const uint16_t* h;
  const float* w;
  const float* score;
  float* normed;  // workspace [rows][n]
  float* logits;  // [rows][labels]
  int32_t* cls;   // [rows]
  int64_t rows, h_rows, ldh, labels;
  int n;
  float eps;
};
hipError_t launch_timestamp_head(int dtype, const HeadParams& p, hipStream_t stream);

// p16: probabilities rounded once to the 16-bit format (else two 16-bit terms).
hipError_t launch_attention(int dtype, const AttnParams& p, bool p16, hipStream_t stream);


}  // namespace qa
