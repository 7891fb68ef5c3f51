/*
 * qa_oracle.h -- CPU restatement of the reference's linear-layer path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (libqa.so, the host mirror,
 * the Python binding) links, loads or calls this code.  Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg use it, and only as
 * the checker / the timed CPU baseline, never as the thing measured on the GPU.
 *
 * What it restates (reference = eclipse005/qwen3-aligner-wgpu):
 *   - 16-bit storage formats and their rounding:
 *       f16  : IEEE binary16 round-to-nearest-even, as half 2.7.1's
 *              f16::from_f32 used by src/cpu_decoder.rs:68,89 and
 *              src/half16.rs:40-47.
 *       bf16 : src/shaders.rs:169-179 rne_bf16_bits,
 *              (u + 0x7FFF + ((u >> 16) & 1)) >> 16.
 *   - the f32 GEMM out = beta*out + x.W^T of the gemm crate 0.18.2 wrapper
 *     gemm_row_major (src/cpu_decoder.rs:583-610, src/cpu_tensor.rs:82-108).
 *   - the linear op with one rounding per output (src/shaders.rs:2045-2073,
 *     src/cpu_decoder.rs:59-97), the SiLU.up loop (src/cpu_decoder.rs:496-505)
 *     and the erf-form GELU (src/audio_encoder.rs:196-202).
 *
 * Parity pins (each function is checked in tests/test_oracle.py):
 *   or_f16_from_f32  : numpy float32->float16 cast over the reference's
 *                      halfway grid + 500k LCG sweep (src/shaders.rs:191-243).
 *   or_bf16_from_f32 : KAT 0.1 -> 0x3DCD (src/half16.rs:113-119); torch's
 *                      float32->bfloat16 cast over the same grid and sweep.
 *   or_gemm_f32      : the reference KAT gemm_row_major_matches_naive
 *                      (src/cpu_decoder.rs:620-646, worst |d| < 1e-3) and
 *                      numpy float64 matmul.
 *   or_gemm_f64      : numpy float64 matmul (to 1e-12 relative).
 *   or_linear        : invariants (zero A keeps C, bias-only, fused-row
 *                      splits), f64 closed forms, SiLU brute force over all
 *                      65536 f16 gate values, GELU against math.erf.
 */
#ifndef QA_ORACLE_H
#define QA_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { OR_F16 = 0, OR_BF16 = 1 };
enum {
  OR_ACCUMULATE = 1u << 0,
  OR_EPI_GELU = 1u << 1,
  OR_EPI_SILU_MUL = 1u << 2,
  OR_TRANSB = 1u << 3,
  OR_BIAS_ROWS = 1u << 4,
  OR_EXACT = 1u << 8, /* accumulate in f64 instead of the blocked f32 GEMM */
};

uint16_t or_f16_from_f32(float x);
float or_f16_to_f32(uint16_t h);
uint16_t or_bf16_from_f32(float x);
float or_bf16_to_f32(uint16_t h);
uint16_t or_h16_from_f32(float x, int dtype);
float or_h16_to_f32(uint16_t h, int dtype);

/* Bulk conversions (n elements). */
void or_h16_to_f32_n(const uint16_t* src, float* dst, int64_t n, int dtype);
void or_f32_to_h16_n(const float* src, uint16_t* dst, int64_t n, int dtype);

/* out[i*ldo+j] = beta*out[i*ldo+j] + sum_p x[i*ldx+p]*w[j*ldw+p]
 * (out is only read when beta != 0, as the gemm crate's read_dst flag). */
void or_gemm_f32(int64_t m, int64_t n, int64_t k, const float* x, int64_t ldx,
                 const float* w, int64_t ldw, float* out, int64_t ldo, float beta);
/* Sequential f32 triple loop -- the naive side of the reference KAT. */
void or_gemm_f32_naive(int64_t m, int64_t n, int64_t k, const float* x, int64_t ldx,
                       const float* w, int64_t ldw, float* out, int64_t ldo);
/* f64 triple loop over f32 inputs: the exact-value pin. */
void or_gemm_f64(int64_t m, int64_t n, int64_t k, const float* x, int64_t ldx,
                 const float* w, int64_t ldw, double* out, int64_t ldo);

float or_silu_mul(float g, float u); /* g/(1+exp(-g)) * u, f32 */
float or_gelu(float x);              /* 0.5x(1+erf(x/sqrt2)), f32 */

/* The linear op, same fields and meaning as qa_linear_desc (include/qa.h). */
typedef struct or_linear_desc {
  uint32_t dtype;
  uint32_t flags;
  int64_t m, n, k;
  int64_t lda, ldb, ldc;
  const uint16_t* a;
  const uint16_t* w;
  uint16_t* c;
  const uint16_t* bias;
  int64_t batch, bsa, bsb, bsc;
} or_linear_desc;

/* Returns 0 on success, -1 on an invalid descriptor. */
int or_linear(const or_linear_desc* d);

/* Number of OpenMP threads the oracle's parallel loops use. */
int or_num_threads(void);
void or_set_threads(int n);

/* ---- decoder prefill ops around the projections (qa_oracle_decoder.c) ----
 * Parity pins (tests/test_oracle_decoder.py): f64 closed forms of RMSNorm and
 * of norm + rotate-half RoPE (including pos 0 = plain norm and the pairwise
 * rotation invariant), brute-force f64 softmax attention, the causal
 * invariant (a row ignores later keys), uniform scores averaging V, and GQA
 * head sharing. */
int64_t or_vperm(int64_t t); /* V-cache column of key t (bits 2 and 3 swapped) */
void or_rms_norm(int dtype, int64_t rows, int64_t n, const uint16_t* x, int64_t ldx,
                 const float* w, float eps, uint16_t* y, int64_t ldy);
void or_qk_norm_rope(int dtype, int64_t rows, int nqh, int nkvh, int hd, const uint16_t* qkv,
                     int64_t ldqkv, const float* qn, const float* kn, const float* cos_t,
                     const float* sin_t, int64_t pos0, float eps, uint16_t* q_out,
                     uint16_t* k_cache, uint16_t* v_cache, int64_t cap, int64_t start);
void or_attention(int dtype, int64_t rows, int nqh, int nkvh, int hd, const uint16_t* q,
                  const uint16_t* k_cache, const uint16_t* v_cache, int64_t cap, int64_t q0,
                  uint16_t* out, int64_t ldo);

/* ---- audio tower ops around the projections (qa_oracle_audio.c) ----
 * Parity pins (tests/test_oracle_audio.py): f64 closed forms of LayerNorm
 * (mean 0 / variance 1 before the affine map, the affine map itself), of
 * per-window softmax attention (brute force, plus: a window ignores every
 * other window, identical keys average V, the last window holds the
 * remainder), the position add (table row r % period), and the sinusoid
 * table against its definition (sin/cos halves, position 0). */
void or_layer_norm(int dtype, int64_t rows, int64_t n, const uint16_t* x, int64_t ldx,
                   const float* w, const float* b, float eps, uint16_t* y, int64_t ldy);
void or_window_attention(int dtype, int64_t s, int nh, int hd, int64_t wlen, const uint16_t* qkv,
                         int64_t ldqkv, uint16_t* out, int64_t ldo);
void or_add_position_table(int dtype, int64_t rows, int64_t n, uint16_t* y, int64_t ldy,
                           const float* table, int64_t period);
void or_sinusoid_table(int64_t positions, int64_t dm, float* table);
/* Pins (tests/test_oracle_audio.py): torch's float64 conv2d (stride 2,
 * padding 1) on the same values in NCHW with the checkpoint weight layout,
 * and a restatement of the reference's im2col + GEMM at small sizes. */
void or_conv3x3s2(int dtype, int64_t batch, int64_t h, int64_t w, int64_t c_in, int64_t c_out,
                  const uint16_t* x, const uint16_t* weight, int64_t ldw, const uint16_t* bias,
                  int gelu, int tmajor, int64_t m0, int64_t m1, uint16_t* y);
/* The log-mel front end (src/mel.rs).  Pins (tests/test_oracle_mel.py):
 * numpy's rfft of the same reflect-padded Hann-windowed frames, the slaney
 * scale's fixed points (1 kHz = mel 15, mel <-> Hz round trip), each filter a
 * triangle of unit area, a pure tone peaking in the bin that holds it, and
 * the uniform log10(c^2) / 4 shift of a signal scaled by c. */
void or_mel_filterbank(int n_mels, int n_fft, int sr, float* out);
void or_stft_power(const float* x, int64_t n, int n_fft, int hop, double* power);
void or_log_mel(const float* x, int64_t n, int n_mels, const float* filt, float* out);
/* The timestamp head.  Pins (tests/test_oracle_head.py): the f64 closed form
 * of the folded norm and the logits, and a constructed case whose argmax is
 * known (score rows aligned with the normed rows, first index on ties). */
void or_timestamp_head(int dtype, int64_t rows, const int32_t* pos, const uint16_t* h,
                       int64_t ldh, int64_t n, const float* w, float eps, const float* score,
                       int64_t labels, double* logits, int32_t* cls);

/* The reference's CPU audio tower in f32 throughout (CpuAudioEncoder::forward,
 * src/audio_encoder.rs:754-832; one f16 narrowing at the end,
 * src/align_inference.rs:124-131).  Pins (tests/test_oracle_audio.py): each
 * equals its 16-bit twin above on inputs that are 16-bit values, up to that
 * twin's final rounding; f64 closed forms (LayerNorm, attention, conv against
 * torch conv2d); the linear against numpy f64 matmul + bias. */
void or_linear_f32(int64_t m, int64_t n, int64_t k, const float* x, int64_t ldx,
                   const uint16_t* w, int dtype, const float* bias, float* y, int64_t ldy);
void or_layer_norm_f32(int64_t rows, int64_t n, const float* x, const float* w, const float* b,
                       float eps, float* y);
void or_gelu_f32_n(float* x, int64_t n);
void or_window_attention_f32(int64_t s, int nh, int hd, int64_t wlen, const float* q,
                             const float* k, const float* v, int64_t ld, float* out);
void or_conv3x3s2_f32(int64_t batch, int64_t h, int64_t w, int64_t c_in, int64_t c_out,
                      const float* x, const float* weight, int64_t ldw, const float* bias,
                      int gelu, int tmajor, float* y);
/* The head's folded norm alone, f32 rows y [rows][n] (src/align_inference.rs:766-783). */
void or_head_fold(int dtype, int64_t rows, const int32_t* pos, const uint16_t* h, int64_t ldh,
                  int64_t n, const float* w, float eps, float* y);

#ifdef __cplusplus
}
#endif
#endif
