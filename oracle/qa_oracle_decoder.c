/*
 * qa_oracle_decoder.c -- CPU restatement of the reference's decoder prefill
 * ops around the projections: RMSNorm, per-head q/k RMSNorm + rotate-half
 * RoPE with the KV-cache write, and causal GQA attention.
 *
 * TEST INFRASTRUCTURE ONLY (see qa_oracle.h): the checker for
 * qa_rms_norm / qa_qk_norm_rope / qa_attention_prefill, never linked into the
 * product.
 *
 * Each function follows the reference's CPU decoder (src/cpu_decoder.rs)
 * step by step, including its accumulation orders and rounding points:
 *   or_rms_norm      rms_norm_row          src/cpu_decoder.rs:288-300
 *   or_qk_norm_rope  norm_rope_head + the
 *                    cache writes          src/cpu_decoder.rs:302-322, :464-491
 *   or_attention     attention             src/cpu_decoder.rs:324-411
 * The cache layouts are the ones qa.h defines for this build (K [h][cap][hd],
 * V transposed [h][hd][cap] with key t at column or_vperm(t)); the reference
 * keeps both as [h][cap][hd] f32 (src/cpu_decoder.rs:470-490), which holds
 * the same values.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>

#include "qa_oracle.h"

/* Column of key t in the transposed V cache: bits 2 and 3 of t swapped
 * (self-inverse; keys stay within their aligned group of 16). */
int64_t or_vperm(int64_t t) { return (t & ~(int64_t)12) | ((t & 4) << 1) | ((t & 8) >> 1); }

/* src/cpu_decoder.rs:288-300: f32 sum of squares in element order,
 * inv = 1/sqrt(sum2/n + eps), out = r16(x * inv * w). */
void or_rms_norm(int dtype, int64_t rows, int64_t n, const uint16_t* x, int64_t ldx,
                 const float* w, float eps, uint16_t* y, int64_t ldy) {
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    const uint16_t* xr = x + r * ldx;
    float sum2 = 0.0f;
    for (int64_t i = 0; i < n; ++i) {
      const float f = or_h16_to_f32(xr[i], dtype);
      sum2 += f * f;
    }
    const float inv = 1.0f / sqrtf(sum2 / (float)n + eps);
    for (int64_t i = 0; i < n; ++i)
      y[r * ldy + i] = or_h16_from_f32(or_h16_to_f32(xr[i], dtype) * inv * w[i], dtype);
  }
}

/* One head row (src/cpu_decoder.rs:302-322): inv from the raw 16-bit values,
 * x_j = raw_j * inv * nw_j, partner p = j +- hd/2 with sign -1 for the first
 * half, out_j = r16(x_j * cos_j + sign * x_p * sin_j). */
static void norm_rope_head(int dtype, const uint16_t* raw, const float* nw, const float* cs,
                           const float* sn, int hd, float eps, uint16_t* out, int64_t ostride) {
  const int half = hd / 2;
  float sum2 = 0.0f;
  for (int j = 0; j < hd; ++j) {
    const float f = or_h16_to_f32(raw[j], dtype);
    sum2 += f * f;
  }
  const float inv = 1.0f / sqrtf(sum2 / (float)hd + eps);
  for (int j = 0; j < hd; ++j) {
    const float xj = or_h16_to_f32(raw[j], dtype) * inv * nw[j];
    const int pj = j < half ? j + half : j - half;
    const float sign = j < half ? -1.0f : 1.0f;
    const float xp = or_h16_to_f32(raw[pj], dtype) * inv * nw[pj];
    out[(int64_t)j * ostride] = or_h16_from_f32(xj * cs[j] + sign * xp * sn[j], dtype);
  }
}

/* src/cpu_decoder.rs:464-491 for rows r = 0..rows-1 at positions pos0 + r:
 * q heads normed + roped into q_out [nqh][rows][hd]; k heads normed + roped
 * into k_cache [nkvh][cap][hd] at row start + r; v heads copied verbatim into
 * the transposed v_cache [nkvh][hd][cap] at column or_vperm(start + r).  cos / sin are
 * [pos][hd] f32 tables (src/mrope.rs:55-82). */
void or_qk_norm_rope(int dtype, int64_t rows, int nqh, int nkvh, int hd, const uint16_t* qkv,
                     int64_t ldqkv, const float* qn, const float* kn, const float* cos_t,
                     const float* sin_t, int64_t pos0, float eps, uint16_t* q_out,
                     uint16_t* k_cache, uint16_t* v_cache, int64_t cap, int64_t start) {
  const int64_t q_dim = (int64_t)nqh * hd, kv_dim = (int64_t)nkvh * hd;
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    const uint16_t* row = qkv + r * ldqkv;
    const float* cs = cos_t + (pos0 + r) * hd;
    const float* sn = sin_t + (pos0 + r) * hd;
    for (int h = 0; h < nqh; ++h)
      norm_rope_head(dtype, row + (int64_t)h * hd, qn, cs, sn, hd, eps,
                     q_out + ((int64_t)h * rows + r) * hd, 1);
    for (int h = 0; h < nkvh; ++h) {
      norm_rope_head(dtype, row + q_dim + (int64_t)h * hd, kn, cs, sn, hd, eps,
                     k_cache + ((int64_t)h * cap + start + r) * hd, 1);
      const uint16_t* v = row + q_dim + kv_dim + (int64_t)h * hd;
      for (int j = 0; j < hd; ++j) v_cache[((int64_t)h * hd + j) * cap + or_vperm(start + r)] = v[j];
    }
  }
}

/* src/cpu_decoder.rs:324-411.  Row r (position q0 + r) of q head h attends to
 * cache rows 0..min(q0 + r, cap - 1) of kv head h / (nqh / nkvh):
 *   s_t = dot(q, k_t) * (1 / sqrt(hd)), the dot in four interleaved f32
 *         partial sums over j = 4i..4i+3, combined (a0 + a1) + (a2 + a3);
 *   p_t = exp(s_t - max_t s_t), sum in key order, inv = 1 / sum;
 *   acc_j = sum_t (p_t * inv) * v_t[j] in key order;  out = r16(acc).
 * q is head-major [nqh][rows][hd]; out is [rows][nqh * hd] (row stride ldo). */
void or_attention(int dtype, int64_t rows, int nqh, int nkvh, int hd, const uint16_t* q,
                  const uint16_t* k_cache, const uint16_t* v_cache, int64_t cap, int64_t q0,
                  uint16_t* out, int64_t ldo) {
  const float scale = 1.0f / sqrtf((float)hd);
  const int rep = nqh / nkvh;
#pragma omp parallel
  {
    float* scores = (float*)malloc(sizeof(float) * (size_t)cap);
    float* acc = (float*)malloc(sizeof(float) * (size_t)hd);
    float* qrow = (float*)malloc(sizeof(float) * (size_t)hd);
    float* krow = (float*)malloc(sizeof(float) * (size_t)hd);
#pragma omp for schedule(dynamic, 4)
    for (int64_t hi = 0; hi < rows * nqh; ++hi) {
      const int64_t r = hi / nqh;
      const int h = (int)(hi % nqh);
      const int64_t pos = q0 + r;
      const int64_t valid = pos + 1 < cap ? pos + 1 : cap;
      for (int j = 0; j < hd; ++j) qrow[j] = or_h16_to_f32(q[((int64_t)h * rows + r) * hd + j], dtype);
      const int kh = h / rep;
      const uint16_t* kb = k_cache + (int64_t)kh * cap * hd;
      const uint16_t* vb = v_cache + (int64_t)kh * hd * cap;
      float best = -INFINITY;
      for (int64_t t = 0; t < valid; ++t) {
        for (int j = 0; j < hd; ++j) krow[j] = or_h16_to_f32(kb[t * hd + j], dtype);
        float a[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        for (int i = 0; i < hd / 4; ++i) {
          const int j = 4 * i;
          a[0] += qrow[j] * krow[j];
          a[1] += qrow[j + 1] * krow[j + 1];
          a[2] += qrow[j + 2] * krow[j + 2];
          a[3] += qrow[j + 3] * krow[j + 3];
        }
        const float dot = (a[0] + a[1]) + (a[2] + a[3]);
        const float s = dot * scale;
        scores[t] = s;
        if (s > best) best = s;
      }
      float sum = 0.0f;
      for (int64_t t = 0; t < valid; ++t) {
        scores[t] = expf(scores[t] - best);
        sum += scores[t];
      }
      const float inv = 1.0f / sum;
      for (int j = 0; j < hd; ++j) acc[j] = 0.0f;
      for (int64_t t = 0; t < valid; ++t) {
        const float wt = scores[t] * inv;
        const int64_t col = or_vperm(t);
        for (int j = 0; j < hd; ++j) acc[j] += wt * or_h16_to_f32(vb[(int64_t)j * cap + col], dtype);
      }
      for (int j = 0; j < hd; ++j) out[r * ldo + (int64_t)h * hd + j] = or_h16_from_f32(acc[j], dtype);
    }
    free(scores);
    free(acc);
    free(qrow);
    free(krow);
  }
}
