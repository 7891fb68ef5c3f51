/*
 * qa_oracle_audio.c -- CPU restatement of the audio tower's non-GEMM ops.
 *
 * TEST INFRASTRUCTURE ONLY (see qa_oracle.h): the checker for
 * qa_layer_norm, qa_window_attention, qa_add_position_table and
 * qa_conv2d_3x3s2.  Compiled
 * with -ffp-contract=off so the f32 arithmetic is the CPU path's, operation
 * for operation.  Inputs and outputs are 16-bit storage (the GPU tower's
 * buffers); every value is widened to f32 and each output rounded once.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>

#include "qa_oracle.h"

/* CpuAudioLayerNorm::forward (src/audio_encoder.rs:147-171): mean and
 * variance by sequential f32 sums, inv_std = 1 / sqrt(var + eps),
 * y = (x - mean) * inv_std * w + b. */
void or_layer_norm(int dtype, int64_t rows, int64_t n, const uint16_t* x, int64_t ldx,
                   const float* w, const float* b, float eps, uint16_t* y, int64_t ldy) {
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    const uint16_t* xr = x + r * ldx;
    float mean = 0.f;
    for (int64_t j = 0; j < n; ++j) mean += or_h16_to_f32(xr[j], dtype);
    mean /= (float)n;
    float var = 0.f;
    for (int64_t j = 0; j < n; ++j) {
      const float d = or_h16_to_f32(xr[j], dtype) - mean;
      var += d * d;
    }
    var /= (float)n;
    const float inv_std = 1.0f / sqrtf(var + eps);
    for (int64_t j = 0; j < n; ++j) {
      const float v = (or_h16_to_f32(xr[j], dtype) - mean) * inv_std * w[j] + b[j];
      y[r * ldy + j] = or_h16_from_f32(v, dtype);
    }
  }
}

/* attention_window (src/audio_encoder.rs:561-616) over every window of
 * `wlen` tokens (CpuAudioAttention::flat, :517-536: the last window holds the
 * remainder; a sequence no longer than one window is one window).  Head h
 * reads q, k, v at columns h*hd, dm + h*hd, 2*dm + h*hd of the fused qkv row
 * (dm = nh*hd); scores = (q.k, sequential f32 dot) * scale, exp(s - max),
 * weights = e * (1 / sum), out = sum_k w v accumulated in key order. */
void or_window_attention(int dtype, int64_t s, int nh, int hd, int64_t wlen, const uint16_t* qkv,
                         int64_t ldqkv, uint16_t* out, int64_t ldo) {
  const int64_t dm = (int64_t)nh * hd;
  const float scale = 1.0f / sqrtf((float)hd);
  const int64_t nwin = (s + wlen - 1) / wlen;
#pragma omp parallel for collapse(2) schedule(dynamic)
  for (int64_t wi = 0; wi < nwin; ++wi)
    for (int h = 0; h < nh; ++h) {
      const int64_t st = wi * wlen;
      const int64_t len = (st + wlen <= s) ? wlen : s - st;
      float* sc = (float*)malloc((size_t)len * sizeof(float));
      float* kq = (float*)malloc((size_t)hd * sizeof(float));
      float* acc = (float*)malloc((size_t)hd * sizeof(float));
      for (int64_t qi = 0; qi < len; ++qi) {
        const uint16_t* q = qkv + (st + qi) * ldqkv + (int64_t)h * hd;
        for (int j = 0; j < hd; ++j) kq[j] = or_h16_to_f32(q[j], dtype);
        float mx = -INFINITY;
        for (int64_t ki = 0; ki < len; ++ki) {
          const uint16_t* k = qkv + (st + ki) * ldqkv + dm + (int64_t)h * hd;
          float dot = 0.f;
          for (int j = 0; j < hd; ++j) dot += kq[j] * or_h16_to_f32(k[j], dtype);
          sc[ki] = dot * scale;
          if (sc[ki] > mx) mx = sc[ki];
        }
        float sum = 0.f;
        for (int64_t ki = 0; ki < len; ++ki) {
          sc[ki] = expf(sc[ki] - mx);
          sum += sc[ki];
        }
        const float inv = 1.0f / sum;
        for (int j = 0; j < hd; ++j) acc[j] = 0.f;
        for (int64_t ki = 0; ki < len; ++ki) {
          const float wgt = sc[ki] * inv;
          const uint16_t* v = qkv + (st + ki) * ldqkv + 2 * dm + (int64_t)h * hd;
          for (int j = 0; j < hd; ++j) acc[j] += wgt * or_h16_to_f32(v[j], dtype);
        }
        uint16_t* o = out + (st + qi) * ldo + (int64_t)h * hd;
        for (int j = 0; j < hd; ++j) o[j] = or_h16_from_f32(acc[j], dtype);
      }
      free(sc);
      free(kq);
      free(acc);
    }
}

/* The sinusoidal position add after conv_out (CpuConvStem::forward_stages,
 * src/audio_encoder.rs:331-343; the GPU tower's add_pe): token r gets the
 * table row r % period (its position within its chunk), y = r16(y + pe). */
void or_add_position_table(int dtype, int64_t rows, int64_t n, uint16_t* y, int64_t ldy,
                           const float* table, int64_t period) {
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    const float* pe = table + (r % period) * n;
    for (int64_t j = 0; j < n; ++j)
      y[r * ldy + j] = or_h16_from_f32(or_h16_to_f32(y[r * ldy + j], dtype) + pe[j], dtype);
  }
}

/* CpuConvStem::load (src/audio_encoder.rs:270-283): pe[p][i] = sin(p * e^(-i lt)),
 * pe[p][half + i] = cos(...), lt = ln(10000) / (half - 1), in f64, stored f32. */
void or_sinusoid_table(int64_t positions, int64_t dm, float* table) {
  const int64_t half = dm / 2;
  const double lt = log(10000.0) / ((double)half - 1.0);
  for (int64_t p = 0; p < positions; ++p)
    for (int64_t i = 0; i < half; ++i) {
      const double a = (double)p * exp(-(double)i * lt);
      table[p * dm + i] = (float)sin(a);
      table[p * dm + half + i] = (float)cos(a);
    }
}

/* One conv level of the stem on the GPU tower's layouts (qa_conv2d_3x3s2):
 * 3x3, stride 2, pad 1 (im2col_3x3_s2p1, src/audio_encoder.rs:204-236), the
 * sum over k = (kh * 3 + kw) * c_in + ic accumulated in f64 (the exact value
 * the f32 GEMM of conv_block approximates, :376-447), + bias, then the erf
 * GELU in f32 when `gelu` (:196-202, 439-441) and one rounding.  x is
 * [batch][h][w][c_in]; weight [c_out][ldw]; rows m0..m1-1 of y [M][c_out],
 * row order (b, ho, wo), or (b, wo, ho) when `tmajor`. */
void or_conv3x3s2(int dtype, int64_t batch, int64_t h, int64_t w, int64_t c_in, int64_t c_out,
                  const uint16_t* x, const uint16_t* weight, int64_t ldw, const uint16_t* bias,
                  int gelu, int tmajor, int64_t m0, int64_t m1, uint16_t* y) {
  const int64_t ho = (h - 1) / 2 + 1, wo = (w - 1) / 2 + 1, plane = ho * wo;
  const int64_t nx = batch * h * w * c_in, nw = c_out * ldw;
  float* xf = (float*)malloc((size_t)nx * sizeof(float));
  float* wf = (float*)malloc((size_t)nw * sizeof(float));
  or_h16_to_f32_n(x, xf, nx, dtype);
  or_h16_to_f32_n(weight, wf, nw, dtype);
#pragma omp parallel for schedule(dynamic, 4)
  for (int64_t m = m0; m < m1; ++m) {
    const int64_t b = m / plane, q = m % plane;
    const int64_t oh = tmajor ? q % ho : q / wo;
    const int64_t ow = tmajor ? q / ho : q % wo;
    for (int64_t oc = 0; oc < c_out; ++oc) {
      const float* wr = wf + oc * ldw;
      double acc = 0.0;  /* products of two f32 values are exact in f64 */
      for (int kh = 0; kh < 3; ++kh)
        for (int kw = 0; kw < 3; ++kw) {
          const int64_t ih = 2 * oh + kh - 1, iw = 2 * ow + kw - 1;
          if (ih < 0 || ih >= h || iw < 0 || iw >= w) continue;
          const float* xp = xf + ((b * h + ih) * w + iw) * c_in;
          const float* wp = wr + (kh * 3 + kw) * c_in;
          for (int64_t ic = 0; ic < c_in; ++ic) acc += (double)xp[ic] * (double)wp[ic];
        }
      if (bias) acc += (double)or_h16_to_f32(bias[oc], dtype);
      float v = (float)acc;
      if (gelu) v = or_gelu(v);
      y[(m - m0) * c_out + oc] = or_h16_from_f32(v, dtype);
    }
  }
  free(xf);
  free(wf);
}

/* create_mel_filterbank (src/mel.rs:100-154), restated: slaney mel scale
 * (linear below 1 kHz at 200/3 Hz per mel, logarithmic above with step
 * ln(6.4) / 27), n_mels + 2 points evenly spaced in mel over 0 .. sr / 2,
 * triangles over bin frequencies j sr / n_fft, each scaled by
 * 2 / (f[i+2] - f[i]); f64 math, f32 storage and f32 scaling. */
static double or_hz_to_mel(double f) {
  const double f_sp = 200.0 / 3.0, min_log_hz = 1000.0, logstep = log(6.4) / 27.0;
  return f < min_log_hz ? f / f_sp : min_log_hz / f_sp + log(f / min_log_hz) / logstep;
}
static double or_mel_to_hz(double m) {
  const double f_sp = 200.0 / 3.0, min_log_hz = 1000.0, logstep = log(6.4) / 27.0;
  const double min_log_mel = min_log_hz / f_sp;
  return m < min_log_mel ? f_sp * m : min_log_hz * exp(logstep * (m - min_log_mel));
}
void or_mel_filterbank(int n_mels, int n_fft, int sr, float* out) {
  const int nf = n_fft / 2 + 1;
  double* ff = (double*)malloc(sizeof(double) * (size_t)(n_mels + 2));
  const double lo = or_hz_to_mel(0.0), hi = or_hz_to_mel(sr / 2.0);
  for (int i = 0; i < n_mels + 2; ++i) ff[i] = or_mel_to_hz(lo + (hi - lo) * i / (double)(n_mels + 1));
  for (int i = 0; i < n_mels; ++i)
    for (int j = 0; j < nf; ++j) {
      const double f = (double)j * sr / n_fft;
      const double down = (f - ff[i]) / (ff[i + 1] - ff[i]);
      const double up = (ff[i + 2] - f) / (ff[i + 2] - ff[i + 1]);
      double v = down < up ? down : up;
      if (v < 0.0) v = 0.0;
      out[i * nf + j] = (float)v * (float)(2.0 / (ff[i + 2] - ff[i]));
    }
  free(ff);
}

/* |X_k|^2 of the centered STFT (src/mel.rs:47-98,203-214): reflect padding of
 * n_fft / 2 without repeating the edge, periodic Hann 0.5 (1 - cos(2 pi j /
 * n_fft)), frames every hop samples, the last frame dropped; a direct DFT in
 * f64.  power [frames][n_fft / 2 + 1], frames = n / hop. */
void or_stft_power(const float* x, int64_t n, int n_fft, int hop, double* power) {
  const int nf = n_fft / 2 + 1;
  const int64_t frames = n / hop, pad = n_fft / 2;
  double* cs = (double*)malloc(sizeof(double) * (size_t)n_fft);
  double* sn = (double*)malloc(sizeof(double) * (size_t)n_fft);
  for (int j = 0; j < n_fft; ++j) {
    cs[j] = cos(2.0 * 3.14159265358979323846 * j / n_fft);
    sn[j] = sin(2.0 * 3.14159265358979323846 * j / n_fft);
  }
#pragma omp parallel for schedule(static)
  for (int64_t f = 0; f < frames; ++f) {
    double fr[4096];
    for (int j = 0; j < n_fft; ++j) {
      int64_t i = f * hop + j - pad;
      const int64_t period = 2 * (n - 1);
      if (n > 1) {
        i %= period;
        if (i < 0) i += period;
        if (i > n - 1) i = period - i;
      } else {
        i = 0;
      }
      fr[j] = (double)x[i] * 0.5 * (1.0 - cs[j]);
    }
    for (int k = 0; k < nf; ++k) {
      double re = 0.0, im = 0.0;
      int idx = 0;
      for (int j = 0; j < n_fft; ++j) {
        re += fr[j] * cs[idx];
        im -= fr[j] * sn[idx];
        idx += k;
        if (idx >= n_fft) idx -= n_fft;
      }
      power[f * nf + k] = re * re + im * im;
    }
  }
  free(cs);
  free(sn);
}

/* The log-mel of MelExtractor::extract (src/mel.rs:203-243) with n_fft 400,
 * hop 160: mel = filterbank . power (f64), log10(max(mel, 1e-10)), clamp at
 * (max over the clip) - 8, (x + 4) / 4.  out f32 [n_mels][frames]. */
void or_log_mel(const float* x, int64_t n, int n_mels, const float* filt, float* out) {
  const int n_fft = 400, hop = 160, nf = n_fft / 2 + 1;
  const int64_t frames = n / hop;
  double* power = (double*)malloc(sizeof(double) * (size_t)(frames * nf));
  or_stft_power(x, n, n_fft, hop, power);
  double* lm = (double*)malloc(sizeof(double) * (size_t)(frames * n_mels));
  double mx = -INFINITY;
#pragma omp parallel for schedule(static) reduction(max : mx)
  for (int64_t f = 0; f < frames; ++f)
    for (int m = 0; m < n_mels; ++m) {
      double acc = 0.0;
      for (int k = 0; k < nf; ++k) acc += (double)filt[m * nf + k] * power[f * nf + k];
      const double v = log10(acc > 1e-10 ? acc : 1e-10);
      lm[f * n_mels + m] = v;
      if (v > mx) mx = v;
    }
  for (int m = 0; m < n_mels; ++m)
    for (int64_t f = 0; f < frames; ++f) {
      const double v = lm[f * n_mels + m];
      out[m * frames + f] = (float)(((v > mx - 8.0 ? v : mx - 8.0) + 4.0) / 4.0);
    }
  free(power);
  free(lm);
}

/* The timestamp head (src/align_inference.rs:738-805): for each position p,
 * the folded final RMSNorm of h[p] in f32 (acc = sum (x w)^2 in order,
 * inv = 1 / sqrt(acc / n + eps), y = x w inv), logits = y . score^T
 * accumulated in f64 (the exact value the reference's f32 GEMM approximates),
 * class = the first index of the largest logit.  logits f64 [rows][labels]. */
void or_timestamp_head(int dtype, int64_t rows, const int32_t* pos, const uint16_t* h,
                       int64_t ldh, int64_t n, const float* w, float eps, const float* score,
                       int64_t labels, double* logits, int32_t* cls) {
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    const uint16_t* x = h + (int64_t)pos[r] * ldh;
    float acc = 0.f;
    for (int64_t j = 0; j < n; ++j) {
      const float v = or_h16_to_f32(x[j], dtype) * w[j];
      acc += v * v;
    }
    const float inv = 1.0f / sqrtf(acc / (float)n + eps);
    float* y = (float*)malloc(sizeof(float) * (size_t)n);
    for (int64_t j = 0; j < n; ++j) y[j] = or_h16_to_f32(x[j], dtype) * w[j] * inv;
    double best = -INFINITY;
    int32_t bi = 0;
    for (int64_t l = 0; l < labels; ++l) {
      double s = 0.0;
      for (int64_t j = 0; j < n; ++j) s += (double)y[j] * (double)score[l * n + j];
      logits[r * labels + l] = s;
      if (s > best) {
        best = s;
        bi = (int32_t)l;
      }
    }
    cls[r] = bi;
    free(y);
  }
}

/* ---- The CPU tower of the reference, in f32 throughout -------------------
 * CpuAudioEncoder::forward (src/audio_encoder.rs:754-832) keeps every value of
 * the tower in f32: its linears add an f32 bias to an f32 GEMM
 * (CpuAudioLinear::forward, :134-143), the residual adds and GELUs are f32
 * (:672-689, :194-202), and only the output is narrowed, once, to f16
 * (src/align_inference.rs:124-131).  The functions below restate those ops
 * on f32 buffers; tests/chains.py composes them into that forward.  (The
 * functions above take and return the GPU tower's 16-bit buffers instead.) */

/* CpuAudioLinear::forward: y = x . W^T with the f32 GEMM (or_gemm_f32, the
 * gemm crate restatement), then y[j] += b[j] in f32.  W is the f16 (or bf16)
 * checkpoint matrix [n][k] widened once, as CpuWeightF16::to_f32 does. */
void or_linear_f32(int64_t m, int64_t n, int64_t k, const float* x, int64_t ldx,
                   const uint16_t* w, int dtype, const float* bias, float* y, int64_t ldy) {
  float* wf = (float*)malloc((size_t)(n * k) * sizeof(float));
  or_h16_to_f32_n(w, wf, n * k, dtype);
  or_gemm_f32(m, n, k, x, ldx, wf, k, y, ldy, 0.0f);
  free(wf);
  if (!bias) return;
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < m; ++i)
    for (int64_t j = 0; j < n; ++j) y[i * ldy + j] += bias[j];
}

/* CpuAudioLayerNorm::forward on f32 rows (the same sums as or_layer_norm). */
void or_layer_norm_f32(int64_t rows, int64_t n, const float* x, const float* w, const float* b,
                       float eps, float* y) {
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    const float* xr = x + r * n;
    float mean = 0.f;
    for (int64_t j = 0; j < n; ++j) mean += xr[j];
    mean /= (float)n;
    float var = 0.f;
    for (int64_t j = 0; j < n; ++j) {
      const float d = xr[j] - mean;
      var += d * d;
    }
    var /= (float)n;
    const float inv_std = 1.0f / sqrtf(var + eps);
    for (int64_t j = 0; j < n; ++j) y[r * n + j] = (xr[j] - mean) * inv_std * w[j] + b[j];
  }
}

/* gelu_inplace (src/audio_encoder.rs:194-202). */
void or_gelu_f32_n(float* x, int64_t n) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n; ++i) x[i] = or_gelu(x[i]);
}

/* attention_window over every window (CpuAudioAttention::flat,
 * src/audio_encoder.rs:493-616) on f32 q, k, v rows [s][ld] (the separate
 * q_proj / k_proj / v_proj outputs; head h at columns h*hd): the arithmetic
 * of or_window_attention without the 16-bit widening and rounding.  out
 * [s][nh*hd] (the [b, s, nh*hd] flat layout). */
void or_window_attention_f32(int64_t s, int nh, int hd, int64_t wlen, const float* q,
                             const float* k, const float* v, int64_t ld, float* out) {
  const float scale = 1.0f / sqrtf((float)hd);
  const int64_t nwin = (s + wlen - 1) / wlen, dm = (int64_t)nh * hd;
#pragma omp parallel for collapse(2) schedule(dynamic)
  for (int64_t wi = 0; wi < nwin; ++wi)
    for (int h = 0; h < nh; ++h) {
      const int64_t st = wi * wlen;
      const int64_t len = (st + wlen <= s) ? wlen : s - st;
      float* sc = (float*)malloc((size_t)len * sizeof(float));
      for (int64_t qi = 0; qi < len; ++qi) {
        const float* qr = q + (st + qi) * ld + (int64_t)h * hd;
        float mx = -INFINITY;
        for (int64_t ki = 0; ki < len; ++ki) {
          const float* kr = k + (st + ki) * ld + (int64_t)h * hd;
          float dot = 0.f;
          for (int j = 0; j < hd; ++j) dot += qr[j] * kr[j];
          sc[ki] = dot * scale;
          if (sc[ki] > mx) mx = sc[ki];
        }
        float sum = 0.f;
        for (int64_t ki = 0; ki < len; ++ki) {
          sc[ki] = expf(sc[ki] - mx);
          sum += sc[ki];
        }
        const float inv = 1.0f / sum;
        float* o = out + (st + qi) * dm + (int64_t)h * hd;
        for (int j = 0; j < hd; ++j) o[j] = 0.f;
        for (int64_t ki = 0; ki < len; ++ki) {
          const float wgt = sc[ki] * inv;
          const float* vr = v + (st + ki) * ld + (int64_t)h * hd;
          for (int j = 0; j < hd; ++j) o[j] += wgt * vr[j];
        }
      }
      free(sc);
    }
}

/* CpuConvStem::conv_block on f32 (src/audio_encoder.rs:376-447): 3x3,
 * stride 2, pad 1, bias, erf GELU, no rounding.  The layouts are the GPU
 * tower's (x [batch][h][w][c_in], weight [c_out][ldw] with k = (kh*3+kw)*c_in
 * + ic, rows (b, ho, wo), or (b, wo, ho) when `tmajor`); the sum is
 * accumulated in f64 and rounded to f32 once, the value the reference's f32
 * im2col GEMM approximates in its own (unpinned) order.  x and weight are f32
 * (the weight the widened f16 checkpoint values, CpuWeightF16::to_f32). */
void or_conv3x3s2_f32(int64_t batch, int64_t h, int64_t w, int64_t c_in, int64_t c_out,
                      const float* x, const float* weight, int64_t ldw, const float* bias,
                      int gelu, int tmajor, float* y) {
  const int64_t ho = (h - 1) / 2 + 1, wo = (w - 1) / 2 + 1, plane = ho * wo;
  const int64_t M = batch * plane;
#pragma omp parallel for schedule(dynamic, 4)
  for (int64_t m = 0; m < M; ++m) {
    const int64_t b = m / plane, q = m % plane;
    const int64_t oh = tmajor ? q % ho : q / wo;
    const int64_t ow = tmajor ? q / ho : q % wo;
    for (int64_t oc = 0; oc < c_out; ++oc) {
      const float* wr = weight + oc * ldw;
      double acc = 0.0;
      for (int kh = 0; kh < 3; ++kh)
        for (int kw = 0; kw < 3; ++kw) {
          const int64_t ih = 2 * oh + kh - 1, iw = 2 * ow + kw - 1;
          if (ih < 0 || ih >= h || iw < 0 || iw >= w) continue;
          const float* xp = x + ((b * h + ih) * w + iw) * c_in;
          const float* wp = wr + (kh * 3 + kw) * c_in;
          for (int64_t ic = 0; ic < c_in; ++ic) acc += (double)xp[ic] * (double)wp[ic];
        }
      float v = (float)acc;
      if (bias) v += bias[oc];
      if (gelu) v = or_gelu(v);
      y[m * c_out + oc] = v;
    }
  }
}

/* The head's folded final norm alone (src/align_inference.rs:766-783), f32:
 * acc = sum (x w)^2 in order, inv = 1 / sqrt(acc / n + eps), y = x w inv,
 * for rows pos[r] of h.  y [rows][n]; the reference then multiplies y by the
 * score matrix with the f32 cpu_tensor::linear (:786-790). */
void or_head_fold(int dtype, int64_t rows, const int32_t* pos, const uint16_t* h, int64_t ldh,
                  int64_t n, const float* w, float eps, float* y) {
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    const uint16_t* x = h + (int64_t)pos[r] * ldh;
    float acc = 0.f;
    for (int64_t j = 0; j < n; ++j) {
      const float v = or_h16_to_f32(x[j], dtype) * w[j];
      acc += v * v;
    }
    const float inv = 1.0f / sqrtf(acc / (float)n + eps);
    for (int64_t j = 0; j < n; ++j) y[r * n + j] = or_h16_to_f32(x[j], dtype) * w[j] * inv;
  }
}
