/*
 * qa_oracle.c -- CPU restatement of the reference's linear-layer path.
 *
 * TEST INFRASTRUCTURE ONLY: see qa_oracle.h.  The product never links this.
 * Each function cites the reference file:line it follows.
 */
#include "qa_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static inline uint32_t f2u(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}
static inline float u2f(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* IEEE binary32 -> binary16, round to nearest, ties to even.  The rule
 * half 2.7.1's f16::from_f32 implements (used at src/cpu_decoder.rs:68,89 and
 * src/half16.rs:42); restated from the IEEE 754 definition. */
uint16_t or_f16_from_f32(float x) {
  const uint32_t u = f2u(x);
  const uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
  const uint32_t a = u & 0x7fffffffu;
  if (a >= 0x7f800000u) { /* inf or NaN */
    if (a == 0x7f800000u) return sign | 0x7c00u;
    return sign | 0x7e00u | (uint16_t)((a >> 13) & 0x3ffu); /* quiet NaN */
  }
  if (a >= 0x477ff000u) return sign | 0x7c00u; /* >= 65520 rounds to inf */
  const int e = (int)(a >> 23);
  if (e >= 113) { /* normal half: exponent e-127 >= -14 */
    const uint32_t mant = a & 0x7fffffu;
    uint32_t q = ((uint32_t)(e - 112) << 10) | (mant >> 13);
    const uint32_t rem = mant & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) q += 1u;
    return sign | (uint16_t)q;
  }
  /* subnormal half (or zero): value = m * 2^(e-150), unit 2^-24 */
  if (e == 0) return sign; /* f32 subnormals are far below 2^-25 */
  const uint32_t m = (a & 0x7fffffu) | 0x800000u;
  const int shift = 126 - e; /* >= 14 */
  if (shift > 25) return sign;
  uint32_t q = m >> shift;
  const uint32_t rem = m & ((1u << shift) - 1u);
  const uint32_t halfway = 1u << (shift - 1);
  if (rem > halfway || (rem == halfway && (q & 1u))) q += 1u;
  return sign | (uint16_t)q;
}

/* binary16 -> binary32 (exact). */
float or_f16_to_f32(uint16_t h) {
  const uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
  const uint32_t e = (h >> 10) & 0x1fu;
  const uint32_t m = h & 0x3ffu;
  if (e == 0x1fu) return u2f(sign | 0x7f800000u | (m << 13));
  if (e == 0) {
    if (m == 0) return u2f(sign);
    /* subnormal: m * 2^-24 is exact in f32 */
    const float v = (float)m * 5.9604644775390625e-08f;
    return sign ? -v : v;
  }
  return u2f(sign | ((e + 112u) << 23) | (m << 13));
}

/* bf16 rounding of src/shaders.rs:169-179 (rne_bf16_bits), the rule the
 * reference pins against half::bf16::from_f32 (src/shaders.rs:191-243).  For
 * NaN inputs it keeps the payload arithmetic as the reference does
 * (src/shaders.rs:247-254 states that gap). */
uint16_t or_bf16_from_f32(float x) {
  const uint32_t u = f2u(x);
  return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

float or_bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

uint16_t or_h16_from_f32(float x, int dtype) {
  return dtype == OR_BF16 ? or_bf16_from_f32(x) : or_f16_from_f32(x);
}
float or_h16_to_f32(uint16_t h, int dtype) {
  return dtype == OR_BF16 ? or_bf16_to_f32(h) : or_f16_to_f32(h);
}

void or_h16_to_f32_n(const uint16_t* src, float* dst, int64_t n, int dtype) {
#pragma omp parallel for schedule(static) if (n > (1 << 16))
  for (int64_t i = 0; i < n; ++i) dst[i] = or_h16_to_f32(src[i], dtype);
}

void or_f32_to_h16_n(const float* src, uint16_t* dst, int64_t n, int dtype) {
#pragma omp parallel for schedule(static) if (n > (1 << 16))
  for (int64_t i = 0; i < n; ++i) dst[i] = or_h16_from_f32(src[i], dtype);
}

int or_num_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

/* Thread count of later parallel regions (the CPU baseline's 1-thread figure). */
void or_set_threads(int n) {
#ifdef _OPENMP
  if (n > 0) omp_set_num_threads(n);
#else
  (void)n;
#endif
}

/* ------------------------------------------------------------------------ */
/* f32 GEMM: restates gemm_row_major (src/cpu_decoder.rs:583-610,
 * src/cpu_tensor.rs:82-108): dst = beta*dst + x.W^T, row-major x [m,k] and
 * W [n,k].  The gemm crate's microkernel order is its own; this one is a
 * blocked dot-product form (8 lane partial sums per output, k blocked by KB),
 * deterministic for any thread count. */

typedef float v8f __attribute__((vector_size(32)));

static inline v8f ld8(const float* p) {
  v8f v;
  memcpy(&v, p, sizeof v);
  return v;
}
static inline float hsum8(v8f v) {
  return ((v[0] + v[4]) + (v[1] + v[5])) + ((v[2] + v[6]) + (v[3] + v[7]));
}

enum { MB = 64, NB = 64, KB = 512 };

/* acc[i][j] (+)= dot(x_i[k0:k1], w_j[k0:k1]) for a 4x4 block. */
static void micro4x4(const float* x, int64_t ldx, const float* w, int64_t ldw,
                     int64_t k0, int64_t k1, float acc[4][4]) {
  v8f s[4][4];
  memset(s, 0, sizeof s);
  int64_t p = k0;
  for (; p + 8 <= k1; p += 8) {
    v8f xa[4], wb[4];
    for (int i = 0; i < 4; ++i) xa[i] = ld8(x + i * ldx + p);
    for (int j = 0; j < 4; ++j) wb[j] = ld8(w + j * ldw + p);
    for (int i = 0; i < 4; ++i)
      for (int j = 0; j < 4; ++j) s[i][j] += xa[i] * wb[j];
  }
  for (int i = 0; i < 4; ++i)
    for (int j = 0; j < 4; ++j) {
      float t = hsum8(s[i][j]);
      for (int64_t q = p; q < k1; ++q) t += x[i * ldx + q] * w[j * ldw + q];
      acc[i][j] += t;
    }
}

static float dot_range(const float* x, const float* w, int64_t k0, int64_t k1) {
  v8f s;
  memset(&s, 0, sizeof s);
  int64_t p = k0;
  for (; p + 8 <= k1; p += 8) s += ld8(x + p) * ld8(w + p);
  float t = hsum8(s);
  for (; p < k1; ++p) t += x[p] * w[p];
  return t;
}

void or_gemm_f32(int64_t m, int64_t n, int64_t k, const float* x, int64_t ldx,
                 const float* w, int64_t ldw, float* out, int64_t ldo, float beta) {
  const int64_t mb = (m + MB - 1) / MB, nb = (n + NB - 1) / NB;
#pragma omp parallel for collapse(2) schedule(dynamic, 1)
  for (int64_t bi = 0; bi < mb; ++bi) {
    for (int64_t bj = 0; bj < nb; ++bj) {
      const int64_t i0 = bi * MB, i1 = i0 + MB < m ? i0 + MB : m;
      const int64_t j0 = bj * NB, j1 = j0 + NB < n ? j0 + NB : n;
      float tile[MB][NB];
      memset(tile, 0, sizeof tile);
      for (int64_t k0 = 0; k0 < k; k0 += KB) {
        const int64_t k1 = k0 + KB < k ? k0 + KB : k;
        int64_t i = i0;
        for (; i + 4 <= i1; i += 4) {
          int64_t j = j0;
          for (; j + 4 <= j1; j += 4) {
            float acc[4][4] = {{0}};
            micro4x4(x + i * ldx, ldx, w + j * ldw, ldw, k0, k1, acc);
            for (int a = 0; a < 4; ++a)
              for (int b = 0; b < 4; ++b) tile[i - i0 + a][j - j0 + b] += acc[a][b];
          }
          for (; j < j1; ++j)
            for (int a = 0; a < 4; ++a)
              tile[i - i0 + a][j - j0] += dot_range(x + (i + a) * ldx, w + j * ldw, k0, k1);
        }
        for (; i < i1; ++i)
          for (int64_t j = j0; j < j1; ++j)
            tile[i - i0][j - j0] += dot_range(x + i * ldx, w + j * ldw, k0, k1);
      }
      for (int64_t i = i0; i < i1; ++i)
        for (int64_t j = j0; j < j1; ++j) {
          float* o = out + i * ldo + j;
          *o = (beta != 0.0f ? beta * *o : 0.0f) + tile[i - i0][j - j0];
        }
    }
  }
}

/* The naive side of gemm_row_major_matches_naive (src/cpu_decoder.rs:633-639):
 * one f32 accumulator, ascending k. */
void or_gemm_f32_naive(int64_t m, int64_t n, int64_t k, const float* x, int64_t ldx,
                       const float* w, int64_t ldw, float* out, int64_t ldo) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < m; ++i)
    for (int64_t j = 0; j < n; ++j) {
      float s = 0.0f;
      for (int64_t p = 0; p < k; ++p) s += x[i * ldx + p] * w[j * ldw + p];
      out[i * ldo + j] = s;
    }
}

void or_gemm_f64(int64_t m, int64_t n, int64_t k, const float* x, int64_t ldx,
                 const float* w, int64_t ldw, double* out, int64_t ldo) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < m; ++i)
    for (int64_t j = 0; j < n; ++j) {
      double s = 0.0;
      for (int64_t p = 0; p < k; ++p) s += (double)x[i * ldx + p] * (double)w[j * ldw + p];
      out[i * ldo + j] = s;
    }
}

/* src/cpu_decoder.rs:498-504: silu = g / (1 + exp(-g)); value = silu * u. */
float or_silu_mul(float g, float u) {
  const float silu = g / (1.0f + expf(-g));
  return silu * u;
}

/* src/audio_encoder.rs:196-202: gelu(x) = 0.5 x (1 + erf(x / sqrt 2)). */
float or_gelu(float x) { return 0.5f * x * (1.0f + erff(x * 0.70710678118654752f)); }

/* ------------------------------------------------------------------------ */
/* The linear op.  Semantics of the reference's prefill_gemm family
 * (src/shaders.rs:1846-2077): acc = sum_k A[m,k] W[n,k] in f32 (W read as
 * [k,n] under TRANSB, src/shaders.rs:1936-1944), then ONE rounding of
 * acc + bias[n] (+ C_old) (src/shaders.rs:2045-2073), the same rounding
 * points as batch_dot / batch_dot_acc (src/cpu_decoder.rs:59-97).
 * SILU_MUL: W = [gate | up] rows (src/decoder.rs:840-871); gate and up are
 * each rounded to 16 bits (src/cpu_decoder.rs:496-497) and the product
 * rounded once (src/cpu_decoder.rs:498-504).  GELU: bias then erf GELU then
 * one rounding (src/audio_encoder.rs:134-143,196-202 compute it in f32; the
 * 16-bit store is the GPU tower's, src/shaders.rs:2599-2652).  BIAS_ROWS indexes
 * the bias by row, the channel-major conv mode of src/shaders.rs:2636-2644. */
int or_linear(const or_linear_desc* d) {
  if (!d || !d->a || !d->w || !d->c) return -1;
  if (d->m < 0 || d->n <= 0 || d->k <= 0) return -1;
  const int dt = (int)d->dtype;
  if (dt != OR_F16 && dt != OR_BF16) return -1;
  const uint32_t fl = d->flags;
  const int silu = (fl & OR_EPI_SILU_MUL) != 0, gelu = (fl & OR_EPI_GELU) != 0;
  const int accum = (fl & OR_ACCUMULATE) != 0, transb = (fl & OR_TRANSB) != 0;
  const int bias_rows = (fl & OR_BIAS_ROWS) != 0;
  if (bias_rows && !d->bias) return -1;
  if (silu && (gelu || accum || transb || d->bias || (d->n & 1))) return -1;
  if (gelu && accum) return -1;
  const int64_t m = d->m, n = d->n, k = d->k;
  const int64_t nout = silu ? n / 2 : n;
  const int64_t batch = d->batch > 0 ? d->batch : 1;
  if (m == 0) return 0;

  float* xa = (float*)malloc(sizeof(float) * (size_t)(m * k));
  float* wf = (float*)malloc(sizeof(float) * (size_t)(n * k));
  float* acc = (float*)malloc(sizeof(float) * (size_t)(m * n));
  double* accd = (fl & OR_EXACT) ? (double*)malloc(sizeof(double) * (size_t)(m * n)) : NULL;
  if (!xa || !wf || !acc || ((fl & OR_EXACT) && !accd)) {
    free(xa); free(wf); free(acc); free(accd);
    return -1;
  }
  for (int64_t z = 0; z < batch; ++z) {
    const uint16_t* A = d->a + z * d->bsa;
    const uint16_t* W = d->w + z * d->bsb;
    uint16_t* C = d->c + z * d->bsc;
    /* widen A (src/cpu_decoder.rs:564-574) and W (:43-51) once per op */
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < m; ++i)
      for (int64_t p = 0; p < k; ++p) xa[i * k + p] = or_h16_to_f32(A[i * d->lda + p], dt);
#pragma omp parallel for schedule(static)
    for (int64_t j = 0; j < n; ++j)
      for (int64_t p = 0; p < k; ++p)
        wf[j * k + p] = or_h16_to_f32(transb ? W[p * d->ldb + j] : W[j * d->ldb + p], dt);
    if (accd) {
      or_gemm_f64(m, n, k, xa, k, wf, k, accd, n);
      for (int64_t i = 0; i < m * n; ++i) acc[i] = (float)accd[i];
    } else {
      or_gemm_f32(m, n, k, xa, k, wf, k, acc, n, 0.0f);
    }
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < m; ++i) {
      for (int64_t j = 0; j < nout; ++j) {
        uint16_t* o = C + i * d->ldc + j;
        if (silu) {
          const float g = or_h16_to_f32(or_h16_from_f32(acc[i * n + j], dt), dt);
          const float u = or_h16_to_f32(or_h16_from_f32(acc[i * n + nout + j], dt), dt);
          *o = or_h16_from_f32(or_silu_mul(g, u), dt);
          continue;
        }
        float v = acc[i * n + j];
        if (d->bias) v += or_h16_to_f32(d->bias[bias_rows ? i : j], dt);
        if (gelu) v = or_gelu(v);
        if (accum) v += or_h16_to_f32(*o, dt);
        *o = or_h16_from_f32(v, dt);
      }
    }
  }
  free(xa);
  free(wf);
  free(acc);
  free(accd);
  return 0;
}
