// qa_mel.hip -- the aligner's log-mel front end on the GPU: 16 kHz samples ->
// centered STFT (n_fft 400, hop 160, periodic Hann, reflect padding) ->
// power -> 128 slaney mel bins -> log10 clamped to max - 8 -> (x + 4) / 4,
// written as the audio tower's 16-bit mel chunks (MelExtractor::extract,
// src/mel.rs:203-243; chunking, src/audio_encoder_gpu.rs:1079-1091).  The
// reference runs this on the CPU with an f32 FFT; here a block transforms 9
// frames at once with a two-level 20 x 20 Cooley-Tukey DFT in f64 (~24k
// FMAs per frame, ~0.7 G for 300 s): an f32
// transform would lose relative accuracy on bins 6+ decades below the frame's
// peak, which the log-mel keeps (its floor is the clip max - 8), so the
// transform is made effectively exact and the mel, log and clamp run in f32
// like the reference's.
#include <algorithm>
#include <utility>

#include "qa_internal.h"

namespace qa {
namespace {

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

constexpr int NFFT = 400, HOP = 160, NBIN = NFFT / 2 + 1;
constexpr int FB = kMelFramesPerBlock;  // frames per block: 3 per wave
constexpr int MT = 192;                 // threads per block (3 waves of 3 x 20 lanes)
constexpr int ZS = 21;                  // complex slots per Z row (20 used; the pad spreads banks)
constexpr int PWS = 204;                // floats per power-spectrum row in LDS

// Reflection index without repeating the edge (src/mel.rs:27-45).
__device__ __forceinline__ int64_t reflect(int64_t i, int64_t n) {
  if (n <= 1) return 0;
  const int64_t period = 2 * (n - 1);
  int64_t x = i % period;
  if (x < 0) x += period;
  return x > n - 1 ? period - x : x;
}

// cos and sin of 2 pi j / 20 from cos 18, 36, 54 and 72 degrees ((1 + sqrt 5) / 4
// and its relatives, to the nearest double), with the quadrant symmetries
// applied exactly: the twiddles of the 20-point DFTs below, as compile-time
// constants once their loops are unrolled (the multiples of 5 fold to 0 / +-1).
__device__ constexpr double cos_q(int j) {  // cos(pi j / 10) for 0 <= j <= 5
  return j == 0 ? 1.0
       : j == 1 ? 0.9510565162951535721
       : j == 2 ? 0.8090169943749474241
       : j == 3 ? 0.5877852522924731292
       : j == 4 ? 0.3090169943749474241
       : 0.0;
}
__device__ constexpr double c20(int j) {
  j %= 20;
  if (j > 10) j = 20 - j;                       // cos is even
  return j <= 5 ? cos_q(j) : -cos_q(10 - j);    // cos(pi - a) = -cos a
}
__device__ constexpr double s20(int j) {
  j %= 20;
  if (j > 10) return -s20(20 - j);              // sin is odd
  return j <= 5 ? cos_q(5 - j) : cos_q(j - 5);  // sin a = cos(pi / 2 - a)
}

// re + i im += (a + i b)(c20(J) - i s20(J)), the products by 0 and +-1 left out
// at compile time (b = 0 for real input).
template <int J, bool REAL>
__device__ __forceinline__ void cmac(double a, double b, double& re, double& im) {
  constexpr double c = c20(J), s = s20(J);
  if constexpr (c == 1.0) {
    re += a;
    if constexpr (!REAL) im += b;
  } else if constexpr (c == -1.0) {
    re -= a;
    if constexpr (!REAL) im -= b;
  } else if constexpr (c != 0.0) {
    re = fma(a, c, re);
    if constexpr (!REAL) im = fma(b, c, im);
  }
  if constexpr (s == 1.0) {
    if constexpr (!REAL) re += b;
    im -= a;
  } else if constexpr (s == -1.0) {
    if constexpr (!REAL) re -= b;
    im += a;
  } else if constexpr (s != 0.0) {
    if constexpr (!REAL) re = fma(b, s, re);
    im = fma(a, -s, im);
  }
}

// out[K] = sum_n (a[n] + i b[n]) W20^(n K) for the K of the sequence: the
// 20-point DFT at those K, every twiddle a compile-time constant.
template <bool REAL, int K, size_t... N>
__device__ __forceinline__ void dft20_bin(const double* a, const double* b, double* ore,
                                          double* oim, std::index_sequence<N...>) {
  double re = 0.0, im = 0.0;
  (cmac<(int)(N * K) % 20, REAL>(a[N], REAL ? 0.0 : b[N], re, im), ...);
  ore[K] = re;
  oim[K] = im;
}
template <bool REAL, size_t... K>
__device__ __forceinline__ void dft20(const double* a, const double* b, double* ore, double* oim,
                                      std::index_sequence<K...>) {
  (dft20_bin<REAL, (int)K>(a, b, ore, oim, std::make_index_sequence<20>{}), ...);
}

// The twiddle table W_400^j = cos - i sin of 2 pi j / 400, and each filter's
// nonzero support [lo, hi) (bins outside it are skipped; bins inside it that
// are zero are skipped one by one, as before).  Block b's waves take filters
// 4b .. 4b + 3; block 0 also fills the table.
__global__ void __launch_bounds__(256) mel_prep_kernel(const MelParams p) {
  if (blockIdx.x == 0) {
    for (int j = threadIdx.x; j < NFFT; j += 256) {
      double s, c;
      sincospi((double)(2 * j) / (double)NFFT, &s, &c);
      p.tw[2 * j] = c;
      p.tw[2 * j + 1] = s;
    }
  }
  const int lane = threadIdx.x & 63;
  const int m = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (m >= p.n_mels) return;
  int lo = NBIN, hi = 0;
  for (int k = lane; k < NBIN; k += 64)
    if (p.filt[(int64_t)m * NBIN + k] != 0.f) {
      lo = min(lo, k);
      hi = max(hi, k + 1);
    }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    lo = min(lo, __shfl_xor(lo, o, 64));
    hi = max(hi, __shfl_xor(hi, o, 64));
  }
  if (lane == 0) {
    p.sup[2 * m] = hi > 0 ? lo : 0;
    p.sup[2 * m + 1] = hi;
  }
}

// FB frames per block: windowed samples -> 400-point DFT -> power -> mel bins
// -> log10.  The DFT is a two-level Cooley-Tukey split of 400 = 20 x 20 in
// f64 (n = 20 n1 + n2, k = k1 + 20 k2):
//   Y[n2][k1] = sum_n1 x[20 n1 + n2] W20^(n1 k1)            (real input)
//   Z[n2][k1] = Y[n2][k1] W400^(n2 k1)
//   X[k1 + 20 k2] = sum_n2 Z[n2][k1] W20^(n2 k2)
// Lane (frame f, i) of a wave computes Y[i][0..10] (Y[i][20 - k1] is its
// conjugate), writes the twiddled row Z[i][*] to LDS, and after a barrier
// reads the column Z[*][i] and forms bins i + 20 k2.  About 1200 f64 FMAs per
// lane, a third of the direct DFT's.  f64 keeps the bins far below the
// frame's peak exact to ~1e-12 relative, as the log-mel needs (its floor is
// the clip maximum - 8 decades of power); the windowing, the mel sums, the
// log and the clamp run in f32 like the reference's.
__global__ void __launch_bounds__(MT) mel_log_kernel(const MelParams p) {
  // Z of the block's frames; the samples before it and the power spectra
  // after it share the space.
  __shared__ __attribute__((aligned(16))) double zb[FB * 20 * ZS * 2];
  __shared__ double tw[2 * NFFT];
  __shared__ float red[MT / 64];
  constexpr int RAW = (FB - 1) * HOP + NFFT;  // samples the block's frames span
  static_assert(RAW * 4 <= sizeof(zb) && FB * PWS * 4 <= sizeof(zb), "aliases");
  static_assert(FB == 3 * (MT / 64), "three frames per wave");
  float* raw = reinterpret_cast<float*>(zb);
  float* pw = reinterpret_cast<float*>(zb);
  const int tid = threadIdx.x, lane = tid & 63;
  const int64_t f0 = (int64_t)blockIdx.x * FB;
  {
    constexpr int R = (2 * NFFT + MT - 1) / MT;
    double t[R];  // all loads in flight before the first store
#pragma unroll
    for (int r = 0; r < R; ++r) t[r] = p.tw[min(r * MT + tid, 2 * NFFT - 1)];
#pragma unroll
    for (int r = 0; r < R; ++r)
      if (r * MT + tid < 2 * NFFT) tw[r * MT + tid] = t[r];
  }
  {
    // the RAW consecutive samples the block's frames span, every load issued
    // before the first is used; centered frames: frame f starts at original
    // index f * hop - n_fft / 2, reflected at both ends
    const int64_t s0 = f0 * HOP - NFFT / 2;
    float v[(RAW + MT - 1) / MT];
#pragma unroll
    for (int r = 0; r < (RAW + MT - 1) / MT; ++r) {
      const int t = r * MT + tid;
      int64_t src = s0 + t;
      if (src < 0 || src >= p.n) src = reflect(src, p.n);
      v[r] = t < RAW ? p.x[src] : 0.f;
    }
#pragma unroll
    for (int r = 0; r < (RAW + MT - 1) / MT; ++r)
      if (r * MT + tid < RAW) raw[r * MT + tid] = v[r];
  }
  __syncthreads();
  // Lanes of frames past the last valid one transform reflected samples; their
  // spectra are never used.
  const bool act = lane < 60;
  const int f = (tid >> 6) * 3 + lane / 20, i = lane % 20;
  double yr[11], yi[11];
  if (act) {
    double x[20];
#pragma unroll
    for (int n1 = 0; n1 < 20; ++n1) {
      // periodic Hann 0.5 (1 - cos(2 pi j / 400)), rounded to f32, times the sample in f32
      const int j = 20 * n1 + i;
      x[n1] = (double)(raw[f * HOP + j] * (float)(0.5 * (1.0 - tw[2 * j])));
    }
    dft20<true>(x, x, yr, yi, std::make_index_sequence<11>{});
  }
  __syncthreads();  // every lane has read its samples: Z may overwrite them
  if (act) {
#pragma unroll
    for (int k1 = 0; k1 < 20; ++k1) {
      const double ar = k1 <= 10 ? yr[k1] : yr[20 - k1];
      const double ai = k1 <= 10 ? yi[k1] : -yi[20 - k1];
      const int t = i * k1;  // < 400
      const double wr = tw[2 * t], wi = -tw[2 * t + 1];
      double* z = zb + ((f * 20 + k1) * ZS + i) * 2;
      z[0] = ar * wr - ai * wi;
      z[1] = ar * wi + ai * wr;
    }
  }
  __syncthreads();
  float pk[11];
  if (act) {
    double zr[20], zi[20];
#pragma unroll
    for (int n2 = 0; n2 < 20; ++n2) {
      const double* z = zb + ((f * 20 + i) * ZS + n2) * 2;
      zr[n2] = z[0];
      zi[n2] = z[1];
    }
    double xr[11], xi[11];
    dft20<false>(zr, zi, xr, xi, std::make_index_sequence<11>{});
#pragma unroll
    for (int k2 = 0; k2 <= 10; ++k2) pk[k2] = (float)(xr[k2] * xr[k2] + xi[k2] * xi[k2]);
  }
  __syncthreads();  // every lane has read its Z column: the spectra may overwrite it
  if (act) {
#pragma unroll
    for (int k2 = 0; k2 <= 10; ++k2) {
      const int k = i + 20 * k2;
      if (k < NBIN) pw[f * PWS + k] = pk[k2];
    }
  }
  __syncthreads();
  // mel m of the block's frames: sum_k filt[m][k] pw[f][k] in k order over the
  // filter's support, skipping its zero bins (adding 0 * pw leaves the sum
  // unchanged), then log10(max(., 1e-10)).
  float mx = -INFINITY;
  for (int m = tid; m < p.n_mels; m += MT) {
    float acc[FB];
#pragma unroll
    for (int g = 0; g < FB; ++g) acc[g] = 0.f;
    const float* fr = p.filt + (int64_t)m * NBIN;
    const int lo = p.sup[2 * m], hi = p.sup[2 * m + 1];
    for (int k = lo; k < hi; k += 4) {  // four weights' loads in flight at once
      float w[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) w[u] = k + u < hi ? fr[k + u] : 0.f;
#pragma unroll
      for (int u = 0; u < 4; ++u)
        if (w[u] != 0.f) {
#pragma unroll
          for (int g = 0; g < FB; ++g) acc[g] += w[u] * pw[g * PWS + k + u];
        }
    }
#pragma unroll
    for (int g = 0; g < FB; ++g) {
      if (f0 + g >= p.frames) continue;
      const float v = logf(fmaxf(acc[g], 1e-10f)) * (1.0f / 2.302585092994046f);
      p.logmel[(int64_t)m * p.frames + f0 + g] = v;
      mx = fmaxf(mx, v);
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
  if (lane == 0) red[tid >> 6] = mx;
  __syncthreads();
  if (tid == 0) {
    float b = red[0];
#pragma unroll
    for (int w = 1; w < MT / 64; ++w) b = fmaxf(b, red[w]);
    p.bmax[blockIdx.x] = b;
  }
}

template <int DT>
__device__ __forceinline__ uint32_t pack2(float a, float b) {  // RNE
  if constexpr (DT == QA_F16)
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){a, b}, f16x2));
  else
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){a, b}, bf16x2));
}

// out[c][m][j] = r16((max(logmel[m][c cs + j], max - 8) + 4) / 4) for valid
// frames, 0 past them (the zero-padded last chunk); two frames per thread.
template <int DT>
__global__ void __launch_bounds__(256) mel_finalize_kernel(const MelParams p) {
  __shared__ float red[256];
  float mx = -INFINITY;
  for (int i = threadIdx.x; i < p.nblocks; i += 256) mx = fmaxf(mx, p.bmax[i]);
  red[threadIdx.x] = mx;
  __syncthreads();
  for (int o = 128; o > 0; o >>= 1) {
    if ((int)threadIdx.x < o) red[threadIdx.x] = fmaxf(red[threadIdx.x], red[threadIdx.x + o]);
    __syncthreads();
  }
  const float lo = red[0] - 8.0f;
  const int64_t pairs = (int64_t)p.n_chunks * p.n_mels * p.cs / 2;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < pairs;
       i += (int64_t)gridDim.x * 256) {
    const int64_t e = 2 * i;
    const int64_t c = e / ((int64_t)p.n_mels * p.cs), r = e - c * p.n_mels * p.cs;
    const int m = (int)(r / p.cs), j = (int)(r - (int64_t)m * p.cs);
    float v[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int64_t t = c * p.cs + j + u;
      v[u] = t < p.frames ? (fmaxf(p.logmel[(int64_t)m * p.frames + t], lo) + 4.0f) / 4.0f : 0.f;
    }
    *reinterpret_cast<uint32_t*>(p.out + e) = pack2<DT>(v[0], v[1]);
  }
}

}  // namespace

hipError_t launch_log_mel(int dtype, const MelParams& p, hipStream_t s) {
  hipLaunchKernelGGL(mel_prep_kernel, dim3((unsigned)((p.n_mels + 3) / 4)), dim3(256), 0, s, p);
  hipLaunchKernelGGL(mel_log_kernel, dim3((unsigned)p.nblocks), dim3(MT), 0, s, p);
  const int64_t pairs = (int64_t)p.n_chunks * p.n_mels * p.cs / 2;
  const unsigned blocks = (unsigned)std::min<int64_t>((pairs + 255) / 256, 4096);
  if (dtype == QA_BF16)
    hipLaunchKernelGGL(mel_finalize_kernel<QA_BF16>, dim3(blocks), dim3(256), 0, s, p);
  else
    hipLaunchKernelGGL(mel_finalize_kernel<QA_F16>, dim3(blocks), dim3(256), 0, s, p);
  return hipGetLastError();
}

}  // namespace qa
