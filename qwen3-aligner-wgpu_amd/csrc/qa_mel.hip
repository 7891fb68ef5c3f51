// qa_mel.hip -- the aligner's log-mel front end on the GPU: 16 kHz samples ->
// centered STFT (n_fft 400, hop 160, periodic Hann, reflect padding) ->
// power -> 128 slaney mel bins -> log10 clamped to max - 8 -> (x + 4) / 4,
// written as the audio tower's 16-bit mel chunks (MelExtractor::extract,
// src/mel.rs:203-243; chunking, src/audio_encoder_gpu.rs:1079-1091).  The
// reference runs this on the CPU with an f32 FFT; here a block transforms 16
// frames at once as a direct DFT from LDS (400 x 201 multiply-adds per
// frame, ~10 GFLOP of f64 for 300 s), accumulated in f64:
// an f32 direct DFT would lose relative accuracy on bins 6+ decades below the
// frame's peak, which the log-mel keeps (its floor is the clip max - 8), so
// the transform is made effectively exact and the mel, log and clamp run in
// f32 like the reference's.
#include <algorithm>

#include "qa_internal.h"

namespace qa {
namespace {

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

constexpr int NFFT = 400, HOP = 160, NBIN = NFFT / 2 + 1, FB = 16;

// Reflection index without repeating the edge (src/mel.rs:27-45).
__device__ __forceinline__ int64_t reflect(int64_t i, int64_t n) {
  if (n <= 1) return 0;
  const int64_t period = 2 * (n - 1);
  int64_t x = i % period;
  if (x < 0) x += period;
  return x > n - 1 ? period - x : x;
}

// Frames f0..f0+15: windowed samples in LDS, power spectra, mel bins, log10.
// The windowed samples sit transposed, xw[j][f], so the DFT loop reads the 16
// frames' sample j as four 16-byte broadcasts.  Each bin's twiddle advances by
// a complex multiply per step (f64) and is re-anchored to the exact table
// value every kAnchor steps, so its drift stays at a few f64 ulps.
constexpr int kAnchor = 50;
__global__ void __launch_bounds__(256) mel_log_kernel(const MelParams p) {
  __shared__ __attribute__((aligned(16))) float xw[NFFT][FB];
  __shared__ float pw[FB][NBIN + 3];
  __shared__ double tc[NFFT], ts[NFFT];
  __shared__ float red[256];
  const int tid = threadIdx.x;
  const int64_t f0 = (int64_t)blockIdx.x * FB;
  for (int j = tid; j < NFFT; j += 256) {
    // twiddles e^{-2 pi i j / 400} and the periodic Hann window 0.5 (1 - cos(2 pi j / 400))
    double s, c;
    sincospi((double)(2 * j) / (double)NFFT, &s, &c);
    tc[j] = c;
    ts[j] = s;
  }
  __syncthreads();
  for (int i = tid; i < FB * NFFT; i += 256) {
    const int f = i / NFFT, j = i - f * NFFT;
    float v = 0.f;
    if (f0 + f < p.frames) {
      // centered frame: padded sample (f0 + f) * hop + j = original index - n_fft / 2
      const int64_t src = reflect((f0 + f) * HOP + j - NFFT / 2, p.n);
      v = p.x[src] * (float)(0.5 * (1.0 - tc[j]));
    }
    xw[j][f] = v;
  }
  __syncthreads();
  // One radix-2 split of the real 400-point DFT.  For bin k = 0..100, lanes
  // 0-31 of a wave sum the even samples (E[k], a 200-point DFT) and lanes
  // 32-63 the odd ones (O[k]) of the same 32 bins; then X[k] = E + w^k O and,
  // since E and O of real input satisfy E[200 - k] = conj(E[k]) (same for O)
  // and w^(200 - k) = -conj(w^k), |X[200 - k]| = |E[k] - w^k O[k]|.
  {
    const int lane = tid & 63, half = lane >> 5;
    const int k = (tid >> 6) * 32 + (lane & 31);
    const bool act = k <= NFFT / 4;
    double re[FB], im[FB];
#pragma unroll
    for (int f = 0; f < FB; ++f) re[f] = im[f] = 0.0;
    if (act) {
      const int step = (2 * k) % NFFT;
      const double rr = tc[step], ri = -ts[step];  // e^{-2 pi i 2k / 400}
      for (int n0 = 0; n0 < NFFT / 2; n0 += kAnchor) {
        const int idx = (2 * n0 * k) % NFFT;
        double wr = tc[idx], wi = -ts[idx];
        for (int n = n0; n < n0 + kAnchor; ++n) {
          typedef float f32x4 __attribute__((ext_vector_type(4)));
          const f32x4* row = reinterpret_cast<const f32x4*>(&xw[2 * n + half][0]);
#pragma unroll
          for (int q = 0; q < FB / 4; ++q) {
            const f32x4 x4 = row[q];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              re[4 * q + e] += (double)x4[e] * wr;
              im[4 * q + e] += (double)x4[e] * wi;
            }
          }
          const double nr = wr * rr - wi * ri;
          wi = wr * ri + wi * rr;
          wr = nr;
        }
      }
    }
    double ore[FB], oim[FB];  // the odd half's sums, in the even lanes
#pragma unroll
    for (int f = 0; f < FB; ++f) {
      ore[f] = __shfl_xor(re[f], 32, 64);
      oim[f] = __shfl_xor(im[f], 32, 64);
    }
    if (act && half == 0) {
      const double cr = tc[k], ci = -ts[k];  // w^k = e^{-2 pi i k / 400}
#pragma unroll
      for (int f = 0; f < FB; ++f) {
        const double tr = cr * ore[f] - ci * oim[f], ti = cr * oim[f] + ci * ore[f];
        const double ar = re[f] + tr, ai = im[f] + ti;
        const double br = re[f] - tr, bi = im[f] - ti;
        pw[f][k] = (float)(ar * ar + ai * ai);
        if (k != NFFT / 4) pw[f][NFFT / 2 - k] = (float)(br * br + bi * bi);
      }
    }
  }
  __syncthreads();
  // mel m of the 16 frames: sum_k filt[m][k] pw[f][k] in k order, skipping the
  // filter's zero bins (adding 0 * pw leaves the sum unchanged), then
  // log10(max(., 1e-10)).
  float mx = -INFINITY;
  for (int m = tid; m < p.n_mels; m += 256) {
    float acc[FB];
#pragma unroll
    for (int f = 0; f < FB; ++f) acc[f] = 0.f;
    const float* fr = p.filt + (int64_t)m * NBIN;
    for (int k = 0; k < NBIN; ++k) {
      const float w = fr[k];
      if (w != 0.f) {
#pragma unroll
        for (int f = 0; f < FB; ++f) acc[f] += w * pw[f][k];
      }
    }
#pragma unroll
    for (int f = 0; f < FB; ++f) {
      if (f0 + f >= p.frames) continue;
      const float v = logf(fmaxf(acc[f], 1e-10f)) * (1.0f / 2.302585092994046f);
      p.logmel[(int64_t)m * p.frames + f0 + f] = v;
      mx = fmaxf(mx, v);
    }
  }
  red[tid] = mx;
  __syncthreads();
  for (int o = 128; o > 0; o >>= 1) {
    if (tid < o) red[tid] = fmaxf(red[tid], red[tid + o]);
    __syncthreads();
  }
  if (tid == 0) p.bmax[blockIdx.x] = red[0];
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
  hipLaunchKernelGGL(mel_log_kernel, dim3((unsigned)p.nblocks), dim3(256), 0, s, p);
  const int64_t pairs = (int64_t)p.n_chunks * p.n_mels * p.cs / 2;
  const unsigned blocks = (unsigned)std::min<int64_t>((pairs + 255) / 256, 4096);
  if (dtype == QA_BF16)
    hipLaunchKernelGGL(mel_finalize_kernel<QA_BF16>, dim3(blocks), dim3(256), 0, s, p);
  else
    hipLaunchKernelGGL(mel_finalize_kernel<QA_F16>, dim3(blocks), dim3(256), 0, s, p);
  return hipGetLastError();
}

}  // namespace qa
