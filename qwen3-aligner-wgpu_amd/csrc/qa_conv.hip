// qa_conv.hip -- the first conv level of the audio tower's stem as a direct
// convolution: 3x3, stride 2, pad 1 over a single-channel input (the mel
// chunk), bias and erf GELU, one rounding per output (CpuConvStem::conv_block,
// src/audio_encoder.rs:376-447, c_in = 1; the GPU tower's im2col + gemm_conv +
// bias_gelu, src/audio_encoder_gpu.rs:1165-1201,1714-1794).  With one input
// channel the im2col row of an output pixel is 9 scattered values, which the
// implicit GEMM's 16-byte channel chunks cannot fetch.  The 9-tap dot
// products run on the matrix cores as a K = 16 product (taps 9..15 zero): a
// wave multiplies 32 output pixels by the weights of 32 output channels per
// v_mfma_f32_32x32x16, every product of two 16-bit values exact in f32.  What
// is left on the VALU per output is the bias add, the erf GELU (a reciprocal
// and an exponential, both at a quarter of the full rate, and ~15 more
// operations) and the rounding: over the 300-chunk stem (461 M outputs) about
// 0.3 ms of the 256 CUs' VALU issue at 2.4 GHz, against ~30 slots per
// output with the taps on the VALU as well (0.43 ms measured before, 0.35
// after).
//
// A block takes 128 output pixels (32 per wave) x every output channel: the
// weights sit in LDS as 16 taps per channel (zero-padded), the bias as f32;
// each lane holds one pixel's taps as the MFMA's B fragment and, per channel
// tile, 16 of that pixel's outputs (4 runs of 4 channels), which leave as
// 8-byte stores.
#include "qa_internal.h"

namespace qa {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

template <int DT>
__device__ __forceinline__ float widen(uint16_t h) {
  if constexpr (DT == QA_F16) return (float)__builtin_bit_cast(_Float16, h);
  else return __uint_as_float((uint32_t)h << 16);
}
template <int DT>
__device__ __forceinline__ uint32_t pack2(float a, float b) {  // RNE
  if constexpr (DT == QA_F16)
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){a, b}, f16x2));
  else
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){a, b}, bf16x2));
}

constexpr int kMaxCout = 1024;
constexpr int kPix = 128;  // output pixels per block

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

template <int DT>
__device__ __forceinline__ f32x16 mfma(u32x4 a, u32x4 b) {
  if constexpr (DT == QA_F16)
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), f32x16{0}, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), f32x16{0}, 0, 0, 0);
}

// MFMA lane layout (v_mfma_f32_32x32x16, A = 32 channels x 16 taps, B = 16
// taps x 32 pixels): lane (r, h) = (lane % 32, lane / 32) supplies taps
// 8h .. 8h + 7 of channel r (A) and of pixel r (B), and receives pixel r's
// outputs for channels 8g + 4h + {0..3}, g = 0..3.
template <int DT, bool GELU>
__global__ void __launch_bounds__(256) conv1_kernel(const Conv1Params p) {
  __shared__ __attribute__((aligned(16))) uint16_t ws[kMaxCout * 16];
  __shared__ __attribute__((aligned(16))) float bs[kMaxCout];
  const int ntile = (p.c_out + 31) / 32;
  for (int i = threadIdx.x; i < ntile * 32 * 16; i += 256) {
    const int c = i >> 4, t = i & 15;
    ws[i] = c < p.c_out && t < 9 ? p.w[(int64_t)c * p.ldw + t] : (uint16_t)0;
  }
  for (int i = threadIdx.x; i < ntile * 32; i += 256)
    bs[i] = p.bias && i < p.c_out ? widen<DT>(p.bias[i]) : 0.f;
  const int lane = threadIdx.x & 63, r = lane & 31, h = lane >> 5;
  const int64_t m = (int64_t)blockIdx.x * kPix + (threadIdx.x >> 6) * 32 + r;
  // this lane's taps 8h .. 8h + 7 of pixel m (zeros past tap 8, in the
  // padding and past the last pixel)
  uint32_t tv[4] = {0, 0, 0, 0};
  if (m < p.M) {
    const int plane = p.ho * p.wo;
    const int64_t b = m / plane;
    const int q = (int)(m - b * plane);
    const int ho = p.tmajor ? q % p.ho : q / p.wo;
    const int wo = p.tmajor ? q / p.ho : q % p.wo;
    const uint16_t* x = p.x + b * p.h * p.w_in;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int t = 8 * h + e;
      if (t < 9) {
        const int kh = t / 3, kw = t % 3;
        const int ih = 2 * ho + kh - 1, iw = 2 * wo + kw - 1;
        if (ih >= 0 && ih < p.h && iw >= 0 && iw < p.w_in)
          tv[e >> 1] |= (uint32_t)x[ih * p.w_in + iw] << (16 * (e & 1));
      }
    }
  }
  const u32x4 bop = {tv[0], tv[1], tv[2], tv[3]};
  __syncthreads();
  uint16_t* y = p.y + m * p.c_out;
  // Per channel tile: bias, GELU and the rounding of the lane's 16 outputs,
  // with no branch between them so their instruction chains interleave.
  auto tile = [&](int ct, float (&v)[16]) {
    const u32x4 aop = *reinterpret_cast<const u32x4*>(ws + (ct * 32 + r) * 16 + 8 * h);
    const f32x16 acc = mfma<DT>(aop, bop);
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const f32x4 b4 = *reinterpret_cast<const f32x4*>(bs + ct * 32 + 8 * g + 4 * h);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float a = acc[4 * g + e] + b4[e];
        v[4 * g + e] = GELU ? gelu_erf(a) : a;
      }
    }
  };
  auto store = [&](int c, const float* v) {
    *reinterpret_cast<u32x2*>(y + c) = u32x2{pack2<DT>(v[0], v[1]), pack2<DT>(v[2], v[3])};
  };
  const int full = p.c_out / 32;  // tiles of 32 channels
  for (int ct = 0; ct < full; ++ct) {
    float v[16];
    tile(ct, v);
    if (m < p.M) {
#pragma unroll
      for (int g = 0; g < 4; ++g) store(ct * 32 + 8 * g + 4 * h, v + 4 * g);
    }
  }
  if (full < ntile) {  // c_out % 32 channels left: runs of 4, all in or all out
    float v[16];
    tile(full, v);
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int c = full * 32 + 8 * g + 4 * h;
      if (m < p.M && c < p.c_out) store(c, v + 4 * g);
    }
  }
}

}  // namespace

hipError_t launch_conv1(int dtype, const Conv1Params& p, hipStream_t s) {
  if (p.c_out > kMaxCout) return hipErrorInvalidValue;  // rejected by validation
  const unsigned blocks = (unsigned)((p.M + kPix - 1) / kPix);
  const dim3 g(blocks), t(256);
  if (dtype == QA_BF16) {
    if (p.gelu) hipLaunchKernelGGL((conv1_kernel<QA_BF16, true>), g, t, 0, s, p);
    else hipLaunchKernelGGL((conv1_kernel<QA_BF16, false>), g, t, 0, s, p);
  } else {
    if (p.gelu) hipLaunchKernelGGL((conv1_kernel<QA_F16, true>), g, t, 0, s, p);
    else hipLaunchKernelGGL((conv1_kernel<QA_F16, false>), g, t, 0, s, p);
  }
  return hipGetLastError();
}

}  // namespace qa
