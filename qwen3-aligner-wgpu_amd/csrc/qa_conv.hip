// qa_conv.hip -- the first conv level of the audio tower's stem as a direct
// convolution: 3x3, stride 2, pad 1 over a single-channel input (the mel
// chunk), bias and erf GELU, one rounding per output (CpuConvStem::conv_block,
// src/audio_encoder.rs:376-447, c_in = 1; the GPU tower's im2col + gemm_conv +
// bias_gelu, src/audio_encoder_gpu.rs:1165-1201,1714-1794).  With one input
// channel the im2col row of an output pixel is 9 scattered values, which the
// implicit GEMM's 16-byte channel chunks cannot fetch.  Per output it costs 9
// multiply-adds and the erf GELU (a reciprocal, an exponential and ~15 more
// VALU operations), ~30 VALU slots in all: over the 300-chunk stem (461 M
// outputs) that is ~0.35 ms of the 256 CUs' VALU issue, which is what the
// measured ~0.43 ms follows (2.1 TB/s of output writes, well under HBM's
// rate; a variant with fully contiguous stores measured the same).
//
// A block takes 64 output pixels x every output channel: the 9 taps of its
// thread's pixel stay in registers, the weights and bias sit in LDS as f32,
// and each output channel group of 8 leaves as one 16-byte store.
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

template <int DT>
__global__ void __launch_bounds__(256) conv1_kernel(const Conv1Params p) {
  __shared__ float ws[kMaxCout * 9];
  __shared__ float bs[kMaxCout];
  for (int i = threadIdx.x; i < p.c_out * 9; i += 256)
    ws[i] = widen<DT>(p.w[(i / 9) * p.ldw + i % 9]);
  for (int i = threadIdx.x; i < p.c_out; i += 256) bs[i] = p.bias ? widen<DT>(p.bias[i]) : 0.f;
  __syncthreads();
  const int64_t m = (int64_t)blockIdx.x * 64 + (threadIdx.x & 63);
  if (m >= p.M) return;
  const int plane = p.ho * p.wo;
  const int64_t b = m / plane;
  const int q = (int)(m - b * plane);
  const int ho = p.tmajor ? q % p.ho : q / p.wo;
  const int wo = p.tmajor ? q / p.ho : q % p.wo;
  const uint16_t* x = p.x + b * p.h * p.w_in;
  float t[9];
#pragma unroll
  for (int kh = 0; kh < 3; ++kh)
#pragma unroll
    for (int kw = 0; kw < 3; ++kw) {
      const int ih = 2 * ho + kh - 1, iw = 2 * wo + kw - 1;
      t[kh * 3 + kw] =
          (ih >= 0 && ih < p.h && iw >= 0 && iw < p.w_in) ? widen<DT>(x[ih * p.w_in + iw]) : 0.f;
    }
  uint16_t* y = p.y + m * p.c_out;
  for (int g = threadIdx.x >> 6; g < p.c_out / 8; g += 4) {
    float v[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const float* wr = ws + (g * 8 + c) * 9;
      float acc = 0.f;
#pragma unroll
      for (int i = 0; i < 9; ++i) acc += wr[i] * t[i];
      acc += bs[g * 8 + c];
      v[c] = p.gelu ? gelu_erf(acc) : acc;
    }
    *reinterpret_cast<u32x4*>(y + g * 8) =
        u32x4{pack2<DT>(v[0], v[1]), pack2<DT>(v[2], v[3]), pack2<DT>(v[4], v[5]),
              pack2<DT>(v[6], v[7])};
  }
}

}  // namespace

hipError_t launch_conv1(int dtype, const Conv1Params& p, hipStream_t s) {
  if (p.c_out > kMaxCout) return hipErrorInvalidValue;  // rejected by validation
  const unsigned blocks = (unsigned)((p.M + 63) / 64);
  if (dtype == QA_BF16)
    hipLaunchKernelGGL(conv1_kernel<QA_BF16>, dim3(blocks), dim3(256), 0, s, p);
  else
    hipLaunchKernelGGL(conv1_kernel<QA_F16>, dim3(blocks), dim3(256), 0, s, p);
  return hipGetLastError();
}

}  // namespace qa
