// qa_audio_ops.hip -- the audio tower's ops around the projections that are
// not GEMMs: LayerNorm, the per-window self-attention and the sinusoidal
// position add (the reference's `layernorm`, extract / win_pack / scores /
// softmax / av / attn_flat and `add_pe` pipelines, src/audio_encoder_gpu.rs:
// 1405-1590, 1838-1866, 1996-2030; WGSL src/shaders.rs:2680-3086; CPU twin
// src/audio_encoder.rs:147-171, 331-343, 517-616).
#include "qa_internal.h"

namespace qa {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

constexpr float kLog2e = 1.44269504088896341f;

template <int DT>
struct H;
template <>
struct H<QA_F16> {
  __device__ static __forceinline__ float widen(uint32_t h) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
  }
  __device__ static __forceinline__ uint32_t pack2(float a, float b) {  // RNE
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){a, b}, f16x2));
  }
  __device__ static __forceinline__ f32x2 unpack2(uint32_t h) {
    return __builtin_convertvector(__builtin_bit_cast(f16x2, h), f32x2);
  }
  __device__ static __forceinline__ f32x16 mfma(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
  // probabilities (<= 1) are formed scaled by 2^15: normal down to p = 2^-29
  static constexpr float kPBias = 15.f;
};
template <>
struct H<QA_BF16> {
  __device__ static __forceinline__ float widen(uint32_t h) { return __uint_as_float(h << 16); }
  // RNE (v_cvt_pk_bf16_f32): for finite values the reference's
  // (u + 0x7fff + ((u >> 16) & 1)) >> 16, src/shaders.rs:169-179
  __device__ static __forceinline__ uint32_t pack2(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){a, b}, bf16x2));
  }
  __device__ static __forceinline__ f32x2 unpack2(uint32_t h) {
    return (f32x2){__uint_as_float(h << 16), __uint_as_float(h & 0xffff0000u)};
  }
  __device__ static __forceinline__ f32x16 mfma(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
  static constexpr float kPBias = 0.f;
};

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// y[r] = r16((x - mean) * inv_std * w + b), one wave per row, 16-byte chunks;
// mean, then the variance of (x - mean), in f32 (src/audio_encoder.rs:147-171).
// NC > 0: rows of at most NC * 512 elements stay in registers (lane l holds
// chunks l and l + 64, ...) and w / b come as 16-byte loads (16-byte aligned);
// NC = 0: any width, re-reading the row.  Both sum in the same lane order.
template <int DT, int NC>
__global__ void __launch_bounds__(256) layer_norm_kernel(const LnParams p) {
  typedef float f32x4 __attribute__((ext_vector_type(4)));
  const int lane = threadIdx.x & 63;
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= p.rows) return;
  const uint16_t* x = p.x + r * p.ldx;
  uint16_t* y = p.y + r * p.ldy;
  if constexpr (NC > 0) {
    u32x4 v[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int i = lane * 8 + c * 512;
      v[c] = i < p.n ? *reinterpret_cast<const u32x4*>(x + i) : u32x4{0, 0, 0, 0};
    }
    float s = 0.f;
#pragma unroll
    for (int c = 0; c < NC; ++c)
      if (lane * 8 + c * 512 < p.n) {
#pragma unroll
        for (int e = 0; e < 4; ++e) s += H<DT>::widen(v[c][e] & 0xffffu) + H<DT>::widen(v[c][e] >> 16);
      }
    const float mean = wave_sum(s) / (float)p.n;
    float q = 0.f;
#pragma unroll
    for (int c = 0; c < NC; ++c)
      if (lane * 8 + c * 512 < p.n) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float a = H<DT>::widen(v[c][e] & 0xffffu) - mean, b = H<DT>::widen(v[c][e] >> 16) - mean;
          q += a * a;
          q += b * b;
        }
      }
    const float inv = 1.0f / sqrtf(wave_sum(q) / (float)p.n + p.eps);
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int i = lane * 8 + c * 512;
      if (i >= p.n) continue;
      const f32x4 w0 = *reinterpret_cast<const f32x4*>(p.w + i), w1 = *reinterpret_cast<const f32x4*>(p.w + i + 4);
      const f32x4 b0 = *reinterpret_cast<const f32x4*>(p.b + i), b1 = *reinterpret_cast<const f32x4*>(p.b + i + 4);
      const float wv[8] = {w0[0], w0[1], w0[2], w0[3], w1[0], w1[1], w1[2], w1[3]};
      const float bv[8] = {b0[0], b0[1], b0[2], b0[3], b1[0], b1[1], b1[2], b1[3]};
      u32x4 o;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float a = (H<DT>::widen(v[c][e] & 0xffffu) - mean) * inv * wv[2 * e] + bv[2 * e];
        const float b = (H<DT>::widen(v[c][e] >> 16) - mean) * inv * wv[2 * e + 1] + bv[2 * e + 1];
        o[e] = H<DT>::pack2(a, b);
      }
      *reinterpret_cast<u32x4*>(y + i) = o;
    }
    return;
  }
  float s = 0.f;
  for (int i = lane * 8; i < p.n; i += 512) {
    const u32x4 v = *reinterpret_cast<const u32x4*>(x + i);
#pragma unroll
    for (int e = 0; e < 4; ++e) s += H<DT>::widen(v[e] & 0xffffu) + H<DT>::widen(v[e] >> 16);
  }
  const float mean = wave_sum(s) / (float)p.n;
  float q = 0.f;
  for (int i = lane * 8; i < p.n; i += 512) {
    const u32x4 v = *reinterpret_cast<const u32x4*>(x + i);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float a = H<DT>::widen(v[e] & 0xffffu) - mean, b = H<DT>::widen(v[e] >> 16) - mean;
      q += a * a;
      q += b * b;
    }
  }
  const float inv = 1.0f / sqrtf(wave_sum(q) / (float)p.n + p.eps);
  for (int i = lane * 8; i < p.n; i += 512) {
    const u32x4 v = *reinterpret_cast<const u32x4*>(x + i);
    u32x4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int j = i + 2 * e;
      const float a = (H<DT>::widen(v[e] & 0xffffu) - mean) * inv * p.w[j] + p.b[j];
      const float b = (H<DT>::widen(v[e] >> 16) - mean) * inv * p.w[j + 1] + p.b[j + 1];
      o[e] = H<DT>::pack2(a, b);
    }
    *reinterpret_cast<u32x4*>(y + i) = o;
  }
}

// y[r][j] = r16(y[r][j] + table[r % period][j]), 8 elements per thread.
template <int DT>
__global__ void __launch_bounds__(256) add_table_kernel(const TableAddParams p) {
  const int64_t chunks = p.n / 8;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= p.rows * chunks) return;
  const int64_t r = i / chunks, c = (i - r * chunks) * 8;
  uint16_t* y = p.y + r * p.ldy + c;
  const float* t = p.table + (r % p.period) * p.n + c;
  const u32x4 v = *reinterpret_cast<const u32x4*>(y);
  u32x4 o;
#pragma unroll
  for (int e = 0; e < 4; ++e)
    o[e] = H<DT>::pack2(H<DT>::widen(v[e] & 0xffffu) + t[2 * e],
                        H<DT>::widen(v[e] >> 16) + t[2 * e + 1]);
  *reinterpret_cast<u32x4*>(y) = o;
}

// ---------------------------------------------------------------------------
// Windowed self-attention, hd = 64, windows of up to 128 tokens.
//
// One block (4 waves) per (head, window); wave w takes query rows 32w..32w+31
// of the window.  K [128 keys][64 d] and V^T [64 d][128 stored keys] of the
// window sit in LDS (32 KB).  S = K.Q^T on v_mfma_f32_32x32x16 (A = 32 keys
// x 16 d from LDS, B = the wave's Q rows from global), so a lane holds one
// query row and 16 of each 32-key tile's scores, 64 in all; the partner lane
// (lane ^ 32) holds the rest of the row.  Keys past the window's length are
// masked.  The row max is exact (every score is in registers), so
// probabilities are <= 1; they enter O^T = V^T.P^T straight from the score
// registers as two 16-bit terms (value and rounding residue), the V^T columns
// stored in the order the score layout holds the keys: within each aligned
// group of 16 keys, 0-3, 8-11, 4-7, 12-15 (bits 2 and 3 swapped).
constexpr int WA_HD = 64, WA_MAXW = 128;


template <int DT>
__global__ void __launch_bounds__(256) window_attention_kernel(const WinAttnParams p) {
  __shared__ __attribute__((aligned(16))) uint16_t ks[WA_MAXW * WA_HD];   // [key][d], 8 chunks/row
  __shared__ __attribute__((aligned(16))) uint16_t vts[WA_HD * WA_MAXW];  // [d][stored key]
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int fr = lane & 31, fh = lane >> 5;
  const int h = (int)(blockIdx.x % p.nh);
  const int64_t win = blockIdx.x / p.nh;
  const int64_t st = win * p.wlen;
  const int len = (int)min((int64_t)p.wlen, p.s - st);
  const int64_t dm = (int64_t)p.nh * WA_HD;
  const uint16_t* qkv = p.qkv + st * p.ldqkv + (int64_t)h * WA_HD;

  // ---- K rows (chunk c of row r at c ^ ((r >> 1) & 7)) into LDS ----
  for (int i = tid; i < WA_MAXW * 8; i += 256) {
    const int r = i >> 3, c = i & 7;
    u32x4 kv = {0, 0, 0, 0};
    if (r < len) kv = *reinterpret_cast<const u32x4*>(qkv + (int64_t)r * p.ldqkv + dm + c * 8);
    *reinterpret_cast<u32x4*>(ks + r * WA_HD + ((c ^ ((r >> 1) & 7)) << 3)) = kv;
  }
  // ---- V^T into LDS, 8 x 8 blocks transposed in registers ----
  // Thread t < 128 takes stored-key chunk sc = t / 8 (8 stored columns) and
  // d chunk c = t % 8: stored columns 16 g + 8 h + 0..7 hold keys
  // 16 g + 4 h + 0..3 and 16 g + 8 + 4 h + 0..3 (bits 2 and 3 of the key
  // swapped), so it loads those
  // 8 key rows of V (16 bytes each) and writes 8 V^T rows d = 8 c .. 8 c + 7,
  // 16 bytes each, at chunk sc ^ (d & 15) (row d: 16 chunks of 8 stored keys).
  if (tid < 128) {
    const int sc = tid >> 3, c = tid & 7;
    const int g = sc >> 1, hh = sc & 1;
    u32x4 vr[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int key = 16 * g + 8 * (j >> 2) + 4 * hh + (j & 3);  // stored column 8 sc + j
      vr[j] = key < len ? *reinterpret_cast<const u32x4*>(qkv + (int64_t)key * p.ldqkv + 2 * dm + c * 8)
                        : u32x4{0, 0, 0, 0};
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int d = c * 8 + e;
      u32x4 o;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint32_t a = vr[2 * q][e >> 1], b = vr[2 * q + 1][e >> 1];
        o[q] = (e & 1) ? ((a >> 16) | (b & 0xffff0000u)) : ((a & 0xffffu) | (b << 16));
      }
      *reinterpret_cast<u32x4*>(vts + d * WA_MAXW + ((sc ^ (d & 15)) << 3)) = o;
    }
  }
  // ---- this wave's query rows as B fragments (4 slices of 16 d) ----
  const int qr = wave * 32 + fr;
  u32x4 qf[4];
#pragma unroll
  for (int sl = 0; sl < 4; ++sl)
    qf[sl] = qr < len ? *reinterpret_cast<const u32x4*>(qkv + (int64_t)qr * p.ldqkv + sl * 16 +
                                                        fh * 8)
                      : u32x4{0, 0, 0, 0};
  __syncthreads();
  if (wave * 32 >= len) return;  // no query rows for this wave (after the barrier)

  // ---- S^T = K.Q^T over the 4 key tiles ----
  f32x16 s[4];
#pragma unroll
  for (int kt = 0; kt < 4; ++kt) {
    s[kt] = f32x16{0};
    const int r = kt * 32 + fr;
#pragma unroll
    for (int sl = 0; sl < 4; ++sl) {
      const int c = 2 * sl + fh;
      const u32x4 kf =
          *reinterpret_cast<const u32x4*>(ks + r * WA_HD + ((c ^ ((r >> 1) & 7)) << 3));
      s[kt] = H<DT>::mfma(kf, qf[sl], s[kt]);
    }
  }
  // ---- softmax over the row (keys >= len masked) ----
  float mx[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
#pragma unroll
  for (int kt = 0; kt < 4; ++kt)
#pragma unroll
    for (int g = 0; g < 4; ++g)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int key = kt * 32 + 8 * g + 4 * fh + e;
        if (key >= len) s[kt][4 * g + e] = -INFINITY;
        mx[e] = fmaxf(mx[e], s[kt][4 * g + e]);
      }
  float m = fmaxf(fmaxf(mx[0], mx[1]), fmaxf(mx[2], mx[3]));
  m = fmaxf(m, __shfl_xor(m, 32, 64));
  const float sc = p.scale * kLog2e;
  const float mb = m * sc - H<DT>::kPBias;
  float rs[4] = {0.f, 0.f, 0.f, 0.f};
  u32x4 pf[8], pl[8];  // slice j = 16 keys: 2 kt + g / 2 of tile kt = j / 2
#pragma unroll
  for (int kt = 0; kt < 4; ++kt)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      float pv[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        pv[e] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[kt][4 * g + e], sc, -mb));
        rs[e] += pv[e];
      }
      const int j = 2 * kt + (g >> 1), half = g & 1;
      pf[j][2 * half] = H<DT>::pack2(pv[0], pv[1]);
      pf[j][2 * half + 1] = H<DT>::pack2(pv[2], pv[3]);
      const f32x2 h01 = H<DT>::unpack2(pf[j][2 * half]), h23 = H<DT>::unpack2(pf[j][2 * half + 1]);
      pl[j][2 * half] = H<DT>::pack2(pv[0] - h01[0], pv[1] - h01[1]);
      pl[j][2 * half + 1] = H<DT>::pack2(pv[2] - h23[0], pv[3] - h23[1]);
    }
  float l = (rs[0] + rs[1]) + (rs[2] + rs[3]);
  l += __shfl_xor(l, 32, 64);
  // ---- O^T = V^T.P^T: 2 d tiles x 8 key slices x 2 terms ----
  f32x16 o[2] = {f32x16{0}, f32x16{0}};
#pragma unroll
  for (int j = 0; j < 8; ++j)
#pragma unroll
    for (int dt = 0; dt < 2; ++dt) {
      const int d = dt * 32 + fr;
      const int c = 2 * j + fh;  // 16 chunks of 8 stored keys per V^T row
      const u32x4 vf = *reinterpret_cast<const u32x4*>(vts + d * WA_MAXW + ((c ^ (d & 15)) << 3));
      o[dt] = H<DT>::mfma(vf, pf[j], o[dt]);
      o[dt] = H<DT>::mfma(vf, pl[j], o[dt]);
    }
  if (qr >= len) return;
  const float inv = 1.0f / l;
  uint16_t* out = p.out + (st + qr) * p.ldo + (int64_t)h * WA_HD;
#pragma unroll
  for (int dt = 0; dt < 2; ++dt)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const u32x2 pk = {H<DT>::pack2(o[dt][4 * g] * inv, o[dt][4 * g + 1] * inv),
                        H<DT>::pack2(o[dt][4 * g + 2] * inv, o[dt][4 * g + 3] * inv)};
      *reinterpret_cast<u32x2*>(out + dt * 32 + 8 * g + 4 * fh) = pk;
    }
}

}  // namespace

hipError_t launch_layer_norm(int dtype, const LnParams& p, hipStream_t s) {
  const unsigned blocks = (unsigned)((p.rows + 3) / 4);
  const bool reg = p.n <= 1024 && (reinterpret_cast<uintptr_t>(p.w) & 15) == 0 &&
                   (reinterpret_cast<uintptr_t>(p.b) & 15) == 0;
  if (dtype == QA_BF16) {
    if (reg) hipLaunchKernelGGL((layer_norm_kernel<QA_BF16, 2>), dim3(blocks), dim3(256), 0, s, p);
    else hipLaunchKernelGGL((layer_norm_kernel<QA_BF16, 0>), dim3(blocks), dim3(256), 0, s, p);
  } else {
    if (reg) hipLaunchKernelGGL((layer_norm_kernel<QA_F16, 2>), dim3(blocks), dim3(256), 0, s, p);
    else hipLaunchKernelGGL((layer_norm_kernel<QA_F16, 0>), dim3(blocks), dim3(256), 0, s, p);
  }
  return hipGetLastError();
}

hipError_t launch_add_table(int dtype, const TableAddParams& p, hipStream_t s) {
  const unsigned blocks = (unsigned)((p.rows * (p.n / 8) + 255) / 256);
  if (dtype == QA_BF16)
    hipLaunchKernelGGL(add_table_kernel<QA_BF16>, dim3(blocks), dim3(256), 0, s, p);
  else
    hipLaunchKernelGGL(add_table_kernel<QA_F16>, dim3(blocks), dim3(256), 0, s, p);
  return hipGetLastError();
}

hipError_t launch_window_attention(int dtype, const WinAttnParams& p, hipStream_t s) {
  const unsigned blocks = (unsigned)(((p.s + p.wlen - 1) / p.wlen) * p.nh);
  if (dtype == QA_BF16)
    hipLaunchKernelGGL(window_attention_kernel<QA_BF16>, dim3(blocks), dim3(256), 0, s, p);
  else
    hipLaunchKernelGGL(window_attention_kernel<QA_F16>, dim3(blocks), dim3(256), 0, s, p);
  return hipGetLastError();
}

}  // namespace qa
