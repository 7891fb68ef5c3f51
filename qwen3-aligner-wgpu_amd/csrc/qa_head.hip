// qa_head.hip -- the aligner's ends around the two towers, on the GPU:
//  * the input rows: the token embedding gather with the audio tower's rows
//    scattered into the audio positions (align_raw_rows, src/align_inference.rs:
//    688-714, done on the host by the reference);
//  * the timestamp head: the final RMSNorm on the <timestamp> rows in its
//    folded form (the weight inside the variance), the f32 score head and the
//    argmax (src/align_inference.rs:738-805, host f32 in the reference).
#include "qa_internal.h"

namespace qa {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <int DT>
__device__ __forceinline__ float widen(uint16_t h) {
  if constexpr (DT == QA_F16) return (float)__builtin_bit_cast(_Float16, h);
  else return __uint_as_float((uint32_t)h << 16);
}

// out[r] = table[src[r]] for src >= 0, audio[-src[r] - 1] for src < 0; an
// index out of range gives a zero row.  One wave per row, 16-byte copies.
__global__ void __launch_bounds__(256) embed_scatter_kernel(const EmbedParams p) {
  const int lane = threadIdx.x & 63;
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= p.rows) return;
  const int s = p.src[r];
  const uint16_t* from = nullptr;
  if (s >= 0 && s < p.vocab) from = p.table + (int64_t)s * p.hidden;
  if (s < 0 && -(int64_t)s - 1 < p.n_audio) from = p.audio + (-(int64_t)s - 1) * p.hidden;
  uint16_t* to = p.out + r * p.hidden;
  for (int i = lane * 8; i < p.hidden; i += 512)
    *reinterpret_cast<u32x4*>(to + i) =
        from ? *reinterpret_cast<const u32x4*>(from + i) : u32x4{0, 0, 0, 0};
}

// normed[r][j] = x_j w_j / sqrt(sum_j (x_j w_j)^2 / n + eps) for x the row
// h[pos[r]] (src/align_inference.rs:760-775); one wave per row.
template <int DT>
__global__ void __launch_bounds__(256) head_norm_kernel(const HeadParams p) {
  const int lane = threadIdx.x & 63;
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= p.rows) return;
  const int pos = p.pos[r];
  const bool ok = pos >= 0 && pos < p.h_rows;
  const uint16_t* x = p.h + (ok ? (int64_t)pos : 0) * p.ldh;
  float s = 0.f;
  for (int j = lane; j < p.n; j += 64) {
    const float v = ok ? widen<DT>(x[j]) * p.w[j] : 0.f;
    s += v * v;
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o, 64);
  const float inv = 1.0f / sqrtf(s / (float)p.n + p.eps);
  for (int j = lane; j < p.n; j += 64)
    p.normed[r * p.n + j] = ok ? widen<DT>(x[j]) * p.w[j] * inv : 0.f;
}

// logits[r][l] = sum_j normed[r][j] score[l][j] in f32, j in order: 64 rows x
// 64 labels per block, k in slabs of 64 through LDS stored k-major, so a
// thread reads its 4 rows and its 4 labels of one k as two 16-byte loads and
// does 16 FMAs with them.  The next slab is loaded into registers while the
// current one multiplies.  VEC: rows of n floats are 16-byte aligned
// (n % 4 == 0 and an aligned score), so each thread fetches 16 consecutive k
// of one row / label as four 16-byte loads.
template <bool VEC>
__global__ void __launch_bounds__(256) head_logits_kernel(const HeadParams p) {
  typedef float f32x4 __attribute__((ext_vector_type(4)));
  constexpr int KS = 64;
  __shared__ __attribute__((aligned(16))) float as[KS][64 + 4], bs[KS][64 + 4];
  const int t = threadIdx.x;
  const int64_t r0 = (int64_t)blockIdx.y * 64, l0 = (int64_t)blockIdx.x * 64;
  const int tr = t >> 4, tl = t & 15;  // rows 4 tr .. 4 tr + 3, labels 4 tl .. 4 tl + 3
  // loader: row / label ld = t / 4, k k0 + 16 (t % 4) .. + 15
  const int ld = t >> 2, lk = (t & 3) * 16;
  const bool arow = r0 + ld < p.rows, brow = l0 + ld < p.labels;
  const float* ap = p.normed + (arow ? (r0 + ld) * p.n : 0);
  const float* bp = p.score + (brow ? (l0 + ld) * p.n : 0);
  float ra[16], rb[16];
  auto load = [&](int k0) {
    if constexpr (VEC) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int k = k0 + lk + 4 * q;
        const bool in = k < p.n;  // n % 4 == 0: a chunk is all in or all out
        const f32x4 va = (arow && in) ? *reinterpret_cast<const f32x4*>(ap + k) : f32x4{0, 0, 0, 0};
        const f32x4 vb = (brow && in) ? *reinterpret_cast<const f32x4*>(bp + k) : f32x4{0, 0, 0, 0};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          ra[4 * q + e] = va[e];
          rb[4 * q + e] = vb[e];
        }
      }
    } else {
#pragma unroll
      for (int e = 0; e < 16; ++e) {
        const int k = k0 + lk + e;
        ra[e] = (arow && k < p.n) ? ap[k] : 0.f;
        rb[e] = (brow && k < p.n) ? bp[k] : 0.f;
      }
    }
  };
  float acc[4][4];
#pragma unroll
  for (int u = 0; u < 4; ++u)
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[u][i] = 0.f;
  load(0);
  for (int k0 = 0; k0 < p.n; k0 += KS) {
#pragma unroll
    for (int e = 0; e < 16; ++e) {
      as[lk + e][ld] = ra[e];
      bs[lk + e][ld] = rb[e];
    }
    __syncthreads();
    if (k0 + KS < p.n) load(k0 + KS);
#pragma unroll 8
    for (int kk = 0; kk < KS; ++kk) {
      const f32x4 a4 = *reinterpret_cast<const f32x4*>(&as[kk][4 * tr]);
      const f32x4 b4 = *reinterpret_cast<const f32x4*>(&bs[kk][4 * tl]);
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[u][i] += a4[u] * b4[i];
    }
    __syncthreads();
  }
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const int64_t r = r0 + 4 * tr + u;
    if (r >= p.rows) continue;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t l = l0 + 4 * tl + i;
      if (l < p.labels) p.logits[r * p.labels + l] = acc[u][i];
    }
  }
}

// cls[r] = the first index of the largest logit of row r (the reference's
// `v > best_v` scan); one wave per row.
__global__ void __launch_bounds__(256) head_argmax_kernel(const HeadParams p) {
  const int lane = threadIdx.x & 63;
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= p.rows) return;
  const float* row = p.logits + r * p.labels;
  float bv = -INFINITY;
  int bi = p.labels;
  for (int l = lane; l < p.labels; l += 64)
    if (row[l] > bv) {
      bv = row[l];
      bi = l;
    }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(bv, o, 64);
    const int oi = __shfl_xor(bi, o, 64);
    if (ov > bv || (ov == bv && oi < bi)) {
      bv = ov;
      bi = oi;
    }
  }
  if (lane == 0) p.cls[r] = bi < p.labels ? bi : 0;
}

}  // namespace

hipError_t launch_embed_scatter(const EmbedParams& p, hipStream_t s) {
  hipLaunchKernelGGL(embed_scatter_kernel, dim3((unsigned)((p.rows + 3) / 4)), dim3(256), 0, s, p);
  return hipGetLastError();
}

hipError_t launch_timestamp_head(int dtype, const HeadParams& p, hipStream_t s) {
  const dim3 rows4((unsigned)((p.rows + 3) / 4));
  if (dtype == QA_BF16)
    hipLaunchKernelGGL(head_norm_kernel<QA_BF16>, rows4, dim3(256), 0, s, p);
  else
    hipLaunchKernelGGL(head_norm_kernel<QA_F16>, rows4, dim3(256), 0, s, p);
  const dim3 lg((unsigned)((p.labels + 63) / 64), (unsigned)((p.rows + 63) / 64));
  if (p.n % 4 == 0 && (reinterpret_cast<uintptr_t>(p.score) & 15) == 0 &&
      (reinterpret_cast<uintptr_t>(p.normed) & 15) == 0)
    hipLaunchKernelGGL(head_logits_kernel<true>, lg, dim3(256), 0, s, p);
  else
    hipLaunchKernelGGL(head_logits_kernel<false>, lg, dim3(256), 0, s, p);
  hipLaunchKernelGGL(head_argmax_kernel, rows4, dim3(256), 0, s, p);
  return hipGetLastError();
}

}  // namespace qa
