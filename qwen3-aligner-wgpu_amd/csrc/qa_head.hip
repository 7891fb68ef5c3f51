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

// logits[r][l] = sum_j normed[r][j] score[l][j] in f32, j in order (each sum
// is one chain of FMAs, as the reference's f32 linear).  A block takes 16 PR
// rows x 64 labels, k in slabs of 64 through LDS stored k-major; a thread
// owns PR rows and 4 labels: per k, PR broadcast reads of its rows' values,
// one 16-byte read of its labels' and 4 PR FMAs.  The next slab is loaded
// into registers while the current one multiplies.  The launch picks the
// smallest PR whose grid fits one block per CU, so each SIMD runs one wave
// and the score matrix (20 MB at 5000 labels) is read by as few row blocks
// as that allows: at 240 rows x 5000 labels, PR = 5 and 3 x 79 blocks.
// VEC: rows of n floats are 16-byte aligned (n % 4 == 0 and aligned
// pointers), so the loaders fetch 16-byte chunks.
template <bool VEC, int PR>
__global__ void __launch_bounds__(256) head_logits_kernel(const HeadParams p) {
  typedef float f32x4 __attribute__((ext_vector_type(4)));
  constexpr int KS = 64, RB = 16 * PR, LB = 64;
  constexpr int AC = RB * KS / 4 / 256;  // A chunks (4 k of one row) per thread per slab
  __shared__ __attribute__((aligned(16))) float as[KS][RB];
  __shared__ __attribute__((aligned(16))) float bs[KS][LB];
  const int t = threadIdx.x;
  const int64_t r0 = (int64_t)blockIdx.y * RB, l0 = (int64_t)blockIdx.x * LB;
  const int tr = t >> 4, tl = t & 15;  // rows tr + 16 u (u < PR), labels 4 tl .. 4 tl + 3
  // loaders: A chunk c = t + 256 j: row c % RB, k 4 (c / RB) .. + 3;
  // B label t % 64, k 16 (t / 64) .. + 15
  const int bl = t & 63, bk = (t >> 6) * 16;
  const bool brow = l0 + bl < p.labels;
  const float* bp = p.score + (brow ? (l0 + bl) * p.n : 0);
  float ra[AC][4], rb[16];
  auto load = [&](int k0) {
#pragma unroll
    for (int j = 0; j < AC; ++j) {
      const int c = t + 256 * j, ar = c % RB, k = k0 + (c / RB) * 4;
      const bool arow = r0 + ar < p.rows;
      const float* ap = p.normed + (arow ? (r0 + ar) * p.n : 0);
      if constexpr (VEC) {
        const f32x4 va = (arow && k < p.n) ? *reinterpret_cast<const f32x4*>(ap + k) : f32x4{0, 0, 0, 0};
#pragma unroll
        for (int e = 0; e < 4; ++e) ra[j][e] = va[e];
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) ra[j][e] = (arow && k + e < p.n) ? ap[k + e] : 0.f;
      }
    }
    if constexpr (VEC) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int kb = k0 + bk + 4 * q;  // n % 4 == 0: a chunk is all in or all out
        const f32x4 vb = (brow && kb < p.n) ? *reinterpret_cast<const f32x4*>(bp + kb) : f32x4{0, 0, 0, 0};
#pragma unroll
        for (int e = 0; e < 4; ++e) rb[4 * q + e] = vb[e];
      }
    } else {
#pragma unroll
      for (int e = 0; e < 16; ++e) rb[e] = (brow && k0 + bk + e < p.n) ? bp[k0 + bk + e] : 0.f;
    }
  };
  float acc[PR][4];
#pragma unroll
  for (int u = 0; u < PR; ++u)
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[u][i] = 0.f;
  load(0);
  for (int k0 = 0; k0 < p.n; k0 += KS) {
#pragma unroll
    for (int j = 0; j < AC; ++j) {
      const int c = t + 256 * j;
#pragma unroll
      for (int e = 0; e < 4; ++e) as[(c / RB) * 4 + e][c % RB] = ra[j][e];
    }
#pragma unroll
    for (int e = 0; e < 16; ++e) bs[bk + e][bl] = rb[e];
    __syncthreads();
    if (k0 + KS < p.n) load(k0 + KS);
#pragma unroll 4
    for (int kk = 0; kk < KS; ++kk) {
      const f32x4 b4 = *reinterpret_cast<const f32x4*>(&bs[kk][4 * tl]);
#pragma unroll
      for (int u = 0; u < PR; ++u) {
        const float a = as[kk][tr + 16 * u];
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[u][i] += a * b4[i];
      }
    }
    __syncthreads();
  }
#pragma unroll
  for (int u = 0; u < PR; ++u) {
    const int64_t r = r0 + tr + 16 * u;
    if (r >= p.rows) continue;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t l = l0 + 4 * tl + i;
      if (l < p.labels) p.logits[r * p.labels + l] = acc[u][i];
    }
  }
}

template <bool VEC>
void launch_logits(const HeadParams& p, hipStream_t s) {
  constexpr int kCUs = 256;
  const int64_t lb = (p.labels + 63) / 64;
  int pr = 1;
  while (pr < 8 && lb * ((p.rows + 16 * pr - 1) / (16 * pr)) > kCUs) ++pr;
  const dim3 g((unsigned)lb, (unsigned)((p.rows + 16 * pr - 1) / (16 * pr))), t(256);
  switch (pr) {
    case 1: hipLaunchKernelGGL((head_logits_kernel<VEC, 1>), g, t, 0, s, p); break;
    case 2: hipLaunchKernelGGL((head_logits_kernel<VEC, 2>), g, t, 0, s, p); break;
    case 3: hipLaunchKernelGGL((head_logits_kernel<VEC, 3>), g, t, 0, s, p); break;
    case 4: hipLaunchKernelGGL((head_logits_kernel<VEC, 4>), g, t, 0, s, p); break;
    case 5: hipLaunchKernelGGL((head_logits_kernel<VEC, 5>), g, t, 0, s, p); break;
    case 6: hipLaunchKernelGGL((head_logits_kernel<VEC, 6>), g, t, 0, s, p); break;
    case 7: hipLaunchKernelGGL((head_logits_kernel<VEC, 7>), g, t, 0, s, p); break;
    default: hipLaunchKernelGGL((head_logits_kernel<VEC, 8>), g, t, 0, s, p); break;
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
  // 8 loads in flight per lane, then its labels in increasing order
  for (int64_t l0 = lane; l0 < p.labels; l0 += 512) {
    float v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = l0 + 64 * u < p.labels ? row[l0 + 64 * u] : -INFINITY;
#pragma unroll
    for (int u = 0; u < 8; ++u)
      if (v[u] > bv) {
        bv = v[u];
        bi = (int)(l0 + 64 * u);
      }
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
  if (p.n % 4 == 0 && (reinterpret_cast<uintptr_t>(p.score) & 15) == 0 &&
      (reinterpret_cast<uintptr_t>(p.normed) & 15) == 0)
    launch_logits<true>(p, s);
  else
    launch_logits<false>(p, s);
  hipLaunchKernelGGL(head_argmax_kernel, rows4, dim3(256), 0, s, p);
  return hipGetLastError();
}

}  // namespace qa
