// qa_decoder_ops.hip -- the decoder's prefill ops around the projections
// that are not GEMMs: RMSNorm, and the per-head q/k RMSNorm + rotate-half
// RoPE that writes the KV cache (the reference's `rms_norm` and
// `qkv_extract` pipelines, src/decoder.rs:1305-1344,1610-1626; WGSL
// src/shaders.rs:331-383,910-1031; CPU twin src/cpu_decoder.rs:288-322,464-491).
//
// All three are HBM-bound elementwise / row-reduction passes: one wave per
// row (or per (row, head)), 16-byte loads and stores, f32 arithmetic, one
// 16-bit rounding per output.  Rounding points follow the CPU path: the
// norm's inverse RMS comes from the 16-bit input values in f32,
// inv = 1 / sqrt(sum2 / n + eps) with IEEE sqrt and divide.
#include "qa_internal.h"

namespace qa {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <int DT>
__device__ __forceinline__ float widen16(uint32_t h) {
  if constexpr (DT == QA_F16) return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
  else return __uint_as_float(h << 16);
}
template <int DT>
__device__ __forceinline__ uint32_t narrow16(float v) {
  if constexpr (DT == QA_F16) {
    return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)v);
  } else {
    const uint32_t u = __float_as_uint(v);  // src/shaders.rs:169-179
    return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
  }
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// y[r] = r16(x[r] * inv * w), one wave per row, 8 elements per lane per step.
// NC > 0: rows of at most NC * 512 elements stay in registers and w comes as
// 16-byte loads (16-byte aligned); NC = 0: any width, re-reading the row.
// Both sum in the same lane order.
template <int DT, int NC>
__global__ void __launch_bounds__(256) rms_norm_kernel(const RmsParams p) {
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
        for (int e = 0; e < 4; ++e) {
          const float lo = widen16<DT>(v[c][e] & 0xffffu), hi = widen16<DT>(v[c][e] >> 16);
          s += lo * lo;
          s += hi * hi;
        }
      }
    s = wave_sum(s);
    const float inv = 1.0f / sqrtf(s / (float)p.n + p.eps);
#pragma unroll
    for (int c = 0; c < NC; ++c) {
      const int i = lane * 8 + c * 512;
      if (i >= p.n) continue;
      const f32x4 w0 = *reinterpret_cast<const f32x4*>(p.w + i), w1 = *reinterpret_cast<const f32x4*>(p.w + i + 4);
      const float wv[8] = {w0[0], w0[1], w0[2], w0[3], w1[0], w1[1], w1[2], w1[3]};
      u32x4 o;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float lo = widen16<DT>(v[c][e] & 0xffffu) * inv * wv[2 * e];
        const float hi = widen16<DT>(v[c][e] >> 16) * inv * wv[2 * e + 1];
        o[e] = narrow16<DT>(lo) | (narrow16<DT>(hi) << 16);
      }
      *reinterpret_cast<u32x4*>(y + i) = o;
    }
    return;
  }
  float s = 0.f;
  for (int i = lane * 8; i < p.n; i += 512) {
    const u32x4 v = *reinterpret_cast<const u32x4*>(x + i);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float lo = widen16<DT>(v[e] & 0xffffu), hi = widen16<DT>(v[e] >> 16);
      s += lo * lo;
      s += hi * hi;
    }
  }
  s = wave_sum(s);
  const float inv = 1.0f / sqrtf(s / (float)p.n + p.eps);
  for (int i = lane * 8; i < p.n; i += 512) {
    const u32x4 v = *reinterpret_cast<const u32x4*>(x + i);
    u32x4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float lo = widen16<DT>(v[e] & 0xffffu) * inv * p.w[i + 2 * e];
      const float hi = widen16<DT>(v[e] >> 16) * inv * p.w[i + 2 * e + 1];
      o[e] = narrow16<DT>(lo) | (narrow16<DT>(hi) << 16);
    }
    *reinterpret_cast<u32x4*>(y + i) = o;
  }
}

// One wave per (row, head slot): slots 0..nqh-1 are q heads (-> q_out
// head-major [nqh][rows][hd]), nqh..nqh+nkvh-1 k heads (-> k_cache
// [nkvh][cap][hd] at row start + r).  Lane l owns the rotate-half pairs
// (j, j + hd/2) for j = l, l + 64, ..., so both partners of every rotation
// are in one lane.
template <int DT>
__global__ void __launch_bounds__(256) qk_norm_rope_kernel(const RopeParams p) {
  const int lane = threadIdx.x & 63;
  const int64_t item = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int slots = p.nqh + p.nkvh;
  if (item >= p.rows * slots) return;
  const int64_t r = item / slots;
  const int slot = (int)(item % slots);
  const bool is_q = slot < p.nqh;
  const int head = is_q ? slot : slot - p.nqh;
  const int hd = p.hd, half = hd / 2;
  const uint16_t* raw = p.qkv + r * p.ldqkv + (is_q ? 0 : (int64_t)p.nqh * hd) + (int64_t)head * hd;
  const float* nw = is_q ? p.qn : p.kn;
  const float* cs = p.cos + (p.pos0 + r) * hd;
  const float* sn = p.sin + (p.pos0 + r) * hd;
  uint16_t* dst = is_q ? p.q_out + ((int64_t)head * p.rows + r) * hd
                       : p.k_cache + ((int64_t)head * p.cap + p.start + r) * hd;
  float s = 0.f;
  for (int j = lane; j < half; j += 64) {
    const float a = widen16<DT>(raw[j]), b = widen16<DT>(raw[j + half]);
    s += a * a;
    s += b * b;
  }
  s = wave_sum(s);
  const float inv = 1.0f / sqrtf(s / (float)hd + p.eps);
  for (int j = lane; j < half; j += 64) {
    const int k = j + half;
    const float xj = widen16<DT>(raw[j]) * inv * nw[j];
    const float xk = widen16<DT>(raw[k]) * inv * nw[k];
    dst[j] = (uint16_t)narrow16<DT>(xj * cs[j] - xk * sn[j]);
    dst[k] = (uint16_t)narrow16<DT>(xk * cs[k] + xj * sn[k]);
  }
}

// The same op with 16-byte accesses, for hd in {64, 128, 256} and 16-byte
// aligned rows: one wave per (row, group of 1024 / hd head slots), hd / 16
// lanes per head.  A lane owns the 8-element chunks c and c + hd / 16 of its
// head, i.e. the rotate-half partners j and j + hd / 2 for the 8 j of chunk
// c, and the head's sum of squares is reduced over its hd / 16 lanes.  The
// arithmetic per element is qk_norm_rope_kernel's; only the order of the
// sum of squares differs.
template <int DT>
__device__ __forceinline__ void qk_norm_rope_vec_body(const RopeParams& p, int64_t bx) {
  const int lane = threadIdx.x & 63;
  const int L = p.hd >> 4;  // lanes per head: 4, 8 or 16
  const int hpw = 64 / L;   // head slots per wave
  const int slots = p.nqh + p.nkvh;
  const int groups = (slots + hpw - 1) / hpw;
  const int64_t item = bx * 4 + (threadIdx.x >> 6);
  if (item >= p.rows * groups) return;
  const int64_t r = item / groups;
  const int slot = (int)(item % groups) * hpw + lane / L;
  const int c = lane % L;
  const bool active = slot < slots;
  const int half = p.hd >> 1;
  const bool is_q = slot < p.nqh;
  const int head = is_q ? slot : slot - p.nqh;
  // q heads then k heads are contiguous at the start of the fused row
  const uint16_t* raw = p.qkv + r * p.ldqkv + (int64_t)(active ? slot : 0) * p.hd;
  u32x4 va = {0, 0, 0, 0}, vb = {0, 0, 0, 0};
  if (active) {
    va = *reinterpret_cast<const u32x4*>(raw + 8 * c);
    vb = *reinterpret_cast<const u32x4*>(raw + half + 8 * c);
  }
  float xa[8], xb[8];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    xa[2 * e] = widen16<DT>(va[e] & 0xffffu);
    xa[2 * e + 1] = widen16<DT>(va[e] >> 16);
    xb[2 * e] = widen16<DT>(vb[e] & 0xffffu);
    xb[2 * e + 1] = widen16<DT>(vb[e] >> 16);
  }
  float s = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    s += xa[e] * xa[e];
    s += xb[e] * xb[e];
  }
  for (int o = 1; o < L; o <<= 1) s += __shfl_xor(s, o, 64);
  if (!active) return;
  const float inv = 1.0f / sqrtf(s / (float)p.hd + p.eps);
  const float* nw = is_q ? p.qn : p.kn;
  const float* cs = p.cos + (p.pos0 + r) * p.hd;
  const float* sn = p.sin + (p.pos0 + r) * p.hd;
  typedef float f32x4 __attribute__((ext_vector_type(4)));
  float wa[8], wb[8], ca[8], cb[8], sa[8], sb[8];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const f32x4 w0 = *reinterpret_cast<const f32x4*>(nw + 8 * c + 4 * h);
    const f32x4 w1 = *reinterpret_cast<const f32x4*>(nw + half + 8 * c + 4 * h);
    const f32x4 c0 = *reinterpret_cast<const f32x4*>(cs + 8 * c + 4 * h);
    const f32x4 c1 = *reinterpret_cast<const f32x4*>(cs + half + 8 * c + 4 * h);
    const f32x4 s0 = *reinterpret_cast<const f32x4*>(sn + 8 * c + 4 * h);
    const f32x4 s1 = *reinterpret_cast<const f32x4*>(sn + half + 8 * c + 4 * h);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      wa[4 * h + e] = w0[e];
      wb[4 * h + e] = w1[e];
      ca[4 * h + e] = c0[e];
      cb[4 * h + e] = c1[e];
      sa[4 * h + e] = s0[e];
      sb[4 * h + e] = s1[e];
    }
  }
  u32x4 oa, ob;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    uint32_t lo[2], hi[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int i = 2 * e + u;
      const float xj = xa[i] * inv * wa[i];
      const float xk = xb[i] * inv * wb[i];
      lo[u] = narrow16<DT>(xj * ca[i] - xk * sa[i]);
      hi[u] = narrow16<DT>(xk * cb[i] + xj * sb[i]);
    }
    oa[e] = lo[0] | (lo[1] << 16);
    ob[e] = hi[0] | (hi[1] << 16);
  }
  uint16_t* dst = is_q ? p.q_out + ((int64_t)head * p.rows + r) * p.hd
                       : p.k_cache + ((int64_t)head * p.cap + p.start + r) * p.hd;
  *reinterpret_cast<u32x4*>(dst + 8 * c) = oa;
  *reinterpret_cast<u32x4*>(dst + half + 8 * c) = ob;
}

// Column of key t in the transposed V cache: bits 2 and 3 of t swapped, so
// each aligned group of 16 keys is stored 0-3, 8-11, 4-7, 12-15 -- the key
// order in which the attention kernel's P.V fragments hold them.
__device__ __forceinline__ int64_t vperm(int64_t t) {
  return (t & ~(int64_t)12) | ((t & 4) << 1) | ((t & 8) >> 1);
}

// V heads into the transposed cache v_cache[h][d][vperm(start + r)] through a
// 64 (rows) x 64 (d) LDS tile, so the row reads are contiguous and the
// transposed writes stay within 32-byte groups.
template <int DT>
__device__ __forceinline__ void v_transpose_body(const RopeParams& p, int64_t bx, int by, int bz) {
  __shared__ uint16_t tile[64][66];
  const int64_t r0 = bx * 64;
  const int d0 = by * 64;
  const int h = bz;
  const int t = threadIdx.x;
  const uint16_t* v = p.qkv + (int64_t)(p.nqh + p.nkvh) * p.hd + (int64_t)h * p.hd + d0;
  {
    const int rr = t >> 2, c = (t & 3) * 16;
    const int64_t r = r0 + rr;
    if (r < p.rows) {
      const uint16_t* src = v + r * p.ldqkv + c;
#pragma unroll
      for (int e = 0; e < 16; ++e) tile[rr][c + e] = src[e];
    }
  }
  __syncthreads();
  {
    const int dd = t >> 2, c = (t & 3) * 16;
    uint16_t* dst = p.v_cache + ((int64_t)h * p.hd + d0 + dd) * p.cap;
    const int64_t k0 = p.start + r0 + c;  // cache position of this thread's first key
    if ((k0 & 15) == 0 && r0 + c + 16 <= p.rows && (reinterpret_cast<uintptr_t>(dst) & 15) == 0) {
      // a whole aligned group of 16 keys: store it permuted, as two 16-byte runs
      uint32_t w[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int a = (int)vperm(2 * i), b = (int)vperm(2 * i + 1);  // stored column -> key
        w[i] = (uint32_t)tile[c + a][dd] | ((uint32_t)tile[c + b][dd] << 16);
      }
      u32x4* out = reinterpret_cast<u32x4*>(dst + k0);
      out[0] = u32x4{w[0], w[1], w[2], w[3]};
      out[1] = u32x4{w[4], w[5], w[6], w[7]};
    } else {
#pragma unroll
      for (int e = 0; e < 16; ++e)
        if (r0 + c + e < p.rows) dst[vperm(k0 + e)] = tile[c + e][dd];
    }
  }
}

template <int DT>
__global__ void __launch_bounds__(256) v_transpose_kernel(const RopeParams p) {
  v_transpose_body<DT>(p, blockIdx.x, blockIdx.y, blockIdx.z);
}

// Both passes in one grid: blocks [0, nvt) are V-transpose tiles (row tile
// fastest, then d tile, then kv head), the rest are 16-byte q/k blocks.  The
// two write disjoint buffers and read only qkv, so they run concurrently and
// share the HBM stream instead of running one after the other.
template <int DT>
__global__ void __launch_bounds__(256) qk_rope_v_kernel(const RopeParams p, int vtx, int vty,
                                                         int64_t nvt) {
  const int64_t b = blockIdx.x;
  if (b < nvt) {
    const int64_t per_head = (int64_t)vtx * vty;
    v_transpose_body<DT>(p, b % vtx, (int)((b % per_head) / vtx), (int)(b / per_head));
  } else {
    qk_norm_rope_vec_body<DT>(p, b - nvt);
  }
}

}  // namespace

hipError_t launch_rms_norm(int dtype, const RmsParams& p, hipStream_t s) {
  const unsigned blocks = (unsigned)((p.rows + 3) / 4);
  const bool reg = p.n <= 1024 && (reinterpret_cast<uintptr_t>(p.w) & 15) == 0;
  if (dtype == QA_BF16) {
    if (reg) hipLaunchKernelGGL((rms_norm_kernel<QA_BF16, 2>), dim3(blocks), dim3(256), 0, s, p);
    else hipLaunchKernelGGL((rms_norm_kernel<QA_BF16, 0>), dim3(blocks), dim3(256), 0, s, p);
  } else {
    if (reg) hipLaunchKernelGGL((rms_norm_kernel<QA_F16, 2>), dim3(blocks), dim3(256), 0, s, p);
    else hipLaunchKernelGGL((rms_norm_kernel<QA_F16, 0>), dim3(blocks), dim3(256), 0, s, p);
  }
  return hipGetLastError();
}

// The 16-byte form needs hd in {64, 128, 256} and every row it touches
// 16-byte aligned (qkv rows, q / k heads, norm weights, cos / sin rows).
bool rope_vec_ok(const RopeParams& p) {
  auto al = [](const void* q) { return (reinterpret_cast<uintptr_t>(q) & 15) == 0; };
  return (p.hd == 64 || p.hd == 128 || p.hd == 256) && p.ldqkv % 8 == 0 && al(p.qkv) &&
         al(p.q_out) && al(p.k_cache) && al(p.qn) && al(p.kn) && al(p.cos) && al(p.sin);
}

hipError_t launch_qk_norm_rope(int dtype, const RopeParams& p, hipStream_t s) {
  const dim3 vt((unsigned)((p.rows + 63) / 64), (unsigned)(p.hd / 64), (unsigned)p.nkvh);
  const bool vec = rope_vec_ok(p);
  const int slots = p.nqh + p.nkvh;
  const int64_t items = vec ? p.rows * ((slots + 1024 / p.hd - 1) / (1024 / p.hd))
                            : p.rows * slots;
  const dim3 grid((unsigned)((items + 3) / 4));
  if (vec) {
    const int64_t nvt = (int64_t)vt.x * vt.y * vt.z;
    const dim3 fused((unsigned)(nvt + grid.x));
    if (dtype == QA_BF16)
      hipLaunchKernelGGL(qk_rope_v_kernel<QA_BF16>, fused, dim3(256), 0, s, p, (int)vt.x, (int)vt.y, nvt);
    else
      hipLaunchKernelGGL(qk_rope_v_kernel<QA_F16>, fused, dim3(256), 0, s, p, (int)vt.x, (int)vt.y, nvt);
    return hipGetLastError();
  }
  if (dtype == QA_BF16) {
    hipLaunchKernelGGL(qk_norm_rope_kernel<QA_BF16>, grid, dim3(256), 0, s, p);
    hipLaunchKernelGGL(v_transpose_kernel<QA_BF16>, vt, dim3(256), 0, s, p);
  } else {
    hipLaunchKernelGGL(qk_norm_rope_kernel<QA_F16>, grid, dim3(256), 0, s, p);
    hipLaunchKernelGGL(v_transpose_kernel<QA_F16>, vt, dim3(256), 0, s, p);
  }
  return hipGetLastError();
}

}  // namespace qa
