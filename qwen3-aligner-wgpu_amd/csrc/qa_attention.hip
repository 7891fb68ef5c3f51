// qa_attention.hip -- causal GQA prefill attention for gfx950 (hd = 128).
//
// Replaces the reference's prefill attention chain (src/decoder.rs:1346-1600:
// repeat_kv, a scores GEMM per key slab, softmax, the P.V GEMM and the slab
// merge; WGSL src/shaders.rs:2079-2505) with one flash-style kernel; the
// arithmetic it must match is the CPU twin, src/cpu_decoder.rs:324-411: f32
// scores q.k / sqrt(hd), softmax in f32, out = round(sum_t p_t v_t).
//
// Block = one kv head x a tile of 64 query rows x its REP q heads; waves:
// NS = 2 key splits x REP heads x 2 row groups of 32.  Split s takes the key
// blocks kb = s, s + 2, ... (64 keys each) below the tile's causal bound, so
// the long rows' key range is processed by two wave groups at once; the two
// partial results merge through LDS at the end in a fixed order.
//
// Per key block, per wave (32 query rows):
//  * S = K . Q^T on v_mfma_f32_32x32x16 (A = 32 keys x 16 d from LDS, B = the
//    wave's Q fragments, kept in registers for the whole kernel): the lane
//    holds one query row and 16 of each 32-key tile's scores.
//  * online softmax in the log2 domain (v_exp_f32): the row max over the
//    lane's values plus its partner lane (lane ^ 32, same row); the running max
//    moves only when a block's max exceeds it by more than 2^8, and then the
//    running output and sum are rescaled by exp2(m_old - m_new); each lane
//    keeps its half of the row sum until the end.
//  * O^T += V^T . P^T: P goes from the score registers straight into the
//    MFMA's B operand.  The reference's GPU path rounds its probabilities to
//    the 16-bit format before its P.V GEMM (PS = 1 here), which costs up to
//    2^-11 (f16) / 2^-8 (bf16) relative per weight; by default (PS = 2) the
//    rounding residue goes through a second MFMA as a second 16-bit term, so
//    the product carries ~2^-22 / 2^-16 and the result tracks the f32 CPU
//    path.  f16 probabilities are formed scaled by 2^7 so that they stay in
//    the normal range (the scale cancels in the final division).  A lane half holds
//    keys {16j+4h..+3, 16j+8+4h..+3} of slice j, so the transposed V cache
//    stores each aligned group of 16 keys in the order 0-3, 8-11, 4-7, 12-15
//    (bits 2 and 3 of the key swapped): one 16-byte read per V fragment.
//  * K and V tiles stream L2 -> LDS with buffer_load ... lds, double-buffered
//    per split group; chunks are XOR-swizzled per row so the 32-row fragment
//    reads hit distinct banks.
#include <type_traits>

#include "qa_internal.h"

namespace qa {

#ifdef QA_PHASE_STAMPS
// Measurement build only (make stamps): every wave of an attention_kernel
// launch adds up s_memtime (shader clock) cycles by phase -- the prologue up
// to the phase loop, the MFMA phases (P.V + S issued), the VALU phases
// (softmax, DMA issue), the phases with no work of its own, the block
// barrier after each phase, the merge and output, and the DMA and LDS waits
// before each barrier -- and counts its MFMA and VALU phases.  Words per
// wave: those seven sums, the two counts.
constexpr int kAttnStampBlocks = 2048, kAttnStampWaves = 8, kAttnStampWords = 9;
__device__ unsigned long long attn_stamp_log[kAttnStampBlocks * kAttnStampWaves * kAttnStampWords];
#endif
namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

#define QA_LDS __attribute__((address_space(3)))

constexpr uint32_t OOB = 0x80000000u;
constexpr int HD = 128;  // head dim
constexpr int QT = 64;   // query rows per block
constexpr int KB = 64;   // keys per block
constexpr int NS = 2;    // key splits per block
constexpr float kLog2e = 1.44269504088896341f;
// The running row max is raised only when a block's max exceeds it by more
// than this (log2 units): probabilities then stay <= 2^kLazy and the output
// rescale runs once per such jump instead of once per block.
constexpr float kLazy = 8.f;

// Max / sum of a value over lane pairs (l, l ^ 32), on v_permlane32_swap: the
// two results hold the wave's lower and upper 32-lane halves exchanged in one
// of them, so a symmetric combination of both is the pair's result on every
// lane, identical on the two lanes of a pair.
__device__ __forceinline__ float pair_max(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float pair_sum(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                  false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

template <int DT>
struct AFmt;
template <>
struct AFmt<QA_F16> {
  __device__ static __forceinline__ f32x16 mfma(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
  // two values, RNE, element a in the low half (v_cvt_pk_f16_f32)
  __device__ static __forceinline__ uint32_t pack2(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){a, b}, f16x2));
  }
  __device__ static __forceinline__ f32x2 unpack2(uint32_t h) {
    return __builtin_convertvector(__builtin_bit_cast(f16x2, h), f32x2);
  }
  // (a, b) minus their 16-bit roundings h (packed: a's in the low half), as
  // two 16-bit values.  Each difference is exact in f32 (a and h agree in
  // their leading bits), so v_fma_mix_f32 (-h) * 1 + a, which reads h
  // straight from its half of the packed word, gives the same bits as
  // widening h and subtracting, in one instruction instead of two.  a and b
  // are v_exp_f32 results, and the compiler puts no wait state ahead of an
  // asm statement; h = pack2(a, b) is a compiler instruction that reads both
  // and precedes these by its data dependency, so the transcendental's
  // one-instruction wait state has passed when they read a and b.
  __device__ static __forceinline__ uint32_t residue2(uint32_t h, float a, float b) {
    float d0, d1;
    asm("v_fma_mix_f32 %0, -%1, 1.0, %2 op_sel_hi:[1,0,0]" : "=v"(d0) : "v"(h), "v"(a));
    asm("v_fma_mix_f32 %0, -%1, 1.0, %2 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(d1) : "v"(h), "v"(b));
    return pack2(d0, d1);
  }
  // Probabilities are formed as p * 2^7; with the running max allowed to lag
  // the true one by up to 2^8 (kLazy) they stay <= 2^15, and the f16 range
  // keeps them normal down to p = 2^-21, so rounding them loses only relative
  // precision (below that, at most 2^-32 absolute).
  static constexpr float kPBias = 7.f;
};
template <>
struct AFmt<QA_BF16> {
  __device__ static __forceinline__ f32x16 mfma(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
  // two values, RNE (v_cvt_pk_bf16_f32): for finite values the reference's
  // (u + 0x7fff + ((u >> 16) & 1)) >> 16, src/shaders.rs:169-179
  __device__ static __forceinline__ uint32_t pack2(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){a, b}, bf16x2));
  }
  __device__ static __forceinline__ f32x2 unpack2(uint32_t h) {
    return (f32x2){__uint_as_float(h << 16), __uint_as_float(h & 0xffff0000u)};
  }
  __device__ static __forceinline__ uint32_t residue2(uint32_t h, float a, float b) {
    const f32x2 hv = unpack2(h);
    return pack2(a - hv[0], b - hv[1]);
  }
  static constexpr float kPBias = 0.f;
};

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}
__device__ __forceinline__ void wait_lds() {
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_waitcnt(0xF | (0x3 << 14) | (0x7 << 4) | (0x0 << 8));
}
__device__ __forceinline__ void exec_barrier() {
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
}

// LDS tile layouts.  K tile: 64 key rows x 256 B (16 chunks of 8 d); chunk c of
// row r at c ^ (r & 15).  V tile: 128 d rows x 128 B (8 chunks of 8 stored key
// positions); chunk c of row d at c ^ ((d >> 1) & 7).
__device__ __forceinline__ int kswz(int r) { return r & 15; }
__device__ __forceinline__ int vswz(int d) { return (d >> 1) & 7; }

template <int DT, int REP, int PS>
__global__ void __launch_bounds__(NS * REP * 2 * 64) attention_kernel(const AttnParams p) {
  constexpr int GW = REP * 2;        // waves per split group
  constexpr int KTILE = KB * HD * 2;  // 16 KB
  constexpr int VTILE = HD * KB * 2;  // 16 KB
  constexpr int KI = KB * HD * 2 / 1024 / GW;  // K DMA instructions per wave per block
  constexpr int VI = HD * KB * 2 / 1024 / GW;  // V DMA instructions per wave per block
  constexpr int LPS = KI + VI;
  static_assert(KI * GW * 4 == KB && VI * GW * 8 == HD, "DMA row coverage");
  __shared__ __attribute__((aligned(1024))) unsigned char smem[NS * 2 * (KTILE + VTILE)];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int split = wave / GW, wg = wave % GW;
  const int hh = wg / 2, rg = wg & 1;
  const int fr = lane & 31, fh = lane >> 5;
#ifdef QA_PHASE_STAMPS
  // s_memtime cycles by phase: prologue, MFMA, VALU, no work, barrier,
  // merge, DMA + LDS waits
  unsigned long long cyc[7] = {0, 0, 0, 0, 0, 0, 0}, nmma = 0, nvalu = 0;
  __builtin_amdgcn_sched_barrier(0);
  unsigned long long c_mark = __builtin_amdgcn_s_memtime();
  __builtin_amdgcn_sched_barrier(0);
#endif

  // Block b -> kv head b % nkvh, row tile T - 1 - b / nkvh: the longest key
  // ranges of every head are dispatched first, and with blocks dealt
  // round-robin over the 8 XCDs all blocks of a head land on one XCD (for
  // nkvh a multiple of 8), whose L2 then holds that head's K and V.
  const int T = (int)((p.rows + QT - 1) / QT);
  const int t = T - 1 - (int)(blockIdx.x / p.nkvh);
  const int kvh = (int)(blockIdx.x % p.nkvh);
  const int head = kvh * REP + hh;
  const int64_t row0 = (int64_t)t * QT;
  const int64_t kend = p.q0 + min(row0 + QT, p.rows);  // keys 0..kend-1 are visible
  const int nkb = (int)((kend + KB - 1) / KB);

  // ---- LDS: per split group, K slots 0/1 then V slots 0/1 (16 KB each) ----
  unsigned char* gsm = smem + split * 2 * (KTILE + VTILE);
  auto kslot = [&](int it) { return gsm + (it & 1) * KTILE; };
  auto vslot = [&](int it) { return gsm + 2 * KTILE + (it & 1) * VTILE; };
  // this group's steps: key blocks split, split + NS, ... below nkb
  const int nst = (nkb - split + NS - 1) / NS;

  // ---- DMA (the group's GW waves share each tile) ----
  const uint16_t* kbase = p.k_cache + (int64_t)kvh * p.cap * HD;
  const uint16_t* vbase = p.v_cache + (int64_t)kvh * HD * p.cap;
  const __amdgpu_buffer_rsrc_t rsk = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(kbase), (short)0, (int)(p.cap * HD * 2), 0x00020000);
  const __amdgpu_buffer_rsrc_t rsv = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(vbase), (short)0, (int)(p.cap * HD * 2), 0x00020000);
  // Per-lane byte offsets of this wave's chunks at key block 0.  K
  // instruction j fills key rows 4 (GW j + wg) + lane / 16 and V instruction j
  // d rows 8 (GW j + wg) + lane / 8; with GW = 4 the K chunk swizzle (row & 15)
  // and for any GW the V chunk swizzle ((d >> 1) & 7) are the same for every
  // j, so instruction j's offset is the lane's offset at j = 0 plus a
  // wave-uniform amount: one add per instruction.  K rows at or past cap lie
  // past the buffer's num_records and read as zeros; a V column at or past cap
  // would not (it lies inside the next d row), so those lanes get OOB.
  // (The lane offsets are recomputed at each refill, a few instructions, from
  // a copy of the lane index the compiler cannot hoist: kept live across the
  // loop they would push the kernel past its register budget.)
  auto lane_opaque = [&]() {
    int l = lane;
    asm volatile("" : "+v"(l));
    return l;
  };
  auto issue_k = [&](int it) {
    unsigned char* sk = kslot(it);
    const int kb = split + NS * it;
    const int l = lane_opaque(), rk = wg * 4 + (l >> 4);
    const uint32_t koff0 = (uint32_t)((rk * HD + (((l & 15) ^ kswz(rk)) << 3)) * 2);
#pragma unroll
    for (int j = 0; j < KI; ++j) {
      const int ins = j * GW + wg;
      uint32_t off;
      if constexpr (GW * 4 % 16 == 0) {
        off = koff0 + (uint32_t)(((int64_t)kb * KB + 4 * GW * j) * HD * 2);
      } else {
        const int r = ins * 4 + (l >> 4);  // key row within the tile
        const int64_t key = (int64_t)kb * KB + r;
        off = key < p.cap ? (uint32_t)((key * HD + (((l & 15) ^ kswz(r)) << 3)) * 2) : OOB;
      }
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rsk, (QA_LDS void*)(sk + ins * 1024), 16, off, 0,
                                               0, 0);
    }
  };
  auto issue_v = [&](int it) {
    unsigned char* sv = vslot(it);
    const int kb = split + NS * it;
    const int l = lane_opaque(), dv = wg * 8 + (l >> 3);
    const int vc = ((l & 7) ^ vswz(dv)) << 3;
    const uint32_t voff0 = (uint32_t)(((int64_t)dv * p.cap + vc) * 2);
    const bool vin = (int64_t)kb * KB + vc < p.cap;
#pragma unroll
    for (int j = 0; j < VI; ++j) {
      const int ins = j * GW + wg;
      const uint32_t off =
          vin ? voff0 + (uint32_t)(((int64_t)8 * GW * j * p.cap + (int64_t)kb * KB) * 2) : OOB;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rsv, (QA_LDS void*)(sv + ins * 1024), 16, off, 0,
                                               0, 0);
    }
  };
  // Loads issued by refill(j), in the VALU phase of step j: K(j + 2) into K
  // slot j & 1 (S(j) has read it) and V(j + 1) into V slot (j + 1) & 1 (P.V of
  // step j - 1 has read it).  The MFMA phase of step i needs K(i) and V(i - 1),
  // issued by refill(i - 1); only refill(i)'s loads may still be in flight.
  auto refill_count = [&](int j) { return (j + 2 < nst ? KI : 0) + (j + 1 < nst ? VI : 0); };
  auto wait_refill = [&](int c) {
    static_assert(KI == VI, "refill counts are 0, VI or KI + VI");
    if (c == LPS)
      wait_vmcnt<LPS>();
    else if (c == VI)
      wait_vmcnt<VI>();
    else
      wait_vmcnt<0>();
  };

  // ---- this wave's 32 query rows, as MFMA B fragments (8 slices of 16 d) ----
  const int64_t qrow = row0 + rg * 32 + fr;
  u32x4 qf[8];
  {
    const uint16_t* q = p.q + ((int64_t)head * p.rows + qrow) * HD + fh * 8;
#pragma unroll
    for (int s = 0; s < 8; ++s)
      qf[s] = qrow < p.rows ? *reinterpret_cast<const u32x4*>(q + s * 16) : u32x4{0, 0, 0, 0};
  }
  const int pos = (int)(p.q0 + qrow);                   // this lane's query position
  const int wpos0 = (int)(p.q0 + row0 + rg * 32);       // the wave's first position
  const float sc = p.scale * kLog2e;

  f32x16 o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) o[i] = f32x16{0};
  float m_run = -INFINITY, l_run = 0.f;
  f32x16 s[2] = {f32x16{0}, f32x16{0}};
  u32x4 pf[4], pl[4];

  // MFMA phase of step it: P.V of step it - 1 (V slot (it - 1) & 1) and
  // S = K.Q^T of step it (K slot it & 1).  Per 16-deep slice st: the P.V
  // MFMAs of the value terms, the two S MFMAs, then the residue terms, so the
  // two MFMAs on one O accumulator are never adjacent; the fragments of
  // slice st + 1 are read from LDS while slice st multiplies (the schedule
  // groups below keep the compiler from sinking the reads next to their use).
  auto mma = [&](auto pv_tag, auto s_tag, int it) {
    constexpr bool PV = decltype(pv_tag)::value, SQ = decltype(s_tag)::value;
    const unsigned char* sk = kslot(it);
    const unsigned char* sv = vslot(it - 1);
    if constexpr (SQ) {
      s[0] = f32x16{0};
      s[1] = f32x16{0};
    }
    auto rd_v = [&](int st, u32x4* vf) {
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int q = 2 * st + u, dt = q & 3, j = q >> 2;
        const int d = dt * 32 + fr;
        vf[u] = *reinterpret_cast<const u32x4*>(sv + d * 128 + (((2 * j + fh) ^ vswz(d)) << 4));
      }
    };
    auto rd_k = [&](int st, u32x4* kf) {
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) {
        const int r = kt * 32 + fr;
        kf[kt] = *reinterpret_cast<const u32x4*>(sk + r * 256 + (((2 * st + fh) ^ kswz(r)) << 4));
      }
    };
    u32x4 vf[2][2], kf[2][2];
    if constexpr (PV) rd_v(0, vf[0]);
    if constexpr (SQ) rd_k(0, kf[0]);
#pragma unroll
    for (int st = 0; st < 8; ++st) {
      const int cur = st & 1, nxt = cur ^ 1;
      if (st + 1 < 8) {
        if constexpr (PV) rd_v(st + 1, vf[nxt]);
        if constexpr (SQ) rd_k(st + 1, kf[nxt]);
      }
      if constexpr (PV) {
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const int q = 2 * st + u, dt = q & 3, j = q >> 2;
          o[dt] = AFmt<DT>::mfma(vf[cur][u], pf[j], o[dt]);
        }
      }
      if constexpr (SQ) {
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) s[kt] = AFmt<DT>::mfma(kf[cur][kt], qf[st], s[kt]);
      }
      if constexpr (PV && PS == 2) {
#pragma unroll
        for (int u = 0; u < 2; ++u) {
          const int q = 2 * st + u, dt = q & 3, j = q >> 2;
          o[dt] = AFmt<DT>::mfma(vf[cur][u], pl[j], o[dt]);
        }
      }
    }
    if constexpr (PV && SQ) {
      // 4 fragment reads, then the slice's 4 or 6 MFMAs, slice by slice
      __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
      for (int st = 0; st < 7; ++st) {
        __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, PS == 2 ? 6 : 4, 0);
      }
      __builtin_amdgcn_sched_group_barrier(0x008, PS == 2 ? 6 : 4, 0);
    }
  };

  // VALU phase of step it: causal mask, online softmax, P to 16-bit terms,
  // rescale of O.
  auto softmax = [&](int it) {
    const int kb = split + NS * it;
    if (kb * KB + KB - 1 > wpos0) {  // only blocks that cross this wave's diagonal
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int g = 0; g < 4; ++g)
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (kb * KB + kt * 32 + 8 * g + 4 * fh + e > pos) s[kt][4 * g + e] = -INFINITY;
    }
    // row max of the raw scores (four independent chains); the scale (> 0)
    // is applied to the max and, fused, in the exponent: exp2(s sc - m)
    float mx[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int i = 0; i < 16; ++i) mx[i & 3] = fmaxf(mx[i & 3], s[kt][i]);
    const float bm = pair_max(fmaxf(fmaxf(mx[0], mx[1]), fmaxf(mx[2], mx[3]))) * sc;
    if (__builtin_amdgcn_ballot_w64(bm > m_run + kLazy)) {  // some row's max jumped
      const float m_new = fmaxf(m_run, bm);
      const float alpha = __builtin_amdgcn_exp2f(m_run - (m_new == -INFINITY ? 0.f : m_new));
      l_run *= alpha;
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) o[dt] *= alpha;
      m_run = m_new;
    }
    const float m_b = (m_run == -INFINITY ? 0.f : m_run) - AFmt<DT>::kPBias;
    float rs[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        float pv[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          pv[e] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[kt][4 * g + e], sc, -m_b));
          rs[e] += pv[e];
        }
        // slice j = 2 kt + g / 2 holds groups g = 2(j%2), 2(j%2)+1 of tile kt
        const int j = 2 * kt + (g >> 1), half = g & 1;
        pf[j][2 * half] = AFmt<DT>::pack2(pv[0], pv[1]);
        pf[j][2 * half + 1] = AFmt<DT>::pack2(pv[2], pv[3]);
        if constexpr (PS == 2) {  // the rounding residue as a second 16-bit term
          pl[j][2 * half] = AFmt<DT>::residue2(pf[j][2 * half], pv[0], pv[1]);
          pl[j][2 * half + 1] = AFmt<DT>::residue2(pf[j][2 * half + 1], pv[2], pv[3]);
        }
      }
    // this lane's half of the row sum; the halves are added once at the end
    l_run += (rs[0] + rs[1]) + (rs[2] + rs[3]);
  };

  // ---- phases: the two split groups run half a step apart ("ping-pong") ----
  // A group's step it is an MFMA phase (P.V(it - 1) + S(it)) followed by a
  // VALU phase (softmax(it)); group 1 runs one phase behind group 0, so on
  // every SIMD (one wave of each group) one wave's MFMAs overlap the other's
  // softmax.  Every phase ends in a block barrier, which also orders each
  // group's LDS reads before the refills that overwrite them.
  const int n0 = (nkb + 1) / 2, n1 = nkb / 2;
  const int phases = max(2 * n0 + 1, 2 * n1 + 2);
  using T_ = std::true_type;
  using F_ = std::false_type;
  if (nst > 0) issue_k(0);  // refill(-2)
  if (nst > 1) issue_k(1);  // refill(-1): K(1), V(0)
  if (nst > 0) issue_v(0);
  if (split == 0) wait_refill(refill_count(-1));
  exec_barrier();
#ifdef QA_PHASE_STAMPS
  auto stamp = [&](int bucket) {  // charge the cycles since the last mark to a bucket
    __builtin_amdgcn_sched_barrier(0);
    const unsigned long long now = __builtin_amdgcn_s_memtime();
    __builtin_amdgcn_sched_barrier(0);
    cyc[bucket] += now - c_mark;
    c_mark = now;
  };
  stamp(0);
#endif
  for (int ph = 0; ph < phases; ++ph) {
    const int my = ph - split;
#ifdef QA_PHASE_STAMPS
    int bucket = 3;
#endif
    if (my >= 0 && my <= 2 * nst) {
      const int it = my >> 1;
      if ((my & 1) == 0) {
        if (it >= 1 && it < nst)
          mma(T_{}, T_{}, it);
        else if (it == 0 && nst > 0)
          mma(F_{}, T_{}, it);
        else if (it == nst && it >= 1)
          mma(T_{}, F_{}, it);
#ifdef QA_PHASE_STAMPS
        bucket = 1;
        ++nmma;
#endif
      } else {
        if (it + 2 < nst) issue_k(it + 2);
        if (it + 1 < nst) issue_v(it + 1);
        softmax(it);
#ifdef QA_PHASE_STAMPS
        bucket = 2;
        ++nvalu;
#endif
      }
    }
#ifdef QA_PHASE_STAMPS
    stamp(bucket);
#endif
    const int nx = ph + 1 - split;  // this wave's next phase
    if (nx >= 0 && (nx & 1) == 0 && (nx >> 1) <= nst) wait_refill(refill_count((nx >> 1) - 1));
    wait_lds();
#ifdef QA_PHASE_STAMPS
    stamp(6);
#endif
    exec_barrier();
#ifdef QA_PHASE_STAMPS
    stamp(4);
#endif
  }

  // ---- merge the two key splits (fixed order) and write the output ----
  l_run = pair_sum(l_run);  // both lane halves of the row
  __syncthreads();
  float* xch = reinterpret_cast<float*>(smem);  // [GW waves][66 values][64 lanes]
  if (split == 1) {
    float* dst = xch + (size_t)wg * 66 * 64 + lane;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int v = 0; v < 16; ++v) dst[(dt * 16 + v) * 64] = o[dt][v];
    dst[64 * 64] = m_run;
    dst[65 * 64] = l_run;
  }
  __syncthreads();
  if (split == 0 && qrow < p.rows) {
    const float* src = xch + (size_t)wg * 66 * 64 + lane;
    const float m1 = src[64 * 64], l1 = src[65 * 64];
    const float mm = fmaxf(m_run, m1);
    const float mu = mm == -INFINITY ? 0.f : mm;
    const float a0 = __builtin_amdgcn_exp2f(m_run - mu), a1 = __builtin_amdgcn_exp2f(m1 - mu);
    const float inv = 1.0f / (l_run * a0 + l1 * a1);
    uint16_t* out = p.out + qrow * p.ldo + (int64_t)head * HD;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        float v[4];
#pragma unroll
        for (int e = 0; e < 4; ++e)
          v[e] = (o[dt][4 * g + e] * a0 + src[(dt * 16 + 4 * g + e) * 64] * a1) * inv;
        const u32x2 pk = {AFmt<DT>::pack2(v[0], v[1]), AFmt<DT>::pack2(v[2], v[3])};
        *reinterpret_cast<u32x2*>(out + dt * 32 + 8 * g + 4 * fh) = pk;
      }
  }
#ifdef QA_PHASE_STAMPS
  stamp(5);
  if (lane == 0 && blockIdx.x < (unsigned)kAttnStampBlocks && wave < kAttnStampWaves) {
    unsigned long long* d =
        attn_stamp_log + ((size_t)blockIdx.x * kAttnStampWaves + wave) * kAttnStampWords;
    for (int i = 0; i < 7; ++i) d[i] = cyc[i];
    d[7] = nmma;
    d[8] = nvalu;
  }
#endif
}

}  // namespace

hipError_t launch_attention(int dtype, const AttnParams& p, bool p16, hipStream_t s) {
  const int rep = p.nqh / p.nkvh;
  const dim3 grid((unsigned)((p.rows + QT - 1) / QT * p.nkvh));
  const dim3 block(NS * rep * 2 * 64);
  void (*k)(AttnParams) = nullptr;
#define QA_ATTN_PICK(R)                                                                      \
  if (dtype == QA_BF16)                                                                      \
    k = p16 ? attention_kernel<QA_BF16, R, 1> : attention_kernel<QA_BF16, R, 2>;             \
  else                                                                                       \
    k = p16 ? attention_kernel<QA_F16, R, 1> : attention_kernel<QA_F16, R, 2>;
  if (rep == 2) {
    QA_ATTN_PICK(2)
  } else if (rep == 1) {
    QA_ATTN_PICK(1)
  } else {
    return hipErrorInvalidValue;  // rejected by qa_attention_prefill's validation
  }
#undef QA_ATTN_PICK
  hipLaunchKernelGGL(k, grid, block, 0, s, p);
  return hipGetLastError();
}

}  // namespace qa

#ifdef QA_PHASE_STAMPS
// The measurement build's attention records: kAttnStampBlocks x
// kAttnStampWaves x kAttnStampWords words (see attn_stamp_log), copied to
// `out`; *blocks, *waves and *words get the sizes.
extern "C" int qa_attn_stamps_read(unsigned long long* out, int* blocks, int* waves, int* words) {
  if (blocks) *blocks = qa::kAttnStampBlocks;
  if (waves) *waves = qa::kAttnStampWaves;
  if (words) *words = qa::kAttnStampWords;
  if (!out) return QA_OK;
  const hipError_t e =
      hipMemcpyFromSymbol(out, HIP_SYMBOL(qa::attn_stamp_log), sizeof(qa::attn_stamp_log));
  return e == hipSuccess ? QA_OK : QA_EDEVICE;
}
// Zeroes every record (synchronous; call outside stream capture).
extern "C" int qa_attn_stamps_clear(void) {
  static unsigned long long zeros[sizeof(qa::attn_stamp_log) / 8];
  const hipError_t e =
      hipMemcpyToSymbol(HIP_SYMBOL(qa::attn_stamp_log), zeros, sizeof(qa::attn_stamp_log));
  return e == hipSuccess ? QA_OK : QA_EDEVICE;
}
#endif
