// qa_gemm.hip -- MFMA GEMM kernels for gfx950 (CDNA4): C = A . W^T + epilogue.
//
// The reference's WGSL `prefill_gemm` (src/shaders.rs:1846-2077) runs this
// contraction as scalar f32 FMAs over a 128x128 tile with f32 LDS; here the
// same contraction runs on the wave64 matrix cores.
//
// Main kernel (gemm_dma_kernel), for W in the checkpoint's [N, K] layout:
//  * v_mfma_f32_32x32x16_{f16,bf16}.  The operands are swapped relative to
//    C = A.W^T: the MFMA's A operand is a 32-row slice of W (32 output columns
//    n), its B operand a 32-row slice of A (32 tokens m), so each lane's
//    accumulators hold ONE token and runs of 4 consecutive columns.  The
//    LDS-staged epilogue stores 8-byte packs; it finds a gate column and its
//    up column (the first and second half of a SiLU tile's W rows, held by
//    different waves) in one row of the parked tile.
//  * Both operands are K-contiguous in HBM, the natural MFMA operand layout:
//    no transposition anywhere.  Tiles stream HBM -> LDS with
//    buffer_load_dwordx4 ... lds (direct to LDS, no VGPR staging) into an
//    S-stage ring; a stage is waited for with an explicit vmcnt that leaves
//    the next S-2 stages in flight, so HBM/L2 latency hides behind S-1 stages
//    of MFMA work.  One s_barrier per stage, without a memory fence (a
//    workgroup fence would drain every in-flight stage).
//  * LDS tile rows are 128 bytes (BK = 64 elements, 8 chunks of 16 B); chunk
//    c of row r sits at c ^ ((r >> 1) & 7), so a fragment read (32 rows x one chunk)
//    spreads over all banks.  A DMA instruction fills 8 rows (1 KB, one 16 B
//    chunk per lane): lane l writes physical chunk l & 7 of row l >> 3 and so
//    fetches that row's logical chunk (l & 7) ^ swz(row).
//  * Out-of-range rows (m >= M, n >= N) and k chunks (>= this split's end)
//    get an offset past the buffer's num_records, which the buffer unit
//    answers with zeros: ragged edges cost nothing and need no padding.
//  * XCD-aware block order: the hardware deals workgroups round-robin over
//    the 8 XCDs; units are renumbered so each XCD gets a contiguous range of
//    a banded tile enumeration (tile_of), sized so its L2 fetches the fewest
//    A and W rows.
//  * Split-K: each split writes f32 partials; splitk_reduce_kernel sums them
//    in split order (deterministic) and runs the epilogue.
//
// Epilogues (one 16-bit rounding per output, src/shaders.rs:2045-2073): bias
// per column (or per row, the channel-major conv), residual add (beta = 1),
// erf GELU (src/audio_encoder.rs:196-202 on the value of
// src/shaders.rs:2586-2652) and SiLU.up (src/cpu_decoder.rs:496-505 on the
// [gate | up] pair src/shaders.rs:1411-1450 reads).
//
// gemm_reg_kernel is the W-as-[K, N] form (the reference's `transb` conv
// operand, src/shaders.rs:1936-1944): register-staged loads that transpose the
// operand into the same K-contiguous LDS layout.
#include <hip/hip_ext.h>

#include "qa_internal.h"

namespace qa {

#ifdef QA_PHASE_STAMPS
// Measurement build only (make stamps): every block of a gemm_dma_kernel
// launch records s_memrealtime (100 MHz) at its start, when ring stage 0 is
// in (after the first barrier), after the main loop, after the park (the
// first store) and at its end, plus its CU id and the launch's N and K, and
// three points of its first DMA-issuing thread's prologue (kernel arguments
// in, tile enumeration done, the first S ring stages issued), in record slot
// p.stamp_slot; the host cycles the slots launch by launch.
constexpr int kStampSlots = 8, kStampBlocks = 2048, kStampWords = 12;
__device__ unsigned long long stamp_log[kStampSlots * kStampBlocks * kStampWords];
#endif

namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

#define QA_LDS __attribute__((address_space(3)))

constexpr int BK = 64;   // k elements per LDS stage: 128-byte tile rows
constexpr int NT = 256;  // threads per block (4 waves)
constexpr uint32_t OOB = 0x80000000u;  // byte offset past every operand's num_records

template <int DT>
struct Fmt;

template <>
struct Fmt<QA_F16> {
  __device__ static __forceinline__ f32x16 mfma(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
  __device__ static __forceinline__ float widen(uint32_t h) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
  }
  // IEEE round-to-nearest-even (v_cvt_f16_f32 in the default round mode).
  __device__ static __forceinline__ uint32_t narrow(float v) {
    return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)v);
  }
};

template <>
struct Fmt<QA_BF16> {
  __device__ static __forceinline__ f32x16 mfma(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
  __device__ static __forceinline__ float widen(uint32_t h) { return __uint_as_float(h << 16); }
  // The storage format's rounding rule, src/shaders.rs:169-179.
  __device__ static __forceinline__ uint32_t narrow(float v) {
    const uint32_t u = __float_as_uint(v);
    return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
  }
};

// 16-byte chunk swizzle of an LDS tile row.  gfx950's LDS serves a 16-lane
// quarter of a ds_read_b128 from 64 banks: rows r and r+1 sit in opposite bank
// halves (128-byte rows), so pairs of rows share a swizzle value and 16
// consecutive rows read one logical chunk without a conflict.
__device__ __forceinline__ int swz(int row) { return (row >> 1) & 7; }

__device__ __forceinline__ int xcd_remap(int b, int n) {
  constexpr unsigned X = 8;  // XCDs per MI355X
  const unsigned ub = (unsigned)b, full = (unsigned)n - (unsigned)n % X;
  if (ub >= full) return b;
  return (int)((ub % X) * (full / X) + ub / X);
}

// Block -> (tile m, tile n, k split).  Workgroups are dealt round-robin over
// the 8 XCDs (block b runs on XCD b % 8), each with its own L2; xcd_remap
// gives each XCD a contiguous range of the tile enumeration below, so what an
// XCD's L2 must fetch is the A rows and W rows one such range touches.  Tiles
// are enumerated in bands of group_m m-tiles (the last band may be shorter):
// within a band, m runs fastest, then n, so a range of r tiles covers about
// group_m m-tiles x r/group_m n-tiles.  group_m = tiles_m enumerates whole
// n-columns (all of A per XCD), group_m = 1 whole m-rows (all of W); the
// planner picks the value that fetches the fewest operand rows.  The k splits
// of a tile are adjacent.
__device__ __forceinline__ void tile_of(const GemmParams& p, int b, int& tm, int& tn,
                                        int& split) {
  const int u = xcd_remap(b, p.tiles_m * p.tiles_n * p.splits);
  const int t = fastdiv(u, p.fd_split);
  split = u - t * p.splits;
  const int g = p.group_m;
  const int band = fastdiv(t, p.fd_band);
  const int i = t - band * g * p.tiles_n;
  const bool last = (band + 1) * g > p.tiles_m;  // a short last band
  const int rows = last ? p.tiles_m - band * g : g;
  tn = fastdiv(i, last ? p.fd_last : p.fd_rows);
  tm = band * g + (i - tn * rows);
}

// A value the caller knows to be equal in every lane, as a scalar register.
__device__ __forceinline__ int wave_uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }

// One 16-byte-per-lane DMA of a buffer into LDS (buffer_load_dwordx4 ... lds):
// lane l's 16 bytes at byte offset `off` land at lds + 16 l.
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t rs, unsigned char* lds, uint32_t off) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (QA_LDS void*)lds, 16, off, 0, 0, 0);
}

// s_waitcnt vmcnt(N) leaving expcnt / lgkmcnt unconstrained (gfx9 encoding).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// s_waitcnt lgkmcnt(0): this wave's LDS reads have returned.  The scheduling
// barrier keeps earlier MFMAs from sinking below the wait.
__device__ __forceinline__ void wait_lds() {
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_waitcnt(0xF | (0x3 << 14) | (0x7 << 4) | (0x0 << 8));
}

// Workgroup execution barrier with no memory fence; the asm statements keep
// the compiler from moving LDS accesses across it.
__device__ __forceinline__ void exec_barrier() {
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
}

// The epilogue math runs on the hardware transcendentals (v_exp_f32 = 2^x,
// v_rcp_f32 = 1/x, about 1 f32 ulp each): a full-precision expf / erff and an
// IEEE divide cost ~30-40 VALU instructions per output, which made the
// SiLU.up epilogue a quarter of the gate|up kernel.  Either error is a few f32
// ulps, far below the 16-bit rounding that follows.
// The erf GELU is gelu_erf, SiLU.up silu_mul / silu_mul_f16x2 (qa_internal.h).

// Output stores carry sc1 (device scope): the lines are written through the
// XCD's L2 as they are stored, so the end-of-kernel release has no dirty
// output to write back, and they stay cacheable for the next kernel, which
// reads them as its A operand or residual.  Measured on the config-3 layer
// sequence: 1.3% faster per step than plain stores.  Nontemporal stores
// shorten the producer too, but then the consumer fetches its operand from
// HBM: the down projection right after gate|up took 18.7 us against 14.9.
// f16 pairs convert as 2-vectors, which gfx950 rounds in one
// v_cvt_pk_f16_f32 (round to nearest even, as the scalar conversion): 2
// instructions per 4 outputs instead of 4 conversions and 2 ORs.
template <int DT>
__device__ __forceinline__ void store4(uint16_t* p, const float* v) {
  u32x2 w;
  if constexpr (DT == QA_F16) {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    w.x = __builtin_bit_cast(uint32_t, h2{(_Float16)v[0], (_Float16)v[1]});
    w.y = __builtin_bit_cast(uint32_t, h2{(_Float16)v[2], (_Float16)v[3]});
  } else {
    w.x = Fmt<DT>::narrow(v[0]) | (Fmt<DT>::narrow(v[1]) << 16);
    w.y = Fmt<DT>::narrow(v[2]) | (Fmt<DT>::narrow(v[3]) << 16);
  }
  asm volatile("global_store_dwordx2 %0, %1, off sc1" ::"v"(p), "v"(w) : "memory");
}

template <int DT>
__device__ __forceinline__ void widen4(u32x2 w, float* v) {
  v[0] = Fmt<DT>::widen(w.x & 0xffffu);
  v[1] = Fmt<DT>::widen(w.x >> 16);
  v[2] = Fmt<DT>::widen(w.y & 0xffffu);
  v[3] = Fmt<DT>::widen(w.y >> 16);
}

// v[e] += the f16 value e of the 4 packed in w (add_f16_half: no widening).
__device__ __forceinline__ void add4_f16(u32x2 w, float* v) {
  v[0] = add_f16_half<false>(w.x, v[0]);
  v[1] = add_f16_half<true>(w.x, v[1]);
  v[2] = add_f16_half<false>(w.y, v[2]);
  v[3] = add_f16_half<true>(w.y, v[3]);
}

// Final values of 4 consecutive output columns [n, n+4) of row m -> C.
// For SiLU, v holds the gate sums and u the up sums.  pre_old, when given,
// holds the group's residual words, loaded earlier; otherwise they are read
// here.  (The loads stay inside their branches: hoisting them out of the
// `accumulate` / `bias` tests makes the compiler wait for every outstanding
// VMEM operation before each store, the previous groups' stores included,
// since vmcnt counts stores too; the qkv store phase measured 2.0 against
// 1.16 us that way.)
// ACC: v_in comes straight from MFMA accumulators (the register-staged
// kernel), which the v_fma_mix forms of the f16 adds must not read (see
// add_f16_half); those launches take the widening adds.
template <int DT, int EPI, bool ACC = false>
__device__ __forceinline__ void epilogue4(const GemmParams& p, uint16_t* C, int m, int n,
                                          const float* v_in, const float* u_in,
                                          const u32x2* pre_old = nullptr,
                                          const u32x2* pre_bias = nullptr) {
  uint16_t* dst = C + (int64_t)m * p.ldc + n;
  if constexpr (EPI == EPI_SILU && DT == QA_F16) {
    u32x2 w;
    w.x = silu_mul_f16x2(v_in[0], v_in[1], u_in[0], u_in[1]);
    w.y = silu_mul_f16x2(v_in[2], v_in[3], u_in[2], u_in[3]);
    asm volatile("global_store_dwordx2 %0, %1, off sc1" ::"v"(dst), "v"(w) : "memory");
    return;
  }
  float v[4];
  if constexpr (EPI == EPI_SILU) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float g = Fmt<DT>::widen(Fmt<DT>::narrow(v_in[e]));
      const float u = Fmt<DT>::widen(Fmt<DT>::narrow(u_in[e]));
      v[e] = silu_mul(g, u);
    }
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = v_in[e];
    if (p.bias) {
      if (p.bias_rows) {
        const float b = Fmt<DT>::widen(p.bias[m]);
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] += b;
      } else if constexpr (DT == QA_F16 && !ACC) {
        const u32x2 bw = pre_bias ? *pre_bias : *reinterpret_cast<const u32x2*>(p.bias + n);
        add4_f16(bw, v);
      } else {
        float b[4];
        widen4<DT>(pre_bias ? *pre_bias : *reinterpret_cast<const u32x2*>(p.bias + n), b);
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] += b[e];
      }
    }
    if constexpr (EPI == EPI_GELU) {
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = gelu_erf(v[e]);
    }
    if (p.accumulate) {
      if constexpr (DT == QA_F16 && !ACC) {
        add4_f16(pre_old ? *pre_old : *reinterpret_cast<const u32x2*>(dst), v);
      } else {
        float old[4];
        widen4<DT>(pre_old ? *pre_old : *reinterpret_cast<const u32x2*>(dst), old);
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] += old[e];
      }
    }
  }
  store4<DT>(dst, v);
}

// W row for tile row r of n-block tn (SiLU: first half of the tile = gate
// rows, second half = up rows), or -1 past the edge.
template <int BN, int EPI>
__device__ __forceinline__ int w_row(const GemmParams& p, int tn, int r) {
  if constexpr (EPI == EPI_SILU) {
    const int half = p.N >> 1, n0h = tn * (BN / 2);
    const int j = n0h + (r < BN / 2 ? r : r - BN / 2);
    if (j >= half) return -1;
    return r < BN / 2 ? j : half + j;
  } else {
    const int n = tn * BN + r;
    return n < p.N ? n : -1;
  }
}

// gemm_reg_kernel's tail: epilogue (splits == 1) or f32 partials (splits >
// 1) straight from the accumulators.  Lane (fr, fh) of MFMA tile (fm, fn)
// holds token m = .. + fr and columns 8g + 4fh + {0,1,2,3} of the wave's
// 32-column subtile wn FN + fn.  No SiLU.up (QA_TRANSB refuses it).
template <int DT, int BM, int BN, int EPI, int FM, int FN, int WTM>
__device__ __forceinline__ void finish_tile(const GemmParams& p, f32x16 (&acc)[FM][FN], uint16_t* C,
                                            int tm, int tn, int split, int wm, int wn, int fr,
                                            int fh) {
  static_assert(EPI != EPI_SILU, "QA_TRANSB takes no SiLU.up");
  const int m0 = tm * BM;
  if (p.splits > 1) {
    f32x4* ws = reinterpret_cast<f32x4*>(p.ws);
#pragma unroll
    for (int fm = 0; fm < FM; ++fm) {
      const int m = m0 + wm * WTM + fm * 32 + fr;
      if (m >= p.M) continue;
      const int64_t rowbase = ((int64_t)split * p.M + m) * p.N;
#pragma unroll
      for (int fn = 0; fn < FN; ++fn) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int n = tn * BN + (wn * FN + fn) * 32 + 8 * g + 4 * fh;
          if (n >= p.N) continue;
          const f32x4 v = {acc[fm][fn][4 * g], acc[fm][fn][4 * g + 1], acc[fm][fn][4 * g + 2],
                           acc[fm][fn][4 * g + 3]};
          ws[(rowbase + n) >> 2] = v;
        }
      }
    }
    return;
  }
#pragma unroll
  for (int fm = 0; fm < FM; ++fm) {
    const int m = m0 + wm * WTM + fm * 32 + fr;
    if (m >= p.M) continue;
#pragma unroll
    for (int fn = 0; fn < FN; ++fn) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int n = tn * BN + (wn * FN + fn) * 32 + 8 * g + 4 * fh;
        if (n >= p.N) continue;
        const float v[4] = {acc[fm][fn][4 * g], acc[fm][fn][4 * g + 1], acc[fm][fn][4 * g + 2],
                            acc[fm][fn][4 * g + 3]};
        epilogue4<DT, EPI, true>(p, C, m, n, v, nullptr);
      }
    }
  }
}

// KG k-groups of 2 x WGN MMA waves; group g multiplies slices
// {g*4/KG .. (g+1)*4/KG - 1} of each 64-deep stage on a 2 (m) x WGN (n)
// wave layout, so the LDS read traffic per stage does not grow with KG.  The
// groups' partial accumulators are summed through LDS at the end, group 0 +
// group 1 + ..., a fixed order.
//
// The 256 x 256 tile (one group of 2 x 4 waves of 128 x 64, two 64 KB
// stages) halves the L2 -> LDS bytes per FLOP of the 128-wide tiles; its f32
// staging tile (266 KB) exceeds the LDS, so it leaves in two row passes.  On
// the prefill shapes (M ~ 4300) it wins where it also cuts the tile rounds:
// gate|up 72 us against 94-102 us with 128 x 192 (408 tiles = 2 rounds
// against 1088 = 5), and the stem's second conv level (1.25 ms against
// 1.5 ms).  Four 128 x 128 waves (one per SIMD, accumulators in AGPRs) read
// a third less LDS but measured 13-25% slower: four waves cannot issue the
// DMA fast enough.
//
// Who streams L2 -> LDS: a wave sustains only ~12 GB/s of DMA however deep
// its queue, so the CU's fill rate grows with the number of waves issuing it
// (~58 GB/s with 4, ~100 with 8, ~120 with 16), and waves that also issue
// MFMAs and fragment reads issue DMA more slowly still.  With PW = 0 the MMA
// waves issue the DMA themselves; with PW > 0, PW producer waves (after the
// MMA waves) issue all of it and only take part in the barriers and the
// epilogue.
//
// With CV = 1 the A operand is implicit: row m is an output pixel of a 3x3,
// stride-2, pad-1 convolution over a channel-last input [b][H][W][C], and
// k = (kh * 3 + kw) * C + ic, so every 16-byte chunk of the row is 8
// consecutive input channels of one tap (C a multiple of 8): the DMA address
// is computed per chunk, and taps in the zero padding read as zeros through
// the buffer resource's range check (the im2col of src/audio_encoder.rs:
// 204-236, never materialised).
//
// With PL > 1 a ring stage holds PL consecutive 64-deep planes (each laid out
// as a 64-deep stage above) behind ONE barrier: the small tiles, whose MMA
// waves issue only a few MFMAs per 64 k, then meet at a barrier PL times less
// often for the same bytes in flight.
//
// EW is a mask of epilogue words each thread loads before the main loop, in
// unsplit launches that have them: EW_RESIDUAL the residual (`pre` below),
// EW_BIAS the column bias (`bpre`).  Other launches run the EW = 0 build,
// which carries none of that code (the extra registers and branches cost the
// plain qkv launch 0.7 us).
constexpr int EW_RESIDUAL = 1, EW_BIAS = 2;

// Smallest p >= 1 with p * nth a multiple of gpr: the store loop's thread ->
// column-group map repeats every p iterations.
constexpr int group_period(int nth, int gpr) {
  int q = 1;
  while ((q * nth) % gpr) ++q;
  return q;
}

template <int DT, int BM, int BN, int S, int EPI, int KG, int PW, int CV = 0, int WGN = 2,
          int PL = 1, int WGM = 2, int EW = 0>
__global__ void __launch_bounds__(64 * (WGM * WGN * KG + PW)) gemm_dma_kernel(const GemmParams p) {
  // WGM waves along m within a group (WGN along n)
  constexpr int GW = WGM * WGN;              // MMA waves per k group
  constexpr int NMW = GW * KG;               // MMA waves
  constexpr int NTH = 64 * (NMW + PW);       // threads
  constexpr int NW = PW > 0 ? PW : NMW;      // DMA-issuing waves
  constexpr int SPG = 4 * PL / KG;           // 16-deep slices per group per stage
  constexpr int WTM = BM / WGM, WTN = BN / WGN;
  constexpr int FM = WTM / 32, FN = WTN / 32;
  constexpr int AJ = BM / (8 * NW), BJ = BN / (8 * NW);  // DMA instructions per wave per stage
  constexpr int LPS = (AJ + BJ) * PL;
  constexpr int SA = BM * 128, PLANE = (BM + BN) * 128, STAGE = PLANE * PL;
  constexpr int SK = BK * PL;  // k elements per ring stage
  // Epilogue staging: the f32 tile (rows padded by 4 floats) in EP row passes.
  constexpr int LDT = BN + 4;
  constexpr int EP = BM * LDT * 4 <= S * STAGE ? 1 : 2;
  constexpr int SMEM = S * STAGE > BM / EP * LDT * 4 ? S * STAGE : BM / EP * LDT * 4;
  static_assert(KG == 1 || KG == 2 || KG == 4, "k groups");
  static_assert(FM >= 1 && FN >= 1 && AJ >= 1 && BJ >= 1, "tile shape");
  static_assert(BM % (8 * NW) == 0 && BN % (8 * NW) == 0, "DMA row groups");
  static_assert(EPI != EPI_SILU || BN % 64 == 0, "SiLU tiles hold whole gate / up subtiles");
  static_assert(S >= 2 && (S - 1) * LPS < 64, "pipeline depth");
  static_assert(KG == 1 || (KG - 1) * 4 * BM * BN <= SMEM, "reduction buffer");
  static_assert(EP == 1 || (WGM % EP == 0 && KG == 1), "row passes take whole wave rows");
  static_assert(SMEM <= 160 * 1024, "LDS");
  __shared__ __attribute__((aligned(1024))) unsigned char smem[SMEM];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const bool mma_wave = PW == 0 || wave < NMW;
  const bool dma_wave = PW == 0 || wave >= NMW;
  const int dwave = PW == 0 ? wave : (wave >= NMW ? wave - NMW : 0);  // index among DMA waves
  const int kg = mma_wave ? wave / GW : KG, w4 = wave % GW;  // producers: no k group
  const int wm = w4 % WGM, wn = w4 / WGM;
  const int fr = lane & 31, fh = lane >> 5;  // fragment row, k-chunk parity

#ifdef QA_PHASE_STAMPS
  unsigned long long st[5] = {__builtin_amdgcn_s_memrealtime(), 0, 0, 0, 0};
  // prologue points of the first DMA-issuing thread; the empty asm statements
  // make each stamp wait for the value it follows
  __shared__ unsigned long long pro[3];
  const int pro_tid = PW > 0 ? NMW * 64 : 0;
  {
    const int kv = p.K;
    asm volatile("" ::"s"(kv));
    if (tid == pro_tid) {
      pro[0] = __builtin_amdgcn_s_memrealtime();
      pro[2] = 0;
    }
  }
#endif
  int tm, tn, split;
  tile_of(p, (int)blockIdx.x, tm, tn, split);
#ifdef QA_PHASE_STAMPS
  asm volatile("" ::"v"(tm), "v"(tn), "v"(split));
  if (tid == pro_tid) pro[1] = __builtin_amdgcn_s_memrealtime();
#endif
  const int64_t z = blockIdx.y;
  const uint16_t* A = p.a + z * p.bsa;
  const uint16_t* W = p.w + z * p.bsb;
  uint16_t* C = p.c + z * p.bsc;
  const __amdgpu_buffer_rsrc_t rsa =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(A), (short)0, p.a_bytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t rsw =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(W), (short)0, p.w_bytes, 0x00020000);

  const int m0 = tm * BM;
  const int kbeg = split * p.kchunk;
  const int kend = min(p.K, kbeg + p.kchunk);
  const int nk = (kend - kbeg + SK - 1) / SK;

  // The residual words of this thread's epilogue groups (the same thread ->
  // group map as the store loop below), loaded here, before the ring's first
  // DMA: they arrive while the main loop runs.  Read after the loop they
  // added their latency to every launch (the 64 x 64 store phase: 1.1 us
  // with a residual against 0.44 us without).  A producer wave's words are
  // older than its DMA loads, so the loop's vmcnt waits, which count only
  // the DMA behind them, complete them too.  Single-pass epilogues (EP = 1)
  // with up to 12 groups per thread; the bias (one small, cached vector) is
  // still read in the epilogue.
  constexpr int EGPR = BN / 4;
  constexpr int EIT = (BM * EGPR + NTH - 1) / NTH;
  constexpr bool PRE = (EW & EW_RESIDUAL) && EP == 1 && EPI != EPI_SILU && EIT <= 12;
  u32x2 pre[PRE ? EIT : 1];
  if constexpr (PRE) {
#pragma unroll
    for (int it = 0; it < EIT; ++it) {
      const int idx = it * NTH + tid;
      const int m = m0 + idx / EGPR, n = tn * BN + (idx % EGPR) * 4;
      if ((BM * EGPR % NTH == 0 || idx < BM * EGPR) && m < p.M && n < p.N)
        pre[it] = *reinterpret_cast<const u32x2*>(C + (int64_t)m * p.ldc + n);
    }
  }
  // The column bias of the same groups, also loaded here.  A thread's groups
  // repeat their columns every BPER store iterations (one to three words
  // for these tiles).  Read in the epilogue, each group's bias word came after
  // the previous groups' stores, and since vmcnt counts stores too, waiting
  // for it waited for those stores to be acknowledged: one write-through
  // round trip per group (the tower's 256 x 256 GELU launch: 15 us of stores
  // with a bias).
  constexpr bool BPRE = (EW & EW_BIAS) && EPI != EPI_SILU;
  constexpr int BPER = BPRE ? group_period(NTH, EGPR) : 1;
  u32x2 bpre[BPER];
  if constexpr (BPRE) {
#pragma unroll
    for (int j = 0; j < BPER; ++j) {
      const int n = tn * BN + ((j * NTH + tid) % EGPR) * 4;
      if (n < p.N) bpre[j] = *reinterpret_cast<const u32x2*>(p.bias + n);
    }
  }

  // Per-lane byte offsets at k = 0 of the row chunk this lane fetches: lane l
  // of DMA instruction j fills LDS row r = (NW*j + dwave)*8 + l/8 at physical
  // chunk l%8, so it fetches logical chunk (l%8) ^ swz(r).
  const int lrow = lane >> 3, pchunk = lane & 7;
  uint32_t aoff[AJ], woff[BJ];
  int akc[AJ], wkc[BJ];  // k offset (elements) of the fetched chunk
  int cpix[AJ], cih[AJ], ciw[AJ];  // CV: image's first pixel, input row / column of tap (0, 0)
  int cg[AJ], cic[AJ];             // CV: tap and channel of the lane's chunk in the next plane issued
#pragma unroll
  for (int j = 0; j < AJ; ++j) {
    const int r = (j * NW + dwave) * 8 + lrow;
    const int m = m0 + r;
    akc[j] = (pchunk ^ swz(r)) * 8;
    aoff[j] = m < p.M ? (uint32_t)(((int64_t)m * p.lda + akc[j]) * 2) : OOB;
    if constexpr (CV) {
      const int plane = p.cv_ho * p.cv_wo, b = m / plane, q = m - b * plane;
      const int ho = p.cv_tmajor ? q % p.cv_ho : q / p.cv_wo;
      const int wo = p.cv_tmajor ? q / p.cv_ho : q % p.cv_wo;
      cpix[j] = b * p.cv_h * p.cv_w;
      cih[j] = m < p.M ? 2 * ho - 1 : INT32_MIN / 2;  // rows >= M never in range
      ciw[j] = 2 * wo - 1;
      cg[j] = (kbeg + akc[j]) / p.cv_c;
      cic[j] = kbeg + akc[j] - cg[j] * p.cv_c;
    }
  }
#pragma unroll
  for (int j = 0; j < BJ; ++j) {
    const int r = (j * NW + dwave) * 8 + lrow;
    const int n = w_row<BN, EPI>(p, tn, r);
    wkc[j] = (pchunk ^ swz(r)) * 8;
    woff[j] = n >= 0 ? (uint32_t)(((int64_t)n * p.ldb + wkc[j]) * 2) : OOB;
  }

  // The DMA's LDS destination goes in M0, which must be wave-uniform: with
  // the wave index in a scalar register it is scalar arithmetic, instead of a
  // v_readfirstlane (and its hazard wait) per instruction.
  const int dwave_s = wave_uniform(dwave);
  // One ring stage's DMA, each chunk checked against the k range (rows past
  // M / N carry OOB, which the buffer unit answers with zeros).
  auto issue_checked = [&](int kidx, int buf) {
#pragma unroll
    for (int pl = 0; pl < PL; ++pl) {
      const int k0 = kbeg + kidx * SK + pl * BK;
      unsigned char* sb = smem + buf * STAGE + pl * PLANE;
#pragma unroll
      for (int j = 0; j < AJ; ++j) {
        uint32_t off;
        if constexpr (CV) {
          const int k = k0 + akc[j];
          const int g = cg[j], ic = cic[j];  // tap g = 3 kh + kw
          cic[j] += BK;  // the next plane: 64 channels on (c >= 64: at most one wrap)
          if (cic[j] >= p.cv_c) {
            cic[j] -= p.cv_c;
            ++cg[j];
          }
          const int kh = (g * 11) >> 5, kw = g - 3 * kh;   // g / 3 for g < 9
          const int ih = cih[j] + kh, iw = ciw[j] + kw;
          const bool ok =
              k < kend && (unsigned)ih < (unsigned)p.cv_h && (unsigned)iw < (unsigned)p.cv_w;
          off = ok ? (uint32_t)(((cpix[j] + ih * p.cv_w + iw) * p.cv_c + ic) * 2) : OOB;
        } else {
          const bool ok = k0 + akc[j] < kend && aoff[j] != OOB;
          off = ok ? aoff[j] + (uint32_t)k0 * 2u : OOB;
        }
        dma16(rsa, sb + (j * NW + dwave_s) * 1024, off);
      }
#pragma unroll
      for (int j = 0; j < BJ; ++j) {
        const bool ok = k0 + wkc[j] < kend && woff[j] != OOB;
        const uint32_t off = ok ? woff[j] + (uint32_t)k0 * 2u : OOB;
        dma16(rsw, sb + SA + (j * NW + dwave_s) * 1024, off);
      }
    }
  };
  // A stage inside the k range needs no per-chunk check: OOB (rows past
  // M / N) plus 2 k0 still lies past every buffer's range, so each
  // instruction is one add.  The last stage of a ragged k range, and the
  // convolution's gathered A, take the checked form.
  auto issue = [&](int kidx, int buf) {
    if (!CV && kbeg + (kidx + 1) * SK <= kend) {
#pragma unroll
      for (int pl = 0; pl < PL; ++pl) {
        const uint32_t k2 = (uint32_t)(kbeg + kidx * SK + pl * BK) * 2u;
        unsigned char* sb = smem + buf * STAGE + pl * PLANE;
#pragma unroll
        for (int j = 0; j < AJ; ++j)
          dma16(rsa, sb + (j * NW + dwave_s) * 1024, aoff[j] + k2);
#pragma unroll
        for (int j = 0; j < BJ; ++j)
          dma16(rsw, sb + SA + (j * NW + dwave_s) * 1024, woff[j] + k2);
      }
    } else {
      issue_checked(kidx, buf);
    }
  };

  f32x16 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = f32x16{0};

  // Fragments of one 16-deep k slice, double-buffered in registers.
  u32x4 fa[2][FN], fb[2][FM];
  auto read_frags = [&](int buf, int kk, int slot) {
    const unsigned char* sA = smem + buf * STAGE + (kk >> 2) * PLANE;  // plane kk / 4
    const unsigned char* sB = sA + SA;
    const int c = (kk & 3) * 2 + fh;
#pragma unroll
    for (int fn = 0; fn < FN; ++fn) {
      const int row = (wn * FN + fn) * 32 + fr;
      fa[slot][fn] = *reinterpret_cast<const u32x4*>(sB + row * 128 + ((c ^ swz(row)) << 4));
    }
#pragma unroll
    for (int fm = 0; fm < FM; ++fm) {
      const int row = wm * WTM + fm * 32 + fr;
      fb[slot][fm] = *reinterpret_cast<const u32x4*>(sA + row * 128 + ((c ^ swz(row)) << 4));
    }
  };
  auto mma = [&](int slot) {
#pragma unroll
    for (int fm = 0; fm < FM; ++fm)
#pragma unroll
      for (int fn = 0; fn < FN; ++fn)
        acc[fm][fn] = Fmt<DT>::mfma(fa[slot][fn], fb[slot][fm], acc[fm][fn]);
  };

  // Pipeline: all S buffers are filled up front; the fragments of the next
  // slice are read while the current one multiplies.  The barrier that
  // publishes stage it+1 (and frees stage it's buffer for stage it+S) sits
  // before the stage's last slice is multiplied: each wave first waits for
  // its own reads of the stage (all of them issued by then), and after the
  // barrier the first fragments of stage it+1 load while the last slice's
  // MFMAs run, so no wave stalls on LDS right after the barrier.
  //
  // With producer waves the roles split but the barrier sequence is the same
  // (one before stage 0, one per later stage): a producer waits for its own
  // DMA of stage it+1, meets the MMA waves at the barrier (after which stage
  // it's buffer is free: every MMA wave waited for its reads of it), and
  // refills that buffer with stage it+S at once.
  static_assert(SPG % 2 == 0, "fragment slots alternate within a stage");
  const int kk0 = kg * SPG;

  // Prefetch of the next kernel's operand (p.pf, a caller hint): each MMA
  // wave loads one dword of PFI x 64 distinct 128-byte lines, so the lines
  // travel HBM -> memory-side cache while this kernel computes, and the next
  // kernel's first stages find them there instead of in HBM.  The loads are
  // ordinary ones: with the nontemporal hint the next kernel measured no
  // faster than with no prefetch at all.  The loaded values are only kept
  // alive until the end of the kernel.  Where the MMA waves also issue the DMA (PW = 0), the
  // loads sit in the same in-order vmcnt stream right after stage S-1: the
  // waits for stages 1 .. S-1 leave them outstanding (+PFI), and the kernel
  // prefetches only when every ring stage is issued up front (nk >= S).
  constexpr int PFI = 2;
  static_assert((S - 1) * LPS + PFI < 64, "vmcnt with the prefetch loads");
  const bool pf_on = p.pf_bytes > 0 && z == 0 && mma_wave && (PW > 0 || nk >= S);
  uint32_t pfv[PFI] = {};
  auto prefetch = [&]() {
    const __amdgpu_buffer_rsrc_t rsp = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(p.pf), (short)0, p.pf_bytes, 0x00020000);
#pragma unroll
    for (int i = 0; i < PFI; ++i) {
      const uint64_t line = (uint64_t)((i * NMW + wave) * 64 + lane) * gridDim.x + blockIdx.x;
      const uint32_t off = line * 128 < (uint64_t)p.pf_bytes ? (uint32_t)(line * 128) : OOB;
      pfv[i] = __builtin_amdgcn_raw_buffer_load_b32(rsp, off, 0, 0);
    }
  };
  if (nk > 0 && !mma_wave) {
#pragma unroll
    for (int s = 0; s < S; ++s)
      if (s < nk) issue(s, s);
#ifdef QA_PHASE_STAMPS
    if (tid == pro_tid) pro[2] = __builtin_amdgcn_s_memrealtime();
#endif
    if (S - 1 < nk)
      wait_vmcnt<(S - 1) * LPS>();
    else
      wait_vmcnt<0>();
    exec_barrier();
    for (int it = 0; it + 1 < nk; ++it) {
      if (it + S - 1 < nk)
        wait_vmcnt<(S - 2) * LPS>();
      else
        wait_vmcnt<0>();
      exec_barrier();
      if (it + S < nk) issue(it + S, it % S);
    }
  } else if (nk > 0) {
    // The MMA waves; they also issue the DMA only without producer waves.
    // Known at compile time for one k group: the conv loader's per-chunk
    // state then stays out of the MMA waves' registers (256 x 160: 256 VGPRs
    // and a 100-byte spill before, 231 after).  The two-group 64-row tiles
    // keep the run-time test: their o / down launches measured 9% slower
    // with the compile-time one (same box, 11.8 -> 12.9 us).
    const bool dma_here = KG == 1 ? PW == 0 : dma_wave;
    if (dma_here) {
#pragma unroll
      for (int s = 0; s < S; ++s)
        if (s < nk) issue(s, s);
#ifdef QA_PHASE_STAMPS
      if (tid == pro_tid) pro[2] = __builtin_amdgcn_s_memrealtime();
#endif
      if (S - 1 < nk)
        wait_vmcnt<(S - 1) * LPS>();
      else
        wait_vmcnt<0>();
    }
    exec_barrier();
#ifdef QA_PHASE_STAMPS
    st[1] = __builtin_amdgcn_s_memrealtime();
#endif
    if (pf_on) prefetch();
    read_frags(0, kk0, 0);
    for (int it = 0; it < nk; ++it) {
      const int buf = it % S;
#pragma unroll
      for (int q = 0; q + 1 < SPG; ++q) {
        read_frags(buf, kk0 + q + 1, (q + 1) & 1);
        mma(q & 1);
      }
      wait_lds();  // unconditional: both paths reach the last MFMAs with ready slots
      if (it + 1 < nk) {
        if (dma_here) {
          if (it + S - 1 < nk) {
            if (PW == 0 && pf_on && it < S - 1)
              wait_vmcnt<(S - 2) * LPS + PFI>();
            else
              wait_vmcnt<(S - 2) * LPS>();
          } else {
            wait_vmcnt<0>();
          }
        }
        exec_barrier();
        read_frags((it + 1) % S, kk0, 0);
      }
      mma((SPG - 1) & 1);
      // Refill the freed buffer behind this wave's LDS reads and MFMAs (issued
      // ahead of them, the DMA writes measurably delay the fragment reads).
      if (dma_here && it + 1 < nk && it + S < nk) {
        __builtin_amdgcn_sched_barrier(0);
        issue(it + S, buf);
      }
    }
  }

  // Epilogue through LDS.  The accumulators (in MFMA lane order: one token,
  // 4-column runs) are parked as an f32 [BM][BN] tile, the k-groups summed
  // into it in group order, and the tile leaves row by row: consecutive
  // threads take consecutive 4-column groups, so bias / residual reads and
  // the 16-bit stores are contiguous row segments.  Rows are padded by 4
  // floats, which puts the 16 rows a quarter-wave writes on distinct banks.
  // With EP = 2 (a tile larger than the LDS) the rows leave in two passes,
  // the m half of the waves with wm = 0, then that of wm = 1.
  constexpr int PR = BM / EP;  // tile rows per pass
  float* tile = reinterpret_cast<float*>(smem);
  constexpr int OUTC = EPI == EPI_SILU ? BN / 2 : BN;  // output columns of the tile
  constexpr int GPR = OUTC / 4;                          // 4-column groups per row
  const int nfull = EPI == EPI_SILU ? p.N / 2 : p.N;
  const int n0 = tn * OUTC;
  // The column bias in LDS for the 16-bit park below (the MMA lanes' column
  // order): the words thread t < BN / 4 preloaded for its store groups.
  constexpr bool PK16 = KG == 1 && ((EPI == EPI_SILU && DT == QA_F16) || EPI == EPI_PLAIN ||
                                    EPI == EPI_GELU);
  __shared__ u32x2 sbias[PK16 && BPRE ? EGPR : 1];
  if constexpr (PK16 && BPRE) {
    if (tid < EGPR) sbias[tid] = tn * BN + tid * 4 < p.N ? bpre[0] : u32x2{0, 0};
  }
  __syncthreads();  // all stages consumed (every DMA was waited for)
#ifdef QA_PHASE_STAMPS
  st[2] = __builtin_amdgcn_s_memrealtime();
#endif
  // 16-bit park (unsplit launches with one k group and no residual): the MMA
  // waves finish each output in registers and park it rounded, as a 16-bit
  // [BM][BN + 4] tile: half the LDS bytes of the f32 tile, in one pass where
  // the f32 tile of a 256-row tile needs two.  Plain and GELU outputs get
  // their bias (from sbias) and GELU in the MMA lanes, in f32, then the one
  // rounding; the store loop only copies rows out.  f16 SiLU.up parks g and u
  // rounded (the epilogue's first step) and the store loop reads the packed
  // pairs straight into silu_mul_h2.  Same bits as the f32 path below, which
  // split launches (f32 partials), residual adds and channel-major bias take.
  bool parked16 = false;
  if constexpr (PK16) {
    if (p.splits == 1 &&
        (EPI == EPI_SILU || (!p.accumulate && !p.bias_rows && (BPRE || !p.bias)))) {
      parked16 = true;
      constexpr int LDH = BN + 4;  // 16-bit values per parked row
      static_assert(BM * LDH * 2 <= SMEM, "16-bit park fits the LDS");
      uint16_t* ht = reinterpret_cast<uint16_t*>(smem);
      typedef _Float16 h2 __attribute__((ext_vector_type(2)));
      if (mma_wave) {
#pragma unroll
        for (int fm = 0; fm < FM; ++fm)
#pragma unroll
          for (int fn = 0; fn < FN; ++fn)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              const int row = wm * WTM + fm * 32 + fr;
              const int col = (wn * FN + fn) * 32 + 8 * q + 4 * fh;
              float x[4];
#pragma unroll
              for (int e = 0; e < 4; ++e) x[e] = acc[fm][fn][4 * q + e];
              if constexpr (EPI != EPI_SILU) {
                if constexpr (BPRE) {
                  float b[4];
                  widen4<DT>(sbias[col >> 2], b);
#pragma unroll
                  for (int e = 0; e < 4; ++e) x[e] += b[e];
                }
                if constexpr (EPI == EPI_GELU) {
#pragma unroll
                  for (int e = 0; e < 4; ++e) x[e] = gelu_erf(x[e]);
                }
              }
              u32x2 w;
              if constexpr (DT == QA_F16) {
                w.x = __builtin_bit_cast(uint32_t, h2{(_Float16)x[0], (_Float16)x[1]});
                w.y = __builtin_bit_cast(uint32_t, h2{(_Float16)x[2], (_Float16)x[3]});
              } else {
                w.x = Fmt<DT>::narrow(x[0]) | (Fmt<DT>::narrow(x[1]) << 16);
                w.y = Fmt<DT>::narrow(x[2]) | (Fmt<DT>::narrow(x[3]) << 16);
              }
              *reinterpret_cast<u32x2*>(ht + row * LDH + col) = w;
            }
      }
      __syncthreads();
#ifdef QA_PHASE_STAMPS
      st[3] = __builtin_amdgcn_s_memrealtime();
#endif
#pragma unroll
      for (int it = 0; it < (BM * GPR + NTH - 1) / NTH; ++it) {
        const int idx = it * NTH + tid;
        if (BM * GPR % NTH != 0 && idx >= BM * GPR) break;
        const int r = idx / GPR, c4 = (idx % GPR) * 4;
        const int m = m0 + r, n = n0 + c4;
        if (m >= p.M || n >= nfull) continue;
        u32x2 w = *reinterpret_cast<const u32x2*>(ht + r * LDH + c4);
        if constexpr (EPI == EPI_SILU) {
          const u32x2 u = *reinterpret_cast<const u32x2*>(ht + r * LDH + BN / 2 + c4);
          w = u32x2{silu_mul_h2(w.x, u.x), silu_mul_h2(w.y, u.y)};
        }
        asm volatile("global_store_dwordx2 %0, %1, off sc1" ::"v"(C + (int64_t)m * p.ldc + n),
                     "v"(w)
                     : "memory");
      }
    }
  }
#pragma unroll
  for (int e = 0; e < (parked16 ? 0 : EP); ++e) {
    if (e > 0) __syncthreads();  // the previous pass's rows have been read
#pragma unroll
    for (int g = 0; g < KG; ++g) {
      if (kg == g && (EP == 1 || wm / (WGM / EP) == e)) {
        auto at = [&](int fm, int fn, int q) {
          const int row = wm * WTM + fm * 32 + fr - e * PR;
          const int col = (wn * FN + fn) * 32 + 8 * q + 4 * fh;
          return reinterpret_cast<f32x4*>(tile + row * LDT + col);
        };
        // Group g > 0 adds its sums to what the groups before it left: every
        // read is issued before the first add, so the LDS round trips overlap
        // instead of running one after another.
        f32x4 prev[FM][FN][4];
        if (g > 0) {
#pragma unroll
          for (int fm = 0; fm < FM; ++fm)
#pragma unroll
            for (int fn = 0; fn < FN; ++fn)
#pragma unroll
              for (int q = 0; q < 4; ++q) prev[fm][fn][q] = *at(fm, fn, q);
        }
#pragma unroll
        for (int fm = 0; fm < FM; ++fm)
#pragma unroll
          for (int fn = 0; fn < FN; ++fn)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              const f32x4 v = {acc[fm][fn][4 * q], acc[fm][fn][4 * q + 1], acc[fm][fn][4 * q + 2],
                               acc[fm][fn][4 * q + 3]};
              *at(fm, fn, q) = g > 0 ? prev[fm][fn][q] + v : v;
            }
      }
      __syncthreads();
    }
#ifdef QA_PHASE_STAMPS
    if (e == 0) st[3] = __builtin_amdgcn_s_memrealtime();
#endif
#pragma unroll
    for (int it = 0; it < (PR * GPR + NTH - 1) / NTH; ++it) {
      const int idx = it * NTH + tid;
      if (PR * GPR % NTH != 0 && idx >= PR * GPR) break;
      const int r = idx / GPR, c4 = (idx % GPR) * 4;
      const int m = m0 + e * PR + r, n = n0 + c4;
      if (m >= p.M || n >= nfull) continue;
      const f32x4 v4 = *reinterpret_cast<const f32x4*>(tile + r * LDT + c4);
      f32x4 u4 = {0.f, 0.f, 0.f, 0.f};
      if constexpr (EPI == EPI_SILU)
        u4 = *reinterpret_cast<const f32x4*>(tile + r * LDT + BN / 2 + c4);
      if (p.splits > 1) {
        f32x4* ws = reinterpret_cast<f32x4*>(p.ws);
        const int64_t rowbase = ((int64_t)split * p.M + m) * p.N;
        ws[(rowbase + n) >> 2] = v4;
        if constexpr (EPI == EPI_SILU) ws[(rowbase + nfull + n) >> 2] = u4;
        continue;
      }
      const float v[4] = {v4.x, v4.y, v4.z, v4.w};
      const float uu[4] = {u4.x, u4.y, u4.z, u4.w};
      const u32x2* bw = nullptr;
      if constexpr (BPRE) bw = &bpre[it % BPER];
      if constexpr (PRE)
        epilogue4<DT, EPI>(p, C, m, n, v, uu, &pre[it], bw);
      else
        epilogue4<DT, EPI>(p, C, m, n, v, uu, nullptr, bw);
    }
  }
  if (pf_on) {
#pragma unroll
    for (int i = 0; i < PFI; ++i) asm volatile("" ::"v"(pfv[i]));
  }
#ifdef QA_PHASE_STAMPS
  __syncthreads();  // every wave's stores issued
  const unsigned b = blockIdx.x + blockIdx.y * gridDim.x;
  if (tid == 0 && b < (unsigned)kStampBlocks) {
    st[4] = __builtin_amdgcn_s_memrealtime();
    unsigned long long* d = stamp_log + ((size_t)p.stamp_slot * kStampBlocks + b) * kStampWords;
    for (int i = 0; i < 5; ++i) d[i] = st[i];
    d[5] = (unsigned long long)__smid();
    d[6] = (unsigned long long)p.N;
    d[7] = (unsigned long long)p.K;
    for (int i = 0; i < 3; ++i) d[8 + i] = pro[i];
  }
#endif
}

// W as [K, N] (row stride ldb): register-staged, double-buffered; each
// 16-byte load (8 consecutive n of one k row) is scattered into the
// K-contiguous LDS layout the MFMA fragments read.
template <int DT, int EPI>
__global__ void __launch_bounds__(NT) gemm_reg_kernel(const GemmParams p) {
  constexpr int BM = 128, BN = 128;
  constexpr int WGM = 2;
  constexpr int WTM = 64;
  constexpr int FM = 2, FN = 2;
  constexpr int AP = BM * 8 / NT, BP = BN * 8 / NT;
  constexpr int SA = BM * 128, SB = BN * 128;
  __shared__ __attribute__((aligned(16))) unsigned char smem[2 * (SA + SB)];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm = wave % WGM, wn = wave / WGM;
  const int fr = lane & 31, fh = lane >> 5;

  int tm, tn, split;
  tile_of(p, (int)blockIdx.x, tm, tn, split);
  const int64_t z = blockIdx.y;
  const uint16_t* __restrict__ A = p.a + z * p.bsa;
  const uint16_t* __restrict__ W = p.w + z * p.bsb;
  uint16_t* C = p.c + z * p.bsc;

  const int m0 = tm * BM;
  const int kbeg = split * p.kchunk;
  const int kend = min(p.K, kbeg + p.kchunk);
  const int nk = (kend - kbeg + BK - 1) / BK;

  const int ch = tid & 7, rsub = tid >> 3;
  const uint16_t* aptr[AP];
  bool arow_ok[AP];
#pragma unroll
  for (int i = 0; i < AP; ++i) {
    const int r = m0 + i * 32 + rsub;
    arow_ok[i] = r < p.M;
    aptr[i] = A + (int64_t)min(r, p.M - 1) * p.lda + ch * 8;
  }

  u32x4 ra[AP], rb[BP];
  auto load_stage = [&](int k0) {
    const bool kin = k0 + ch * 8 < kend;
#pragma unroll
    for (int i = 0; i < AP; ++i)
      ra[i] = (kin && arow_ok[i]) ? *reinterpret_cast<const u32x4*>(aptr[i] + k0)
                                  : u32x4{0, 0, 0, 0};
#pragma unroll
    for (int i = 0; i < BP; ++i) {
      const int q = i * NT + tid;
      const int krow = q / (BN / 8), nc = q % (BN / 8);
      const int gk = k0 + krow, gn = tn * BN + nc * 8;
      rb[i] = (gk < kend && gn < p.N)
                  ? *reinterpret_cast<const u32x4*>(W + (int64_t)gk * p.ldb + gn)
                  : u32x4{0, 0, 0, 0};
    }
  };
  auto store_stage = [&](int stage) {
    unsigned char* sA = smem + stage * (SA + SB);
    unsigned char* sB = sA + SA;
#pragma unroll
    for (int i = 0; i < AP; ++i) {
      const int row = i * 32 + rsub;
      *reinterpret_cast<u32x4*>(sA + row * 128 + ((ch ^ swz(row)) << 4)) = ra[i];
    }
#pragma unroll
    for (int i = 0; i < BP; ++i) {
      const int q = i * NT + tid;
      const int krow = q / (BN / 8), nc = q % (BN / 8);
      const uint32_t w4[4] = {rb[i].x, rb[i].y, rb[i].z, rb[i].w};
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int row = nc * 8 + e;
        const uint16_t v = (uint16_t)(w4[e >> 1] >> ((e & 1) * 16));
        *reinterpret_cast<uint16_t*>(sB + row * 128 + (((krow >> 3) ^ swz(row)) << 4) +
                                     (krow & 7) * 2) = v;
      }
    }
  };

  f32x16 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = f32x16{0};

  auto compute_stage = [&](int stage) {
    const unsigned char* sA = smem + stage * (SA + SB);
    const unsigned char* sB = sA + SA;
#pragma unroll
    for (int kk = 0; kk < BK / 16; ++kk) {
      const int c = kk * 2 + fh;
      u32x4 fa[FN], fb[FM];
#pragma unroll
      for (int fn = 0; fn < FN; ++fn) {
        const int row = (wn * FN + fn) * 32 + fr;
        fa[fn] = *reinterpret_cast<const u32x4*>(sB + row * 128 + ((c ^ swz(row)) << 4));
      }
#pragma unroll
      for (int fm = 0; fm < FM; ++fm) {
        const int row = wm * WTM + fm * 32 + fr;
        fb[fm] = *reinterpret_cast<const u32x4*>(sA + row * 128 + ((c ^ swz(row)) << 4));
      }
#pragma unroll
      for (int fm = 0; fm < FM; ++fm)
#pragma unroll
        for (int fn = 0; fn < FN; ++fn) acc[fm][fn] = Fmt<DT>::mfma(fa[fn], fb[fm], acc[fm][fn]);
    }
  };

  if (nk > 0) {
    load_stage(kbeg);
    store_stage(0);
    __syncthreads();
    for (int it = 0; it < nk; ++it) {
      const bool more = it + 1 < nk;
      if (more) load_stage(kbeg + (it + 1) * BK);
      compute_stage(it & 1);
      if (more) store_stage((it + 1) & 1);
      __syncthreads();
    }
  }
  finish_tile<DT, BM, BN, EPI, FM, FN, WTM>(p, acc, C, tm, tn, split, wm, wn, fr, fh);
}

// Sum the split-K partials [splits][M][N] (f32) in split order and run the
// epilogue: one thread per 4 output columns of one row.
template <int DT, int EPI>
__global__ void __launch_bounds__(256) splitk_reduce_kernel(const GemmParams p) {
  const int nout = EPI == EPI_SILU ? p.N / 2 : p.N;
  const int groups = nout / 4;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (int64_t)p.M * groups) return;
  const int m = (int)(idx / groups), n = (int)(idx % groups) * 4;
  const f32x4* ws = reinterpret_cast<const f32x4*>(p.ws);
  f32x4 s = {0.f, 0.f, 0.f, 0.f}, su = {0.f, 0.f, 0.f, 0.f};
  for (int sp = 0; sp < p.splits; ++sp) {
    const int64_t row = ((int64_t)sp * p.M + m) * p.N;
    s += ws[(row + n) >> 2];
    if constexpr (EPI == EPI_SILU) su += ws[(row + nout + n) >> 2];
  }
  const float v[4] = {s.x, s.y, s.z, s.w};
  const float uu[4] = {su.x, su.y, su.z, su.w};
  epilogue4<DT, EPI>(p, p.c, m, n, v, uu);
}

// Launch timing events (launch_gemm's t0 / t1), null for none.
struct Stamps {
  hipEvent_t t0, t1;
};

template <class K>
hipError_t launch_kernel(K k, dim3 grid, dim3 block, hipStream_t s, const Stamps& ts,
                         const GemmParams& p) {
  if (ts.t0 || ts.t1)
    hipExtLaunchKernelGGL(k, grid, block, 0, s, ts.t0, ts.t1, 0, p);
  else
    hipLaunchKernelGGL(k, grid, block, 0, s, p);
  return hipGetLastError();
}

template <int DT, int BM, int BN, int S, int EPI, int KG, int PW, int CV = 0, int WGN = 2,
          int PL = 1, int WGM = 2>
hipError_t launch_dma(const Plan& plan, const GemmParams& p, int batch, hipStream_t s,
                      const Stamps& ts) {
  const unsigned units = (unsigned)(plan.tiles_m * plan.tiles_n * plan.splits);
  const dim3 grid(units, (unsigned)batch), block(64 * (WGM * WGN * KG + PW));
  // The preloading builds only where their words exist (unsplit launches: a
  // split launch's epilogue runs in the reduce kernel): the residual where
  // the kernel can hold it, the column bias on every non-SiLU tile.
  constexpr int EP = BM * (BN + 4) * 4 <= S * (BM + BN) * 128 * PL ? 1 : 2;
  constexpr int NTH = 64 * (WGM * WGN * KG + PW);
  constexpr bool RES_OK =
      CV == 0 && EPI == EPI_PLAIN && EP == 1 && (BM * BN / 4 + NTH - 1) / NTH <= 12;
  const bool res = RES_OK && plan.splits == 1 && p.accumulate;
  const bool bw = EPI != EPI_SILU && plan.splits == 1 && p.bias && !p.bias_rows;
  if constexpr (EPI != EPI_SILU) {
    if constexpr (RES_OK) {
      if (res && bw)
        return launch_kernel(
            gemm_dma_kernel<DT, BM, BN, S, EPI, KG, PW, CV, WGN, PL, WGM, EW_RESIDUAL | EW_BIAS>,
            grid, block, s, ts, p);
      if (res)
        return launch_kernel(
            gemm_dma_kernel<DT, BM, BN, S, EPI, KG, PW, CV, WGN, PL, WGM, EW_RESIDUAL>, grid,
            block, s, ts, p);
    }
    if (bw)
      return launch_kernel(gemm_dma_kernel<DT, BM, BN, S, EPI, KG, PW, CV, WGN, PL, WGM, EW_BIAS>,
                           grid, block, s, ts, p);
  }
  return launch_kernel(gemm_dma_kernel<DT, BM, BN, S, EPI, KG, PW, CV, WGN, PL, WGM, 0>, grid,
                       block, s, ts, p);
}

template <int DT, int EPI>
hipError_t launch_reg(const Plan& plan, const GemmParams& p, int batch, hipStream_t s,
                      const Stamps& ts) {
  const unsigned units = (unsigned)(plan.tiles_m * plan.tiles_n * plan.splits);
  return launch_kernel(gemm_reg_kernel<DT, EPI>, dim3(units, (unsigned)batch), dim3(NT), s, ts, p);
}

template <int DT, int EPI>
hipError_t launch_reduce(const GemmParams& p, hipStream_t s, const Stamps& ts) {
  const int nout = EPI == EPI_SILU ? p.N / 2 : p.N;
  const int64_t threads = (int64_t)p.M * (nout / 4);
  return launch_kernel(splitk_reduce_kernel<DT, EPI>, dim3((unsigned)((threads + 255) / 256)),
                       dim3(256), s, ts, p);
}

template <int DT, int EPI>
hipError_t launch_epi(const Plan& plan, const GemmParams& p, int batch, hipStream_t s,
                      const Stamps& ts_in) {
  // split K: the GEMM's dispatch stamps the start, the reduce's the end
  const Stamps ts = plan.splits > 1 ? Stamps{ts_in.t0, nullptr} : ts_in;
  hipError_t e;
  if (plan.conv) {  // implicit-GEMM convolution (qa_conv2d_3x3s2)
    if constexpr (EPI == EPI_SILU) return hipErrorInvalidValue;  // never planned
    else if (plan.tile == TILE_256x128)
      e = launch_dma<DT, 256, 128, 3, EPI, 1, 4, 1>(plan, p, batch, s, ts);
    else if (plan.tile == TILE_128x256)
      e = launch_dma<DT, 128, 256, 3, EPI, 1, 4, 1>(plan, p, batch, s, ts);
    else if (plan.tile == TILE_256x256)
      e = launch_dma<DT, 256, 256, 2, EPI, 1, 0, 1, 4>(plan, p, batch, s, ts);
    else if (plan.tile == TILE_256x160)  // 4 x 1 waves of 64 x 160: N = 480 in three tiles
      e = launch_dma<DT, 256, 160, 3, EPI, 1, 4, 1, 1, 1, 4>(plan, p, batch, s, ts);
    else
      e = launch_dma<DT, 128, 128, 3, EPI, 1, 8, 1>(plan, p, batch, s, ts);
  } else if (plan.transb) {
    if constexpr (EPI == EPI_SILU) return hipErrorInvalidValue;  // rejected by validation
    else e = launch_reg<DT, EPI>(plan, p, batch, s, ts);
  } else {
    switch (plan.tile) {
      // (one k group of MMA waves plus 4 producer waves: 2-10% faster than two
      // k groups that issue their own DMA, on the prefill and tower shapes)
      case TILE_256x128: e = launch_dma<DT, 256, 128, 3, EPI, 1, 4>(plan, p, batch, s, ts); break;
      case TILE_128x256: e = launch_dma<DT, 128, 256, 3, EPI, 1, 4>(plan, p, batch, s, ts); break;
      case TILE_64x128: e = launch_dma<DT, 64, 128, 4, EPI, 2, 8>(plan, p, batch, s, ts); break;
      // 64x64: waves of 32 (m) x 64 (n) and an 8-deep ring (less LDS read per
      // FLOP than 32 x 32 waves with 6 stages): 7-8% faster at M = N = 1024 on
      // repeated launches over L2-resident operands, ~1% in the decoder-layer
      // sequence, where each launch starts on cold weights.
      case TILE_64x64: e = launch_dma<DT, 64, 64, 8, EPI, 2, 8, 0, 1>(plan, p, batch, s, ts); break;
      case TILE_64x64_P2:
        e = launch_dma<DT, 64, 64, 4, EPI, 2, 8, 0, 1, 2>(plan, p, batch, s, ts);
        break;
      // 128x192 and 128x128: one k group of 2 x 2 MMA waves that run the
      // whole 64-deep stage, plus producer waves that only issue the DMA.
      // Against two k groups of MMA waves that also issue the DMA (PW = 0)
      // or share it with producers, the stage's L2 -> LDS stream is faster
      // and the epilogue has no k-group sum: config 3 -3 / -1.3%, the
      // 4352-token prefill -3%, the 300 s forward -2% (same box).
      case TILE_128x192: e = launch_dma<DT, 128, 192, 3, EPI, 1, 4>(plan, p, batch, s, ts); break;
      case TILE_256x256: e = launch_dma<DT, 256, 256, 2, EPI, 1, 0, 0, 4>(plan, p, batch, s, ts); break;
      // 256 x 192: one round where 128 x 192 needs two (the tower's qkv at M = 3900)
      case TILE_256x192:
        e = launch_dma<DT, 256, 192, 2, EPI, 1, 0, 0, 2, 1, 4>(plan, p, batch, s, ts);
        break;
      default: e = launch_dma<DT, 128, 128, 3, EPI, 1, 8>(plan, p, batch, s, ts); break;
    }
  }
  if (e != hipSuccess || plan.splits == 1) return e;
  return launch_reduce<DT, EPI>(p, s, Stamps{nullptr, ts_in.t1});
}

template <int DT>
hipError_t launch_dt(const Plan& plan, const GemmParams& p, int batch, hipStream_t s,
                     const Stamps& ts) {
  switch (plan.epi) {
    case EPI_GELU: return launch_epi<DT, EPI_GELU>(plan, p, batch, s, ts);
    case EPI_SILU: return launch_epi<DT, EPI_SILU>(plan, p, batch, s, ts);
    default: return launch_epi<DT, EPI_PLAIN>(plan, p, batch, s, ts);
  }
}

}  // namespace

#ifdef QA_PHASE_STAMPS
static int g_stamp_next = 0;  // the next launch's record slot
#endif

hipError_t launch_gemm(int dtype, const Plan& plan, const GemmParams& p_in, int batch,
                       hipStream_t stream, hipEvent_t t0, hipEvent_t t1) {
  const Stamps ts{t0, t1};
  GemmParams p = p_in;
  const int g = p.group_m > 0 ? p.group_m : 1, bands = (p.tiles_m + g - 1) / g;
  p.fd_split = fastdiv_make((uint32_t)p.splits);
  p.fd_band = fastdiv_make((uint32_t)(g * p.tiles_n));
  p.fd_rows = fastdiv_make((uint32_t)g);
  p.fd_last = fastdiv_make((uint32_t)(p.tiles_m - (bands - 1) * g));
#ifdef QA_PHASE_STAMPS
  p.stamp_slot = g_stamp_next;
  g_stamp_next = (g_stamp_next + 1) % kStampSlots;
#endif
  if (dtype == QA_BF16) return launch_dt<QA_BF16>(plan, p, batch, stream, ts);
  return launch_dt<QA_F16>(plan, p, batch, stream, ts);
}

}  // namespace qa

#ifdef QA_PHASE_STAMPS
// The measurement build's stamp records: kStampSlots x kStampBlocks x
// kStampWords words (see stamp_log), copied to `out`; *slots, *blocks and
// *words get the sizes.
extern "C" int qa_phase_stamps_read(unsigned long long* out, int* slots, int* blocks,
                                    int* words) {
  if (slots) *slots = qa::kStampSlots;
  if (blocks) *blocks = qa::kStampBlocks;
  if (words) *words = qa::kStampWords;
  if (!out) return QA_OK;
  const hipError_t e = hipMemcpyFromSymbol(out, HIP_SYMBOL(qa::stamp_log), sizeof(qa::stamp_log));
  return e == hipSuccess ? QA_OK : QA_EDEVICE;
}
// Zeroes every record (synchronous; call outside stream capture).
extern "C" int qa_phase_stamps_clear(void) {
  static unsigned long long zeros[sizeof(qa::stamp_log) / 8];
  const hipError_t e = hipMemcpyToSymbol(HIP_SYMBOL(qa::stamp_log), zeros, sizeof(qa::stamp_log));
  return e == hipSuccess ? QA_OK : QA_EDEVICE;
}
#endif
