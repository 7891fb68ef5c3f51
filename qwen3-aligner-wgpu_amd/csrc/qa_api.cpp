// qa_api.cpp -- the C ABI of include/qa.h over HIP.
//
// Replaces, for the linear-layer path, the reference's wgpu device runtime
// (src/gpu.rs: storage/upload/readback/flush, :672-762) and the GEMM dispatch
// helpers (src/decoder.rs:1030-1104, src/audio_encoder_gpu.rs:1895-1944).
// There is no pipeline compile or cache (src/gpu.rs:774-890): the kernels are
// gfx950 code objects linked into this library.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "half_bits.h"
#include "qa.h"
#include "qa_internal.h"

struct qa_ctx {
  int device = 0;
  hipStream_t stream = nullptr;
  int num_cus = 256;
  float* ws = nullptr;  // split-K partials
  size_t ws_floats = 0;
  float* scratch = nullptr;  // this device's copy of `scratch` (qa_linear_noalloc)
  // qa_prefetch_hint: bytes the projection after the next one reads; the next
  // projection launch takes it over and clears it
  const void* pf = nullptr;
  size_t pf_bytes = 0;
  // qa_time_next_launch: events the next projection's GEMM kernel stamps
  hipEvent_t t0 = nullptr, t1 = nullptr;
};

// The allocation-free linear's split-K partials (qa_linear_noalloc): one
// file-scope device array, 16 MiB of f32, which every GPU the library runs on
// holds until the process ends.  Host code never passes its name to a kernel
// (on the host the name is a stand-in, not a device address): each device's
// address comes from hipGetSymbolAddress at context creation, with that
// device current, and is kept per device.  Every qa_linear_noalloc call on a
// GPU shares that GPU's array, so calls that overlap on one GPU (two contexts'
// streams running at once) race on it.  Each split-K launch writes every
// partial it later reads, so nothing needs clearing between calls.
constexpr size_t kScratchFloats = (size_t)4 << 20;
static __device__ __align__(256) float scratch[kScratchFloats];

namespace {

thread_local std::string g_err;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

int ok() { return QA_OK; }

int hip_fail(hipError_t e, const char* what) {
  return fail(e == hipErrorOutOfMemory ? QA_ENOMEM : QA_EDEVICE, "%s: %s (%d)", what,
              hipGetErrorString(e), (int)e);
}

bool aligned(const void* p, size_t a) { return ((uintptr_t)p % a) == 0; }

constexpr uint32_t kKnownFlags =
    QA_ACCUMULATE | QA_EPI_GELU | QA_EPI_SILU_MUL | QA_TRANSB | QA_BIAS_ROWS;
constexpr int64_t kI32 = 0x7fffffff;

// Byte span [lo, hi) an operand covers over all batches.
struct Span {
  uintptr_t lo, hi;
};
Span span_of(const void* p, int64_t rows, int64_t cols, int64_t ld, int64_t batch, int64_t bs) {
  const uintptr_t lo = (uintptr_t)p;
  const int64_t last = (batch - 1) * bs + (rows - 1) * ld + cols;  // elements
  return {lo, lo + (uintptr_t)(last * 2)};
}
bool overlap(Span a, Span b) { return a.lo < b.hi && b.lo < a.hi; }

int validate(const qa_linear_desc* d) {
  if (!d) return fail(QA_EINVAL, "qa_linear: null descriptor");
  if (d->dtype != QA_F16 && d->dtype != QA_BF16)
    return fail(QA_EINVAL, "qa_linear: dtype %u is neither QA_F16 nor QA_BF16", d->dtype);
  if (d->flags & ~kKnownFlags) return fail(QA_EINVAL, "qa_linear: unknown flags 0x%x", d->flags);
  const bool silu = d->flags & QA_EPI_SILU_MUL, gelu = d->flags & QA_EPI_GELU;
  const bool accum = d->flags & QA_ACCUMULATE, transb = d->flags & QA_TRANSB;
  const bool brow = d->flags & QA_BIAS_ROWS;
  if (d->m < 0 || d->n <= 0 || d->k <= 0)
    return fail(QA_EINVAL, "qa_linear: bad shape m=%lld n=%lld k=%lld", (long long)d->m,
                (long long)d->n, (long long)d->k);
  if (d->m > kI32 || d->n > kI32 || d->k > kI32 || d->lda > kI32 || d->ldb > kI32 ||
      d->ldc > kI32)
    return fail(QA_EINVAL, "qa_linear: dimensions and strides must be below 2^31");
  if (!d->a || !d->w || !d->c) return fail(QA_EINVAL, "qa_linear: null operand pointer");
  if (d->k % 8) return fail(QA_EINVAL, "qa_linear: k=%lld is not a multiple of 8", (long long)d->k);
  if (d->lda < d->k || d->lda % 8)
    return fail(QA_EINVAL, "qa_linear: lda=%lld must be >= k and a multiple of 8",
                (long long)d->lda);
  if (silu && (gelu || accum || transb || brow || d->bias))
    return fail(QA_EINVAL, "qa_linear: QA_EPI_SILU_MUL takes no bias, residual, GELU or TRANSB");
  if (gelu && accum) return fail(QA_EINVAL, "qa_linear: QA_EPI_GELU with QA_ACCUMULATE");
  if (brow && !d->bias) return fail(QA_EINVAL, "qa_linear: QA_BIAS_ROWS without a bias");
  if (silu && d->n % 8)
    return fail(QA_EINVAL, "qa_linear: SiLU-mul needs n (= 2*inter) a multiple of 8, got %lld",
                (long long)d->n);
  if (transb) {
    if (d->n % 8) return fail(QA_EINVAL, "qa_linear: TRANSB needs n a multiple of 8");
    if (d->ldb < d->n || d->ldb % 8)
      return fail(QA_EINVAL, "qa_linear: TRANSB needs ldb >= n and a multiple of 8");
  } else if (d->ldb < d->k || d->ldb % 8) {
    return fail(QA_EINVAL, "qa_linear: ldb=%lld must be >= k and a multiple of 8",
                (long long)d->ldb);
  }
  const int64_t nout = silu ? d->n / 2 : d->n;
  if (nout % 4) return fail(QA_EINVAL, "qa_linear: output columns %lld not a multiple of 4",
                            (long long)nout);
  if (d->ldc < nout || d->ldc % 4)
    return fail(QA_EINVAL, "qa_linear: ldc=%lld must be >= %lld and a multiple of 4",
                (long long)d->ldc, (long long)nout);
  const int64_t batch = d->batch > 0 ? d->batch : 1;
  if (batch > 65535) return fail(QA_EINVAL, "qa_linear: batch %lld > 65535", (long long)batch);
  if (batch > 1) {
    if (d->bsa < 0 || d->bsb < 0 || d->bsc < 0 || d->bsa % 8 || d->bsb % 8 || d->bsc % 4)
      return fail(QA_EINVAL,
                  "qa_linear: batch strides must be >= 0, bsa/bsb multiples of 8, bsc of 4");
  }
  if (!aligned(d->a, 16) || !aligned(d->w, 16))
    return fail(QA_EINVAL, "qa_linear: a and w must be 16-byte aligned");
  if (!aligned(d->c, 8) || (d->bias && !aligned(d->bias, 8)))
    return fail(QA_EINVAL, "qa_linear: c and bias must be 8-byte aligned");
  if (((d->m > 0 ? d->m - 1 : 0) * d->lda + d->k) * 2 >= (int64_t)1 << 31 ||
      (((transb ? d->k : d->n) - 1) * d->ldb + (transb ? d->n : d->k)) * 2 >= (int64_t)1 << 31)
    return fail(QA_EUNSUPPORTED, "qa_linear: an operand spans 2 GiB or more (one batch)");
  if (d->m > 0) {
    const Span sa = span_of(d->a, d->m, d->k, d->lda, batch, d->bsa);
    const Span sw = transb ? span_of(d->w, d->k, d->n, d->ldb, batch, d->bsb)
                           : span_of(d->w, d->n, d->k, d->ldb, batch, d->bsb);
    const Span sc = span_of(d->c, d->m, nout, d->ldc, batch, d->bsc);
    if (overlap(sa, sc) || overlap(sw, sc))
      return fail(QA_EINVAL, "qa_linear: c overlaps an input operand");
  }
  return ok();
}

// Measured on MI355X (gfx950) with the kernels of qa_gemm.hip: time per
// 64-deep k stage of one tile with one block per CU (the L2 -> LDS stream
// sets it, not the matrix cores), and the fixed cost of a tile (block start
// skew + prologue fill + epilogue), in microseconds.
double stage_us(int tile) {
  switch (tile) {
    case qa::TILE_256x128:
    case qa::TILE_128x256: return 0.95;
    case qa::TILE_128x192: return 0.72;
    case qa::TILE_64x128: return 0.36;
    case qa::TILE_64x64: return 0.25;
    case qa::TILE_64x64_P2: return 0.21;
    case qa::TILE_256x256: return 1.75;
    // 256 x 192 (set between its neighbours; picked for the tower's qkv,
    // where it measured 31.0 against 34.9 us on 128 x 192)
    case qa::TILE_256x192: return 1.40;
    default: return 0.56;
  }
}
// 64-deep planes per ring stage: a split's k range runs in whole stages (the
// planes past its end read zeros), so its cost rounds up to that multiple.
int planes(int tile) { return tile == qa::TILE_64x64_P2 ? 2 : 1; }
double stages_of(int tile, int64_t kchunk) {
  const int64_t pl = planes(tile);
  return (double)(((kchunk + 63) / 64 + pl - 1) / pl * pl);
}
constexpr double kTileFixedUs = 3.0;
constexpr double kLaunchUs = 2.0;       // one more kernel in the stream (split-K reduce)
constexpr double kReduceGBs = 3000.0;   // split-K reduce kernel, partials from L2/MALL

// Tile / split-K choice: the modelled time of each candidate is
// rounds x (fixed + stages x stage_us) (+ the reduce kernel when K is split),
// where rounds = ceil(units / CUs); the cheapest candidate wins.
void choose_group_m(qa::Plan& pl, int64_t span = 0);

qa::Plan plan_linear(const qa_linear_desc& d, int num_cus, size_t max_ws_floats = SIZE_MAX) {
  qa::Plan pl{};
  const bool silu = d.flags & QA_EPI_SILU_MUL;
  pl.epi = silu ? qa::EPI_SILU : (d.flags & QA_EPI_GELU) ? qa::EPI_GELU : qa::EPI_PLAIN;
  pl.transb = (d.flags & QA_TRANSB) != 0;
  const int64_t M = d.m, N = d.n, K = d.k;
  const int64_t nout = silu ? N / 2 : N;

  int forced_tile = -1, forced_splits = 0;
  if (const char* e = getenv("QA_TILE")) forced_tile = atoi(e);
  if (const char* e = getenv("QA_SPLITS")) forced_splits = atoi(e);
  // A batch runs each problem as its own grid row (blockIdx.y) with no room
  // for split-K partials, so batched calls are never split: the planner, not
  // the shape, must not decide whether a valid batched call can run.
  if (d.batch > 1) forced_splits = 1;

  // every tile shape of the plain loader (TILE_256x160 is the conv loader's)
  int cands[] = {qa::TILE_128x128, qa::TILE_256x128, qa::TILE_128x256, qa::TILE_64x128,
                 qa::TILE_64x64,   qa::TILE_128x192, qa::TILE_256x256, qa::TILE_64x64_P2,
                 qa::TILE_256x192};
  int ncand = (int)(sizeof cands / sizeof cands[0]);
  if (pl.transb) ncand = 1;  // the conv operand path has one tile shape
  if (forced_tile >= 0 && forced_tile < qa::TILE_COUNT && forced_tile != qa::TILE_256x160 &&
      !pl.transb) {
    cands[0] = forced_tile;
    ncand = 1;
  }
  double best = 1e300;
  for (int ci = 0; ci < ncand; ++ci) {
    const qa::TileShape ts = qa::tile_shape(cands[ci]);
    const int64_t tbn = silu ? ts.bn / 2 : ts.bn;
    const int64_t tm = (M + ts.bm - 1) / ts.bm, tn = (nout + tbn - 1) / tbn;
    const int64_t tiles = tm * tn;
    const int64_t max_splits = forced_splits > 0 ? forced_splits : (pl.transb ? 1 : 8);
    for (int64_t want = forced_splits > 0 ? forced_splits : 1; want <= max_splits; want *= 2) {
      int64_t kchunk = ((K + want - 1) / want + 63) / 64 * 64;
      const int64_t splits = (K + kchunk - 1) / kchunk;
      if (splits > 1 && kchunk < 256 && forced_splits <= 0) break;  // keep >= 4 stages per split
      // partials that would not fit the caller's workspace bound (the
      // allocation-free entry point's scratch) rule a split count out
      if (splits > 1 && forced_splits <= 0 && (size_t)(splits * M * N) > max_ws_floats) break;
      const int64_t units = tiles * splits;
      const int64_t rounds = (units + num_cus - 1) / num_cus;
      double cost = (double)rounds * (kTileFixedUs + stages_of(cands[ci], kchunk) * stage_us(cands[ci]));
      if (splits > 1)
        cost += kLaunchUs + (double)(splits * 4 + 2) * (double)M * (double)N / (kReduceGBs * 1e3);
      if (cost < best * 0.999) {
        best = cost;
        pl.tile = cands[ci];
        pl.tiles_m = (int)tm;
        pl.tiles_n = (int)tn;
        pl.splits = (int)splits;
        pl.kchunk = (int)kchunk;
      }
      if (forced_splits > 0) break;
    }
  }
  if (pl.splits > 1) pl.ws_floats = (size_t)pl.splits * (size_t)M * (size_t)N;
  choose_group_m(pl);
  return pl;
}

// Tile enumeration bands (tile_of): each XCD takes a contiguous range of
// about per = tiles/8 tiles, which with bands of g m-tiles covers g m-tiles
// x ceil(per/g) n-tiles; its L2 fetches those A rows (bm each) and W rows
// (bn each, both halves of a SiLU tile).  The cheapest g wins, the whole
// n-column order (g = tiles_m) on ties.  With span > 0 the count is taken
// over the first `span` tiles of the range instead of all of it (see
// plan_conv).  QA_GROUP_M forces g.
void choose_group_m(qa::Plan& pl, int64_t span) {
  {
    const qa::TileShape ts = qa::tile_shape(pl.tile);
    const int64_t tm = pl.tiles_m, tn = pl.tiles_n;
    int64_t per = std::max<int64_t>(1, (tm * tn + 7) / 8);
    if (span > 0) per = std::min(per, span);
    pl.group_m = (int)tm;
    double best = 1e300;
    for (int64_t g = tm; g >= 1; g = g > 1 ? (g + 1) / 2 : 0) {
      // a range longer than a band spans whole bands: ceil(per / tn) m-tiles
      const int64_t rows = per > g * tn ? (per + tn - 1) / tn : std::min(g, per);
      const int64_t cols = std::min((per + g - 1) / g, tn);
      const double cost = (double)rows * ts.bm + (double)cols * ts.bn;
      if (cost < best * 0.999) {
        best = cost;
        pl.group_m = (int)g;
      }
    }
    if (const char* e = getenv("QA_GROUP_M")) {
      const int g = atoi(e);
      if (g >= 1) pl.group_m = (int)std::min<int64_t>(g, tm);
    }
  }
}

// The implicit-GEMM convolution: M = output pixels, N = c_out, K = 9 c_in,
// never split (K is long), on the tile shapes the CV loader is built for.
// The A operand is an input slab that nine taps re-read; at the stem's sizes
// (a 921 MB input for the second level over 300 chunks) an XCD's range of
// tiles touches far more of it than its 4 MB L2 holds, so only the tiles
// its CUs run at the same time (one per CU) can share what the L2 fetched:
// the band height is chosen for that window.  For the same reason the
// 128 x 256 tile comes first among equal costs: it gathers each input slab
// for half as many n-tiles as 256 x 128.  Measured on the 300-chunk second
// level (c = 480) with two k groups of MMA waves that issue their own DMA:
// 256 x 128 took 2.07 ms with the whole-range band (118 m-tiles, each slab
// re-fetched once per n-tile) and 1.50 ms with bands of 8; 128 x 256 with
// the window's band 1.37-1.41 ms, and 256 x 256 1.13-1.28 ms.  With one k
// group plus producer waves (the kernels now) 128 x 256 takes 1.08 ms and
// 256 x 128 1.21 ms; the third level (62400 pixels) 264 us on 128 x 256
// against 259 us on 256 x 256.  The per-stage costs of the CV loader, whose
// address arithmetic per chunk and 9-tap gather cost more than the plain
// loader's, are those kernel-trace times over the rounds and stages
// (conv_stage_us).
double conv_stage_us(int tile) {
  switch (tile) {
    case qa::TILE_128x256: return 1.09;
    case qa::TILE_256x128: return 1.21;
    case qa::TILE_256x256: return 2.27;
    // 256 x 160: same-box runs of the 300-chunk second level put its stage
    // at ~1.2x the 128 x 256 one (1.25x the FLOPs, 11 rounds against 15)
    case qa::TILE_256x160: return 1.30;
    default: return 0.74;  // 128 x 128
  }
}
qa::Plan plan_conv(int64_t M, int64_t N, int64_t K, bool gelu, int num_cus) {
  qa::Plan pl{};
  pl.epi = gelu ? qa::EPI_GELU : qa::EPI_PLAIN;
  pl.conv = true;
  pl.splits = 1;
  pl.kchunk = (int)((K + 63) / 64 * 64);
  double best = 1e300;
  int forced_tile = -1;
  if (const char* e = getenv("QA_TILE")) forced_tile = atoi(e);
  for (const int tile : {qa::TILE_128x256, qa::TILE_256x128, qa::TILE_128x128, qa::TILE_256x256,
                         qa::TILE_256x160}) {
    if (forced_tile >= 0 && forced_tile != tile) continue;
    const qa::TileShape ts = qa::tile_shape(tile);
    const int64_t tm = (M + ts.bm - 1) / ts.bm, tn = (N + ts.bn - 1) / ts.bn;
    const int64_t rounds = (tm * tn + num_cus - 1) / num_cus;
    const double cost = (double)rounds * (kTileFixedUs + (double)pl.kchunk / 64.0 * conv_stage_us(tile));
    if (cost < best * 0.999) {
      best = cost;
      pl.tile = tile;
      pl.tiles_m = (int)tm;
      pl.tiles_n = (int)tn;
    }
  }
  if (best == 1e300) {  // a forced tile the conv path does not have
    pl.tile = qa::TILE_128x128;
    pl.tiles_m = (int)((M + 127) / 128);
    pl.tiles_n = (int)((N + 127) / 128);
  }
  choose_group_m(pl, std::max(1, num_cus / 8));
  return pl;
}

int ensure_workspace(qa_ctx* ctx, size_t floats) {
  if (floats <= ctx->ws_floats) return ok();
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(ctx->stream, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone)
    return fail(QA_EINVAL,
                "the context workspace must grow (%zu floats) but the stream is being "
                "captured; run the same call once before capture",
                floats);
  hipError_t e = hipStreamSynchronize(ctx->stream);
  if (e != hipSuccess) return hip_fail(e, "hipStreamSynchronize");
  if (ctx->ws) (void)hipFree(ctx->ws);
  ctx->ws = nullptr;
  ctx->ws_floats = 0;
  e = hipMalloc(&ctx->ws, floats * sizeof(float));
  if (e != hipSuccess) return hip_fail(e, "hipMalloc(context workspace)");
  ctx->ws_floats = floats;
  return ok();
}

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
float* g_scratch[kMaxDevices] = {};

// This device's address of `scratch`; the device must be current.
int scratch_address(int device, float** out) {
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (device < 0 || device >= kMaxDevices)
    return fail(QA_EUNSUPPORTED, "device %d: at most %d devices", device, kMaxDevices);
  if (!g_scratch[device]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(scratch)");
    g_scratch[device] = (float*)p;
  }
  *out = g_scratch[device];
  return ok();
}

int set_device(qa_ctx* ctx) {
  const hipError_t e = hipSetDevice(ctx->device);
  return e == hipSuccess ? ok() : hip_fail(e, "hipSetDevice");
}

// What the next projection launch takes over from the context: the
// qa_prefetch_hint range and the qa_time_next_launch events.  Every
// projection entry point takes them first thing, before any check or early
// return, so a hint or an event pair never outlives the call it was set for
// (a hint left behind would make a later launch read a buffer that may have
// been freed in between).
struct NextLaunch {
  const void* pf = nullptr;
  size_t pf_bytes = 0;
  hipEvent_t t0 = nullptr, t1 = nullptr;
};
NextLaunch take_next_launch(qa_ctx* ctx) {
  NextLaunch n{ctx->pf, ctx->pf_bytes, ctx->t0, ctx->t1};
  ctx->pf = nullptr;
  ctx->pf_bytes = 0;
  ctx->t0 = ctx->t1 = nullptr;
  return n;
}

// Launch a validated, planned projection with split-K partials in `ws`.
int launch_linear(qa_ctx* ctx, const qa_linear_desc* d, const qa::Plan& plan, float* ws,
                  const NextLaunch& nl) {
  qa::GemmParams p{};
  p.a = (const uint16_t*)d->a;
  p.w = (const uint16_t*)d->w;
  p.c = (uint16_t*)d->c;
  p.bias = (const uint16_t*)d->bias;
  p.ws = ws;
  p.a_bytes = (int)(((d->m - 1) * d->lda + d->k) * 2);
  p.w_bytes = (int)((((d->flags & QA_TRANSB) ? d->k : d->n) - 1) * d->ldb +
                    ((d->flags & QA_TRANSB) ? d->n : d->k)) * 2;
  p.M = (int)d->m;
  p.N = (int)d->n;
  p.K = (int)d->k;
  p.lda = (int)d->lda;
  p.ldb = (int)d->ldb;
  p.ldc = (int)d->ldc;
  p.bsa = d->bsa;
  p.bsb = d->bsb;
  p.bsc = d->bsc;
  p.tiles_m = plan.tiles_m;
  p.tiles_n = plan.tiles_n;
  p.splits = plan.splits;
  p.kchunk = plan.kchunk;
  p.accumulate = (d->flags & QA_ACCUMULATE) ? 1 : 0;
  p.bias_rows = (d->flags & QA_BIAS_ROWS) ? 1 : 0;
  p.group_m = plan.group_m;
  if (nl.pf && !plan.transb) {
    p.pf = (const uint16_t*)nl.pf;
    p.pf_bytes = (int)std::min<size_t>(nl.pf_bytes, (size_t)INT32_MAX & ~(size_t)127);
  }
  const hipEvent_t t0 = nl.t0, t1 = nl.t1;
  if (t0 || t1) {
    // a captured dispatch does not stamp them on replay (the graph keeps an
    // event node that reads back as garbage)
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(ctx->stream, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone)
      return fail(QA_EINVAL,
                  "qa_linear: timing events from qa_time_next_launch cannot be recorded under "
                  "stream capture");
  }
  const int batch = d->batch > 0 ? (int)d->batch : 1;
  if (plan.splits > 1 && batch > 1)
    return fail(QA_EUNSUPPORTED, "qa_linear: split-K with batch > 1");
  const hipError_t e = qa::launch_gemm((int)d->dtype, plan, p, batch, ctx->stream, t0, t1);
  return e == hipSuccess ? ok() : hip_fail(e, "qa_linear launch");
}

}  // namespace

extern "C" {

const char* qa_last_error(void) { return g_err.c_str(); }

const char* qa_version(void) { return "qa 0.2.0 (abi 2, gfx950)"; }

int qa_ctx_create(int device, qa_ctx** out) {
  if (!out) return fail(QA_EINVAL, "qa_ctx_create: null output pointer");
  *out = nullptr;
  int count = 0;
  hipError_t e = hipGetDeviceCount(&count);
  if (e != hipSuccess || count <= 0)
    return fail(QA_EDEVICE, "qa_ctx_create: no HIP device visible (%s)",
                e == hipSuccess ? "device count 0" : hipGetErrorString(e));
  if (device < 0 || device >= count)
    return fail(QA_EINVAL, "qa_ctx_create: device %d out of range [0, %d)", device, count);
  hipDeviceProp_t prop;
  e = hipGetDeviceProperties(&prop, device);
  if (e != hipSuccess) return hip_fail(e, "hipGetDeviceProperties");
  if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
    return fail(QA_EUNSUPPORTED, "qa_ctx_create: device %d is %s; this library runs on gfx950",
                device, prop.gcnArchName);
  e = hipSetDevice(device);
  if (e != hipSuccess) return hip_fail(e, "hipSetDevice");
  qa_ctx* ctx = new qa_ctx;
  ctx->device = device;
  ctx->num_cus = prop.multiProcessorCount > 0 ? prop.multiProcessorCount : 256;
  if (int rc = scratch_address(device, &ctx->scratch)) {
    delete ctx;
    return rc;
  }
  e = hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking);
  if (e != hipSuccess) {
    delete ctx;
    return hip_fail(e, "hipStreamCreateWithFlags");
  }
  *out = ctx;
  return ok();
}

int qa_ctx_destroy(qa_ctx* ctx) {
  if (!ctx) return ok();
  (void)hipSetDevice(ctx->device);
  (void)hipStreamSynchronize(ctx->stream);
  if (ctx->ws) (void)hipFree(ctx->ws);
  const hipError_t e = hipStreamDestroy(ctx->stream);
  delete ctx;
  return e == hipSuccess ? ok() : hip_fail(e, "hipStreamDestroy");
}

void* qa_ctx_stream(qa_ctx* ctx) { return ctx ? (void*)ctx->stream : nullptr; }

int qa_alloc(qa_ctx* ctx, size_t bytes, void** out) {
  if (!ctx || !out) return fail(QA_EINVAL, "qa_alloc: null argument");
  *out = nullptr;
  if (int rc = set_device(ctx)) return rc;
  const size_t padded = std::max<size_t>(16, (bytes + 15) & ~(size_t)15);
  void* p = nullptr;
  hipError_t e = hipMalloc(&p, padded);
  if (e != hipSuccess) return hip_fail(e, "hipMalloc");
  // Zero-filled, as wgpu storage buffers are (the attention reads cache
  // entries past the written rows with weight zero; they must be finite).
  e = hipMemsetAsync(p, 0, padded, ctx->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
  if (e != hipSuccess) {
    (void)hipFree(p);
    return hip_fail(e, "hipMemsetAsync(qa_alloc)");
  }
  *out = p;
  return ok();
}

int qa_free(qa_ctx* ctx, void* ptr) {
  if (!ctx) return fail(QA_EINVAL, "qa_free: null context");
  if (!ptr) return ok();
  if (int rc = set_device(ctx)) return rc;
  const hipError_t e = hipFree(ptr);
  return e == hipSuccess ? ok() : hip_fail(e, "hipFree");
}

int qa_upload(qa_ctx* ctx, void* dst, size_t off, const void* src, size_t bytes) {
  if (!ctx || !dst || (!src && bytes)) return fail(QA_EINVAL, "qa_upload: null argument");
  if (!bytes) return ok();
  if (int rc = set_device(ctx)) return rc;
  hipError_t e = hipMemcpyAsync((char*)dst + off, src, bytes, hipMemcpyHostToDevice, ctx->stream);
  if (e != hipSuccess) return hip_fail(e, "hipMemcpyAsync(H2D)");
  e = hipStreamSynchronize(ctx->stream);
  return e == hipSuccess ? ok() : hip_fail(e, "hipStreamSynchronize");
}

int qa_download(qa_ctx* ctx, void* dst, const void* src, size_t off, size_t bytes) {
  if (!ctx || !src || (!dst && bytes)) return fail(QA_EINVAL, "qa_download: null argument");
  if (!bytes) return ok();
  if (int rc = set_device(ctx)) return rc;
  hipError_t e =
      hipMemcpyAsync(dst, (const char*)src + off, bytes, hipMemcpyDeviceToHost, ctx->stream);
  if (e != hipSuccess) return hip_fail(e, "hipMemcpyAsync(D2H)");
  e = hipStreamSynchronize(ctx->stream);
  return e == hipSuccess ? ok() : hip_fail(e, "hipStreamSynchronize");
}

int qa_sync(qa_ctx* ctx) {
  if (!ctx) return fail(QA_EINVAL, "qa_sync: null context");
  if (int rc = set_device(ctx)) return rc;
  const hipError_t e = hipStreamSynchronize(ctx->stream);
  return e == hipSuccess ? ok() : hip_fail(e, "qa_sync");
}

int qa_linear_validate(const qa_linear_desc* desc) { return validate(desc); }


int qa_linear(qa_ctx* ctx, const qa_linear_desc* d) {
  if (!ctx) return fail(QA_EINVAL, "qa_linear: null context");
  const NextLaunch nl = take_next_launch(ctx);
  if (int rc = validate(d)) return rc;
  if (d->m == 0) return ok();
  if (int rc = set_device(ctx)) return rc;
  const qa::Plan plan = plan_linear(*d, ctx->num_cus);
  if (plan.splits > 1) {
    if (int rc = ensure_workspace(ctx, plan.ws_floats)) return rc;
  }
  return launch_linear(ctx, d, plan, ctx->ws, nl);
}

int qa_linear_noalloc(qa_ctx* ctx, const qa_linear_desc* d) {
  if (!ctx) return fail(QA_EINVAL, "qa_linear_noalloc: null context");
  const NextLaunch nl = take_next_launch(ctx);
  if (int rc = validate(d)) return rc;
  if (d->m == 0) return ok();
  if (int rc = set_device(ctx)) return rc;
  // split counts whose partials exceed the scratch are never planned; only a
  // split forced through QA_SPLITS can ask for more
  const qa::Plan plan = plan_linear(*d, ctx->num_cus, kScratchFloats);
  if (plan.splits > 1 && plan.ws_floats > kScratchFloats)
    return fail(QA_EINVAL,
                "qa_linear_noalloc: %d K splits of a %lld x %lld output need %zu f32 partials; the "
                "scratch holds %zu",
                plan.splits, (long long)d->m, (long long)d->n, plan.ws_floats, kScratchFloats);
  return launch_linear(ctx, d, plan, ctx->scratch, nl);
}

size_t qa_linear_noalloc_scratch_floats(void) { return kScratchFloats; }

int qa_prefetch_hint(qa_ctx* ctx, const void* ptr, size_t bytes) {
  if (!ctx) return fail(QA_EINVAL, "qa_prefetch_hint: null context");
  if (!ptr && bytes) return fail(QA_EINVAL, "qa_prefetch_hint: null pointer with %zu bytes", bytes);
  ctx->pf = bytes ? ptr : nullptr;
  ctx->pf_bytes = ptr ? bytes : 0;
  return ok();
}

int qa_time_next_launch(qa_ctx* ctx, void* start_event, void* stop_event) {
  if (!ctx) return fail(QA_EINVAL, "qa_time_next_launch: null context");
  ctx->t0 = (hipEvent_t)start_event;
  ctx->t1 = (hipEvent_t)stop_event;
  return ok();
}

int qa_mlp_fused(qa_ctx* ctx, const qa_mlp_desc* d) {
  if (!ctx) return fail(QA_EINVAL, "qa_mlp_fused: null context");
  // the caller's hint and timing events belong to this call whatever happens
  // below; they go to the gate|up launch
  const NextLaunch nl = take_next_launch(ctx);
  if (!d) return fail(QA_EINVAL, "qa_mlp_fused: null descriptor");
  if (d->flags) return fail(QA_EINVAL, "qa_mlp_fused: flags must be 0");
  if (d->m < 0 || d->hidden <= 0 || d->inter <= 0)
    return fail(QA_EINVAL, "qa_mlp_fused: bad shape");
  qa_linear_desc gu{};
  gu.dtype = d->dtype;
  gu.flags = QA_EPI_SILU_MUL;
  gu.m = d->m;
  gu.n = 2 * d->inter;
  gu.k = d->hidden;
  gu.lda = d->hidden;
  gu.ldb = d->hidden;
  gu.ldc = d->inter;
  gu.a = d->x;
  gu.w = d->w_gu;
  gu.c = d->act;
  gu.batch = 1;
  qa_linear_desc down{};
  down.dtype = d->dtype;
  down.flags = QA_ACCUMULATE;
  down.m = d->m;
  down.n = d->hidden;
  down.k = d->inter;
  down.lda = d->inter;
  down.ldb = d->inter;
  down.ldc = d->hidden;
  down.a = d->act;
  down.w = d->w_down;
  down.c = d->h;
  down.batch = 1;
  if (int rc = validate(&gu)) return rc;
  if (int rc = validate(&down)) return rc;
  if (d->m == 0) return ok();
  // a caller's hint stays with the gate|up launch; otherwise it pulls the
  // down projection's weights toward the caches
  ctx->pf = nl.pf ? nl.pf : d->w_down;
  ctx->pf_bytes = nl.pf ? nl.pf_bytes : (size_t)(d->hidden * d->inter) * 2;
  ctx->t0 = nl.t0;
  ctx->t1 = nl.t1;
  if (int rc = qa_linear(ctx, &gu)) return rc;
  return qa_linear(ctx, &down);
}

int qa_rms_norm(qa_ctx* ctx, const qa_rms_norm_desc* d) {
  if (!ctx || !d) return fail(QA_EINVAL, "qa_rms_norm: null argument");
  if (d->dtype != QA_F16 && d->dtype != QA_BF16)
    return fail(QA_EINVAL, "qa_rms_norm: dtype %u is neither QA_F16 nor QA_BF16", d->dtype);
  if (d->flags) return fail(QA_EINVAL, "qa_rms_norm: flags must be 0");
  if (d->rows < 0 || d->n <= 0 || d->n % 8 || d->n > kI32)
    return fail(QA_EINVAL, "qa_rms_norm: rows >= 0 and n a positive multiple of 8, got %lld x %lld",
                (long long)d->rows, (long long)d->n);
  if (d->ldx < d->n || d->ldy < d->n || d->ldx % 8 || d->ldy % 8)
    return fail(QA_EINVAL, "qa_rms_norm: row strides must be >= n and multiples of 8");
  if (!d->x || !d->y || !d->w) return fail(QA_EINVAL, "qa_rms_norm: null pointer");
  if (!aligned(d->x, 16) || !aligned(d->y, 16) || !aligned(d->w, 4))
    return fail(QA_EINVAL, "qa_rms_norm: x and y must be 16-byte aligned");
  if (!(d->eps >= 0.0f)) return fail(QA_EINVAL, "qa_rms_norm: eps must be >= 0");
  if (d->rows == 0) return ok();
  if (int rc = set_device(ctx)) return rc;
  qa::RmsParams p{};
  p.x = (const uint16_t*)d->x;
  p.w = d->w;
  p.y = (uint16_t*)d->y;
  p.rows = d->rows;
  p.ldx = d->ldx;
  p.ldy = d->ldy;
  p.n = (int)d->n;
  p.eps = d->eps;
  const hipError_t e = qa::launch_rms_norm((int)d->dtype, p, ctx->stream);
  return e == hipSuccess ? ok() : hip_fail(e, "qa_rms_norm launch");
}

int qa_qk_norm_rope(qa_ctx* ctx, const qa_qk_rope_desc* d) {
  if (!ctx || !d) return fail(QA_EINVAL, "qa_qk_norm_rope: null argument");
  if (d->dtype != QA_F16 && d->dtype != QA_BF16)
    return fail(QA_EINVAL, "qa_qk_norm_rope: dtype %u is neither QA_F16 nor QA_BF16", d->dtype);
  if (d->flags) return fail(QA_EINVAL, "qa_qk_norm_rope: flags must be 0");
  if (d->rows < 0 || d->nqh <= 0 || d->nkvh <= 0 || d->nqh % d->nkvh)
    return fail(QA_EINVAL, "qa_qk_norm_rope: need rows >= 0 and nqh a multiple of nkvh > 0");
  if (d->hd <= 0 || d->hd % 64 || d->hd > 256)
    return fail(QA_EINVAL, "qa_qk_norm_rope: hd=%d must be a multiple of 64 up to 256", d->hd);
  if (d->ldqkv < (int64_t)(d->nqh + 2 * d->nkvh) * d->hd)
    return fail(QA_EINVAL, "qa_qk_norm_rope: ldqkv below the fused q|k|v width");
  if (d->pos0 < 0 || d->start < 0 || d->start + d->rows > d->cap || d->cap % 16 || d->cap > kI32)
    return fail(QA_EINVAL,
                "qa_qk_norm_rope: need pos0, start >= 0, start + rows <= cap, cap a multiple of 16");
  if (!d->qkv || !d->qn_w || !d->kn_w || !d->cos || !d->sin || !d->q_out || !d->k_cache ||
      !d->v_cache)
    return fail(QA_EINVAL, "qa_qk_norm_rope: null pointer");
  if (!aligned(d->qkv, 2) || !aligned(d->q_out, 2) || !aligned(d->k_cache, 2) ||
      !aligned(d->v_cache, 2) || !aligned(d->qn_w, 4) || !aligned(d->kn_w, 4) ||
      !aligned(d->cos, 4) || !aligned(d->sin, 4))
    return fail(QA_EINVAL, "qa_qk_norm_rope: misaligned pointer");
  if (!(d->eps >= 0.0f)) return fail(QA_EINVAL, "qa_qk_norm_rope: eps must be >= 0");
  if (d->rows == 0) return ok();
  if (int rc = set_device(ctx)) return rc;
  qa::RopeParams p{};
  p.qkv = (const uint16_t*)d->qkv;
  p.qn = d->qn_w;
  p.kn = d->kn_w;
  p.cos = d->cos;
  p.sin = d->sin;
  p.q_out = (uint16_t*)d->q_out;
  p.k_cache = (uint16_t*)d->k_cache;
  p.v_cache = (uint16_t*)d->v_cache;
  p.rows = d->rows;
  p.ldqkv = d->ldqkv;
  p.pos0 = d->pos0;
  p.cap = d->cap;
  p.start = d->start;
  p.nqh = d->nqh;
  p.nkvh = d->nkvh;
  p.hd = d->hd;
  p.eps = d->eps;
  const hipError_t e = qa::launch_qk_norm_rope((int)d->dtype, p, ctx->stream);
  return e == hipSuccess ? ok() : hip_fail(e, "qa_qk_norm_rope launch");
}

int qa_attention_prefill(qa_ctx* ctx, const qa_attention_desc* d) {
  if (!ctx || !d) return fail(QA_EINVAL, "qa_attention_prefill: null argument");
  if (d->dtype != QA_F16 && d->dtype != QA_BF16)
    return fail(QA_EINVAL, "qa_attention_prefill: dtype %u is neither QA_F16 nor QA_BF16",
                d->dtype);
  if (d->flags & ~QA_ATTN_P16)
    return fail(QA_EINVAL, "qa_attention_prefill: unknown flags 0x%x", d->flags & ~QA_ATTN_P16);
  if (d->rows < 0 || d->nqh <= 0 || d->nkvh <= 0 || d->nqh % d->nkvh)
    return fail(QA_EINVAL, "qa_attention_prefill: need rows >= 0 and nqh a multiple of nkvh > 0");
  if (d->hd != 128) return fail(QA_EUNSUPPORTED, "qa_attention_prefill: hd=%d (only 128)", d->hd);
  if (d->q0 < 0 || d->q0 + d->rows > d->cap || d->cap * d->hd * 2 > kI32)
    return fail(QA_EINVAL,
                "qa_attention_prefill: need q0 >= 0, q0 + rows <= cap and a cache head below 2 GiB");
  if (d->cap % 16) return fail(QA_EINVAL, "qa_attention_prefill: cap must be a multiple of 16");
  if (d->nqh / d->nkvh > 2)
    return fail(QA_EUNSUPPORTED, "qa_attention_prefill: nqh / nkvh = %d (1 or 2 supported)",
                d->nqh / d->nkvh);
  if (d->ldo < (int64_t)d->nqh * d->hd || d->ldo % 8)
    return fail(QA_EINVAL, "qa_attention_prefill: ldo must be >= nqh*hd and a multiple of 8");
  if (!d->q || !d->k_cache || !d->v_cache || !d->out)
    return fail(QA_EINVAL, "qa_attention_prefill: null pointer");
  if (!aligned(d->q, 16) || !aligned(d->k_cache, 16) || !aligned(d->v_cache, 16) ||
      !aligned(d->out, 16))
    return fail(QA_EINVAL, "qa_attention_prefill: buffers must be 16-byte aligned");
  if (d->rows == 0) return ok();
  if (int rc = set_device(ctx)) return rc;
  qa::AttnParams p{};
  p.q = (const uint16_t*)d->q;
  p.k_cache = (const uint16_t*)d->k_cache;
  p.v_cache = (const uint16_t*)d->v_cache;
  p.out = (uint16_t*)d->out;
  p.rows = d->rows;
  p.cap = d->cap;
  p.q0 = d->q0;
  p.ldo = d->ldo;
  p.nqh = d->nqh;
  p.nkvh = d->nkvh;
  p.hd = d->hd;
  p.scale = 1.0f / sqrtf((float)d->hd);
  const hipError_t e = qa::launch_attention((int)d->dtype, p, (d->flags & QA_ATTN_P16) != 0, ctx->stream);
  return e == hipSuccess ? ok() : hip_fail(e, "qa_attention_prefill launch");
}

int qa_conv2d_3x3s2(qa_ctx* ctx, const qa_conv_desc* d) {
  if (!ctx || !d) return fail(QA_EINVAL, "qa_conv2d_3x3s2: null argument");
  if (d->dtype != QA_F16 && d->dtype != QA_BF16)
    return fail(QA_EINVAL, "qa_conv2d_3x3s2: dtype %u is neither QA_F16 nor QA_BF16", d->dtype);
  if (d->flags & ~(uint32_t)(QA_CONV_GELU | QA_CONV_TOKEN_MAJOR))
    return fail(QA_EINVAL, "qa_conv2d_3x3s2: unknown flags 0x%x",
                d->flags & ~(uint32_t)(QA_CONV_GELU | QA_CONV_TOKEN_MAJOR));
  if (d->batch < 0 || d->h <= 0 || d->w <= 0 || d->c_in <= 0 || d->c_out <= 0)
    return fail(QA_EINVAL, "qa_conv2d_3x3s2: bad shape");
  if (d->c_out % 8) return fail(QA_EINVAL, "qa_conv2d_3x3s2: c_out must be a multiple of 8");
  const bool direct = d->c_in == 1;
  if (!direct && (d->c_in % 8 || d->c_in < 64))
    return fail(QA_EUNSUPPORTED,
                "qa_conv2d_3x3s2: c_in=%lld (1, or a multiple of 8 >= 64)", (long long)d->c_in);
  if (direct && d->c_out > 1024)
    return fail(QA_EUNSUPPORTED, "qa_conv2d_3x3s2: c_out=%lld > 1024 with c_in = 1",
                (long long)d->c_out);
  const int64_t ho = (d->h - 1) / 2 + 1, wo = (d->w - 1) / 2 + 1;
  const int64_t M = d->batch * ho * wo;
  const int64_t K = 9 * d->c_in, ldw = (K + 7) / 8 * 8;
  if (d->batch * d->h * d->w * d->c_in * 2 > kI32 || M * d->c_out > kI32 * 4LL ||
      d->c_out * ldw * 2 > kI32 || M > kI32)
    return fail(QA_EINVAL, "qa_conv2d_3x3s2: operands must stay below 2 GiB");
  if (!d->x || !d->weight || !d->y) return fail(QA_EINVAL, "qa_conv2d_3x3s2: null pointer");
  if (!aligned(d->x, 16) || !aligned(d->weight, 16) || !aligned(d->y, 16) ||
      (d->bias && !aligned(d->bias, 8)))
    return fail(QA_EINVAL, "qa_conv2d_3x3s2: x, weight and y must be 16-byte aligned, bias 8");
  if (M == 0) return ok();
  if (int rc = set_device(ctx)) return rc;
  const bool gelu = (d->flags & QA_CONV_GELU) != 0, tmajor = (d->flags & QA_CONV_TOKEN_MAJOR) != 0;
  if (direct) {
    qa::Conv1Params p{};
    p.x = (const uint16_t*)d->x;
    p.w = (const uint16_t*)d->weight;
    p.bias = (const uint16_t*)d->bias;
    p.y = (uint16_t*)d->y;
    p.M = M;
    p.h = (int)d->h;
    p.w_in = (int)d->w;
    p.ho = (int)ho;
    p.wo = (int)wo;
    p.c_out = (int)d->c_out;
    p.ldw = (int)ldw;
    p.tmajor = tmajor;
    p.gelu = gelu;
    const hipError_t e = qa::launch_conv1((int)d->dtype, p, ctx->stream);
    return e == hipSuccess ? ok() : hip_fail(e, "qa_conv2d_3x3s2 launch");
  }
  const qa::Plan plan = plan_conv(M, d->c_out, K, gelu, ctx->num_cus);
  qa::GemmParams p{};
  p.a = (const uint16_t*)d->x;
  p.w = (const uint16_t*)d->weight;
  p.c = (uint16_t*)d->y;
  p.bias = (const uint16_t*)d->bias;
  p.a_bytes = (int)(d->batch * d->h * d->w * d->c_in * 2);
  p.w_bytes = (int)(d->c_out * ldw * 2);
  p.M = (int)M;
  p.N = (int)d->c_out;
  p.K = (int)K;
  p.lda = (int)K;
  p.ldb = (int)ldw;
  p.ldc = (int)d->c_out;
  p.tiles_m = plan.tiles_m;
  p.tiles_n = plan.tiles_n;
  p.splits = 1;
  p.kchunk = plan.kchunk;
  p.group_m = plan.group_m;
  p.cv_c = (int)d->c_in;
  p.cv_h = (int)d->h;
  p.cv_w = (int)d->w;
  p.cv_ho = (int)ho;
  p.cv_wo = (int)wo;
  p.cv_tmajor = tmajor;
  const hipError_t e = qa::launch_gemm((int)d->dtype, plan, p, 1, ctx->stream);
  return e == hipSuccess ? ok() : hip_fail(e, "qa_conv2d_3x3s2 launch");
}

int qa_mel_filterbank(int n_mels, int n_fft, int sample_rate, float* out) {
  if (!out || n_mels <= 0 || n_fft <= 0 || sample_rate <= 0)
    return fail(QA_EINVAL, "qa_mel_filterbank: bad argument");
  // create_mel_filterbank (src/mel.rs:100-154): slaney mel scale (linear below
  // 1 kHz at 200/3 Hz per mel, logarithmic above with step ln(6.4) / 27),
  // n_mels + 2 points evenly spaced in mel from 0 to sr / 2, triangles over
  // the FFT bin frequencies, each scaled by 2 / (width in Hz).  f64, stored f32.
  const int n_freqs = n_fft / 2 + 1;
  const double sr = sample_rate, f_sp = 200.0 / 3.0, min_log_hz = 1000.0;
  const double min_log_mel = min_log_hz / f_sp, logstep = std::log(6.4) / 27.0;
  auto hz_to_mel = [&](double f) {
    return f < min_log_hz ? f / f_sp : min_log_mel + std::log(f / min_log_hz) / logstep;
  };
  auto mel_to_hz = [&](double m) {
    return m < min_log_mel ? f_sp * m : min_log_hz * std::exp(logstep * (m - min_log_mel));
  };
  const double mel_lo = hz_to_mel(0.0), mel_hi = hz_to_mel(sr / 2.0);
  std::vector<double> ff((size_t)n_mels + 2);
  for (int i = 0; i < n_mels + 2; ++i)
    ff[(size_t)i] = mel_to_hz(mel_lo + (mel_hi - mel_lo) * i / (double)(n_mels + 1));
  for (int i = 0; i < n_mels; ++i) {
    const double enorm = 2.0 / (ff[(size_t)i + 2] - ff[(size_t)i]);
    for (int j = 0; j < n_freqs; ++j) {
      const double f = j * sr / n_fft;
      const double down = (f - ff[(size_t)i]) / (ff[(size_t)i + 1] - ff[(size_t)i]);
      const double up = (ff[(size_t)i + 2] - f) / (ff[(size_t)i + 2] - ff[(size_t)i + 1]);
      out[(size_t)i * n_freqs + j] = (float)std::max(0.0, std::min(down, up)) * (float)enorm;
    }
  }
  return ok();
}

int qa_log_mel(qa_ctx* ctx, const qa_mel_desc* d) {
  if (!ctx || !d) return fail(QA_EINVAL, "qa_log_mel: null argument");
  if (d->dtype != QA_F16 && d->dtype != QA_BF16)
    return fail(QA_EINVAL, "qa_log_mel: dtype %u is neither QA_F16 nor QA_BF16", d->dtype);
  if (d->flags) return fail(QA_EINVAL, "qa_log_mel: flags must be 0");
  if (d->n_samples < 160 || d->n_samples > kI32 || d->n_mels <= 0 || d->n_mels > 1024 ||
      d->cs <= 0 || d->cs % 2)
    return fail(QA_EINVAL, "qa_log_mel: need n_samples >= 160, 0 < n_mels <= 1024 and cs even");
  if (!d->samples || !d->filterbank || !d->out) return fail(QA_EINVAL, "qa_log_mel: null pointer");
  if (!aligned(d->samples, 4) || !aligned(d->filterbank, 4) || !aligned(d->out, 4))
    return fail(QA_EINVAL, "qa_log_mel: misaligned pointer");
  if (int rc = set_device(ctx)) return rc;
  qa::MelParams p{};
  p.frames = d->n_samples / 160;
  p.n = d->n_samples;
  p.n_mels = d->n_mels;
  p.cs = d->cs;
  p.n_chunks = (int)((p.frames + d->cs - 1) / d->cs);
  p.nblocks = (int)((p.frames + qa::kMelFramesPerBlock - 1) / qa::kMelFramesPerBlock);
  // workspace: logmel, block maxima, then (from a 64-float boundary) the
  // twiddle table and the filters' supports
  const size_t tw_at = ((size_t)p.n_mels * (size_t)p.frames + (size_t)p.nblocks + 63) & ~(size_t)63;
  const size_t floats = tw_at + 800 * 2 + 2 * (size_t)p.n_mels;
  if (int rc = ensure_workspace(ctx, floats)) return rc;
  p.x = d->samples;
  p.filt = d->filterbank;
  p.logmel = ctx->ws;
  p.bmax = ctx->ws + (size_t)p.n_mels * (size_t)p.frames;
  p.tw = reinterpret_cast<double*>(ctx->ws + tw_at);
  p.sup = reinterpret_cast<int32_t*>(ctx->ws + tw_at + 800 * 2);
  p.out = (uint16_t*)d->out;
  const hipError_t e = qa::launch_log_mel((int)d->dtype, p, ctx->stream);
  return e == hipSuccess ? ok() : hip_fail(e, "qa_log_mel launch");
}

// The run's 16-bit rounding of an f32 value, widened back to f32: IEEE RNE for
// f16; (u + 0x7FFF + ((u >> 16) & 1)) >> 16 for bf16 (src/shaders.rs:169-179).
float round16(float v, uint32_t dtype) {
  if (dtype == QA_BF16) return qa_half::bf16_to_f32(qa_half::bf16_from_f32(v));
  return qa_half::f16_to_f32(qa_half::f16_from_f32(v));
}

int qa_rope_tables(int64_t positions, int hd, double theta, uint32_t dtype, float* cos_out,
                   float* sin_out) {
  if (positions <= 0 || hd <= 0 || hd % 2 || !(theta > 0.0) || !cos_out || !sin_out)
    return fail(QA_EINVAL, "qa_rope_tables: bad argument");
  if (dtype != QA_F16 && dtype != QA_BF16)
    return fail(QA_EINVAL, "qa_rope_tables: dtype %u is neither QA_F16 nor QA_BF16", dtype);
  const int half = hd / 2;
  std::vector<double> inv((size_t)half);
  for (int j = 0; j < half; ++j) inv[(size_t)j] = 1.0 / std::pow(theta, 2.0 * j / hd);
  for (int64_t p = 0; p < positions; ++p)
    for (int j = 0; j < half; ++j) {
      const double a = (double)p * inv[(size_t)j];
      const float c = round16((float)std::cos(a), dtype), s = round16((float)std::sin(a), dtype);
      cos_out[p * hd + j] = cos_out[p * hd + j + half] = c;
      sin_out[p * hd + j] = sin_out[p * hd + j + half] = s;
    }
  return ok();
}

int qa_embed_scatter(qa_ctx* ctx, const qa_embed_desc* d) {
  if (!ctx || !d) return fail(QA_EINVAL, "qa_embed_scatter: null argument");
  if (d->dtype != QA_F16 && d->dtype != QA_BF16)
    return fail(QA_EINVAL, "qa_embed_scatter: dtype %u is neither QA_F16 nor QA_BF16", d->dtype);
  if (d->flags) return fail(QA_EINVAL, "qa_embed_scatter: flags must be 0");
  if (d->rows < 0 || d->hidden <= 0 || d->hidden % 8 || d->hidden > kI32 || d->vocab < 0 ||
      d->n_audio < 0)
    return fail(QA_EINVAL, "qa_embed_scatter: bad shape");
  if (!d->src || !d->out || (d->vocab && !d->table) || (d->n_audio && !d->audio))
    return fail(QA_EINVAL, "qa_embed_scatter: null pointer");
  if (!aligned(d->out, 16) || (d->table && !aligned(d->table, 16)) ||
      (d->audio && !aligned(d->audio, 16)) || !aligned(d->src, 4))
    return fail(QA_EINVAL, "qa_embed_scatter: table, audio and out must be 16-byte aligned");
  if (d->rows == 0) return ok();
  if (int rc = set_device(ctx)) return rc;
  qa::EmbedParams p{};
  p.src = d->src;
  p.table = (const uint16_t*)d->table;
  p.audio = (const uint16_t*)d->audio;
  p.out = (uint16_t*)d->out;
  p.rows = d->rows;
  p.vocab = d->vocab;
  p.n_audio = d->n_audio;
  p.hidden = (int)d->hidden;
  const hipError_t e = qa::launch_embed_scatter(p, ctx->stream);
  return e == hipSuccess ? ok() : hip_fail(e, "qa_embed_scatter launch");
}

int qa_timestamp_head(qa_ctx* ctx, const qa_head_desc* d) {
  if (!ctx || !d) return fail(QA_EINVAL, "qa_timestamp_head: null argument");
  if (d->dtype != QA_F16 && d->dtype != QA_BF16)
    return fail(QA_EINVAL, "qa_timestamp_head: dtype %u is neither QA_F16 nor QA_BF16", d->dtype);
  if (d->flags) return fail(QA_EINVAL, "qa_timestamp_head: flags must be 0");
  if (d->rows < 0 || d->n <= 0 || d->n > kI32 || d->labels <= 0 || d->labels > kI32 ||
      d->h_rows < 0 || d->ldh < d->n || (d->rows + 15) / 16 > 65535)
    return fail(QA_EINVAL, "qa_timestamp_head: bad shape");
  if (!d->positions || !d->h || !d->norm_w || !d->score || !d->logits || !d->classes)
    return fail(QA_EINVAL, "qa_timestamp_head: null pointer");
  if (!aligned(d->h, 2) || !aligned(d->norm_w, 4) || !aligned(d->score, 4) ||
      !aligned(d->logits, 4) || !aligned(d->classes, 4) || !aligned(d->positions, 4))
    return fail(QA_EINVAL, "qa_timestamp_head: misaligned pointer");
  if (!(d->eps >= 0.0f)) return fail(QA_EINVAL, "qa_timestamp_head: eps must be >= 0");
  if (d->rows == 0) return ok();
  if (int rc = set_device(ctx)) return rc;
  if (int rc = ensure_workspace(ctx, (size_t)(d->rows * d->n))) return rc;
  qa::HeadParams p{};
  p.pos = d->positions;
  p.h = (const uint16_t*)d->h;
  p.w = d->norm_w;
  p.score = d->score;
  p.normed = ctx->ws;
  p.logits = d->logits;
  p.cls = d->classes;
  p.rows = d->rows;
  p.h_rows = d->h_rows;
  p.ldh = d->ldh;
  p.labels = d->labels;
  p.n = (int)d->n;
  p.eps = d->eps;
  const hipError_t e = qa::launch_timestamp_head((int)d->dtype, p, ctx->stream);
  return e == hipSuccess ? ok() : hip_fail(e, "qa_timestamp_head launch");
}

int qa_layer_norm(qa_ctx* ctx, const qa_layer_norm_desc* d) {
  if (!ctx || !d) return fail(QA_EINVAL, "qa_layer_norm: null argument");
  if (d->dtype != QA_F16 && d->dtype != QA_BF16)
    return fail(QA_EINVAL, "qa_layer_norm: dtype %u is neither QA_F16 nor QA_BF16", d->dtype);
  if (d->flags) return fail(QA_EINVAL, "qa_layer_norm: flags must be 0");
  if (d->rows < 0 || d->n <= 0 || d->n % 8 || d->n > kI32)
    return fail(QA_EINVAL, "qa_layer_norm: rows >= 0 and n a positive multiple of 8, got %lld x %lld",
                (long long)d->rows, (long long)d->n);
  if (d->ldx < d->n || d->ldy < d->n || d->ldx % 8 || d->ldy % 8)
    return fail(QA_EINVAL, "qa_layer_norm: row strides must be >= n and multiples of 8");
  if (!d->x || !d->y || !d->w || !d->b) return fail(QA_EINVAL, "qa_layer_norm: null pointer");
  if (!aligned(d->x, 16) || !aligned(d->y, 16) || !aligned(d->w, 4) || !aligned(d->b, 4))
    return fail(QA_EINVAL, "qa_layer_norm: x and y must be 16-byte aligned");
  if (!(d->eps >= 0.0f)) return fail(QA_EINVAL, "qa_layer_norm: eps must be >= 0");
  if (d->rows == 0) return ok();
  if (int rc = set_device(ctx)) return rc;
  qa::LnParams p{};
  p.x = (const uint16_t*)d->x;
  p.w = d->w;
  p.b = d->b;
  p.y = (uint16_t*)d->y;
  p.rows = d->rows;
  p.ldx = d->ldx;
  p.ldy = d->ldy;
  p.n = (int)d->n;
  p.eps = d->eps;
  const hipError_t e = qa::launch_layer_norm((int)d->dtype, p, ctx->stream);
  return e == hipSuccess ? ok() : hip_fail(e, "qa_layer_norm launch");
}

int qa_window_attention(qa_ctx* ctx, const qa_window_attention_desc* d) {
  if (!ctx || !d) return fail(QA_EINVAL, "qa_window_attention: null argument");
  if (d->dtype != QA_F16 && d->dtype != QA_BF16)
    return fail(QA_EINVAL, "qa_window_attention: dtype %u is neither QA_F16 nor QA_BF16",
                d->dtype);
  if (d->flags) return fail(QA_EINVAL, "qa_window_attention: flags must be 0");
  if (d->s < 0 || d->nh <= 0 || d->wlen <= 0)
    return fail(QA_EINVAL, "qa_window_attention: need s >= 0, nh > 0 and wlen > 0");
  if (d->hd != 64) return fail(QA_EUNSUPPORTED, "qa_window_attention: hd=%d (only 64)", d->hd);
  if (d->wlen > 128)
    return fail(QA_EUNSUPPORTED, "qa_window_attention: wlen=%lld (at most 128)", (long long)d->wlen);
  const int64_t dm = (int64_t)d->nh * d->hd;
  if (d->ldqkv < 3 * dm || d->ldqkv % 8 || d->ldo < dm || d->ldo % 8)
    return fail(QA_EINVAL,
                "qa_window_attention: ldqkv must be >= 3 nh hd, ldo >= nh hd, both multiples of 8");
  if ((d->s + d->wlen - 1) / d->wlen * d->nh > kI32)
    return fail(QA_EINVAL, "qa_window_attention: too many windows");
  if (!d->qkv || !d->out) return fail(QA_EINVAL, "qa_window_attention: null pointer");
  if (!aligned(d->qkv, 16) || !aligned(d->out, 16))
    return fail(QA_EINVAL, "qa_window_attention: qkv and out must be 16-byte aligned");
  if (d->s == 0) return ok();
  if (int rc = set_device(ctx)) return rc;
  qa::WinAttnParams p{};
  p.qkv = (const uint16_t*)d->qkv;
  p.out = (uint16_t*)d->out;
  p.s = d->s;
  p.wlen = d->wlen;
  p.ldqkv = d->ldqkv;
  p.ldo = d->ldo;
  p.nh = d->nh;
  p.scale = 1.0f / sqrtf((float)d->hd);
  const hipError_t e = qa::launch_window_attention((int)d->dtype, p, ctx->stream);
  return e == hipSuccess ? ok() : hip_fail(e, "qa_window_attention launch");
}

int qa_add_position_table(qa_ctx* ctx, const qa_position_add_desc* d) {
  if (!ctx || !d) return fail(QA_EINVAL, "qa_add_position_table: null argument");
  if (d->dtype != QA_F16 && d->dtype != QA_BF16)
    return fail(QA_EINVAL, "qa_add_position_table: dtype %u is neither QA_F16 nor QA_BF16",
                d->dtype);
  if (d->flags) return fail(QA_EINVAL, "qa_add_position_table: flags must be 0");
  if (d->rows < 0 || d->n <= 0 || d->n % 8 || d->period <= 0)
    return fail(QA_EINVAL, "qa_add_position_table: need rows >= 0, n a positive multiple of 8, "
                           "period > 0");
  if (d->ldy < d->n || d->ldy % 8)
    return fail(QA_EINVAL, "qa_add_position_table: ldy must be >= n and a multiple of 8");
  if (!d->y || !d->table) return fail(QA_EINVAL, "qa_add_position_table: null pointer");
  if (!aligned(d->y, 16) || !aligned(d->table, 4))
    return fail(QA_EINVAL, "qa_add_position_table: y must be 16-byte aligned");
  if (d->rows * (d->n / 8) > kI32 * 256LL)
    return fail(QA_EINVAL, "qa_add_position_table: too many elements");
  if (d->rows == 0) return ok();
  if (int rc = set_device(ctx)) return rc;
  qa::TableAddParams p{};
  p.y = (uint16_t*)d->y;
  p.table = d->table;
  p.rows = d->rows;
  p.ldy = d->ldy;
  p.n = d->n;
  p.period = d->period;
  const hipError_t e = qa::launch_add_table((int)d->dtype, p, ctx->stream);
  return e == hipSuccess ? ok() : hip_fail(e, "qa_add_position_table launch");
}

}  // extern "C"
