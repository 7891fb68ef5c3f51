/*
 * qa.h -- C ABI of the MI355X (gfx950) linear-layer GEMM path of
 * eclipse005/qwen3-aligner-wgpu.
 *
 * The reference dispatches every dense projection of its prefill forward
 * through one WGSL GEMM family, `prefill_gemm` (src/shaders.rs:1785-2077), from
 * two call surfaces: the text decoder's `gemm!` / `gemm_at!` macros
 * (src/decoder.rs:1030-1104, uniform `GDims` at src/decoder.rs:194-212) and the
 * audio tower's `GpuAudioEncoder::{gemm, gemm_beta, gemm_conv, dispatch_gemm}`
 * (src/audio_encoder_gpu.rs:1614-1944).  Buffers come from `Gpu::storage`
 * (src/gpu.rs:672-682), data moves with `Gpu::upload` / `write_at` /
 * `readback` (src/gpu.rs:697-762) and `flush` / `pump` wait for the queue
 * (src/gpu.rs:709-728).  This header is the C replacement for exactly that
 * surface, so a Rust `extern "C"` shim can swap the bodies of those helpers.
 *
 * Conventions:
 *  - Every function returns an int status: QA_OK (0) or a negative QA_E*
 *    code; the message of the last failure on the calling thread is
 *    qa_last_error().  Shapes are validated synchronously, before any launch;
 *    launches are asynchronous on the context's one in-order stream, so an
 *    asynchronous device fault surfaces at qa_sync (as it does at the
 *    reference's poll, src/decoder.rs:1670-1672).
 *  - All strides and sizes are in ELEMENTS (16-bit values).  The reference's
 *    GDims carries bsa/bsb in u32 words but bsc in elements
 *    (src/shaders.rs:1805-1810); a caller converting from GDims doubles
 *    bsa/bsb.
 *  - 16-bit data is little-endian f16 or bf16 bits, the reference's storage
 *    format (src/shaders.rs:27-97, src/half16.rs:22-84).  The format is a
 *    per-call field, not the process-wide setting of src/shaders.rs:99-158.
 *  - A context owns one in-order HIP stream and is not safe for concurrent
 *    calls; separate contexts on separate threads are (the reference records
 *    its dispatches on one thread into one queue, src/align_inference.rs:485).
 */
#ifndef QA_H
#define QA_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define QA_ABI_VERSION 1

typedef struct qa_ctx qa_ctx;

/* Status codes (the reference's anyhow errors, src/decoder.rs:927-950). */
enum {
  QA_OK = 0,
  QA_EINVAL = -1,       /* bad argument or shape                          */
  QA_ENOMEM = -2,       /* device allocation failed                       */
  QA_EDEVICE = -3,      /* no usable device, or a HIP runtime failure      */
  QA_EUNSUPPORTED = -4  /* valid request this build does not implement     */
};

/* 16-bit storage formats (src/shaders.rs:27-40, `Half`). */
enum { QA_F16 = 0, QA_BF16 = 1 };

/* qa_linear_desc.flags */
enum {
  /* C = round(acc + bias + C_old): the `beta = 1` residual form
   * (src/shaders.rs:2067-2072; `gemm_acc`, src/decoder.rs:1602-1608,1652-1657;
   * `gemm_beta`, src/audio_encoder_gpu.rs:1614-1632). */
  QA_ACCUMULATE = 1u << 0,
  /* C = round(gelu(acc + bias)), erf GELU: the GEMM followed by
   * `audio_bias_gelu` (src/audio_encoder_gpu.rs:1594-1602, src/shaders.rs:2599)
   * as one kernel.  Not combinable with QA_ACCUMULATE. */
  QA_EPI_GELU = 1u << 1,
  /* W holds n = 2*inter rows, [gate | up] (src/decoder.rs:1628-1634);
   * C[:, j] = round(silu(round(g_j)) * round(u_j)) for j < n/2: the gate|up GEMM
   * followed by `silu_mul_split` (src/decoder.rs:1636-1650) as one kernel.
   * Not combinable with a bias, QA_ACCUMULATE, QA_EPI_GELU or QA_TRANSB. */
  QA_EPI_SILU_MUL = 1u << 2,
  /* W is read as [k, n] row-major (the conv GEMM's im2col operand,
   * `gemm_conv`, src/audio_encoder_gpu.rs:1714-1721). */
  QA_TRANSB = 1u << 3,
  /* The bias is indexed by output ROW m instead of column: the channel-major
   * conv activation, `audio_bias_gelu` mode 1 (src/shaders.rs:2636-2644,
   * src/audio_encoder_gpu.rs:1777-1790).  Requires a bias. */
  QA_BIAS_ROWS = 1u << 4
};

/* One projection C = A . W^T (+ epilogue).  Replaces a `GDims` uniform plus
 * its bind group and dispatch (src/decoder.rs:1070-1104,
 * src/audio_encoder_gpu.rs:1895-1944).
 *
 *   a    [m, k]  row stride lda            (the activations)
 *   w    [n, k]  row stride ldb            (checkpoint [out, in] layout;
 *                                           [k, n] under QA_TRANSB)
 *   c    [m, n]  row stride ldc            ([m, n/2] under QA_EPI_SILU_MUL)
 *   bias [n] or NULL                       (per output column; [m] per
 *                                           output row under QA_BIAS_ROWS)
 *   batch >= 1 independent problems, element offsets bsa/bsb/bsc apart
 *   (the reference's wgid.z batch, src/shaders.rs:1870-1874).
 *
 * Requirements: k, lda, ldb multiples of 8 (16-byte rows, the reference pads
 * k to 16, src/audio_encoder_gpu.rs:2266-2268); output columns and ldc
 * multiples of 4; n a multiple of 8 under QA_TRANSB or QA_EPI_SILU_MUL;
 * pointers 16-byte aligned (qa_alloc returns 256-byte aligned memory).
 * m may be any value >= 0 (no padding to a tile multiple is needed, unlike
 * the reference's `mp`, src/decoder.rs:907-910). */
typedef struct qa_linear_desc {
  uint32_t dtype; /* QA_F16 / QA_BF16 */
  uint32_t flags; /* QA_ACCUMULATE | QA_EPI_* | QA_TRANSB */
  int64_t m, n, k;
  int64_t lda, ldb, ldc;
  const void* a;
  const void* w;
  void* c;
  const void* bias;
  int64_t batch;
  int64_t bsa, bsb, bsc;
} qa_linear_desc;

/* The decoder MLP block h += down(silu(x.Wg^T) * (x.Wu^T)): the gu GEMM,
 * `silu_mul_split` and the down GEMM of src/decoder.rs:1628-1657 (CPU twin:
 * src/cpu_decoder.rs:495-506).  `act` is caller-owned scratch (the reference's
 * `activated` buffer); h may alias x (out = MLP(x) + x). */
typedef struct qa_mlp_desc {
  uint32_t dtype;
  uint32_t flags;       /* reserved, must be 0 */
  int64_t m, hidden, inter;
  const void* x;        /* [m, hidden]                                 */
  const void* w_gu;     /* [2*inter, hidden]: gate rows, then up rows  */
  const void* w_down;   /* [hidden, inter]                             */
  void* act;            /* [m, inter] scratch                          */
  void* h;              /* [m, hidden] residual, updated in place      */
} qa_mlp_desc;

/* Context: device selection plus one in-order stream.  Replaces Gpu::new_with
 * (src/gpu.rs:475-622) for this path.  Fails with QA_EDEVICE when no device is
 * visible and QA_EUNSUPPORTED when the device is not gfx950. */
int qa_ctx_create(int device, qa_ctx** out);
int qa_ctx_destroy(qa_ctx* ctx);
/* The context's hipStream_t, for callers that record events or capture
 * graphs around qa_* launches (the reference exposes its queue the same way,
 * `gpu.queue`). */
void* qa_ctx_stream(qa_ctx* ctx);

/* Device memory (Gpu::storage, src/gpu.rs:672-682: sizes padded to 16 B,
 * contents zero-filled as wgpu's are). */
int qa_alloc(qa_ctx* ctx, size_t bytes, void** out);
int qa_free(qa_ctx* ctx, void* ptr);
/* Host -> device copy at byte offset `off`; the host bytes are consumed
 * before return (Gpu::upload / write_at, src/gpu.rs:697-705). */
int qa_upload(qa_ctx* ctx, void* dst, size_t off, const void* src, size_t bytes);
/* Device -> host copy; waits for prior work (Gpu::readback, src/gpu.rs:735-762). */
int qa_download(qa_ctx* ctx, void* dst, const void* src, size_t off, size_t bytes);
/* Wait for every launch so far; reports asynchronous faults (Gpu::flush/pump,
 * src/gpu.rs:709-728). */
int qa_sync(qa_ctx* ctx);

/* Launch one projection (see qa_linear_desc). */
int qa_linear(qa_ctx* ctx, const qa_linear_desc* desc);
/* Validate a descriptor without a device or a launch (the size guards of
 * src/decoder.rs:927-950 and src/audio_encoder_gpu.rs:216-245). */
int qa_linear_validate(const qa_linear_desc* desc);
/* qa_linear without any allocation, for callers that cannot call hipMalloc
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * allocation).  No counterpart in the reference.  Same descriptor, kernels
 * and results as qa_linear; where qa_linear would grow its context's
 * workspace for split-K partials, this keeps them in a file-scope device
 * array of qa_linear_noalloc_scratch_floats() f32 (16 MiB), one per GPU,
 * held until the process ends.  The planner never picks a split whose
 * partials exceed it; a split forced larger (QA_SPLITS) is refused with
 * QA_EINVAL.  All calls on one GPU share that GPU's array: calls that overlap
 * on one GPU (contexts whose streams run at the same time) race on it. */
int qa_linear_noalloc(qa_ctx* ctx, const qa_linear_desc* desc);
size_t qa_linear_noalloc_scratch_floats(void);
/* Name `bytes` of device memory at `ptr` -- normally the weights of the
 * projection that follows -- for the NEXT projection launched on this context
 * (qa_linear, qa_linear_noalloc, either GEMM of qa_mlp_fused) to pull from HBM
 * into the memory-side cache while it computes, so the following launch
 * starts on cached weights.  A hint only: results never depend on it, the
 * launch that takes it over clears it, and a hint past what one launch
 * touches (a few tens of MB) is cut short.  No counterpart in the reference;
 * for layer loops that stream a model's weights once per step
 * (src/decoder.rs:1321-1657 runs qkv, o, gate|up, down per layer). */
int qa_prefetch_hint(qa_ctx* ctx, const void* ptr, size_t bytes);
/* Timing hook: the NEXT projection launched on this context (as for
 * qa_prefetch_hint) records the start and the end of its GEMM kernel into
 * these HIP events (hipEvent_t, created by the caller; either may be null),
 * stamped by the kernel's dispatch itself (hipExtLaunchKernel) rather than by
 * event packets queued between kernels, which add a gap of their own.  With
 * K split, the GEMM kernel stamps the start and the split-K reduce kernel
 * after it the end, so the pair spans both.  The launch
 * that takes the events over clears them; under stream capture that launch
 * fails with QA_EINVAL (a captured dispatch does not stamp them on replay).
 * No counterpart in the reference; for per-kernel timing in harnesses
 * (bench.py's per-site figures). */
int qa_time_next_launch(qa_ctx* ctx, void* start_event, void* stop_event);
/* Launch the MLP block (see qa_mlp_desc). */
int qa_mlp_fused(qa_ctx* ctx, const qa_mlp_desc* desc);

/* ---- decoder prefill ops around the projections ----------------------- */

/* y[r] = round(x[r] * inv_r * w), inv_r = 1 / sqrt(mean(x[r]^2) + eps) in
 * f32: the input and post-attention norms.  Replaces the `rms_norm` pipeline
 * dispatch (src/decoder.rs:1305-1319,1610-1626; WGSL src/shaders.rs:331-383;
 * CPU twin `rms_norm_row`, src/cpu_decoder.rs:288-300).  n and the row
 * strides are multiples of 8; x, y 16-byte aligned. */
typedef struct qa_rms_norm_desc {
  uint32_t dtype;
  uint32_t flags; /* reserved, must be 0 */
  int64_t rows, n;
  const void* x;
  int64_t ldx;
  const float* w; /* [n], the norm weight widened to f32 */
  void* y;
  int64_t ldy;
  float eps;
} qa_rms_norm_desc;
int qa_rms_norm(qa_ctx* ctx, const qa_rms_norm_desc* desc);

/* Per-head q / k RMSNorm + rotate-half RoPE and the KV-cache write, for
 * `rows` positions pos0.. of the fused qkv GEMM output: replaces the
 * `qkv_extract` dispatch (src/decoder.rs:1330-1344; WGSL
 * src/shaders.rs:910-1031; CPU twin src/cpu_decoder.rs:302-322,464-491).
 *   qkv     [rows][(nqh + 2 nkvh) hd], row stride ldqkv: q heads, k, v
 *   cos,sin [pos][hd] f32 tables (src/mrope.rs:55-82); row pos0 + r is used
 *   q_out   [nqh][rows][hd]   q heads, normed + roped (head-major)
 *   k_cache [nkvh][cap][hd]   k heads, normed + roped, at rows start..
 *   v_cache [nkvh][hd][cap]   v heads verbatim, TRANSPOSED: key t at column
 *                             t with bits 2 and 3 swapped (each aligned group
 *                             of 16 keys stored 0-3, 8-11, 4-7, 12-15)
 * The V cache is kept transposed (and so ordered) so that qa_attention_prefill's
 * P.V matrix product reads each fragment's keys as one 16-byte run.  hd is a
 * multiple of 64 (<= 256); cap is a multiple of 16; start + rows <= cap. */
typedef struct qa_qk_rope_desc {
  uint32_t dtype;
  uint32_t flags; /* reserved, must be 0 */
  int64_t rows;
  int32_t nqh, nkvh, hd;
  float eps;
  const void* qkv;
  int64_t ldqkv;
  const float* qn_w; /* [hd] */
  const float* kn_w; /* [hd] */
  const float* cos;
  const float* sin;
  int64_t pos0;
  void* q_out;
  void* k_cache;
  void* v_cache;
  int64_t cap, start;
} qa_qk_rope_desc;
int qa_qk_norm_rope(qa_ctx* ctx, const qa_qk_rope_desc* desc);

/* Causal GQA attention for `rows` query positions q0.. (q head h reads kv
 * head h / (nqh / nkvh); row r attends to cache rows 0..q0 + r), softmax of
 * q.k / sqrt(hd) in f32, out[r][h hd + j] = round(sum_t p_t v_t[j]).  Replaces
 * the prefill attention chain repeat_kv -> scores -> softmax -> P.V (-> slab
 * merge) (src/decoder.rs:1346-1600; WGSL src/shaders.rs:2079-2505; CPU twin
 * `attention`, src/cpu_decoder.rs:324-411).  q, k_cache and v_cache are laid
 * out as qa_qk_norm_rope writes them; out is [rows][nqh hd] with row stride
 * ldo, the o projection's input.  hd = 128, nqh / nkvh in {1, 2}; cap is a
 * multiple of 16; q0 + rows <= cap.  Cache entries from q0 + rows up to the
 * next multiple of 64 keys are read (and weighted by zero): they must hold
 * finite values, as qa_alloc's zero-filled memory does.
 * By default the probabilities enter the P.V product as two 16-bit terms
 * (value + rounding residue), so the result tracks the f32 CPU twin; with
 * QA_ATTN_P16 they are rounded once to the 16-bit format, as the reference's
 * GPU path rounds them (its softmax writes 16-bit P for the P.V GEMM,
 * src/shaders.rs:2226-2294; it also rounds the scores, which this kernel keeps
 * in f32) -- faster, up to 2^-11 (f16) / 2^-8 (bf16) relative error per
 * weight. */
enum { QA_ATTN_P16 = 1u << 0 };
typedef struct qa_attention_desc {
  uint32_t dtype;
  uint32_t flags; /* 0 or QA_ATTN_P16 */
  int64_t rows;
  int32_t nqh, nkvh, hd;
  const void* q;
  const void* k_cache;
  const void* v_cache;
  int64_t cap, q0;
  void* out;
  int64_t ldo;
} qa_attention_desc;
int qa_attention_prefill(qa_ctx* ctx, const qa_attention_desc* desc);

/* ---- audio tower ops around the projections ---- */

/* qa_conv_desc.flags */
enum {
  QA_CONV_GELU = 1u << 0,        /* y = gelu(conv + bias), the stem's activation */
  QA_CONV_TOKEN_MAJOR = 1u << 1  /* output rows ordered (b, wo, ho), not (b, ho, wo) */
};
/* One conv level of the audio tower's stem: 3x3 kernel, stride 2, padding 1,
 * + bias (+ erf GELU), f32 accumulation, one rounding per output.  Replaces
 * the im2col + gemm_conv + bias_gelu dispatches of a level
 * (src/audio_encoder_gpu.rs:1165-1201,1714-1794; CPU twin
 * CpuConvStem::conv_block, src/audio_encoder.rs:204-236,376-447).
 *   x      [batch][h][w][c_in]  channel-last (the reference keeps [b][c][h][w];
 *                               channel-last makes each tap's channels one
 *                               contiguous run, so no im2col is materialised)
 *   weight [c_out][ldw], ldw = 9 c_in rounded up to 8 (zero-padded):
 *          k = (kh * 3 + kw) * c_in + ic, i.e. the checkpoint's
 *          [c_out][c_in][3][3] with c_in moved last
 *   bias   [c_out] or NULL
 *   y      [batch * ho * wo][c_out], ho = (h - 1) / 2 + 1, wo = (w - 1) / 2 + 1;
 *          rows (b, ho, wo), or (b, wo, ho) with QA_CONV_TOKEN_MAJOR -- the
 *          layout conv_out reads after the last level: row (b, t) then holds
 *          [f][c], contiguous (the reference's permute,
 *          src/audio_encoder_gpu.rs:1795-1837, becomes a weight permutation).
 * c_in = 1 (the mel input) or a multiple of 8 >= 64; c_out a multiple of 8
 * (<= 1024 when c_in = 1); every operand below 2 GiB. */
typedef struct qa_conv_desc {
  uint32_t dtype;
  uint32_t flags;
  int64_t batch, h, w, c_in, c_out;
  const void* x;
  const void* weight;
  const void* bias;
  void* y;
} qa_conv_desc;
int qa_conv2d_3x3s2(qa_ctx* ctx, const qa_conv_desc* desc);

/* LayerNorm over each row: y = r16((x - mean) / sqrt(var + eps) * w + b),
 * mean and variance in f32 from the 16-bit inputs.  Replaces the
 * `layernorm` dispatches (src/audio_encoder_gpu.rs:1308,1411,1592,1996-2030;
 * WGSL src/shaders.rs:2680-2754; CPU twin CpuAudioLayerNorm::forward,
 * src/audio_encoder.rs:147-171).  n a multiple of 8; w, b f32 [n]. */
typedef struct qa_layer_norm_desc {
  uint32_t dtype;
  uint32_t flags; /* reserved, must be 0 */
  int64_t rows, n;
  const void* x;
  int64_t ldx;
  const float* w;
  const float* b;
  void* y;
  int64_t ldy;
  float eps;
} qa_layer_norm_desc;
int qa_layer_norm(qa_ctx* ctx, const qa_layer_norm_desc* desc);

/* Windowed self-attention of the audio tower: tokens 0..s-1 in windows of
 * wlen (the last holds the remainder); within a window every token attends
 * to every token, softmax of q.k / sqrt(hd) in f32.  Head h reads q, k, v at
 * columns h hd, nh hd + h hd, 2 nh hd + h hd of the fused qkv projection
 * output [s][ldqkv] and writes out[t][h hd + j].  Replaces the reference's
 * extract -> win_pack -> scores -> softmax -> av -> attn_flat chain
 * (src/audio_encoder_gpu.rs:1420-1577; WGSL src/shaders.rs:2756-3086; CPU twin
 * attention_window, src/audio_encoder.rs:517-616).  hd = 64 and
 * wlen <= 128 (QA_EUNSUPPORTED otherwise).  The probabilities enter the
 * P.V product as two 16-bit terms, as in qa_attention_prefill's default. */
typedef struct qa_window_attention_desc {
  uint32_t dtype;
  uint32_t flags; /* reserved, must be 0 */
  int64_t s;
  int32_t nh, hd;
  int64_t wlen;
  const void* qkv;
  int64_t ldqkv;
  void* out;
  int64_t ldo;
} qa_window_attention_desc;
int qa_window_attention(qa_ctx* ctx, const qa_window_attention_desc* desc);

/* y[r][j] = r16(y[r][j] + table[r % period][j]): the sinusoidal position add
 * after conv_out, row r taking its position within its chunk (`add_pe`,
 * src/audio_encoder_gpu.rs:1838-1866; WGSL src/shaders.rs:2957-3000; CPU twin src/audio_encoder.rs:331-343).
 * table f32 [period][n]; n a multiple of 8. */
typedef struct qa_position_add_desc {
  uint32_t dtype;
  uint32_t flags; /* reserved, must be 0 */
  int64_t rows, n;
  void* y;
  int64_t ldy;
  const float* table;
  int64_t period;
} qa_position_add_desc;
int qa_add_position_table(qa_ctx* ctx, const qa_position_add_desc* desc);

/* ---- the aligner's host-side formats, on the device ---- */

/* The slaney mel filterbank [n_mels][n_fft / 2 + 1] (f32, slaney scale and
 * area normalisation, 0 Hz .. sample_rate / 2), create_mel_filterbank
 * (src/mel.rs:100-154).  Host function, no device needed; returns QA_EINVAL
 * on a null output or non-positive sizes. */
int qa_mel_filterbank(int n_mels, int n_fft, int sample_rate, float* out);

/* Log-mel of 16 kHz samples straight into the audio tower's input chunks:
 * centered STFT (n_fft 400, hop 160, periodic Hann, reflect padding), power,
 * the filterbank, log10(max(., 1e-10)), clamp to (clip max - 8), (x + 4) / 4
 * (MelExtractor::extract, src/mel.rs:203-243), frames = n_samples / 160.
 * out [ceil(frames / cs)][n_mels][cs] in the 16-bit format, frames past the
 * last zero (the chunking of encode, src/audio_encoder_gpu.rs:1079-1091).
 * samples and filterbank are device f32 buffers; needs n_samples >= 160
 * (at least one frame) and cs even.  Uses the context's workspace
 * (n_mels * frames floats plus ~8 KB), which grows only outside graph
 * capture. */
typedef struct qa_mel_desc {
  uint32_t dtype;
  uint32_t flags; /* reserved, must be 0 */
  int64_t n_samples;
  const float* samples;
  const float* filterbank;
  int32_t n_mels, cs;
  void* out;
} qa_mel_desc;
int qa_log_mel(qa_ctx* ctx, const qa_mel_desc* desc);

/* RoPE tables for text positions 0..positions-1 (all three M-RoPE axes equal,
 * as the aligner prefills them, src/mrope.rs:55-89 with text_positions):
 * angle(p, j) = p / theta^(2j / hd) in f64, cos / sin rounded to f32 and then
 * to the run's 16-bit format `dtype` (QA_F16 / QA_BF16), as the reference
 * narrows both tables before either decoder reads them
 * (src/align_inference.rs:371-372 on the GPU path, :394-395 on the CPU path,
 * src/cpu_decoder.rs:247); stored widened back to f32 [positions][hd], the
 * second half repeating the first.  The aligner uses theta = 1e6
 * (src/align_inference.rs:322-327).  Host function, no device needed. */
int qa_rope_tables(int64_t positions, int hd, double theta, uint32_t dtype, float* cos_out,
                   float* sin_out);

/* The decoder's input rows: out[r] = table[src[r]] (the token embedding) for
 * src[r] >= 0 and audio[-src[r] - 1] (the audio tower's output row) for
 * src[r] < 0 -- the host gather + scatter of align_raw_rows
 * (src/align_inference.rs:688-714).  An index out of range gives a zero row.
 * src is a device int32 array; hidden a multiple of 8; table, audio and out
 * 16-byte aligned, in the 16-bit format of the decoder. */
typedef struct qa_embed_desc {
  uint32_t dtype;
  uint32_t flags; /* reserved, must be 0 */
  int64_t rows, hidden;
  const int32_t* src;
  const void* table;
  int64_t vocab;
  const void* audio;
  int64_t n_audio;
  void* out;
} qa_embed_desc;
int qa_embed_scatter(qa_ctx* ctx, const qa_embed_desc* desc);

/* The timestamp head (src/align_inference.rs:738-805): for each of `rows`
 * positions p (device int32), the final RMSNorm of h[p] in its folded form,
 * x w / sqrt(sum (x w)^2 / n + eps), then logits = normed . score^T (f32) and
 * classes = the first index of each row's largest logit (the caller
 * multiplies by the segment time, 80 ms).  h [h_rows][ldh] in the 16-bit
 * format; norm_w f32 [n]; score f32 [labels][n]; logits f32 [rows][labels]
 * and classes int32 [rows] are device outputs.  A position out of range
 * gives a zero row.  Uses the context's workspace (rows * n floats). */
typedef struct qa_head_desc {
  uint32_t dtype;
  uint32_t flags; /* reserved, must be 0 */
  int64_t rows;
  const int32_t* positions;
  const void* h;
  int64_t h_rows, ldh, n;
  const float* norm_w;
  float eps;
  const float* score;
  int64_t labels;
  float* logits;
  int32_t* classes;
} qa_head_desc;
int qa_timestamp_head(qa_ctx* ctx, const qa_head_desc* desc);

/* Message of the last failure on this thread ("" if none). */
const char* qa_last_error(void);
/* Library version string, e.g. "qa 0.2.0 (abi 2, gfx950)".  The abi number
 * changes whenever an exported signature changes (abi 2: qa_rope_tables takes
 * the run's 16-bit format before its output pointers); a caller built against
 * another abi must not bind this library. */
const char* qa_version(void);

#ifdef __cplusplus
}
#endif
#endif /* QA_H */
