/*
 * qa_host.h -- C surface of the C++ host mirror (linear_sites.cpp) for the
 * Python harness (tests, bench, smoke).
 *
 * The mirror re-creates, on top of the C ABI in include/qa.h only, what the
 * reference's Rust host does around its GEMM dispatches:
 *   - the text decoder's per-layer projections of WgpuTextDecoder::prefill
 *     (src/decoder.rs:1321-1327 qkv, :1602-1608 o + residual, :1628-1650
 *     gate|up + SiLU, :1652-1657 down + residual) over the fused
 *     [q|k|v] / [gate|up] weights of convert_layer / fused_pieces
 *     (src/decoder.rs:816-871);
 *   - the audio tower's linears of GpuAudioEncoder::layer
 *     (src/audio_encoder_gpu.rs:1414-1419 qkv + bias, :1579-1581 o + bias +
 *     residual, :1594-1602 fc1 + bias + GELU, :1603-1605 fc2 + bias + residual)
 *     and a conv block as an im2col GEMM + bias + GELU
 *     (src/audio_encoder.rs:376-447, the CPU conv block).
 * The projection-only objects (qah_decoder, qah_encoder) take the non-GEMM
 * ops' outputs as fixed synthetic inputs; qah_tdec runs whole decoder layers,
 * norms, RoPE + KV-cache write and attention included
 * (WgpuTextDecoder::prefill's layer loop, src/decoder.rs:1305-1657).
 *
 * It is not part of the product boundary (include/qa.h): a Rust caller keeps
 * its own host code and binds only include/qa.h.
 */
#ifndef QA_HOST_H
#define QA_HOST_H

#include <stddef.h>
#include <stdint.h>

#include "qa.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Seeded synthetic values: SplitMix64 counter stream salted by tensor id,
 * Box-Muller in f64, mean + std*z rounded to f32 then RNE to the 16-bit
 * format.  Deterministic for any thread count. */
void qah_synth_normal_h16(uint64_t seed, uint64_t tensor_id, float mean, float std_dev,
                          int dtype, uint16_t* out, size_t n);
/* Same stream, as f32 values (no 16-bit rounding). */
void qah_synth_normal_f32(uint64_t seed, uint64_t tensor_id, float mean, float std_dev,
                          float* out, size_t n);
/* f32 -> 16-bit RNE narrowing (weights.rs narrow_h16_into, src/weights.rs:57-89). */
void qah_narrow_f32(const float* src, uint16_t* dst, size_t n, int dtype);
/* Rows [rows, cols] of `parts` concatenated along the output dimension
 * (PackedWeight::concat_rows, src/weights.rs:345-360; fused_pieces,
 * src/decoder.rs:840-871). */
void qah_concat_rows(const uint16_t* const* parts, const int64_t* rows, int nparts, int64_t cols,
                     uint16_t* dst);

/* ---- text decoder projections ---- */
typedef struct qah_decoder qah_decoder;
int qah_decoder_create(qa_ctx* ctx, int dtype, int layers, int hidden, int q_dim, int kv_dim,
                       int inter, int max_rows, qah_decoder** out);
/* Uploads layer `li`'s weights, each row-major [out, in]; q|k|v and gate|up
 * are fused into one matrix each, as the reference uploads them. */
int qah_decoder_load_layer(qah_decoder* d, int li, const uint16_t* q, const uint16_t* k,
                           const uint16_t* v, const uint16_t* o, const uint16_t* gate,
                           const uint16_t* up, const uint16_t* down);
/* The non-GEMM ops' outputs the projections read: normed [rows, hidden]
 * (input RMSNorm), attn [rows, q_dim] (attention), norm2 [rows, hidden]
 * (post-attention RMSNorm), and the residual stream h [rows, hidden]. */
int qah_decoder_set_inputs(qah_decoder* d, int rows, const uint16_t* normed,
                           const uint16_t* attn, const uint16_t* norm2, const uint16_t* h);
/* Enqueue every layer's four projections (no wait). */
int qah_decoder_prefill_linears(qah_decoder* d, int rows);
/* Enqueue layer `li`'s four projections alone, with the same prefetch hints
 * as in the whole pass (its down launch pulls layer li + 1's qkv weights). */
int qah_decoder_layer(qah_decoder* d, int li, int rows);
/* Copy back: which = 0 h [rows, hidden], 1 qkv [rows, q+2kv] of the last
 * layer run, 2 act [rows, inter] of the last layer run. */
int qah_decoder_read(qah_decoder* d, int which, int rows, uint16_t* host);
/* Time `steps` forward passes after `warmup`: HIP events on the context's
 * stream (ms_per_step) and the host clock from the first launch to the
 * completed synchronize (wall_ms_per_step, may be NULL).  use_graph = 1
 * replays one captured hipGraph per step. */
int qah_decoder_time(qah_decoder* d, int rows, int warmup, int steps, int use_graph,
                     double* ms_per_step, double* wall_ms_per_step);
/* Per-site average kernel duration (ms) over `steps` eager passes, each GEMM
 * kernel stamping its own start / end events at dispatch (qa_time_next_launch):
 * site_ms[0..3] = qkv, o, gu, down. */
int qah_decoder_profile_sites(qah_decoder* d, int rows, int steps, double* site_ms);
void qah_decoder_destroy(qah_decoder* d);

/* ---- audio tower linears ---- */
typedef struct qah_encoder qah_encoder;
int qah_encoder_create(qa_ctx* ctx, int dtype, int layers, int d_model, int ffn, int conv_k,
                       int max_rows, qah_encoder** out);
/* Layer li: qkv_w [3d, d] (fused q|k|v rows, src/audio_encoder_gpu.rs:292-313)
 * with qkv_b [3d]; o_w [d, d], o_b [d]; fc1_w [ffn, d], fc1_b [ffn];
 * fc2_w [d, ffn], fc2_b [d]. */
int qah_encoder_load_layer(qah_encoder* e, int li, const uint16_t* qkv_w, const uint16_t* qkv_b,
                           const uint16_t* o_w, const uint16_t* o_b, const uint16_t* fc1_w,
                           const uint16_t* fc1_b, const uint16_t* fc2_w, const uint16_t* fc2_b);
/* The conv block as a GEMM: w [d, conv_k] (conv weight flattened to im2col k
 * order, src/audio_encoder_gpu.rs:262-285), b [d]. */
int qah_encoder_load_conv(qah_encoder* e, const uint16_t* w, const uint16_t* b);
/* col [rows, conv_k] im2col operand; normed [rows, d] (LayerNorm 1 output);
 * attn [rows, d] (attention output); norm2 [rows, d] (LayerNorm 2 output);
 * h [rows, d] residual stream. */
int qah_encoder_set_inputs(qah_encoder* e, int rows, const uint16_t* col, const uint16_t* normed,
                           const uint16_t* attn, const uint16_t* norm2, const uint16_t* h);
/* conv GEMM (+bias+GELU) into `conv_out`, then every layer's 4 linears. */
int qah_encoder_forward_linears(qah_encoder* e, int rows);
/* which = 0 h [rows, d], 1 conv_out [rows, d], 2 qkv [rows, 3d] and
 * 3 act [rows, ffn] of the last layer run. */
int qah_encoder_read(qah_encoder* e, int which, int rows, uint16_t* host);
int qah_encoder_time(qah_encoder* e, int rows, int warmup, int steps, int use_graph,
                     double* ms_per_step, double* wall_ms_per_step);
/* The same per GEMM site of the tower (qa_time_next_launch stamps):
 * site_ms[0..4] = conv, qkv, o, fc1, fc2 */
int qah_encoder_profile_sites(qah_encoder* e, int rows, int steps, double* site_ms);
void qah_encoder_destroy(qah_encoder* e);

/* ---- whole text-decoder layers (decoder_prefill.cpp) ---- */
typedef struct qah_tdec qah_tdec;
/* Qwen3 decoder: hidden, nqh x hd query heads over nkvh kv heads, SwiGLU MLP
 * of width inter; RMSNorm epsilon eps; up to max_rows positions. */
int qah_tdec_create(qa_ctx* ctx, int dtype, int layers, int hidden, int nqh, int nkvh, int hd,
                    int inter, int max_rows, float eps, qah_tdec** out);
/* Layer li: the seven projections as qah_decoder_load_layer, plus f32 norm
 * weights iln, pln [hidden] (input / post-attention RMSNorm) and qn, kn [hd]
 * (q / k head RMSNorm). */
int qah_tdec_load_layer(qah_tdec* t, int li, const uint16_t* q, const uint16_t* k,
                        const uint16_t* v, const uint16_t* o, const uint16_t* gate,
                        const uint16_t* up, const uint16_t* down, const float* iln,
                        const float* pln, const float* qn, const float* kn);
/* RoPE tables cos / sin [positions][hd] (src/mrope.rs:55-82); a prefill of
 * `rows` positions needs positions >= rows. */
int qah_tdec_set_rope(qah_tdec* t, const float* cos, const float* sin, int positions);
/* qa_attention_desc.flags used by the layers' attention (0 or QA_ATTN_P16). */
int qah_tdec_set_attention_flags(qah_tdec* t, uint32_t flags);
/* The residual stream h [rows, hidden] the first layer reads. */
int qah_tdec_set_hidden(qah_tdec* t, int rows, const uint16_t* h);
/* Enqueue every layer over positions 0..rows-1 (no wait); h is updated in place. */
int qah_tdec_prefill(qah_tdec* t, int rows);
/* which = 0 h [rows, hidden], 1 attn [rows, nqh hd], 2 qkv [rows, (nqh + 2 nkvh) hd],
 * 3 act [rows, inter], 4 normed, 5 norm2 [rows, hidden], 6 q heads [nqh, rows, hd]
 * of the last layer run; 7 K cache [nkvh, cap, hd] and 8 V cache (transposed,
 * [nkvh, hd, cap]) of the last layer, cap = max_rows rounded up to 64. */
int qah_tdec_read(qah_tdec* t, int which, int rows, uint16_t* host);
int qah_tdec_time(qah_tdec* t, int rows, int warmup, int steps, int use_graph,
                  double* ms_per_step, double* wall_ms_per_step);
/* Average ms per layer of each op over `steps` prefills, every launch
 * bracketed by its own HIP events: op_ms[0..7] = rms_norm, qkv, qk_norm_rope,
 * attention, o, rms_norm 2, gate|up, down. */
int qah_tdec_profile_ops(qah_tdec* t, int rows, int steps, double* op_ms);
void qah_tdec_destroy(qah_tdec* t);

/* ---- the whole audio tower (audio_encoder.cpp) ---- */
typedef struct qah_aenc qah_aenc;
/* Qwen3-ASR audio tower (GpuAudioEncoder::encode, src/audio_encoder_gpu.rs:
 * 1060-1347): n_mels bins in chunks of cs frames, conv stem of c_conv
 * channels, `layers` transformer layers of d_model = nh x 64 with an ffn-wide
 * GELU MLP, windows of wlen tokens, projector to out_dim; up to max_chunks
 * chunks. */
int qah_aenc_create(qa_ctx* ctx, int dtype, int layers, int n_mels, int cs, int c_conv,
                    int d_model, int nh, int ffn, int out_dim, int wlen, int max_chunks,
                    qah_aenc** out);
/* Conv level 0..2: weight in the checkpoint's [c_out][c_in][3][3] layout, bias [c_out]. */
int qah_aenc_load_conv(qah_aenc* a, int level, const uint16_t* w, const uint16_t* b);
/* conv_out: weight [d_model][c_conv * f] in the checkpoint's (c, f) column order. */
int qah_aenc_load_conv_out(qah_aenc* a, const uint16_t* w, const uint16_t* b);
/* Layer li: LayerNorm weights / biases f32 [d_model]; qkv_w [3 d_model][d_model]
 * (fused q|k|v rows) + qkv_b; o; fc1 [ffn][d_model]; fc2 [d_model][ffn]. */
int qah_aenc_load_layer(qah_aenc* a, int li, const float* ln1_w, const float* ln1_b,
                        const uint16_t* qkv_w, const uint16_t* qkv_b, const uint16_t* o_w,
                        const uint16_t* o_b, const float* ln2_w, const float* ln2_b,
                        const uint16_t* fc1_w, const uint16_t* fc1_b, const uint16_t* fc2_w,
                        const uint16_t* fc2_b);
/* ln_post (f32), proj1 [d_model][d_model], proj2 [out_dim][d_model], with biases. */
int qah_aenc_load_post(qah_aenc* a, const float* ln_w, const float* ln_b, const uint16_t* p1_w,
                       const uint16_t* p1_b, const uint16_t* p2_w, const uint16_t* p2_b);
/* Mel chunks [n_chunks][n_mels][cs] (the last zero-padded past its frames). */
int qah_aenc_set_mel(qah_aenc* a, int n_chunks, const uint16_t* mel);
/* Tokens of n_chunks chunks whose last has tail_frames frames (0 = full). */
int64_t qah_aenc_tokens(qah_aenc* a, int n_chunks, int tail_frames);
/* Enqueue the whole tower (no wait). */
int qah_aenc_forward(qah_aenc* a, int n_chunks, int tail_frames);
/* which = 0 out [rows, out_dim], 1 h [rows, d_model] (the residual stream
 * after the last layer), 2 conv1 / 3 conv2 output rows [rows, c_conv],
 * 4 conv_out operand [rows, c_conv * f], 5 the last LayerNorm output
 * [rows, d_model], 6 qkv [rows, 3 d_model], 7 attention [rows, d_model],
 * 8 fc1 activation [rows, ffn], 9 proj1 activation [rows, d_model]. */
int qah_aenc_read(qah_aenc* a, int which, int64_t rows, uint16_t* host);
int qah_aenc_time(qah_aenc* a, int n_chunks, int tail_frames, int warmup, int steps,
                  int use_graph, double* ms_per_step, double* wall_ms_per_step);
/* Event-bracketed ms over `steps` forwards: ms[0..2] conv levels, 3 conv_out +
 * position add, 4..10 the layer ops summed over all layers (LayerNorm, qkv,
 * attention, out_proj, LayerNorm 2, fc1, fc2), 11 ln_post + projector. */
int qah_aenc_profile(qah_aenc* a, int n_chunks, int tail_frames, int steps, double* ms);
void qah_aenc_destroy(qah_aenc* a);

/* The aligner's forward pass (Aligner::align_raw_rows,
 * src/align_inference.rs:646-805): samples -> log-mel -> the encoder `enc`
 * -> embedding gather + audio scatter -> the decoder `dec` -> timestamp head,
 * then fix_timestamps on the host.  enc and dec stay owned by the caller and
 * must outlive the aligner. */
typedef struct qah_aligner qah_aligner;
/* The timestamp repair alone (src/postprocess.rs:33-111); out may not alias data. */
void qah_fix_timestamps(const int64_t* data, int64_t n, int64_t* out);
int qah_aligner_create(qa_ctx* ctx, qah_aenc* enc, qah_tdec* dec, int64_t vocab, int64_t labels,
                       double segment_ms, int64_t max_samples, qah_aligner** out);
/* Token embedding [vocab][hidden] in the decoder's 16-bit format. */
int qah_aligner_load_embed(qah_aligner* h, const uint16_t* table);
/* Final RMSNorm weight f32 [hidden] and score head f32 [labels][hidden]. */
int qah_aligner_load_head(qah_aligner* h, const float* norm_w, const float* score);
/* Assemble and upload one input: f32 samples at 16 kHz, and n_words words
 * given as token ids (word_lens[w] ids each, concatenated in word_ids).
 * info (optional, 5 entries): sequence length, audio tokens, timestamp
 * slots, mel chunks, frames in the last chunk (0 = full). */
int qah_aligner_prepare(qah_aligner* h, const float* samples, int64_t n_samples, int n_words,
                        const int32_t* word_lens, const int32_t* word_ids, int64_t* info);
/* Enqueue the device pass (no wait). */
int qah_aligner_forward(qah_aligner* h);
/* Classes -> raw ms (class x segment) and repaired ms, 2 per word. */
int qah_aligner_result(qah_aligner* h, int64_t* raw_ms, int64_t* fixed_ms);
/* which = 0 classes int32 [slots], 1 logits f32 [slots][labels], 2 input ids
 * int32 [seq], 3 timestamp positions int32 [slots], 4 row sources int32
 * [seq] (token id, or -1 - k for audio row k). */
int qah_aligner_read(qah_aligner* h, int which, void* host);
int qah_aligner_time(qah_aligner* h, int warmup, int steps, int use_graph, double* ms_per_step,
                     double* wall_ms_per_step);
/* Event-bracketed ms over `steps` forwards: mel, tower, scatter, prefill, head. */
int qah_aligner_profile(qah_aligner* h, int steps, double* ms);
void qah_aligner_destroy(qah_aligner* h);

/* ---- the real-checkpoint loader (checkpoint.cpp) ---- */
/* A Qwen3-ForcedAligner checkpoint directory (src/weights.rs:207-290):
 * model.safetensors, or model.safetensors.index.json and its shards, mapped
 * read-only; tensor names of the `-hf` conversion are mapped onto the
 * original ones (model.language_model. -> thinker.model., model.audio_tower.
 * -> thinker.audio_tower., model.multi_modal_projector.linear_{1,2} ->
 * thinker.audio_tower.proj{1,2}, thinker.lm_head. -> score.). */
typedef struct qah_ckpt qah_ckpt;
/* The dimensions config.json records, in its original (thinker_config) or
 * `-hf` (audio_config / text_config) layout, with the reference's defaults
 * for absent fields (src/config.rs:36-150,186-235). */
typedef struct qah_ckpt_config {
  int64_t vocab, hidden, inter, layers, nqh, nkvh, hd;
  double rms_eps, rope_theta;
  int64_t d_model, enc_layers, enc_heads, enc_ffn, n_mels, c_conv, n_window, n_window_infer,
      out_dim;
  int64_t num_labels, timestamp_token_id, audio_start, audio_end, audio_token;
  double segment_ms;
} qah_ckpt_config;
int qah_ckpt_open(const char* dir, qah_ckpt** out);
/* The message of the last failing qah_ckpt_* call on this thread. */
const char* qah_ckpt_error(void);
/* Tensor metadata: dtype 0 f16, 1 bf16, 2 f32, 3 other; up to 8 dims. */
int qah_ckpt_tensor(qah_ckpt* c, const char* name, int* dtype, int* ndim, int64_t* shape);
/* The tensor converted to QA_F16 / QA_BF16 (round to nearest even; a copy
 * when it is stored so) or to f32; elems must equal its element count. */
int qah_ckpt_read_h16(qah_ckpt* c, const char* name, int dtype, uint16_t* dst, int64_t elems);
int qah_ckpt_read_f32(qah_ckpt* c, const char* name, float* dst, int64_t elems);
int qah_ckpt_read_config(qah_ckpt* c, qah_ckpt_config* out);
/* Build the aligner from the checkpoint: an audio tower sized for
 * max_seconds of audio, a decoder of max_rows positions (RoPE tables of
 * config.json's theta), the embedding and the head.  Linear and conv
 * weights go to the run's 16-bit format; the decoder's and the tower's norm
 * weights are rounded to it too (src/decoder.rs:823-826,
 * src/audio_encoder_gpu.rs:330-331); the final norm and the score head stay
 * f32 (src/align_inference.rs:405-430).  Absent linear biases read as zero.
 * On success the caller owns all three (destroy the aligner first). */
int qah_ckpt_load_aligner(qah_ckpt* c, qa_ctx* ctx, int dtype, double max_seconds, int max_rows,
                          qah_aenc** enc, qah_tdec** dec, qah_aligner** al);
/* The tower geometry load_aligner uses for config.json and max_seconds:
 * out[0] frames per chunk (2 n_window), out[1] the attention window in tokens
 * (feo(cs) * (n_window_infer / cs), src/audio_encoder.rs:807-810), out[2] mel
 * rows after the stem, out[3] chunks for max_seconds.  QA_EINVAL /
 * QA_EUNSUPPORTED for a geometry the kernels cannot run (n_window,
 * n_mels or n_window_infer not positive, a window shorter than a chunk,
 * decoder heads not 128 wide, a GQA ratio above 2). */
int qah_ckpt_geometry(qah_ckpt* c, double max_seconds, int64_t* out);
void qah_ckpt_close(qah_ckpt* c);

/* Time `iters` back-to-back launches of one descriptor (HIP events around the
 * whole run on the context's stream); ms per launch. */
int qah_time_linear(qa_ctx* ctx, const qa_linear_desc* desc, int warmup, int iters,
                    double* ms_per_launch);

/* `iters` back-to-back launches cycling through descs[0..ndesc), an event
 * recorded before each launch and after the last on the context's stream:
 * ms_each[i] is launch i's duration including its share of the launch gap
 * (the per-launch figures whose median / p10 / p90 the benchmark reports). */
int qah_time_linears_each(qa_ctx* ctx, const qa_linear_desc* descs, int ndesc, int warmup,
                          int iters, float* ms_each);

/* Checks the f16 SiLU.up epilogue's packed arithmetic (silu_mul_f16x2 in
 * qa_internal.h) on the device against silu_mul in f32 followed by a separate
 * round-to-nearest-even to f16, on 2 * pairs inputs generated from `seed`
 * (special values, random f32 bit patterns, values in [-16, 16)):
 * *mismatches = outputs that differ (two NaNs count as equal). */
int qah_check_silu_f16x2(qa_ctx* ctx, int64_t pairs, uint64_t seed, int64_t* mismatches);

/* The same launches, each timed by its own kernels' dispatches
 * (qa_time_next_launch): ms_each[i] is launch i's kernel time alone, from
 * the GEMM's start to its end (to the split-K reduce's end when K is split),
 * without the gap between launches. */
int qah_time_linears_stamped(qa_ctx* ctx, const qa_linear_desc* descs, int ndesc, int warmup,
                             int iters, float* ms_each);

/* A plain 16-byte-per-thread copy of `bytes` between two fresh buffers,
 * `reps` times: the known-size reference that calibrates the FETCH_SIZE /
 * WRITE_SIZE counters. */
int qah_copy_calibration(qa_ctx* ctx, size_t bytes, int reps);

#ifdef __cplusplus
}
#endif
#endif
