/*
 * wavo_hip.h — the C ABI of the MI355X (gfx950) backend for wavo's encoder/decoder compute path.
 *
 * The entry points mirror wavo's crate-internal GPU operator API one to one (src/gpu/mod.rs: `Gpu`,
 * `Linear`, `Channels`, `Epilogue`, `Pass`), so that a Rust `src/gpu/hip.rs` binds them through a
 * thin `extern "C"` block.  Each declaration cites the reference interface it
 * replaces.  Plain pointers and sizes only: no HIP or torch types cross this boundary.
 *
 * Conventions
 *  - Every entry returns 0 on success or a negative WH_E* code; wh_last_error(ctx) gives the text
 *    that the Rust side turns into Error::Gpu (device failures) or Error::Model (shapes/arguments).
 *  - Device pointers come from wh_alloc().  Activations are f32 row-major [rows][cols], as in the
 *    reference.  Ops are queued on the context's stream in call order (the reference records them
 *    into one compute pass); wh_sync()/wh_read() wait for them and report deferred device errors,
 *    as Gpu::run's final poll does (src/gpu/mod.rs:969-1002).
 *  - A context is not internally synchronized (the reference serializes calls with Gpu::busy,
 *    src/gpu/mod.rs:232-233): one thread at a time per context.
 */
#ifndef WAVO_HIP_H
#define WAVO_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Error codes.  WH_EARG ≙ Error::Model (bad shape or argument, not fatal); WH_EGPU and WH_EOOM ≙
 * Error::Gpu (Error::is_fatal, src/error.rs:129-140: the caller reloads). */
#define WH_OK 0
#define WH_EARG (-1)
#define WH_EGPU (-2)
#define WH_EOOM (-3)

/* ggml tensor types of GGUF weights (src/gguf.rs:14-38, plus ggml's Q4_0 = 2). */
#define WH_F32 0
#define WH_F16 1
#define WH_Q4_0 2
#define WH_Q8_0 8

/* Epilogue modes, equal to Epilogue::params (src/gpu/mod.rs:430-456). */
#define WH_BIAS 0
#define WH_SILU 1
#define WH_RELU 2
#define WH_RESIDUAL 3 /* c += alpha * v */
#define WH_GELU 4
#define WH_GELU_RESIDUAL 5
#define WH_TANH 6

typedef struct wh_ctx wh_ctx;
typedef struct wh_linear wh_linear;
typedef struct wh_model wh_model;

/* ------------------------------------------------------------------------- device and memory */

/* Gpu::new(fast, index) (src/gpu/mod.rs:461).  device_index < 0 picks device 0. */
int wh_open(int device_index, wh_ctx **out);
/* Drop for Gpu. */
void wh_close(wh_ctx *ctx);
/* The message of the last failed call on ctx (or of the last failed wh_open when ctx is NULL). */
const char *wh_last_error(const wh_ctx *ctx);
/* Gpu::info / Device (src/gpu/mod.rs:580, :30-46): name, compute units, wavefront size. */
int wh_device_info(wh_ctx *ctx, char *name, size_t name_len, int *compute_units, int *wave);
/* Gpu::buffer / readback (src/gpu/mod.rs:675-697): n_f32 floats of device memory, uninitialized. */
int wh_alloc(wh_ctx *ctx, size_t n_f32, float **dptr);
int wh_free(wh_ctx *ctx, void *dptr);
/* Page-locked host memory for wh_write / wh_read (the DMA engines copy it without a bounce buffer):
 * the counterpart of the mapped staging and readback buffers of Gpu::write and Gpu::run
 * (src/gpu/mod.rs:687-697, :741-750, :969-1002).  wh_host_free waits for the queued work first. */
int wh_host_alloc(wh_ctx *ctx, size_t bytes, void **host);
int wh_host_free(wh_ctx *ctx, void *host);
/* Gpu::write / upload (src/gpu/mod.rs:741-750): bytes from host memory, complete on return. */
int wh_write(wh_ctx *ctx, void *dst, const void *src, size_t bytes);
/* Device-to-device copy on the stream. */
int wh_copy(wh_ctx *ctx, void *dst, const void *src, size_t bytes);
/* Zero `bytes` of device memory with a fill kernel (safe inside stream capture). */
int wh_zero(wh_ctx *ctx, void *dst, size_t bytes);
/* The readback of Gpu::run / finish (src/gpu/mod.rs:969-1002): waits for the queued work, reports
 * deferred device errors, then copies `bytes` from device memory to host memory. */
int wh_read(wh_ctx *ctx, void *host, const void *dptr, size_t bytes);
/* Waits for the queued work; reports deferred device errors (Gpu::complete's poll). */
int wh_sync(wh_ctx *ctx);
/* The context's hipStream_t as an opaque pointer, for callers that time with HIP events. */
void *wh_stream(wh_ctx *ctx);
/* Tuning and measurement overrides (no counterpart in the reference, whose kernel choices are fixed
 * per device tier, src/gpu/mod.rs:50-107).  Only an explicit call changes them; a fresh context
 * chooses every launch plan itself.  Keys:
 *   "gemm_plan"        "bm,bn,wm,wn,slots,split[,pipeline[,kgroups]]" for every GEMM of the main kernel
 *                      ("" clears);
 *   "gemm_shape_plans" "m,cols,k:bm,bn,wm,wn,slots,split[,pipeline[,kgroups]];..." per call shape ("" clears);
 *   "gemm_kernel_only" "1": a k-split GEMM call stops after its GEMM kernel and leaves c unwritten
 *                      (to time that kernel alone, as a model step runs it); "0" restores;
 *   "gemm_group"       "n": the GEMM's XCDs take tiles in groups of n row tiles, column by column inside a
 *                      group (0 = chosen per plan; the output is the same bit for bit);
 *   "attn_split"       "n": attention splits its key range n ways (0 = chosen per shape);
 *   "position_cache"   "0": the Parakeet encoder recomputes its relative-position projection every call
 *                      instead of keeping it for the frame count its buffer holds (to time it); "1" restores;
 *   "mel_raw"          "1": wh_model_mel writes each filter's sum before the logarithm, without the
 *                      normalization or scaling (to check the transforms bit for bit); "0" restores;
 *   "whisper_host"     "1": wh_whisper_decode reads every step's logits back and picks on the host
 *                      (wh_whisper_pick), the check of its device search; "0" restores;
 *   "whisper_logprobs" "1": wh_whisper_decode sums the log-probabilities whatever the no-speech
 *                      probability (to check them); "0" restores;
 *   "attend_merge"     "1": wh_attend merges its 256-key parts in the launch's last workgroup (the
 *                      path of a decoder step's self-attention) instead of a second kernel; "0" restores;
 *   "epilogue_fusion"  "0": the encoders run in launches of their own what GEMM epilogues do otherwise
 *                      (attention's packed K, Vᵀ and position rows for one window, as the padded-batch
 *                      path does; the Parakeet subsampling's flatten; the conv module's GLU), the check
 *                      of those epilogues; "1" restores.
 * Unknown keys and malformed values return WH_EARG. */
int wh_tune(wh_ctx *ctx, const char *key, const char *value);
/* Profiling (no counterpart in the reference, whose timing lives in `wavo bench` and GPU timestamp
 * queries, docs/perf.md:54).  mode 1: every kernel launch gets HIP events on the stream around it
 * (each pair adds the event's own overhead, a few microseconds, to what it measures); mode 2: only
 * the regions bracketed by wh_region.  wh_profile_read waits, then writes JSON text: per kernel
 * variant or region name its count, total milliseconds and algorithmic flops and bytes.  Setting
 * the mode clears the records. */
int wh_profile(wh_ctx *ctx, int mode);
int wh_profile_read(wh_ctx *ctx, char *out, size_t len);
/* Begins (name != NULL) or ends (name == NULL, with the region's algorithmic flops and bytes) a
 * timed region: HIP events on the stream around whatever is queued in between. */
int wh_region(wh_ctx *ctx, const char *name, double flops, double bytes);

/* ----------------------------------------------------------------------- recorded passes */

/* Gpu::record / finish (src/gpu/mod.rs:922-943): the ops queued on ctx between wh_record_begin and
 * wh_record_end are recorded, not run, into a pass (a HIP graph); wh_replay queues the whole pass
 * again, with the buffers and arguments it was recorded with, as often as asked.  Nothing may
 * allocate while recording: an op that would grow the context's scratch fails (run it once first),
 * and wh_replay refuses a pass recorded before the scratch moved.  Profiling must be off.  Free a
 * pass before its context. */
typedef struct wh_pass wh_pass;
int wh_record_begin(wh_ctx *ctx);
int wh_record_end(wh_ctx *ctx, wh_pass **out);
int wh_replay(wh_ctx *ctx, const wh_pass *pass);
void wh_pass_free(wh_pass *pass);

/* -------------------------------------------------------------------------------- weights */

/* One GGUF weight tensor [rows][k] in its file bytes (ggml dims [k, rows], dims[0] contiguous:
 * src/gguf.rs:109-111), type WH_F32/F16/Q4_0/Q8_0. */
typedef struct wh_tensor {
  const void *data;
  int type;
  int k;
  int rows;
} wh_tensor;

/* Gpu::linear (src/gpu/mod.rs:758) and, with pad_k != 0, Gpu::conv (:766): the tensors stacked
 * along n, kept on the device in their GGUF bytes (Q8_0 34-byte / Q4_0 18-byte blocks as stored),
 * with the bias of the stacked rows (n_bias == 0: zeros).  A bias with `dual` more values than the
 * rows writes the first `dual` outputs again after the others with those biases (upload_linear,
 * :770-834).  k % 32 == 0 unless pad_k, which pads k to 32 with zero columns in F32 (exact, as the
 * GEMM rounds W to f16 either way). */
int wh_linear_new(wh_ctx *ctx, const wh_tensor *ws, int count, const float *bias, int n_bias,
                  int pad_k, wh_linear **out);
/* Linear::width (src/gpu/mod.rs:406-412): output columns per row of c, `cols + dual`, where cols =
 * rows when rows % 32 == 0, else rows rounded up to 64. */
int wh_linear_width(const wh_linear *l);
/* The (padded) k the layer takes, and its weight type. */
int wh_linear_k(const wh_linear *l);
int wh_linear_type(const wh_linear *l);
void wh_linear_free(wh_ctx *ctx, wh_linear *l);

/* --------------------------------------------------------------------------------- Pass ops */

/* Pass::gemm (src/gpu/mod.rs:1394-1426): c = epi(h(a)·h(W)ᵀ + b) for m rows of a [m][k], h =
 * round-to-f16, f32 accumulation; rows of c are wh_linear_width() wide; columns rows..cols get
 * epi(0); dual columns get acc + bias with no epilogue.  Residual modes read c. */
int wh_gemm(wh_ctx *ctx, const float *a, const wh_linear *l, float *c, int m, int epi,
            float alpha);
/* wh_gemm with `a` already rounded to f16 (a16: m rows of k halves) and, with out16 != 0, f16
 * outputs (not for the residual epilogues, which accumulate into f32): the form the graph drivers
 * use between ops whose consumer is a GEMM.  No counterpart in the reference, whose GEMM reads f32
 * and rounds it (gemm.wgsl:1-9). */
int wh_gemm_h(wh_ctx *ctx, const void *a16, const wh_linear *l, void *c, int m, int epi,
              float alpha, int out16);
/* wh_gemm that allocates nothing: no counterpart in the reference.  For callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * The same kernels and results as wh_gemm; the f16 copy of `a` and the split-k partial sums go to a
 * fixed workspace of wh_gemm_noalloc_limit() bytes (32 MiB) that each device holds for the life of
 * the process, instead of the context's growable scratch.  A call whose workspace would exceed it
 * returns WH_EARG without launching.  Calls on one device share the workspace, so callers must
 * serialize them: a call from another stream (or context) while the device's previous call may still
 * be running is refused with WH_EARG (calls under stream capture are not checked; their replays must
 * not overlap either).  Not while per-launch profiling (wh_profile 1) is on. */
int wh_gemm_noalloc(wh_ctx *ctx, const float *a, const wh_linear *l, float *c, int m, int epi, float alpha);
size_t wh_gemm_noalloc_limit(void);
/* Pass::gemv (src/gpu/mod.rs:1461-1467): c[offset + j] = epi(a·W[j] + b[j]) for one row a, W not
 * rounded. */
int wh_gemv(wh_ctx *ctx, const float *a, const wh_linear *l, float *c, int epi, float alpha,
            int offset);
/* Pass::embed (src/gpu/mod.rs:1469-1482): c = W[ids[i]] + pos[offset..] + b, k values. */
int wh_embed(wh_ctx *ctx, const wh_linear *l, const float *pos, float *c, const uint32_t *ids,
             int i, int offset);
/* Pass::layer_norm (src/gpu/mod.rs:1428-1446): LayerNorm (eps 1e-5) of rows x [rows][cols] with
 * gain g and bias b into y; with table != NULL also into yr with RoPE (NEOX split-half per head of
 * head_dim; table [rows][cos(hd/2) | sin(hd/2)]).  Pass::layer_norm_row is rows = 1. */
int wh_layer_norm(wh_ctx *ctx, const float *x, const float *g, const float *b, float *y, int rows,
                  int cols, const float *table, float *yr, int head_dim);
/* Pass::attend (src/gpu/mod.rs:1484-1505): one query per head q [heads·hd] over keys 0..n of an f16
 * cache of `cols` positions (wh_pack's layout) into o, through `part` (wh_attend_len floats). */
int wh_attend(wh_ctx *ctx, const float *q, const uint32_t *kv, float *part, float *o, int n,
              int cols, int heads, int hd);
size_t wh_attend_len(int n, int heads, int hd); /* attend_len (src/gpu/mod.rs:1045-1049) */
/* Pass::pack (src/gpu/mod.rs:1507-1523): rows of x (from float src, stride floats apart, each K
 * then V of d floats) into the f16 cache y of cols positions at positions col..: K transposed (pair
 * i of position j at word i·cols + j), then V by position (word d/2·cols + j·d/2 + i). */
int wh_pack(wh_ctx *ctx, const float *x, int src, int stride, uint32_t *y, int rows, int d,
            int cols, int col);
/* Pass::im2col (src/gpu/mod.rs:1525-1533): columns col[i][c·kernel + k] = x[stride·i + k − pad][c],
 * rows padded with zeros to a multiple of 32. */
int wh_im2col(wh_ctx *ctx, const float *x, float *col, int t, int ch, int kernel, int stride,
              int pad);
/* Pass::conv_glu (src/gpu/mod.rs:1535-1557): GLU of h [t][2ch], depthwise conv (odd kernel,
 * centred; taps dw_w [ch][kernel] + dw_b), LayerNorm (layer_norm != 0) or affine x·g + b, SiLU,
 * into y [t][ch].  `valid` (< t) zeroes the GLU output of frames >= valid first (a padded window's
 * frame mask, src/ane/conformer.rs:301-309); valid >= t is unmasked.  ch % 4 == 0, ch <= 1024,
 * kernel <= 31, 16-byte aligned buffers. */
int wh_conv_glu(wh_ctx *ctx, const float *h, const float *dw_w, const float *dw_b, int kernel,
                const float *g, const float *b, int layer_norm, float *y, int t, int ch,
                int valid);
/* Pass::attention (src/gpu/mod.rs:1559-1601): multi-head attention, scale 1/√head_dim, into o
 * [t][heads·hd]:
 *   v != NULL, pos == NULL: qk [t][q | k], v [t][heads·hd]            (rotary, GigaAM)
 *   v == NULL, pos == NULL: qk [t][q | k | v]                          (Whisper)
 *   v == NULL, pos != NULL: qk [t][q + u | k | v | q + v], pos [2t + 15][heads·hd] (row r is
 *     position t + 15 − r); score (i, j) = ((q+u)_i·k_j + (q+v)_i·pos[j − i + t + 15]) / √hd.
 * `valid` (< t) masks keys >= valid (additive key mask, src/ane/mod.rs:463-466).  The products
 * use f16 operands with f32 accumulation and softmax, as the reference's f16 flash tier. */
int wh_attention(wh_ctx *ctx, const float *qk, const float *v, const float *pos, float *o, int t,
                 int heads, int hd, int valid);
/* Pass::depthwise (src/gpu/mod.rs:1603-1630): 3×3 stride-2 pad-1 depthwise conv + bias (w [9][ch])
 * over the image [t][f][ch] into output rows t0..t0+rows of y; x holds the image's rows from
 * 2·t0 − 1.  With first_w (the first conv, 1 → ch, + first_b, then ReLU, never stored) x is the
 * one-channel image [t][f] and y gets `rows` rows of [⌈f/4⌉][ch] from output row 2·t0 − 1, rows
 * from ⌈t/4⌉ on zero. */
int wh_depthwise(wh_ctx *ctx, const float *x, const float *first_w, const float *first_b,
                 const float *w, const float *b, float *y, int t, int f, int ch, int t0,
                 int rows);
/* Pass::flatten (src/gpu/mod.rs:1674-1678): [t][f][ch] -> [t][ch·f]. */
int wh_flatten(wh_ctx *ctx, const float *x, float *y, int t, int f, int ch);
/* Pass::argmax (src/gpu/mod.rs:1669-1672): index of the first maximum of x[..n] into out[0]. */
int wh_argmax(wh_ctx *ctx, const float *x, uint32_t *out, int n);

/* --------------------------------------------------------------------- model graph drivers */

/* Model::load_with for the GGUF families on this backend (src/lib.rs:580-617): reads the file's
 * header and weights (src/gguf.rs) and uploads them (gigaam: src/gigaam/encoder.rs:39-57; parakeet:
 * src/parakeet/encoder.rs:51-74; whisper: src/whisper/encoder.rs:32-45, src/transformer.rs:180-212). */
int wh_model_load(wh_ctx *ctx, const char *gguf_path, wh_model **out);
void wh_model_free(wh_model *m);
/* arch: 0 gigaam, 1 parakeet, 2 whisper; d_model, encoder layers, mel bins, output width. */
int wh_model_info(const wh_model *m, int *arch, int *d, int *layers, int *mels, int *width);
/* Encoder frames and output width for mel_frames mel frames (src/parakeet/mod.rs:44-46 etc.). */
int wh_model_frames(const wh_model *m, int mel_frames, int *frames, int *width);
/* The family's Encoder::record on device buffers (src/gigaam/encoder.rs:83-93,
 * src/parakeet/encoder.rs:103-124, src/whisper/encoder.rs:67-74): mel_dev [mel_frames][mels] →
 * out_dev [frames][width].  `valid` < mel_frames marks the frames past it as padding (kestrel
 * length masking, src/parakeet/encoder.rs:77-80).  Queued; wh_sync waits. */
int wh_model_encode(wh_model *m, const float *mel_dev, int mel_frames, int valid, float *out_dev);
/* A batch of padded windows through the Parakeet encoder (one segment per window, each padded to
 * mel_frames): valid[b] mel frames of window b are real; keys and conv inputs past a window's valid
 * frames are masked, as the Neural Engine graph masks them (src/ane/conformer.rs:161-178, :301-309;
 * src/ane/mod.rs:463-466).  mel_dev [batch][mel_frames][mels] → out_dev [batch][frames][width]. */
int wh_model_encode_batch(wh_model *m, const float *mel_dev, int batch, int mel_frames,
                          const int *valid, float *out_dev);
/* Replay of repeated encoder calls (no counterpart in the reference, whose wgpu passes are recorded
 * anew per call, src/gpu/mod.rs:906-1002).  With on != 0 (the default) the second wh_model_encode /
 * wh_model_encode_batch call with the same arguments (same device buffers and sizes) is recorded
 * into a HIP graph and later such calls replay it: the same kernels in the same order, without
 * their host-side launch cost.  on == 0 drops the recordings and launches every call eagerly. */
int wh_model_graphs(wh_model *m, int on);
/* Conformer blocks only, over x_dev [t][d] in place (layers = how many of them). */
int wh_model_blocks(wh_model *m, float *x_dev, int t, int layers);
/* Greedy token ids of an encoder output on the host: CTC (GigaAM, src/gigaam/decoder.rs:135-151)
 * or TDT (Parakeet, src/parakeet/decoder.rs:91-191).  Writes up to cap (token, frame) pairs;
 * returns the count or a negative error. */
int wh_model_greedy(wh_model *m, const float *enc_host, int frames, int width, uint32_t *out,
                    int cap);
/* The same decoders over an encoder output in device memory, run on the device; replaces the
 * encoder readback plus host decode of Model::transcribe (src/parakeet/mod.rs:135-141,
 * src/gigaam/mod.rs:144-152).  CTC: per-frame first-maximum argmax and the collapse.  TDT: the
 * joint, decision and LSTM predictor with the loop's state in device memory (runs of decisions
 * recorded and replayed; the host reads the state between runs).  Same results as wh_model_greedy
 * up to float rounding of the decoder's products (ties of near-equal logits may differ). */
int wh_model_greedy_device(wh_model *m, const float *enc_dev, int frames, int width, uint32_t *out,
                           int cap);
/* The family's log-mel frontend, Frontend::compute (src/parakeet/frontend.rs:52-72,
 * src/gigaam/frontend.rs:50-71, src/whisper/frontend.rs:45-85), on the device: pcm_dev holds
 * `samples` 16 kHz samples; writes the features [frames][mels] to mel_dev and their count to *frames
 * (mel_dev NULL: the count only).  Parakeet: samples / 160 + 1 frames (0 below 3), normalized;
 * GigaAM: full 320-sample frames; Whisper: 3000 frames for up to 30 s, else samples / 160.  GigaAM and
 * Whisper take the window and filterbank the model file holds.  The transforms use the reference's
 * operation order and tables, so the spectra are bit-identical; the logarithms are the device's
 * (within an ulp of the host's). */
int wh_model_mel(wh_model *m, const float *pcm_dev, int samples, float *mel_dev, int *frames);
/* Whisper decoding on the device: wh_whisper_begin computes every layer's cross-attention K/V from
 * the encoder output (Decoder::record_cross, src/transformer.rs:243-248); wh_whisper_step runs one
 * token at position pos (Decoder::record_step, :254-290) and leaves the logits in logits_dev. */
int wh_whisper_begin(wh_model *m, const float *enc_dev, int frames);
int wh_whisper_step(wh_model *m, int token, int pos, float *logits_dev);

/* ------------------------------------------------------------------- Whisper window search */

/* The reference's `Ids` (src/whisper/search.rs:16-23): EOT, <|notimestamps|>, the first timestamp
 * <|0.00|> (begin; timestamps run to the end of the vocabulary) and the two suppression lists, plus
 * SOT (src/whisper/mod.rs:177). */
typedef struct wh_whisper_ids {
  int eot, no_timestamps, begin, sot;
  const int *suppress;
  int n_suppress;
  const int *begin_suppress;
  int n_begin_suppress;
} wh_whisper_ids;
/* The model's ids as Whisper::load reads them (src/whisper/mod.rs:131-141); the lists point into
 * the model. */
int wh_whisper_ids_of(const wh_model *m, wh_whisper_ids *out);
/* search::decode's choice of the next token (`pick`, src/whisper/search.rs:46-59, with
 * timestamp_rules :73-111 and argmax :113-127), in place on host logits[vocab]: the suppression list,
 * the begin-suppression list while n == 0, the timestamp rules over the n ids generated so far, then
 * the first maximum; with logprob != NULL also its log-softmax.  Returns the id (or WH_EARG).  Host
 * code only: it needs no device. */
int wh_whisper_pick(const wh_whisper_ids *ids, float *logits, int vocab, const uint32_t *generated, int n,
                    float *logprob);
/* search::probability (src/whisper/search.rs:129-135): the softmax probability of id. */
float wh_whisper_probability(const float *logits, int vocab, int id);
/* search::retrieve (src/whisper/search.rs:137-181): the segments of a window's generated ids as
 * (start in 20 ms steps, first index, end index) triples in seg[3i..3i+2] (their text: the ids < eot
 * in that range); returns the count (writes at most cap); *advance = the mel frames the next window
 * moves on.  Host code only. */
int wh_whisper_retrieve(const wh_whisper_ids *ids, const uint32_t *generated, int n, int frames, int *seg, int cap,
                        int *advance);
/* The decoding of one window of Whisper::transcribe (src/whisper/mod.rs:226-239, search::decode
 * src/whisper/search.rs:35-71) on the device: the cross K/V of enc_dev [frames][d] (wh_whisper_begin),
 * the decoder over the prompt (n_prompt ids from SOT; 0 = [SOT], the prompt of a model without
 * language tokens), then greedy steps under the rules until EOT, 256 new tokens or position
 * min(448, context).  The search runs on the device: each pick (suppression, timestamp rules, first
 * argmax, log-softmax) is a kernel over the step's logits that also writes the next step's token and
 * position, and recorded runs of 8 (step, pick) pairs replay with one small read of the search's
 * state between runs (the reference reads every step's logits back, Gpu::finish).  Log-probabilities
 * are summed when the no-speech probability on SOT's logits is above 0.6, as the reference asks for them.
 * Writes the generated ids (without EOT) to out and returns their count (or an error); *no_speech and
 * *avg_logprob (0 when not summed) may be NULL. */
int wh_whisper_decode(wh_model *m, const float *enc_dev, int frames, const uint32_t *prompt, int n_prompt,
                      uint32_t *out, int cap, float *no_speech, float *avg_logprob);

#ifdef __cplusplus
}
#endif
#endif
