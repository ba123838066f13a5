// Internal declarations of the gfx950 backend: the context, weights, and the kernel launchers that
// the C ABI (include/wavo_hip.h) and the graph drivers call.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <cstdint>
#include <string>
#include <array>
#include <vector>

#include "../../include/wavo_hip.h"

// One profiled launch (or named region) and its algorithmic work: a start and a stop event.  A launch's
// events are stamped by the runtime at the kernel's own start and end (hipExtLaunchKernel); a region's
// are recorded on the stream around whatever is queued in between.  `used` = the events were queued.
struct wh_prof_rec {
  std::string kernel;
  double flops = 0, bytes = 0;
  int ev0 = -1, ev1 = -1;
  bool used = false;
};

constexpr int ATTEND_HEADS = 1024;  // heads of one attend launch, at most
constexpr int ROW_REGS = 32;  // row values per lane the row kernels hold in registers: rows up to 2048
// An internal GEMM epilogue (beside WH_BIAS .. WH_TANH): the GLU of the Conformer conv module over a
// weight whose output columns come in groups of 8, [a₀..a₃ | g₀..g₃] (4 channels, rows permuted at
// load): output row r, column col/2 + q = (x_q + b_q)·σ(x_{q+4} + b_{q+4}) for the group at col, σ as
// 1/(1 + e^−x) by the hardware reciprocal (conv_glu_kernel's arithmetic); c is cols/2 wide (ldc), f32,
// and the GEMM does not split k.
constexpr int EPI_GLU = 7;

struct wh_ctx {
  int device = 0;
  hipStream_t stream = nullptr;
  int cus = 0;
  // Per head, the parts of an attend launch done so far (0 between launches: the last part resets it).
  int *attend_count = nullptr;
  // GEMM launch-plan override set by wh_tune("gemm_plan", "bm,bn,wm,wn,slots,split[,pipeline[,kgroups]]") (tuning
  // sweeps only): all zero = chosen per shape.
  int gemm_plan[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  // wh_tune("gemm_kernel_only", "1") (measurement only): a split GEMM call stops after the GEMM kernel, leaving
  // its partial sums unfinished, so that the kernel can be timed alone as it runs inside a model step
  // (where the next kernel finishes the sums).
  int gemm_kernel_only = 0;
  // Per-shape overrides set by wh_tune("gemm_shape_plans", "m,cols,k:bm,bn,wm,wn,slots,split[,pipeline[,kgroups]];…")
  // (tuning sweeps inside a model's step only).
  std::vector<std::array<int, 11>> gemm_shape_plans;
  // GEMM tile-order override set by wh_tune("gemm_group", "n") (tuning sweeps only): n row tiles per
  // group of the order; 0 = chosen per shape.
  int gemm_group = 0;
  // Attention key-split override set by wh_tune("attn_split", "n") (tuning sweeps only): 0 = chosen per shape.
  int attn_split = 0;
  // Set by a caller around one GEMM call (null otherwise): the main kernel skips when *gemm_skip ==
  // gemm_skip_val (its output already holds the product).
  const int *gemm_skip = nullptr;
  int gemm_skip_val = 0;
  // wh_tune("position_cache", "0") (measurement): the Parakeet encoder recomputes its position
  // projection every call instead of keeping it per frame count; "1" restores.
  int no_position_cache = 0;
  // wh_tune("mel_raw", "1") (checks only): the frontends write each filter's sum before the logarithm.
  int mel_raw = 0;
  // wh_tune("whisper_host", "1") (checks only): wh_whisper_decode picks each token on the host.
  int whisper_host = 0;
  // wh_tune("whisper_logprobs", "1") (checks only): the window search sums the picks' log-probabilities
  // whatever the no-speech probability.
  int whisper_logprobs = 0;
  // wh_tune("attend_merge", "1") (checks only): attention over a key count known at launch merges its
  // parts in its last workgroup, as for a count in device memory, instead of a second kernel.
  int attend_merge = 0;
  // Bumped by every wh_tune call: the model's recorded calls carry it in their keys, so that a call
  // recorded before a tuning change is not replayed after it.
  long tune_epoch = 0;
  // wh_tune("epilogue_fusion", "0") (checks only): the encoders run in launches of their own what
  // GEMM epilogues do otherwise — attention's K, Vᵀ and position rows packed (as for padded batches),
  // the Parakeet subsampling's image flattened, the conv module's GLU; "1" restores.
  int unfused = 0;
  std::string name;
  std::string error;
  // Profiling (wh_profile): 0 off (default), 1 events around every launch, 2 named regions only.
  int prof = 0;
  int open_region = -1;
  int prof_pending = -1;  // mode 1: the record whose events the next wh_launch carries
  std::vector<hipEvent_t> events;
  size_t next_event = 0;
  std::vector<wh_prof_rec> recs;
  // Device scratch of the ops that stage data between kernels of one call (attention's split
  // operands): grown on demand, reused by every later call on this stream.
  void *scratch = nullptr;
  size_t scratch_bytes = 0;
  long scratch_epoch = 0;  // incremented whenever scratch moves (recorded graphs hold its address)
  int recording = 0;       // between wh_record_begin and wh_record_end: the stream is being captured
  // The device address of wh_gemm_noalloc's file-scope workspace on this device (nullptr if the
  // lookup failed, with its error).
  void *noalloc = nullptr;
  hipError_t noalloc_error = hipSuccess;
  // Staged uploads (stage_upload): a second stream for host-to-device copies, a ring of pinned host
  // buffers (allocated at the first upload), per slot the event of its last copy, and the fill of
  // the current slot.
  hipStream_t upload = nullptr;
  static constexpr int STAGE_SLOTS = 4;
  void *pinned[STAGE_SLOTS] = {};
  hipEvent_t pinned_done[STAGE_SLOTS] = {};
  bool pinned_used[STAGE_SLOTS] = {};
  int pinned_slot = 0;
  size_t pinned_fill = 0;
  hipEvent_t upload_fence = nullptr;
};

// A file whose mapping [base, base + size) a staged upload reads with pread instead of through the
// mapping: no page faults, the kernel copies from the page cache (or the disk) into pinned memory.
struct StageFile {
  int fd;
  const uint8_t *base;
  size_t size;
};
// Copies `bytes` of host memory (read from `file` where they lie in its mapping) into pinned staging
// and queues their copy to `dst` on the context's upload stream; returns once `src` may be reused.
int stage_upload(wh_ctx *ctx, void *dst, const void *src, size_t bytes, const StageFile *file = nullptr);
// Work queued on ctx->stream after this call waits for every staged upload so far.
int stage_fence(wh_ctx *ctx);
// Waits for every staged upload and reports their errors.
int stage_wait(wh_ctx *ctx);
// wh_linear_new with the weights read through `file` where they lie in its mapping.
int linear_new(wh_ctx *ctx, const wh_tensor *ws, int count, const float *bias, int n_bias, int pad_k,
               wh_linear **out, const StageFile *file);

// Looks up the device address of wh_gemm_noalloc's workspace on ctx's device (current), once per device.
int gemm_noalloc_init(wh_ctx *ctx);

// At least `bytes` of device scratch (256-byte aligned), or nullptr with ctx->error set.  Growing
// it drains the stream first; a caller that must not allocate reserves the size up front.
void *wh_scratch(wh_ctx *ctx, size_t bytes);

// Profiling scope of one launch: with per-launch profiling on (wh_profile 1) it reserves a record with
// a start/stop event pair, which the next wh_launch inside the scope carries; a scope left without a
// launch drops its record.
struct ProfScope {
  ProfScope(wh_ctx *ctx, const char *kernel, double flops, double bytes);
  ~ProfScope();
  wh_ctx *ctx;
  int rec = -1;
};

// The event pair of the pending profiled launch (nullptr when none), which the call clears.
void wh_prof_take(wh_ctx *ctx, hipEvent_t *start, hipEvent_t *stop);

// Queues kernel<<<grid, block, shm, ctx->stream>>>(args...).  Under a ProfScope with per-launch
// profiling on, the launch goes through hipExtLaunchKernelGGL with the scope's events, which the
// runtime stamps at the kernel's own start and end (no marker packets around it).
template <typename F, typename... Args>
inline void wh_launch(wh_ctx *ctx, F kernel, dim3 grid, dim3 block, size_t shm, Args... args) {
  if (ctx->prof == 1 && ctx->prof_pending >= 0) {
    hipEvent_t e0 = nullptr, e1 = nullptr;
    wh_prof_take(ctx, &e0, &e1);
    hipExtLaunchKernelGGL(kernel, grid, block, (std::uint32_t)shm, ctx->stream, e0, e1, 0u, args...);
    return;
  }
  kernel<<<grid, block, shm, ctx->stream>>>(args...);
}

// A linear layer on the device (src/gpu/mod.rs:390-413): W [rows][k] in its GGUF bytes, rows
// contiguous; the bias padded to `cols + dual`.
struct wh_linear {
  int rows = 0;   // real rows of W (stacked)
  int cols = 0;   // output columns before the dual ones
  int dual = 0;
  int k = 0;      // inner size (padded to 32 for a conv)
  int type = 0;   // WH_F32 / WH_F16 / WH_Q4_0 / WH_Q8_0
  size_t row_bytes = 0;
  uint8_t *w = nullptr;
  float *bias = nullptr;  // cols + dual values
};

// Sets ctx->error and returns code.
int wh_fail(wh_ctx *ctx, int code, const char *fmt, ...);
// Checks the last launch; returns WH_OK or WH_EGPU with the HIP error text.
int wh_launched(wh_ctx *ctx, const char *what);

// Bytes of n weights of a GGUF type.
size_t wh_type_bytes(int type, size_t n);

// ---- launchers (each validates its shapes, then queues on ctx->stream) ----
int launch_gemm(wh_ctx *ctx, const float *a, const wh_linear *l, float *c, int m, int ldc, int epi,
                float alpha);
// The same with `a` already rounded to f16 (its producer wrote f16): half the A traffic.  With
// out16 the outputs are stored as f16 (for a consumer that rounds them to f16 anyway); residual
// epilogues need f32 outputs.
// Whether launch_gemm_h can run l with EPI_GLU into c (the main kernel, whole groups of 8 real columns).
bool gemm_glu_ok(const wh_linear *l, const void *c);
int launch_gemm_h(wh_ctx *ctx, const void *a16, const wh_linear *l, void *c, int m, int ldc, int epi,
                  float alpha, int out16);
// x += alpha·(l(a16) + bias) followed by y = LayerNorm(x; g, b) (y f16 with out16): a GEMM with the
// residual epilogue whose output row feeds a LayerNorm.  When the GEMM splits k, the split finish
// and the norm run as one kernel (launch_split_residual_ln); otherwise the GEMM's own epilogue adds
// the residual and the norm follows.  Needs l->cols == cols of x and no dual outputs.  keep_x = 0:
// x is not needed afterwards (the fused kernel need not store it).  g2: a second LayerNorm of y (f32)
// into y2 (f16) — the next block's first norm.  residual = 0: x = l(a16) + bias (the bias epilogue; x
// is not read), then the norm.
// A GEMM whose columns col0 .. col0 + cols − 1, heads of hd, go to dst in attention's packed layout
// instead of into c: rows per head (tr false: [head][rs][hd], this call's rows from row r0, rows m ..
// rs − r0 − 1 as zeros where tiles reach them) or transposed (tr: [head][hd][rs], r0 = 0, zeros for
// rows m .. rs − 1).  Transposed with blk > 0 (one head, hd = cols, blk % 8 == 0): rows in blocks of
// blk, [row / blk][col − col0][row % blk] — a [t][f][ch] image flattened to [t][ch·f] rows (blk = f) —
// rows from rs on not written.
struct HeadsOut {
  _Float16 *dst;
  int col0, cols, hd, rs, r0;
  bool tr;
  int blk;
};
int launch_gemm_h_heads(wh_ctx *ctx, const void *a16, const wh_linear *l, void *c, int m, int ldc, int epi,
                        const HeadsOut *outs, int n);
int launch_gemm_h_ln(wh_ctx *ctx, const void *a16, const wh_linear *l, float *x, int m, float alpha, const float *g,
                     const float *b, void *y, int out16, int keep_x = 1, const float *g2 = nullptr,
                     const float *b2 = nullptr, void *y2 = nullptr, int residual = 1);
int launch_split_residual_ln(wh_ctx *ctx, const float *part, int splits, const float *bias, int wrows, float alpha,
                             float *x, const float *g, const float *b, void *y, int rows, int cols, int out16,
                             int keep_x = 1, const float *g2 = nullptr, const float *b2 = nullptr, void *y2 = nullptr,
                             int residual = 1);
// f32 → f16 (RNE) of n values (n % 4 == 0).
int launch_to_half(wh_ctx *ctx, const float *x, void *y, size_t n);
// A decoder cache column written by a GEMV as well: outputs lo .. lo + 2d (a K row then a V row of d
// values) go, as f16, to column col (or *dcol) of `cache` (cols positions; launch_pack's layout).
struct GemvPack {
  uint32_t *cache;
  int lo, d, cols, col;
  const int *dcol;
};
// With ln_g: the product takes LayerNorm(a; ln_g, ln_b) (one row of k): inside the streaming kernel,
// or written to ln_y (k floats) by its own launch before the general kernel.  With pack: see GemvPack
// (inside the streaming kernel, or by launch_pack after the general one).
int launch_gemv(wh_ctx *ctx, const float *a, const wh_linear *l, float *c, int epi, float alpha,
                int offset, const float *ln_g = nullptr, const float *ln_b = nullptr, float *ln_y = nullptr,
                const GemvPack *pack = nullptr);
// With dpos (device memory), the position offset is (*dpos)·dstride instead of `offset`: a recorded
// decoder step reads its position from the device.
int launch_embed(wh_ctx *ctx, const wh_linear *l, const float *pos, float *c, const uint32_t *ids,
                 int i, int offset, const int *dpos = nullptr, int dstride = 0);
// out16: y (and yr) as f16, for consumers that are GEMMs.
int launch_layer_norm(wh_ctx *ctx, const float *x, const float *g, const float *b, void *y, int rows,
                      int cols, const float *table, void *yr, int head_dim, int out16 = 0);
int launch_im2col(wh_ctx *ctx, const float *x, float *col, int t, int ch, int kernel, int stride,
                  int pad, int batch, long x_batch_stride, long col_batch_stride);
// layout of h: 0 [x | gates] per frame, 1 groups of 8 [x₀..x₃ | g₀..g₃] per 4 channels, 2 the GLU
// already applied ([t][ch]; EPI_GLU).
int launch_conv_glu(wh_ctx *ctx, const float *h, const float *w, const float *wb, int kernel,
                    const float *g, const float *b, int layer_norm, void *y, int t, int ch,
                    const int *valid_dev, int valid, int batch, int out16 = 0, int layout = 0);
// qk / v / pos are f32 (in16 == 0) or f16; o is f32 or f16 (out16).  pos rows are pos_stride
// elements apart (0: heads · hd).
// The packed attention operands' shape for one window of t keys (relative: with position rows).
void attention_layout(int t, int heads, int hd, int rel, int *tk, int *pfront, int *prows);
int launch_attention_packed(wh_ctx *ctx, const _Float16 *q, int qs, const _Float16 *qv, const _Float16 *kp,
                            const _Float16 *vt, const _Float16 *pp, void *o, int t, int heads, int hd, int out16);
int launch_attention(wh_ctx *ctx, const void *qk, const void *v, const void *pos, void *o, int t,
                     int heads, int hd, const int *valid_dev, int valid, int batch, int out16 = 0,
                     int in16 = 0, int pos_stride = 0);
// Scratch bytes launch_attention uses for t frames × batch windows (rel: relative positions) on
// this context's device (its CU count sets the key splits).
size_t attention_scratch_bytes(const wh_ctx *ctx, int t, int heads, int hd, int batch, int rel);
// y f32, or f16 with out16 (for a consumer that rounds its input to f16 anyway: a GEMM).
int launch_depthwise(wh_ctx *ctx, const float *x, const float *w0, const float *b0, const float *w,
                     const float *b, void *y, int t, int f, int ch, int t0, int rows, int out16 = 0);
// x and y f32, or both f16 (f16).
int launch_flatten(wh_ctx *ctx, const void *x, void *y, int t, int f, int ch, int f16 = 0);
int launch_argmax(wh_ctx *ctx, const float *x, uint32_t *out, int n);
int launch_step_args(wh_ctx *ctx, uint32_t *ids, int token, int pos);
// With dn (device memory), the key count is *dn + n (at most cols).
int launch_attend(wh_ctx *ctx, const float *q, const uint32_t *kv, float *part, float *o, int n,
                  int cols, int heads, int hd, const int *dn = nullptr);
// With dcol (device memory), the first cache column is *dcol instead of `col` (columns past the
// cache are not written).
int launch_pack(wh_ctx *ctx, const float *x, int src, int stride, uint32_t *y, int rows, int d,
                int cols, int col, const int *dcol = nullptr);
int launch_zero(wh_ctx *ctx, void *dst, size_t bytes);
// *dst = v (one thread, on the context's stream).
int launch_set_int(wh_ctx *ctx, int *dst, int v);
// Device-to-device copy with a kernel (a graph node like any other launch).
int launch_copy(wh_ctx *ctx, void *dst, const void *src, size_t bytes);
int launch_add_rows(wh_ctx *ctx, float *x, const float *add, size_t n);

// ---- greedy decoding on the device (greedy.hip) ----
// The TDT loop's state (src/parakeet/decoder.rs:158-191), in device memory: the call's encoder output
// and (token, frame) list too, so a recorded decision serves every call.
struct TdtState {
  int t, symbols, left, count, token, done, idle, decisions;
  int frames, width, cap, pad;
  const float *enc;
  uint32_t *out;
};
// The decoder's constants (src/parakeet/decoder.rs:46-89).
struct TdtConfig {
  int classes, ndur, blank, max_symbols, global;
  int durations[16];
};
// The fused decision's arguments: the decoder's weights as stored (one type for all), the state
// records (current and next), the LSTM state [layers][n] (old and new h, c), the joint's predictor
// projection, and the joint's per-workgroup partial maxima [parts][4].
struct TdtArgs {
  const uint8_t *out_w, *pred_w;
  const uint8_t *lstm_w[4];
  const float *out_b, *pred_b;
  const float *lstm_b[4];
  size_t out_rb, pred_rb, lstm_rb;
  int type, n, joint, layers, out_rows, parts;
  const float *embed;  // [classes][n] f32
  TdtState *st, *nx;
  float *h_old, *h_new, *c, *pred, *part;
  float *erow, *z;  // the next frame's encoder row [joint], the next joint input [joint]
  TdtConfig cfg;
};
enum { TDT_JOINT = 0, TDT_STEP = 1, TDT_PRED = 2, TDT_INIT = 3 };
// Both state records from `init` (the next one not idle: the first predict runs).
int launch_tdt_init(wh_ctx *ctx, TdtState *st, TdtState *nx, const TdtState &init);
// One part of a decision (TDT_JOINT, TDT_STEP with the further LSTM layers, TDT_PRED), or the first
// predict(None) (TDT_INIT, then TDT_PRED).
int launch_tdt(wh_ctx *ctx, const TdtArgs &a, int what);
// The joint's workgroups (and partial maxima) for `out_rows` output rows of weight type `type`.
int tdt_parts(int type, int out_rows);
// Greedy CTC (src/gigaam/decoder.rs:135-151) over `frames` rows of `width` logits (the first
// `classes` columns): ids (frames ints) is scratch; up to cap (token, frame) pairs into out, the
// count into *count (all device memory).
int launch_ctc(wh_ctx *ctx, const float *logits, int frames, int width, int classes, int blank, int *ids,
               uint32_t *out, int cap, int *count);

// ---- the log-mel frontends on the device (frontend.hip) ----
// One call's arguments: the audio, the transform's tables (as the element type: double for
// Parakeet, float otherwise), the window, the filterbank [mels][n_fft / 2 + 1] and per filter its
// span (Parakeet: nonzero bins; GigaAM: bins widened to 16; Whisper: 4-bin groups), the output.
struct MelArgs {
  const float *pcm;
  int samples, len, hop, mels, leaf, stages;
  const int *perm;
  const void *leaf_cos, *leaf_sin, *tw_cos, *tw_sin, *window;
  const float *filters;
  const int *span;
  float *out;
  float silent;  // Whisper: the value of a frame of zeros
  int raw;       // write each filter's sum before the logarithm; no normalization or scale
};
// kind 0 Parakeet, 1 GigaAM, 2 Whisper; `frames` frames into a.out; scratch: one float (Whisper).
int launch_mel(wh_ctx *ctx, const MelArgs &a, int kind, int frames, float *scratch);

// Whisper's window search on the device (greedy.hip): the loop's state, and one pick's arguments
// (the suppression lists as a per-id mask: bit 0 suppress, bit 1 suppress before the first token).
struct WhisperState {
  int n, pos, done, picks, np, limit, max_new, logprobs, last_ts, pad;
  double sum;
};
// One workgroup's share of a pick (greedy.hip): sums of exp(v − its maxima), the maxima, the first
// maxima over all its ids and over its timestamps.
struct WhisperPart {
  double s_ts, s_all;
  float tmax, text, fmax, best_v, ts_v;
  int best_i, ts_i, pad;
};
struct WhisperPickArgs {
  const float *logits;
  int vocab, eot, no_ts, begin, max_initial;
  const uint8_t *mask;
  WhisperState *st;
  uint32_t *gen, *ids;
  WhisperPart *part;  // a partial per 1024 ids
};
int launch_whisper_init(wh_ctx *ctx, WhisperState *st, const WhisperState &init);
int launch_whisper_pick(wh_ctx *ctx, const WhisperPickArgs &a);
