// Greedy decoders of an encoder output on the device: CTC (src/gigaam/decoder.rs:135-151) and the
// TDT loop with its LSTM predictor and joint (src/parakeet/decoder.rs:91-191).  The reference runs
// both on the host; here the encoder output never leaves the device and only the (token, frame)
// pairs come back.
//
// TDT: the loop's control state lives in device memory (TdtState), so one decision is a fixed
// sequence of launches that a caller records once and replays until the state says done: the joint
// input z = ReLU(enc[t] + pred) (tdt_joint_in_kernel), the joint's output layer (a GEMV), the
// decision (tdt_decide_kernel: both first-maximum argmaxes and the reference's frame / symbol-budget
// rules), then the predictor on the emitted token (the embedding row, per LSTM layer the gate GEMVs
// and tdt_cell_kernel, the joint's predictor projection), whose launches a device-side flag switches
// off when the decision emitted nothing or the loop is done.
#include <cfloat>

#include "internal.h"

namespace {

__device__ __forceinline__ bool better(float v, int i, float bv, int bi) {
  // The first maximum: a larger value, or an equal one at a smaller index.
  return v > bv || (v == bv && i < bi);
}

// (value, index) of the first maximum of x[0..n) over a workgroup of 256 threads; every thread gets it.
__device__ __forceinline__ void wg_argmax(const float *__restrict__ x, int n, float *sv, int *si, float &v, int &i) {
  const int tid = threadIdx.x;
  float bv = -FLT_MAX;
  int bi = n;
  for (int j = tid; j < n; j += 256) {
    const float y = x[j];
    if (bi == n || better(y, j, bv, bi)) bv = y, bi = j;
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(bv, o, 64);
    const int oi = __shfl_xor(bi, o, 64);
    if (oi < n && (bi == n || better(ov, oi, bv, bi))) bv = ov, bi = oi;
  }
  if ((tid & 63) == 0) sv[tid >> 6] = bv, si[tid >> 6] = bi;
  __syncthreads();
  v = sv[0], i = si[0];
  for (int w = 1; w < 4; w++)
    if (si[w] < n && (i == n || better(sv[w], si[w], v, i))) v = sv[w], i = si[w];
  __syncthreads();
}

// z[j] = max(enc[t·width + j] + pred[j], 0) for the current frame t (Decoder::joint's input,
// src/parakeet/decoder.rs:135-142).
__global__ __launch_bounds__(256) void tdt_joint_in_kernel(const float *__restrict__ pred, float *__restrict__ z,
                                                           int joint, const TdtState *__restrict__ st) {
  if (st->done) return;
  const float *e = st->enc + (size_t)st->t * st->width;
  for (int j = threadIdx.x; j < joint; j += 256) z[j] = fmaxf(e[j] + pred[j], 0.0f);
}

// The predictor's input: the embedding row of the last emitted token (Decoder::predict,
// src/parakeet/decoder.rs:111-114).
__global__ __launch_bounds__(256) void tdt_embed_kernel(const float *__restrict__ table, int n, float *__restrict__ x,
                                                        const TdtState *__restrict__ st) {
  if (st->idle) return;
  const float *row = table + (size_t)st->token * n;
  for (int j = threadIdx.x; j < n; j += 256) x[j] = row[j];
}

// One decision of the TDT greedy loop (src/parakeet/decoder.rs:158-191) on the joint's logits
// [classes + durations]: the token and duration argmaxes (first maximum), the emission, and the
// frame / symbol-budget update.  One workgroup.
__global__ __launch_bounds__(256) void tdt_decide_kernel(const float *__restrict__ logits, TdtState *__restrict__ st,
                                                         TdtConfig cfg) {
  __shared__ float sv[4];
  __shared__ int si[4];
  if (st->done) return;
  float v;
  int token, di;
  wg_argmax(logits, cfg.classes, sv, si, v, token);
  wg_argmax(logits + cfg.classes, cfg.ndur, sv, si, v, di);
  if (threadIdx.x != 0) return;
  const int t = st->t, dur = cfg.durations[di];
  const bool emit = token != cfg.blank;
  if (emit) {
    if (st->count < st->cap) {
      st->out[2 * st->count] = (uint32_t)token;
      st->out[2 * st->count + 1] = (uint32_t)t;
    }
    st->count++;
    st->token = token;
  }
  int nt = t;
  if (cfg.global) {
    st->left--;
    nt = t + (token == cfg.blank ? max(dur, 1) : dur);
  } else {
    nt = t + dur;
    int symbols = st->symbols + 1;
    if (dur != 0) {
      symbols = 0;
    } else if (symbols >= cfg.max_symbols || token == cfg.blank) {
      nt++;
      symbols = 0;
    }
    st->symbols = symbols;
  }
  st->t = nt;
  st->decisions++;
  const int done = nt >= st->frames || (cfg.global && st->left <= 0);
  st->done = done;
  st->idle = (!emit || done) ? 1 : 0;
}

// One LSTM layer's cell (Decoder::predict, src/parakeet/decoder.rs:115-128): the gates [i | f | g | o]
// (one GEMV of [Wx | Wh] over [x | h] with the bias), c' = σ(f)·c + σ(i)·tanh(g), h' = σ(o)·tanh(c'),
// in place.
__global__ __launch_bounds__(256) void tdt_cell_kernel(const float *__restrict__ gates, float *__restrict__ h,
                                                       float *__restrict__ c, int n, const int *__restrict__ idle) {
  if (idle && *idle) return;
  for (int k = blockIdx.x * 256 + threadIdx.x; k < n; k += gridDim.x * 256) {
    const float ig = gates[k], fg = gates[n + k], gg = gates[2 * n + k], og = gates[3 * n + k];
    const float si = 1.0f / (1.0f + expf(-ig)), sf = 1.0f / (1.0f + expf(-fg)), so = 1.0f / (1.0f + expf(-og));
    const float cc = sf * c[k] + si * tanhf(gg);
    c[k] = cc;
    h[k] = so * tanhf(cc);
  }
}

__global__ void tdt_init_kernel(TdtState *st, TdtState init) {
  if (threadIdx.x == 0) *st = init;
}

// Greedy CTC, step 1: the first maximum of each frame's first `classes` logits.
__global__ __launch_bounds__(256) void ctc_argmax_kernel(const float *__restrict__ logits, int width, int classes,
                                                         int *__restrict__ ids) {
  __shared__ float sv[4];
  __shared__ int si[4];
  float v;
  int i;
  wg_argmax(logits + (size_t)blockIdx.x * width, classes, sv, si, v, i);
  if (threadIdx.x == 0) ids[blockIdx.x] = i;
}

// Greedy CTC, step 2 (src/gigaam/decoder.rs:135-151): a frame's id is emitted when it is not blank and
// differs from the previous frame's; (token, frame) pairs in order, the count in out_count.  One
// workgroup: each thread flags its frames, a prefix sum over the flags places the pairs.
__global__ __launch_bounds__(256) void ctc_collapse_kernel(const int *__restrict__ ids, int frames, int blank,
                                                           uint32_t *__restrict__ out, int cap, int *__restrict__ count) {
  __shared__ int part[256];
  const int tid = threadIdx.x, per = (frames + 255) / 256, f0 = tid * per, f1 = min(f0 + per, frames);
  int n = 0;
  for (int f = f0; f < f1; f++) n += ids[f] != blank && (f == 0 || ids[f] != ids[f - 1]);
  part[tid] = n;
  __syncthreads();
  for (int o = 1; o < 256; o <<= 1) {  // inclusive prefix sum
    const int add = tid >= o ? part[tid - o] : 0;
    __syncthreads();
    part[tid] += add;
    __syncthreads();
  }
  int at = part[tid] - n;
  for (int f = f0; f < f1; f++)
    if (ids[f] != blank && (f == 0 || ids[f] != ids[f - 1])) {
      if (at < cap) out[2 * at] = (uint32_t)ids[f], out[2 * at + 1] = (uint32_t)f;
      at++;
    }
  if (tid == 255) *count = part[255];
}

}  // namespace

int launch_tdt_init(wh_ctx *ctx, TdtState *st, const TdtState &init) {
  wh_launch(ctx, tdt_init_kernel, 1, 64, 0, st, init);
  return wh_launched(ctx, "tdt init");
}

int launch_tdt_joint_in(wh_ctx *ctx, const float *pred, float *z, int joint, const TdtState *st) {
  ProfScope prof(ctx, "tdt_joint_in", 0.0, 12.0 * joint);
  wh_launch(ctx, tdt_joint_in_kernel, 1, 256, 0, pred, z, joint, st);
  return wh_launched(ctx, "tdt joint input");
}

int launch_tdt_embed(wh_ctx *ctx, const float *table, int n, float *x, const TdtState *st) {
  ProfScope prof(ctx, "tdt_embed", 0.0, 8.0 * n);
  wh_launch(ctx, tdt_embed_kernel, 1, 256, 0, table, n, x, st);
  return wh_launched(ctx, "tdt embed");
}

int launch_tdt_decide(wh_ctx *ctx, const float *logits, TdtState *st, const TdtConfig &cfg) {
  if (cfg.classes <= 0 || cfg.ndur <= 0 || cfg.ndur > 16 || cfg.blank < 0 || cfg.blank >= cfg.classes ||
      cfg.max_symbols <= 0)
    return wh_fail(ctx, WH_EARG, "tdt: bad decoder configuration");
  ProfScope prof(ctx, "tdt_decide", 0.0, 4.0 * (cfg.classes + cfg.ndur));
  wh_launch(ctx, tdt_decide_kernel, 1, 256, 0, logits, st, cfg);
  return wh_launched(ctx, "tdt decide");
}

int launch_tdt_cell(wh_ctx *ctx, const float *gates, float *h, float *c, int n, const int *idle) {
  ProfScope prof(ctx, "tdt_cell", 0.0, 28.0 * n);
  wh_launch(ctx, tdt_cell_kernel, (n + 255) / 256, 256, 0, gates, h, c, n, idle);
  return wh_launched(ctx, "tdt cell");
}

int launch_ctc(wh_ctx *ctx, const float *logits, int frames, int width, int classes, int blank, int *ids,
               uint32_t *out, int cap, int *count) {
  if (frames <= 0 || classes <= 0 || classes > width || blank < 0 || blank >= classes)
    return wh_fail(ctx, WH_EARG, "ctc: bad arguments");
  {
    ProfScope prof(ctx, "ctc_argmax", 0.0, 4.0 * frames * classes);
    wh_launch(ctx, ctc_argmax_kernel, frames, 256, 0, logits, width, classes, ids);
    if (int rc = wh_launched(ctx, "ctc argmax")) return rc;
  }
  ProfScope prof(ctx, "ctc_collapse", 0.0, 4.0 * frames);
  wh_launch(ctx, ctc_collapse_kernel, 1, 256, 0, ids, frames, blank, out, cap, count);
  return wh_launched(ctx, "ctc collapse");
}
