// Row-wise and convolution side kernels of the encoders over time-major [t][ch] f32 activations:
// LayerNorm (+RoPE), im2col, the Conformer conv module's middle (GLU, depthwise conv, norm, SiLU),
// Parakeet's 3×3 stride-2 subsampling convs and flatten, argmax, and fills.  Semantics follow
// src/gpu/ops.wgsl and src/gpu/spatial.wgsl (cited per kernel); the layout is one wavefront per row
// (64 lanes over the channels, reductions across the lanes) instead of a 256-thread
// workgroup per row, so a row's data stays in registers and short rows keep every lane busy.
#include <algorithm>

#include "internal.h"
#include "xlane.h"

namespace {

using xlane::wave_max;
using xlane::wave_sum;


__device__ __forceinline__ void store4(float *p, float4 v) { *(float4 *)p = v; }
// The f32 values rounded to f16 (RNE), as a GEMM rounds an f32 input: the empty asm keeps the compiler
// from fusing the last multiply-add into an f16-rounding one (v_fma_mix*), which rounds once from the
// exact sum instead.
__device__ __forceinline__ float as_f32(float v) {
  asm volatile("" : "+v"(v));
  return v;
}
__device__ __forceinline__ void store4(_Float16 *p, float4 v) {
  typedef _Float16 h4 __attribute__((ext_vector_type(4)));
  v.x = as_f32(v.x), v.y = as_f32(v.y), v.z = as_f32(v.z), v.w = as_f32(v.w);
  *(h4 *)p = h4{(_Float16)v.x, (_Float16)v.y, (_Float16)v.z, (_Float16)v.w};
}

// LayerNorm (eps 1e-5) of row `row`, one wavefront per row; with a table, the NEOX split-half RoPE
// of each head into yr (ops.wgsl:44-95; src/cpu/ops.rs:68-110).  OT = float, or _Float16 when every
// consumer of y (and yr) is a GEMM, which rounds its input to f16 anyway.  NJ: float4 groups per lane
// when cols == 256·NJ (the models' widths), else 0 (any cols ≤ ROW_REGS·64).  Every load of the row
// and of the norm's weights is issued before the first use, so the wave waits for one memory round
// trip (a loop that loads and then stores waits once per iteration).
template <typename OT, int NJ>
__global__ __launch_bounds__(256) void layer_norm_kernel(const float *__restrict__ x, const float *__restrict__ g,
                                                         const float *__restrict__ b, OT *__restrict__ y,
                                                         int rows, int cols, const float *__restrict__ table,
                                                         OT *__restrict__ yr, int hd) {
  extern __shared__ float srow[];  // 4 rows of cols (RoPE only)
  constexpr int J = NJ ? NJ : ROW_REGS / 4;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int row = blockIdx.x * 4 + w;
  const bool active = row < rows;
  float *sr = srow + w * cols;
  const int q4 = cols / 4;  // float4 per row (cols % 4 == 0)
  if (active) {
    const float4 *xr = (const float4 *)(x + (size_t)row * cols);
    const float4 *g4 = (const float4 *)g, *b4 = (const float4 *)b;
    float4 v[J], gg[J], bb[J];
#pragma unroll
    for (int j = 0; j < J; j++) {
      const int i = lane + 64 * j;
      const bool in = NJ || i < q4;
      v[j] = in ? xr[i] : make_float4(0, 0, 0, 0);
      gg[j] = in ? g4[i] : make_float4(0, 0, 0, 0);
      bb[j] = in ? b4[i] : make_float4(0, 0, 0, 0);
    }
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < J; j++) s += (v[j].x + v[j].y) + (v[j].z + v[j].w);
    const float mean = wave_sum(s) / (float)cols;
    float q = 0.0f;
#pragma unroll
    for (int j = 0; j < J; j++) {
      if (NJ || lane + 64 * j < q4) {
        float dx = v[j].x - mean, dy = v[j].y - mean, dz = v[j].z - mean, dw = v[j].w - mean;
        q += (dx * dx + dy * dy) + (dz * dz + dw * dw);
      }
    }
    const float rstd = rsqrtf(wave_sum(q) / (float)cols + 1e-5f);
    OT *yy = y + (size_t)row * cols;
#pragma unroll
    for (int j = 0; j < J; j++) {
      const int i = lane + 64 * j;
      if (NJ || i < q4) {
        float4 o;
        o.x = (v[j].x - mean) * rstd * gg[j].x + bb[j].x;
        o.y = (v[j].y - mean) * rstd * gg[j].y + bb[j].y;
        o.z = (v[j].z - mean) * rstd * gg[j].z + bb[j].z;
        o.w = (v[j].w - mean) * rstd * gg[j].w + bb[j].w;
        store4(yy + 4 * i, o);
        if (table) *(float4 *)(sr + 4 * i) = o;
      }
    }
  }
  if (!table) return;  // uniform across the workgroup
  __syncthreads();
  if (!active) return;
  const int half = hd / 2;
  const float *tr = table + (size_t)row * hd;
  OT *out = yr + (size_t)row * cols;
  for (int i = lane; i < cols; i += 64) {
    int d = i % hd, f = d % half;
    float c = tr[f], sn = tr[half + f];
    out[i] = (OT)(d < half ? sr[i] * c - sr[i + half] * sn : sr[i] * c + sr[i - half] * sn);
  }
}

// Same for rows longer than ROW_REGS·64: the row is read three times.
__global__ __launch_bounds__(64) void layer_norm_long(const float *__restrict__ x, const float *__restrict__ g,
                                                      const float *__restrict__ b, float *__restrict__ y, int cols) {
  const int lane = threadIdx.x;
  const float *xr = x + (size_t)blockIdx.x * cols;
  float s = 0.0f;
  for (int i = lane; i < cols; i += 64) s += xr[i];
  const float mean = wave_sum(s) / (float)cols;
  float q = 0.0f;
  for (int i = lane; i < cols; i += 64) {
    float d = xr[i] - mean;
    q += d * d;
  }
  const float rstd = rsqrtf(wave_sum(q) / (float)cols + 1e-5f);
  float *yy = y + (size_t)blockIdx.x * cols;
  for (int i = lane; i < cols; i += 64) yy[i] = (xr[i] - mean) * rstd * g[i] + b[i];
}

// im2col (ops.wgsl:97-119): col[i][c·kernel + k] = x[stride·i + k − pad][c], zero-padded to
// `width` (a multiple of 32).  blockIdx.z is the batch item.
__global__ void im2col_kernel(const float *__restrict__ x, float *__restrict__ col, int t, int ch, int kernel,
                              int stride, int pad, int rows, int width, long xs, long cs) {
  const int i = blockIdx.y;
  const int e = blockIdx.x * 256 + threadIdx.x;
  if (e >= width || i >= rows) return;
  x += xs * blockIdx.z;
  col += cs * blockIdx.z;
  float v = 0.0f;
  int s = stride * i + e % kernel;
  if (e < ch * kernel && s >= pad && s - pad < t) v = x[(size_t)(s - pad) * ch + e / kernel];
  col[(size_t)i * width + e] = v;
}

// The Conformer conv module between the pointwise convs (ops.wgsl:121-164; src/cpu/ops.rs:137-182):
// h [t][2ch] → GLU x·σ(gate) (zero from the window's valid frames on) → depthwise conv (odd kernel,
// centred, w [ch][kernel]) + bias → LayerNorm or affine → SiLU.  Layouts of h (GLU_*): x in columns
// 0..ch−1 and the gates after them; interleaved in groups of 8, [x₀..x₃ | g₀..g₃] per 4 channels (the
// pointwise conv's rows permuted at load); or the GLU already applied, [t][ch] (by that GEMM's
// epilogue, with this kernel's arithmetic).  A workgroup takes CF consecutive
// frames of one window with one thread per 4 channels: each thread slides over the CF + kernel − 1
// frames its outputs need, keeping their GLU values and its 4·kernel taps in registers (the taps of
// 4 channels are 4·kernel consecutive floats), so h is read once per workgroup plus the kernel − 1
// frames of overlap.  The norm's row sums go through wavefront reductions and LDS.  Frames are
// [batch][t]; the conv does not cross windows.  OT = float, or _Float16 for a consumer GEMM.
constexpr int CF = 4;  // 4 frames per workgroup: a 750-frame window spreads over 188 CUs
enum { GLU_PLAIN = 0, GLU_GROUPS = 1, GLU_DONE = 2 };
constexpr int CG_MAXK = 31;

template <typename OT, int K>
__global__ __launch_bounds__(256) void conv_glu_kernel(const float *__restrict__ h, const float *__restrict__ w,
                                                       const float *__restrict__ wb, int kernel,
                                                       const float *__restrict__ g, const float *__restrict__ gb,
                                                       int layer_norm, OT *__restrict__ y, int t, int ch,
                                                       const int *__restrict__ valid_dev, int valid, int layout) {
  constexpr int SPAN = CF + K - 1;
  __shared__ float red[2][4][CF];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, nw = blockDim.x >> 6;
  const int seg = blockIdx.y, f0 = blockIdx.x * CF;
  const int lim = valid_dev ? min(valid_dev[seg], t) : min(valid, t);
  const int pad = K / 2;
  const int c = 4 * tid;
  const bool on = c < ch;
  // Floats per frame of h, and this thread's offsets of its x and gate quads in a frame.
  const int fw = layout == GLU_DONE ? ch : 2 * ch;
  const int ox = layout == GLU_GROUPS ? 2 * c : c, og = layout == GLU_GROUPS ? 2 * c + 4 : c + ch;
  const float *hs = h + (size_t)seg * t * fw;
  float4 acc[CF];
  // The norm's weights, loaded with the inputs (they are used after the reductions).
  const float4 gg = on ? *(const float4 *)(g + c) : make_float4(0, 0, 0, 0);
  const float4 bb = on ? *(const float4 *)(gb + c) : make_float4(0, 0, 0, 0);
  {
    float4 tap[K];
    const float4 bias = on ? *(const float4 *)(wb + c) : make_float4(0, 0, 0, 0);
    if (on) {
      // Taps of channels c..c+3: w[(c + q)·K + k] = 4·K consecutive floats from c·K.
      const float *wc = w + (size_t)c * K;
#pragma unroll
      for (int k = 0; k < K; k++) tap[k] = make_float4(wc[k], wc[K + k], wc[2 * K + k], wc[3 * K + k]);
    }
#pragma unroll
    for (int i = 0; i < CF; i++) acc[i] = bias;
    // Every input frame's loads first (from a clamped in-bounds address, zeroed after), so the wave
    // waits for one memory round trip rather than one per frame.
    float4 xs[SPAN], gs[SPAN];
#pragma unroll
    for (int r = 0; r < SPAN; r++) {
      const int src = f0 - pad + r;
      const size_t at = (size_t)(src >= 0 && src < lim ? src : 0) * fw;
      xs[r] = *(const float4 *)(hs + at + (on ? ox : 0));
      if (layout != GLU_DONE) gs[r] = *(const float4 *)(hs + at + (on ? og : 0));
    }
#pragma unroll
    for (int r = 0; r < SPAN; r++) {
      const int src = f0 - pad + r;
      float4 v = make_float4(0, 0, 0, 0);
      if (on && src >= 0 && src < lim) {
        const float4 x = xs[r];
        if (layout == GLU_DONE) {
          v = x;
        } else {
          // GLU: a·σ(b), σ by the hardware reciprocal (1 ulp) as a·(1 / (1 + e^−b)), the reference's
          // two roundings, instead of an IEEE division (~10 instructions) on every input frame of the span.
          const float4 gt = gs[r];
          v.x = x.x * __builtin_amdgcn_rcpf(1.0f + __expf(-gt.x));
          v.y = x.y * __builtin_amdgcn_rcpf(1.0f + __expf(-gt.y));
          v.z = x.z * __builtin_amdgcn_rcpf(1.0f + __expf(-gt.z));
          v.w = x.w * __builtin_amdgcn_rcpf(1.0f + __expf(-gt.w));
        }
      }
      // Output frame i takes tap k = r − i.
#pragma unroll
      for (int i = 0; i < CF; i++) {
        const int k = r - i;
        if (k >= 0 && k < K) {
          acc[i].x += tap[k].x * v.x;
          acc[i].y += tap[k].y * v.y;
          acc[i].z += tap[k].z * v.z;
          acc[i].w += tap[k].w * v.w;
        }
      }
    }
  }
  float mean[CF], rstd[CF];
#pragma unroll
  for (int i = 0; i < CF; i++) mean[i] = 0.0f, rstd[i] = 1.0f;
  if (layer_norm) {
    // Mean, then the variance about it, over the ch channels of each frame.
#pragma unroll
    for (int i = 0; i < CF; i++) {
      const float s = on ? (acc[i].x + acc[i].y) + (acc[i].z + acc[i].w) : 0.0f;
      const float ws = wave_sum(s);
      if (lane == 0) red[0][wave][i] = ws;
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < CF; i++) {
      float s = 0.0f;
      for (int q = 0; q < nw; q++) s += red[0][q][i];
      mean[i] = s / (float)ch;
      float qv = 0.0f;
      if (on) {
        const float dx = acc[i].x - mean[i], dy = acc[i].y - mean[i], dz = acc[i].z - mean[i], dw = acc[i].w - mean[i];
        qv = (dx * dx + dy * dy) + (dz * dz + dw * dw);
      }
      const float ws = wave_sum(qv);
      if (lane == 0) red[1][wave][i] = ws;
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < CF; i++) {
      float s = 0.0f;
      for (int q = 0; q < nw; q++) s += red[1][q][i];
      rstd[i] = rsqrtf(s / (float)ch + 1e-5f);
    }
  }
  if (!on) return;
#pragma unroll
  for (int i = 0; i < CF; i++) {
    const int f = f0 + i;
    if (f >= t) break;
    float4 v;
    v.x = (acc[i].x - mean[i]) * rstd[i] * gg.x + bb.x;
    v.y = (acc[i].y - mean[i]) * rstd[i] * gg.y + bb.y;
    v.z = (acc[i].z - mean[i]) * rstd[i] * gg.z + bb.z;
    v.w = (acc[i].w - mean[i]) * rstd[i] * gg.w + bb.w;
    v.x = v.x * __builtin_amdgcn_rcpf(1.0f + __expf(-v.x));  // SiLU, as the GLU above
    v.y = v.y * __builtin_amdgcn_rcpf(1.0f + __expf(-v.y));
    v.z = v.z * __builtin_amdgcn_rcpf(1.0f + __expf(-v.z));
    v.w = v.w * __builtin_amdgcn_rcpf(1.0f + __expf(-v.w));
    store4(y + ((size_t)seg * t + f) * ch + c, v);
  }
}

__host__ __device__ __forceinline__ int half_len(int n) { return (n - 1) / 2 + 1; }

// Depthwise 3×3 stride-2 pad-1 conv + bias over the image [t][f][ch]; x holds rows 2·t0 − 1..;
// output rows t0 + blockIdx.y of y [⌈t/2⌉][⌈f/2⌉][ch] (spatial.wgsl:31-48), f32 or, for a consumer
// that rounds it to f16 anyway (a GEMM), f16 (TO).
template <typename TO>
__global__ void depthwise_kernel(const float *__restrict__ x, const float *__restrict__ w, const float *__restrict__ b,
                                 TO *__restrict__ y, int t, int f, int ch, int t0) {
  const int fo = blockIdx.x, k = blockIdx.y, fh = half_len(f);
  for (int c = threadIdx.x; c < ch; c += blockDim.x) {
    // The 9 taps and inputs loaded first (clamped to an in-bounds element, unused ones skipped
    // below): one memory round trip rather than one per tap behind its bounds test.
    float wv[9], xv[9];
#pragma unroll
    for (int i = 0; i < 3; i++) {
      const int ti = 2 * (t0 + k) + i;
#pragma unroll
      for (int j = 0; j < 3; j++) {
        const int fi = 2 * fo + j;
        const bool in = ti >= 1 && ti <= t && fi >= 1 && fi <= f;
        wv[i * 3 + j] = w[(i * 3 + j) * ch + c];
        xv[i * 3 + j] = x[in ? ((size_t)(2 * k + i) * f + fi - 1) * ch + c : (size_t)c];
      }
    }
    float acc = b[c];
#pragma unroll
    for (int i = 0; i < 3; i++) {
      const int ti = 2 * (t0 + k) + i;
#pragma unroll
      for (int j = 0; j < 3; j++) {
        const int fi = 2 * fo + j;
        if (ti >= 1 && ti <= t && fi >= 1 && fi <= f) acc = fmaf(wv[i * 3 + j], xv[i * 3 + j], acc);
      }
    }
    y[((size_t)(t0 + k) * fh + fo) * ch + c] = (TO)as_f32(acc);
  }
}

// The same conv for ch % 4 == 0 and 16-byte aligned rows: a thread makes DW_COLS consecutive output
// columns of 4 channels (item (row, column group, channel quad), quads fastest), its 3 × (2·DW_COLS + 1)
// input quads and 9 tap quads all loaded before the first product (one memory round trip; adjacent
// outputs share their edge column), the sums in the same tap order as depthwise_kernel.
constexpr int DW_COLS = 4;
template <typename TO>
__global__ __launch_bounds__(256) void depthwise4_kernel(const float *__restrict__ x, const float *__restrict__ w,
                                                         const float *__restrict__ b, TO *__restrict__ y, int t, int f,
                                                         int ch, int t0, int rows) {
  constexpr int NI = 2 * DW_COLS + 1;
  const int q4 = ch / 4, fh = half_len(f), groups = (fh + DW_COLS - 1) / DW_COLS;
  const long item = (long)blockIdx.x * blockDim.x + threadIdx.x;
  if (item >= (long)rows * groups * q4) return;
  const int c4 = (int)(item % q4), grp = (int)((item / q4) % groups), k = (int)(item / ((long)q4 * groups));
  const int fo0 = grp * DW_COLS, c = 4 * c4;
  float4 xv[3][NI], wv[9];
#pragma unroll
  for (int i = 0; i < 3; i++) {
    const int ti = 2 * (t0 + k) + i;
#pragma unroll
    for (int jj = 0; jj < NI; jj++) {
      const int fi = 2 * fo0 + jj;  // input column fi − 1 (padding at fi = 0 and past f)
      const bool in = ti >= 1 && ti <= t && fi >= 1 && fi <= f;
      xv[i][jj] = *(const float4 *)(x + (in ? ((size_t)(2 * k + i) * f + fi - 1) * ch + c : (size_t)c));
    }
  }
#pragma unroll
  for (int q = 0; q < 9; q++) wv[q] = *(const float4 *)(w + (size_t)q * ch + c);
  const float4 bias = *(const float4 *)(b + c);
#pragma unroll
  for (int o = 0; o < DW_COLS; o++) {
    const int fo = fo0 + o;
    if (fo >= fh) break;
    float4 acc = bias;
#pragma unroll
    for (int i = 0; i < 3; i++) {
      const int ti = 2 * (t0 + k) + i;
#pragma unroll
      for (int j = 0; j < 3; j++) {
        const int fi = 2 * fo + j;
        if (ti >= 1 && ti <= t && fi >= 1 && fi <= f) {
          const float4 a = wv[i * 3 + j], v = xv[i][2 * o + j];
          acc.x = fmaf(a.x, v.x, acc.x), acc.y = fmaf(a.y, v.y, acc.y);
          acc.z = fmaf(a.z, v.z, acc.z), acc.w = fmaf(a.w, v.w, acc.w);
        }
      }
    }
    store4(y + ((size_t)(t0 + k) * fh + fo) * ch + c, acc);
  }
}

// conv0 (1 → ch, 3×3 s2 p1) + ReLU, never stored, then the depthwise conv2 + bias, into rows
// 2·blockIdx.y and 2·blockIdx.y + 1 of a chunk (chunk row q is output row 2·t0 − 1 + q; rows from ⌈t/4⌉
// on zero, as masked) (spatial.wgsl:50-107; src/parakeet/cpu.rs:103-152).  A workgroup makes two
// whole output rows, one thread per channel: their 11 × (4·f2 + 3) input patch goes to LDS once, each
// thread keeps its channel's 18 taps in registers across the f2 positions, and the two rows share the
// conv0 row between them (5 conv0 rows per column, not 6).  Along the columns, the conv0 values and
// the input chunk a column shares with the next are carried over.  Output f32 or f16 (TO), as above.
template <typename TO>
__global__ void first_depthwise_kernel(const float *__restrict__ x, const float *__restrict__ w,
                                       const float *__restrict__ b, TO *__restrict__ y,
                                       const float *__restrict__ w0, const float *__restrict__ b0, int t,
                                       int f, int ch, int t0, int rows) {
  // FD_ROWS rows × pw columns; column 4·fo + j is input column 4·fo + j − 3
  extern __shared__ __attribute__((aligned(16))) float xs[];
  constexpr int FD_ROWS = 11;
  const int t1 = half_len(t), f1 = half_len(f), f2 = half_len(f1);
  const int q0 = 2 * blockIdx.y;  // the workgroup's first chunk row
  const int r = 2 * t0 + q0;      // its output row + 1
  const int pw = 4 * f2 + 4;      // the 4·f2 + 3 columns used, rows padded to 16 bytes
  // The patch (input rows 4r − 7 .. 4r + 3): every load of a thread issued before its stores (one
  // round trip, not one per element group), from clamped addresses, for the first 8 groups of
  // blockDim.x elements (the whole patch of 128 mel bins with 256 threads); any rest by the loop after.
  {
    constexpr int G = 8;
    float v[G];
#pragma unroll
    for (int q = 0; q < G; q++) {
      const int e = min((int)threadIdx.x + q * (int)blockDim.x, FD_ROWS * pw - 1);
      const int tm = 4 * r + e / pw - 7, fm = e % pw - 3;
      const bool in = tm >= 0 && tm < t && fm >= 0 && fm < f;
      const float xv = x[in ? (size_t)tm * f + fm : 0];
      v[q] = in ? xv : 0.0f;
    }
#pragma unroll
    for (int q = 0; q < G; q++) xs[min((int)threadIdx.x + q * (int)blockDim.x, FD_ROWS * pw - 1)] = v[q];
    for (int e = threadIdx.x + G * blockDim.x; e < FD_ROWS * pw; e += blockDim.x) {
      const int tm = 4 * r + e / pw - 7, fm = e % pw - 3;
      xs[e] = (tm >= 0 && tm < t && fm >= 0 && fm < f) ? x[(size_t)tm * f + fm] : 0.0f;
    }
  }
  __syncthreads();
  const bool masked0 = r > half_len(t1), masked1 = r + 1 > half_len(t1), second = q0 + 1 < rows;
  for (int c = threadIdx.x; c < ch; c += blockDim.x) {
    float a[9], wd[9];
#pragma unroll
    for (int q = 0; q < 9; q++) a[q] = w0[q * ch + c], wd[q] = w[q * ch + c];
    const float bias0 = b0[c], bias = b[c];
    // ReLU(conv0) at conv1 rows 2r − 2 + u (u = 0..4) and columns 2·fo + jj (jj = 0..2).  Taps on
    // padding (a row or column outside 1..t1, 1..f1) contribute zero, so every tap is summed without a
    // branch: the rows' factor is folded into output row o's taps wm[o] once, the columns' into the
    // values (column 2·fo + 1 ≤ 2·f2 − 1 ≤ f1 is always inside; 2·fo + 2 not at the last column when
    // f1 is odd; column jj = 0 is the previous column's jj = 2, and padding for fo = 0).  The factors
    // are multiplied in, not selected: a select lets the compiler branch around each conv0 sum, which
    // splits the column into dozens of blocks.
    float wm[2][9];
#pragma unroll
    for (int o = 0; o < 2; o++)
#pragma unroll
      for (int i = 0; i < 3; i++) {
        const int ti = 2 * (r + o) + i - 2;
        const float rv = ti >= 1 && ti <= t1 ? 1.0f : 0.0f;
#pragma unroll
        for (int j = 0; j < 3; j++) wm[o][i * 3 + j] = wd[i * 3 + j] * rv;
      }
    float cv[5][3];
#pragma unroll
    for (int u = 0; u < 5; u++) cv[u][2] = 0.0f;
    // The 11 × 8 input window of column fo (patch columns 4·fo .. 4·fo + 7) as two 16-byte chunks per
    // row, the second of which is the next column's first: two buffers that swap roles every column
    // (the loop unrolled by two, so no chunk is copied).
    float4 ca[FD_ROWS], cb[FD_ROWS];
    const auto column = [&](int fo, const float4 *lo, float4 *hi) {
#pragma unroll
      for (int rr = 0; rr < FD_ROWS; rr++) hi[rr] = ((const float4 *)xs)[rr * (pw / 4) + fo + 1];
      const float c2 = 2 * fo + 2 <= f1 ? 1.0f : 0.0f;
#pragma unroll
      for (int u = 0; u < 5; u++) {
        cv[u][0] = cv[u][2];
#pragma unroll
        for (int jj = 1; jj < 3; jj++) {
          float v = bias0;
#pragma unroll
          for (int d = 0; d < 3; d++) {
            const float4 l = lo[2 * u + d], h = hi[2 * u + d];
            const float row[8] = {l.x, l.y, l.z, l.w, h.x, h.y, h.z, h.w};
#pragma unroll
            for (int e = 0; e < 3; e++) v = fmaf(a[3 * d + e], row[2 * jj + e], v);
          }
          cv[u][jj] = jj == 2 ? fmaxf(v, 0.0f) * c2 : fmaxf(v, 0.0f);
        }
      }
#pragma unroll
      for (int o = 0; o < 2; o++) {
        float acc = bias;
#pragma unroll
        for (int i = 0; i < 3; i++)
#pragma unroll
          for (int j = 0; j < 3; j++) acc = fmaf(wm[o][i * 3 + j], cv[2 * o + i][j], acc);
        acc = as_f32(acc);
        if (o == 0) y[((size_t)q0 * f2 + fo) * ch + c] = (TO)(masked0 ? 0.0f : acc);
        else if (second) y[((size_t)(q0 + 1) * f2 + fo) * ch + c] = (TO)(masked1 ? 0.0f : acc);
      }
    };
#pragma unroll
    for (int rr = 0; rr < FD_ROWS; rr++) ca[rr] = ((const float4 *)xs)[rr * (pw / 4)];
    for (int fo = 0; fo < f2; fo += 2) {
      column(fo, ca, cb);
      if (fo + 1 < f2) column(fo + 1, cb, ca);
    }
  }
}

// [t][f][ch] → [t][ch·f] (spatial.wgsl:112-119), f and ch powers of two with f·ch ≤ 256·P: a frame's
// f × ch block through LDS, read and written coalesced (the strided reads of the plain kernel below
// touch one float per 1 KiB), every load before any store.  LDS rows are padded by 4 floats, so the
// transposed reads of 64 lanes (16 rows × 4 columns) hit 64 distinct banks when ch % 64 == 0.
// Elements of type T (f32, or f16 between a GEMM's f16 output and the next GEMM).
template <int P, typename T>
__global__ __launch_bounds__(256) void flatten_lds_kernel(const T *__restrict__ x, T *__restrict__ y, int lf, int lch) {
  extern __shared__ float tl[];
  const int n = 1 << (lf + lch), cp = (1 << lch) + 4, tid = threadIdx.x;
  const T *xr = x + (size_t)blockIdx.x * n;
  T *yr = y + (size_t)blockIdx.x * n;
  float v[P];
#pragma unroll
  for (int q = 0; q < P; q++) v[q] = (float)xr[min(tid + 256 * q, n - 1)];  // clamped: no branch
#pragma unroll
  for (int q = 0; q < P; q++) {
    const int e = min(tid + 256 * q, n - 1);  // input element e = fi·ch + c (past n: the last again)
    tl[(e >> lch) * cp + (e & ((1 << lch) - 1))] = v[q];
  }
  __syncthreads();
#pragma unroll
  for (int q = 0; q < P; q++) {
    const int e = tid + 256 * q;  // output element e = c·f + fi
    if (e < n) yr[e] = (T)tl[(e & ((1 << lf) - 1)) * cp + (e >> lf)];
  }
}

template <typename T>
__global__ void flatten_kernel(const T *__restrict__ x, T *__restrict__ y, int f, int ch) {
  const int n = f * ch;
  const T *xr = x + (size_t)blockIdx.x * n;
  T *yr = y + (size_t)blockIdx.x * n;
  for (int e = threadIdx.x; e < n; e += blockDim.x) yr[e] = xr[(e % f) * ch + e / f];
}

// Index of the first maximum of x[..n] (ops.wgsl:266-287), one workgroup.
__global__ __launch_bounds__(256) void argmax_kernel(const float *__restrict__ x, uint32_t *out, int n) {
  __shared__ float bv[4];
  __shared__ int bi[4];
  float best = -INFINITY;
  int idx = 0x7fffffff;
  for (int i = threadIdx.x; i < n; i += 256) {
    float v = x[i];
    if (v > best || (v == best && i < idx)) best = v, idx = i;
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    float ov = __shfl_xor(best, o, 64);
    int oi = __shfl_xor(idx, o, 64);
    if (ov > best || (ov == best && oi < idx)) best = ov, idx = oi;
  }
  if ((threadIdx.x & 63) == 0) bv[threadIdx.x >> 6] = best, bi[threadIdx.x >> 6] = idx;
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < 4; w++)
      if (bv[w] > best || (bv[w] == best && bi[w] < idx)) best = bv[w], idx = bi[w];
    // All NaN or n == 0: index 0.
    out[0] = (uint32_t)(idx == 0x7fffffff ? 0 : idx);
  }
}

__global__ void zero_kernel(uint32_t *p, size_t words) {
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  for (; i < words; i += (size_t)gridDim.x * blockDim.x) p[i] = 0u;
}

__global__ void zero_bytes_kernel(uint8_t *p, size_t bytes) {
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < bytes) p[i] = 0;
}

// 16-byte copy: each thread moves four 16-byte pieces per round (a workgroup's 16 KiB in flight
// before any store), streaming past the caches (non-temporal loads and stores).
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
__global__ __launch_bounds__(256) void copy16_kernel(u32x4 *__restrict__ y, const u32x4 *__restrict__ x, size_t n) {
  constexpr int U = 4;
  for (size_t i = (size_t)blockIdx.x * 256 * U + threadIdx.x; i < n; i += (size_t)gridDim.x * 256 * U) {
    u32x4 v[U];
#pragma unroll
    for (int u = 0; u < U; u++)
      if (i + 256 * u < n) v[u] = __builtin_nontemporal_load(x + i + 256 * u);
#pragma unroll
    for (int u = 0; u < U; u++)
      if (i + 256 * u < n) __builtin_nontemporal_store(v[u], y + i + 256 * u);
  }
}

// The finish of a k-split GEMM with the residual epilogue, fused with the LayerNorm of its result:
// x[row] += alpha·(Σ_z part[z][row] + bias) (the partial sums added in split order from 0, the W
// padding columns ≥ wrows contributing epi(0 + bias) as the GEMM gives them), then y = LN(x[row])
// with the arithmetic of layer_norm_kernel.  res = 0: the bias epilogue instead, x[row] = Σ + bias
// (alpha 1, x not read).  One wavefront per row; NJ as in layer_norm_kernel, and
// every load (partial sums, bias, x, the norms' weights) issued before the first use.
template <typename OT, int NSPLIT, int NJ>
__global__ __launch_bounds__(256) void split_residual_ln_kernel(const float *__restrict__ part, int splits,
                                                                const float *__restrict__ bias, int wrows, float alpha,
                                                                float *__restrict__ x, const float *__restrict__ g,
                                                                const float *__restrict__ b, OT *__restrict__ y,
                                                                int rows, int cols, int keep_x,
                                                                const float *__restrict__ g2,
                                                                const float *__restrict__ b2,
                                                                _Float16 *__restrict__ y2, int res) {
  constexpr int J = NJ ? NJ : ROW_REGS / 4;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int row = blockIdx.x * 4 + w;
  if (row >= rows) return;
  const int q4 = cols / 4;
  const size_t plane = (size_t)rows * cols;
  float4 *xr = (float4 *)(x + (size_t)row * cols);
  const float4 *pr = (const float4 *)(part + (size_t)row * cols), *b4 = (const float4 *)bias;
  const float4 *g4 = (const float4 *)g, *lb4 = (const float4 *)b;
  const float4 *g24 = (const float4 *)g2, *b24 = (const float4 *)b2;
  const float4 z4 = make_float4(0, 0, 0, 0);
  auto in = [&](int j) { return NJ || lane + 64 * j < q4; };
  float4 v[J], gg[J], bb[J], gg2[J], bb2[J];
  if constexpr (NSPLIT > 0) {
    float4 p[NSPLIT][J], bi[J], c[J];
#pragma unroll
    for (int j = 0; j < J; j++) {
      const int i = lane + 64 * j;
#pragma unroll
      for (int z = 0; z < NSPLIT; z++) p[z][j] = in(j) ? pr[z * (plane / 4) + i] : z4;
      bi[j] = in(j) ? b4[i] : z4;
      c[j] = res && in(j) ? xr[i] : z4;
    }
#pragma unroll
    for (int j = 0; j < J; j++) {
      gg[j] = in(j) ? g4[lane + 64 * j] : z4;
      bb[j] = in(j) ? lb4[lane + 64 * j] : z4;
      if (g2) gg2[j] = in(j) ? g24[lane + 64 * j] : z4, bb2[j] = in(j) ? b24[lane + 64 * j] : z4;
    }
#pragma unroll
    for (int j = 0; j < J; j++) {
      float4 acc = z4;
#pragma unroll
      for (int z = 0; z < NSPLIT; z++) acc.x += p[z][j].x, acc.y += p[z][j].y, acc.z += p[z][j].z, acc.w += p[z][j].w;
      const int i = lane + 64 * j;
      if (4 * i + 0 >= wrows) acc.x = 0.0f;
      if (4 * i + 1 >= wrows) acc.y = 0.0f;
      if (4 * i + 2 >= wrows) acc.z = 0.0f;
      if (4 * i + 3 >= wrows) acc.w = 0.0f;
      v[j] = make_float4(c[j].x + alpha * (acc.x + bi[j].x), c[j].y + alpha * (acc.y + bi[j].y),
                         c[j].z + alpha * (acc.z + bi[j].z), c[j].w + alpha * (acc.w + bi[j].w));
    }
  } else {
#pragma unroll
    for (int j = 0; j < J; j++) {
      const int i = lane + 64 * j;
      v[j] = z4;
      if (in(j)) {
        float4 acc = z4;
        for (int z = 0; z < splits; z++) {
          const float4 p = pr[z * (plane / 4) + i];
          acc.x += p.x, acc.y += p.y, acc.z += p.z, acc.w += p.w;
        }
        if (4 * i + 0 >= wrows) acc.x = 0.0f;
        if (4 * i + 1 >= wrows) acc.y = 0.0f;
        if (4 * i + 2 >= wrows) acc.z = 0.0f;
        if (4 * i + 3 >= wrows) acc.w = 0.0f;
        const float4 bi = b4[i], c = res ? xr[i] : z4;
        v[j] = make_float4(c.x + alpha * (acc.x + bi.x), c.y + alpha * (acc.y + bi.y), c.z + alpha * (acc.z + bi.z),
                           c.w + alpha * (acc.w + bi.w));
      }
    }
#pragma unroll
    for (int j = 0; j < J; j++) {
      gg[j] = in(j) ? g4[lane + 64 * j] : z4;
      bb[j] = in(j) ? lb4[lane + 64 * j] : z4;
      if (g2) gg2[j] = in(j) ? g24[lane + 64 * j] : z4, bb2[j] = in(j) ? b24[lane + 64 * j] : z4;
    }
  }
  float s = 0.0f;
#pragma unroll
  for (int j = 0; j < J; j++) {
    if (keep_x && in(j)) xr[lane + 64 * j] = v[j];
    s += (v[j].x + v[j].y) + (v[j].z + v[j].w);
  }
  const float mean = wave_sum(s) / (float)cols;
  float q = 0.0f;
#pragma unroll
  for (int j = 0; j < J; j++) {
    if (in(j)) {
      float dx = v[j].x - mean, dy = v[j].y - mean, dz = v[j].z - mean, dw = v[j].w - mean;
      q += (dx * dx + dy * dy) + (dz * dz + dw * dw);
    }
  }
  const float rstd = rsqrtf(wave_sum(q) / (float)cols + 1e-5f);
  OT *yy = y + (size_t)row * cols;
#pragma unroll
  for (int j = 0; j < J; j++) {
    if (in(j)) {
      float4 o;
      o.x = (v[j].x - mean) * rstd * gg[j].x + bb[j].x;
      o.y = (v[j].y - mean) * rstd * gg[j].y + bb[j].y;
      o.z = (v[j].z - mean) * rstd * gg[j].z + bb[j].z;
      o.w = (v[j].w - mean) * rstd * gg[j].w + bb[j].w;
      store4(yy + 4 * (lane + 64 * j), o);
      v[j] = o;
    }
  }
  if (!g2) return;
  // A second LayerNorm of y (the next block's first norm) into y2, from the registers.
  s = 0.0f;
#pragma unroll
  for (int j = 0; j < J; j++)
    if (in(j)) s += (v[j].x + v[j].y) + (v[j].z + v[j].w);
  const float mean2 = wave_sum(s) / (float)cols;
  q = 0.0f;
#pragma unroll
  for (int j = 0; j < J; j++) {
    if (in(j)) {
      float dx = v[j].x - mean2, dy = v[j].y - mean2, dz = v[j].z - mean2, dw = v[j].w - mean2;
      q += (dx * dx + dy * dy) + (dz * dz + dw * dw);
    }
  }
  const float rstd2 = rsqrtf(wave_sum(q) / (float)cols + 1e-5f);
  _Float16 *y2r = y2 + (size_t)row * cols;
#pragma unroll
  for (int j = 0; j < J; j++) {
    if (in(j)) {
      float4 o;
      o.x = (v[j].x - mean2) * rstd2 * gg2[j].x + bb2[j].x;
      o.y = (v[j].y - mean2) * rstd2 * gg2[j].y + bb2[j].y;
      o.z = (v[j].z - mean2) * rstd2 * gg2[j].z + bb2[j].z;
      o.w = (v[j].w - mean2) * rstd2 * gg2[j].w + bb2[j].w;
      store4(y2r + 4 * (lane + 64 * j), o);
    }
  }
}

__global__ void copy_bytes_kernel(uint8_t *__restrict__ y, const uint8_t *__restrict__ x, size_t n) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) y[i] = x[i];
}

__global__ void add_kernel(float *x, const float *a, size_t n) {
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  for (; i < n; i += (size_t)gridDim.x * blockDim.x) x[i] += a[i];
}

}  // namespace

int launch_layer_norm(wh_ctx *ctx, const float *x, const float *g, const float *b, void *y, int rows,
                      int cols, const float *table, void *yr, int hd, int out16) {
  if (rows < 0 || cols <= 0 || (rows && (!x || !g || !b || !y)))
    return wh_fail(ctx, WH_EARG, "layer_norm: bad arguments (%d x %d)", rows, cols);
  if (table && (!yr || hd <= 0 || hd % 2 || cols % hd))
    return wh_fail(ctx, WH_EARG, "layer_norm: rope needs cols %% head_dim == 0 and even head_dim");
  if (!rows) return WH_OK;
  ProfScope prof(ctx, "layer_norm", 0.0, (double)rows * cols * (4 + (out16 ? 2 : 4) * (table ? 2 : 1)));
  if (cols <= ROW_REGS * 64 && cols % 4 == 0 && (uintptr_t)x % 16 == 0 && (uintptr_t)y % 16 == 0 &&
      (uintptr_t)g % 16 == 0 && (uintptr_t)b % 16 == 0) {
    size_t lds = table ? (size_t)4 * cols * sizeof(float) : 0;
#define LN(OT, NJ) \
  wh_launch(ctx, layer_norm_kernel<OT, NJ>, (rows + 3) / 4, 256, lds, x, g, b, (OT *)y, rows, cols, table, (OT *)yr, hd)
    const int nj = cols % 256 ? 0 : cols / 256;
    if (out16) {
      if (nj == 3) LN(_Float16, 3);
      else if (nj == 4) LN(_Float16, 4);
      else if (nj == 5) LN(_Float16, 5);
      else LN(_Float16, 0);
    } else {
      if (nj == 3) LN(float, 3);
      else if (nj == 4) LN(float, 4);
      else if (nj == 5) LN(float, 5);
      else LN(float, 0);
    }
#undef LN
  } else {
    if (table || out16)
      return wh_fail(ctx, WH_EARG, "layer_norm: rope and f16 rows need cols %% 4 == 0, at most %d", ROW_REGS * 64);
    wh_launch(ctx, layer_norm_long, rows, 64, 0, x, g, b, (float *)y, cols);
  }
  return wh_launched(ctx, "layer_norm");
}

int launch_split_residual_ln(wh_ctx *ctx, const float *part, int splits, const float *bias, int wrows, float alpha,
                             float *x, const float *g, const float *b, void *y, int rows, int cols, int out16,
                             int keep_x, const float *g2, const float *b2, void *y2, int residual) {
  if (rows <= 0 || cols <= 0 || cols % 4 || cols > ROW_REGS * 64 || splits < 1 || !part || !bias || !x || !g || !b || !y ||
      (uintptr_t)part % 16 || (uintptr_t)bias % 16 || (uintptr_t)x % 16 || (uintptr_t)g % 16 || (uintptr_t)b % 16 ||
      (uintptr_t)y % 16 || (g2 && (!b2 || !y2 || (uintptr_t)g2 % 16 || (uintptr_t)b2 % 16 || (uintptr_t)y2 % 16)))
    return wh_fail(ctx, WH_EARG, "split_residual_ln: bad arguments (%d x %d, %d splits)", rows, cols, splits);
  ProfScope prof(ctx, "split_residual_ln", 0.0,
                 (double)rows * cols *
                     (4.0 * splits + (residual ? 4 : 0) + (keep_x ? 4 : 0) + (out16 ? 2 : 4) + (g2 ? 2 : 0)));
  const int grid = (rows + 3) / 4;
#define SRL(OT, N)                                                                                                   \
  do {                                                                                                               \
    if (cols == 1024 && N > 0)                                                                                       \
      wh_launch(ctx, split_residual_ln_kernel<OT, N, 4>, grid, 256, 0, part, splits, bias, wrows, alpha, x, g, b,      \
                (OT *)y, rows, cols, keep_x, g2, b2, (_Float16 *)y2, residual);                                 \
    else if (cols == 1280 && N > 0)                                                                                  \
      wh_launch(ctx, split_residual_ln_kernel<OT, N, 5>, grid, 256, 0, part, splits, bias, wrows, alpha, x, g, b,      \
                (OT *)y, rows, cols, keep_x, g2, b2, (_Float16 *)y2, residual);                                 \
    else                                                                                                             \
      wh_launch(ctx, split_residual_ln_kernel<OT, N, 0>, grid, 256, 0, part, splits, bias, wrows, alpha, x, g, b,      \
                (OT *)y, rows, cols, keep_x, g2, b2, (_Float16 *)y2, residual);                                 \
  } while (0)
  if (out16) {
    if (splits == 2) SRL(_Float16, 2);
    else if (splits == 4) SRL(_Float16, 4);
    else SRL(_Float16, 0);
  } else {
    if (splits == 2) SRL(float, 2);
    else if (splits == 4) SRL(float, 4);
    else SRL(float, 0);
  }
#undef SRL
  return wh_launched(ctx, "split_residual_ln");
}

int launch_im2col(wh_ctx *ctx, const float *x, float *col, int t, int ch, int kernel, int stride, int pad,
                  int batch, long xs, long cs) {
  if (t <= 0 || ch <= 0 || kernel <= 0 || stride <= 0 || pad < 0 || t + 2 * pad < kernel || batch <= 0)
    return wh_fail(ctx, WH_EARG, "im2col: bad shape");
  int rows = (t + 2 * pad - kernel) / stride + 1;
  int width = (ch * kernel + 31) / 32 * 32;
  dim3 grid((width + 255) / 256, rows, batch);
  ProfScope prof(ctx, "im2col", 0.0, 4.0 * batch * ((double)rows * width + (double)t * ch));
  wh_launch(ctx, im2col_kernel, grid, 256, 0, x, col, t, ch, kernel, stride, pad, rows, width, xs, cs);
  return wh_launched(ctx, "im2col");
}

template <typename OT>
static void conv_glu_k(wh_ctx *ctx, dim3 grid, int threads, const float *h, const float *w, const float *wb, int kernel,
                const float *g, const float *b, int layer_norm, OT *y, int t, int ch, const int *valid_dev, int valid,
                int layout) {
#define CG(K)                                                                                                      \
  case K:                                                                                                          \
    wh_launch(ctx, conv_glu_kernel<OT, K>, grid, threads, 0, h, w, wb, kernel, g, b, layer_norm, y, t, ch, valid_dev, \
              valid, layout);                                                                                      \
    break;
  switch (kernel) {
    CG(1) CG(3) CG(5) CG(7) CG(9) CG(11) CG(13) CG(15) CG(17) CG(19) CG(21) CG(23) CG(25) CG(27) CG(29) CG(31)
  }
#undef CG
}

int launch_conv_glu(wh_ctx *ctx, const float *h, const float *w, const float *wb, int kernel, const float *g,
                    const float *b, int layer_norm, void *y, int t, int ch, const int *valid_dev, int valid,
                    int batch, int out16, int layout) {
  if (t <= 0 || ch <= 0 || ch > 1024 || ch % 4 || kernel <= 0 || kernel % 2 == 0 || kernel > CG_MAXK || batch <= 0 ||
      layout < GLU_PLAIN || layout > GLU_DONE)
    return wh_fail(ctx, WH_EARG, "conv_glu: bad shape (t %d, ch %d, kernel %d): ch %% 4 == 0, ch <= 1024, odd kernel <= %d",
                   t, ch, kernel, CG_MAXK);
  if ((uintptr_t)h % 16 || (uintptr_t)w % 16 || (uintptr_t)wb % 16 || (uintptr_t)g % 16 || (uintptr_t)b % 16 ||
      (uintptr_t)y % 16)
    return wh_fail(ctx, WH_EARG, "conv_glu: buffers must be 16-byte aligned");
  const int frames = t * batch;
  ProfScope prof(ctx, "conv_glu", 0.0, ((layout == GLU_DONE ? 4.0 : 8.0) + (out16 ? 2.0 : 4.0)) * frames * ch);
  dim3 grid((t + CF - 1) / CF, batch);
  const int threads = (ch / 4 + 63) / 64 * 64;
  if (out16)
    conv_glu_k<_Float16>(ctx, grid, threads, h, w, wb, kernel, g, b, layer_norm, (_Float16 *)y, t, ch, valid_dev,
                         valid < 0 ? t : valid, layout);
  else
    conv_glu_k<float>(ctx, grid, threads, h, w, wb, kernel, g, b, layer_norm, (float *)y, t, ch, valid_dev,
                      valid < 0 ? t : valid, layout);
  return wh_launched(ctx, "conv_glu");
}

int launch_depthwise(wh_ctx *ctx, const float *x, const float *w0, const float *b0, const float *w,
                     const float *b, void *y, int t, int f, int ch, int t0, int rows, int out16) {
  if (t <= 0 || f <= 0 || ch <= 0 || t0 < 0 || rows < 0) return wh_fail(ctx, WH_EARG, "depthwise: bad shape");
  if (!rows) return WH_OK;
  int threads = ch >= 256 ? 256 : ((ch + 63) / 64) * 64;
  const double ob = out16 ? 2.0 : 4.0;  // output bytes per value
  ProfScope prof(ctx, w0 ? "first_depthwise" : "depthwise", 0.0,
                 rows * half_len(w0 ? half_len(f) : f) * ch * (w0 ? ob : ob + 4.0 * 4));
  if (w0) {
    const size_t lds = sizeof(float) * 11 * (4 * (size_t)half_len(half_len(f)) + 4);
    if (lds > 64 * 1024) return wh_fail(ctx, WH_EARG, "depthwise: %d mel bins is more than one workgroup's patch holds", f);
    const dim3 grid(1, (rows + 1) / 2);
    const int nt = threads < 64 ? 64 : threads;
    if (out16)
      wh_launch(ctx, first_depthwise_kernel<_Float16>, grid, nt, lds, x, w, b, (_Float16 *)y, w0, b0, t, f, ch, t0, rows);
    else wh_launch(ctx, first_depthwise_kernel<float>, grid, nt, lds, x, w, b, (float *)y, w0, b0, t, f, ch, t0, rows);
  } else if (ch % 4 == 0 && (uintptr_t)x % 16 == 0 && (uintptr_t)w % 16 == 0 && (uintptr_t)b % 16 == 0 &&
             (uintptr_t)y % (out16 ? 8 : 16) == 0) {
    const long items = (long)rows * ((half_len(f) + DW_COLS - 1) / DW_COLS) * (ch / 4);
    const int blocks = (int)((items + 255) / 256);
    if (out16) wh_launch(ctx, depthwise4_kernel<_Float16>, blocks, 256, 0, x, w, b, (_Float16 *)y, t, f, ch, t0, rows);
    else wh_launch(ctx, depthwise4_kernel<float>, blocks, 256, 0, x, w, b, (float *)y, t, f, ch, t0, rows);
  } else {
    const dim3 grid(half_len(f), rows);
    if (out16) wh_launch(ctx, depthwise_kernel<_Float16>, grid, threads, 0, x, w, b, (_Float16 *)y, t, f, ch, t0);
    else wh_launch(ctx, depthwise_kernel<float>, grid, threads, 0, x, w, b, (float *)y, t, f, ch, t0);
  }
  return wh_launched(ctx, "depthwise");
}

template <typename T>
static void flatten_t(wh_ctx *ctx, const T *x, T *y, int t, int f, int ch) {
  const bool pow2 = (f & (f - 1)) == 0 && (ch & (ch - 1)) == 0;
  if (pow2 && (long)f * ch <= 16 * 256) {
    const int lf = __builtin_ctz(f), lch = __builtin_ctz(ch);
    wh_launch(ctx, flatten_lds_kernel<16, T>, t, 256, sizeof(float) * (size_t)f * (ch + 4), x, y, lf, lch);
  } else {
    wh_launch(ctx, flatten_kernel<T>, t, 256, 0, x, y, f, ch);
  }
}

int launch_flatten(wh_ctx *ctx, const void *x, void *y, int t, int f, int ch, int f16) {
  if (t < 0 || f <= 0 || ch <= 0) return wh_fail(ctx, WH_EARG, "flatten: bad shape");
  if (!t) return WH_OK;
  ProfScope prof(ctx, "flatten", 0.0, (f16 ? 4.0 : 8.0) * t * f * ch);
  if (f16) flatten_t(ctx, (const _Float16 *)x, (_Float16 *)y, t, f, ch);
  else flatten_t(ctx, (const float *)x, (float *)y, t, f, ch);
  return wh_launched(ctx, "flatten");
}

int launch_argmax(wh_ctx *ctx, const float *x, uint32_t *out, int n) {
  if (n < 0 || !out) return wh_fail(ctx, WH_EARG, "argmax: bad arguments");
  wh_launch(ctx, argmax_kernel, 1, 256, 0, x, out, n);
  return wh_launched(ctx, "argmax");
}

__global__ void set_int_kernel(int *__restrict__ dst, int v) {
  if (threadIdx.x == 0) *dst = v;
}

int launch_set_int(wh_ctx *ctx, int *dst, int v) {
  if (!dst) return wh_fail(ctx, WH_EARG, "set_int: NULL");
  wh_launch(ctx, set_int_kernel, 1, 64, 0, dst, v);
  return wh_launched(ctx, "set_int");
}

int launch_zero(wh_ctx *ctx, void *dst, size_t bytes) {
  if (!bytes) return WH_OK;
  if (!dst) return wh_fail(ctx, WH_EARG, "zero: NULL");
  size_t words = bytes / 4;
  if ((uintptr_t)dst % 4 == 0 && words) {
    size_t blocks = (words + 255) / 256;
    wh_launch(ctx, zero_kernel, (unsigned)(blocks > 65535 ? 65535 : blocks), 256, 0, (uint32_t *)dst, words);
    if (bytes % 4)
      wh_launch(ctx, zero_bytes_kernel, 1, 4, 0, (uint8_t *)dst + words * 4, bytes % 4);
  } else {
    wh_launch(ctx, zero_bytes_kernel, (unsigned)((bytes + 255) / 256), 256, 0, (uint8_t *)dst, bytes);
  }
  return wh_launched(ctx, "zero");
}

int launch_copy(wh_ctx *ctx, void *dst, const void *src, size_t bytes) {
  if (!bytes) return WH_OK;
  if (!dst || !src) return wh_fail(ctx, WH_EARG, "copy: NULL");
  ProfScope prof(ctx, "copy", 0.0, 2.0 * bytes);
  const size_t n16 = ((uintptr_t)dst % 16 == 0 && (uintptr_t)src % 16 == 0) ? bytes / 16 : 0;
  if (n16) {
    const size_t blocks = std::min<size_t>((n16 + 1023) / 1024, 16384);
    wh_launch(ctx, copy16_kernel, (unsigned)blocks, 256, 0, (u32x4 *)dst, (const u32x4 *)src, n16);
  }
  const size_t rest = bytes - 16 * n16;
  if (rest) {
    const size_t blocks = std::min<size_t>((rest + 255) / 256, 8192);
    wh_launch(ctx, copy_bytes_kernel, (unsigned)blocks, 256, 0, (uint8_t *)dst + 16 * n16, (const uint8_t *)src + 16 * n16,
                                                                 rest);
  }
  return wh_launched(ctx, "copy");
}

int launch_add_rows(wh_ctx *ctx, float *x, const float *a, size_t n) {
  if (!n) return WH_OK;
  size_t blocks = (n + 255) / 256;
  wh_launch(ctx, add_kernel, (unsigned)(blocks > 65535 ? 65535 : blocks), 256, 0, x, a, n);
  return wh_launched(ctx, "add");
}
