// Decoder kernels for one token: the HBM-bound GEMV over GGUF weight bytes (Pass::gemv,
// src/gpu/mod.rs:1461-1467; gemm.wgsl:244-307), the embedding row (Pass::embed, :1469-1482;
// gemm.wgsl:309-327), attention of one query per head over an f16 K/V cache split into parts of
// 256 keys and their merge, in one launch (Pass::attend, :1484-1505; decode.wgsl:56-147), and packing f32 rows
// into that cache (Pass::pack, :1507-1523; decode.wgsl:148-173).
//
// The GEMV streams W once: a workgroup takes a run of whole rows, contiguous in HBM, and each thread
// one 16-byte (F16/F32) or block-pair (Q8_0/Q4_0) item of a row per step, so the workgroup's loads
// sweep the run's bytes in order; `a` sits in LDS.  Per block the int8 (or nibble) products are
// summed in f32 and scaled once, as ggml's mul_mv (gemm.wgsl:244-262); W is not rounded to f16.
#include <algorithm>

#include <cstdio>

#include "internal.h"
#include "xlane.h"

namespace {

__device__ __forceinline__ float half_bits(uint32_t h) { return (float)__builtin_bit_cast(_Float16, (uint16_t)h); }

__device__ __forceinline__ float gelu(float x) {
  float z = fabsf(0.70710678118654752440f * x);
  float t = 1.0f / (1.0f + 0.3275911f * z);
  float e = 1.0f - (((((1.061405429f * t - 1.453152027f) * t) + 1.421413741f) * t - 0.284496736f) * t +
                     0.254829592f) * t * __expf(-z * z);
  float s = x > 0.0f ? 1.0f : (x < 0.0f ? -1.0f : 0.0f);
  return 0.5f * x * (1.0f + s * e);
}

__device__ __forceinline__ float epilogue(int epi, float alpha, float v, float c) {
  switch (epi) {
    case WH_SILU: return v / (1.0f + __expf(-v));
    case WH_RELU: return fmaxf(v, 0.0f);
    case WH_RESIDUAL: return c + alpha * v;
    case WH_GELU: return gelu(v);
    case WH_GELU_RESIDUAL: return c + gelu(v);
    case WH_TANH: return tanhf(fminf(fmaxf(v, -10.0f), 10.0f));
    default: return v;
  }
}

// Items per row and weights per item of each type's GEMV.
template <int WT, bool PAIR>
struct Item {
  static constexpr int W = WT == WH_F32 ? 4 : (WT == WH_F16 ? 8 : (PAIR ? 64 : 32));
};

// Σ over one item of W (row bytes `wr`, item index `it`) times a (in LDS).
template <int WT, bool PAIR>
__device__ __forceinline__ float item_dot(const uint8_t *__restrict__ wr, int it, const float *as) {
  if constexpr (WT == WH_F32) {
    float4 w = *(const float4 *)(wr + (size_t)it * 16);
    const float *x = as + 4 * it;
    return w.x * x[0] + w.y * x[1] + w.z * x[2] + w.w * x[3];
  } else if constexpr (WT == WH_F16) {
    uint4 w = *(const uint4 *)(wr + (size_t)it * 16);
    const float *x = as + 8 * it;
    uint32_t u[4] = {w.x, w.y, w.z, w.w};
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; i++) s += half_bits(u[i] & 0xffffu) * x[2 * i] + half_bits(u[i] >> 16) * x[2 * i + 1];
    return s;
  } else {
    constexpr int BLK = WT == WH_Q8_0 ? 34 : 18;
    constexpr int NB = PAIR ? 2 : 1;
    float total = 0.0f;
    if constexpr (PAIR) {
      constexpr int DW = WT == WH_Q8_0 ? 17 : 9;
      const uint32_t *p = (const uint32_t *)(wr + (size_t)it * 2 * BLK);
      uint32_t q[DW + 1];
#pragma unroll
      for (int i = 0; i < DW; i++) q[i] = p[i];
      q[DW] = 0;
#pragma unroll
      for (int b = 0; b < 2; b++) {
        // Block 0: scale in q[0] low half, data from byte 2; block 1: scale in the high half of
        // dword BLK/4 (byte BLK), data from byte BLK + 2 (dword-aligned).
        constexpr int S1 = BLK / 4;
        float d = half_bits(b ? (q[S1] >> 16) : (q[0] & 0xffffu));
        const float *x = as + 32 * (2 * it + b);
        float s = 0.0f;
        if constexpr (WT == WH_Q8_0) {
#pragma unroll
          for (int j = 0; j < 8; j++) {
            uint32_t v = b ? q[S1 + 1 + j] : __builtin_amdgcn_alignbyte(q[j + 1], q[j], 2);
#pragma unroll
            for (int e = 0; e < 4; e++) s += (float)(int8_t)(v >> (8 * e)) * x[4 * j + e];
          }
        } else {
#pragma unroll
          for (int j = 0; j < 4; j++) {
            uint32_t v = b ? q[S1 + 1 + j] : __builtin_amdgcn_alignbyte(q[j + 1], q[j], 2);
#pragma unroll
            for (int e = 0; e < 4; e++) {
              uint32_t by = (v >> (8 * e)) & 0xffu;
              s += (float)((int)(by & 15u) - 8) * x[4 * j + e] + (float)((int)(by >> 4) - 8) * x[16 + 4 * j + e];
            }
          }
        }
        total += s * d;
      }
    } else {
      constexpr int HW = WT == WH_Q8_0 ? 17 : 9;
      const uint16_t *p = (const uint16_t *)(wr + (size_t)it * BLK);
      uint16_t h[HW];
#pragma unroll
      for (int i = 0; i < HW; i++) h[i] = p[i];
      float d = half_bits(h[0]);
      const float *x = as + 32 * it;
      float s = 0.0f;
#pragma unroll
      for (int i = 1; i < HW; i++) {
        uint32_t lo = h[i] & 0xffu, hi = h[i] >> 8;
        int e = 2 * (i - 1);
        if constexpr (WT == WH_Q8_0) {
          s += (float)(int8_t)lo * x[e] + (float)(int8_t)hi * x[e + 1];
        } else {
          s += (float)((int)(lo & 15u) - 8) * x[e] + (float)((int)(lo >> 4) - 8) * x[16 + e];
          s += (float)((int)(hi & 15u) - 8) * x[e + 1] + (float)((int)(hi >> 4) - 8) * x[16 + e + 1];
        }
      }
      total = s * d;
    }
    (void)NB;
    return total;
  }
}

// c[offset + j] = epi(a·W[j] + bias[j]): one wavefront per pair of rows, lanes striding over the
// row's items, reduced by shuffles; a workgroup of 4 waves covers 8 consecutive rows.  Rows past W's
// real ones are epi(0) up to `cols` (the reference's padding columns).
template <int WT, bool PAIR>
__global__ __launch_bounds__(256) void gemv_wave_kernel(const float *__restrict__ a, const uint8_t *__restrict__ w,
                                                        const float *__restrict__ bias, float *__restrict__ c,
                                                        int rows, int cols, int k, size_t row_bytes, int epi,
                                                        float alpha, int offset) {
  extern __shared__ float as[];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  for (int i = tid; i < k; i += 256) as[i] = a[i];
  __syncthreads();
  constexpr int WPI = Item<WT, PAIR>::W;
  const int items = k / WPI;
  // Rows of this wave: 2 at a time so two rows' loads are in flight.
  const int row0 = (blockIdx.x * 4 + wave) * 2;
#pragma unroll
  for (int rr = 0; rr < 2; rr++) {
    const int row = row0 + rr;
    if (row >= cols) break;
    float s = 0.0f;
    if (row < rows) {
      const uint8_t *wr = w + (size_t)row * row_bytes;
      for (int it = lane; it < items; it += 64) s += item_dot<WT, PAIR>(wr, it, as);
    }
    s = xlane::wave_sum(s);
    if (lane == 0) {
      float *cp = c + offset + row;
      *cp = epilogue(epi, alpha, s + bias[row], *cp);
    }
  }
}

// ------------------------------------------------------------------- streaming GEMV (k % 64 == 0)

// LDS DMA from a wave-uniform base plus a per-lane byte offset (16 bytes or 4 bytes per lane) to LDS
// lds + 16·lane (4·lane); counted by vmcnt.
__device__ __forceinline__ void gv_dma16(const void *base, uint32_t off, uint32_t lds) {
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(base), "{m0}"(lds) : "memory");
}
__device__ __forceinline__ void gv_dma4(const void *base, uint32_t off, uint32_t lds) {
  asm volatile("s_nop 0\n\tglobal_load_lds_dword %0, %1" ::"v"(off), "s"(base), "{m0}"(lds) : "memory");
}
__device__ __forceinline__ uint32_t gv_lds_addr(const void *p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)p;
}
template <int N>
__device__ __forceinline__ void gv_wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

struct GemvArgs {
  const float *a;
  const uint8_t *w;
  const float *bias;
  float *c;
  int rows, cols, k, epi, offset;
  const float *ln_g, *ln_b;  // non-null: the product takes LayerNorm(a; ln_g, ln_b)
  GemvPack pack;             // pack.cache non-null: outputs lo .. lo + 2d also into the cache column
  float alpha;
  int row_bytes;
  int rps;        // rows per stage
  int stages;     // ceil(rows / rps)
  int per_wg;     // stages per workgroup
  size_t total;   // rows · row_bytes
};

constexpr int GV_NS = 3;       // LDS stages per workgroup (two in flight while one is used)
constexpr int GV_STAGE = 16384;  // bytes per stage (whole DMA instructions of 1 KiB)

// c[offset + j] = epi(a·W[j] + bias[j]) for rows j of W streamed from HBM: a workgroup takes a run
// of stages, each `rps` consecutive rows (≤ 16 KiB, contiguous in HBM), and keeps GV_NS − 1 stages
// in flight by LDS DMA (16-byte lanes when rows are 16-byte multiples, else 4-byte lanes), so the
// chip holds tens of MB of loads in flight.  Each thread takes one 64-weight item (a Q8_0 or Q4_0
// block pair, or 64 F16 weights) of one row of the stage from LDS, `a` from LDS, and sums the
// products in f32 (per block Σ q·a, then × d, as gemm.wgsl:244-262); a row's items are summed in
// order through LDS.  W is not rounded (Pass::gemv semantics).
__device__ __forceinline__ float gv_wave_sum(float v) { return xlane::wave_sum(v); }

template <int WT, bool D16>
__global__ __launch_bounds__(256) void gemv_stream_kernel(GemvArgs P) {
  constexpr int ITEM = WT == WH_Q8_0 ? 68 : WT == WH_Q4_0 ? 36 : 128;  // bytes of 64 weights
  constexpr int LANE = D16 ? 16 : 4;                                   // bytes per lane per DMA
  constexpr int NI = GV_STAGE / (64 * LANE);                           // DMA instructions per stage
  constexpr int PER = NI / 4;                                          // per wave (4 waves)
  constexpr int AS = 68;  // floats per item of a in LDS: 64 + 4, so items start 4 banks apart
  static_assert(NI % 4 == 0 && (GV_NS - 2) * PER < 64, "vmcnt range");
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  uint8_t *st = smem;                                                  // GV_NS stages
  const int items = P.k / 64;
  float *as = (float *)(smem + GV_NS * GV_STAGE);                      // a: items × AS
  float *part = as + items * AS;          // every stage's 256 partial sums (per_wg × 256), summed after the loop
  float *rsum = part + 256 * P.per_wg;    // the workgroup's row sums
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int s0 = blockIdx.x * P.per_wg, s1 = min(s0 + P.per_wg, P.stages);
  const size_t stage_bytes = (size_t)P.rps * P.row_bytes;
  const uint32_t lds0 = gv_lds_addr(st);
  auto issue = [&](int s) {  // stage s of the matrix into ring slot (s - s0) % GV_NS
    const uint8_t *base = P.w + (size_t)s * stage_bytes;
    const size_t left = P.total - (size_t)s * stage_bytes;  // bytes from this stage's start to the end
    const uint32_t slot = lds0 + ((s - s0) % GV_NS) * GV_STAGE;
#pragma unroll
    for (int i = 0; i < PER; i++) {
      const int n = wave + 4 * i;
      // Bytes past the matrix end read its last chunk again (never used as a real row).
      const uint32_t off = (uint32_t)min((size_t)(n * 64 + lane) * LANE, left - LANE);
      if constexpr (D16) gv_dma16(base, off, slot + n * 64 * LANE);
      else gv_dma4(base, off, slot + n * 64 * LANE);
    }
  };
#pragma unroll
  for (int i = 0; i < GV_NS - 1; i++)
    if (s0 + i < s1) issue(s0 + i);
  // `a` (and the norm's g, b) into LDS.  Every load is issued before any is used, wavefront 0's loads
  // for the norm's statistics with the rest and all from clamped addresses (a load behind a branch
  // waits there), so the prologue costs one round trip, with the first stages' DMA.
  // The epilogue's bias and output (residual modes) of this thread's first row and the cache column,
  // loaded with the prologue's loads (pinned below, where the prologue waits anyway) instead of after
  // the streaming loop.
  const int r0 = s0 * P.rps, r1 = min(s1 * P.rps, P.rows);
  const bool res = P.epi == WH_RESIDUAL || P.epi == WH_GELU_RESIDUAL;
  const int er = min(r0 + tid, P.rows - 1);
  const float eb = P.bias[er], ec = res ? P.c[P.offset + er] : 0.0f;
  const int pcol = P.pack.dcol ? *P.pack.dcol : P.pack.col;  // the cache column (the step's position)
  const int q4 = P.k / 4;
  constexpr int AV = 8;  // float4 of `a` per thread on the vector path: k ≤ 8192
  const bool vec = ((uintptr_t)P.a % 16 == 0) && q4 <= AV * 256;
  const float4 *a4 = (const float4 *)P.a;
  float4 av[AV], gv[AV], bv[AV];
  if (vec) {
#pragma unroll
    for (int t = 0; t < AV; t++)
      if (256 * t < q4) {  // uniform: only the rounds that hold part of the row
        const int i = min(tid + 256 * t, q4 - 1);
        av[t] = a4[i];
        if (P.ln_g) gv[t] = ((const float4 *)P.ln_g)[i], bv[t] = ((const float4 *)P.ln_b)[i];
      }
  }
  __shared__ float stat[2];
  if (P.ln_g && wave == 0) {
    // The norm before this product, with layer_norm_kernel's arithmetic (one wave sums in the same
    // order, zeros past the row), so the normalized row equals the standalone kernel's bit for bit.
    float sm = 0.0f, q = 0.0f, mean;
    if (q4 <= 16 * 64) {
      float4 v[16];
#pragma unroll
      for (int t = 0; t < 16; t++) {
        v[t] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        if (64 * t < q4) {  // uniform
          const float4 x = a4[min(lane + 64 * t, q4 - 1)];
          if (lane + 64 * t < q4) v[t] = x;
        }
      }
#pragma unroll
      for (int t = 0; t < 16; t++) sm += (v[t].x + v[t].y) + (v[t].z + v[t].w);
      mean = gv_wave_sum(sm) / (float)P.k;
#pragma unroll
      for (int t = 0; t < 16; t++)
        if (lane + 64 * t < q4) {
          const float dx = v[t].x - mean, dy = v[t].y - mean, dz = v[t].z - mean, dw = v[t].w - mean;
          q += (dx * dx + dy * dy) + (dz * dz + dw * dw);
        }
    } else {
      for (int i = lane; i < q4; i += 64) {
        const float4 v = a4[i];
        sm += (v.x + v.y) + (v.z + v.w);
      }
      mean = gv_wave_sum(sm) / (float)P.k;
      for (int i = lane; i < q4; i += 64) {
        const float4 v = a4[i];
        const float dx = v.x - mean, dy = v.y - mean, dz = v.z - mean, dw = v.w - mean;
        q += (dx * dx + dy * dy) + (dz * dz + dw * dw);
      }
    }
    const float rstd = rsqrtf(gv_wave_sum(q) / (float)P.k + 1e-5f);
    if (lane == 0) stat[0] = mean, stat[1] = rstd;
  }
  if (vec) {
    if (P.ln_g) {
      __syncthreads();  // the norm's statistics
      const float mean = stat[0], rstd = stat[1];
#pragma unroll
      for (int t = 0; t < AV; t++) {
        if (256 * t >= q4) break;
        av[t].x = (av[t].x - mean) * rstd * gv[t].x + bv[t].x;
        av[t].y = (av[t].y - mean) * rstd * gv[t].y + bv[t].y;
        av[t].z = (av[t].z - mean) * rstd * gv[t].z + bv[t].z;
        av[t].w = (av[t].w - mean) * rstd * gv[t].w + bv[t].w;
      }
    }
#pragma unroll
    for (int t = 0; t < AV; t++) {
      if (256 * t >= q4) break;
      // float4 i: elements 4i .. 4i + 3 of item 4i / 64 (threads past the row store the last one again)
      const int i = min(tid + 256 * t, q4 - 1);
      *(float4 *)(as + (i >> 4) * AS + 4 * (i & 15)) = av[t];
    }
  } else {
    if (P.ln_g) __syncthreads();
    const float mean = P.ln_g ? stat[0] : 0.0f, rstd = P.ln_g ? stat[1] : 1.0f;
    for (int i = tid; i < P.k; i += 256)
      as[(i >> 6) * AS + (i & 63)] = P.ln_g ? (P.a[i] - mean) * rstd * P.ln_g[i] + P.ln_b[i] : P.a[i];
  }
  asm volatile("" : : "v"(eb), "v"(ec), "v"(pcol));
  const int row_l = tid / items, it = tid % items;
  for (int s = s0; s < s1; s++) {
    if (s + GV_NS - 2 < s1) gv_wait_vm<(GV_NS - 2) * PER>();
    else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();  // stage s landed everywhere; the slot of stage s − 1 and `part` are free
    if (s + GV_NS - 1 < s1) issue(s + GV_NS - 1);
    const int nrows = min(P.rps, P.rows - s * P.rps);
    float sum = 0.0f;
    if (row_l < nrows) {
      const uint8_t *ip = st + ((s - s0) % GV_NS) * GV_STAGE + row_l * P.row_bytes + it * ITEM;
      const float *x = as + AS * it;
      if constexpr (WT == WH_F16) {
#pragma unroll
        for (int q = 0; q < 8; q++) {
          const uint4 v = *(const uint4 *)(ip + 16 * q);
          const uint32_t u[4] = {v.x, v.y, v.z, v.w};
          const float4 x0 = *(const float4 *)(x + 8 * q), x1 = *(const float4 *)(x + 8 * q + 4);
          const float xs[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
          for (int e = 0; e < 4; e++) sum += half_bits(u[e] & 0xffffu) * xs[2 * e] + half_bits(u[e] >> 16) * xs[2 * e + 1];
        }
      } else {
        constexpr int DW = ITEM / 4;  // 17 or 9 dwords
        const uint32_t *p = (const uint32_t *)ip;
        uint32_t q[DW + 1];
#pragma unroll
        for (int i = 0; i < DW; i++) q[i] = p[i];
        q[DW] = 0;
        constexpr int S1 = ITEM / 8;  // block 1's scale sits in the high half of dword S1
#pragma unroll
        for (int b = 0; b < 2; b++) {
          const float d = half_bits(b ? (q[S1] >> 16) : (q[0] & 0xffffu));
          const float *xb = x + 32 * b;
          float bs = 0.0f;
          if constexpr (WT == WH_Q8_0) {
#pragma unroll
            for (int j = 0; j < 8; j++) {
              const uint32_t v = b ? q[S1 + 1 + j] : __builtin_amdgcn_alignbyte(q[j + 1], q[j], 2);
              const float4 xv = *(const float4 *)(xb + 4 * j);
              bs += (float)(int8_t)(v) * xv.x + (float)(int8_t)(v >> 8) * xv.y + (float)(int8_t)(v >> 16) * xv.z +
                    (float)(int8_t)(v >> 24) * xv.w;
            }
          } else {
#pragma unroll
            for (int j = 0; j < 4; j++) {
              const uint32_t v = b ? q[S1 + 1 + j] : __builtin_amdgcn_alignbyte(q[j + 1], q[j], 2);
              const float4 xl = *(const float4 *)(xb + 4 * j), xh = *(const float4 *)(xb + 16 + 4 * j);
              bs += (float)((int)(v & 15u) - 8) * xl.x + (float)((int)((v >> 8) & 15u) - 8) * xl.y +
                    (float)((int)((v >> 16) & 15u) - 8) * xl.z + (float)((int)((v >> 24) & 15u) - 8) * xl.w;
              bs += (float)((int)((v >> 4) & 15u) - 8) * xh.x + (float)((int)((v >> 12) & 15u) - 8) * xh.y +
                    (float)((int)((v >> 20) & 15u) - 8) * xh.z + (float)((int)((v >> 28) & 15u) - 8) * xh.w;
            }
          }
          sum += bs * d;
        }
      }
    }
    part[(s - s0) * 256 + tid] = sum;  // the thread's own slot: no barrier until after the loop
  }
  // The rows' items in order, 4 at a time (items % 4 == 0 when k % 256 == 0; else a tail), for
  // every stage of the workgroup at once, off the streaming loop; then the epilogue.
  __syncthreads();
  const int nsr = (s1 - s0) * P.rps;  // the workgroup's stage rows (the last stage's may pass `rows`)
  for (int j = tid; j < nsr; j += 256) {
    const int st = j / P.rps, rl = j - st * P.rps;
    const float *pr = part + st * 256 + rl * items;
    float acc = 0.0f;
    int i = 0;
    if ((items & 3) == 0) {
#pragma unroll 4
      for (; i < items; i += 4) {
        const float4 v = *(const float4 *)(pr + i);
        acc += ((v.x + v.y) + (v.z + v.w));
      }
    }
    for (; i < items; i++) acc += pr[i];
    rsum[j] = acc;
  }
  __syncthreads();
  for (int row = r0 + tid; row < r1; row += 256) {
    float *cp = P.c + P.offset + row;
    const bool first = row == r0 + tid;
    const float v = epilogue(P.epi, P.alpha, rsum[row - r0] + (first ? eb : P.bias[row]), res ? (first ? ec : *cp) : 0.0f);
    *cp = v;
    const int x = row - P.pack.lo;  // the cache's K then V values: pair x / 2, half x % 2 of launch_pack
    if (P.pack.cache && x >= 0 && x < 2 * P.pack.d && pcol < P.pack.cols) {
      const int pi = x >> 1, half = P.pack.d / 2;
      const size_t word = pi < half ? (size_t)pi * P.pack.cols + pcol
                                    : (size_t)half * P.pack.cols + (size_t)pcol * half + pi - half;
      ((uint16_t *)P.pack.cache)[2 * word + (x & 1)] = __builtin_bit_cast(uint16_t, (_Float16)v);
    }
  }
  // Rows rows..cols (the padding rows of the linear): epi(0 + bias), by the first workgroup.
  if (blockIdx.x == 0)
    for (int row = P.rows + tid; row < P.cols; row += 256) {
      float *cp = P.c + P.offset + row;
      *cp = epilogue(P.epi, P.alpha, P.bias[row], res ? *cp : 0.0f);
    }
}

template <int WT>
int gemv_stream(wh_ctx *ctx, const float *a, const wh_linear *l, float *c, int epi, float alpha, int offset,
                const float *ln_g, const float *ln_b, const GemvPack *pack) {
  const int items = l->k / 64;
  GemvArgs P{a, l->w, l->bias, c, l->rows, l->cols, l->k, epi, offset, ln_g, ln_b,
             pack ? *pack : GemvPack{}, alpha, (int)l->row_bytes, 0, 0, 0, 0};
  P.rps = std::min(256 / items, GV_STAGE / (int)l->row_bytes);
  P.stages = (l->rows + P.rps - 1) / P.rps;
  // Two workgroups per CU (48 KiB of stages each), each streaming a run of stages: measured on
  // MI355X, 16 KiB stages three deep at two per CU stream the 70.5 MB head at 4.6 TB/s, against
  // 3.2 TB/s for 20 KiB stages four deep at one per CU.
  const int cus = ctx->cus > 0 ? ctx->cus : 256;
  const int wgs = std::min(P.stages, 2 * cus);
  P.per_wg = (P.stages + wgs - 1) / wgs;
  const int grid = (P.stages + P.per_wg - 1) / P.per_wg;
  P.total = (size_t)l->rows * l->row_bytes;
  const size_t lds = (size_t)GV_NS * GV_STAGE + 4 * (size_t)items * 68 + 4 * (256 + (size_t)P.rps) * P.per_wg;
  if (lds > 160 * 1024) return 1;  // (positive: not an error) the caller takes the general kernel
  // Named by type and shape (rows x k): the profile tells the decoder's GEMVs apart.
  char tn[64];
  snprintf(tn, sizeof tn, "gemv_%s %dx%d", WT == WH_F16 ? "f16" : WT == WH_Q8_0 ? "q8_0" : "q4_0", l->rows, l->k);
  const double bytes = (double)P.total + 4.0 * l->k + 4.0 * l->cols * (epi == WH_RESIDUAL || epi == WH_GELU_RESIDUAL ? 2 : 1);
  ProfScope prof(ctx, tn, 2.0 * l->rows * l->k, bytes);
  if (l->row_bytes % 16 == 0)
    wh_launch(ctx, gemv_stream_kernel<WT, true>, grid, 256, lds, P);
  else
    wh_launch(ctx, gemv_stream_kernel<WT, false>, grid, 256, lds, P);
  return wh_launched(ctx, "gemv");
}

template <int WT, bool PAIR>
int gemv_t(wh_ctx *ctx, const float *a, const wh_linear *l, float *c, int epi, float alpha, int offset) {
  int waves = (l->cols + 1) / 2;
  int grid = (waves + 3) / 4;
  size_t lds = sizeof(float) * (size_t)l->k;
  char tn[64];
  snprintf(tn, sizeof tn, "gemv_%s %dx%d", WT == WH_F32 ? "f32" : WT == WH_F16 ? "f16" : WT == WH_Q8_0 ? "q8_0" : "q4_0",
           l->rows, l->k);
  // Algorithmic bytes: W as stored + a + c (+ c read by the residual epilogues).
  double bytes = (double)l->rows * l->row_bytes + 4.0 * l->k + 4.0 * l->cols * (epi == WH_RESIDUAL || epi == WH_GELU_RESIDUAL ? 2 : 1);
  ProfScope prof(ctx, tn, 2.0 * l->rows * l->k, bytes);
  wh_launch(ctx, gemv_wave_kernel<WT, PAIR>, grid, 256, lds, a, l->w, l->bias, c, l->rows, l->cols, l->k,
                                                              l->row_bytes, epi, alpha, offset);
  return wh_launched(ctx, "gemv");
}

// c[i] = W[ids[idx]][i] + pos[offset + i] + bias[i] (gemm.wgsl:309-327).
__global__ void embed_kernel(const uint8_t *__restrict__ w, int type, size_t row_bytes, const float *__restrict__ pos,
                             const float *__restrict__ bias, float *__restrict__ c, const uint32_t *__restrict__ ids,
                             int idx, int k, int offset, const int *__restrict__ dpos, int dstride) {
  int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= k) return;
  if (dpos) offset = *dpos * dstride;
  const uint8_t *wr = w + (size_t)ids[idx] * row_bytes;
  float v;
  switch (type) {
    case WH_F32: v = ((const float *)wr)[i]; break;
    case WH_F16: v = half_bits(((const uint16_t *)wr)[i]); break;
    case WH_Q8_0: {
      const uint8_t *blk = wr + (size_t)(i / 32) * 34;
      v = (float)(int8_t)blk[2 + i % 32] * half_bits((uint32_t)blk[0] | ((uint32_t)blk[1] << 8));
      break;
    }
    default: {
      const uint8_t *blk = wr + (size_t)(i / 32) * 18;
      int e = i % 32;
      uint32_t by = blk[2 + (e & 15)];
      int q = (int)(e < 16 ? (by & 15u) : (by >> 4)) - 8;
      v = (float)q * half_bits((uint32_t)blk[0] | ((uint32_t)blk[1] << 8));
    }
  }
  c[i] = v + pos[offset + i] + bias[i];
}

// RNE to f16 keeping subnormals; values past the f16 range keep their exponent only in the
// reference's WGSL, here they become ±inf (the cache is f16 storage).
__device__ __forceinline__ uint32_t h16(float x) { return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)x); }

constexpr int KEYS = 256;  // keys per workgroup, one per thread (the parts of attend_len)

// Part (c, h): head h's query against keys c·KEYS .. (c+1)·KEYS − 1 (decode.wgsl:56-119).
//
// Every load is issued at the start: thread t's key K (all its pairs: K is transposed per head, so a
// wave's 64 keys read 256 contiguous bytes per pair) and, for p·V, the value pair t % pairs of every
// (KEYS / pairs)-th key from t / pairs on (a key's pairs are contiguous); then q.  Scores, the
// softmax over the part and p·V follow from registers and LDS.  A head of one part writes its output;
// otherwise each part writes (Σ e·v, max, Σ e) for the merge (decode.wgsl:121-147): by combine_kernel
// when the key count is known at launch (a second launch costs less than the fences below), or with
// MERGE by whichever of the head's parts finishes last, for a count in device memory (a recorded
// decoder step, mostly one part: no second launch and no fence then).  There wave 0, which wrote the
// part, makes it visible device-wide (release fence: the XCDs' L2s are written back) and counts it
// done on the head's counter; the part that completes the count (acquire fence) merges and puts the
// counter back to 0 for the next launch.  No workgroup waits on another.
template <int P, bool MERGE>  // P: pairs per head, at most
__global__ __launch_bounds__(KEYS) void attend_kernel(const float *__restrict__ q, const uint32_t *__restrict__ kv,
                                                      float *__restrict__ part, float *__restrict__ o,
                                                      int *__restrict__ count, int n, int hd, float scale, int cols,
                                                      int heads, const int *__restrict__ dn) {
  if (dn) n = min(*dn + n, cols);
  const int j0 = blockIdx.x * KEYS;
  if (j0 >= n) return;  // a grid sized for the most keys: parts past n are unused
  __shared__ float qs[2 * P];
  __shared__ float p[KEYS];
  __shared__ float red[8];
  __shared__ float2 rv[KEYS];
  __shared__ int last;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int pairs = hd / 2, h = blockIdx.y, parts = (n + KEYS - 1) / KEYS;
  const int cnt = min(n - j0, KEYS);
  const size_t v_stride = (size_t)heads * pairs;
  // K of key j0 + tid (clamped into the part; its score is dropped below).
  const uint32_t *kp = kv + (size_t)h * pairs * cols + j0 + min(tid, cnt - 1);
  uint32_t ku[P];
#pragma unroll
  for (int i = 0; i < P; i++) ku[i] = kp[(size_t)min(i, pairs - 1) * cols];
  // V: pair c of keys g, g + groups, … of the part (key j is (j % groups, j / groups): j / groups < P
  // since groups ≥ KEYS / P; clamped into the part, weighted 0 past cnt).
  const int groups = KEYS / pairs, c = tid % pairs, g = tid / pairs;
  const uint32_t *vp = kv + v_stride * cols + (size_t)h * pairs + c;
  uint32_t vu[P];
#pragma unroll
  for (int t = 0; t < P; t++) vu[t] = vp[(size_t)(j0 + min(g + groups * t, cnt - 1)) * v_stride];
  for (int i = tid; i < hd; i += KEYS) qs[i] = (float)(_Float16)q[h * hd + i];
  __syncthreads();
  float acc = 0.0f;
#pragma unroll
  for (int i = 0; i < P; i++)
    if (i < pairs) acc += qs[2 * i] * half_bits(ku[i] & 0xffffu) + qs[2 * i + 1] * half_bits(ku[i] >> 16);
  const float x = tid < cnt ? acc * scale : -INFINITY;
  float m = x;
  m = xlane::wave_max(m);
  if (lane == 0) red[wave] = m;
  __syncthreads();
  m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  const float e = tid < cnt ? __expf(x - m) : 0.0f;
  p[tid] = e;
  float l = e;
  l = xlane::wave_sum(l);
  if (lane == 0) red[4 + wave] = l;
  __syncthreads();
  l = red[4] + red[5] + red[6] + red[7];
  float2 ov = make_float2(0.0f, 0.0f);
  if (g < groups)
#pragma unroll
    for (int t = 0; t < P; t++) {
      const int j = g + groups * t;
      if (j < cnt) {
        ov.x += p[j] * half_bits(vu[t] & 0xffffu);
        ov.y += p[j] * half_bits(vu[t] >> 16);
      }
    }
  rv[tid] = ov;
  __syncthreads();
  float2 sum = make_float2(0.0f, 0.0f);
  if (tid < pairs)
    for (int k = 0; k < groups; k++) sum.x += rv[k * pairs + tid].x, sum.y += rv[k * pairs + tid].y;
  if (parts == 1) {
    if (tid < pairs) {
      const float inv = 1.0f / l;
      o[h * hd + 2 * tid] = sum.x * inv;
      o[h * hd + 2 * tid + 1] = sum.y * inv;
    }
    return;
  }
  float *pp = part + ((size_t)h * parts + blockIdx.x) * (hd + 2);
  if (tid < pairs) pp[2 * tid] = sum.x, pp[2 * tid + 1] = sum.y;  // wave 0 (pairs ≤ 64)
  if (tid == 0) pp[hd] = m, pp[hd + 1] = l;
  if (!MERGE) return;
  if (wave == 0) {
    __threadfence();
    if (tid == 0) last = atomicAdd(&count[h], 1) == parts - 1;
  }
  __syncthreads();
  if (!last) return;
  __threadfence();
  // The merge: every part rescaled to the common maximum.
  const float *base = part + (size_t)h * parts * (hd + 2);
  float mx = -INFINITY;
  for (int k = 0; k < parts; k++) mx = fmaxf(mx, base[k * (hd + 2) + hd]);
  float lt = 0.0f;
  for (int k = 0; k < parts; k++) lt += __expf(base[k * (hd + 2) + hd] - mx) * base[k * (hd + 2) + hd + 1];
  if (tid < hd) {
    float r = 0.0f;
    for (int k = 0; k < parts; k++) r += __expf(base[k * (hd + 2) + hd] - mx) * base[k * (hd + 2) + tid];
    o[h * hd + tid] = r / lt;
  }
  if (tid == 0) count[h] = 0;
}

// Per head, the parts of attend_kernel rescaled to their common maximum, summed and normalized
// (decode.wgsl:121-147).  Up to CP parts (the 1500-frame cross attention has 6) and 128 dimensions,
// every part's values are loaded first (clamped: one round trip, not one per part and pass), then
// combined in the order of the general loop below, so both give the same bits.
constexpr int CP = 8;
__global__ void combine_kernel(const float *__restrict__ part, float *__restrict__ o, int n, int hd) {
  const int parts = (n + KEYS - 1) / KEYS;
  const float *base = part + (size_t)blockIdx.x * parts * (hd + 2);
  if (parts <= CP && hd <= 2 * 64 && blockDim.x == 64) {
    const int tid = threadIdx.x;
    float pm[CP], pl[CP], pv[CP][2];
#pragma unroll
    for (int c = 0; c < CP; c++) {
      const float *bc = base + min(c, parts - 1) * (hd + 2);
      pm[c] = bc[hd], pl[c] = bc[hd + 1];
#pragma unroll
      for (int j = 0; j < 2; j++) pv[c][j] = bc[min(tid + 64 * j, hd - 1)];
    }
    float m = -INFINITY;
#pragma unroll
    for (int c = 0; c < CP; c++)
      if (c < parts) m = fmaxf(m, pm[c]);
    float l = 0.0f;
#pragma unroll
    for (int c = 0; c < CP; c++)
      if (c < parts) l += __expf(pm[c] - m) * pl[c];
#pragma unroll
    for (int j = 0; j < 2; j++) {
      const int i = tid + 64 * j;
      float acc = 0.0f;
#pragma unroll
      for (int c = 0; c < CP; c++)
        if (c < parts) acc += __expf(pm[c] - m) * pv[c][j];
      if (i < hd) o[blockIdx.x * hd + i] = acc / l;
    }
    return;
  }
  float m = -INFINITY;
  for (int c = 0; c < parts; c++) m = fmaxf(m, base[c * (hd + 2) + hd]);
  float l = 0.0f;
  for (int c = 0; c < parts; c++) l += __expf(base[c * (hd + 2) + hd] - m) * base[c * (hd + 2) + hd + 1];
  for (int i = threadIdx.x; i < hd; i += blockDim.x) {
    float acc = 0.0f;
    for (int c = 0; c < parts; c++) acc += __expf(base[c * (hd + 2) + hd] - m) * base[c * (hd + 2) + i];
    o[blockIdx.x * hd + i] = acc / l;
  }
}

// Rows of x (K then V, d floats each) into the f16 cache at positions col.. (decode.wgsl:148-173).
__global__ void pack_kernel(const float *__restrict__ x, uint32_t *__restrict__ y, int n, int d, int cols, int col,
                            int src, int stride, const int *__restrict__ dcol) {
  if (dcol) col = *dcol;
  int i, j;
  if (n > 1) {
    i = blockIdx.y * 4 + threadIdx.x / 64;
    j = blockIdx.x * 64 + threadIdx.x % 64;
  } else {
    i = blockIdx.x * 256 + threadIdx.x;
    j = 0;
  }
  const int half = d / 2;
  if (i >= d || j >= n || col + j >= cols) return;
  const float *p = x + src + (size_t)j * stride + 2 * i;
  size_t at = i < half ? (size_t)i * cols + col + j : (size_t)half * cols + (size_t)(col + j) * half + i - half;
  y[at] = h16(p[0]) | (h16(p[1]) << 16);
}

}  // namespace

int launch_gemv(wh_ctx *ctx, const float *a, const wh_linear *l, float *c, int epi, float alpha, int offset,
                const float *ln_g, const float *ln_b, float *ln_y, const GemvPack *pack) {
  if (pack && (!pack->cache || pack->d <= 0 || pack->d % 2 || pack->lo < 0 || pack->lo + 2 * pack->d > l->rows ||
               pack->cols <= 0 || pack->col < 0 || pack->col >= pack->cols))
    return wh_fail(ctx, WH_EARG, "gemv: bad cache column");
  if (!a || !c || offset < 0 || epi < WH_BIAS || epi > WH_TANH) return wh_fail(ctx, WH_EARG, "gemv: bad arguments");
  if ((size_t)l->k * 4 > 64 * 1024) return wh_fail(ctx, WH_EARG, "gemv: k %d too large", l->k);
  if (ln_g && (!ln_b || !ln_y || l->k % 4 || (uintptr_t)a % 16 || (uintptr_t)ln_g % 16 || (uintptr_t)ln_b % 16))
    return wh_fail(ctx, WH_EARG, "gemv: the fused norm needs g, b, a row buffer, k %% 4 == 0 and an aligned a");
  bool pair = l->k % 64 == 0;
  // The streaming kernel: whole 64-weight items, at most 256 of them per row, rows 4-byte aligned.
  if (pair && l->k / 64 <= 256 && l->row_bytes % 4 == 0 && (int)l->row_bytes <= GV_STAGE && l->rows > 0) {
    int rc = 1;
    switch (l->type) {
      case WH_Q8_0: rc = gemv_stream<WH_Q8_0>(ctx, a, l, c, epi, alpha, offset, ln_g, ln_b, pack); break;
      case WH_Q4_0: rc = gemv_stream<WH_Q4_0>(ctx, a, l, c, epi, alpha, offset, ln_g, ln_b, pack); break;
      case WH_F16: rc = gemv_stream<WH_F16>(ctx, a, l, c, epi, alpha, offset, ln_g, ln_b, pack); break;
    }
    if (rc != 1) return rc;
  }
  if (pack) {  // the general kernel, then the cache column by its own launch
    if (int rc = launch_gemv(ctx, a, l, c, epi, alpha, offset, ln_g, ln_b, ln_y, nullptr)) return rc;
    return launch_pack(ctx, c + offset, pack->lo, 0, pack->cache, 1, pack->d, pack->cols, pack->col, pack->dcol);
  }
  if (ln_g) {  // the general kernel takes the norm from its own launch
    if (int rc = launch_layer_norm(ctx, a, ln_g, ln_b, ln_y, 1, l->k, nullptr, nullptr, 0)) return rc;
    a = ln_y;
  }
  switch (l->type) {
    case WH_F32: return gemv_t<WH_F32, false>(ctx, a, l, c, epi, alpha, offset);
    case WH_F16: return gemv_t<WH_F16, false>(ctx, a, l, c, epi, alpha, offset);
    case WH_Q8_0: return pair ? gemv_t<WH_Q8_0, true>(ctx, a, l, c, epi, alpha, offset)
                              : gemv_t<WH_Q8_0, false>(ctx, a, l, c, epi, alpha, offset);
    case WH_Q4_0: return pair ? gemv_t<WH_Q4_0, true>(ctx, a, l, c, epi, alpha, offset)
                              : gemv_t<WH_Q4_0, false>(ctx, a, l, c, epi, alpha, offset);
  }
  return wh_fail(ctx, WH_EARG, "gemv: weight type %d", l->type);
}

// A decoder step's token and position into device memory (ids[0], ids[1]), where a recorded step
// reads them: a kernel argument, so the host neither copies nor waits.
__global__ void step_args_kernel(uint32_t *ids, uint32_t token, uint32_t pos) {
  if (threadIdx.x == 0) {
    ids[0] = token;
    ids[1] = pos;
  }
}

int launch_step_args(wh_ctx *ctx, uint32_t *ids, int token, int pos) {
  if (!ids || token < 0 || pos < 0) return wh_fail(ctx, WH_EARG, "step arguments: bad arguments");
  wh_launch(ctx, step_args_kernel, 1, 64, 0, ids, (uint32_t)token, (uint32_t)pos);
  return wh_launched(ctx, "step_args");
}

int launch_embed(wh_ctx *ctx, const wh_linear *l, const float *pos, float *c, const uint32_t *ids, int i,
                 int offset, const int *dpos, int dstride) {
  if (!pos || !c || !ids || i < 0 || offset < 0) return wh_fail(ctx, WH_EARG, "embed: bad arguments");
  ProfScope prof(ctx, "embed", 0.0, 12.0 * l->k);
  wh_launch(ctx, embed_kernel, (l->k + 255) / 256, 256, 0, l->w, l->type, l->row_bytes, pos, l->bias, c, ids, i,
                                                            l->k, offset, dpos, dstride);
  return wh_launched(ctx, "embed");
}

int launch_attend(wh_ctx *ctx, const float *q, const uint32_t *kv, float *part, float *o, int n, int cols,
                  int heads, int hd, const int *dn) {
  if (n <= 0 || n > cols || heads <= 0 || heads > ATTEND_HEADS || hd <= 0 || hd > 128 || hd % 2 || !q || !kv || !part ||
      !o)
    return wh_fail(ctx, WH_EARG, "attend: bad arguments (n %d, cols %d, heads %d, hd %d)", n, cols, heads, hd);
  if (!ctx->attend_count) return wh_fail(ctx, WH_EGPU, "attend: the context has no part counters");
  const float scale = 1.0f / sqrtf((float)hd);
  // A key count in device memory: the grid covers the whole cache and parts past it return.
  const int most = dn ? cols : n;
  const dim3 grid((most + KEYS - 1) / KEYS, heads);
  int *count = ctx->attend_count;
  ProfScope prof(ctx, dn ? "attend_self" : "attend", 4.0 * most * heads * hd, 2.0 * most * heads * hd * 2 + 4.0 * heads * hd);
  if (dn || most <= KEYS || ctx->attend_merge) {  // one launch: one part, or the merge by the last part
    if (hd <= 64)
      wh_launch(ctx, (attend_kernel<32, true>), grid, KEYS, 0, q, kv, part, o, count, n, hd, scale, cols, heads, dn);
    else
      wh_launch(ctx, (attend_kernel<64, true>), grid, KEYS, 0, q, kv, part, o, count, n, hd, scale, cols, heads, dn);
    return wh_launched(ctx, "attend");
  }
  if (hd <= 64)
    wh_launch(ctx, (attend_kernel<32, false>), grid, KEYS, 0, q, kv, part, o, count, n, hd, scale, cols, heads, dn);
  else
    wh_launch(ctx, (attend_kernel<64, false>), grid, KEYS, 0, q, kv, part, o, count, n, hd, scale, cols, heads, dn);
  if (int rc = wh_launched(ctx, "attend")) return rc;
  ProfScope pc(ctx, "attend_combine", 0.0, 4.0 * grid.x * heads * (hd + 2.0) + 4.0 * heads * hd);
  wh_launch(ctx, combine_kernel, heads, 64, 0, part, o, n, hd);
  return wh_launched(ctx, "combine");
}

int launch_pack(wh_ctx *ctx, const float *x, int src, int stride, uint32_t *y, int rows, int d, int cols, int col,
                const int *dcol) {
  if (rows <= 0 || d <= 0 || d % 2 || cols <= 0 || col < 0 || col + rows > cols || src < 0 || !x || !y)
    return wh_fail(ctx, WH_EARG, "pack: bad arguments");
  ProfScope prof(ctx, "pack", 0.0, 4.0 * rows * 2 * d + 2.0 * rows * 2 * d);
  if (rows == 1) {
    wh_launch(ctx, pack_kernel, (d + 255) / 256, 256, 0, x, y, rows, d, cols, col, src, stride, dcol);
  } else {
    dim3 grid((rows + 63) / 64, (d + 3) / 4);
    wh_launch(ctx, pack_kernel, grid, 256, 0, x, y, rows, d, cols, col, src, stride, dcol);
  }
  return wh_launched(ctx, "pack");
}
