// Decoder kernels for one token: the HBM-bound GEMV over GGUF weight bytes (Pass::gemv,
// src/gpu/mod.rs:1461-1467; gemm.wgsl:244-307), the embedding row (Pass::embed, :1469-1482;
// gemm.wgsl:309-327), attention of one query per head over an f16 K/V cache split into parts of
// 256 keys and their merge (Pass::attend, :1484-1505; decode.wgsl:56-147), and packing f32 rows
// into that cache (Pass::pack, :1507-1523; decode.wgsl:148-173).
//
// The GEMV streams W once: a workgroup takes a run of whole rows, contiguous in HBM, and each thread
// one 16-byte (F16/F32) or block-pair (Q8_0/Q4_0) item of a row per step, so the workgroup's loads
// sweep the run's bytes in order; `a` sits in LDS.  Per block the int8 (or nibble) products are
// summed in f32 and scaled once, as ggml's mul_mv (gemm.wgsl:244-262); W is not rounded to f16.
#include "internal.h"

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
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o, 64);
    if (lane == 0) {
      float *cp = c + offset + row;
      *cp = epilogue(epi, alpha, s + bias[row], *cp);
    }
  }
}

template <int WT, bool PAIR>
int gemv_t(wh_ctx *ctx, const float *a, const wh_linear *l, float *c, int epi, float alpha, int offset) {
  int waves = (l->cols + 1) / 2;
  int grid = (waves + 3) / 4;
  size_t lds = sizeof(float) * (size_t)l->k;
  static const char *tn = WT == WH_F32 ? "gemv_f32" : WT == WH_F16 ? "gemv_f16" : WT == WH_Q8_0 ? "gemv_q8_0" : "gemv_q4_0";
  // Algorithmic bytes: W as stored + a + c (+ c read by the residual epilogues).
  double bytes = (double)l->rows * l->row_bytes + 4.0 * l->k + 4.0 * l->cols * (epi == WH_RESIDUAL || epi == WH_GELU_RESIDUAL ? 2 : 1);
  ProfScope prof(ctx, tn, 2.0 * l->rows * l->k, bytes);
  gemv_wave_kernel<WT, PAIR><<<grid, 256, lds, ctx->stream>>>(a, l->w, l->bias, c, l->rows, l->cols, l->k,
                                                              l->row_bytes, epi, alpha, offset);
  return wh_launched(ctx, "gemv");
}

// c[i] = W[ids[idx]][i] + pos[offset + i] + bias[i] (gemm.wgsl:309-327).
__global__ void embed_kernel(const uint8_t *__restrict__ w, int type, size_t row_bytes, const float *__restrict__ pos,
                             const float *__restrict__ bias, float *__restrict__ c, const uint32_t *__restrict__ ids,
                             int idx, int k, int offset) {
  int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= k) return;
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

constexpr int KEYS = 256;

// Part (c, h): head h's query against keys c·KEYS.. (decode.wgsl:56-119).
__global__ __launch_bounds__(256) void attend_kernel(const float *__restrict__ q, const uint32_t *__restrict__ kv,
                                                     float *__restrict__ part, int n, int hd, float scale,
                                                     int cols, int heads) {
  __shared__ float qs[128];
  __shared__ float s[KEYS];
  __shared__ float red[8];
  __shared__ float2 rv[256];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int pairs = hd / 2, h = blockIdx.y;
  const size_t k0 = (size_t)h * pairs * cols;
  const size_t v_stride = (size_t)heads * pairs;
  const size_t v0 = v_stride * cols + (size_t)h * pairs;
  for (int i = tid; i < hd; i += 256) qs[i] = (float)(_Float16)q[h * hd + i];
  __syncthreads();
  const int j0 = blockIdx.x * KEYS;
  const int cnt = min(n - j0, KEYS);
  float x = -INFINITY;
  if (tid < cnt) {
    float acc = 0.0f;
    for (int i = 0; i < pairs; i++) {
      uint32_t u = kv[k0 + (size_t)i * cols + j0 + tid];
      acc += qs[2 * i] * half_bits(u & 0xffffu) + qs[2 * i + 1] * half_bits(u >> 16);
    }
    x = acc * scale;
  }
  float m = x;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
  if (lane == 0) red[wave] = m;
  __syncthreads();
  m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  float e = tid < cnt ? __expf(x - m) : 0.0f;
  s[tid] = e;
  float l = e;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) l += __shfl_xor(l, o, 64);
  if (lane == 0) red[4 + wave] = l;
  __syncthreads();
  l = red[4] + red[5] + red[6] + red[7];
  const int groups = 256 / pairs;
  const int c = tid % pairs, g = tid / pairs;
  float2 o = make_float2(0.0f, 0.0f);
  if (g < groups)
    for (int j = g; j < cnt; j += groups) {
      uint32_t u = kv[v0 + (size_t)(j0 + j) * v_stride + c];
      o.x += s[j] * half_bits(u & 0xffffu);
      o.y += s[j] * half_bits(u >> 16);
    }
  rv[tid] = o;
  __syncthreads();
  const int nparts = (n + KEYS - 1) / KEYS;
  float *pp = part + ((size_t)h * nparts + blockIdx.x) * (hd + 2);
  if (tid < pairs) {
    float2 t = make_float2(0.0f, 0.0f);
    for (int k = 0; k < groups; k++) {
      t.x += rv[k * pairs + tid].x;
      t.y += rv[k * pairs + tid].y;
    }
    pp[2 * tid] = t.x;
    pp[2 * tid + 1] = t.y;
  }
  if (tid == 0) {
    pp[hd] = m;
    pp[hd + 1] = l;
  }
}

// Per head: the parts rescaled to their common maximum, summed and normalized (decode.wgsl:121-147).
__global__ void combine_kernel(const float *__restrict__ part, float *__restrict__ o, int n, int hd) {
  const int parts = (n + KEYS - 1) / KEYS;
  const float *base = part + (size_t)blockIdx.x * parts * (hd + 2);
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
                            int src, int stride) {
  int i, j;
  if (n > 1) {
    i = blockIdx.y * 4 + threadIdx.x / 64;
    j = blockIdx.x * 64 + threadIdx.x % 64;
  } else {
    i = blockIdx.x * 256 + threadIdx.x;
    j = 0;
  }
  const int half = d / 2;
  if (i >= d || j >= n) return;
  const float *p = x + src + (size_t)j * stride + 2 * i;
  size_t at = i < half ? (size_t)i * cols + col + j : (size_t)half * cols + (size_t)(col + j) * half + i - half;
  y[at] = h16(p[0]) | (h16(p[1]) << 16);
}

}  // namespace

int launch_gemv(wh_ctx *ctx, const float *a, const wh_linear *l, float *c, int epi, float alpha, int offset) {
  if (!a || !c || offset < 0 || epi < WH_BIAS || epi > WH_TANH) return wh_fail(ctx, WH_EARG, "gemv: bad arguments");
  if ((size_t)l->k * 4 > 64 * 1024) return wh_fail(ctx, WH_EARG, "gemv: k %d too large", l->k);
  bool pair = l->k % 64 == 0;
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

int launch_embed(wh_ctx *ctx, const wh_linear *l, const float *pos, float *c, const uint32_t *ids, int i,
                 int offset) {
  if (!pos || !c || !ids || i < 0 || offset < 0) return wh_fail(ctx, WH_EARG, "embed: bad arguments");
  ProfScope prof(ctx, "embed", 0.0, 12.0 * l->k);
  embed_kernel<<<(l->k + 255) / 256, 256, 0, ctx->stream>>>(l->w, l->type, l->row_bytes, pos, l->bias, c, ids, i,
                                                            l->k, offset);
  return wh_launched(ctx, "embed");
}

int launch_attend(wh_ctx *ctx, const float *q, const uint32_t *kv, float *part, float *o, int n, int cols,
                  int heads, int hd) {
  if (n <= 0 || n > cols || heads <= 0 || hd <= 0 || hd > 128 || hd % 2 || !q || !kv || !part || !o)
    return wh_fail(ctx, WH_EARG, "attend: bad arguments (n %d, cols %d, hd %d)", n, cols, hd);
  float scale = 1.0f / sqrtf((float)hd);
  dim3 grid((n + KEYS - 1) / KEYS, heads);
  ProfScope prof(ctx, "attend", 4.0 * n * heads * hd, 2.0 * n * heads * hd * 2 + 4.0 * heads * hd);
  attend_kernel<<<grid, 256, 0, ctx->stream>>>(q, kv, part, n, hd, scale, cols, heads);
  int rc = wh_launched(ctx, "attend");
  if (rc) return rc;
  combine_kernel<<<heads, 64, 0, ctx->stream>>>(part, o, n, hd);
  return wh_launched(ctx, "combine");
}

int launch_pack(wh_ctx *ctx, const float *x, int src, int stride, uint32_t *y, int rows, int d, int cols, int col) {
  if (rows <= 0 || d <= 0 || d % 2 || cols <= 0 || col < 0 || col + rows > cols || src < 0 || !x || !y)
    return wh_fail(ctx, WH_EARG, "pack: bad arguments");
  ProfScope prof(ctx, "pack", 0.0, 4.0 * rows * 2 * d + 2.0 * rows * 2 * d);
  if (rows == 1) {
    pack_kernel<<<(d + 255) / 256, 256, 0, ctx->stream>>>(x, y, rows, d, cols, col, src, stride);
  } else {
    dim3 grid((rows + 63) / 64, (d + 3) / 4);
    pack_kernel<<<grid, 256, 0, ctx->stream>>>(x, y, rows, d, cols, col, src, stride);
  }
  return wh_launched(ctx, "pack");
}
