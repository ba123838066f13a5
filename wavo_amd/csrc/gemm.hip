// The quantized GEMM of Pass::gemm (src/gpu/mod.rs:1394-1426) on gfx950 matrix cores:
//   c[m][j] = epi(Σ_k h(a[m][k]) · h(W[j][k]) + bias[j]),  h = round to f16 (RNE), f32 accumulate,
// as gemm.wgsl:170-242 and the CPU backend (src/cpu/gemm.rs:126-177) define it.  W stays in HBM as
// the GGUF stores it (src/gguf.rs:14-38): Q8_0 34-byte blocks (f16 scale + 32 int8), Q4_0 18-byte
// blocks (f16 scale + 16 bytes of nibbles), F16 or F32 rows.  Each workgroup stages a BM×64 tile of
// `a` (converted to f16) and a BN×64 tile of W (dequantized to f16(q·d), the reference's exact
// rounding) in LDS and runs v_mfma_f32_32x32x16_f16 over them; the epilogues of Epilogue::params
// (src/gpu/mod.rs:445-455; gemm.wgsl:72-94) and the dual outputs are fused into the store.
#include <cstdio>

#include "internal.h"

namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int BK = 64;       // k per stage: two quantized blocks
constexpr int LDS_ROW = 72;  // halves per LDS row (144 B: 16-byte aligned rows, banks staggered)

__device__ __forceinline__ float gelu(float x) {
  // Abramowitz–Stegun 7.1.26 erf, as gemm.wgsl:65-70 and src/cpu/ops.rs:33-40.
  float z = fabsf(0.70710678118654752440f * x);
  float t = 1.0f / (1.0f + 0.3275911f * z);
  float e = 1.0f - (((((1.061405429f * t - 1.453152027f) * t) + 1.421413741f) * t - 0.284496736f) * t +
                     0.254829592f) * t * __expf(-z * z);
  float s = x > 0.0f ? 1.0f : (x < 0.0f ? -1.0f : 0.0f);
  return 0.5f * x * (1.0f + s * e);
}

__device__ __forceinline__ float epilogue(int epi, float alpha, float v, const float *c) {
  switch (epi) {
    case WH_SILU: return v / (1.0f + __expf(-v));
    case WH_RELU: return fmaxf(v, 0.0f);
    case WH_RESIDUAL: return *c + alpha * v;
    case WH_GELU: return gelu(v);
    case WH_GELU_RESIDUAL: return *c + gelu(v);
    case WH_TANH: return tanhf(fminf(fmaxf(v, -10.0f), 10.0f));
    default: return v;
  }
}

__device__ __forceinline__ float half_bits(uint32_t h) { return (float)__builtin_bit_cast(_Float16, (uint16_t)h); }

// What one thread carries from HBM between two stages: its share of the `a` tile and of W.
template <int WT, int BM, int BN>
struct Stage {
  static constexpr int A4 = BM * BK / 4 / 256;  // float4 of `a` per thread
  float4 a[A4];
  // W: F32 BN*16 float4, F16 BN*8 uint4, quantized one (row, block) item of up to 9 dwords.
  static constexpr int W4 = WT == WH_F32 ? BN * 16 / 256 : (WT == WH_F16 ? BN * 8 / 256 : 0);
  uint4 w[W4 > 0 ? W4 : 1];
  uint32_t q[9];
};

template <int WT, int BM, int BN, bool ALIGNED>
__device__ __forceinline__ void load_stage(Stage<WT, BM, BN> &s, const float *__restrict__ a,
                                           const uint8_t *__restrict__ w, int m, int rows, int k,
                                           size_t row_bytes, int m0, int n0, int k0, int tid) {
#pragma unroll
  for (int p = 0; p < Stage<WT, BM, BN>::A4; p++) {
    int f = tid + 256 * p, r = f >> 4, q = f & 15;
    int row = m0 + r, col = k0 + 4 * q;
    s.a[p] = (row < m && col < k) ? *(const float4 *)(a + (size_t)row * k + col) : make_float4(0, 0, 0, 0);
  }
  if constexpr (WT == WH_F32 || WT == WH_F16) {
    constexpr int PER_ROW = WT == WH_F32 ? 16 : 8;
    constexpr int EL = WT == WH_F32 ? 4 : 8;  // elements per 16 bytes
#pragma unroll
    for (int p = 0; p < Stage<WT, BM, BN>::W4; p++) {
      int f = tid + 256 * p, r = f / PER_ROW, q = f % PER_ROW;
      int row = n0 + r, col = k0 + EL * q;
      s.w[p] = (row < rows && col < k) ? *(const uint4 *)(w + (size_t)row * row_bytes + (size_t)col * (16 / EL))
                                       : make_uint4(0, 0, 0, 0);
    }
  } else {
    // Item (row r, block b) of the stage: thread tid < 2·BN.
    constexpr int DW = WT == WH_Q8_0 ? 9 : 5;    // dwords per item on the aligned path
    constexpr int HW = WT == WH_Q8_0 ? 17 : 9;   // u16 per block on the unaligned path
    constexpr int BLK = WT == WH_Q8_0 ? 34 : 18; // bytes per block
    int r = tid >> 1, b = tid & 1;
    int row = n0 + r, blk = (k0 >> 5) + b;
    bool ok = tid < 2 * BN && row < rows && blk < (k >> 5);
    const uint8_t *base = w + (size_t)row * row_bytes;
    if (ALIGNED) {
      // Row starts and block pairs are 4-byte aligned (k % 64 == 0): the pair of blocks k0/64 is
      // 2·BLK bytes; item b reads dwords from (b ? BLK - 2 : 0) bytes in.
      const uint32_t *p = (const uint32_t *)(base + (size_t)(k0 >> 6) * 2 * BLK + (b ? (BLK - 2) : 0));
#pragma unroll
      for (int i = 0; i < DW; i++) s.q[i] = ok ? p[i] : 0u;
    } else {
      const uint16_t *p = (const uint16_t *)(base + (size_t)blk * BLK);
      uint16_t h[HW];
#pragma unroll
      for (int i = 0; i < HW; i++) h[i] = ok ? p[i] : (uint16_t)0;
      // As the aligned path's even items: dword j holds bytes 4j..4j+3 of the block.
#pragma unroll
      for (int j = 0; j < DW; j++) {
        uint32_t lo = 2 * j < HW ? h[2 * j] : 0u, hi = 2 * j + 1 < HW ? h[2 * j + 1] : 0u;
        s.q[j] = lo | (hi << 16);
      }
    }
  }
}

// Stage → LDS: `a` rounded to f16; W dequantized to f16(q·d).
template <int WT, int BM, int BN, bool ALIGNED>
__device__ __forceinline__ void store_stage(const Stage<WT, BM, BN> &s, _Float16 *As, _Float16 *Bs, int tid) {
#pragma unroll
  for (int p = 0; p < Stage<WT, BM, BN>::A4; p++) {
    int f = tid + 256 * p, r = f >> 4, q = f & 15;
    half4 h = {(_Float16)s.a[p].x, (_Float16)s.a[p].y, (_Float16)s.a[p].z, (_Float16)s.a[p].w};
    *(half4 *)(As + r * LDS_ROW + 4 * q) = h;
  }
  if constexpr (WT == WH_F32) {
#pragma unroll
    for (int p = 0; p < Stage<WT, BM, BN>::W4; p++) {
      int f = tid + 256 * p, r = f >> 4, q = f & 15;
      float4 v = __builtin_bit_cast(float4, s.w[p]);
      half4 h = {(_Float16)v.x, (_Float16)v.y, (_Float16)v.z, (_Float16)v.w};
      *(half4 *)(Bs + r * LDS_ROW + 4 * q) = h;
    }
  } else if constexpr (WT == WH_F16) {
#pragma unroll
    for (int p = 0; p < Stage<WT, BM, BN>::W4; p++) {
      int f = tid + 256 * p, r = f >> 3, q = f & 7;
      *(uint4 *)(Bs + r * LDS_ROW + 8 * q) = s.w[p];
    }
  } else {
    if (tid >= 2 * BN) return;
    int r = tid >> 1, b = tid & 1;
    // Even items (and the unaligned path) have the scale in the low half of q[0] and the data
    // from byte 2; odd aligned items have the scale in the high half and the data from q[1].
    bool odd = ALIGNED && b;
    uint32_t d16 = odd ? (s.q[0] >> 16) : (s.q[0] & 0xffffu);
    float d = half_bits(d16);
    constexpr int NDW = WT == WH_Q8_0 ? 8 : 4;  // data dwords of a block
    uint32_t dw[NDW];
#pragma unroll
    for (int i = 0; i < NDW; i++)
      dw[i] = odd ? s.q[i + 1] : __builtin_amdgcn_alignbyte(s.q[i + 1], s.q[i], 2);
    _Float16 *dst = Bs + r * LDS_ROW + 32 * b;
    if constexpr (WT == WH_Q8_0) {
#pragma unroll
      for (int g = 0; g < 4; g++) {
        half8 h;
#pragma unroll
        for (int e = 0; e < 8; e++) {
          int q = (int)(int8_t)(dw[2 * g + e / 4] >> (8 * (e & 3)));
          h[e] = (_Float16)((float)q * d);
        }
        *(half8 *)(dst + 8 * g) = h;
      }
    } else {
      // ggml block_q4_0: element i < 16 is the low nibble of byte i, 16 + i the high one.
#pragma unroll
      for (int g = 0; g < 4; g++) {
        half8 h;
#pragma unroll
        for (int e = 0; e < 8; e++) {
          int i = 8 * g + e;  // element
          int byte = i & 15;
          uint32_t v = (dw[byte >> 2] >> (8 * (byte & 3))) & 0xffu;
          int q = (int)(i < 16 ? (v & 15u) : (v >> 4)) - 8;
          h[e] = (_Float16)((float)q * d);
        }
        *(half8 *)(dst + 8 * g) = h;
      }
    }
  }
}

template <int WT, int BM, int BN, bool ALIGNED>
__global__ __launch_bounds__(256) void gemm_kernel(const float *__restrict__ a, const uint8_t *__restrict__ w,
                                                   const float *__restrict__ bias, float *__restrict__ c,
                                                   int m, int rows, int cols, int k, int dual, int ldc,
                                                   int epi, float alpha, size_t row_bytes) {
  __shared__ __attribute__((aligned(16))) _Float16 As[BM * LDS_ROW];
  __shared__ __attribute__((aligned(16))) _Float16 Bs[BN * LDS_ROW];
  constexpr int TM = BM / 64, TN = BN / 64;  // 32×32 MFMA tiles per wave (2×2 waves)
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int n0 = blockIdx.x * BN, m0 = blockIdx.y * BM;
  const int wm = (wave >> 1) * (BM / 2), wn = (wave & 1) * (BN / 2);
  floatx16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; i++)
#pragma unroll
    for (int j = 0; j < TN; j++) acc[i][j] = floatx16{};

  Stage<WT, BM, BN> st;
  load_stage<WT, BM, BN, ALIGNED>(st, a, w, m, rows, k, row_bytes, m0, n0, 0, tid);
  const int lrow = lane & 31, lk = 8 * (lane >> 5);
  for (int k0 = 0; k0 < k; k0 += BK) {
    store_stage<WT, BM, BN, ALIGNED>(st, As, Bs, tid);
    __syncthreads();
    if (k0 + BK < k) load_stage<WT, BM, BN, ALIGNED>(st, a, w, m, rows, k, row_bytes, m0, n0, k0 + BK, tid);
#pragma unroll
    for (int s = 0; s < BK / 16; s++) {
      half8 af[TM], bf[TN];
#pragma unroll
      for (int i = 0; i < TM; i++) af[i] = *(const half8 *)(As + (wm + 32 * i + lrow) * LDS_ROW + 16 * s + lk);
#pragma unroll
      for (int j = 0; j < TN; j++) bf[j] = *(const half8 *)(Bs + (wn + 32 * j + lrow) * LDS_ROW + 16 * s + lk);
#pragma unroll
      for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
    }
    __syncthreads();
  }
  // D[i][j] of a 32×32 tile sits in lane j (mod 32), register v: i = 8·(v/4) + 4·(lane/32) + v%4.
#pragma unroll
  for (int i = 0; i < TM; i++)
#pragma unroll
    for (int j = 0; j < TN; j++) {
      int col = n0 + wn + 32 * j + lrow;
      if (col >= cols) continue;
      float bv = bias[col];
      float b2 = col < dual ? bias[cols + col] : 0.0f;
#pragma unroll
      for (int v = 0; v < 16; v++) {
        int row = m0 + wm + 32 * i + 8 * (v >> 2) + 4 * (lane >> 5) + (v & 3);
        if (row >= m) continue;
        float *cp = c + (size_t)row * ldc + col;
        float x = acc[i][j][v];
        *cp = epilogue(epi, alpha, x + bv, cp);
        if (col < dual) cp[cols] = x + b2;
      }
    }
}

template <int WT, bool ALIGNED>
int launch_t(wh_ctx *ctx, const float *a, const wh_linear *l, float *c, int m, int ldc, int epi, float alpha) {
  // Tile: the largest whose grid still gives every CU a workgroup, else the smallest.
  const int cus = ctx->cus > 0 ? ctx->cus : 256;
  auto tiles = [&](int bm, int bn) { return (long)((l->cols + bn - 1) / bn) * ((m + bm - 1) / bm); };
  int bm = 64, bn = 64;
  if (tiles(128, 128) >= cus) bm = 128, bn = 128;
  else if (tiles(64, 128) >= cus) bm = 64, bn = 128;
  dim3 grid((l->cols + bn - 1) / bn, (m + bm - 1) / bm);
  hipStream_t s = ctx->stream;
  // Algorithmic work: 2·m·rows·k flops over the real rows; bytes of W as stored, a, c (and c read
  // back by the residual epilogues).
  static const char *tn = WT == WH_F32 ? "f32" : WT == WH_F16 ? "f16" : WT == WH_Q8_0 ? "q8_0" : "q4_0";
  char name[64];
  snprintf(name, sizeof name, "gemm_%s_%dx%d", tn, bm, bn);
  double width = l->cols + l->dual;
  double bytes = (double)l->rows * l->row_bytes + 4.0 * m * l->k + 4.0 * m * width * (epi == WH_RESIDUAL || epi == WH_GELU_RESIDUAL ? 2 : 1);
  ProfScope prof(ctx, name, 2.0 * m * l->rows * l->k, bytes);
  if (bm == 128)
    gemm_kernel<WT, 128, 128, ALIGNED><<<grid, 256, 0, s>>>(a, l->w, l->bias, c, m, l->rows, l->cols, l->k, l->dual, ldc, epi, alpha, l->row_bytes);
  else if (bn == 128)
    gemm_kernel<WT, 64, 128, ALIGNED><<<grid, 256, 0, s>>>(a, l->w, l->bias, c, m, l->rows, l->cols, l->k, l->dual, ldc, epi, alpha, l->row_bytes);
  else
    gemm_kernel<WT, 64, 64, ALIGNED><<<grid, 256, 0, s>>>(a, l->w, l->bias, c, m, l->rows, l->cols, l->k, l->dual, ldc, epi, alpha, l->row_bytes);
  return wh_launched(ctx, "gemm");
}

}  // namespace

int launch_gemm(wh_ctx *ctx, const float *a, const wh_linear *l, float *c, int m, int ldc, int epi,
                float alpha) {
  if (m < 0 || !l || (m && (!a || !c))) return wh_fail(ctx, WH_EARG, "gemm: bad arguments (m %d)", m);
  if (epi < WH_BIAS || epi > WH_TANH) return wh_fail(ctx, WH_EARG, "gemm: epilogue %d", epi);
  if (m == 0) return WH_OK;
  if ((uintptr_t)a % 16) return wh_fail(ctx, WH_EARG, "gemm: a must be 16-byte aligned");
  bool aligned = l->k % 64 == 0;
  switch (l->type) {
    case WH_F32: return launch_t<WH_F32, true>(ctx, a, l, c, m, ldc, epi, alpha);
    case WH_F16: return launch_t<WH_F16, true>(ctx, a, l, c, m, ldc, epi, alpha);
    case WH_Q8_0:
      return aligned ? launch_t<WH_Q8_0, true>(ctx, a, l, c, m, ldc, epi, alpha)
                     : launch_t<WH_Q8_0, false>(ctx, a, l, c, m, ldc, epi, alpha);
    case WH_Q4_0:
      return aligned ? launch_t<WH_Q4_0, true>(ctx, a, l, c, m, ldc, epi, alpha)
                     : launch_t<WH_Q4_0, false>(ctx, a, l, c, m, ldc, epi, alpha);
  }
  return wh_fail(ctx, WH_EARG, "gemm: weight type %d", l->type);
}
