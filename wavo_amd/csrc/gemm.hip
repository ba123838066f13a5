// The quantized GEMM of Pass::gemm (src/gpu/mod.rs:1394-1426) on gfx950 matrix cores:
//   c[m][j] = epi(Σ_k h(a[m][k]) · h(W[j][k]) + bias[j]),  h = round to f16 (RNE), f32 accumulate,
// as gemm.wgsl:170-242 and the CPU backend (src/cpu/gemm.rs:126-177) define it.  W stays in HBM as
// the GGUF stores it (src/gguf.rs:14-38): Q8_0 34-byte blocks (f16 scale + 32 int8), Q4_0 18-byte
// blocks (f16 scale + 16 bytes of nibbles), F16 or F32 rows.  Each workgroup stages a BM×64 tile of
// `a` (rounded to f16, or already f16 from its producer) in LDS, double-buffered, while each lane
// loads its own GGUF block of W from HBM straight into registers and dequantizes it to f16(q·d) —
// the reference's exact rounding — as the operand of v_mfma_f32_32x32x16_f16; the epilogues of
// Epilogue::params (src/gpu/mod.rs:445-455; gemm.wgsl:72-94) and the dual outputs are fused into
// the store.
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

// A operand staging: the BM×64 tile of `a` for one k step, f32 (rounded to f16 when stored to
// LDS) or already f16.
template <int BM, bool A16>
struct AStage {
  static constexpr int N = A16 ? BM * 64 / 8 / 256 : BM * 64 / 4 / 256;  // 16-byte loads per thread
  uint4 v[N];
};

template <int BM, bool A16>
__device__ __forceinline__ void load_a(AStage<BM, A16> &s, const void *__restrict__ a, int m, int k, int m0, int k0,
                                       int tid) {
  constexpr int PER_ROW = A16 ? 8 : 16;  // 16-byte pieces per 64-wide row
  constexpr int EL = A16 ? 8 : 4;
#pragma unroll
  for (int p = 0; p < AStage<BM, A16>::N; p++) {
    int f = tid + 256 * p, r = f / PER_ROW, q = f % PER_ROW;
    int row = m0 + r, col = k0 + EL * q;
    const uint8_t *src = (const uint8_t *)a + ((size_t)row * k + col) * (A16 ? 2 : 4);
    s.v[p] = (row < m && col < k) ? *(const uint4 *)src : make_uint4(0, 0, 0, 0);
  }
}

template <int BM, bool A16>
__device__ __forceinline__ void store_a(const AStage<BM, A16> &s, _Float16 *As, int tid) {
#pragma unroll
  for (int p = 0; p < AStage<BM, A16>::N; p++) {
    int f = tid + 256 * p;
    if constexpr (A16) {
      int r = f >> 3, q = f & 7;
      *(uint4 *)(As + r * LDS_ROW + 8 * q) = s.v[p];
    } else {
      int r = f >> 4, q = f & 15;
      float4 x = __builtin_bit_cast(float4, s.v[p]);
      half4 h = {(_Float16)x.x, (_Float16)x.y, (_Float16)x.z, (_Float16)x.w};
      *(half4 *)(As + r * LDS_ROW + 4 * q) = h;
    }
  }
}

// B operand: each lane of a wave holds, per 32-row MFMA tile j of the wave's W rows, row
// n = n0 + wn + 32j + lane%32 and the k half g = lane/32 of the 64-wide step — for Q8_0/Q4_0 exactly
// one GGUF block.  The MFMA's k slots of lane group g at substep s are then k = 32g + 8s..+8 of the
// step, and the A fragments are read with the same permutation, so the products pair up as in
// Σ_k a[m][k]·W[n][k].
template <int WT>
struct BRaw {
  static constexpr int D = WT == WH_Q8_0 ? 9 : WT == WH_Q4_0 ? 5 : WT == WH_F16 ? 16 : 32;  // dwords
  uint32_t d[D];
};

template <int WT, bool ALIGNED>
__device__ __forceinline__ void load_b(BRaw<WT> &s, const uint8_t *__restrict__ w, int rows, int k,
                                       size_t row_bytes, int n, int k0, int g) {
  const int blk = (k0 >> 5) + g;  // the lane's 32-wide k block
  const bool ok = n < rows && blk < (k >> 5);
  const uint8_t *base = w + (size_t)n * row_bytes;
  if constexpr (WT == WH_F16 || WT == WH_F32) {
    const uint4 *p = (const uint4 *)(base + (size_t)blk * 32 * (WT == WH_F16 ? 2 : 4));
#pragma unroll
    for (int i = 0; i < BRaw<WT>::D / 4; i++) {
      uint4 v = ok ? p[i] : make_uint4(0, 0, 0, 0);
      s.d[4 * i] = v.x, s.d[4 * i + 1] = v.y, s.d[4 * i + 2] = v.z, s.d[4 * i + 3] = v.w;
    }
  } else {
    constexpr int BLK = WT == WH_Q8_0 ? 34 : 18;
    if (ALIGNED) {
      // k % 64 == 0: block pairs are 4-byte aligned; block g starts at byte g·BLK of its pair, so
      // block 1 is read from byte BLK − 2 (its scale is then the high half of the first dword).
      const uint32_t *p = (const uint32_t *)(base + (size_t)(k0 >> 6) * 2 * BLK + (g ? BLK - 2 : 0));
#pragma unroll
      for (int i = 0; i < BRaw<WT>::D; i++) s.d[i] = ok ? p[i] : 0u;
    } else {
      constexpr int HW = BLK / 2;
      const uint16_t *p = (const uint16_t *)(base + (size_t)blk * BLK);
#pragma unroll
      for (int j = 0; j < BRaw<WT>::D; j++) {
        uint32_t lo = ok && 2 * j < HW ? p[2 * j] : 0u, hi = ok && 2 * j + 1 < HW ? p[2 * j + 1] : 0u;
        s.d[j] = lo | (hi << 16);
      }
    }
  }
}

// The lane's block as 4 MFMA fragments of 8 halves: f16(q·d) (Q8_0/Q4_0), f16(w) (F32), or as stored.
template <int WT, bool ALIGNED>
__device__ __forceinline__ void dequant_b(const BRaw<WT> &s, int g, half8 f[4]) {
  if constexpr (WT == WH_F16) {
#pragma unroll
    for (int q = 0; q < 4; q++) {
      uint4 v = make_uint4(s.d[4 * q], s.d[4 * q + 1], s.d[4 * q + 2], s.d[4 * q + 3]);
      f[q] = __builtin_bit_cast(half8, v);
    }
  } else if constexpr (WT == WH_F32) {
#pragma unroll
    for (int q = 0; q < 4; q++)
#pragma unroll
      for (int e = 0; e < 8; e++) f[q][e] = (_Float16)__builtin_bit_cast(float, s.d[8 * q + e]);
  } else {
    // Scale in the low half of d[0] (data from byte 2), or for an aligned odd block in the high
    // half (data dword-aligned from d[1]).
    const bool odd = ALIGNED && g;
    const float d = half_bits(odd ? (s.d[0] >> 16) : (s.d[0] & 0xffffu));
    constexpr int NDW = WT == WH_Q8_0 ? 8 : 4;
    uint32_t dw[NDW];
#pragma unroll
    for (int i = 0; i < NDW; i++) dw[i] = odd ? s.d[i + 1] : __builtin_amdgcn_alignbyte(s.d[i + 1], s.d[i], 2);
    if constexpr (WT == WH_Q8_0) {
#pragma unroll
      for (int q = 0; q < 4; q++)
#pragma unroll
        for (int e = 0; e < 8; e++) f[q][e] = (_Float16)((float)(int8_t)(dw[2 * q + e / 4] >> (8 * (e & 3))) * d);
    } else {
      // ggml block_q4_0: element i < 16 is the low nibble of byte i, 16 + i the high one.
#pragma unroll
      for (int q = 0; q < 4; q++)
#pragma unroll
        for (int e = 0; e < 8; e++) {
          const int i = 8 * q + e, byte = i & 15;
          const uint32_t v = (dw[byte >> 2] >> (8 * (byte & 3))) & 0xffu;
          f[q][e] = (_Float16)((float)((int)(i < 16 ? (v & 15u) : (v >> 4)) - 8) * d);
        }
    }
  }
}

template <int WT, int BM, int BN, bool ALIGNED, bool A16>
__global__ __launch_bounds__(256) void gemm_kernel(const void *__restrict__ a, const uint8_t *__restrict__ w,
                                                   const float *__restrict__ bias, float *__restrict__ c,
                                                   int m, int rows, int cols, int k, int dual, int ldc,
                                                   int epi, float alpha, size_t row_bytes) {
  __shared__ __attribute__((aligned(16))) _Float16 As[2][BM * LDS_ROW];
  constexpr int TM = BM / 64, TN = BN / 64;  // 32×32 MFMA tiles per wave (2×2 waves)
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int n0 = blockIdx.x * BN, m0 = blockIdx.y * BM;
  const int wm = (wave >> 1) * (BM / 2), wn = (wave & 1) * (BN / 2);
  const int lrow = lane & 31, g = lane >> 5;
  floatx16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; i++)
#pragma unroll
    for (int j = 0; j < TN; j++) acc[i][j] = floatx16{};

  AStage<BM, A16> as;
  BRaw<WT> bs[TN];
  load_a<BM, A16>(as, a, m, k, m0, 0, tid);
#pragma unroll
  for (int j = 0; j < TN; j++) load_b<WT, ALIGNED>(bs[j], w, rows, k, row_bytes, n0 + wn + 32 * j + lrow, 0, g);
  store_a<BM, A16>(as, As[0], tid);
  __syncthreads();
  int buf = 0;
  for (int k0 = 0; k0 < k; k0 += BK) {
    half8 bf[TN][4];
#pragma unroll
    for (int j = 0; j < TN; j++) dequant_b<WT, ALIGNED>(bs[j], g, bf[j]);
    const bool more = k0 + BK < k;
    if (more) {
      load_a<BM, A16>(as, a, m, k, m0, k0 + BK, tid);
#pragma unroll
      for (int j = 0; j < TN; j++) load_b<WT, ALIGNED>(bs[j], w, rows, k, row_bytes, n0 + wn + 32 * j + lrow, k0 + BK, g);
    }
    const _Float16 *at = As[buf];
#pragma unroll
    for (int s = 0; s < 4; s++) {
      half8 af[TM];
#pragma unroll
      for (int i = 0; i < TM; i++) af[i] = *(const half8 *)(at + (wm + 32 * i + lrow) * LDS_ROW + 32 * g + 8 * s);
#pragma unroll
      for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j][s], acc[i][j], 0, 0, 0);
    }
    if (more) store_a<BM, A16>(as, As[buf ^ 1], tid);
    __syncthreads();
    buf ^= 1;
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

template <int WT, bool ALIGNED, bool A16>
int launch_t(wh_ctx *ctx, const void *a, const wh_linear *l, float *c, int m, int ldc, int epi, float alpha) {
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
  snprintf(name, sizeof name, "gemm_%s%s_%dx%d", tn, A16 ? "_a16" : "", bm, bn);
  double width = l->cols + l->dual;
  double bytes = (double)l->rows * l->row_bytes + (A16 ? 2.0 : 4.0) * m * l->k +
                 4.0 * m * width * (epi == WH_RESIDUAL || epi == WH_GELU_RESIDUAL ? 2 : 1);
  ProfScope prof(ctx, name, 2.0 * m * l->rows * l->k, bytes);
  if (bm == 128)
    gemm_kernel<WT, 128, 128, ALIGNED, A16><<<grid, 256, 0, s>>>(a, l->w, l->bias, c, m, l->rows, l->cols, l->k, l->dual, ldc, epi, alpha, l->row_bytes);
  else if (bn == 128)
    gemm_kernel<WT, 64, 128, ALIGNED, A16><<<grid, 256, 0, s>>>(a, l->w, l->bias, c, m, l->rows, l->cols, l->k, l->dual, ldc, epi, alpha, l->row_bytes);
  else
    gemm_kernel<WT, 64, 64, ALIGNED, A16><<<grid, 256, 0, s>>>(a, l->w, l->bias, c, m, l->rows, l->cols, l->k, l->dual, ldc, epi, alpha, l->row_bytes);
  return wh_launched(ctx, "gemm");
}

template <bool A16>
int launch_typed(wh_ctx *ctx, const void *a, const wh_linear *l, float *c, int m, int ldc, int epi, float alpha) {
  const bool aligned = l->k % 64 == 0;
  switch (l->type) {
    case WH_F32: return launch_t<WH_F32, true, A16>(ctx, a, l, c, m, ldc, epi, alpha);
    case WH_F16: return launch_t<WH_F16, true, A16>(ctx, a, l, c, m, ldc, epi, alpha);
    case WH_Q8_0:
      return aligned ? launch_t<WH_Q8_0, true, A16>(ctx, a, l, c, m, ldc, epi, alpha)
                     : launch_t<WH_Q8_0, false, A16>(ctx, a, l, c, m, ldc, epi, alpha);
    case WH_Q4_0:
      return aligned ? launch_t<WH_Q4_0, true, A16>(ctx, a, l, c, m, ldc, epi, alpha)
                     : launch_t<WH_Q4_0, false, A16>(ctx, a, l, c, m, ldc, epi, alpha);
  }
  return wh_fail(ctx, WH_EARG, "gemm: weight type %d", l->type);
}

}  // namespace

int launch_gemm(wh_ctx *ctx, const float *a, const wh_linear *l, float *c, int m, int ldc, int epi,
                float alpha) {
  if (m < 0 || !l || (m && (!a || !c))) return wh_fail(ctx, WH_EARG, "gemm: bad arguments (m %d)", m);
  if (epi < WH_BIAS || epi > WH_TANH) return wh_fail(ctx, WH_EARG, "gemm: epilogue %d", epi);
  if (m == 0) return WH_OK;
  if ((uintptr_t)a % 16) return wh_fail(ctx, WH_EARG, "gemm: a must be 16-byte aligned");
  return launch_typed<false>(ctx, a, l, c, m, ldc, epi, alpha);
}

int launch_gemm_h(wh_ctx *ctx, const void *a16, const wh_linear *l, float *c, int m, int ldc, int epi,
                  float alpha) {
  if (m < 0 || !l || (m && (!a16 || !c))) return wh_fail(ctx, WH_EARG, "gemm: bad arguments (m %d)", m);
  if (epi < WH_BIAS || epi > WH_TANH) return wh_fail(ctx, WH_EARG, "gemm: epilogue %d", epi);
  if (m == 0) return WH_OK;
  if ((uintptr_t)a16 % 16) return wh_fail(ctx, WH_EARG, "gemm: a must be 16-byte aligned");
  return launch_typed<true>(ctx, a16, l, c, m, ldc, epi, alpha);
}
