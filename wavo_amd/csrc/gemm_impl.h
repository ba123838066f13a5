// The GEMM kernels and their launch templates, shared by gemm.hip and the per-weight-type
// translation units gemm_lds_{q8_0,q4_0,f16}.hip (each instantiates the LDS-DMA kernel for one
// weight type, so that the three compile in parallel).  The kernels are described in gemm.hip.
#pragma once
#include <algorithm>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <type_traits>
#include <utility>
#include "internal.h"
#include "xlane.h"

// Launch shapes of the LDS-DMA kernel: tile, wavefronts per tile row and column, ring slots, k split
// over workgroups, loop variant, k groups (wavefront sets that take the k steps in turn).
struct GemmPlan {
  int bm, bn, wm, wn, ns, split, pipe = 0, wk = 1;
};

// The launch plan of an m × cols × k GEMM (gemm.hip).
GemmPlan gemm_plan_for(const wh_ctx *ctx, int m, int cols, int k);

namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef _Float16 half2 __attribute__((ext_vector_type(2)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

constexpr int BK = 64;       // k per stage: two quantized blocks
constexpr int LDS_ROW = 72;  // halves per LDS row (144 B: 16-byte aligned rows, banks staggered)

__device__ __forceinline__ float gelu(float x) {
  // Abramowitz–Stegun 7.1.26 erf, as gemm.wgsl:65-70 and src/cpu/ops.rs:33-40.
  float z = fabsf(0.70710678118654752440f * x);
  float t = __builtin_amdgcn_rcpf(1.0f + 0.3275911f * z);  // 1 ulp, against ~10 instructions of IEEE division
  float e = 1.0f - (((((1.061405429f * t - 1.453152027f) * t) + 1.421413741f) * t - 0.284496736f) * t +
                     0.254829592f) * t * __expf(-z * z);
  float s = x > 0.0f ? 1.0f : (x < 0.0f ? -1.0f : 0.0f);
  return 0.5f * x * (1.0f + s * e);
}

__device__ __forceinline__ float epilogue(int epi, float alpha, float v, const float *c) {
  switch (epi) {
    case WH_SILU: return v * __builtin_amdgcn_rcpf(1.0f + __expf(-v));
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

template <int WT, int BM, int BN, bool ALIGNED, bool A16, bool OUT16>
__global__ __launch_bounds__(256) void gemm_reg_kernel(const void *__restrict__ a, const uint8_t *__restrict__ w,
                                                   const float *__restrict__ bias, void *__restrict__ c,
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
        const size_t at = (size_t)row * ldc + col;
        float x = col < rows ? acc[i][j][v] : 0.0f;
        if constexpr (OUT16) {
          _Float16 *cp = (_Float16 *)c + at;
          *cp = (_Float16)epilogue(epi, alpha, x + bv, nullptr);
          if (col < dual) cp[cols] = (_Float16)(x + b2);
        } else {
          float *cp = (float *)c + at;
          *cp = epilogue(epi, alpha, x + bv, cp);
          if (col < dual) cp[cols] = x + b2;
        }
      }
    }
}


// ------------------------------------------------------------------------------------ LDS-DMA path

__device__ __forceinline__ uint32_t lds_addr(const void *p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)p;
}

// LDS DMA (counted by vmcnt): each lane copies 16 (dma16) or 4 (dma4) bytes at `src` to LDS byte
// lds + 16·lane (4·lane); `lds` is wave-uniform.
__device__ __forceinline__ void dma16(const void *src, uint32_t lds) {
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "{m0}"(__builtin_amdgcn_readfirstlane(lds))
               : "memory");
}
__device__ __forceinline__ void dma4(const void *src, uint32_t lds) {
  asm volatile("s_nop 0\n\tglobal_load_lds_dword %0, off" ::"v"(src), "{m0}"(__builtin_amdgcn_readfirstlane(lds))
               : "memory");
}
__device__ __forceinline__ void dma_wait() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }
// The same from a wave-uniform base address (SGPRs) plus a per-lane 32-bit byte offset, so that a
// loop moves the whole DMA by scalar adds.  `lds` must be wave-uniform (it goes to M0).
__device__ __forceinline__ void dma16s(const void *base, uint32_t off, uint32_t lds) {
  // (the base through readfirstlane: a scalar value even where the scalar registers run short; the
  // halves as unsigned 32-bit values, since readfirstlane returns int and must not sign-extend)
  const uint64_t b = (uint64_t)(uintptr_t)base;
  const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(b >> 32));
  const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)b);
  const uint64_t bs = ((uint64_t)hi << 32) | (uint64_t)lo;
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(bs), "{m0}"(lds) : "memory");
}
__device__ __forceinline__ void dma4s(const void *base, uint32_t off, uint32_t lds) {
  asm volatile("s_nop 0\n\tglobal_load_lds_dword %0, %1" ::"v"(off), "s"(base), "{m0}"(lds) : "memory");
}

// Two f16 values 1024 + byte0, 1024 + byte1 of x (bytes 0-1, or 2-3 with HI).
template <bool HI>
__device__ __forceinline__ half2 magic_pair(uint32_t x) {
  return __builtin_bit_cast(half2, __builtin_amdgcn_perm(0x64646464u, x, HI ? 0x04030402u : 0x04010400u));
}

// Two int8 of x (bytes 0-1, or 2-3 with HI) as two f16 (exact: |q| ≤ 128), by sub-dword operand
// selection of the conversion itself (SDWA: sign-extended byte in, one half of the result out).
template <bool HI>
__device__ __forceinline__ half2 i8_pair(uint32_t x) {
  uint32_t r;
  if constexpr (HI)
    asm("v_cvt_f16_i16_sdwa %0, sext(%1) dst_sel:WORD_0 dst_unused:UNUSED_PAD src0_sel:BYTE_2\n\t"
        "v_cvt_f16_i16_sdwa %0, sext(%1) dst_sel:WORD_1 dst_unused:UNUSED_PRESERVE src0_sel:BYTE_3"
        : "=&v"(r) : "v"(x));
  else
    asm("v_cvt_f16_i16_sdwa %0, sext(%1) dst_sel:WORD_0 dst_unused:UNUSED_PAD src0_sel:BYTE_0\n\t"
        "v_cvt_f16_i16_sdwa %0, sext(%1) dst_sel:WORD_1 dst_unused:UNUSED_PRESERVE src0_sel:BYTE_1"
        : "=&v"(r) : "v"(x));
  return __builtin_bit_cast(half2, r);
}

// Q8_0 MFMA fragment of substep S: elements 16·(S % 2) + 8g .. + 8 of block S / 2 of the lane's W
// row pair, f16(q·d) — the exact conversion of q, then one packed f16 multiply by the block scale.
// w = the lane's dwords (read_w): for block 0 (data from byte 2 of the pair) three dwords per
// substep holding the elements from byte 2, for block 1 (data from byte 36) two aligned dwords.
template <int S>
__device__ __forceinline__ half8 dequant_q8(const uint32_t *w, half2 d2) {
  half2 p[4];
  if constexpr (S < 2) {
    const uint32_t *x = w + 3 * S;
    p[0] = i8_pair<true>(x[0]), p[1] = i8_pair<false>(x[1]), p[2] = i8_pair<true>(x[1]), p[3] = i8_pair<false>(x[2]);
  } else {
    const uint32_t *x = w + 6 + 2 * (S - 2);
    p[0] = i8_pair<false>(x[0]), p[1] = i8_pair<true>(x[0]), p[2] = i8_pair<false>(x[1]), p[3] = i8_pair<true>(x[1]);
  }
  half8 f;
#pragma unroll
  for (int h = 0; h < 4; h++) {
    const half2 v = p[h] * d2;
    f[2 * h] = v[0], f[2 * h + 1] = v[1];
  }
  return f;
}

// The MFMA fragment of substep s (elements 8s .. 8s + 7) of one block.  dw = the block's data
// dwords as read from LDS at the lane's offset, `sh` = bytes of that offset before the data (2 for
// the even block of a pair: data from byte 2; 0 for the odd one: data dword-aligned), d2 = the
// block's scale twice.
template <int WT>
__device__ __forceinline__ half8 dequant_frag(const uint32_t *dw, uint32_t sh, half2 d2, int s) {
  half8 f;
  if constexpr (WT == WH_Q8_0) {
    const half2 bias = {(_Float16)1152.0f, (_Float16)1152.0f};  // 1024 + 128
#pragma unroll
    for (int h = 0; h < 2; h++) {
      const uint32_t x = __builtin_amdgcn_alignbyte(dw[2 * s + h + 1], dw[2 * s + h], sh) ^ 0x80808080u;
      const half2 p0 = (magic_pair<false>(x) - bias) * d2, p1 = (magic_pair<true>(x) - bias) * d2;
      f[4 * h] = p0[0], f[4 * h + 1] = p0[1], f[4 * h + 2] = p1[0], f[4 * h + 3] = p1[1];
    }
  } else {
    // ggml block_q4_0: element i < 16 is the low nibble of byte i, 16 + i the high one; value
    // (nibble − 8)·d.  Substeps 0-1 take low nibbles of bytes 0-15, substeps 2-3 high ones.
    const half2 bias = {(_Float16)1032.0f, (_Float16)1032.0f};  // 1024 + 8
#pragma unroll
    for (int h = 0; h < 2; h++) {
      const int q = 2 * (s & 1) + h;
      const uint32_t x = __builtin_amdgcn_alignbyte(dw[q + 1], dw[q], sh);
      const uint32_t nib = s < 2 ? x & 0x0f0f0f0fu : (x >> 4) & 0x0f0f0f0fu;
      const half2 p0 = (magic_pair<false>(nib) - bias) * d2, p1 = (magic_pair<true>(nib) - bias) * d2;
      f[4 * h] = p0[0], f[4 * h + 1] = p0[1], f[4 * h + 2] = p1[0], f[4 * h + 3] = p1[1];
    }
  }
  return f;
}

// Work of one gemm_lds_kernel launch.
struct LdsArgs {
  const _Float16 *a;
  const uint8_t *w;
  const float *bias;
  void *c;          // output, or f32 partial sums [split][m][cols] with SPLIT
  int m, rows, cols, k, dual, ldc, epi;
  float alpha;
  size_t row_bytes;
  HeadsOut ho[2];  // column ranges written in attention's packed layout instead of into c (f16 outputs)
  int nho;
  // Non-null: the launch does nothing when *skip == skip_val (c already holds this product: an
  // input-independent GEMM whose output is kept between calls, tagged on the device).
  const int *skip;
  int skip_val;
  // Row tiles per group of the tile order (1: row by row; see the kernel's tile order).
  int group;
};

// s_waitcnt with vmcnt = N (0..63) and no wait on the other counters (gfx9 encoding: vmcnt bits
// 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8).
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// f(integral_constant<S>, kt0 + S) for S = I .. N − 1 while kt0 + S < nk: a loop body unrolled with
// its step index known at compile time.
template <int I, int N, class F>
__device__ __forceinline__ void unrolled_steps(F &f, int kt0, int nk) {
  if constexpr (I < N) {
    if (kt0 + I < nk) {
      f(std::integral_constant<int, I>{}, kt0 + I);
      unrolled_steps<I + 1, N>(f, kt0, nk);
    }
  }
}

// f(integral_constant<I>) for I = B, B + S, .. < E.
template <int B, int E, int S, class F>
__device__ __forceinline__ void static_for(F &&f) {
  if constexpr (B < E) {
    f(std::integral_constant<int, B>{});
    static_for<B + S, E, S>(f);
  }
}

// The row-major epilogue's lane order and the half of its 8 columns a lane reads first (rows of
// BN + 8 floats in LDS).  gfx950 serves a 16-byte LDS read in four passes of 16 lanes (the two
// half-waves, each split by the parity of lane bits 2-4), and a lane's two reads of one row land in
// the low and the high half of a 32-byte slot, so reading the low halves first everywhere gives every
// pass of a 64-column tile, which holds four rows, a 3-way bank conflict.  There lane bits 1 and 2 and
// bits 4 and 5 are swapped and odd rows read their high half first: each pass then hits 16 distinct
// 4-bank groups (found by enumerating lane-bit permutations and half rules over every pass; the
// 750-frame step 4.06-4.09 -> 4.04 ms).  128- and 256-column tiles keep the plain order (2-way
// conflicts): their conflict-free orders measured slower, the 128-column one in the 750-frame step
// (4.05 against 4.04 ms), the 256-column one in the 16-window batch (24.69 against 24.50 ms).
template <int BN>
__device__ __forceinline__ int epi_lane(int tid) {
  if constexpr (BN == 64) {
    const int l = tid & 63;
    return (tid & ~63) | (l & 0b001001) | ((l >> 1) & 0b000010) | ((l << 1) & 0b000100) | ((l >> 1) & 0b010000) |
           ((l << 1) & 0b100000);
  } else {
    return tid;
  }
}
template <int BN>
__device__ __forceinline__ int epi_half(int r) {
  return BN == 64 ? r & 1 : 0;
}

// The epilogue's store of NR rows × BN columns of a tile whose f32 sums sit in LDS (cl, rows of `crow`
// floats): NT threads take 8 consecutive columns each (16-byte loads of c for the residual modes,
// 16-byte stores), applying the bias (bb, loaded by the caller for the thread's fixed column group),
// the epilogue, the dual columns (bd) and the padding columns (epi(0 + bias), as the reference's zero
// rows give); a split GEMM stores its plain partial sums into plane tz instead.  A pass holds, for
// every row group of RPW tile rows (one per row of wavefronts), PGR of its rows from row 32·i0: LDS
// row r is tile row (r / PGR)·RPW + 32·i0 + r % PGR (PGR = RPW, i0 = 0: the whole tile in order).
template <int NR, int RPW, int PGR, int BN, int NT, bool SPLIT, bool OUT16, bool TWO = false>
__device__ __forceinline__ void store_c_tile(const LdsArgs &P, const float *cl, int crow, int tid, int m0, int n0,
                                             int tz, int i0, const float (&bb)[8], const float (&bd)[8],
                                             const float *cl2 = nullptr, int ccol = 0) {
  constexpr int G8 = BN / 8;
  // The tile's sums: with TWO the two k groups' planes added as they are read (group 0's + group 1's).
  auto rd4 = [&](int off) {
    float4 a = *(const float4 *)(cl + off);
    if constexpr (TWO) {
      const float4 b = *(const float4 *)(cl2 + off);
      a.x += b.x, a.y += b.y, a.z += b.z, a.w += b.w;
    }
    return a;
  };
  auto rd1 = [&](int off) {
    float a = cl[off];
    if constexpr (TWO) a += cl2[off];
    return a;
  };
  // Row r's 8 columns from c8, in the read order of epi_half (x in column order).
  auto rd8 = [&](int r, int c8, float (&x)[8]) {
    const int h = epi_half<BN>(r);
    const float4 u = rd4(r * crow + c8 + 4 * h), v = rd4(r * crow + c8 + 4 - 4 * h);
    const float4 lo = h ? v : u, hi = h ? u : v;
    x[0] = lo.x, x[1] = lo.y, x[2] = lo.z, x[3] = lo.w, x[4] = hi.x, x[5] = hi.y, x[6] = hi.z, x[7] = hi.w;
  };
  const int et = epi_lane<BN>(tid);  // the lane's place in the row-major rounds below
  const int m = P.m, rows = P.rows;
  static_assert((NR * G8) % NT == 0, "whole rounds of column groups");
  static_assert(PGR % 32 == 0 && RPW % PGR == 0, "passes of whole 32-row groups");
  const int m0p = m0 + 32 * i0;  // tile row of LDS row r: m0p + trow(r)
  auto trow = [](int r) { return (r / PGR) * RPW + r % PGR; };
  constexpr int BM = NR;
  if constexpr (OUT16 && !SPLIT) {
    // A tile inside a packed range (the host keeps each range on whole tiles): f16 rows per head or,
    // transposed, 8 rows of one column per store; the epilogue as below (no residual, no dual).
#pragma unroll
    for (int o = 0; o < 2; o++) {  // constant indices: the ranges stay in the kernel arguments
      if (o >= P.nho) break;
      const HeadsOut &h = P.ho[o];
      if (n0 < h.col0 || n0 >= h.col0 + h.cols) continue;
      if (h.tr && ccol) {
        // The tile staged column by column (ccol floats per LDS column): a column's 8 rows are two
        // 16-byte reads.  Lanes down the rows of a column (rows per head of Vᵀ are contiguous), or,
        // blocked, along the columns in pairs of 8-row halves (a block's columns follow each other).
        // Every item's bias loaded before the first store (a load after a store to memory that may
        // alias it would wait for a round trip per item).
        constexpr int ITS = (BM * G8 + NT - 1) / NT;
        float bi[ITS];
#pragma unroll
        for (int it = 0; it < ITS; it++) {
          const int e = tid + it * NT, c = h.blk ? (e >> 1) % BN : e / (BM / 8);
          bi[it] = e < BM * G8 && n0 + c < P.cols ? P.bias[n0 + c] : 0.0f;
        }
#pragma unroll
        for (int it = 0; it < ITS; it++) {
          const int e = tid + it * NT;
          if (e >= BM * G8) break;
          const int c = h.blk ? (e >> 1) % BN : e / (BM / 8);
          const int r0 = h.blk ? 8 * ((e & 1) + 2 * (e / (2 * BN))) : 8 * (e % (BM / 8));
          const int row0 = m0p + trow(r0), col = n0 + c;
          if (row0 >= h.rs || col >= P.cols) continue;
          const float b = bi[it];
          const float4 x0 = rd4(c * ccol + r0), x1 = rd4(c * ccol + r0 + 4);
          const float x[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
          half8 y;
#pragma unroll
          for (int q = 0; q < 8; q++) y[q] = (_Float16)(row0 + q < m ? epilogue(P.epi, 0.0f, x[q] + b, nullptr) : 0.0f);
          const size_t at = h.blk ? (size_t)(row0 / h.blk) * h.cols * h.blk + (size_t)(col - h.col0) * h.blk + row0 % h.blk
                                  : (size_t)(col - h.col0) * h.rs + row0;
          *(half8 *)(h.dst + at) = y;
        }
      } else if (h.tr) {
        // A lane's column is the same in every round (NT % BN == 0): its bias loaded once, before the
        // stores.
        static_assert(NT % BN == 0, "a fixed column per lane");
        const float b = n0 + tid % BN < P.cols ? P.bias[n0 + tid % BN] : 0.0f;
#pragma unroll
        for (int it = 0; it < BM * G8 / NT; it++) {
          const int e = tid + it * NT, c = e % BN, r0 = 8 * (e / BN), row0 = m0p + trow(r0), col = n0 + c;
          if (row0 >= h.rs || col >= P.cols) continue;
          half8 y;
#pragma unroll
          for (int q = 0; q < 8; q++)
            y[q] = (_Float16)(row0 + q < m ? epilogue(P.epi, 0.0f, rd1((r0 + q) * crow + c) + b, nullptr) : 0.0f);
          // head j, dim i: row j·hd + i; blocked: 8 rows of one block (row0 % 8 == 0, blk % 8 == 0)
          const size_t at = h.blk ? (size_t)(row0 / h.blk) * h.cols * h.blk + (size_t)(col - h.col0) * h.blk + row0 % h.blk
                                  : (size_t)(col - h.col0) * h.rs + row0;
          *(half8 *)(h.dst + at) = y;
        }
      } else {
#pragma unroll
        for (int it = 0; it < BM * G8 / NT; it++) {
          const int e = et + it * NT, r = e / G8, c8 = 8 * (e % G8), row = m0p + trow(r), col = n0 + c8;
          if (row + h.r0 >= h.rs || col >= P.cols) continue;
          half8 y;
          if (row < m) {
            float x[8];
            rd8(r, c8, x);
#pragma unroll
            for (int q = 0; q < 8; q++) y[q] = (_Float16)epilogue(P.epi, 0.0f, x[q] + bb[q], nullptr);
          } else {
#pragma unroll
            for (int q = 0; q < 8; q++) y[q] = (_Float16)0.0f;
          }
          const int v = col - h.col0;  // 8 columns of one head (hd % 8 == 0)
          *(half8 *)(h.dst + ((size_t)(v / h.hd) * h.rs + h.r0 + row) * h.hd + v % h.hd) = y;
        }
      }
      return;
    }
  }
  if constexpr (!SPLIT) {
    // A tile of real, non-dual columns only (every tile but the edge ones): the epilogue mode chosen
    // once per tile, no per-column checks, pairs converted to f16 by one instruction.
    if (n0 + BN <= rows && n0 >= P.dual) {
      auto run = [&](auto E_c) {
        constexpr int E = decltype(E_c)::value;
#pragma unroll
        for (int it = 0; it < BM * G8 / NT; it++) {
          const int e = et + it * NT, r = e / G8, c8 = 8 * (e % G8), row = m0p + trow(r), col = n0 + c8;
          if (row >= m) continue;
          float x[8];
          rd8(r, c8, x);
          if constexpr (E == EPI_GLU) {  // 4 channels from the group [a₀..a₃ | g₀..g₃] at col
            float4 v;
            v.x = (x[0] + bb[0]) * __builtin_amdgcn_rcpf(1.0f + __expf(-(x[4] + bb[4])));
            v.y = (x[1] + bb[1]) * __builtin_amdgcn_rcpf(1.0f + __expf(-(x[5] + bb[5])));
            v.z = (x[2] + bb[2]) * __builtin_amdgcn_rcpf(1.0f + __expf(-(x[6] + bb[6])));
            v.w = (x[3] + bb[3]) * __builtin_amdgcn_rcpf(1.0f + __expf(-(x[7] + bb[7])));
            *(float4 *)((float *)P.c + (size_t)row * P.ldc + col / 2) = v;
            continue;
          }
          const size_t at = (size_t)row * P.ldc + col;
          float y[8];
          if constexpr (!OUT16 && (E == WH_RESIDUAL || E == WH_GELU_RESIDUAL)) {
            const float4 c0 = *(const float4 *)((const float *)P.c + at), c1 = *(const float4 *)((const float *)P.c + at + 4);
            const float cc[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
#pragma unroll
            for (int q = 0; q < 8; q++) y[q] = E == WH_RESIDUAL ? cc[q] + P.alpha * (x[q] + bb[q]) : cc[q] + gelu(x[q] + bb[q]);
          } else {
#pragma unroll
            for (int q = 0; q < 8; q++) y[q] = epilogue(E, 0.0f, x[q] + bb[q], nullptr);
          }
          if constexpr (OUT16) {
            typedef float float2v __attribute__((ext_vector_type(2)));
            half8 h;
#pragma unroll
            for (int q = 0; q < 4; q++) {
              const half2 p = __builtin_convertvector(float2v{y[2 * q], y[2 * q + 1]}, half2);
              h[2 * q] = p[0], h[2 * q + 1] = p[1];
            }
            *(half8 *)((_Float16 *)P.c + at) = h;
          } else {
            *(float4 *)((float *)P.c + at) = make_float4(y[0], y[1], y[2], y[3]);
            *(float4 *)((float *)P.c + at + 4) = make_float4(y[4], y[5], y[6], y[7]);
          }
        }
      };
      switch (P.epi) {
        case WH_SILU: run(std::integral_constant<int, WH_SILU>{}); return;
        case WH_RELU: run(std::integral_constant<int, WH_RELU>{}); return;
        case WH_GELU: run(std::integral_constant<int, WH_GELU>{}); return;
        case WH_TANH: run(std::integral_constant<int, WH_TANH>{}); return;
        case WH_RESIDUAL:
          if constexpr (!OUT16) { run(std::integral_constant<int, WH_RESIDUAL>{}); return; }
          break;
        case WH_GELU_RESIDUAL:
          if constexpr (!OUT16) { run(std::integral_constant<int, WH_GELU_RESIDUAL>{}); return; }
          break;
        case EPI_GLU:
          if constexpr (!OUT16) { run(std::integral_constant<int, EPI_GLU>{}); return; }
          break;
        default: run(std::integral_constant<int, WH_BIAS>{}); return;
      }
    }
  }
#pragma unroll
  for (int it = 0; it < BM * G8 / NT; it++) {
    const int e = et + it * NT, r = e / G8, c8 = 8 * (e % G8), row = m0p + trow(r), col = n0 + c8;
    if (row >= m || col >= P.cols) continue;  // cols % 32 == 0: a group is inside or past
    float x[8];
    rd8(r, c8, x);
    if constexpr (SPLIT) {
      float *cp = (float *)P.c + ((size_t)tz * m + row) * P.cols + col;
      *(float4 *)cp = make_float4(x[0], x[1], x[2], x[3]);
      *(float4 *)(cp + 4) = make_float4(x[4], x[5], x[6], x[7]);
      continue;
    }
#pragma unroll
    for (int q = 0; q < 8; q++)
      if (col + q >= rows) x[q] = 0.0f;
    if (!OUT16 && P.epi == EPI_GLU) {  // as in the interior path (the host keeps whole groups of real columns)
      float4 v;
      v.x = (x[0] + bb[0]) * __builtin_amdgcn_rcpf(1.0f + __expf(-(x[4] + bb[4])));
      v.y = (x[1] + bb[1]) * __builtin_amdgcn_rcpf(1.0f + __expf(-(x[5] + bb[5])));
      v.z = (x[2] + bb[2]) * __builtin_amdgcn_rcpf(1.0f + __expf(-(x[6] + bb[6])));
      v.w = (x[3] + bb[3]) * __builtin_amdgcn_rcpf(1.0f + __expf(-(x[7] + bb[7])));
      *(float4 *)((float *)P.c + (size_t)row * P.ldc + col / 2) = v;
      continue;
    }
    const size_t at = (size_t)row * P.ldc + col;
    float y[8];
    if (!OUT16 && (P.epi == WH_RESIDUAL || P.epi == WH_GELU_RESIDUAL)) {
      const float4 c0 = *(const float4 *)((const float *)P.c + at), c1 = *(const float4 *)((const float *)P.c + at + 4);
      const float cc[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
      if (P.epi == WH_RESIDUAL)
#pragma unroll
        for (int q = 0; q < 8; q++) y[q] = cc[q] + P.alpha * (x[q] + bb[q]);
      else
#pragma unroll
        for (int q = 0; q < 8; q++) y[q] = cc[q] + gelu(x[q] + bb[q]);
    } else {
      switch (P.epi) {
#define EPI_CASE(E)                                                               \
  case E:                                                                         \
    _Pragma("unroll") for (int q = 0; q < 8; q++) y[q] = epilogue(E, 0.0f, x[q] + bb[q], nullptr); \
    break;
        EPI_CASE(WH_SILU)
        EPI_CASE(WH_RELU)
        EPI_CASE(WH_GELU)
        EPI_CASE(WH_TANH)
#undef EPI_CASE
        default:
#pragma unroll
          for (int q = 0; q < 8; q++) y[q] = x[q] + bb[q];
      }
    }
    const bool dual = col < P.dual;  // dual % 8 == 0 is not required: per column below
    if constexpr (OUT16) {
      half8 h;
#pragma unroll
      for (int q = 0; q < 8; q++) h[q] = (_Float16)y[q];
      *(half8 *)((_Float16 *)P.c + at) = h;
    } else {
      *(float4 *)((float *)P.c + at) = make_float4(y[0], y[1], y[2], y[3]);
      *(float4 *)((float *)P.c + at + 4) = make_float4(y[4], y[5], y[6], y[7]);
    }
    if (dual) {
#pragma unroll
      for (int q = 0; q < 8; q++) {
        if (col + q >= P.dual) break;
        const float d = x[q] + bd[q];
        if constexpr (OUT16) ((_Float16 *)P.c)[at + P.cols + q] = (_Float16)d;
        else ((float *)P.c)[at + P.cols + q] = d;
      }
    }
  }
}

// c tile BM × BN per workgroup of WM × WN wavefronts, each a (BM/WM) × (BN/WN) block of 32×32 MFMA
// tiles, over the k range of its split (the 64-wide k steps divided evenly over gridDim.z).
//
// Pipeline.  The k loop moves in 64-wide steps through a ring of NS LDS slots that the LDS DMA
// fills NS steps ahead, from scalar base addresses (a step costs the vector units nothing but the
// dequantization).  A step is 4 substeps of 16 k; each wave reads the a fragments of substep s + 1
// while the MFMAs of substep s run, and the W data of the next step after the one barrier of the
// step, which sits after substep 2: there every wave has waited for the next stage's DMA and has read
// everything it needs of the current slot into registers (the last substep's a fragments before the
// third substep's MFMAs, the step's W data one step earlier), so the DMA of step kt + NS goes into
// the current slot right after the barrier, and a stage has NS − 1 steps to land.  The loop is
// unrolled by the ring length so that every LDS offset is an immediate.  The DMA of a stage is spread
// over the wavefronts, each instruction issued once (an instruction costs the memory pipeline the same
// ~16 cycles whatever its width, so W rows move in 16-byte chunks too).
//
// LDS layout: the a stages (rows of 8 16-byte chunks, chunk c of row r at (c + r/2) % 8 — the 16
// lanes that LDS serves together read 16 rows and hit all 64 banks once), then the W stages: F16
// rows like a, or quantized rows of one block pair (68 or 36 bytes, as stored) in LDS rows of 80 or
// 48 bytes (whole 16-byte chunks from the pair's start).  At substep s, the
// lane of MFMA column n and k half g takes k slots 32g + 8s .. + 8 — block g of its W row's pair —
// and the a fragments the same slots.
//
// Epilogue.  The accumulators go through LDS (f32, rows padded so the two lane halves of a tile hit
// distinct banks) and leave as 8 consecutive columns per lane: 16-byte loads of c for the residual
// modes and 16-byte stores, with the bias, the epilogue, the dual columns and the padding columns
// (epi(0 + bias), as the reference's zero rows give) applied on the way.  A tile whose f32 sums do
// not fit in the ring's LDS goes through in passes of whole 32-row MFMA tiles of every wavefront.
template <int WT, int BM, int BN, int WM, int WN, int NSQ, bool SPLIT, bool OUT16, int PIPE, int WK>
__global__ __launch_bounds__(64 * WM * WN * WK) void gemm_lds_kernel(LdsArgs P) {
  constexpr int NW = WM * WN;  // wavefronts of one k group
  constexpr int NWT = NW * WK;  // of the workgroup
  static_assert(WK == 1 || (WK == 2 && PIPE == 0), "k groups in the plain loop");
  constexpr int TM = BM / WM / 32, TN = BN / WN / 32;
  static_assert(TM >= 1 && TN >= 1, "32×32 MFMA tiles per wave");
  constexpr int PAIR1 = WT == WH_Q8_0 ? 68 : WT == WH_Q4_0 ? 36 : 128;  // W bytes of 64 weights
  constexpr bool WCH = WT == WH_F16;                                     // W moves in 16-byte chunks
  // A quantized W row's block pair moves as whole 16-byte chunks from its (4-byte aligned) start: 5
  // chunks (80 LDS bytes) for Q8_0, 3 (48) for Q4_0; the bytes past the pair are the next pair's (or
  // the allocation's tail slack) and are never read.  F16 rows move like a.
  constexpr int WROW = WCH ? 128 : (PAIR1 + 15) / 16 * 16, WCK = WROW / 16;  // LDS bytes, chunks per W row
  // A ring slot holds WK consecutive 64-wide k steps (sub-stages): the a tile's, then the W rows'.
  constexpr int A_ST0 = BM * 128, W_ST0 = BN * WROW;
  constexpr int A_ST = WK * A_ST0, W_ST = WK * W_ST0, ST = A_ST + W_ST;
  constexpr int CROW = BN + 8;                                           // f32 per epilogue LDS row
  // NSQ slots asked for, as many as fit in the 160 KiB of LDS.
  constexpr int NS = NSQ * ST + 16 <= 160 * 1024 ? NSQ : (160 * 1024 - 16) / ST;
  static_assert(NS >= 2, "at least two slots");
  static_assert(A_ST0 % 1024 == 0 && W_ST0 % 1024 == 0, "whole DMA instructions per sub-stage");
  constexpr int W_RG = NS * A_ST;                               // the W stages follow the a stages
  constexpr int NIA = A_ST / 1024;                              // a: 16-byte DMA instructions per stage
  constexpr int NIW = W_ST / 1024;                              // W: 16-byte DMA instructions per stage
  // The wavefronts that issue the DMA: all of them; in the ping-pong loop the a tile by all of them
  // and the W rows by the four of the second group.
  constexpr int NWA = NWT, NWI = PIPE == 2 ? 4 : NWT;
  // Instructions per wavefront and stage: PA / PW at most; the first NIA % NWI (NIW % NWI) wavefronts
  // take one more than the others.  vmcnt immediates count PI = the fewest a wavefront issues per stage:
  // loads complete in order, so waiting until at most m·PI remain waits for everything older than the
  // wavefront's last m stages (and at most a few of their instructions besides).
  constexpr int PA = (NIA + NWA - 1) / NWA, PW = (NIW + NWI - 1) / NWI, PI = NIA / NWA + NIW / NWI;
  static_assert((NS - 1) * PI < 64, "vmcnt holds the DMA of NS - 1 steps");
  // (+16: the odd block of the last W row reads one dword past its row, unused)
  constexpr int RING = NS * ST + 16;
  // Epilogue passes: PG of each wavefront's TM 32-row tiles at a time, the most that fit in the ring
  // (the whole tile when it fits).
  // (k groups: one plane of the pass per group)
  constexpr int PG = WK * BM * CROW * 4 <= RING ? TM
                     : (TM % 2 == 0 && WK * BM / 2 * CROW * 4 <= RING) ? TM / 2
                     : (TM % 4 == 0 && WK * BM / 4 * CROW * 4 <= RING) ? TM / 4 : 1;
  constexpr int CPL = WM * 32 * PG * CROW;  // floats of one plane of a pass
  constexpr int C_BYTES = WK * CPL * 4;
  constexpr int LDS_BYTES = RING > C_BYTES ? RING : C_BYTES;
  __shared__ __attribute__((aligned(16))) uint8_t lds[LDS_BYTES];

  if (P.skip && *P.skip == P.skip_val) return;  // c already holds this product
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // Tile order.  Workgroups go to the 8 XCDs round-robin by linear id, and each XCD has its own L2.
  // The grid is renumbered so that an XCD takes a contiguous run l of tiles of one k split, and the
  // run is ordered in groups of P.group row tiles, column by column inside a group: an XCD's tiles
  // then form a rectangle of row tiles x column tiles, whose rows of a and of w its L2 fetches once.
  // (P.group 1: a band of row tiles over all column tiles, which fetches the whole of w per XCD.)
  // (XCD x takes the linear ids ≡ x mod 8: total / 8 of them, one more for the first total % 8.)
  int tx = blockIdx.x, ty = blockIdx.y, tz = blockIdx.z;
  {
    const int nx = gridDim.x, ny = gridDim.y, total = nx * ny * gridDim.z;
    const int lin = tx + nx * (ty + ny * tz), x = lin % 8, l = x * (total / 8) + min(x, total % 8) + lin / 8;
    tz = l / (nx * ny);
    const int e = l % (nx * ny), g0 = e / (P.group * nx) * P.group, gh = min(P.group, ny - g0), w = e - g0 * nx;
    ty = g0 + w % gh;
    tx = w / gh;
  }
  const int n0 = tx * BN, m0 = ty * BM;
  // k group kg of the wavefront (it computes sub-stage kg of every slot) and its place wv in the group.
  const int kg = WK == 1 ? 0 : wave / NW, wv = WK == 1 ? wave : wave % NW;
  const int wm = (wv / WN) * (BM / WM), wn = (wv % WN) * (BN / WN);
  const int lrow = lane & 31, g = lane >> 5;
  const int m = P.m, k = P.k, rows = P.rows;
  // Slots of WK k steps: the split's range kb .. kb + nk − 1.
  const int nkt = k / (64 * WK), kb = nkt * tz / (int)gridDim.z, nk = nkt * (tz + 1) / (int)gridDim.z - kb;

  // Per-lane byte offsets of this wave's DMA instructions from the step's base addresses (rows past
  // m or rows are clamped: their products land in outputs that are discarded or zeroed), and the
  // instructions' LDS offsets in a stage.
  const int wi = PIPE == 2 ? wave % 4 : wave;  // the wavefront's index among the W-issuing ones
  uint32_t aoff[PA], alds[PA];
#pragma unroll
  for (int i = 0; i < PA; i++) {
    const int n = (wave + NWA * i) % NIA, sub = n / (A_ST0 / 1024), nn = n % (A_ST0 / 1024);
    const int r = 8 * nn + lane / 8, lc = ((lane % 8) - (r >> 1)) & 7;
    aoff[i] = (uint32_t)(((size_t)min(m0 + r, m - 1) * k + 8 * lc) * 2 + 128 * sub);
    alds[i] = 1024 * n;
  }
  uint32_t woff[PW], wlds[PW];
#pragma unroll
  for (int i = 0; i < PW; i++) {
    const int n = (wi + NWI * i) % NIW, sub = n / (W_ST0 / 1024), nn = n % (W_ST0 / 1024);
    if constexpr (WCH) {
      const int r = 8 * nn + lane / 8, lc = ((lane % 8) - (r >> 1)) & 7;
      woff[i] = (uint32_t)((size_t)min(n0 + r, rows - 1) * P.row_bytes + 16 * lc + PAIR1 * sub);
      wlds[i] = 1024 * n;
    } else {
      // (Q8_0: rows 16-31 of each 32-row block start 8 bytes into their LDS row, see read_w; a
      // clamped row 0 — a one-row W, never read — is not moved, as nothing precedes it)
      const int t = 64 * nn + lane, r = t / WCK, c = t % WCK, row = min(n0 + r, rows - 1);
      const int shift = WT == WH_Q8_0 && (r & 16) && row > 0 ? 8 : 0;
      woff[i] = (uint32_t)((size_t)row * P.row_bytes + 16 * c + PAIR1 * sub - shift);
      wlds[i] = 1024 * n;
    }
  }
  const uint8_t *abase = (const uint8_t *)P.a + (size_t)kb * 128 * WK;
  const uint8_t *wbase = P.w + (size_t)kb * PAIR1 * WK;
  const uint32_t lds0 = lds_addr(lds);
  auto issue_a = [&](int kt, int slot) {
    const uint8_t *ab = abase + (size_t)kt * 128 * WK;
#pragma unroll
    for (int i = 0; i < PA; i++)
      if (NIA % NWA == 0 || i < NIA / NWA || wave + NWA * i < NIA) dma16s(ab, aoff[i], lds0 + slot * A_ST + alds[i]);
  };
  auto issue_w = [&](int kt, int slot) {
    const uint8_t *wb = wbase + (size_t)kt * PAIR1 * WK;
#pragma unroll
    for (int i = 0; i < PW; i++)
      if (NIW % NWI == 0 || i < NIW / NWI || wi + NWI * i < NIW) dma16s(wb, woff[i], lds0 + W_RG + slot * W_ST + wlds[i]);
  };
  auto issue = [&](int kt, int slot) {
    issue_a(kt, slot);
    issue_w(kt, slot);
  };

  // The lane's k chunk (of 8 in a step) at substep s.  Q8_0: 2s + g — block s/2 of the pair at
  // every lane of a substep, so the bytes of a substep sit at the same place in every lane's dwords;
  // Q4_0 and F16: 4g + s — block g.  a and W fragments take the same chunk.
  constexpr bool Q8 = WT == WH_Q8_0;
  auto chunk = [&](int s) { return Q8 ? 2 * s + g : 4 * g + s; };
  // LDS read offsets of the lane: a chunk of row wm + lrow (+32i), rotated by row/2; the lane's W
  // dwords (Q8_0: from byte 8g of its row pair, the scales in dwords 0 and 8 of the row; Q4_0:
  // g = 0 reads dwords 0.. with the data from byte 2, g = 1 the dwords from byte BLK + 2 with the
  // scale in the high half of the dword before); F16 chunks like a.
  uint32_t a_off[4];
#pragma unroll
  for (int s = 0; s < 4; s++) a_off[s] = kg * A_ST0 + (wm + lrow) * 128 + 16 * ((chunk(s) + (lrow >> 1)) & 7);
  constexpr int ND = Q8 ? 10 : WT == WH_Q4_0 ? 5 : 16;  // dwords per lane per W row and step
  constexpr int NSC = Q8 ? 2 : 1;                       // scale dwords per lane per W row and step
  constexpr int BLK = PAIR1 / 2;
  const uint32_t w_row = W_RG + kg * W_ST0 + (wn + lrow) * WROW + (Q8 ? 8 * ((lrow >> 4) & 1) : 0);
  const uint32_t w_dat = Q8 ? w_row + 8 * g : w_row + (g ? BLK + 2 : 0), w_sc = w_row + (g ? BLK - 2 : 0);
  uint32_t wf_off[4];
#pragma unroll
  for (int s = 0; s < 4; s++) wf_off[s] = w_row + 16 * ((chunk(s) + (lrow >> 1)) & 7);

  auto read_a = [&](half8 (&f)[TM], int slot, int s) {
#pragma unroll
    for (int i = 0; i < TM; i++) f[i] = *(const half8 *)(lds + a_off[s] + slot * A_ST + i * 4096);
  };
  auto read_w = [&](uint32_t (&w)[TN][ND], uint32_t (&sc)[TN][NSC], int slot) {
#pragma unroll
    for (int j = 0; j < TN; j++) {
      if constexpr (WCH) {
#pragma unroll
        for (int s = 0; s < 4; s++) {
          const uint4 x = *(const uint4 *)(lds + wf_off[s] + slot * W_ST + j * 32 * WROW);
          w[j][4 * s] = x.x, w[j][4 * s + 1] = x.y, w[j][4 * s + 2] = x.z, w[j][4 * s + 3] = x.w;
        }
        sc[j][0] = 0;
      } else if constexpr (Q8) {
        // Pair bytes 2 + 8g .. (block 0, substeps 0-1: dwords 0-2 and 4-6 from byte 8g) and
        // 36 + 8g .. (block 1, substeps 2-3: dwords 9-10 and 13-14), read as the 16 dwords from byte
        // 8g in 8-byte reads: with 80-byte LDS rows, rows r and r + 16 of a 32-row block would share
        // banks, so rows 16-31 sit 8 bytes further into their LDS row (measured on gfx950: single
        // dwords from the rows as stored cost 6 bank-conflict cycles per read, 8-byte reads from the
        // moved rows none).  The scales at bytes 0 and 34: dword 0 of lane group 0's span (lanes
        // 32-63 take it from lane − 32) and dword 8 − 2g.
        const uint2 *q = (const uint2 *)(lds + w_dat + slot * W_ST + j * 32 * WROW);
        uint32_t d[16];
#pragma unroll
        for (int i = 0; i < 8; i++) {
          const uint2 v = q[i];
          d[2 * i] = v.x, d[2 * i + 1] = v.y;
        }
        constexpr int at[10] = {0, 1, 2, 4, 5, 6, 9, 10, 13, 14};
#pragma unroll
        for (int i = 0; i < 10; i++) w[j][i] = d[at[i]];
        uint32_t s0 = d[0], s0b = d[0];
        xlane::swap32(s0, s0b);  // lanes 32-63: lane − 32's dword 0
        sc[j][0] = s0, sc[j][1] = g ? d[6] : d[8];
      } else {
        const uint32_t *q = (const uint32_t *)(lds + w_dat + slot * W_ST + j * 32 * WROW);
#pragma unroll
        for (int i = 0; i < ND; i++) w[j][i] = q[i];
        sc[j][0] = *(const uint32_t *)(lds + w_sc + slot * W_ST + j * 32 * WROW);
      }
    }
  };

  floatx16 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; i++)
#pragma unroll
    for (int j = 0; j < TN; j++) acc[i][j] = floatx16{};
  const uint32_t sh = g ? 0u : 2u;
  // The MFMA operand of W column block j at substep s: f16 chunks as read (F16), or the lane's
  // quantized dwords dequantized (f16(q·d)).
  auto wfrag = [&](const uint32_t (&w)[TN][ND], const uint32_t (&scl)[TN][NSC], int j, auto s_c) -> half8 {
    constexpr int s = decltype(s_c)::value;
    if constexpr (WCH) return __builtin_bit_cast(half8, make_uint4(w[j][4 * s], w[j][4 * s + 1], w[j][4 * s + 2], w[j][4 * s + 3]));
    else if constexpr (Q8) {
      const half2 sv = __builtin_bit_cast(half2, scl[j][s >> 1]);  // block 0: low half; block 1: high
      const _Float16 d = s < 2 ? sv[0] : sv[1];
      return dequant_q8<s>(w[j], half2{d, d});
    } else {
      const _Float16 d = __builtin_bit_cast(_Float16, (uint16_t)(g ? scl[j][0] >> 16 : scl[j][0] & 0xffffu));
      return dequant_frag<WT>(w[j], sh, half2{d, d}, s);
    }
  };
  if constexpr (PIPE == 2) {
    // Ping-pong.  Two groups of four wavefronts (group 1 = waves 4-7; a workgroup's wavefronts go to
    // the SIMDs round-robin, so every SIMD holds one of each) take turns, offset by half a step: while
    // one group runs the 4·TM·TN MFMAs of a k step from registers (its a fragments read one substep
    // ahead), the other group reads and dequantizes its W fragments of its next step.  So the
    // dequantization's VALU runs beside the other group's MFMAs on every SIMD.  One barrier per half
    // step; group 1 starts one barrier later.  Stage i is read by group 0 between barriers 2i + 1 and
    // 2i + 3 and by group 1 between 2i + 2 and 2i + 4, so its slot refills after barrier 2i + 4 with
    // stage i + NS: the a tile by all eight wavefronts during their MFMAs of step i + 1 (one DMA
    // instruction after the first MFMA of each substep), the W rows by group 1 during its
    // dequantization of step i + 1.  Stage i + 1 must land by barrier 2i + 3: group 0 waits for its part
    // at the end of its MFMAs of step i, group 1 at the end of its dequantization of step i.
    static_assert(WM == 2 && WN == 4 && NS >= 3, "two groups of four wavefronts, three or more slots");
    static_assert(NIA % NW == 0 && NIA / NW <= 4, "at most one a-tile DMA instruction per wavefront and substep");
    const bool g1 = wave >= 4;
    constexpr int QA = NIA / NW, QW = NIW / 4;  // DMA instructions per wavefront and stage (W: the fewest)
    uint32_t wq[TN][ND], sc[TN][NSC];
    half8 af[2][TM], wf[4][TN];
    // The MFMAs of substep s; a-tile DMA instruction s of stage kd (if any) after the first.
    auto mm = [&](const half8 (&f)[TM], const half8 (&b)[TN], const uint8_t *ab, int slot_d, auto s_c) {
      constexpr int SS = decltype(s_c)::value;
#pragma unroll
      for (int j = 0; j < TN; j++)
#pragma unroll
        for (int i = 0; i < TM; i++) {
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(f[i], b[j], acc[i][j], 0, 0, 0);
          if constexpr (SS < QA)
            if (i == 0 && j == 0) dma16s(ab, aoff[SS], lds0 + slot_d * A_ST + alds[SS]);
        }
    };
    // Prologue: stages 0 .. NS − 2, the a tiles by all, the W rows by group 1.
#pragma unroll
    for (int s = 0; s < NS - 1; s++)
      if (s < nk) {
        issue_a(s, s);
        if (g1) issue_w(s, s);
      }
    if (nk >= NS - 1) {  // stage 0 has landed
      if (g1) wait_vm<(NS - 2) * (QA + QW)>();
      else wait_vm<(NS - 2) * QA>();
    } else {
      dma_wait();
    }
    __syncthreads();
    if (g1) __syncthreads();
    auto step = [&](auto S_c, int kt) {
      constexpr int S = decltype(S_c)::value, slot = S % NS, dslot = (S + NS - 1) % NS;
      const bool more = kt + NS - 1 < nk;  // stage kt + NS − 1 exists (into the slot of step kt − 1)
      // Preparation of step kt.
      read_w(wq, sc, slot);
      static_for<0, 4, 1>([&](auto s_c) {
#pragma unroll
        for (int j = 0; j < TN; j++) wf[decltype(s_c)::value][j] = wfrag(wq, sc, j, s_c);
      });
      read_a(af[0], slot, 0);
      // The fragments exist in registers here (kept from being recomputed inside the MFMA phase).
#pragma unroll
      for (int s = 0; s < 4; s++)
#pragma unroll
        for (int j = 0; j < TN; j++) asm volatile("" : "+v"(wf[s][j]));
      if (g1) {
        if (more) issue_w(kt + NS - 1, dslot);
        // Group 1's a-tile part of stage kt + 1 (issued in its MFMAs of step kt − 1) and W rows of it
        // have landed: only the W rows just issued may remain.
        if (kt + 1 < nk) {
          if (more) wait_vm<QW>();
          else dma_wait();
        }
      }
      __syncthreads();
      __builtin_amdgcn_sched_barrier(0);
      // The MFMAs of step kt, with this wavefront's a-tile DMA of stage kt + NS − 1; each substep's a
      // fragments read before the previous substep's MFMAs.
      // (After the last stage, the last one again: into the slot of step kt − 1, which nothing reads
      // any more, so that every step issues the same instructions with no branch between MFMAs.)
      const uint8_t *ab = abase + (size_t)(uint32_t)__builtin_amdgcn_readfirstlane(more ? kt + NS - 1 : nk - 1) * 128;
      read_a(af[1], slot, 1);
      mm(af[0], wf[0], ab, dslot, std::integral_constant<int, 0>{});
      read_a(af[0], slot, 2);
      mm(af[1], wf[1], ab, dslot, std::integral_constant<int, 1>{});
      read_a(af[1], slot, 3);
      mm(af[0], wf[2], ab, dslot, std::integral_constant<int, 2>{});
      mm(af[1], wf[3], ab, dslot, std::integral_constant<int, 3>{});
      if (!g1 && kt + 1 < nk) wait_vm<QA>();  // group 0's part of stage kt + 1 has landed (this step's may remain)
      __builtin_amdgcn_sched_barrier(0);
      if (!g1 || kt + 1 < nk) __syncthreads();
    };
    constexpr int UNR = NS;
    for (int kt0 = 0; kt0 < nk; kt0 += UNR) unrolled_steps<0, UNR>(step, kt0, nk);
    dma_wait();  // the repeated stages of the last steps, before the epilogue reuses the LDS
  } else {
#pragma unroll
    for (int s = 0; s < NS; s++)
      if (s < nk) issue(s, s);
    uint32_t wq[2][TN][ND], sc[2][TN][NSC];
    half8 af[2][TM];
    // Substep s of a step: dequantize the lane's W fragment (quantized) and run the TM × TN MFMAs.
    auto mma = [&](const half8 (&f)[TM], const uint32_t (&w)[TN][ND], const uint32_t (&scl)[TN][NSC], auto s_c) {
#pragma unroll
      for (int j = 0; j < TN; j++) {
        const half8 b = wfrag(w, scl, j, s_c);
#pragma unroll
        for (int i = 0; i < TM; i++) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(f[i], b, acc[i][j], 0, 0, 0);
      }
    };
    if (nk > 0) {
      if (nk >= NS) wait_vm<(NS - 1) * PI>();  // stages 1 .. NS - 1 may be in flight
      else dma_wait();
      __syncthreads();
      read_w(wq[0], sc[0], 0);
      read_a(af[0], 0, 0);
    }
    // Step kt (S = kt modulo the unroll: ring slot S % NS, register set S % 2).
    auto step = [&](auto S_c, int kt) {
      constexpr int S = decltype(S_c)::value, slot = S % NS, cur = S & 1;
      read_a(af[1], slot, 1);
      mma(af[0], wq[cur], sc[cur], std::integral_constant<int, 0>{});
      read_a(af[0], slot, 2);
      mma(af[1], wq[cur], sc[cur], std::integral_constant<int, 1>{});
      read_a(af[1], slot, 3);
      mma(af[0], wq[cur], sc[cur], std::integral_constant<int, 2>{});
      if (kt + 1 < nk) {
        // Stage kt + 1 has landed for every wave, and every wave is done reading slot kt.
        if (kt + NS - 1 < nk) wait_vm<(NS - 2) * PI>();  // stages kt + 2 .. kt + NS - 1 may be in flight
        else dma_wait();
        __syncthreads();
        if (kt + NS < nk) issue(kt + NS, slot);  // into the slot this step has finished reading
        read_w(wq[cur ^ 1], sc[cur ^ 1], (slot + 1) % NS);
        read_a(af[0], (slot + 1) % NS, 0);
      }
      mma(af[1], wq[cur], sc[cur], std::integral_constant<int, 3>{});
    };
    constexpr int UNR = NS % 2 ? 2 * NS : NS;
    for (int kt0 = 0; kt0 < nk; kt0 += UNR) unrolled_steps<0, UNR>(step, kt0, nk);
  }

  // Epilogue through LDS: every DMA has landed (the last step waited for it) and the barrier below
  // ends every wavefront's reads of the stages.  A thread's 8-column group is the same on every row
  // it stores (64·NW is a multiple of BN / 8), so its bias values are loaded once, before the barrier.
  constexpr int G8 = BN / 8;  // 8-column groups per row
  static_assert((64 * NWT) % G8 == 0, "fixed column group per thread");
  const int ecol = n0 + 8 * (epi_lane<BN>(tid) % G8);
  float bb[8] = {}, bd[8] = {};
  if (!SPLIT && ecol < P.cols) {
    const float4 b0 = *(const float4 *)(P.bias + ecol), b1 = *(const float4 *)(P.bias + ecol + 4);
    bb[0] = b0.x, bb[1] = b0.y, bb[2] = b0.z, bb[3] = b0.w, bb[4] = b1.x, bb[5] = b1.y, bb[6] = b1.z, bb[7] = b1.w;
#pragma unroll
    for (int q = 0; q < 8; q++)
      if (ecol + q < P.dual) bd[q] = P.bias[P.cols + ecol + q];
  }
  float *cl = (float *)lds;
  // Pass i0: 32-row tiles i0 .. i0 + PG − 1 of every wavefront; LDS row (wave row)·32·PG + 32·(i − i0)
  // + the row in the MFMA tile.
  const int crow0 = (wv / WN) * 32 * PG;
  // A tile of a transposed packed range (Vᵀ, flattened image rows) is staged column by column, CCOL
  // floats per column (its 4-row runs written 16 bytes at a time; the padding spreads a 16-lane pass
  // over every bank), when that fits in a plane.
  constexpr int NRP = WM * 32 * PG, CCOL = NRP + 4;
  constexpr bool TCM = OUT16 && !SPLIT && BN * CCOL <= CPL;
  bool trt = false;
  if constexpr (TCM) {
#pragma unroll
    for (int o = 0; o < 2; o++)
      if (o < P.nho && P.ho[o].tr && n0 >= P.ho[o].col0 && n0 < P.ho[o].col0 + P.ho[o].cols) trt = true;
  }
  // (passes unrolled at compile time, so that the accumulators are only ever indexed by constants)
  auto pass = [&](auto I0_c) {
    constexpr int i0 = decltype(I0_c)::value;
    __syncthreads();
    // Each k group stores its sums in a plane of its own, both at once; the stores below add group
    // 0's and group 1's (a fixed order of the two halves' sums).
    float *mine = cl + kg * CPL;
    if (TCM && trt) {
#pragma unroll
      for (int i = i0; i < i0 + PG; i++)
#pragma unroll
        for (int j = 0; j < TN; j++)
#pragma unroll
          for (int v4 = 0; v4 < 4; v4++)
            *(float4 *)(mine + (wn + 32 * j + lrow) * CCOL + crow0 + 32 * (i - i0) + 8 * v4 + 4 * g) =
                make_float4(acc[i][j][4 * v4], acc[i][j][4 * v4 + 1], acc[i][j][4 * v4 + 2], acc[i][j][4 * v4 + 3]);
    } else {
#pragma unroll
      for (int i = i0; i < i0 + PG; i++)
#pragma unroll
        for (int j = 0; j < TN; j++)
#pragma unroll
          for (int v = 0; v < 16; v++)
            mine[(crow0 + 32 * (i - i0) + 8 * (v >> 2) + 4 * g + (v & 3)) * CROW + wn + 32 * j + lrow] = acc[i][j][v];
    }
    __syncthreads();
    store_c_tile<WM * 32 * PG, BM / WM, 32 * PG, BN, 64 * NWT, SPLIT, OUT16, (WK > 1)>(
        P, cl, CROW, tid, m0, n0, tz, i0, bb, bd, cl + CPL, TCM && trt ? CCOL : 0);
  };
  static_for<0, TM, PG>(pass);
}

// Split-k finish: c = epi(Σ_z part[z] + bias) with the partial sums added in split order (the same
// result on every run), dual outputs and padding columns as in the kernel above.
template <bool OUT16>
__global__ __launch_bounds__(256) void split_finish_kernel(const float *__restrict__ part, int splits, const float *__restrict__ bias,
                                                           void *__restrict__ c, int m, int rows, int cols, int dual,
                                                           int ldc, int epi, float alpha) {
  const size_t n = (size_t)m * cols, plane = n;
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) {
    const int row = (int)(i / cols), col = (int)(i % cols);
    float x = 0.0f;
    for (int z = 0; z < splits; z++) x += part[z * plane + i];
    if (col >= rows) x = 0.0f;
    const size_t at = (size_t)row * ldc + col;
    if constexpr (OUT16) {
      _Float16 *cp = (_Float16 *)c + at;
      *cp = (_Float16)epilogue(epi, alpha, x + bias[col], nullptr);
      if (col < dual) cp[cols] = (_Float16)(x + bias[cols + col]);
    } else {
      float *cp = (float *)c + at;
      *cp = epilogue(epi, alpha, x + bias[col], cp);
      if (col < dual) cp[cols] = x + bias[cols + col];
    }
  }
}

template <int WT, int BM, int BN, int WM, int WN, int NS, int PIPE, int WK>
int lds_launch(wh_ctx *ctx, dim3 grid, const LdsArgs &a, bool split, bool out16) {
  constexpr int WROW = WT == WH_Q8_0 ? 80 : WT == WH_Q4_0 ? 48 : 128;  // LDS bytes per W row (the kernel's)
  if constexpr (PIPE == 2 && (WT == WH_F16 || NS * (BM * 128 + BN * WROW) + 16 > 160 * 1024)) {
    // (not built: the ring would exceed the LDS, or F16 rows, which need no dequantization to hide)
    return wh_fail(ctx, WH_EARG, "gemm: no ping-pong kernel for %d slots of a %dx%d tile of this weight type", NS, BM, BN);
  } else {
    constexpr int NT = 64 * WM * WN * WK;
    if (split) wh_launch(ctx, gemm_lds_kernel<WT, BM, BN, WM, WN, NS, true, false, PIPE, WK>, grid, NT, 0, a);
    else if (out16) wh_launch(ctx, gemm_lds_kernel<WT, BM, BN, WM, WN, NS, false, true, PIPE, WK>, grid, NT, 0, a);
    else wh_launch(ctx, gemm_lds_kernel<WT, BM, BN, WM, WN, NS, false, false, PIPE, WK>, grid, NT, 0, a);
    return WH_OK;
  }
}

template <int WT>
int launch_lds_t(wh_ctx *ctx, const _Float16 *a, const wh_linear *l, void *c, int m, int ldc, int epi, float alpha,
                 bool out16, float *part, int *splits, const HeadsOut *ho, int nho) {
  GemmPlan p = gemm_plan_for(ctx, m, l->cols, l->k);
  if ((p.split > 1 && !part) || nho) p.split = 1;  // packed ranges are written by the tiles' own epilogue
  if (splits) *splits = p.split;
  LdsArgs args{a, l->w, l->bias, p.split > 1 ? (void *)part : c, m, l->rows, l->cols, l->k, l->dual, ldc, epi, alpha,
               l->row_bytes, {}, nho, nullptr, 0, 1};
  // A tagged output (ctx->gemm_skip, set by the caller for this launch): whole-k plans only (a split
  // launch's partial sums are finished by another kernel).
  if (ctx->gemm_skip && p.split == 1) args.skip = ctx->gemm_skip, args.skip_val = ctx->gemm_skip_val;
  if (nho < 0 || nho > 2) return wh_fail(ctx, WH_EARG, "gemm: %d packed ranges", nho);
  for (int i = 0; i < nho; i++) {
    const HeadsOut &h = ho[i];
    // Whole tiles, inside the real columns, no dual columns; 16-byte stores.
    if (!out16 || h.col0 % p.bn || h.cols % p.bn || h.col0 + h.cols > l->rows || h.col0 < l->dual || h.hd % 8 ||
        h.cols % h.hd || (uintptr_t)h.dst % 16 || h.r0 < 0 || (h.tr ? h.r0 || h.rs % 8 || h.rs < m : h.rs < h.r0 + m) ||
        h.blk < 0 || (h.blk && (!h.tr || h.blk % 8 || h.hd != h.cols)))
      return wh_fail(ctx, WH_EARG, "gemm: packed output %d off the %d-column tiles or its layout", i, p.bn);
    args.ho[i] = h;
  }
  dim3 grid((l->cols + p.bn - 1) / p.bn, (m + p.bm - 1) / p.bm, p.split);
  // Tile order: k-group plans under 1024 rows (few tiles per CU, w from HBM) in groups of 2 row
  // tiles, the others row by row (Parakeet 60 s in-step: the 750x4096x1024 up projections 15.5 ->
  // 14.8 us, while the 64x64 qkv projection, a single k group, slows with every group size above 1;
  // Whisper's 1500x1280x1280 k-group projection takes 17.5 us in groups of 2, 15.0 row by row).
  const int group = ctx->gemm_group ? ctx->gemm_group : p.wk > 1 && m < 1024 ? 2 : 1;
  args.group = std::max(1, std::min(group, (int)grid.y));
  static const char *tn = WT == WH_F16 ? "f16" : WT == WH_Q8_0 ? "q8_0" : "q4_0";
  // Named by kernel variant and call shape: m x rows x k, epilogue, output type, row width.
  char name[128];
  char sp[24] = "";
  if (p.split > 1) snprintf(sp, sizeof sp, "_s%d", p.split);
  if (p.pipe) snprintf(sp + strlen(sp), sizeof sp - strlen(sp), "_p%d", p.pipe);
  if (p.wk > 1) snprintf(sp + strlen(sp), sizeof sp - strlen(sp), "_k%d", p.wk);
  snprintf(name, sizeof name, "gemm_%s_%dx%d_w%dx%d_n%d%s %dx%dx%d e%d %s w%d%s", tn, p.bm, p.bn, p.wm, p.wn, p.ns, sp,
           m, l->rows, l->k, epi, out16 ? "f16" : "f32", l->cols + l->dual, args.skip ? " (tagged)" : "");
  const double width = epi == EPI_GLU ? l->cols / 2 : l->cols + l->dual;
  const double bytes = (double)l->rows * l->row_bytes + 2.0 * m * l->k +
                       (out16 ? 2.0 : 4.0) * m * width * (epi == WH_RESIDUAL || epi == WH_GELU_RESIDUAL ? 2 : 1);
  {
    // (a tagged launch is profiled as no work: it skips whenever its tag matches)
    ProfScope prof(ctx, name, args.skip ? 0.0 : 2.0 * m * l->rows * l->k, args.skip ? 0.0 : bytes);
    const bool sp = p.split > 1;
    bool ok = false;
#define PLANK(BM, BN, WM, WN, NS, PIPE, WK)                                                                       \
  if (!ok && p.bm == BM && p.bn == BN && p.wm == WM && p.wn == WN && p.ns == NS && p.pipe == PIPE && p.wk == WK) { \
    if (int rc = lds_launch<WT, BM, BN, WM, WN, NS, PIPE, WK>(ctx, grid, args, sp, out16)) return rc;               \
    ok = true;                                                                                                      \
  }
#define PLANP(BM, BN, WM, WN, NS, PIPE) PLANK(BM, BN, WM, WN, NS, PIPE, 1)
#define PLAN(BM, BN, WM, WN, NS) PLANK(BM, BN, WM, WN, NS, 0, 1)
    PLAN(128, 128, 2, 4, 3)
    PLAN(64, 64, 2, 2, 3)
    PLAN(128, 128, 2, 4, 2)
    PLAN(128, 128, 2, 2, 2)
    PLAN(256, 128, 4, 2, 2)
    PLAN(96, 64, 1, 2, 2)
    PLAN(192, 128, 2, 2, 2)
    PLAN(256, 256, 2, 4, 2)
    PLAN(96, 128, 1, 4, 3)
    PLANK(64, 64, 2, 2, 4, 0, 2)
    PLANK(96, 64, 1, 2, 2, 0, 2)
    PLANK(96, 128, 1, 4, 3, 0, 2)
    PLANP(256, 256, 2, 4, 3, 2)  // the ping-pong loop (tuning only: not faster than the plain one)
#undef PLAN
#undef PLANP
#undef PLANK
    if (!ok)
      return wh_fail(ctx, WH_EARG, "gemm: no kernel for tile %dx%d, %dx%d waves, %d stages, %d k groups", p.bm, p.bn,
                     p.wm, p.wn, p.ns, p.wk);
    if (int rc = wh_launched(ctx, "gemm")) return rc;
  }
  if (p.split > 1 && !splits && !ctx->gemm_kernel_only) {
    ProfScope prof(ctx, "gemm_split_finish", 0.0, 4.0 * p.split * m * l->cols + 4.0 * m * width);
    const size_t n = (size_t)m * l->cols;
    const int blocks = (int)std::min<size_t>((n + 255) / 256, 8192);
    if (out16)
      wh_launch(ctx, split_finish_kernel<true>, blocks, 256, 0, part, p.split, l->bias, c, m, l->rows, l->cols, l->dual, ldc, epi, alpha);
    else
      wh_launch(ctx, split_finish_kernel<false>, blocks, 256, 0, part, p.split, l->bias, c, m, l->rows, l->cols, l->dual, ldc, epi, alpha);
    return wh_launched(ctx, "gemm split finish");
  }
  return WH_OK;
}

}  // namespace

// The LDS-DMA GEMM for one weight type (gemm_lds_<type>.hip); arguments as launch_lds in gemm.hip.
int gemm_lds_q8_0(wh_ctx *ctx, const _Float16 *a, const wh_linear *l, void *c, int m, int ldc, int epi, float alpha,
                bool out16, float *part, int *splits, const HeadsOut *ho, int nho);
int gemm_lds_q4_0(wh_ctx *ctx, const _Float16 *a, const wh_linear *l, void *c, int m, int ldc, int epi, float alpha,
                bool out16, float *part, int *splits, const HeadsOut *ho, int nho);
int gemm_lds_f16(wh_ctx *ctx, const _Float16 *a, const wh_linear *l, void *c, int m, int ldc, int epi, float alpha,
                bool out16, float *part, int *splits, const HeadsOut *ho, int nho);
