// The log-mel frontends on the device (src/fft.rs, src/parakeet/frontend.rs, src/gigaam/frontend.rs,
// src/whisper/frontend.rs), so that audio goes to the device once and the encoder reads its features
// where they are made.  The reference runs them on the CPU.
//
// One workgroup per frame: the frame's samples (padding, pre-emphasis, window) in the transform's
// input order, the leaves' naive DFTs and the radix-2 stages in LDS with the reference's operations
// in its order (src/fft.rs:106-148: every mul_add an fma, the same cos/sin tables, computed on the
// host), then the power spectrum and each filter's sum as the family defines it, and the logarithm.
// This file is built with -ffp-contract=off: a product and a sum the reference rounds separately stay
// separate, and fma() is written where the reference fuses.  A second kernel normalizes Parakeet's
// bins over the frames (f64 sums; their order differs from the reference's sequential sums, a
// difference far below the f32 result's rounding) or applies Whisper's global clamp and scale.
#include <algorithm>
#include <cfloat>

#include "internal.h"

namespace {

// Parakeet's padded, pre-emphasized sample q of frame t (src/parakeet/frontend.rs:80-87).
__device__ __forceinline__ double parakeet_sample(const float *pcm, int samples, long q) {
  q -= 256;  // N_FFT / 2 zeros before the audio
  if (q < 0) return 0.0;
  if (q == 0) return (double)pcm[0];
  if (q < samples) return (double)pcm[q] - (double)0.97f * (double)pcm[q - 1];
  return 0.0;
}

// Whisper's reflect-padded sample p (src/whisper/frontend.rs:47-54): the audio zero-padded to len,
// then 200 samples of reflection on each side.
__device__ __forceinline__ float whisper_sample(const float *pcm, int samples, int len, long p) {
  const int pad = 200;
  long q;
  if (p < pad) q = pad - p;
  else if (p < pad + len) q = p - pad;
  else q = len - 2 - (p - pad - len);
  return q < samples ? pcm[q] : 0.0f;
}

// ln of an f32, rounded once from the f64 logarithm: the correctly rounded value except in the rare
// double-rounding case, which is what the C library's logf returns nearly always.
__device__ __forceinline__ float log_f32(float x) { return (float)log((double)x); }

template <typename T>
__device__ __forceinline__ T fma_t(T a, T b, T c);
template <>
__device__ __forceinline__ double fma_t<double>(double a, double b, double c) {
  return fma(a, b, c);
}
template <>
__device__ __forceinline__ float fma_t<float>(float a, float b, float c) {
  return fmaf(a, b, c);
}

// One frame per workgroup of 256 threads.  KIND: 0 Parakeet (T = double), 1 GigaAM, 2 Whisper (float).
template <typename T, int KIND>
__global__ __launch_bounds__(256) void mel_kernel(MelArgs a) {
  constexpr int N = KIND == 0 ? 512 : KIND == 1 ? 320 : 400;
  constexpr int BINS = N / 2 + 1;
  __shared__ T bufa[2 * N], bufb[2 * N];
  __shared__ T xs[N];
  __shared__ double pw[BINS];
  const int t = blockIdx.x, tid = threadIdx.x;
  const T *tw_c = (const T *)a.tw_cos, *tw_s = (const T *)a.tw_sin;
  const T *lc = (const T *)a.leaf_cos, *ls = (const T *)a.leaf_sin;
  const T *win = (const T *)a.window;

  // The frame in the transform's input order: xs[j] = x[perm[j]].
  int nonzero = 0;
  for (int j = tid; j < N; j += 256) {
    const int i = a.perm[j];
    T s;
    if constexpr (KIND == 0) s = (T)parakeet_sample(a.pcm, a.samples, (long)t * a.hop + i);
    else if constexpr (KIND == 1) s = (T)a.pcm[(long)t * a.hop + i];
    else s = (T)whisper_sample(a.pcm, a.samples, a.len, (long)t * a.hop + i);
    nonzero |= s != (T)0;
    xs[j] = s * win[i];
  }
  if constexpr (KIND == 2) {
    // A frame of zeros is the same constant (src/whisper/frontend.rs:62-68).
    if (!__syncthreads_or(nonzero)) {
      for (int m = tid; m < a.mels; m += 256) a.out[(size_t)t * a.mels + m] = a.raw ? 0.0f : a.silent;
      return;
    }
  } else {
    __syncthreads();
  }

  // The leaves: naive DFTs of the odd factor (src/fft.rs:106-122), output o = k·blocks + g.
  const int leaf = a.leaf, blocks = N / leaf;
  for (int o = tid; o < N; o += 256) {
    const int k = o / blocks, g = o - k * blocks;
    T re = xs[g], im = (T)0;
    for (int j = 1; j < leaf; j++) {
      const T c = lc[j * leaf + k], s = ls[j * leaf + k], v = xs[j * blocks + g];
      re = fma_t<T>(v, c, re);
      im = fma_t<T>(-v, s, im);
    }
    bufa[o] = re;
    bufa[N + o] = im;
  }
  __syncthreads();

  // The radix-2 stages (src/fft.rs:140-148).
  T *src = bufa, *dst = bufb;
  constexpr int HALF = N / 2;
  for (int st = 0; st < a.stages; st++) {
    for (int i = tid; i < HALF; i += 256) {
      const T c = tw_c[st * HALF + i], s = tw_s[st * HALF + i];
      const T av = src[2 * i], x = src[2 * i + 1], b = src[N + 2 * i], y = src[N + 2 * i + 1];
      dst[i] = fma_t<T>(s, y, fma_t<T>(c, x, av));
      dst[N + i] = fma_t<T>(-s, x, fma_t<T>(c, y, b));
      dst[i + HALF] = fma_t<T>(-s, y, fma_t<T>(-c, x, av));
      dst[N + i + HALF] = fma_t<T>(s, x, fma_t<T>(-c, y, b));
    }
    __syncthreads();
    T *tmp = src;
    src = dst, dst = tmp;
  }

  // The power spectrum as each family rounds it.
  for (int k = tid; k < BINS; k += 256) {
    const T re = src[k], im = src[N + k];
    if constexpr (KIND == 0) pw[k] = (double)(float)(re * re + im * im);   // f64, then f32
    else if constexpr (KIND == 1) pw[k] = (double)(re * re + im * im);     // f32, unfused
    else pw[k] = (double)fmaf(re, re, im * im);                            // f32 fma, then f64
  }
  __syncthreads();

  for (int m = tid; m < a.mels; m += 256) {
    const float *f = a.filters + (size_t)m * BINS;
    const int lo = a.span[2 * m], hi = a.span[2 * m + 1];
    float v;
    if constexpr (KIND == 0) {
      // Each filter as a chain of f32 fused multiply-adds in bin order (src/parakeet/frontend.rs:99-104).
      float e = 0.0f;
      for (int k = lo; k < hi; k++) e = fmaf(f[k], (float)pw[k], e);
      v = a.raw ? e : log_f32(e + 1.0f / 16777216.0f);
    } else if constexpr (KIND == 1) {
      // dot over the span (src/cpu/mod.rs:20-43): 16 lanes of fmas, summed pairwise, then the tail.
      float acc[16];
#pragma unroll
      for (int l = 0; l < 16; l++) acc[l] = 0.0f;
      const int n = hi - lo, n16 = n / 16 * 16;
      for (int i = 0; i < n16; i += 16)
#pragma unroll
        for (int l = 0; l < 16; l++) acc[l] = fmaf(f[lo + i + l], (float)pw[lo + i + l], acc[l]);
#pragma unroll
      for (int w = 8; w >= 1; w >>= 1)
#pragma unroll
        for (int l = 0; l < w; l++) acc[l] += acc[l + w];
      float tail = 0.0f;
      for (int i = n16; i < n; i++) tail += f[lo + i] * (float)pw[lo + i];
      float e = acc[0] + tail;
      if (a.raw) {
        v = e;
      } else {
        e = e < 1e-9f ? 1e-9f : e > 1e9f ? 1e9f : e;
        v = log_f32(e);
      }
    } else {
      // f64 sums in groups of 4 bins and the last bin alone (src/whisper/frontend.rs:88-105).
      double sum = 0.0;
      for (int g = lo; g < hi; g++) {
        const int k = 4 * g;
        sum += (((double)f[k] * pw[k] + (double)f[k + 1] * pw[k + 1]) + (double)f[k + 2] * pw[k + 2]) +
               (double)f[k + 3] * pw[k + 3];
      }
      sum += (double)f[BINS - 1] * pw[BINS - 1];
      v = a.raw ? (float)sum : (float)log10(sum > 1e-10 ? sum : 1e-10);
    }
    a.out[(size_t)t * a.mels + m] = v;
  }
}

// Parakeet's normalization of bin m over all frames but the last (src/parakeet/frontend.rs:58-70):
// one workgroup per bin; the last frame is zero.
__global__ __launch_bounds__(256) void mel_normalize_kernel(float *__restrict__ mel, int frames, int mels) {
  __shared__ double part[256];
  const int m = blockIdx.x, tid = threadIdx.x, n = frames - 1;
  double s = 0.0;
  for (int t = tid; t < n; t += 256) s += (double)mel[(size_t)t * mels + m];
  part[tid] = s;
  __syncthreads();
  for (int o = 128; o > 0; o >>= 1) {
    if (tid < o) part[tid] += part[tid + o];
    __syncthreads();
  }
  const double mean = part[0] / (double)n;
  __syncthreads();
  s = 0.0;
  for (int t = tid; t < n; t += 256) {
    const double d = (double)mel[(size_t)t * mels + m] - mean;
    s += d * d;
  }
  part[tid] = s;
  __syncthreads();
  for (int o = 128; o > 0; o >>= 1) {
    if (tid < o) part[tid] += part[tid + o];
    __syncthreads();
  }
  const double inv = 1.0 / (sqrt(part[0] / (double)(n - 1)) + (double)1e-5f);
  for (int t = tid; t < n; t += 256) {
    float *p = mel + (size_t)t * mels + m;
    *p = (float)(((double)*p - mean) * inv);
  }
  if (tid == 0) mel[(size_t)n * mels + m] = 0.0f;
}

// Whisper: the maximum over every value (one workgroup), then (max(v, max − 8) + 4) / 4 in f64
// (src/whisper/frontend.rs:80-84).
__global__ __launch_bounds__(1024) void mel_max_kernel(const float *__restrict__ mel, size_t n, float *__restrict__ mx) {
  __shared__ float part[1024];
  float v = -INFINITY;
  for (size_t i = threadIdx.x; i < n; i += 1024) v = fmaxf(v, mel[i]);
  part[threadIdx.x] = v;
  __syncthreads();
  for (int o = 512; o > 0; o >>= 1) {
    if ((int)threadIdx.x < o) part[threadIdx.x] = fmaxf(part[threadIdx.x], part[threadIdx.x + o]);
    __syncthreads();
  }
  if (threadIdx.x == 0) *mx = part[0];
}

__global__ __launch_bounds__(256) void mel_scale_kernel(float *__restrict__ mel, size_t n, const float *__restrict__ mx) {
  const double top = (double)*mx - 8.0;
  for (size_t i = blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) {
    double v = (double)mel[i];
    v = v > top ? v : top;
    mel[i] = (float)((v + 4.0) / 4.0);
  }
}

}  // namespace

int launch_mel(wh_ctx *ctx, const MelArgs &a, int kind, int frames, float *scratch) {
  if (frames <= 0 || !a.pcm || !a.out || a.mels <= 0) return wh_fail(ctx, WH_EARG, "mel: bad arguments");
  {
    ProfScope prof(ctx, kind == 0 ? "mel_parakeet" : kind == 1 ? "mel_gigaam" : "mel_whisper", 0.0,
                   4.0 * ((double)frames * a.hop + (double)frames * a.mels));
    switch (kind) {
      case 0: wh_launch(ctx, mel_kernel<double, 0>, frames, 256, 0, a); break;
      case 1: wh_launch(ctx, mel_kernel<float, 1>, frames, 256, 0, a); break;
      default: wh_launch(ctx, mel_kernel<float, 2>, frames, 256, 0, a); break;
    }
    if (int rc = wh_launched(ctx, "mel")) return rc;
  }
  const size_t n = (size_t)frames * a.mels;
  if (a.raw) return WH_OK;
  if (kind == 0) {
    ProfScope prof(ctx, "mel_normalize", 0.0, 12.0 * n);
    wh_launch(ctx, mel_normalize_kernel, a.mels, 256, 0, a.out, frames, a.mels);
    return wh_launched(ctx, "mel normalize");
  }
  if (kind == 2) {
    if (!scratch) return wh_fail(ctx, WH_EARG, "mel: no scratch for the maximum");
    {
      ProfScope prof(ctx, "mel_max", 0.0, 4.0 * n);
      wh_launch(ctx, mel_max_kernel, 1, 1024, 0, (const float *)a.out, n, scratch);
      if (int rc = wh_launched(ctx, "mel max")) return rc;
    }
    ProfScope prof(ctx, "mel_scale", 0.0, 8.0 * n);
    const int blocks = (int)std::min<size_t>((n + 255) / 256, 4096);
    wh_launch(ctx, mel_scale_kernel, blocks, 256, 0, a.out, n, (const float *)scratch);
    return wh_launched(ctx, "mel scale");
  }
  return WH_OK;
}
