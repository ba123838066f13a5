/*
 * Op-level CPU restatement of wavo's CPU backend (portable arithmetic).  TEST INFRASTRUCTURE ONLY:
 * see oracle.h.  Built with -ffp-contract=off so that a*b+c stays two roundings wherever the
 * reference's Rust writes it so; fused multiply-adds are spelled fmaf() where the reference uses
 * FMA tiles (src/cpu/gemm.rs:503-529, src/cpu/mod.rs:20-43).
 */
#include "oracle.h"

#include <math.h>
#include <omp.h>
#include <stdlib.h>
#include <string.h>

static int g_threads = 0;
int ox_threads(void) { return g_threads > 0 ? g_threads : omp_get_max_threads(); }
void ox_set_threads(int n) { g_threads = n; }

static inline uint32_t f2u(float x) { uint32_t u; memcpy(&u, &x, 4); return u; }
static inline float u2f(uint32_t u) { float x; memcpy(&x, &u, 4); return x; }

/* src/cpu/gemm.rs:213-221: RNE to f16; subnormal halves are multiples of 2^-24; values past the
 * f16 range keep their exponent. */
float ox_to_half(float x) {
  if (fabsf(x) < u2f(0x38800000u)) return nearbyintf(x * 16777216.0f) / 16777216.0f;
  uint32_t b = f2u(x);
  return u2f((b + 0xfffu + ((b >> 13) & 1u)) & 0xffffe000u);
}

/* IEEE binary16 -> f32. */
float ox_half_to_float(uint16_t h) {
  uint32_t s = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 0x1f, m = h & 0x3ff;
  if (e == 0) {
    float v = (float)m * 5.9604644775390625e-8f; /* m * 2^-24 */
    return s ? -v : v;
  }
  if (e == 31) return u2f(s | 0x7f800000u | (m << 13));
  return u2f(s | ((e + 112) << 23) | (m << 13));
}

/* f32 -> IEEE binary16 bits, round to nearest even, overflow to inf (half::f16::from_f32). */
uint16_t ox_float_to_half_bits(float x) {
  uint32_t u = f2u(x), s = (u >> 16) & 0x8000u;
  uint32_t a = u & 0x7fffffffu;
  if (a >= 0x7f800000u) return (uint16_t)(s | 0x7c00u | (a > 0x7f800000u ? 0x200u : 0));
  if (a >= 0x477ff000u) return (uint16_t)(s | 0x7c00u); /* rounds past 65504 */
  if (a < 0x38800000u) {                                  /* subnormal half or zero */
    float v = u2f(a) * 16777216.0f;                       /* exact scaling, then RNE */
    return (uint16_t)(s | (uint32_t)nearbyintf(v));
  }
  uint32_t e = (a >> 23) - 112, m = a & 0x7fffffu;
  uint32_t h = (e << 10) | (m >> 13);
  uint32_t rest = m & 0x1fffu;
  if (rest > 0x1000u || (rest == 0x1000u && (h & 1u))) h++;
  return (uint16_t)(s | h);
}

/* src/cpu/ops.rs:16-26, Cephes expf without branches. */
float ox_exp(float x) {
  const float MAGIC = 12582912.0f;
  x = x < -87.0f ? -87.0f : (x > 88.0f ? 88.0f : x);
  float t = x * 1.44269504088896340736f + MAGIC;
  float n = t - MAGIC;
  float r = x - n * 0.6933594f + n * 2.1219444e-4f;
  float p = 1.9875691e-4f * r + 1.3981999e-3f;
  p = ((((p * r + 8.333452e-3f) * r + 4.1665796e-2f) * r + 0.16666665f) * r + 0.5f) * r * r;
  float scale = u2f((uint32_t)(((int32_t)f2u(t) - 0x4B400000 + 127) << 23));
  return (p + r + 1.0f) * scale;
}

float ox_silu(float x) { return x / (1.0f + ox_exp(-x)); }

/* src/cpu/ops.rs:33-40: Abramowitz-Stegun 7.1.26 erf. */
float ox_gelu(float x) {
  float z = fabsf(0.70710678118654752440f * x);
  float t = 1.0f / (1.0f + 0.3275911f * z);
  float p = (((1.0614054f * t - 1.453152f) * t + 1.4214138f) * t - 0.28449674f) * t + 0.2548296f;
  float sg = x > 0.0f ? 1.0f : (x < 0.0f ? -1.0f : 0.0f);
  if (x == 0.0f) sg = signbit(x) ? -1.0f : 1.0f; /* f32::signum(±0) = ±1 */
  return 0.5f * x * (1.0f + sg * (1.0f - p * t * ox_exp(-z * z)));
}

/* src/cpu/mod.rs:20-43: 16 FMA lanes, summed pairwise, then the tail. */
float ox_dot(const float *a, const float *b, size_t n) {
  float acc[16] = {0};
  size_t n16 = n / 16 * 16;
  for (size_t i = 0; i < n16; i += 16)
    for (int l = 0; l < 16; l++) acc[l] = fmaf(a[i + l], b[i + l], acc[l]);
  for (int w = 8; w >= 1; w >>= 1)
    for (int l = 0; l < w; l++) acc[l] += acc[l + w];
  float tail = 0.0f;
  for (size_t i = n16; i < n; i++) tail += a[i] * b[i];
  return acc[0] + tail;
}

/* 8-lane sum (src/cpu/ops.rs:57-63). */
static float sum8(const float *v, int n) {
  float acc[8] = {0};
  for (int i = 0; i < n; i++) acc[i % 8] += v[i];
  float s = 0.0f;
  for (int i = 0; i < 8; i++) s += acc[i];
  return s;
}

/* Mean and 1/sqrt(var + 1e-5) (src/cpu/ops.rs:48-54). */
static void moments(const float *x, int n, float *mean, float *rstd, float *tmp) {
  float m = sum8(x, n) / (float)n;
  for (int i = 0; i < n; i++) tmp[i] = (x[i] - m) * (x[i] - m);
  float var = sum8(tmp, n) / (float)n;
  *mean = m;
  *rstd = 1.0f / sqrtf(var + 1e-5f);
}

/* ---------------------------------------------------------------------------------------------- */

size_t ox_type_size(int type, size_t n) {
  switch (type) {
    case OX_F32: return n * 4;
    case OX_F16: return n * 2;
    case OX_Q8_0: return n / 32 * 34;
    case OX_Q4_0: return n / 32 * 18;
  }
  return 0;
}

static inline uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

int ox_dequant(int type, const void *src, float *dst, size_t n) {
  const uint8_t *s = (const uint8_t *)src;
  switch (type) {
    case OX_F32: memcpy(dst, src, n * 4); return 0;
    case OX_F16:
      for (size_t i = 0; i < n; i++) dst[i] = ox_half_to_float(rd16(s + 2 * i));
      return 0;
    case OX_Q8_0: /* src/gguf.rs:281-285: w = i8 * f32(d) */
      for (size_t b = 0; b < n / 32; b++) {
        const uint8_t *blk = s + 34 * b;
        float d = ox_half_to_float(rd16(blk));
        for (int i = 0; i < 32; i++) dst[32 * b + i] = (float)(int8_t)blk[2 + i] * d;
      }
      return 0;
    case OX_Q4_0: /* ggml block_q4_0: d, then 16 bytes; element i < 16 is the low nibble of byte i,
                     element 16 + i the high nibble; w = (nibble - 8) * d */
      for (size_t b = 0; b < n / 32; b++) {
        const uint8_t *blk = s + 18 * b;
        float d = ox_half_to_float(rd16(blk));
        for (int i = 0; i < 16; i++) {
          dst[32 * b + i] = (float)((int)(blk[2 + i] & 15) - 8) * d;
          dst[32 * b + 16 + i] = (float)((int)(blk[2 + i] >> 4) - 8) * d;
        }
      }
      return 0;
  }
  return -1;
}

/* ggml quantize_row_q8_0_ref: d = amax/127 stored as f16; q = round(x * (1/d)) half away from 0. */
void ox_quantize_q8_0(const float *x, void *dst, size_t n) {
  uint8_t *o = (uint8_t *)dst;
  for (size_t b = 0; b < n / 32; b++) {
    float amax = 0.0f;
    for (int i = 0; i < 32; i++) amax = fmaxf(amax, fabsf(x[32 * b + i]));
    float d = amax / 127.0f, id = d != 0.0f ? 1.0f / d : 0.0f;
    uint16_t h = ox_float_to_half_bits(d);
    o[34 * b] = (uint8_t)h;
    o[34 * b + 1] = (uint8_t)(h >> 8);
    for (int i = 0; i < 32; i++) o[34 * b + 2 + i] = (uint8_t)(int8_t)roundf(x[32 * b + i] * id);
  }
}

/* ggml quantize_row_q4_0_ref: max = the value of largest magnitude (signed), d = max / -8,
 * q = min(15, (int8)(x * (1/d) + 8.5)). */
void ox_quantize_q4_0(const float *x, void *dst, size_t n) {
  uint8_t *o = (uint8_t *)dst;
  for (size_t b = 0; b < n / 32; b++) {
    const float *v = x + 32 * b;
    float amax = 0.0f, max = 0.0f;
    for (int i = 0; i < 32; i++)
      if (amax < fabsf(v[i])) { amax = fabsf(v[i]); max = v[i]; }
    float d = max / -8.0f, id = d != 0.0f ? 1.0f / d : 0.0f;
    uint16_t h = ox_float_to_half_bits(d);
    o[18 * b] = (uint8_t)h;
    o[18 * b + 1] = (uint8_t)(h >> 8);
    for (int i = 0; i < 16; i++) {
      int q0 = (int)(int8_t)(v[i] * id + 8.5f), q1 = (int)(int8_t)(v[16 + i] * id + 8.5f);
      q0 = q0 > 15 ? 15 : q0;
      q1 = q1 > 15 ? 15 : q1;
      o[18 * b + 2 + i] = (uint8_t)(q0 | (q1 << 4));
    }
  }
}

/* ---------------------------------------------------------------------------------------------- */

ox_linear *ox_linear_new(int type, int k, int count, const void *const *ws, const int *rows,
                         const float *bias) {
  if (k <= 0 || ((type == OX_Q8_0 || type == OX_Q4_0) && k % 32)) return NULL;
  if (type != OX_F32 && type != OX_F16 && type != OX_Q8_0 && type != OX_Q4_0) return NULL;
  int n = 0;
  for (int i = 0; i < count; i++) n += rows[i];
  ox_linear *l = (ox_linear *)calloc(1, sizeof *l);
  l->n = n;
  l->k = k;
  l->type = type;
  size_t row = ox_type_size(type, (size_t)k);
  l->w = (uint8_t *)malloc(row * (size_t)n + 64);
  size_t at = 0;
  for (int i = 0; i < count; i++) {
    memcpy(l->w + at, ws[i], row * (size_t)rows[i]);
    at += row * (size_t)rows[i];
  }
  l->bias = (float *)calloc((size_t)n, sizeof(float));
  if (bias) memcpy(l->bias, bias, (size_t)n * sizeof(float));
  return l;
}

void ox_linear_free(ox_linear *l) {
  if (!l) return;
  free(l->w);
  free(l->bias);
  free(l);
}

void ox_linear_row(const ox_linear *l, int r, float *out) {
  size_t row = ox_type_size(l->type, (size_t)l->k);
  ox_dequant(l->type, l->w + row * (size_t)r, out, (size_t)l->k);
}

/* v = acc + bias, then the epilogue into c (src/cpu/gemm.rs:339-352). */
static inline float epilogue(int epi, float alpha, float v, float c) {
  switch (epi) {
    case OX_SILU: return ox_silu(v);
    case OX_RELU: return v > 0.0f ? v : 0.0f;
    case OX_RESIDUAL: return c + alpha * v;
    case OX_GELU: return ox_gelu(v);
    case OX_GELU_RESIDUAL: return c + ox_gelu(v);
    case OX_TANH: return tanhf(v < -10.0f ? -10.0f : (v > 10.0f ? 10.0f : v));
    default: return v;
  }
}

#define NR 16
#define MR 6
#define GROUP_BYTES (384 << 10)

/* Panel p of W: [k][NR] of to_half(w), zeros past n (src/cpu/gemm.rs:87-122). */
static void pack_panel(const ox_linear *l, int p, float *out, float *wide) {
  int k = l->k;
  for (int j = 0; j < NR; j++) {
    int row = NR * p + j;
    if (row >= l->n) {
      for (int kk = 0; kk < k; kk++) out[kk * NR + j] = 0.0f;
      continue;
    }
    ox_linear_row(l, row, wide);
    /* F16 weights are already halves; F32 and Q8_0 (q * d, exact in f32) are rounded. */
    for (int kk = 0; kk < k; kk++) out[kk * NR + j] = ox_to_half(wide[kk]);
  }
}

/* MR rows of a times a panel: acc[r][j] = sum over kk in order of fma (src/cpu/gemm.rs:356-375). */
static void tile(const float *const a[MR], const float *b, int k, float acc[MR][NR]) {
  for (int r = 0; r < MR; r++)
    for (int j = 0; j < NR; j++) acc[r][j] = 0.0f;
  for (int kk = 0; kk < k; kk++) {
    const float *bk = b + (size_t)kk * NR;
    for (int r = 0; r < MR; r++) {
      float av = a[r][kk];
      for (int j = 0; j < NR; j++) acc[r][j] = fmaf(av, bk[j], acc[r][j]);
    }
  }
}

/* Runs the GEMM's jobs (src/cpu/gemm.rs:228-269).  The accumulators (without bias) go to
 * store(c_ctx, row, col0, ncols, acc_row). */
typedef void (*store_fn)(void *ctx, int row, int col0, int ncols, const float *acc);

static void gemm_jobs(const float *ah, const ox_linear *l, int m, store_fn store, void *ctx) {
  int k = l->k, n = l->n;
  int panels = (n + NR - 1) / NR;
  int per_group = GROUP_BYTES / (4 * k * NR);
  if (per_group < 1) per_group = 1;
  if (per_group > panels) per_group = panels;
  int groups = (panels + per_group - 1) / per_group;
  int threads = ox_threads();
  int splits = (4 * threads + groups - 1) / groups;
  int maxs = (m + 8 * MR - 1) / (8 * MR);
  if (splits > maxs) splits = maxs;
  if (splits < 1) splits = 1;
  int rows = (m + splits - 1) / splits;
  rows = (rows + MR - 1) / MR * MR;
  int jobs = groups * splits;
#pragma omp parallel num_threads(threads)
  {
    float *buf = (float *)malloc(sizeof(float) * (size_t)per_group * k * NR);
    float *wide = (float *)malloc(sizeof(float) * (size_t)k);
#pragma omp for schedule(dynamic, 1)
    for (int job = 0; job < jobs; job++) {
      int g = job / splits, s = job % splits;
      int p0 = g * per_group, p1 = (g + 1) * per_group < panels ? (g + 1) * per_group : panels;
      for (int p = p0; p < p1; p++) pack_panel(l, p, buf + (size_t)(p - p0) * k * NR, wide);
      int r0 = s * rows, r1 = (s + 1) * rows < m ? (s + 1) * rows : m;
      for (int row = r0; row < r1; row += MR) {
        const float *a[MR];
        for (int r = 0; r < MR; r++) {
          int rr = row + r < r1 ? row + r : r1 - 1;
          a[r] = ah + (size_t)rr * k;
        }
        for (int p = p0; p < p1; p++) {
          float acc[MR][NR];
          tile(a, buf + (size_t)(p - p0) * k * NR, k, acc);
          int c0 = NR * p, nc = n - c0 < NR ? n - c0 : NR;
          for (int r = 0; r < MR && row + r < r1; r++) store(ctx, row + r, c0, nc, acc[r]);
        }
      }
    }
    free(buf);
    free(wide);
  }
}

struct plain_ctx {
  float *c;
  const float *bias;
  int ld, epi;
  float alpha;
};

static void store_plain(void *p, int row, int c0, int nc, const float *acc) {
  struct plain_ctx *x = (struct plain_ctx *)p;
  float *c = x->c + (size_t)row * x->ld + c0;
  for (int j = 0; j < nc; j++) c[j] = epilogue(x->epi, x->alpha, acc[j] + x->bias[c0 + j], c[j]);
}

static float *round_rows(const float *a, size_t len) {
  float *ah = (float *)malloc(sizeof(float) * (len ? len : 1));
#pragma omp parallel for num_threads(ox_threads()) schedule(static)
  for (size_t i = 0; i < len; i++) ah[i] = ox_to_half(a[i]);
  return ah;
}

void ox_gemm(const float *a, const ox_linear *l, float *c, int m, int epi, float alpha) {
  if (m <= 0) return;
  float *ah = round_rows(a, (size_t)m * l->k);
  struct plain_ctx ctx = {c, l->bias, l->n, epi, alpha};
  gemm_jobs(ah, l, m, store_plain, &ctx);
  free(ah);
}

struct wide_ctx {
  float *c;
  const float *bias, *bias2;
  int ld, cols, dual, epi;
  float alpha;
};

static void store_wide(void *p, int row, int c0, int nc, const float *acc) {
  struct wide_ctx *x = (struct wide_ctx *)p;
  float *c = x->c + (size_t)row * x->ld;
  for (int j = 0; j < nc; j++) {
    int col = c0 + j;
    c[col] = epilogue(x->epi, x->alpha, acc[j] + x->bias[col], c[col]);
    if (col < x->dual) c[x->cols + col] = acc[j] + x->bias2[col];
  }
}

void ox_gemm_wide(const float *a, const ox_linear *l, float *c, int m, int epi, float alpha,
                  const float *bias2, int dual) {
  if (m <= 0) return;
  int n = l->n;
  int cols = n % 32 == 0 ? n : (n + 63) / 64 * 64;
  int ld = cols + dual;
  float *ah = round_rows(a, (size_t)m * l->k);
  struct wide_ctx ctx = {c, l->bias, bias2, ld, cols, dual, epi, alpha};
  gemm_jobs(ah, l, m, store_wide, &ctx);
  /* The padding columns: epilogue of v = 0. */
  for (int r = 0; r < m; r++)
    for (int j = n; j < cols; j++) c[(size_t)r * ld + j] = epilogue(epi, alpha, 0.0f, c[(size_t)r * ld + j]);
  free(ah);
}

void ox_gemv(const float *x, const ox_linear *l, float *c, int epi, float alpha) {
  int n = l->n, k = l->k;
#pragma omp parallel num_threads(ox_threads())
  {
    float *w = (float *)malloc(sizeof(float) * (size_t)k);
#pragma omp for schedule(static)
    for (int r = 0; r < n; r++) {
      ox_linear_row(l, r, w);
      float v = ox_dot(w, x, (size_t)k) + l->bias[r];
      c[r] = epilogue(epi, alpha, v, c[r]);
    }
    free(w);
  }
}

/* ---------------------------------------------------------------------------------------------- */

void ox_layer_norm(const float *x, const float *w, const float *b, float *y, int rows, int cols,
                   const float *table, float *yr, int hd) {
#pragma omp parallel num_threads(ox_threads())
  {
    float *tmp = (float *)malloc(sizeof(float) * (size_t)cols);
#pragma omp for schedule(static)
    for (int r = 0; r < rows; r++) {
      const float *xr = x + (size_t)r * cols;
      float *yy = y + (size_t)r * cols;
      float mean, rstd;
      moments(xr, cols, &mean, &rstd, tmp);
      for (int i = 0; i < cols; i++) yy[i] = (xr[i] - mean) * rstd * w[i] + b[i];
      if (table) {
        int half = hd / 2;
        const float *cs = table + (size_t)r * hd, *sn = cs + half;
        float *o = yr + (size_t)r * cols;
        for (int h0 = 0; h0 < cols; h0 += hd)
          for (int i = 0; i < half; i++) {
            float y0 = yy[h0 + i], y1 = yy[h0 + half + i];
            o[h0 + i] = y0 * cs[i] - y1 * sn[i];
            o[h0 + half + i] = y1 * cs[i] + y0 * sn[i];
          }
      }
    }
    free(tmp);
  }
}

void ox_im2col(const float *x, int t, int ch, int kernel, int stride, int pad, float *col,
               int width) {
  int rows = (t + 2 * pad - kernel) / stride + 1;
  if (width < ch * kernel) width = ch * kernel;
  for (int i = 0; i < rows; i++) {
    float *cr = col + (size_t)i * width;
    memset(cr, 0, sizeof(float) * (size_t)width);
    for (int k = 0; k < kernel; k++) {
      int s = stride * i + k;
      if (s < pad || s - pad >= t) continue;
      const float *xr = x + (size_t)(s - pad) * ch;
      for (int c = 0; c < ch; c++) cr[c * kernel + k] = xr[c];
    }
  }
}

void ox_conv_glu(float *h, const float *taps, const float *tb, int kernel, const float *g,
                 const float *beta, int layer_norm, float *y, int t, int ch, int valid) {
  if (valid < 0 || valid > t) valid = t;
#pragma omp parallel for num_threads(ox_threads()) schedule(static)
  for (int s = 0; s < t; s++) {
    float *x = h + (size_t)s * 2 * ch, *gate = x + ch;
    for (int c = 0; c < ch; c++) x[c] /= 1.0f + ox_exp(-gate[c]);
    if (s >= valid)
      for (int c = 0; c < ch; c++) x[c] = 0.0f;
  }
#pragma omp parallel num_threads(ox_threads())
  {
    float *acc = (float *)malloc(sizeof(float) * (size_t)ch);
    float *tmp = (float *)malloc(sizeof(float) * (size_t)ch);
#pragma omp for schedule(static)
    for (int i = 0; i < t; i++) {
      memcpy(acc, tb, sizeof(float) * (size_t)ch);
      for (int k = 0; k < kernel; k++) {
        int src = i + k - kernel / 2;
        if (src < 0 || src >= t) continue;
        const float *xs = h + (size_t)src * 2 * ch, *w = taps + (size_t)k * ch;
        for (int c = 0; c < ch; c++) acc[c] += w[c] * xs[c];
      }
      float mean = 0.0f, rstd = 1.0f;
      if (layer_norm) moments(acc, ch, &mean, &rstd, tmp);
      float *yy = y + (size_t)i * ch;
      for (int c = 0; c < ch; c++) yy[c] = ox_silu((acc[c] - mean) * rstd * g[c] + beta[c]);
    }
    free(acc);
    free(tmp);
  }
}

/* Softmax of scale * s over the first n of the row, zero past `valid` (src/cpu/ops.rs:278-289). */
static void softmax_row(float *s, int n, int valid, float scale) {
  float mx = -INFINITY;
  for (int j = 0; j < valid; j++) mx = fmaxf(mx, s[j]);
  mx *= scale;
  for (int j = 0; j < valid; j++) s[j] = ox_exp(s[j] * scale - mx);
  for (int j = valid; j < n; j++) s[j] = 0.0f;
  float inv = 1.0f / sum8(s, valid);
  for (int j = 0; j < valid; j++) s[j] *= inv;
}

/* sum_c a[c] * b[c] by in-order fma (the `product` tile's per-output order). */
static inline float fdot(const float *a, const float *b, int n) {
  float acc = 0.0f;
  for (int c = 0; c < n; c++) acc = fmaf(a[c], b[c], acc);
  return acc;
}

void ox_attention(const float *qk, int ld, const float *v, int ldv, float *o, int t, int heads,
                  int hd, int valid) {
  int ch = heads * hd;
  if (valid <= 0 || valid > t) valid = t;
  float scale = 1.0f / sqrtf((float)hd);
#pragma omp parallel num_threads(ox_threads())
  {
    float *s = (float *)malloc(sizeof(float) * (size_t)t);
    float *acc = (float *)malloc(sizeof(float) * (size_t)hd);
    float *kh = (float *)malloc(sizeof(float) * (size_t)t * hd);
#pragma omp for schedule(dynamic, 1) collapse(2)
    for (int h = 0; h < heads; h++)
      for (int i0 = 0; i0 < t; i0 += 48) {
        for (int j = 0; j < t; j++) memcpy(kh + (size_t)j * hd, qk + (size_t)j * ld + ch + h * hd, sizeof(float) * hd);
        int i1 = i0 + 48 < t ? i0 + 48 : t;
        for (int i = i0; i < i1; i++) {
          const float *q = qk + (size_t)i * ld + h * hd;
          for (int j = 0; j < t; j++) s[j] = fdot(q, kh + (size_t)j * hd, hd);
          softmax_row(s, t, valid, scale);
          for (int c = 0; c < hd; c++) acc[c] = 0.0f;
          for (int j = 0; j < valid; j++) {
            const float *vr = v + (size_t)j * ldv + h * hd;
            for (int c = 0; c < hd; c++) acc[c] = fmaf(s[j], vr[c], acc[c]);
          }
          memcpy(o + (size_t)i * ch + h * hd, acc, sizeof(float) * hd);
        }
      }
    free(s);
    free(acc);
    free(kh);
  }
}

void ox_relative_attention(const float *qkv, const float *pos, const float *u, const float *vb,
                           float *o, int t, int heads, int hd, int valid) {
  int ch = heads * hd;
  if (valid <= 0 || valid > t) valid = t;
  float scale = 1.0f / sqrtf((float)hd);
#pragma omp parallel num_threads(ox_threads())
  {
    float *s = (float *)malloc(sizeof(float) * (size_t)t);
    float *acc = (float *)malloc(sizeof(float) * (size_t)hd);
    float *qu = (float *)malloc(sizeof(float) * (size_t)hd);
    float *qv = (float *)malloc(sizeof(float) * (size_t)hd);
#pragma omp for schedule(dynamic, 1) collapse(2)
    for (int h = 0; h < heads; h++)
      for (int i0 = 0; i0 < t; i0 += 48) {
        int i1 = i0 + 48 < t ? i0 + 48 : t;
        for (int i = i0; i < i1; i++) {
          const float *q = qkv + (size_t)i * 3 * ch + h * hd;
          for (int c = 0; c < hd; c++) {
            qu[c] = q[c] + u[h * hd + c];
            qv[c] = q[c] + vb[h * hd + c];
          }
          for (int j = 0; j < t; j++) {
            float a = fdot(qu, qkv + (size_t)j * 3 * ch + ch + h * hd, hd);
            float p = fdot(qv, pos + (size_t)(j - i + t + 15) * ch + h * hd, hd);
            s[j] = a + p;
          }
          softmax_row(s, t, valid, scale);
          for (int c = 0; c < hd; c++) acc[c] = 0.0f;
          for (int j = 0; j < valid; j++) {
            const float *vr = qkv + (size_t)j * 3 * ch + 2 * ch + h * hd;
            for (int c = 0; c < hd; c++) acc[c] = fmaf(s[j], vr[c], acc[c]);
          }
          memcpy(o + (size_t)i * ch + h * hd, acc, sizeof(float) * hd);
        }
      }
    free(s);
    free(acc);
    free(qu);
    free(qv);
  }
}

void ox_attend(const float *q, const float *kv, int cols, int n, float *o, int heads, int hd) {
  float scale = 1.0f / sqrtf((float)hd);
  const float *k = kv, *v = kv + (size_t)heads * cols * hd;
  float *qh = (float *)malloc(sizeof(float) * (size_t)hd);
  float *s = (float *)malloc(sizeof(float) * (size_t)(n > 0 ? n : 1));
  for (int h = 0; h < heads; h++) {
    for (int c = 0; c < hd; c++) qh[c] = ox_half_to_float(ox_float_to_half_bits(q[h * hd + c]));
    const float *kh = k + (size_t)h * cols * hd, *vh = v + (size_t)h * cols * hd;
    for (int j = 0; j < n; j++) s[j] = ox_dot(qh, kh + (size_t)j * hd, (size_t)hd) * scale;
    float mx = -INFINITY;
    for (int j = 0; j < n; j++) mx = fmaxf(mx, s[j]);
    for (int j = 0; j < n; j++) s[j] = ox_exp(s[j] - mx);
    float inv = 1.0f / sum8(s, n);
    float *oh = o + (size_t)h * hd;
    for (int c = 0; c < hd; c++) oh[c] = 0.0f;
    for (int j = 0; j < n; j++)
      for (int c = 0; c < hd; c++) oh[c] += s[j] * vh[(size_t)j * hd + c];
    for (int c = 0; c < hd; c++) oh[c] *= inv;
  }
  free(qh);
  free(s);
}

void ox_pack(const float *x, int src, int stride, uint32_t *cache, int rows, int d, int cols,
             int col) {
  int half = d / 2;
  for (int j = 0; j < rows; j++)
    for (int i = 0; i < d; i++) {
      const float *p = x + src + (size_t)j * stride + 2 * i;
      uint32_t w = (uint32_t)ox_float_to_half_bits(ox_to_half(p[0])) |
                   ((uint32_t)ox_float_to_half_bits(ox_to_half(p[1])) << 16);
      size_t at = i < half ? (size_t)i * cols + col + j
                           : (size_t)half * cols + (size_t)(col + j) * half + (i - half);
      cache[at] = w;
    }
}

void ox_rope_table(int frames, int hd, double theta, float *out) {
  int half = hd / 2;
  for (int t = 0; t < frames; t++)
    for (int i = 0; i < half; i++) {
      double a = (double)t * pow(theta, -2.0 * (double)i / (double)hd);
      out[(size_t)t * hd + i] = (float)cos(a);
      out[(size_t)t * hd + half + i] = (float)sin(a);
    }
}

void ox_rel_positions(int d, long first, int rows, float *out) {
  int half = d / 2;
  float *div = (float *)malloc(sizeof(float) * (size_t)half);
  for (int k = 0; k < half; k++) div[k] = expf((float)(2 * k) * (-logf(10000.0f) / (float)d));
  for (int r = 0; r < rows; r++) {
    float p = (float)(first - r);
    for (int k = 0; k < half; k++) {
      out[(size_t)r * d + 2 * k] = sinf(p * div[k]);
      out[(size_t)r * d + 2 * k + 1] = cosf(p * div[k]);
    }
  }
  free(div);
}

void ox_batch_norm(const float *w, const float *b, const float *mean, const float *var, int d,
                   float *scale, float *shift) {
  for (int i = 0; i < d; i++) {
    scale[i] = w[i] / sqrtf(var[i] + 1e-5f);
    shift[i] = b[i] - mean[i] * scale[i];
  }
}

/* ---------------------------------------------------------------------------------------------- */

static inline int half_len(int n) { return (n - 1) / 2 + 1; }

void ox_sub_first(const float *mel, int valid, int mels, const float *w0, const float *b0,
                  const float *w2, const float *b2, int ch, float *y, int rows, int t0) {
  int t1 = half_len(valid), f1 = half_len(mels), f2 = half_len(f1);
#pragma omp parallel num_threads(ox_threads())
  {
    float *c0 = (float *)malloc(sizeof(float) * (size_t)3 * f1 * ch);
#pragma omp for schedule(static)
    for (int k = 0; k < rows; k++) {
      for (int i = 0; i < 3; i++) {
        float *row = c0 + (size_t)i * f1 * ch;
        long r = 4L * t0 + 2L * k + i - 3;
        if (r < 0 || r >= t1) {
          memset(row, 0, sizeof(float) * (size_t)f1 * ch);
          continue;
        }
        for (int c = 0; c < f1; c++) {
          float *px = row + (size_t)c * ch;
          memcpy(px, b0, sizeof(float) * (size_t)ch);
          for (int tap = 0; tap < 9; tap++) {
            long tm = 2 * r + tap / 3 - 1, fm = 2L * c + tap % 3 - 1;
            float x = (tm >= 0 && tm < valid && fm >= 0 && fm < mels) ? mel[tm * mels + fm] : 0.0f;
            const float *w = w0 + (size_t)tap * ch;
            for (int e = 0; e < ch; e++) px[e] += w[e] * x;
          }
          for (int e = 0; e < ch; e++) px[e] = px[e] > 0.0f ? px[e] : 0.0f;
        }
      }
      int masked = 2 * t0 + k > half_len(t1);
      for (int fo = 0; fo < f2; fo++) {
        float *yy = y + ((size_t)k * f2 + fo) * ch;
        if (masked) {
          memset(yy, 0, sizeof(float) * (size_t)ch);
          continue;
        }
        memcpy(yy, b2, sizeof(float) * (size_t)ch);
        for (int tap = 0; tap < 9; tap++) {
          int c = 2 * fo + tap % 3 - 1;
          if (c < 0 || c >= f1) continue;
          const float *x = c0 + ((size_t)(tap / 3) * f1 + c) * ch, *w = w2 + (size_t)tap * ch;
          for (int e = 0; e < ch; e++) yy[e] += w[e] * x[e];
        }
      }
    }
    free(c0);
  }
}

void ox_depthwise(const float *x, const float *w, const float *b, int t, int f, int ch, float *y,
                  int n, int t0) {
  int fo_n = half_len(f);
#pragma omp parallel for num_threads(ox_threads()) schedule(static)
  for (int k = 0; k < n; k++)
    for (int fo = 0; fo < fo_n; fo++) {
      float *yy = y + ((size_t)k * fo_n + fo) * ch;
      memcpy(yy, b, sizeof(float) * (size_t)ch);
      for (int tap = 0; tap < 9; tap++) {
        int ti = 2 * (t0 + k) + tap / 3, fi = 2 * fo + tap % 3;
        if (ti < 1 || ti > t || fi < 1 || fi > f) continue;
        const float *xx = x + (((size_t)2 * k + tap / 3) * f + fi - 1) * ch, *ww = w + (size_t)tap * ch;
        for (int e = 0; e < ch; e++) yy[e] += ww[e] * xx[e];
      }
    }
}

void ox_flatten(const float *x, float *y, int t, int f, int ch) {
  size_t n = (size_t)f * ch;
  for (int r = 0; r < t; r++)
    for (size_t e = 0; e < n; e++) y[r * n + e] = x[r * n + (e % f) * ch + e / f];
}

/* ---------------------------------------------------------------------------------------------- */

int ox_argmax(const float *v, int n) {
  int best = 0;
  for (int i = 1; i < n; i++)
    if (v[i] > v[best]) best = i;
  return best;
}

int ox_ctc(const float *logits, int frames, int classes, int blank, uint32_t *out) {
  int count = 0, prev = -1;
  for (int t = 0; t < frames; t++) {
    int best = ox_argmax(logits + (size_t)t * classes, classes);
    if (prev != best && best != blank) {
      out[2 * count] = (uint32_t)best;
      out[2 * count + 1] = (uint32_t)t;
      count++;
    }
    prev = best;
  }
  return count;
}

/* The TDT loop of src/parakeet/decoder.rs:158-191 over a decision source. */
typedef void (*tdt_joint)(void *ctx, int t, int emitted, int *token, int *dur);

int ox_tdt_loop(int frames, int blank, const int *durations, int max_symbols, int global,
                tdt_joint joint, void *ctx, uint32_t *out, int cap) {
  int count = 0, t = 0, symbols = 0, emitted = -1;
  long left = global ? (long)max_symbols * frames : -1;
  while (t < frames && (left < 0 || left > 0)) {
    int token, d;
    joint(ctx, t, emitted, &token, &d);
    emitted = -1;
    if (token != blank) {
      if (count < cap) {
        out[2 * count] = (uint32_t)token;
        out[2 * count + 1] = (uint32_t)t;
      }
      count++;
      emitted = token;
    }
    if (global) {
      left--;
      int step = durations[d];
      t += token == blank ? (step > 1 ? step : 1) : step;
      continue;
    }
    t += durations[d];
    symbols++;
    if (durations[d] != 0) symbols = 0;
    else if (symbols >= max_symbols || token == blank) {
      t++;
      symbols = 0;
    }
  }
  return count;
}

struct scripted {
  const int *script;
  int len, used;
  int *calls;
};

static void scripted_joint(void *p, int t, int emitted, int *token, int *dur) {
  struct scripted *s = (struct scripted *)p;
  if (s->calls) {
    s->calls[2 * s->used] = t;
    s->calls[2 * s->used + 1] = emitted;
  }
  if (s->used < s->len) {
    *token = s->script[2 * s->used];
    *dur = s->script[2 * s->used + 1];
  } else {
    *token = -2; /* script too short: caller sees used > len */
    *dur = 0;
  }
  s->used++;
}

int ox_tdt_scripted(int frames, int blank, const int *durations, int max_symbols, int global,
                    const int *script, int script_len, uint32_t *out, int *calls, int *used) {
  struct scripted s = {script, script_len, 0, calls};
  int n = ox_tdt_loop(frames, blank, durations, max_symbols, global, scripted_joint, &s, out, 1 << 20);
  *used = s.used;
  return n;
}
