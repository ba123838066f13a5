/*
 * Parity oracle (test infrastructure only; the product never links it): the log-mel frontends of
 * src/fft.rs, src/parakeet/frontend.rs, src/gigaam/frontend.rs and src/whisper/frontend.rs, restated in C
 * with the reference's operations in its order.  Every multiply-add the reference writes as mul_add is
 * fma()/fmaf() here; every other product and sum is rounded on its own (the Makefile builds with
 * -ffp-contract=off).  cos, sin, ln, exp and log10 come from the C library, as the reference's f64/f32
 * methods do on Linux.
 *
 *   Fft::new / forward / leaves / stage ... src/fft.rs:47-148
 *   Parakeet Frontend .................... src/parakeet/frontend.rs:29-141
 *   GigaAM Frontend ...................... src/gigaam/frontend.rs:25-71
 *   Whisper Frontend ..................... src/whisper/frontend.rs:28-106
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"

/* With g_raw set, the frontends write each filter's sum (the value the logarithm would take, before
 * Parakeet's epsilon, GigaAM's clamp or Whisper's floor; 0 for Whisper's silent frames) and skip the
 * normalization or scaling: the check of the transform and filter arithmetic bit for bit. */
static int g_raw = 0;
void ox_mel_raw(int on) { g_raw = on; }

/* ------------------------------------------------------------------------------------------ FFT */

/* The transform's tables for n = leaf · 2^stages (src/fft.rs:47-70). */
typedef struct {
  int n, leaf, blocks, stages;
  int *perm;
  double *lc, *ls; /* leaf cos / sin, [j][k] */
  double *tc, *ts; /* per stage, the twiddle of each output i < n / 2 */
} fft_plan;

static void trig(int i, int n, double *c, double *s) {
  double phase = 6.283185307179586 * (double)i / (double)n; /* TAU · i / n */
  *c = cos(phase);
  *s = sin(phase);
}

static int fft_plan_init(fft_plan *p, int n) {
  memset(p, 0, sizeof *p);
  int leaf = n;
  while (leaf % 2 == 0) leaf /= 2;
  int blocks = n / leaf;
  p->n = n, p->leaf = leaf, p->blocks = blocks;
  /* The first sample of each leaf: the recursion puts even samples before odd ones. */
  int *starts = (int *)malloc(sizeof(int) * blocks), len = 1;
  starts[0] = 0;
  int *next = (int *)malloc(sizeof(int) * blocks);
  while (len < blocks) {
    for (int i = 0; i < len; i++) next[i] = 2 * starts[i], next[len + i] = 2 * starts[i] + 1;
    len *= 2;
    memcpy(starts, next, sizeof(int) * len);
  }
  free(next);
  p->perm = (int *)malloc(sizeof(int) * n);
  for (int i = 0; i < n; i++) p->perm[i] = starts[i % blocks] + i / blocks * blocks;
  free(starts);
  p->lc = (double *)malloc(sizeof(double) * leaf * leaf);
  p->ls = (double *)malloc(sizeof(double) * leaf * leaf);
  for (int i = 0; i < leaf * leaf; i++) trig((int)((long)(i / leaf) * (i % leaf) * blocks % n), n, &p->lc[i], &p->ls[i]);
  int stages = 0;
  for (int size = 2 * leaf; size <= n; size *= 2) stages++;
  p->stages = stages;
  p->tc = (double *)malloc(sizeof(double) * (stages * (n / 2) + 1));
  p->ts = (double *)malloc(sizeof(double) * (stages * (n / 2) + 1));
  int st = 0;
  for (int size = 2 * leaf; size <= n; size *= 2, st++)
    for (int i = 0; i < n / 2; i++) {
      int g = n / size;
      trig(i / g * g, n, &p->tc[st * (n / 2) + i], &p->ts[st * (n / 2) + i]);
    }
  return 0;
}

static void fft_plan_free(fft_plan *p) {
  free(p->perm), free(p->lc), free(p->ls), free(p->tc), free(p->ts);
}

/* Fft::forward over x[n]: re and im into buf[0..n) and buf[n..2n) (buf holds 4n). */
#define FFT_FORWARD(NAME, T, FMA)                                                                  \
  static void NAME(const fft_plan *p, const T *x, T *buf) {                                         \
    const int n = p->n, leaf = p->leaf, blocks = p->blocks;                                         \
    T *front = buf, *back = buf + 2 * n;                                                            \
    T *src = p->stages % 2 == 0 ? back : front, *dst = p->stages % 2 == 0 ? front : back;           \
    for (int j = 0; j < n; j++) src[j] = x[p->perm[j]];                                             \
    /* leaves (src/fft.rs:106-122) */                                                               \
    T *re = dst, *im = dst + n;                                                                     \
    for (int k = 0; k < leaf; k++) {                                                                \
      T *rk = re + k * blocks, *ik = im + k * blocks;                                               \
      for (int g = 0; g < blocks; g++) rk[g] = src[g], ik[g] = (T)0;                                \
      for (int j = 1; j < leaf; j++) {                                                              \
        const T c = (T)p->lc[j * leaf + k], s = (T)p->ls[j * leaf + k];                             \
        const T *xs = src + j * blocks;                                                             \
        for (int g = 0; g < blocks; g++) {                                                          \
          rk[g] = FMA(xs[g], c, rk[g]);                                                             \
          ik[g] = FMA(-xs[g], s, ik[g]);                                                            \
        }                                                                                           \
      }                                                                                             \
    }                                                                                               \
    /* radix-2 stages (src/fft.rs:124-138) */                                                       \
    const int half = n / 2;                                                                         \
    for (int st = 0; st < p->stages; st++) {                                                        \
      T *t = src;                                                                                   \
      src = dst, dst = t;                                                                           \
      const T *sr = src, *si = src + n;                                                             \
      T *dr = dst, *di = dst + n;                                                                   \
      for (int i = 0; i < half; i++) {                                                              \
        const T c = (T)p->tc[st * half + i], s = (T)p->ts[st * half + i];                           \
        const T a = sr[2 * i], xo = sr[2 * i + 1], b = si[2 * i], y = si[2 * i + 1];                \
        dr[i] = FMA(s, y, FMA(c, xo, a));                                                           \
        di[i] = FMA(-s, xo, FMA(c, y, b));                                                          \
        dr[i + half] = FMA(-s, y, FMA(-c, xo, a));                                                  \
        di[i + half] = FMA(s, xo, FMA(-c, y, b));                                                   \
      }                                                                                             \
    }                                                                                               \
  }

FFT_FORWARD(fft_forward64, double, fma)
FFT_FORWARD(fft_forward32, float, fmaf)

int ox_fft(int n, int f64, const void *x, void *re, void *im) {
  if (n <= 0) return -1;
  fft_plan p;
  fft_plan_init(&p, n);
  if (f64) {
    double *buf = (double *)malloc(sizeof(double) * 4 * n);
    fft_forward64(&p, (const double *)x, buf);
    memcpy(re, buf, sizeof(double) * n);
    memcpy(im, buf + n, sizeof(double) * n);
    free(buf);
  } else {
    float *buf = (float *)malloc(sizeof(float) * 4 * n);
    fft_forward32(&p, (const float *)x, buf);
    memcpy(re, buf, sizeof(float) * n);
    memcpy(im, buf + n, sizeof(float) * n);
    free(buf);
  }
  fft_plan_free(&p);
  return 0;
}

int ox_fft_tables(int n, int *perm, double *leaf_cos, double *leaf_sin, double *tw_cos, double *tw_sin,
                  int *leaf, int *stages) {
  fft_plan p;
  fft_plan_init(&p, n);
  *leaf = p.leaf, *stages = p.stages;
  if (perm) memcpy(perm, p.perm, sizeof(int) * n);
  if (leaf_cos) memcpy(leaf_cos, p.lc, sizeof(double) * p.leaf * p.leaf);
  if (leaf_sin) memcpy(leaf_sin, p.ls, sizeof(double) * p.leaf * p.leaf);
  if (tw_cos) memcpy(tw_cos, p.tc, sizeof(double) * p.stages * (n / 2));
  if (tw_sin) memcpy(tw_sin, p.ts, sizeof(double) * p.stages * (n / 2));
  fft_plan_free(&p);
  return 0;
}

/* ------------------------------------------------------------------------------------ Parakeet */

#define PK_MELS 128
#define PK_FFT 512
#define PK_WIN 400
#define PK_HOP 160
#define PK_BINS (PK_FFT / 2 + 1)

/* slaney_filterbank (src/parakeet/frontend.rs:113-141): [128][257]. */
void ox_parakeet_filterbank(float *out) {
  const double fsp = 200.0 / 3.0, min_log_hz = 1000.0, min_log_mel = min_log_hz / fsp;
  const double log_step = log(6.4) / 27.0;
  const double fmax = 8000.0;
  const double mel_max = fmax < min_log_hz ? fmax / fsp : min_log_mel + log(fmax / min_log_hz) / log_step;
  double hz[PK_MELS + 2];
  for (int m = 0; m < PK_MELS + 2; m++) {
    double mel = mel_max * (double)m / (double)(PK_MELS + 1);
    hz[m] = mel < min_log_mel ? mel * fsp : min_log_hz * exp(log_step * (mel - min_log_mel));
  }
  for (int m = 0; m < PK_MELS; m++) {
    double enorm = 2.0 / (hz[m + 2] - hz[m]);
    for (int k = 0; k < PK_BINS; k++) {
      double f = 16000.0 * (double)k / (double)PK_FFT;
      double lower = (f - hz[m]) / (hz[m + 1] - hz[m]);
      double upper = (hz[m + 2] - f) / (hz[m + 2] - hz[m + 1]);
      double v = lower < upper ? lower : upper;
      if (!(v > 0.0)) v = 0.0;
      out[m * PK_BINS + k] = (float)(v * enorm);
    }
  }
}

/* The symmetric Hann(400) centred in 512 (src/parakeet/frontend.rs:33-39). */
static void parakeet_window(double *w) {
  const int pad = (PK_FFT - PK_WIN) / 2;
  for (int i = 0; i < PK_FFT; i++) {
    int k = i - pad;
    w[i] = k >= 0 && k < PK_WIN ? 0.5 - 0.5 * cos(2.0 * 3.141592653589793 * (double)k / (double)(PK_WIN - 1)) : 0.0;
  }
}

/* Frontend::log_mel (src/parakeet/frontend.rs:74-108) for frames [t0, t1) of the whole pcm. */
int ox_parakeet_log_mel(const float *pcm, int samples, int t0, int t1, float *out) {
  const int frames = samples / PK_HOP + 1;
  if (t0 < 0 || t1 > frames || t0 > t1) return -1;
  double window[PK_FFT];
  parakeet_window(window);
  float *filters = (float *)malloc(sizeof(float) * PK_MELS * PK_BINS);
  ox_parakeet_filterbank(filters);
  int lo[PK_MELS], hi[PK_MELS];
  for (int m = 0; m < PK_MELS; m++) {
    const float *f = filters + m * PK_BINS;
    int a = 0, b = -1;
    while (a < PK_BINS && f[a] == 0.0f) a++;
    if (a == PK_BINS) a = 0;
    for (int k = PK_BINS - 1; k >= 0; k--)
      if (f[k] != 0.0f) {
        b = k;
        break;
      }
    lo[m] = a, hi[m] = b < 0 ? a : b + 1;
  }
  fft_plan p;
  fft_plan_init(&p, PK_FFT);
  const int pad = t0 * PK_HOP, len = (t1 - t0 > 0 ? t1 - t0 - 1 : 0) * PK_HOP + PK_FFT;
  double *padded = (double *)malloc(sizeof(double) * len);
  for (int q = 0; q < len; q++) {
    long j = (long)pad + q - PK_FFT / 2;
    if (j < 0) padded[q] = 0.0;
    else if (j == 0) padded[q] = (double)pcm[0];
    else if (j < samples) padded[q] = (double)pcm[j] - (double)0.97f * (double)pcm[j - 1];
    else padded[q] = 0.0;
  }
  double frame[PK_FFT], buf[4 * PK_FFT];
  float power[PK_BINS];
  for (int t = 0; t < t1 - t0; t++) {
    for (int i = 0; i < PK_FFT; i++) frame[i] = padded[t * PK_HOP + i] * window[i];
    fft_forward64(&p, frame, buf);
    for (int k = 0; k < PK_BINS; k++) power[k] = (float)(buf[k] * buf[k] + buf[PK_FFT + k] * buf[PK_FFT + k]);
    for (int m = 0; m < PK_MELS; m++) {
      float e = 0.0f;
      for (int k = lo[m]; k < hi[m]; k++) e = fmaf(filters[m * PK_BINS + k], power[k], e);
      out[t * PK_MELS + m] = g_raw ? e : logf(e + 1.0f / (float)(1 << 24));
    }
  }
  free(padded);
  free(filters);
  fft_plan_free(&p);
  return t1 - t0;
}

/* Frontend::compute (src/parakeet/frontend.rs:52-72): [samples / 160 + 1][128], 0 frames below 3. */
int ox_parakeet_mel(const float *pcm, int samples, float *out) {
  const int frames = samples / PK_HOP + 1;
  if (frames < 3) return 0;
  if (!out) return frames;
  ox_parakeet_log_mel(pcm, samples, 0, frames, out);
  if (g_raw) return frames;
  const int n = frames - 1;
  for (int m = 0; m < PK_MELS; m++) {
    double mean = 0.0, var = 0.0;
    for (int t = 0; t < n; t++) mean += (double)out[t * PK_MELS + m];
    mean /= (double)n;
    for (int t = 0; t < n; t++) {
      double d = (double)out[t * PK_MELS + m] - mean;
      var += d * d;
    }
    var /= (double)(n - 1);
    const double inv = 1.0 / (sqrt(var) + (double)1e-5f);
    for (int t = 0; t < n; t++) out[t * PK_MELS + m] = (float)(((double)out[t * PK_MELS + m] - mean) * inv);
    out[n * PK_MELS + m] = 0.0f;
  }
  return frames;
}

/* -------------------------------------------------------------------------------------- GigaAM */

#define GA_FFT 320
#define GA_HOP 160
#define GA_BINS (GA_FFT / 2 + 1)

/* Frontend::compute (src/gigaam/frontend.rs:50-71) with the GGUF's window [320] and filterbank
 * [mels][161]: [(samples − 320) / 160 + 1][mels], 0 frames below 320 samples. */
int ox_gigaam_mel(const float *pcm, int samples, const float *window, const float *filters, int mels, float *out) {
  const int frames = samples >= GA_FFT ? (samples - GA_FFT) / GA_HOP + 1 : 0;
  if (!out || frames == 0) return frames;
  int *lo = (int *)malloc(sizeof(int) * mels), *hi = (int *)malloc(sizeof(int) * mels);
  for (int m = 0; m < mels; m++) { /* spans widened to dot's 16-bin chunks (src/gigaam/frontend.rs:31-38) */
    const float *f = filters + m * GA_BINS;
    int a = 0, b = 0;
    while (a < GA_BINS && f[a] == 0.0f) a++;
    if (a == GA_BINS) a = 0;
    for (int k = GA_BINS - 1; k >= 0; k--)
      if (f[k] != 0.0f) {
        b = k + 1;
        break;
      }
    a = a / 16 * 16;
    b = b > GA_BINS / 16 * 16 ? GA_BINS : (b + 15) / 16 * 16;
    lo[m] = a, hi[m] = b > a ? b : a;
  }
  fft_plan p;
  fft_plan_init(&p, GA_FFT);
  float frame[GA_FFT], buf[4 * GA_FFT], power[GA_BINS];
  for (int t = 0; t < frames; t++) {
    for (int i = 0; i < GA_FFT; i++) frame[i] = pcm[t * GA_HOP + i] * window[i];
    fft_forward32(&p, frame, buf);
    for (int k = 0; k < GA_BINS; k++) power[k] = buf[k] * buf[k] + buf[GA_FFT + k] * buf[GA_FFT + k];
    for (int m = 0; m < mels; m++) {
      float v = ox_dot(filters + m * GA_BINS + lo[m], power + lo[m], (size_t)(hi[m] - lo[m]));
      if (g_raw) {
        out[t * mels + m] = v;
        continue;
      }
      v = v < 1e-9f ? 1e-9f : v > 1e9f ? 1e9f : v;
      out[t * mels + m] = logf(v);
    }
  }
  fft_plan_free(&p);
  free(lo);
  free(hi);
  return frames;
}

/* ------------------------------------------------------------------------------------- Whisper */

#define WS_FFT 400
#define WS_HOP 160
#define WS_BINS (WS_FFT / 2 + 1)
#define WS_SAMPLES 480000

/* Frontend::compute (src/whisper/frontend.rs:45-85) with the GGUF's window [400] and filterbank
 * [mels][201]: [max(samples, 480000) / 160][mels]. */
int ox_whisper_mel(const float *pcm, int samples, const float *window, const float *filters, int mels, float *out) {
  const int len = samples > WS_SAMPLES ? samples : WS_SAMPLES, pad = WS_FFT / 2, frames = len / WS_HOP;
  if (!out) return frames;
  float *padded = (float *)calloc((size_t)len + WS_FFT, sizeof(float));
  memcpy(padded + pad, pcm, sizeof(float) * samples);
  for (int i = 0; i < pad; i++) {
    padded[i] = padded[2 * pad - i];
    padded[pad + len + i] = padded[pad + len - 2 - i];
  }
  int *glo = (int *)malloc(sizeof(int) * mels), *ghi = (int *)malloc(sizeof(int) * mels);
  for (int m = 0; m < mels; m++) { /* 4-bin groups below bin 200 (src/whisper/frontend.rs:34-39) */
    const float *f = filters + m * WS_BINS;
    int a = 0, b = 0;
    while (a < WS_BINS && f[a] == 0.0f) a++;
    if (a == WS_BINS) a = 0;
    for (int k = WS_BINS - 1; k >= 0; k--)
      if (f[k] != 0.0f) {
        b = k / 4 + 1;
        break;
      }
    a /= 4;
    const int top = (WS_BINS - 1) / 4;
    b = b < a ? a : b > top ? top : b;
    glo[m] = a, ghi[m] = b;
  }
  const float silent = (float)log10(1e-10);
  fft_plan p;
  fft_plan_init(&p, WS_FFT);
  float frame[WS_FFT], buf[4 * WS_FFT];
  double power[WS_BINS];
  for (int t = 0; t < frames; t++) {
    const float *x = padded + (size_t)t * WS_HOP;
    int zero = 1;
    for (int i = 0; i < WS_FFT; i++) zero &= x[i] == 0.0f;
    if (zero) {
      for (int m = 0; m < mels; m++) out[(size_t)t * mels + m] = g_raw ? 0.0f : silent;
      continue;
    }
    for (int i = 0; i < WS_FFT; i++) frame[i] = x[i] * window[i];
    fft_forward32(&p, frame, buf);
    for (int k = 0; k < WS_BINS; k++) {
      const float re = buf[k], im = buf[WS_FFT + k];
      power[k] = (double)fmaf(re, re, im * im);
    }
    for (int m = 0; m < mels; m++) {
      const float *f = filters + m * WS_BINS;
      double sum = 0.0;
#define W(k) ((double)f[k] * power[k])
      for (int g = glo[m]; g < ghi[m]; g++) sum += ((W(4 * g) + W(4 * g + 1)) + W(4 * g + 2)) + W(4 * g + 3);
      sum += W(WS_BINS - 1);
#undef W
      out[(size_t)t * mels + m] = g_raw ? (float)sum : (float)log10(sum > 1e-10 ? sum : 1e-10);
    }
  }
  if (g_raw) {
    fft_plan_free(&p);
    free(padded), free(glo), free(ghi);
    return frames;
  }
  float mx = -INFINITY;
  for (size_t i = 0; i < (size_t)frames * mels; i++) mx = out[i] > mx ? out[i] : mx;
  const double top = (double)mx;
  for (size_t i = 0; i < (size_t)frames * mels; i++) {
    double v = (double)out[i];
    v = v > top - 8.0 ? v : top - 8.0;
    out[i] = (float)((v + 4.0) / 4.0);
  }
  fft_plan_free(&p);
  free(padded);
  free(glo);
  free(ghi);
  return frames;
}
