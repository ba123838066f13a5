/*
 * Model-level CPU restatement (the parity oracle's encoders and decoders).  TEST INFRASTRUCTURE
 * ONLY: see oracle.h.  A GGUF v3 reader (src/gguf.rs), the Conformer blocks on the CPU
 * (src/cpu/conformer.rs:72-200), the GigaAM encoder (src/gigaam/cpu.rs:23-54), the Parakeet
 * encoder (src/parakeet/cpu.rs:36-174), its TDT greedy decoder (src/parakeet/decoder.rs:91-191),
 * and Whisper's encoder (src/whisper/cpu.rs:40-47, src/cpu/transformer.rs:94-117) and decoder step
 * (src/cpu/transformer.rs:186-266).
 */
#include "oracle.h"

#include <fcntl.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

/* ------------------------------------------------------------------ GGUF v3 (src/gguf.rs:121-181) */

typedef struct {
  const char *name;
  size_t name_len;
  int n_dims;
  size_t dims[4];
  int type;
  size_t offset;
} gg_tensor;

typedef struct {
  const char *key;
  size_t key_len;
  unsigned type;
  const uint8_t *val;
} gg_kv;

typedef struct {
  uint8_t *map;
  size_t len;
  gg_kv *kv;
  size_t n_kv;
  gg_tensor *t;
  size_t n_t;
  size_t data;
} gguf;

typedef struct {
  const uint8_t *p, *end;
  int bad;
} rd;

static uint64_t rd_n(rd *r, int n) {
  if (r->p + n > r->end) {
    r->bad = 1;
    return 0;
  }
  uint64_t v = 0;
  for (int i = 0; i < n; i++) v |= (uint64_t)r->p[i] << (8 * i);
  r->p += n;
  return v;
}

static const char *rd_str(rd *r, size_t *len) {
  *len = (size_t)rd_n(r, 8);
  if (r->bad || r->p + *len > r->end) {
    r->bad = 1;
    return NULL;
  }
  const char *s = (const char *)r->p;
  r->p += *len;
  return s;
}

static size_t scalar_size(unsigned t) {
  static const size_t sz[] = {1, 1, 2, 2, 4, 4, 4, 1, 0, 0, 8, 8, 8};
  return t < 13 ? sz[t] : 0;
}

static void rd_skip(rd *r, unsigned t) {
  if (t == 8) {
    size_t l;
    rd_str(r, &l);
  } else if (t == 9) {
    unsigned it = (unsigned)rd_n(r, 4);
    uint64_t n = rd_n(r, 8);
    for (uint64_t i = 0; i < n && !r->bad; i++) rd_skip(r, it);
  } else {
    size_t s = scalar_size(t);
    if (!s || r->p + s > r->end) r->bad = 1;
    else r->p += s;
  }
}

static void gguf_close(gguf *g) {
  if (g->map) munmap(g->map, g->len);
  free(g->kv);
  free(g->t);
  memset(g, 0, sizeof *g);
}

static int gguf_open(gguf *g, const char *path, char *err, size_t errlen) {
  memset(g, 0, sizeof *g);
  int fd = open(path, O_RDONLY);
  if (fd < 0) {
    snprintf(err, errlen, "cannot open %s", path);
    return -1;
  }
  struct stat st;
  fstat(fd, &st);
  g->len = (size_t)st.st_size;
  g->map = (uint8_t *)mmap(NULL, g->len, PROT_READ, MAP_PRIVATE, fd, 0);
  close(fd);
  if (g->map == MAP_FAILED) {
    g->map = NULL;
    snprintf(err, errlen, "cannot map %s", path);
    return -1;
  }
  rd r = {g->map, g->map + g->len, 0};
  if (g->len < 4 || memcmp(g->map, "GGUF", 4)) {
    snprintf(err, errlen, "not a GGUF file");
    gguf_close(g);
    return -1;
  }
  r.p += 4;
  unsigned version = (unsigned)rd_n(&r, 4);
  if (version != 3) {
    snprintf(err, errlen, "unsupported GGUF version %u", version);
    gguf_close(g);
    return -1;
  }
  g->n_t = (size_t)rd_n(&r, 8);
  g->n_kv = (size_t)rd_n(&r, 8);
  if (g->n_t > (1u << 24) || g->n_kv > (1u << 24)) r.bad = 1;
  g->kv = (gg_kv *)calloc(g->n_kv + 1, sizeof(gg_kv));
  g->t = (gg_tensor *)calloc(g->n_t + 1, sizeof(gg_tensor));
  size_t align = 32;
  for (size_t i = 0; i < g->n_kv && !r.bad; i++) {
    gg_kv *kv = &g->kv[i];
    kv->key = rd_str(&r, &kv->key_len);
    kv->type = (unsigned)rd_n(&r, 4);
    kv->val = r.p;
    if (kv->key_len == 17 && !memcmp(kv->key, "general.alignment", 17) && kv->type == 4) {
      rd v = r;
      align = (size_t)rd_n(&v, 4);
    }
    rd_skip(&r, kv->type);
  }
  for (size_t i = 0; i < g->n_t && !r.bad; i++) {
    gg_tensor *t = &g->t[i];
    t->name = rd_str(&r, &t->name_len);
    t->n_dims = (int)rd_n(&r, 4);
    if (t->n_dims < 1 || t->n_dims > 4) r.bad = 1;
    for (int d = 0; d < t->n_dims && !r.bad; d++) t->dims[d] = (size_t)rd_n(&r, 8);
    t->type = (int)rd_n(&r, 4);
    t->offset = (size_t)rd_n(&r, 8);
  }
  if (r.bad) {
    snprintf(err, errlen, "truncated GGUF header");
    gguf_close(g);
    return -1;
  }
  size_t end = (size_t)(r.p - g->map);
  g->data = (end + align - 1) / align * align;
  for (size_t i = 0; i < g->n_t; i++) {
    gg_tensor *t = &g->t[i];
    size_t n = 1;
    for (int d = 0; d < t->n_dims; d++) n *= t->dims[d];
    size_t size = ox_type_size(t->type, n);
    if (!size || g->data + t->offset + size > g->len) {
      snprintf(err, errlen, "tensor %.*s is out of file bounds or of an unsupported type",
               (int)t->name_len, t->name);
      gguf_close(g);
      return -1;
    }
  }
  return 0;
}

static const gg_kv *gg_find(const gguf *g, const char *key) {
  size_t l = strlen(key);
  for (size_t i = 0; i < g->n_kv; i++)
    if (g->kv[i].key_len == l && !memcmp(g->kv[i].key, key, l)) return &g->kv[i];
  return NULL;
}

static long gg_int(const gguf *g, const char *key, long dflt) {
  const gg_kv *kv = gg_find(g, key);
  if (!kv) return dflt;
  rd r = {kv->val, g->map + g->len, 0};
  switch (kv->type) {
    case 0: return (long)rd_n(&r, 1);
    case 1: return (long)(int8_t)rd_n(&r, 1);
    case 2: return (long)rd_n(&r, 2);
    case 3: return (long)(int16_t)rd_n(&r, 2);
    case 4: return (long)(uint32_t)rd_n(&r, 4);
    case 5: return (long)(int32_t)rd_n(&r, 4);
    case 7: return (long)rd_n(&r, 1);
    case 10: case 11: return (long)rd_n(&r, 8);
  }
  return dflt;
}

static double gg_float(const gguf *g, const char *key, double dflt) {
  const gg_kv *kv = gg_find(g, key);
  if (!kv) return dflt;
  rd r = {kv->val, g->map + g->len, 0};
  if (kv->type == 6) {
    uint32_t u = (uint32_t)rd_n(&r, 4);
    float f;
    memcpy(&f, &u, 4);
    return f;
  }
  if (kv->type == 12) {
    uint64_t u = rd_n(&r, 8);
    double d;
    memcpy(&d, &u, 8);
    return d;
  }
  return (double)gg_int(g, key, (long)dflt);
}

static int gg_streq(const gguf *g, const char *key, const char *want) {
  const gg_kv *kv = gg_find(g, key);
  if (!kv || kv->type != 8) return 0;
  rd r = {kv->val, g->map + g->len, 0};
  size_t l;
  const char *s = rd_str(&r, &l);
  return s && l == strlen(want) && !memcmp(s, want, l);
}

/* Integer array items (i32 arrays: TDT durations, suppress lists). */
static int gg_int_array(const gguf *g, const char *key, int *out, int cap) {
  const gg_kv *kv = gg_find(g, key);
  if (!kv || kv->type != 9) return -1;
  rd r = {kv->val, g->map + g->len, 0};
  unsigned it = (unsigned)rd_n(&r, 4);
  uint64_t n = rd_n(&r, 8);
  size_t s = scalar_size(it);
  if (!s || s > 8) return -1;
  for (uint64_t i = 0; i < n && (int)i < cap; i++) {
    uint64_t v = rd_n(&r, (int)s);
    out[i] = s == 4 ? (int)(int32_t)v : (int)v;
  }
  return (int)n;
}

static const gg_tensor *gg_tensor_find(const gguf *g, const char *name) {
  size_t l = strlen(name);
  for (size_t i = 0; i < g->n_t; i++)
    if (g->t[i].name_len == l && !memcmp(g->t[i].name, name, l)) return &g->t[i];
  return NULL;
}

static const uint8_t *gg_data(const gguf *g, const gg_tensor *t) { return g->map + g->data + t->offset; }

static size_t gg_count(const gg_tensor *t) {
  size_t n = 1;
  for (int d = 0; d < t->n_dims; d++) n *= t->dims[d];
  return n;
}

/* ------------------------------------------------------------------------------ model loading */

typedef struct {
  char err[256];
  gguf *g;
} loader;

static const gg_tensor *need(loader *L, const char *name) {
  const gg_tensor *t = gg_tensor_find(L->g, name);
  if (!t && !L->err[0]) snprintf(L->err, sizeof L->err, "missing tensor %.200s", name);
  return t;
}

static float *f32s(loader *L, const char *name, size_t want) {
  const gg_tensor *t = need(L, name);
  if (!t) return NULL;
  size_t n = gg_count(t);
  if (want && n != want) {
    if (!L->err[0]) snprintf(L->err, sizeof L->err, "tensor %s has %zu values, expected %zu", name, n, want);
    return NULL;
  }
  float *o = (float *)malloc(sizeof(float) * n);
  ox_dequant(t->type, gg_data(L->g, t), o, n);
  return o;
}

/* Linear layer over `count` stacked tensors (src/cpu/gemm.rs:45-72): weights named `names[i]` +
 * ".weight", biases ".bias" when bias (NULL name = zeros, as Whisper's k). */
static ox_linear *linear_n(loader *L, const char *const *names, int count, int bias, int zero_idx) {
  const void *ws[4];
  int rows[4], type = -1, k = -1, n = 0;
  char buf[256];
  for (int i = 0; i < count; i++) {
    snprintf(buf, sizeof buf, "%s.weight", names[i]);
    const gg_tensor *t = need(L, buf);
    if (!t) return NULL;
    int tk = (int)t->dims[0];
    for (int d = 1; d < t->n_dims - 1; d++) tk *= (int)t->dims[d];
    if (type >= 0 && (t->type != type || tk != k)) {
      snprintf(L->err, sizeof L->err, "stacked weights differ in type or shape");
      return NULL;
    }
    type = t->type;
    k = tk;
    rows[i] = (int)t->dims[t->n_dims - 1];
    n += rows[i];
    ws[i] = gg_data(L->g, t);
  }
  float *b = NULL;
  if (bias) {
    b = (float *)calloc((size_t)n, sizeof(float));
    int at = 0;
    for (int i = 0; i < count; i++) {
      if (i != zero_idx) {
        snprintf(buf, sizeof buf, "%s.bias", names[i]);
        float *bi = f32s(L, buf, (size_t)rows[i]);
        if (!bi) {
          free(b);
          return NULL;
        }
        memcpy(b + at, bi, sizeof(float) * rows[i]);
        free(bi);
      }
      at += rows[i];
    }
  }
  ox_linear *l = ox_linear_new(type, k, count, ws, rows, b);
  free(b);
  if (!l && !L->err[0]) snprintf(L->err, sizeof L->err, "bad linear layer %s", names[0]);
  return l;
}

/* A matrix stored under its exact tensor name (no ".weight"), without a bias. */
static ox_linear *matrix(loader *L, const char *tensor) {
  const gg_tensor *t = need(L, tensor);
  if (!t) return NULL;
  int k = (int)t->dims[0], rows = (int)t->dims[t->n_dims - 1];
  const void *ws[1] = {gg_data(L->g, t)};
  ox_linear *l = ox_linear_new(t->type, k, 1, ws, &rows, NULL);
  if (!l && !L->err[0]) snprintf(L->err, sizeof L->err, "bad matrix %s", tensor);
  return l;
}

static ox_linear *linear1(loader *L, const char *name, int bias) {
  const char *names[1] = {name};
  return linear_n(L, names, 1, bias, -1);
}

/* ------------------------------------------------------------------------------- Conformer */

typedef struct {
  float *w, *b;
} chan;

typedef struct {
  chan norm_ff1, norm_attn, norm_conv, norm_ff2, norm_out, conv_norm, dw;
  ox_linear *ff1[2], *ff2[2], *out, *pw1, *pw2;
  ox_linear *qk, *v;            /* rotary */
  ox_linear *qkv, *pos;         /* relative */
  float *u, *vb;                /* relative [heads][hd] */
} block;

enum { ARCH_GIGAAM = 0, ARCH_PARAKEET = 1, ARCH_WHISPER = 2 };

typedef struct {
  chan norm_self, norm_cross, norm_ffn;
  ox_linear *qkv, *self_out, *cross_q, *cross_kv, *cross_out, *fc1, *fc2;
} dec_layer;

struct ox_model {
  int arch;
  gguf g;
  /* Conformer config (src/conformer.rs:34-61). */
  int layers, d, heads, d_ff, kernel, layer_norm_conv, relative, bias;
  block *blocks;
  int mels;
  /* GigaAM */
  double theta;
  ox_linear *conv0, *conv2, *head;
  /* Parakeet subsampling */
  int ch;
  chan sc0, sc2, sc5;
  ox_linear *conv3, *conv6, *pre_out, *joint_enc;
  /* Parakeet TDT decoder */
  int hidden, joint, classes, blank, n_dur, max_symbols, global, lstm_layers;
  int durations[16];
  ox_linear *embed, *pred_w, *out_w;
  ox_linear **wx, **wh;
  float **lstm_b, *pred_b, *out_b;
  /* Whisper */
  int frames, dec_layers, dec_heads, dec_ff, vocab, context;
  float *enc_pos, *dec_pos;
  ox_linear *wconv0, *wconv1;
  chan enc_norm, dec_norm;
  struct {
    chan norm_attn, norm_ffn;
    ox_linear *qkv, *out, *fc1, *fc2;
  } *wblocks;
  dec_layer *dl;
  ox_linear *token_embd;
  /* Whisper decoding caches (src/cpu/transformer.rs:146-223): per layer K then V. */
  float **own, **cross;
  int cross_frames;
  /* Whisper's special ids and suppression lists (src/whisper/mod.rs:131-141, :177). */
  int eot, no_timestamps, sot, n_suppress, n_begin_suppress;
  int suppress[512], begin_suppress[64];
};

static chan norm(loader *L, const char *name, int d, int bias) {
  char buf[256];
  chan c = {0, 0};
  snprintf(buf, sizeof buf, "%s.weight", name);
  c.w = f32s(L, buf, (size_t)d);
  if (bias) {
    snprintf(buf, sizeof buf, "%s.bias", name);
    c.b = f32s(L, buf, (size_t)d);
  } else {
    c.b = (float *)calloc((size_t)d, sizeof(float));
  }
  return c;
}

static void block_load(loader *L, ox_model *m, int i, block *k) {
  char p[128], b1[192], b2[192], b3[192];
  int d = m->d;
#define P(s) (snprintf(p, sizeof p, "enc.blocks.%d.%s", i, s), p)
  k->norm_ff1 = norm(L, P("norm_ff1"), d, 1);
  k->ff1[0] = linear1(L, P("ff1.linear1"), m->bias);
  k->ff1[1] = linear1(L, P("ff1.linear2"), m->bias);
  k->norm_attn = norm(L, P("norm_attn"), d, 1);
  snprintf(b1, sizeof b1, "enc.blocks.%d.attn.linear_q", i);
  snprintf(b2, sizeof b2, "enc.blocks.%d.attn.linear_k", i);
  snprintf(b3, sizeof b3, "enc.blocks.%d.attn.linear_v", i);
  if (!m->relative) {
    const char *qk[2] = {b1, b2};
    k->qk = linear_n(L, qk, 2, m->bias, -1);
    k->v = linear1(L, b3, m->bias);
  } else {
    const char *qkv[3] = {b1, b2, b3};
    k->qkv = linear_n(L, qkv, 3, m->bias, -1);
    k->pos = linear1(L, P("attn.linear_pos"), 0);
    k->u = f32s(L, P("attn.pos_bias_u"), (size_t)d);
    k->vb = f32s(L, P("attn.pos_bias_v"), (size_t)d);
  }
  k->out = linear1(L, P("attn.linear_out"), m->bias);
  k->norm_conv = norm(L, P("norm_conv"), d, 1);
  k->pw1 = linear1(L, P("conv.pointwise1"), m->bias);
  if (m->layer_norm_conv) {
    k->conv_norm = norm(L, P("conv.ln"), d, 1);
  } else {
    float *bw = f32s(L, P("conv.bn.weight"), (size_t)d), *bb = f32s(L, P("conv.bn.bias"), (size_t)d);
    float *mean = f32s(L, P("conv.bn.running_mean"), (size_t)d);
    float *var = f32s(L, P("conv.bn.running_var"), (size_t)d);
    k->conv_norm.w = (float *)malloc(sizeof(float) * d);
    k->conv_norm.b = (float *)malloc(sizeof(float) * d);
    if (bw && bb && mean && var) ox_batch_norm(bw, bb, mean, var, d, k->conv_norm.w, k->conv_norm.b);
    free(bw);
    free(bb);
    free(mean);
    free(var);
  }
  /* [d][kernel] in the file, [kernel][d] here (src/cpu/conformer.rs:124-126). */
  float *w = f32s(L, P("conv.depthwise.weight"), (size_t)d * m->kernel);
  k->dw.w = (float *)malloc(sizeof(float) * (size_t)d * m->kernel);
  if (w)
    for (int t = 0; t < m->kernel; t++)
      for (int c = 0; c < d; c++) k->dw.w[t * d + c] = w[c * m->kernel + t];
  free(w);
  k->dw.b = m->bias ? f32s(L, P("conv.depthwise.bias"), (size_t)d) : (float *)calloc((size_t)d, 4);
  k->pw2 = linear1(L, P("conv.pointwise2"), m->bias);
  k->norm_ff2 = norm(L, P("norm_ff2"), d, 1);
  k->ff2[0] = linear1(L, P("ff2.linear1"), m->bias);
  k->ff2[1] = linear1(L, P("ff2.linear2"), m->bias);
  k->norm_out = norm(L, P("norm_out"), d, 1);
#undef P
}

/* Block::run (src/cpu/conformer.rs:159-200): from x into y; x is scratch. */
static void block_run(const ox_model *m, const block *k, float *x, float *y, float *h, float *qk,
                      float *yr, int t, const float *pos, int valid) {
  int d = m->d, hd = d / m->heads;
  ox_layer_norm(x, k->norm_ff1.w, k->norm_ff1.b, y, t, d, NULL, NULL, 0);
  ox_gemm(y, k->ff1[0], h, t, OX_SILU, 0);
  ox_gemm(h, k->ff1[1], x, t, OX_RESIDUAL, 0.5f);
  if (!m->relative) {
    ox_layer_norm(x, k->norm_attn.w, k->norm_attn.b, y, t, d, pos, yr, hd);
    ox_gemm(yr, k->qk, qk, t, OX_BIAS, 0);
    ox_gemm(y, k->v, h, t, OX_BIAS, 0);
    ox_attention(qk, 2 * d, h, d, y, t, m->heads, hd, valid);
  } else {
    int pr = 2 * t + 15;
    ox_layer_norm(x, k->norm_attn.w, k->norm_attn.b, y, t, d, NULL, NULL, 0);
    ox_gemm(y, k->qkv, qk, t, OX_BIAS, 0);
    ox_gemm(pos, k->pos, yr, pr, OX_BIAS, 0);
    ox_relative_attention(qk, yr, k->u, k->vb, y, t, m->heads, hd, valid);
  }
  ox_gemm(y, k->out, x, t, OX_RESIDUAL, 1.0f);
  ox_layer_norm(x, k->norm_conv.w, k->norm_conv.b, y, t, d, NULL, NULL, 0);
  ox_gemm(y, k->pw1, qk, t, OX_BIAS, 0);
  ox_conv_glu(qk, k->dw.w, k->dw.b, m->kernel, k->conv_norm.w, k->conv_norm.b, m->layer_norm_conv,
              y, t, d, valid);
  ox_gemm(y, k->pw2, x, t, OX_RESIDUAL, 1.0f);
  ox_layer_norm(x, k->norm_ff2.w, k->norm_ff2.b, y, t, d, NULL, NULL, 0);
  ox_gemm(y, k->ff2[0], h, t, OX_SILU, 0);
  ox_gemm(h, k->ff2[1], x, t, OX_RESIDUAL, 0.5f);
  ox_layer_norm(x, k->norm_out.w, k->norm_out.b, y, t, d, NULL, NULL, 0);
}

/* Conformer::run (src/cpu/conformer.rs:72-91) over x [t][d] in place, `layers` blocks. */
static void conformer_run(const ox_model *m, float *x, int t, const float *pos, int layers, int valid) {
  int d = m->d;
  size_t hsz = (size_t)t * (m->d_ff > d ? m->d_ff : d);
  float *y = (float *)malloc(sizeof(float) * (size_t)t * d);
  float *h = (float *)malloc(sizeof(float) * hsz);
  float *qk = (float *)malloc(sizeof(float) * (size_t)t * 3 * d);
  float *yr = (float *)malloc(sizeof(float) * (size_t)(2 * t + 15) * d);
  float *cur = x, *nxt = y;
  for (int i = 0; i < layers; i++) {
    block_run(m, &m->blocks[i], cur, nxt, h, qk, yr, t, pos, valid);
    float *s = cur;
    cur = nxt;
    nxt = s;
  }
  if (cur != x) memcpy(x, cur, sizeof(float) * (size_t)t * d);
  free(cur == x ? nxt : cur);
  free(h);
  free(qk);
  free(yr);
}

static int half_len(int n) { return (n - 1) / 2 + 1; }

/* The positional table of a call over t frames. */
static float *positions(const ox_model *m, int t) {
  int hd = m->d / m->heads;
  if (!m->relative) {
    float *p = (float *)malloc(sizeof(float) * (size_t)t * hd);
    ox_rope_table(t, hd, m->theta, p);
    return p;
  }
  float *p = (float *)malloc(sizeof(float) * (size_t)(2 * t + 15) * m->d);
  ox_rel_positions(m->d, (long)t + 15, 2 * t + 15, p);
  return p;
}

/* ------------------------------------------------------------------------------ load */

static int conformer_config(loader *L, ox_model *m, const char *arch) {
  char k[160];
#define U(name) (snprintf(k, sizeof k, "stt.%s.encoder.%s", arch, name), gg_int(L->g, k, -1))
  m->layers = (int)U("n_layers");
  m->d = (int)U("d_model");
  m->heads = (int)U("n_heads");
  m->d_ff = (int)U("d_ff");
  m->kernel = (int)U("conv_kernel");
  snprintf(k, sizeof k, "stt.%s.encoder.conv_norm_type", arch);
  m->layer_norm_conv = gg_streq(L->g, k, "layer_norm");
  if (!m->layer_norm_conv && !gg_streq(L->g, k, "batch_norm")) {
    snprintf(L->err, sizeof L->err, "unsupported conv_norm_type");
    return -1;
  }
#undef U
  int d = m->d, heads = m->heads;
  if (m->layers <= 0 || d <= 0 || heads <= 0 || d % heads || d > 1024 || d / heads > 128 ||
      (d / heads) % 2 || m->kernel % 2 == 0) {
    snprintf(L->err, sizeof L->err, "unsupported attention shape: d_model %d, %d heads", d, heads);
    return -1;
  }
  return 0;
}

static int load_conformer_blocks(loader *L, ox_model *m) {
  m->blocks = (block *)calloc((size_t)m->layers, sizeof(block));
  for (int i = 0; i < m->layers && !L->err[0]; i++) block_load(L, m, i, &m->blocks[i]);
  return L->err[0] ? -1 : 0;
}

static int load_gigaam(loader *L, ox_model *m) {
  if (!gg_streq(L->g, "stt.gigaam.encoder.self_attention_model", "rotary")) {
    snprintf(L->err, sizeof L->err, "stt.gigaam.encoder.self_attention_model must be rotary");
    return -1;
  }
  m->relative = 0;
  m->bias = 1;
  if (conformer_config(L, m, "gigaam")) return -1;
  m->mels = (int)gg_int(L->g, "stt.frontend.num_mels", -1);
  m->theta = (double)gg_int(L->g, "stt.gigaam.encoder.pos_emb_max_len", 5000);
  m->conv0 = linear1(L, "enc.pre_encode.conv.0", 1);
  m->conv2 = linear1(L, "enc.pre_encode.conv.2", 1);
  m->head = gg_streq(L->g, "stt.gigaam.head_kind", "rnnt") ? linear1(L, "joint.enc", 1)
                                                           : linear1(L, "head.ctc", 1);
  m->blank = (int)gg_int(L->g, "tokenizer.ggml.blank_token_id", -1);
  return load_conformer_blocks(L, m);
}

static chan taps3(loader *L, int i, int ch) {
  char buf[128];
  chan c = {0, 0};
  snprintf(buf, sizeof buf, "enc.pre_encode.conv.%d.weight", i);
  float *w = f32s(L, buf, (size_t)9 * ch);
  snprintf(buf, sizeof buf, "enc.pre_encode.conv.%d.bias", i);
  c.b = f32s(L, buf, (size_t)ch);
  /* [ch][time tap][freq tap] -> [tap][ch] (src/parakeet/cpu.rs:41-45). */
  c.w = (float *)malloc(sizeof(float) * 9 * (size_t)ch);
  if (w)
    for (int e = 0; e < 9 * ch; e++) c.w[e] = w[(e % ch) * 9 + e / ch];
  free(w);
  return c;
}

static int load_parakeet(loader *L, ox_model *m) {
  m->relative = 1;
  m->bias = 0;
  if (conformer_config(L, m, "parakeet")) return -1;
  m->mels = (int)gg_int(L->g, "stt.frontend.num_mels", -1);
  m->ch = (int)gg_int(L->g, "stt.parakeet.encoder.subsampling_channels", -1);
  m->sc0 = taps3(L, 0, m->ch);
  m->sc2 = taps3(L, 2, m->ch);
  m->sc5 = taps3(L, 5, m->ch);
  m->conv3 = linear1(L, "enc.pre_encode.conv.3", 1);
  m->conv6 = linear1(L, "enc.pre_encode.conv.6", 1);
  m->pre_out = linear1(L, "enc.pre_encode.out", 1);
  m->joint_enc = linear1(L, "joint.enc", 1);
  if (load_conformer_blocks(L, m)) return -1;
  /* TDT decoder (src/parakeet/decoder.rs:46-89). */
  m->hidden = (int)gg_int(L->g, "stt.parakeet.predictor.hidden", -1);
  m->joint = (int)gg_int(L->g, "stt.parakeet.joint.hidden", -1);
  m->blank = (int)gg_int(L->g, "tokenizer.ggml.blank_token_id", -1);
  m->max_symbols = (int)gg_int(L->g, "stt.parakeet.tdt.max_symbols", 10);
  m->global = gg_streq(L->g, "stt.parakeet.tdt.symbol_budget", "global");
  m->n_dur = gg_int_array(L->g, "stt.parakeet.tdt.durations", m->durations, 16);
  m->lstm_layers = (int)gg_int(L->g, "stt.parakeet.predictor.n_layers", 1);
  if (gg_tensor_find(L->g, "pred.embed.weight") && m->n_dur > 0 && m->n_dur <= 16) {
    m->embed = linear1(L, "pred.embed", 0);
    m->classes = m->embed ? m->embed->n : 0;
    m->wx = (ox_linear **)calloc((size_t)m->lstm_layers, sizeof(void *));
    m->wh = (ox_linear **)calloc((size_t)m->lstm_layers, sizeof(void *));
    m->lstm_b = (float **)calloc((size_t)m->lstm_layers, sizeof(void *));
    char buf[128];
    for (int l = 0; l < m->lstm_layers; l++) {
      snprintf(buf, sizeof buf, "pred.lstm.%d.Wx", l);
      m->wx[l] = matrix(L, buf);
      snprintf(buf, sizeof buf, "pred.lstm.%d.Wh", l);
      m->wh[l] = matrix(L, buf);
      snprintf(buf, sizeof buf, "pred.lstm.%d.bias", l);
      m->lstm_b[l] = f32s(L, buf, (size_t)4 * m->hidden);
    }
    m->pred_w = linear1(L, "joint.pred", 0);
    m->pred_b = f32s(L, "joint.pred.bias", (size_t)m->joint);
    m->out_w = linear1(L, "joint.out", 0);
    m->out_b = f32s(L, "joint.out.bias", (size_t)(m->classes + m->n_dur));
  }
  return L->err[0] ? -1 : 0;
}

static int load_whisper(loader *L, ox_model *m) {
  m->d = (int)gg_int(L->g, "stt.whisper.encoder.d_model", -1);
  m->heads = (int)gg_int(L->g, "stt.whisper.encoder.n_heads", -1);
  m->layers = (int)gg_int(L->g, "stt.whisper.encoder.n_layers", -1);
  m->d_ff = (int)gg_int(L->g, "stt.whisper.encoder.ffn_dim", -1);
  m->dec_heads = (int)gg_int(L->g, "stt.whisper.decoder.n_heads", -1);
  m->dec_layers = (int)gg_int(L->g, "stt.whisper.decoder.n_layers", -1);
  m->dec_ff = (int)gg_int(L->g, "stt.whisper.decoder.ffn_dim", -1);
  m->vocab = (int)gg_int(L->g, "stt.whisper.decoder.vocab_size", -1);
  m->context = (int)gg_int(L->g, "stt.whisper.decoder.max_target_positions", -1);
  m->mels = (int)gg_int(L->g, "stt.whisper.encoder.num_mel_bins", -1);
  m->frames = (int)gg_int(L->g, "stt.whisper.encoder.max_source_positions", 1500);
  int d = m->d;
  if (d <= 0 || m->heads <= 0 || d % m->heads || d / m->heads > 64 || (d / m->heads) % 8) {
    snprintf(L->err, sizeof L->err, "unsupported shape: d_model %d, %d heads", d, m->heads);
    return -1;
  }
  m->wconv0 = linear1(L, "enc.conv.0", 1);
  m->wconv1 = linear1(L, "enc.conv.1", 1);
  m->enc_pos = f32s(L, "enc.pos_emb.weight", (size_t)d * m->frames);
  m->wblocks = calloc((size_t)m->layers, sizeof *m->wblocks);
  char p[160], q[160], k[160], v[160];
  for (int i = 0; i < m->layers && !L->err[0]; i++) {
#define P(s) (snprintf(p, sizeof p, "enc.blocks.%d.%s", i, s), p)
    m->wblocks[i].norm_attn = norm(L, P("norm_attn"), d, 1);
    snprintf(q, sizeof q, "enc.blocks.%d.attn.q", i);
    snprintf(k, sizeof k, "enc.blocks.%d.attn.k", i);
    snprintf(v, sizeof v, "enc.blocks.%d.attn.v", i);
    const char *qkv[3] = {q, k, v};
    m->wblocks[i].qkv = linear_n(L, qkv, 3, 1, 1);
    m->wblocks[i].out = linear1(L, P("attn.out"), 1);
    m->wblocks[i].norm_ffn = norm(L, P("norm_ffn"), d, 1);
    m->wblocks[i].fc1 = linear1(L, P("ffn.fc1"), 1);
    m->wblocks[i].fc2 = linear1(L, P("ffn.fc2"), 1);
#undef P
  }
  m->enc_norm = norm(L, "enc.final_norm", d, 1);
  m->dl = (dec_layer *)calloc((size_t)m->dec_layers, sizeof(dec_layer));
  for (int i = 0; i < m->dec_layers && !L->err[0]; i++) {
    dec_layer *l = &m->dl[i];
#define P(s) (snprintf(p, sizeof p, "dec.blocks.%d.%s", i, s), p)
    l->norm_self = norm(L, P("norm_self"), d, 1);
    snprintf(q, sizeof q, "dec.blocks.%d.self_attn.q", i);
    snprintf(k, sizeof k, "dec.blocks.%d.self_attn.k", i);
    snprintf(v, sizeof v, "dec.blocks.%d.self_attn.v", i);
    const char *qkv[3] = {q, k, v};
    l->qkv = linear_n(L, qkv, 3, 1, 1);
    l->self_out = linear1(L, P("self_attn.out"), 1);
    l->norm_cross = norm(L, P("norm_cross"), d, 1);
    l->cross_q = linear1(L, P("cross_attn.q"), 1);
    snprintf(k, sizeof k, "dec.blocks.%d.cross_attn.k", i);
    snprintf(v, sizeof v, "dec.blocks.%d.cross_attn.v", i);
    const char *kv[2] = {k, v};
    /* stacked(k, v): k has no bias (src/cpu/transformer.rs:28-38). */
    l->cross_kv = linear_n(L, kv, 2, 1, 0);
    l->cross_out = linear1(L, P("cross_attn.out"), 1);
    l->norm_ffn = norm(L, P("norm_ffn"), d, 1);
    l->fc1 = linear1(L, P("ffn.fc1"), 1);
    l->fc2 = linear1(L, P("ffn.fc2"), 1);
#undef P
  }
  m->dec_norm = norm(L, "dec.final_norm", d, 1);
  m->eot = (int)gg_int(L->g, "tokenizer.ggml.eos_token_id", -1);
  m->no_timestamps = (int)gg_int(L->g, "stt.whisper.no_timestamps_token_id", -1);
  m->sot = (int)gg_int(L->g, "stt.whisper.sot_token_id", -1);
  /* Optional lists: the converter writes them only when not empty (src/whisper/mod.rs:131-133). */
  m->n_suppress = gg_int_array(L->g, "stt.whisper.suppress_tokens", m->suppress, 512);
  m->n_begin_suppress = gg_int_array(L->g, "stt.whisper.begin_suppress_tokens", m->begin_suppress, 64);
  if (m->n_suppress < 0) m->n_suppress = 0;
  if (m->n_begin_suppress < 0) m->n_begin_suppress = 0;
  if (m->n_suppress > 512 || m->n_begin_suppress > 64 || m->eot < 0 || m->no_timestamps < 0 ||
      m->no_timestamps + 1 >= m->vocab) {
    snprintf(L->err, sizeof L->err, "bad Whisper special token ids");
    return -1;
  }
  for (int i = 0; i < m->n_suppress + m->n_begin_suppress; i++) {
    int id = i < m->n_suppress ? m->suppress[i] : m->begin_suppress[i - m->n_suppress];
    if (id < 0 || id >= m->vocab) {
      snprintf(L->err, sizeof L->err, "special token ids out of the vocabulary");
      return -1;
    }
  }
  m->token_embd = linear1(L, "dec.token_embd", 0);
  m->dec_pos = f32s(L, "dec.pos_emb.weight", (size_t)d * m->context);
  return L->err[0] ? -1 : 0;
}

ox_model *ox_model_load(const char *path, char *err, size_t errlen) {
  ox_model *m = (ox_model *)calloc(1, sizeof *m);
  if (gguf_open(&m->g, path, err, errlen)) {
    free(m);
    return NULL;
  }
  loader L;
  memset(&L, 0, sizeof L);
  L.g = &m->g;
  int rc;
  if (gg_streq(&m->g, "general.architecture", "gigaam")) {
    m->arch = ARCH_GIGAAM;
    rc = load_gigaam(&L, m);
  } else if (gg_streq(&m->g, "general.architecture", "parakeet")) {
    m->arch = ARCH_PARAKEET;
    rc = load_parakeet(&L, m);
  } else if (gg_streq(&m->g, "general.architecture", "whisper")) {
    m->arch = ARCH_WHISPER;
    rc = load_whisper(&L, m);
  } else {
    snprintf(L.err, sizeof L.err, "unsupported general.architecture");
    rc = -1;
  }
  if (rc) {
    snprintf(err, errlen, "%s", L.err);
    ox_model_free(m);
    return NULL;
  }
  return m;
}

static void chan_free(chan *c) {
  free(c->w);
  free(c->b);
}

void ox_model_free(ox_model *m) {
  if (!m) return;
  for (int i = 0; m->blocks && i < m->layers; i++) {
    block *k = &m->blocks[i];
    chan_free(&k->norm_ff1), chan_free(&k->norm_attn), chan_free(&k->norm_conv);
    chan_free(&k->norm_ff2), chan_free(&k->norm_out), chan_free(&k->conv_norm), chan_free(&k->dw);
    ox_linear *ls[] = {k->ff1[0], k->ff1[1], k->ff2[0], k->ff2[1], k->out, k->pw1, k->pw2,
                       k->qk, k->v, k->qkv, k->pos};
    for (size_t j = 0; j < sizeof ls / sizeof *ls; j++) ox_linear_free(ls[j]);
    free(k->u);
    free(k->vb);
  }
  free(m->blocks);
  ox_linear *ls[] = {m->conv0, m->conv2, m->head, m->conv3, m->conv6, m->pre_out, m->joint_enc,
                     m->embed, m->pred_w, m->out_w, m->wconv0, m->wconv1, m->token_embd};
  for (size_t j = 0; j < sizeof ls / sizeof *ls; j++) ox_linear_free(ls[j]);
  chan_free(&m->sc0), chan_free(&m->sc2), chan_free(&m->sc5);
  for (int l = 0; m->wx && l < m->lstm_layers; l++) {
    ox_linear_free(m->wx[l]);
    ox_linear_free(m->wh[l]);
    free(m->lstm_b[l]);
  }
  free(m->wx), free(m->wh), free(m->lstm_b), free(m->pred_b), free(m->out_b);
  for (int i = 0; m->wblocks && i < m->layers; i++) {
    chan_free(&m->wblocks[i].norm_attn), chan_free(&m->wblocks[i].norm_ffn);
    ox_linear_free(m->wblocks[i].qkv), ox_linear_free(m->wblocks[i].out);
    ox_linear_free(m->wblocks[i].fc1), ox_linear_free(m->wblocks[i].fc2);
  }
  free(m->wblocks);
  for (int i = 0; m->dl && i < m->dec_layers; i++) {
    dec_layer *l = &m->dl[i];
    chan_free(&l->norm_self), chan_free(&l->norm_cross), chan_free(&l->norm_ffn);
    ox_linear *dls[] = {l->qkv, l->self_out, l->cross_q, l->cross_kv, l->cross_out, l->fc1, l->fc2};
    for (size_t j = 0; j < sizeof dls / sizeof *dls; j++) ox_linear_free(dls[j]);
  }
  free(m->dl);
  chan_free(&m->enc_norm), chan_free(&m->dec_norm);
  free(m->enc_pos), free(m->dec_pos);
  for (int i = 0; m->own && i < m->dec_layers; i++) free(m->own[i]), free(m->cross[i]);
  free(m->own), free(m->cross);
  gguf_close(&m->g);
  free(m);
}

int ox_model_info(ox_model *m, int *arch, int *d, int *layers, int *mels, int *width) {
  *arch = m->arch;
  *d = m->d;
  *layers = m->layers;
  *mels = m->mels;
  switch (m->arch) {
    case ARCH_GIGAAM: *width = m->head->n; break;
    case ARCH_PARAKEET: *width = m->joint_enc->n; break;
    default: *width = m->d;
  }
  return 0;
}

int ox_model_blocks(ox_model *m, float *x, int t, int layers) {
  if (m->arch == ARCH_WHISPER || layers > m->layers) return -1;
  float *pos = positions(m, t);
  conformer_run(m, x, t, pos, layers, t);
  free(pos);
  return 0;
}

/* Encoder frames of Parakeet (src/parakeet/mod.rs:44-46). */
static int parakeet_frames(int mel_frames) { return half_len(half_len(half_len(mel_frames - 1))); }

/* Whisper encoder (src/whisper/cpu.rs:40-47 and src/cpu/transformer.rs:94-117). */
static void whisper_encode(ox_model *m, const float *mel, float *out) {
  int t = m->frames, d = m->d, mels = m->mels, hd = d / m->heads;
  int k0 = 3 * mels, k1 = 3 * d;
  float *col = (float *)malloc(sizeof(float) * (size_t)2 * t * (k0 > k1 ? k0 : k1));
  float *h = (float *)malloc(sizeof(float) * (size_t)2 * t * d);
  ox_im2col(mel, 2 * t, mels, 3, 1, 1, col, k0);
  ox_gemm(col, m->wconv0, h, 2 * t, OX_GELU, 0);
  float *x = (float *)malloc(sizeof(float) * (size_t)t * d);
  memcpy(x, m->enc_pos, sizeof(float) * (size_t)t * d);
  ox_im2col(h, 2 * t, d, 3, 2, 1, col, k1);
  ox_gemm(col, m->wconv1, x, t, OX_GELU_RESIDUAL, 0);
  free(col);
  free(h);
  float *y = (float *)malloc(sizeof(float) * (size_t)t * d);
  float *qkv = (float *)malloc(sizeof(float) * (size_t)t * 3 * d);
  float *hh = (float *)malloc(sizeof(float) * (size_t)t * m->d_ff);
  for (int i = 0; i < m->layers; i++) {
    ox_layer_norm(x, m->wblocks[i].norm_attn.w, m->wblocks[i].norm_attn.b, y, t, d, NULL, NULL, 0);
    ox_gemm(y, m->wblocks[i].qkv, qkv, t, OX_BIAS, 0);
    ox_attention(qkv, 3 * d, qkv + 2 * d, 3 * d, y, t, m->heads, hd, t);
    ox_gemm(y, m->wblocks[i].out, x, t, OX_RESIDUAL, 1.0f);
    ox_layer_norm(x, m->wblocks[i].norm_ffn.w, m->wblocks[i].norm_ffn.b, y, t, d, NULL, NULL, 0);
    ox_gemm(y, m->wblocks[i].fc1, hh, t, OX_GELU, 0);
    ox_gemm(hh, m->wblocks[i].fc2, x, t, OX_RESIDUAL, 1.0f);
  }
  ox_layer_norm(x, m->enc_norm.w, m->enc_norm.b, out, t, d, NULL, NULL, 0);
  free(x);
  free(y);
  free(qkv);
  free(hh);
}

int ox_model_encode(ox_model *m, const float *mel, int mel_frames, int valid, float *out,
                    int *frames_out, int *width_out) {
  if (m->arch == ARCH_GIGAAM) {
    int t1 = half_len(mel_frames), t = half_len(t1), d = m->d, mels = m->mels;
    *frames_out = t;
    *width_out = m->head->n;
    if (!out) return 0;
    int w0 = 5 * mels, w1 = 5 * d;
    float *col = (float *)malloc(sizeof(float) * (size_t)t1 * (w0 > w1 ? w0 : w1));
    float *h = (float *)malloc(sizeof(float) * (size_t)t1 * d);
    ox_im2col(mel, mel_frames, mels, 5, 2, 2, col, w0);
    ox_gemm(col, m->conv0, h, t1, OX_RELU, 0);
    float *x = (float *)malloc(sizeof(float) * (size_t)t * d);
    ox_im2col(h, t1, d, 5, 2, 2, col, w1);
    ox_gemm(col, m->conv2, x, t, OX_RELU, 0);
    free(col);
    free(h);
    float *pos = positions(m, t);
    conformer_run(m, x, t, pos, m->layers, t);
    free(pos);
    ox_gemm(x, m->head, out, t, OX_BIAS, 0);
    free(x);
    return 0;
  }
  if (m->arch == ARCH_WHISPER) {
    *frames_out = m->frames;
    *width_out = m->d;
    if (!out) return 0;
    if (mel_frames != 2 * m->frames) return -1;
    whisper_encode(m, mel, out);
    return 0;
  }
  /* Parakeet (src/parakeet/cpu.rs:66-98). */
  int ch = m->ch, mels = m->mels, d = m->d;
  int t2 = half_len(half_len(mel_frames)), f2 = half_len(half_len(mels));
  int t = parakeet_frames(mel_frames), f = half_len(f2);
  *frames_out = t;
  *width_out = m->joint_enc->n;
  if (!out) return 0;
  const int CHUNK = 64;
  size_t csz = (size_t)(2 * CHUNK + 1) * f2 * ch;
  float *a = (float *)malloc(sizeof(float) * csz), *b = (float *)malloc(sizeof(float) * csz);
  float *h = (float *)malloc(sizeof(float) * (size_t)t * f * ch);
  for (int t0 = 0; t0 < t; t0 += CHUNK) {
    int n = CHUNK < t - t0 ? CHUNK : t - t0, rows = 2 * n + 1;
    ox_sub_first(mel, valid, mels, m->sc0.w, m->sc0.b, m->sc2.w, m->sc2.b, ch, a, rows, t0);
    ox_gemm(a, m->conv3, b, rows * f2, OX_RELU, 0);
    ox_depthwise(b, m->sc5.w, m->sc5.b, t2, f2, ch, h + (size_t)t0 * f * ch, n, t0);
  }
  free(a);
  free(b);
  float *y = (float *)malloc(sizeof(float) * (size_t)t * f * ch);
  ox_gemm(h, m->conv6, y, t * f, OX_RELU, 0);
  ox_flatten(y, h, t, f, ch);
  free(y);
  float *x = (float *)malloc(sizeof(float) * (size_t)t * d);
  ox_gemm(h, m->pre_out, x, t, OX_BIAS, 0);
  free(h);
  float *pos = positions(m, t);
  conformer_run(m, x, t, pos, m->layers, t);
  free(pos);
  ox_gemm(x, m->joint_enc, out, t, OX_BIAS, 0);
  free(x);
  return 0;
}

/* ------------------------------------------------------------------------- TDT greedy decode */

/* Row of a decoder matrix times x, as matvecs (src/cpu/mod.rs:449-469): dot on the dequantized
 * row. */
static void matvec(const ox_linear *l, const float *x, float *out) {
  float *w = (float *)malloc(sizeof(float) * (size_t)l->k);
  for (int r = 0; r < l->n; r++) {
    ox_linear_row(l, r, w);
    out[r] = ox_dot(w, x, (size_t)l->k);
  }
  free(w);
}

typedef struct {
  ox_model *m;
  const float *enc;
  int width;
  float *state, *next, *pred;
  /* Optional trace per decision: (frame, token, duration index) and the smaller top-2 gap of its
   * token and duration logits (how far the decision is from flipping). */
  int *trace_frame;
  float *trace_gap;
  int decisions, cap;
} tdt_ctx;

static float top2_gap(const float *v, int n) {
  float a = -INFINITY, b = -INFINITY;
  for (int i = 0; i < n; i++) {
    if (v[i] > a) {
      b = a;
      a = v[i];
    } else if (v[i] > b) {
      b = v[i];
    }
  }
  return n > 1 ? a - b : INFINITY;
}

/* Decoder::predict (src/parakeet/decoder.rs:111-133). */
static void predict(ox_model *m, int token, const float *state, float *next, float *pred) {
  int n = m->hidden;
  float *x = (float *)calloc((size_t)n, sizeof(float));
  if (token >= 0) ox_linear_row(m->embed, token, x);
  float *gx = (float *)malloc(sizeof(float) * 4 * n), *gh = (float *)malloc(sizeof(float) * 4 * n);
  for (int l = 0; l < m->lstm_layers; l++) {
    const float *h = state + (size_t)2 * n * l, *c = h + n;
    float *nh = next + (size_t)2 * n * l, *nc = nh + n;
    matvec(m->wx[l], x, gx);
    matvec(m->wh[l], h, gh);
    for (int k = 0; k < n; k++) {
#define GATE(i) (gx[i] + gh[i] + m->lstm_b[l][i])
      float ig = GATE(k), fg = GATE(n + k), gg = GATE(2 * n + k), og = GATE(3 * n + k);
#undef GATE
      float sf = 1.0f / (1.0f + expf(-fg)), si = 1.0f / (1.0f + expf(-ig)), so = 1.0f / (1.0f + expf(-og));
      nc[k] = sf * c[k] + si * tanhf(gg);
      nh[k] = so * tanhf(nc[k]);
    }
    memcpy(x, nh, sizeof(float) * n);
  }
  matvec(m->pred_w, x, pred);
  for (int j = 0; j < m->joint; j++) pred[j] = pred[j] + m->pred_b[j];
  free(x);
  free(gx);
  free(gh);
}

int ox_tdt_loop(int frames, int blank, const int *durations, int max_symbols, int global,
                void (*joint)(void *, int, int, int *, int *), void *ctx, uint32_t *out, int cap);

static void tdt_joint_fn(void *p, int t, int emitted, int *token, int *dur) {
  tdt_ctx *c = (tdt_ctx *)p;
  ox_model *m = c->m;
  int S = 2 * m->lstm_layers * m->hidden;
  if (emitted >= 0) {
    memcpy(c->state, c->next, sizeof(float) * S);
    predict(m, emitted, c->state, c->next, c->pred);
  }
  float *z = (float *)malloc(sizeof(float) * m->joint);
  const float *e = c->enc + (size_t)t * c->width;
  for (int j = 0; j < m->joint; j++) {
    float v = e[j] + c->pred[j];
    z[j] = v > 0.0f ? v : 0.0f;
  }
  float *logits = (float *)malloc(sizeof(float) * (m->classes + m->n_dur));
  matvec(m->out_w, z, logits);
  for (int i = 0; i < m->classes + m->n_dur; i++) logits[i] = logits[i] + m->out_b[i];
  *token = ox_argmax(logits, m->classes);
  *dur = ox_argmax(logits + m->classes, m->n_dur);
  if (c->trace_gap && c->decisions < c->cap) {
    float g1 = top2_gap(logits, m->classes), g2 = top2_gap(logits + m->classes, m->n_dur);
    c->trace_frame[3 * c->decisions] = t;
    c->trace_frame[3 * c->decisions + 1] = *token;
    c->trace_frame[3 * c->decisions + 2] = *dur;
    c->trace_gap[c->decisions] = g1 < g2 ? g1 : g2;
  }
  c->decisions++;
  free(z);
  free(logits);
}

int ox_model_tdt_trace(ox_model *m, const float *enc, int frames, int width, uint32_t *out, int cap,
                       int *trace_frame, float *trace_gap, int trace_cap) {
  if (m->arch != ARCH_PARAKEET || !m->embed) return -1;
  int S = 2 * m->lstm_layers * m->hidden;
  tdt_ctx c = {m, enc, width, (float *)calloc((size_t)S, 4), (float *)calloc((size_t)S, 4),
               (float *)calloc((size_t)m->joint, 4), trace_frame, trace_gap, 0, trace_cap};
  predict(m, -1, c.state, c.next, c.pred);
  int n = ox_tdt_loop(frames, m->blank, m->durations, m->max_symbols, m->global, tdt_joint_fn, &c,
                      out, cap);
  free(c.state);
  free(c.next);
  free(c.pred);
  return n;
}

int ox_model_predict(ox_model *m, int token, const float *state, float *next, float *pred) {
  if (m->arch != ARCH_PARAKEET || !m->embed || token >= m->classes) return -1;
  predict(m, token, state, next, pred);
  return 0;
}

/* Decoder::joint's logits (src/parakeet/decoder.rs:135-142) before the two argmaxes. */
int ox_model_joint(ox_model *m, const float *enc_row, const float *pred, float *logits) {
  if (m->arch != ARCH_PARAKEET || !m->embed) return -1;
  float *z = (float *)malloc(sizeof(float) * m->joint);
  for (int j = 0; j < m->joint; j++) {
    float v = enc_row[j] + pred[j];
    z[j] = v > 0.0f ? v : 0.0f;
  }
  matvec(m->out_w, z, logits);
  for (int i = 0; i < m->classes + m->n_dur; i++) logits[i] = logits[i] + m->out_b[i];
  free(z);
  return 0;
}

int ox_model_tdt(ox_model *m, const float *enc, int frames, int width, uint32_t *out, int cap) {
  return ox_model_tdt_trace(m, enc, frames, width, out, cap, NULL, NULL, 0);
}

/* max_i Σ_j |W_ij| of the joint's output layer: with the same predictor state, encoder rows that
 * differ by at most ε per value give joint logits that differ by at most this times ε. */
float ox_model_tdt_lipschitz(ox_model *m) {
  if (m->arch != ARCH_PARAKEET || !m->out_w) return -1.0f;
  float *w = (float *)malloc(sizeof(float) * (size_t)m->out_w->k), best = 0.0f;
  for (int r = 0; r < m->out_w->n; r++) {
    ox_linear_row(m->out_w, r, w);
    float s = 0.0f;
    for (int j = 0; j < m->out_w->k; j++) s += fabsf(w[j]);
    if (s > best) best = s;
  }
  free(w);
  return best;
}

/* ------------------------------------------------------------------------ Whisper decoding */

int ox_whisper_begin(ox_model *m, const float *enc, int frames) {
  if (m->arch != ARCH_WHISPER) return -1;
  int d = m->d, hd = d / m->dec_heads, heads = m->dec_heads;
  if (!m->own) {
    m->own = (float **)calloc((size_t)m->dec_layers, sizeof(float *));
    m->cross = (float **)calloc((size_t)m->dec_layers, sizeof(float *));
  }
  float *kv = (float *)malloc(sizeof(float) * (size_t)frames * 2 * d);
  for (int i = 0; i < m->dec_layers; i++) {
    free(m->own[i]);
    free(m->cross[i]);
    m->own[i] = (float *)calloc((size_t)m->context * 2 * d, sizeof(float));
    m->cross[i] = (float *)malloc(sizeof(float) * (size_t)frames * 2 * d);
    ox_gemm(enc, m->dl[i].cross_kv, kv, frames, OX_BIAS, 0);
    /* Decoder::pack (src/cpu/transformer.rs:211-223): [2*heads][cols][hd], f16-rounded. */
    for (int j = 0; j < frames; j++)
      for (int h = 0; h < 2 * heads; h++)
        for (int c = 0; c < hd; c++)
          m->cross[i][((size_t)h * frames + j) * hd + c] =
              ox_half_to_float(ox_float_to_half_bits(kv[(size_t)j * 2 * d + h * hd + c]));
  }
  free(kv);
  m->cross_frames = frames;
  return 0;
}

int ox_model_whisper_ids(ox_model *m, ox_whisper_ids *ids) {
  if (m->arch != ARCH_WHISPER) return -1;
  ids->eot = m->eot;
  ids->no_timestamps = m->no_timestamps;
  ids->begin = m->no_timestamps + 1;
  ids->sot = m->sot;
  ids->suppress = m->suppress;
  ids->n_suppress = m->n_suppress;
  ids->begin_suppress = m->begin_suppress;
  ids->n_begin_suppress = m->n_begin_suppress;
  return 0;
}

int ox_model_context(ox_model *m) { return m->arch == ARCH_WHISPER ? m->context : 0; }

/* Decoder::step (src/cpu/transformer.rs:226-266). */
int ox_whisper_step(ox_model *m, int token, int pos, float *logits) {
  if (m->arch != ARCH_WHISPER || !m->own || pos >= m->context) return -1;
  int d = m->d, heads = m->dec_heads, hd = d / heads, f = m->dec_ff;
  float *x = (float *)malloc(sizeof(float) * d), *y = (float *)malloc(sizeof(float) * d);
  float *qkv = (float *)malloc(sizeof(float) * 3 * d), *att = (float *)malloc(sizeof(float) * d);
  float *h = (float *)malloc(sizeof(float) * f);
  ox_linear_row(m->token_embd, token, x);
  for (int i = 0; i < d; i++) x[i] += m->dec_pos[(size_t)pos * d + i];
  for (int i = 0; i < m->dec_layers; i++) {
    dec_layer *l = &m->dl[i];
    ox_layer_norm(x, l->norm_self.w, l->norm_self.b, y, 1, d, NULL, NULL, 0);
    ox_gemv(y, l->qkv, qkv, OX_BIAS, 0);
    for (int hh = 0; hh < 2 * heads; hh++)
      for (int c = 0; c < hd; c++)
        m->own[i][((size_t)hh * m->context + pos) * hd + c] =
            ox_half_to_float(ox_float_to_half_bits(qkv[d + hh * hd + c]));
    ox_attend(qkv, m->own[i], m->context, pos + 1, att, heads, hd);
    ox_gemv(att, l->self_out, x, OX_RESIDUAL, 1.0f);
    ox_layer_norm(x, l->norm_cross.w, l->norm_cross.b, y, 1, d, NULL, NULL, 0);
    ox_gemv(y, l->cross_q, qkv, OX_BIAS, 0);
    ox_attend(qkv, m->cross[i], m->cross_frames, m->cross_frames, att, heads, hd);
    ox_gemv(att, l->cross_out, x, OX_RESIDUAL, 1.0f);
    ox_layer_norm(x, l->norm_ffn.w, l->norm_ffn.b, y, 1, d, NULL, NULL, 0);
    ox_gemv(y, l->fc1, h, OX_GELU, 0);
    ox_gemv(h, l->fc2, x, OX_RESIDUAL, 1.0f);
  }
  ox_layer_norm(x, m->dec_norm.w, m->dec_norm.b, y, 1, d, NULL, NULL, 0);
  ox_gemv(y, m->token_embd, logits, OX_BIAS, 0);
  free(x), free(y), free(qkv), free(att), free(h);
  return 0;
}
