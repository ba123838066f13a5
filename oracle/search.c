/*
 * Whisper's greedy window search on the CPU (the parity oracle's restatement of
 * src/whisper/search.rs).  TEST INFRASTRUCTURE ONLY: see oracle.h.
 *
 *   pick / decode ............. src/whisper/search.rs:35-71
 *   timestamp_rules ........... src/whisper/search.rs:73-111
 *   argmax (+ log-softmax) .... src/whisper/search.rs:113-127
 *   probability ............... src/whisper/search.rs:129-135
 *   retrieve .................. src/whisper/search.rs:137-181
 *
 * Arithmetic as the reference spells it: f32 differences `v - max` widened to f64 before the
 * exponential, f64 sums, the logarithm narrowed to f32 and added in f32.
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"

#define MAX_NEW 256     /* src/whisper/search.rs:10 */
#define CONTEXT 448     /* src/whisper/search.rs:11 */
#define MAX_INITIAL 50  /* src/whisper/search.rs:13 */

static int is_ts(const ox_whisper_ids *ids, uint32_t id) { return (int)id >= ids->begin; }

static void fill(float *v, int lo, int hi) {
  for (int i = lo; i < hi; i++) v[i] = -INFINITY;
}

void ox_timestamp_rules(const ox_whisper_ids *ids, float *logits, int vocab, const uint32_t *gen, int n) {
  const int begin = ids->begin;
  logits[ids->no_timestamps] = -INFINITY;
  const int last = n > 0 && is_ts(ids, gen[n - 1]);
  const int penultimate = n < 2 || is_ts(ids, gen[n - 2]);
  if (last) {
    if (penultimate) fill(logits, begin, vocab);
    else fill(logits, 0, ids->eot);
  }
  for (int i = n - 1; i >= 0; i--)
    if (is_ts(ids, gen[i])) {
      int low = last && !penultimate ? (int)gen[i] : (int)gen[i] + 1;
      fill(logits, begin, low < vocab ? low : vocab);
      break;
    }
  if (n == 0) {
    fill(logits, 0, begin);
    int hi = begin + MAX_INITIAL + 1;
    fill(logits, hi < vocab ? hi : vocab, vocab);
  }
  float max = -INFINITY;
  for (int i = begin; i < vocab; i++) max = fmaxf(max, logits[i]);
  float mass = -INFINITY;
  if (isfinite(max)) {
    double sum = 0.0;
    for (int i = begin; i < vocab; i++)
      if (isfinite(logits[i])) sum += exp((double)(logits[i] - max));
    if (sum > 0.0) mass = max + (float)log(sum);
  }
  float text = -INFINITY;
  for (int i = 0; i < begin; i++) text = fmaxf(text, logits[i]);
  if (mass > text) fill(logits, 0, begin);
}

int ox_whisper_argmax(const float *logits, int vocab, int logprob, float *lp) {
  int best = 0;
  for (int i = 0; i < vocab; i++)
    if (logits[i] > logits[best]) best = i;
  if (lp) *lp = 0.0f;
  if (!logprob) return best;
  float max = -INFINITY;
  for (int i = 0; i < vocab; i++)
    if (isfinite(logits[i])) max = fmaxf(max, logits[i]);
  double sum = 0.0;
  for (int i = 0; i < vocab; i++)
    if (isfinite(logits[i])) sum += exp((double)(logits[i] - max));
  if (lp) *lp = logits[best] - (max + (float)log(sum));
  return best;
}

int ox_whisper_pick(const ox_whisper_ids *ids, float *logits, int vocab, const uint32_t *gen, int n, int logprob,
                    float *lp) {
  for (int i = 0; i < ids->n_suppress; i++) logits[ids->suppress[i]] = -INFINITY;
  if (n == 0)
    for (int i = 0; i < ids->n_begin_suppress; i++) logits[ids->begin_suppress[i]] = -INFINITY;
  ox_timestamp_rules(ids, logits, vocab, gen, n);
  return ox_whisper_argmax(logits, vocab, logprob, lp);
}

float ox_probability(const float *logits, int vocab, int id) {
  float max = -INFINITY;
  for (int i = 0; i < vocab; i++)
    if (isfinite(logits[i])) max = fmaxf(max, logits[i]);
  double sum = 0.0, mine = 0.0;
  for (int i = 0; i < vocab; i++) {
    double e = isfinite(logits[i]) ? exp((double)(logits[i] - max)) : 0.0;
    sum += e;
    if (i == id) mine = e;
  }
  return (float)(mine / sum);
}

int ox_whisper_decode(ox_model *m, const ox_whisper_ids *ids, float *logits, int vocab, int prompt, int logprobs,
                      uint32_t *out, int cap, float *avg, float *gaps) {
  double sum = 0.0;
  int picks = 0, n = 0;
  int limit = ox_model_context(m);
  if (limit > CONTEXT) limit = CONTEXT;
  float lp = 0.0f;
  if (gaps) gaps[0] = ox_top2_gap(logits, vocab, ids, out, 0);
  int next = ox_whisper_pick(ids, logits, vocab, out, 0, logprobs, &lp);
  sum += lp, picks++;
  for (int pos = prompt; pos < prompt + MAX_NEW; pos++) {
    if (next == ids->eot) break;
    if (n >= cap) return -1;
    out[n++] = (uint32_t)next;
    if (pos + 1 > limit) break;
    if (ox_whisper_step(m, next, pos, logits)) return -1;
    if (gaps) gaps[n] = ox_top2_gap(logits, vocab, ids, out, n);
    next = ox_whisper_pick(ids, logits, vocab, out, n, logprobs, &lp);
    sum += lp, picks++;
  }
  if (avg) *avg = logprobs ? (float)(sum / picks) : 0.0f;
  return n;
}

/* The gap between the two largest logits that the rules leave (+inf when one or none is left), on a
 * copy: the margin of that step's choice. */
float ox_top2_gap(const float *logits, int vocab, const ox_whisper_ids *ids, const uint32_t *gen, int n) {
  float *c = (float *)malloc(sizeof(float) * (size_t)vocab);
  memcpy(c, logits, sizeof(float) * (size_t)vocab);
  for (int i = 0; i < ids->n_suppress; i++) c[ids->suppress[i]] = -INFINITY;
  if (n == 0)
    for (int i = 0; i < ids->n_begin_suppress; i++) c[ids->begin_suppress[i]] = -INFINITY;
  ox_timestamp_rules(ids, c, vocab, gen, n);
  float a = -INFINITY, b = -INFINITY;
  for (int i = 0; i < vocab; i++) {
    if (c[i] > a) b = a, a = c[i];
    else if (c[i] > b) b = c[i];
  }
  free(c);
  return isfinite(b) ? a - b : INFINITY;
}

int ox_whisper_retrieve(const ox_whisper_ids *ids, const uint32_t *gen, int n, int frames, int *seg, int cap,
                        int *advance) {
#define TS(i) is_ts(ids, gen[i])
  int *slices = (int *)malloc(sizeof(int) * (size_t)(n + 1));
  int ns = 0;
  for (int i = 0; i + 1 < n; i++)
    if (TS(i) && TS(i + 1)) slices[ns++] = i + 1;
  int count = 0;
  if (ns == 0) {
    if (n > 0) {
      if (cap > 0) seg[0] = 0, seg[1] = 0, seg[2] = n;
      count = 1;
    }
    *advance = frames;
    free(slices);
    return count;
  }
  const int single = n >= 2 && !TS(n - 2) && TS(n - 1);
  if (single) slices[ns++] = n;
  else slices[ns - 1] += 1;
  int last = 0;
  for (int k = 0; k < ns; k++) {
    const int end = slices[k];
    const int closing = k + 1 < ns || single ? end - 1 : end - 2;
    if (end > last && TS(last) && closing >= last && closing < n && TS(closing)) {
      if (count < cap) seg[3 * count] = (int)gen[last] - ids->begin, seg[3 * count + 1] = last, seg[3 * count + 2] = end;
      count++;
    }
    last = end;
  }
  if (single) *advance = frames;
  else if (last >= 2 && last - 2 < n && TS(last - 2)) *advance = ((int)gen[last - 2] - ids->begin) * 2;
  else *advance = frames;
  free(slices);
  return count;
#undef TS
}
