// Whisper's greedy window search on the host (src/whisper/search.rs), the consumer of the decoder's
// logits: the suppression lists, the timestamp rules, the first argmax with its log-softmax, the
// no-speech probability and the cut of a window's tokens into timestamped segments.  Host code only:
// these functions touch no device memory, so the C ABI offers them to a caller without a GPU too.
//
//   pick ...................... src/whisper/search.rs:46-59
//   timestamp_rules ........... src/whisper/search.rs:73-111
//   argmax (+ log-softmax) .... src/whisper/search.rs:113-127
//   probability ............... src/whisper/search.rs:129-135
//   retrieve .................. src/whisper/search.rs:137-181
//
// The arithmetic follows the reference: f32 differences `v - max` widened to f64 before the
// exponential, f64 sums, the logarithm narrowed to f32 and added in f32.
#include <cmath>
#include <vector>

#include "../../include/wavo_hip.h"

namespace {

constexpr int MAX_INITIAL = 50;  // the first timestamp is at most 1.0 s in (src/whisper/search.rs:13)

bool is_ts(const wh_whisper_ids *ids, uint32_t id) { return (int)id >= ids->begin; }

void neg_inf(float *v, int lo, int hi) {
  for (int i = lo; i < hi; i++) v[i] = -INFINITY;
}

void timestamp_rules(const wh_whisper_ids *ids, float *logits, int vocab, const uint32_t *gen, int n) {
  const int begin = ids->begin;
  logits[ids->no_timestamps] = -INFINITY;
  const bool last = n > 0 && is_ts(ids, gen[n - 1]);
  const bool penultimate = n < 2 || is_ts(ids, gen[n - 2]);
  if (last) {
    // A timestamp pair closes (only text or EOT may follow) or a single one opens (only timestamps).
    if (penultimate) neg_inf(logits, begin, vocab);
    else neg_inf(logits, 0, ids->eot);
  }
  for (int i = n - 1; i >= 0; i--)  // timestamps never decrease
    if (is_ts(ids, gen[i])) {
      const int low = last && !penultimate ? (int)gen[i] : (int)gen[i] + 1;
      neg_inf(logits, begin, std::min(low, vocab));
      break;
    }
  if (n == 0) {  // the first token is a timestamp of at most MAX_INITIAL steps
    neg_inf(logits, 0, begin);
    neg_inf(logits, std::min(begin + MAX_INITIAL + 1, vocab), vocab);
  }
  float max = -INFINITY;
  for (int i = begin; i < vocab; i++) max = std::fmax(max, logits[i]);
  float mass = -INFINITY;
  if (std::isfinite(max)) {
    double sum = 0.0;
    for (int i = begin; i < vocab; i++)
      if (std::isfinite(logits[i])) sum += std::exp((double)(logits[i] - max));
    if (sum > 0.0) mass = max + (float)std::log(sum);
  }
  float text = -INFINITY;
  for (int i = 0; i < begin; i++) text = std::fmax(text, logits[i]);
  if (mass > text) neg_inf(logits, 0, begin);  // the timestamps' total probability wins
}

int argmax(const float *logits, int vocab, float *lp) {
  int best = 0;
  for (int i = 0; i < vocab; i++)
    if (logits[i] > logits[best]) best = i;
  if (!lp) return best;
  float max = -INFINITY;
  for (int i = 0; i < vocab; i++)
    if (std::isfinite(logits[i])) max = std::fmax(max, logits[i]);
  double sum = 0.0;
  for (int i = 0; i < vocab; i++)
    if (std::isfinite(logits[i])) sum += std::exp((double)(logits[i] - max));
  *lp = logits[best] - (max + (float)std::log(sum));
  return best;
}

bool ids_ok(const wh_whisper_ids *ids, int vocab) {
  if (!ids || ids->eot < 0 || ids->eot >= vocab || ids->no_timestamps < 0 || ids->no_timestamps >= vocab ||
      ids->begin <= 0 || ids->begin > vocab || (ids->n_suppress && !ids->suppress) ||
      (ids->n_begin_suppress && !ids->begin_suppress))
    return false;
  for (int i = 0; i < ids->n_suppress; i++)
    if (ids->suppress[i] < 0 || ids->suppress[i] >= vocab) return false;
  for (int i = 0; i < ids->n_begin_suppress; i++)
    if (ids->begin_suppress[i] < 0 || ids->begin_suppress[i] >= vocab) return false;
  return true;
}

}  // namespace

extern "C" {

int wh_whisper_pick(const wh_whisper_ids *ids, float *logits, int vocab, const uint32_t *gen, int n, float *logprob) {
  if (!logits || vocab <= 0 || n < 0 || (n && !gen) || !ids_ok(ids, vocab)) return WH_EARG;
  for (int i = 0; i < ids->n_suppress; i++) logits[ids->suppress[i]] = -INFINITY;
  if (n == 0)
    for (int i = 0; i < ids->n_begin_suppress; i++) logits[ids->begin_suppress[i]] = -INFINITY;
  timestamp_rules(ids, logits, vocab, gen, n);
  return argmax(logits, vocab, logprob);
}

float wh_whisper_probability(const float *logits, int vocab, int id) {
  if (!logits || id < 0 || id >= vocab) return NAN;
  float max = -INFINITY;
  for (int i = 0; i < vocab; i++)
    if (std::isfinite(logits[i])) max = std::fmax(max, logits[i]);
  double sum = 0.0, mine = 0.0;
  for (int i = 0; i < vocab; i++) {
    const double e = std::isfinite(logits[i]) ? std::exp((double)(logits[i] - max)) : 0.0;
    sum += e;
    if (i == id) mine = e;
  }
  return (float)(mine / sum);
}

int wh_whisper_retrieve(const wh_whisper_ids *ids, const uint32_t *gen, int n, int frames, int *seg, int cap,
                        int *advance) {
  if (!ids || n < 0 || (n && !gen) || !advance || cap < 0 || (cap && !seg)) return WH_EARG;
  auto ts = [&](int i) { return is_ts(ids, gen[i]); };
  // Slices after every pair of consecutive timestamps.
  std::vector<int> slices;
  for (int i = 0; i + 1 < n; i++)
    if (ts(i) && ts(i + 1)) slices.push_back(i + 1);
  int count = 0;
  auto put = [&](int start, int lo, int hi) {
    if (count < cap) seg[3 * count] = start, seg[3 * count + 1] = lo, seg[3 * count + 2] = hi;
    count++;
  };
  if (slices.empty()) {  // no pair: one segment from the window's start, and a full advance
    if (n > 0) put(0, 0, n);
    *advance = frames;
    return count;
  }
  const bool single = n >= 2 && !ts(n - 2) && ts(n - 1);
  if (single) slices.push_back(n);
  else slices.back() += 1;
  int last = 0;
  for (size_t k = 0; k < slices.size(); k++) {
    const int end = slices[k];
    const int closing = k + 1 < slices.size() || single ? end - 1 : end - 2;
    if (end > last && ts(last) && closing >= last && closing < n && ts(closing))
      put((int)gen[last] - ids->begin, last, end);
    last = end;
  }
  if (single) *advance = frames;
  else if (last >= 2 && last - 2 < n && ts(last - 2)) *advance = ((int)gen[last - 2] - ids->begin) * 2;
  else *advance = frames;
  return count;
}

}  // extern "C"
