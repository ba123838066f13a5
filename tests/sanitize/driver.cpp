// CPU program for tests/test_sanitize.py, built with AddressSanitizer and UBSan (tests/sanitize/Makefile):
// runs the oracle's model paths (GGUF load, encoders, CTC, TDT with its trace, Whisper steps and window
// search) on the small synthetic models named on the command line, then the product's host-side Whisper
// search (wavo_amd/csrc/search.cpp) against the oracle's on seeded random logits and token histories.
// Exit status 0: every comparison held and neither sanitizer reported (they abort on the first report).
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "oracle.h"
#include "wavo_hip.h"

namespace {

uint64_t g_state = 0x9e3779b97f4a7c15ull;

uint32_t next_u32() {
  g_state = g_state * 6364136223846793005ull + 1442695040888963407ull;
  return (uint32_t)(g_state >> 33);
}

float next_f32() { return (float)((int)(next_u32() % 20001) - 10000) / 2500.0f; }  // [-4, 4]

int failures = 0;

void check(bool ok, const char *what, int i) {
  if (!ok) {
    std::fprintf(stderr, "MISMATCH %s (case %d)\n", what, i);
    failures++;
  }
}

ox_model *load(const char *path) {
  char err[256] = {0};
  ox_model *m = ox_model_load(path, err, sizeof err);
  if (!m) std::fprintf(stderr, "load %s: %s\n", path, err);
  return m;
}

// Encoder output of random mel frames; frames and width through the pointers.
std::vector<float> encode(ox_model *m, int mel_frames, int *frames, int *width) {
  int arch = 0, d = 0, layers = 0, mels = 0, w = 0;
  ox_model_info(m, &arch, &d, &layers, &mels, &w);
  std::vector<float> mel((size_t)mel_frames * mels);
  for (float &v : mel) v = next_f32();
  if (ox_model_encode(m, mel.data(), mel_frames, mel_frames, nullptr, frames, width)) return {};
  std::vector<float> out((size_t)*frames * *width);
  if (ox_model_encode(m, mel.data(), mel_frames, mel_frames, out.data(), frames, width)) return {};
  return out;
}

int run_gigaam(const char *path) {
  ox_model *m = load(path);
  if (!m) return 1;
  int frames = 0, width = 0;
  std::vector<float> enc = encode(m, 200, &frames, &width);
  check(!enc.empty(), "gigaam encode", 0);
  std::vector<uint32_t> out(2 * (size_t)frames + 2);
  int n = ox_ctc(enc.data(), frames, width, width - 1, out.data());
  check(n >= 0 && n <= frames, "gigaam ctc count", 0);
  ox_model_free(m);
  return 0;
}

int run_parakeet(const char *path) {
  ox_model *m = load(path);
  if (!m) return 1;
  int frames = 0, width = 0;
  std::vector<float> enc = encode(m, 160, &frames, &width);
  check(!enc.empty(), "parakeet encode", 0);
  const int cap = 16 * frames + 16;
  std::vector<uint32_t> out(2 * (size_t)cap), out2(2 * (size_t)cap);
  std::vector<int> trace(3 * (size_t)cap);
  std::vector<float> gaps(cap);
  int n = ox_model_tdt(m, enc.data(), frames, width, out.data(), cap);
  int n2 = ox_model_tdt_trace(m, enc.data(), frames, width, out2.data(), cap, trace.data(), gaps.data(), cap);
  check(n >= 0 && n == n2 && std::memcmp(out.data(), out2.data(), 8 * (size_t)n) == 0, "parakeet tdt", 0);
  ox_model_free(m);
  return 0;
}

wh_whisper_ids product_ids(const ox_whisper_ids &o) {
  wh_whisper_ids w;
  w.eot = o.eot;
  w.no_timestamps = o.no_timestamps;
  w.begin = o.begin;
  w.sot = o.sot;
  w.suppress = o.suppress;
  w.n_suppress = o.n_suppress;
  w.begin_suppress = o.begin_suppress;
  w.n_begin_suppress = o.n_begin_suppress;
  return w;
}

// A token history: text ids below eot and timestamps from begin, in runs.
std::vector<uint32_t> history(const ox_whisper_ids &ids, int vocab, int n) {
  std::vector<uint32_t> g(n);
  int ts = ids.begin;
  for (int i = 0; i < n; i++) {
    if (next_u32() % 3 == 0) {
      ts = std::min(vocab - 1, ts + (int)(next_u32() % 40));
      g[i] = (uint32_t)ts;
    } else {
      g[i] = next_u32() % (uint32_t)ids.eot;
    }
  }
  return g;
}

int run_whisper(const char *path, int V) {
  ox_model *m = load(path);
  if (!m) return 1;
  int frames = 0, width = 0;
  std::vector<float> enc = encode(m, 200, &frames, &width);
  check(!enc.empty(), "whisper encode", 0);
  ox_whisper_ids ids;
  if (ox_model_whisper_ids(m, &ids)) return 1;
  std::vector<float> logits(V);
  check(ox_whisper_begin(m, enc.data(), frames) == 0, "whisper begin", 0);
  check(ox_whisper_step(m, ids.sot, 0, logits.data()) == 0, "whisper step", 0);
  std::vector<uint32_t> out(512);
  std::vector<float> gaps(513);
  float avg = 0.0f;
  int n = ox_whisper_decode(m, &ids, logits.data(), V, 1, 1, out.data(), 512, &avg, gaps.data());
  check(n >= 0, "whisper decode", 0);

  // The product's search against the oracle's.
  const wh_whisper_ids pw = product_ids(ids);
  for (int i = 0; i < 400; i++) {
    const int len = (int)(next_u32() % 48);
    std::vector<uint32_t> g = history(ids, V, len);
    std::vector<float> a(V), b(V);
    for (int j = 0; j < V; j++) a[j] = b[j] = next_f32();
    if (i % 7 == 0) a[ids.begin] = b[ids.begin] = 50.0f;  // a dominant timestamp
    float lpa = 0.0f, lpb = 0.0f;
    const int want = ox_whisper_pick(&ids, a.data(), V, g.data(), len, 1, &lpa);
    const int got = wh_whisper_pick(&pw, b.data(), V, g.data(), len, &lpb);
    check(want == got && lpa == lpb && std::memcmp(a.data(), b.data(), 4 * (size_t)V) == 0, "pick", i);
    const int id = (int)(next_u32() % (uint32_t)V);
    check(ox_probability(b.data(), V, id) == wh_whisper_probability(b.data(), V, id), "probability", i);
    std::vector<int> sa(3 * (size_t)(len + 2)), sb(3 * (size_t)(len + 2));
    int adva = -1, advb = -1;
    const int ca = ox_whisper_retrieve(&ids, g.data(), len, frames, sa.data(), len + 2, &adva);
    const int cb = wh_whisper_retrieve(&pw, g.data(), len, frames, sb.data(), len + 2, &advb);
    check(ca == cb && adva == advb && (ca <= 0 || std::memcmp(sa.data(), sb.data(), 12 * (size_t)ca) == 0),
          "retrieve", i);
  }
  ox_model_free(m);
  return 0;
}

}  // namespace

int main(int argc, char **argv) {
  if (argc != 5) {
    std::fprintf(stderr, "usage: %s gigaam.gguf parakeet.gguf whisper.gguf whisper_vocab\n", argv[0]);
    return 2;
  }
  if (run_gigaam(argv[1]) || run_parakeet(argv[2]) || run_whisper(argv[3], std::atoi(argv[4]))) return 1;
  std::printf("sanitized run done, %d mismatches\n", failures);
  return failures ? 1 : 0;
}
