// Graph drivers of the family encoders and the Whisper decoder on the gfx950 kernels, and the host
// greedy decoders of their outputs.  They record the ops in the order the reference's GPU graph
// builders do:
//   GGUF v3 reading ............ src/gguf.rs:121-287
//   Conformer blocks ........... src/conformer.rs:34-61 (Config::load), :107-116, :180-265
//   GigaAM encoder ............. src/gigaam/encoder.rs:39-118, rope table src/gigaam/mod.rs:86-97
//   Parakeet encoder ........... src/parakeet/encoder.rs:51-153, frames src/parakeet/mod.rs:44-46
//   Whisper encoder/decoder .... src/whisper/encoder.rs:32-74, src/transformer.rs:103-290
//   CTC greedy ................. src/gigaam/decoder.rs:135-151
//   TDT greedy ................. src/parakeet/decoder.rs:91-191 (host, as the reference runs it)
// Activations live in an arena of device buffers sized for the longest input so far (the
// reference's per-family Arena, e.g. src/gigaam/encoder.rs:25-35, :61-72).  The Parakeet
// subsampling runs unchunked: the reference splits it into 8 chunks to bound memory
// (src/parakeet/encoder.rs:17-19), which 288 GB of HBM does not need, and one launch per conv keeps
// its GEMM large.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <climits>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <map>
#include <memory>
#include <string>
#include <vector>

#include "internal.h"

namespace {

// ------------------------------------------------------------------------------- GGUF reader

struct Tensor {
  std::vector<size_t> dims;
  int type = 0;
  const uint8_t *data = nullptr;
  size_t count() const {
    size_t n = 1;
    for (size_t d : dims) n *= d;
    return n;
  }
};

struct Value {
  unsigned type = 0;
  const uint8_t *p = nullptr;
};

class Gguf {
 public:
  ~Gguf() {
    if (map_) munmap(map_, len_);
    if (fd_ >= 0) ::close(fd_);
  }

  // The mapping as a source of staged uploads: weight bytes are read with pread into pinned memory.
  StageFile file() const { return StageFile{fd_, map_, len_}; }

  bool open(const char *path, std::string &err) {
    int fd = ::open(path, O_RDONLY);
    if (fd < 0) return err = std::string("cannot open ") + path, false;
    fd_ = fd;
    struct stat st;
    fstat(fd, &st);
    len_ = (size_t)st.st_size;
    void *m = mmap(nullptr, len_, PROT_READ, MAP_PRIVATE, fd, 0);
    if (m == MAP_FAILED) return err = "cannot map the file", false;
    map_ = (uint8_t *)m;
    p_ = map_;
    end_ = map_ + len_;
    if (len_ < 4 || memcmp(map_, "GGUF", 4)) return err = "not a GGUF file", false;
    p_ += 4;
    uint32_t version = (uint32_t)rd(4);
    if (version != 3) return err = "unsupported GGUF version " + std::to_string(version), false;
    uint64_t n_t = rd(8), n_kv = rd(8);
    if (bad_ || n_t > (1u << 24) || n_kv > (1u << 24)) return err = "truncated GGUF header", false;
    size_t align = 32;
    for (uint64_t i = 0; i < n_kv && !bad_; i++) {
      std::string key = str();
      Value v;
      v.type = (unsigned)rd(4);
      v.p = p_;
      if (key == "general.alignment" && v.type == 4) {
        uint32_t a;
        memcpy(&a, p_, 4);
        align = a;
      }
      skip(v.type);
      kv_[key] = v;
    }
    std::vector<std::pair<std::string, std::pair<Tensor, uint64_t>>> infos;
    for (uint64_t i = 0; i < n_t && !bad_; i++) {
      std::string name = str();
      uint32_t nd = (uint32_t)rd(4);
      if (nd < 1 || nd > 4) bad_ = true;
      Tensor t;
      for (uint32_t d = 0; d < nd && !bad_; d++) t.dims.push_back((size_t)rd(8));
      t.type = (int)rd(4);
      uint64_t off = rd(8);
      infos.push_back({name, {t, off}});
    }
    if (bad_) return err = "truncated GGUF header", false;
    size_t data = ((size_t)(p_ - map_) + align - 1) / align * align;
    for (auto &in : infos) {
      Tensor t = in.second.first;
      size_t bytes = wh_type_bytes(t.type, t.count());
      if (!bytes || data + in.second.second + bytes > len_)
        return err = "tensor " + in.first + " is out of file bounds or of an unsupported type", false;
      t.data = map_ + data + in.second.second;
      tensors_[in.first] = t;
    }
    return true;
  }

  const Tensor *tensor(const std::string &name) const {
    auto it = tensors_.find(name);
    return it == tensors_.end() ? nullptr : &it->second;
  }

  bool has(const std::string &key) const { return kv_.count(key) != 0; }

  long integer(const std::string &key, long dflt) const {
    auto it = kv_.find(key);
    if (it == kv_.end()) return dflt;
    const uint8_t *p = it->second.p;
    switch (it->second.type) {
      case 0: return p[0];
      case 1: return (int8_t)p[0];
      case 2: { uint16_t v; memcpy(&v, p, 2); return v; }
      case 3: { int16_t v; memcpy(&v, p, 2); return v; }
      case 4: { uint32_t v; memcpy(&v, p, 4); return v; }
      case 5: { int32_t v; memcpy(&v, p, 4); return v; }
      case 7: return p[0];
      case 10: case 11: { int64_t v; memcpy(&v, p, 8); return (long)v; }
    }
    return dflt;
  }

  std::string string(const std::string &key) const {
    auto it = kv_.find(key);
    if (it == kv_.end() || it->second.type != 8) return "";
    uint64_t n;
    memcpy(&n, it->second.p, 8);
    return std::string((const char *)it->second.p + 8, n);
  }

  std::vector<long> ints(const std::string &key) const {
    std::vector<long> out;
    auto it = kv_.find(key);
    if (it == kv_.end() || it->second.type != 9) return out;
    uint32_t item;
    uint64_t n;
    memcpy(&item, it->second.p, 4);
    memcpy(&n, it->second.p + 4, 8);
    const uint8_t *p = it->second.p + 12;
    size_t s = item == 4 || item == 5 ? 4 : (item == 10 || item == 11 ? 8 : 0);
    for (uint64_t i = 0; s && i < n; i++, p += s) {
      if (s == 4) {
        int32_t v;
        memcpy(&v, p, 4);
        out.push_back(item == 4 ? (long)(uint32_t)v : (long)v);
      } else {
        int64_t v;
        memcpy(&v, p, 8);
        out.push_back((long)v);
      }
    }
    return out;
  }

 private:
  uint64_t rd(int n) {
    if (p_ + n > end_) {
      bad_ = true;
      return 0;
    }
    uint64_t v = 0;
    for (int i = 0; i < n; i++) v |= (uint64_t)p_[i] << (8 * i);
    p_ += n;
    return v;
  }
  std::string str() {
    uint64_t n = rd(8);
    if (bad_ || p_ + n > end_) {
      bad_ = true;
      return "";
    }
    std::string s((const char *)p_, n);
    p_ += n;
    return s;
  }
  void skip(unsigned t) {
    static const int sz[] = {1, 1, 2, 2, 4, 4, 4, 1, 0, 0, 8, 8, 8};
    if (t == 8) {
      str();
    } else if (t == 9) {
      unsigned it = (unsigned)rd(4);
      uint64_t n = rd(8);
      for (uint64_t i = 0; i < n && !bad_; i++) skip(it);
    } else if (t < 13 && sz[t]) {
      if (p_ + sz[t] > end_) bad_ = true;
      else p_ += sz[t];
    } else {
      bad_ = true;
    }
  }

  uint8_t *map_ = nullptr;
  size_t len_ = 0;
  int fd_ = -1;
  const uint8_t *p_ = nullptr, *end_ = nullptr;
  bool bad_ = false;
  std::map<std::string, Value> kv_;
  std::map<std::string, Tensor> tensors_;
};

float half_to_float(uint16_t h) {
  uint32_t s = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 31, m = h & 0x3ff, u;
  if (e == 0) {
    float v = (float)m * 5.9604644775390625e-8f;
    return s ? -v : v;
  }
  u = e == 31 ? (s | 0x7f800000u | (m << 13)) : (s | ((e + 112) << 23) | (m << 13));
  float f;
  memcpy(&f, &u, 4);
  return f;
}

// Tensor::to_f32 (src/gguf.rs:274-287), plus Q4_0.
std::vector<float> to_f32(const Tensor &t) {
  size_t n = t.count();
  std::vector<float> out(n);
  const uint8_t *s = t.data;
  switch (t.type) {
    case WH_F32: memcpy(out.data(), s, n * 4); break;
    case WH_F16:
      for (size_t i = 0; i < n; i++) {
        uint16_t h;
        memcpy(&h, s + 2 * i, 2);
        out[i] = half_to_float(h);
      }
      break;
    case WH_Q8_0:
      for (size_t b = 0; b < n / 32; b++) {
        uint16_t h;
        memcpy(&h, s + 34 * b, 2);
        float d = half_to_float(h);
        for (int i = 0; i < 32; i++) out[32 * b + i] = (float)(int8_t)s[34 * b + 2 + i] * d;
      }
      break;
    case WH_Q4_0:
      for (size_t b = 0; b < n / 32; b++) {
        uint16_t h;
        memcpy(&h, s + 18 * b, 2);
        float d = half_to_float(h);
        for (int i = 0; i < 16; i++) {
          out[32 * b + i] = (float)((int)(s[18 * b + 2 + i] & 15) - 8) * d;
          out[32 * b + 16 + i] = (float)((int)(s[18 * b + 2 + i] >> 4) - 8) * d;
        }
      }
      break;
  }
  return out;
}

// ----------------------------------------------------------------------------- device helpers

// A device f32 array owned by the model.
struct DevArray {
  float *p = nullptr;
  size_t n = 0;
};

struct Chan {
  float *w = nullptr, *b = nullptr;
};

class Loader {
 public:
  Loader(wh_ctx *ctx, const Gguf &g) : ctx_(ctx), g_(g) {}
  std::string err;

  const Tensor *need(const std::string &name, size_t want = 0) {
    const Tensor *t = g_.tensor(name);
    if (!t) {
      fail("missing tensor " + name);
      return nullptr;
    }
    if (want && t->count() != want) {
      fail("tensor " + name + " has " + std::to_string(t->count()) + " values, expected " + std::to_string(want));
      return nullptr;
    }
    return t;
  }

  std::vector<float> f32s(const std::string &name, size_t want) {
    const Tensor *t = need(name, want);
    return t ? to_f32(*t) : std::vector<float>(want, 0.0f);
  }

  float *upload(const std::vector<float> &v) {
    if (!err.empty()) return nullptr;
    float *p = nullptr;
    if (wh_alloc(ctx_, v.size(), &p)) {
      fail(ctx_->error);
      return nullptr;
    }
    owned.push_back(p);
    if (!v.empty() && stage_upload(ctx_, p, v.data(), v.size() * 4)) fail(ctx_->error);
    return p;
  }

  Chan norm(const std::string &name, int d, bool bias) {
    Chan c;
    c.w = upload(f32s(name + ".weight", d));
    c.b = upload(bias ? f32s(name + ".bias", d) : std::vector<float>(d, 0.0f));
    return c;
  }

  // conformer::linear / transformer::stacked: the weights `names[i].weight` stacked along n with
  // their biases (index `zero` has none: Whisper's k); `extra` appended after (dual outputs).
  wh_linear *linear(const std::vector<std::string> &names, bool bias, int zero = -1,
                    const std::vector<float> &override_bias = {}, int pad_k = 0) {
    if (!err.empty()) return nullptr;
    std::vector<wh_tensor> ws;
    std::vector<float> b;
    for (size_t i = 0; i < names.size(); i++) {
      const Tensor *t = need(names[i] + ".weight");
      if (!t) return nullptr;
      int k = (int)t->dims[0];
      for (size_t d = 1; d + 1 < t->dims.size(); d++) k *= (int)t->dims[d];
      int rows = (int)t->dims.back();
      ws.push_back(wh_tensor{t->data, t->type, k, rows});
      if (bias) {
        if ((int)i == zero) b.insert(b.end(), rows, 0.0f);
        else {
          auto bi = f32s(names[i] + ".bias", rows);
          b.insert(b.end(), bi.begin(), bi.end());
        }
      }
    }
    const std::vector<float> &bb = override_bias.empty() ? b : override_bias;
    wh_linear *l = nullptr;
    const StageFile file = g_.file();
    if (linear_new(ctx_, ws.data(), (int)ws.size(), bb.empty() ? nullptr : bb.data(), (int)bb.size(), pad_k, &l,
                   &file)) {
      fail(names[0] + ": " + ctx_->error);
      return nullptr;
    }
    linears.push_back(l);
    return l;
  }

  // The conv module's first pointwise conv (2·ch output rows: the GLU's x rows, then its gates) with
  // its rows permuted into groups of 8, [x 4j .. 4j+3 | gates 4j .. 4j+3] for j = 0 .. ch/4 − 1, so
  // that a GEMM epilogue holds every channel's x and gate in one lane (EPI_GLU); *groups says whether
  // it did (ch % 4 == 0), else the rows stay as stored.  Whole rows move: the products are unchanged.
  wh_linear *glu_groups(const std::string &name, bool bias, bool *groups) {
    *groups = false;
    if (!err.empty()) return nullptr;
    const Tensor *t = need(name + ".weight");
    if (!t) return nullptr;
    int k = (int)t->dims[0];
    for (size_t d = 1; d + 1 < t->dims.size(); d++) k *= (int)t->dims[d];
    const int rows = (int)t->dims.back(), ch = rows / 2;
    if (rows % 8) return linear({name}, bias);
    const size_t rb = wh_type_bytes(t->type, (size_t)k);
    std::vector<uint8_t> host(rb * rows);
    std::vector<float> b, bo = bias ? f32s(name + ".bias", rows) : std::vector<float>();
    for (int r = 0; r < rows; r++) {
      const int j = r / 8, q = r % 8, src = q < 4 ? 4 * j + q : ch + 4 * j + q - 4;
      memcpy(host.data() + (size_t)r * rb, t->data + (size_t)src * rb, rb);
      if (bias) b.push_back(bo[src]);
    }
    wh_tensor w{host.data(), t->type, k, rows};
    wh_linear *l = nullptr;
    if (linear_new(ctx_, &w, 1, b.empty() ? nullptr : b.data(), (int)b.size(), 0, &l, nullptr)) {
      fail(name + ": " + ctx_->error);
      return nullptr;
    }
    linears.push_back(l);
    *groups = true;
    return l;
  }

  // One linear layer from weight tensors joined along k: row r is [names[0] row r | names[1] row r |
  // ...] (the LSTM's [Wx | Wh] over [x | h]).  Same type and rows; whole 32-weight blocks each.
  wh_linear *joined(const std::vector<std::string> &names, const std::vector<float> &bias) {
    if (!err.empty()) return nullptr;
    std::vector<const Tensor *> ts;
    std::vector<size_t> rb;
    int k = 0, rows = -1, type = -1;
    for (const std::string &name : names) {
      const Tensor *t = need(name);
      if (!t) return nullptr;
      const int ki = (int)t->dims[0], ri = (int)(t->count() / t->dims[0]);
      if ((type >= 0 && t->type != type) || (rows >= 0 && ri != rows) || ki % 32) {
        fail(name + ": joined weights differ in type or rows, or k is not a multiple of 32");
        return nullptr;
      }
      type = t->type, rows = ri, k += ki;
      ts.push_back(t);
      rb.push_back(wh_type_bytes(type, (size_t)ki));
    }
    size_t row_bytes = 0;
    for (size_t b : rb) row_bytes += b;
    std::vector<uint8_t> host(row_bytes * rows);
    for (int r = 0; r < rows; r++) {
      uint8_t *dst = host.data() + (size_t)r * row_bytes;
      for (size_t i = 0; i < ts.size(); dst += rb[i], i++) memcpy(dst, ts[i]->data + (size_t)r * rb[i], rb[i]);
    }
    wh_tensor w{host.data(), type, k, rows};
    wh_linear *l = nullptr;
    if (linear_new(ctx_, &w, 1, bias.data(), (int)bias.size(), 0, &l, nullptr)) {
      fail(names[0] + ": " + ctx_->error);
      return nullptr;
    }
    linears.push_back(l);
    return l;
  }

  void fail(const std::string &m) {
    if (err.empty()) err = m;
  }

  std::vector<float *> owned;
  std::vector<wh_linear *> linears;

 private:
  wh_ctx *ctx_;
  const Gguf &g_;
};

// ----------------------------------------------------------------------------------- model

enum Arch { GIGAAM = 0, PARAKEET = 1, WHISPER = 2 };
constexpr intptr_t WHISPER_STEP = 16;  // the recording key of a Whisper decoder step
constexpr intptr_t TDT_CHUNK = 17;     // the recording key of a run of TDT decisions
constexpr int TDT_DECISIONS = 32;      // decisions per recorded run (the host looks at the state between runs)
constexpr intptr_t WHISPER_LOOP = 18;  // the recording key of a run of Whisper (step, pick) pairs
constexpr int WHISPER_PICKS = 8;       // (step, pick) pairs per recorded run
constexpr int WHISPER_MAX_NEW = 256, WHISPER_CONTEXT = 448;  // src/whisper/search.rs:10-11

struct Block {
  Chan norm_ff1, norm_attn, norm_conv, norm_ff2, norm_out, conv_norm, dw;
  wh_linear *ff1[2] = {}, *ff2[2] = {}, *out = nullptr, *pw1 = nullptr, *pw2 = nullptr;
  bool pw1_groups = false;  // pw1's output columns in GLU groups of 8 (Loader::glu_groups)
  wh_linear *qk = nullptr, *v = nullptr;     // rotary: q stacked over k, and v
  wh_linear *qkv = nullptr;  // relative: [q + u | k | v | q + v]
};

struct WBlock {
  Chan norm_attn, norm_ffn;
  wh_linear *qkv = nullptr, *out = nullptr, *fc1 = nullptr, *fc2 = nullptr;
};

struct DLayer {
  Chan norm_self, norm_cross, norm_ffn;
  wh_linear *qkv = nullptr, *self_out = nullptr, *cross_q = nullptr, *cross_kv = nullptr, *cross_out = nullptr,
            *fc1 = nullptr, *fc2 = nullptr;
};

// A decoder matrix on the host for the TDT greedy loop: rows of f32 (dequantized, exact).
struct HostMat {
  int rows = 0, k = 0;
  std::vector<float> w;
};

int half_len(int n) { return (n - 1) / 2 + 1; }

}  // namespace

struct wh_model {
  wh_ctx *ctx = nullptr;
  Arch arch = GIGAAM;
  std::unique_ptr<Gguf> g;
  std::vector<float *> owned;
  std::vector<wh_linear *> linears;
  // Conformer config.
  int layers = 0, d = 0, heads = 0, d_ff = 0, kernel = 0, mels = 0;
  bool layer_norm_conv = false, relative = false;
  std::vector<Block> blocks;
  // GigaAM
  double theta = 5000.0;
  wh_linear *conv0 = nullptr, *conv2 = nullptr, *head = nullptr;
  int outputs = 0, blank = 0;
  // Parakeet
  int ch = 0;
  Chan sc0, sc2, sc5;
  wh_linear *conv3 = nullptr, *conv6 = nullptr, *pre_out = nullptr, *joint_enc = nullptr;
  // TDT decoder (host)
  int hidden = 0, joint = 0, classes = 0, max_symbols = 10, lstm_layers = 0;
  bool global = false;
  std::vector<int> durations;
  HostMat embed_h, pred_w, out_w;
  std::vector<HostMat> wx, wh;
  std::vector<std::vector<float>> lstm_b;
  std::vector<float> pred_b, out_b;
  // The same decoder on the device (greedy.hip): [Wx | Wh] per LSTM layer with its bias, the joint's
  // projections, the embedding table in f32; the loop's buffers (tdt_bufs) and (token, frame) list.
  std::vector<wh_linear *> tdt_lstm;
  wh_linear *tdt_pred = nullptr, *tdt_out = nullptr;
  float *tdt_embed = nullptr, *tdt_buf = nullptr;
  uint32_t *tdt_list = nullptr;
  int tdt_list_cap = 0;
  // Greedy CTC on the device: [ids (frames) | count | pairs], sized for ctc_cap frames.
  int *ctc_buf = nullptr;
  int ctc_cap = 0;
  // The log-mel frontend: GigaAM's and Whisper's window and filterbank [mels][n_fft / 2 + 1] from the
  // GGUF (empty when the file has none), and the device plan built at the first wh_model_mel.
  std::vector<float> fe_window, fe_filters;
  struct MelDev {
    bool ready = false;
    int kind = 0, n = 0, mels = 0, leaf = 0, stages = 0;
    float silent = 0.0f;
    uint8_t *buf = nullptr;  // every table and the scratch float in one allocation
    MelArgs args{};
    float *scratch = nullptr;
  } mel;
  // Whisper
  int frames = 1500, dec_layers = 0, dec_heads = 0, dec_ff = 0, vocab = 0, context = 0;
  wh_linear *wconv0 = nullptr, *wconv1 = nullptr, *token_embd = nullptr;
  float *enc_pos = nullptr, *dec_pos = nullptr;
  std::vector<WBlock> wblocks;
  std::vector<DLayer> dl;
  Chan enc_norm, dec_norm;
  // Arena (device activations), sized for `cap` encoder frames × `cap_batch` windows.
  int cap = 0, cap_batch = 0;
  float *x = nullptr, *y = nullptr, *h = nullptr, *qk = nullptr, *yr = nullptr, *pos = nullptr, *sub = nullptr;
  void *pos16 = nullptr;            // Parakeet: the position table as f16 (the pos GEMM's input)
  // Parakeet: every block's linear_pos stacked along rows, and the projected position rows of a call,
  // f16 [2t + 15][layers · d] (block i's at column i · d).
  wh_linear *pos_all = nullptr;
  void *posp = nullptr;
  // Device tags of the position projection's outputs: the frame count t whose projection posp ([0])
  // and ppk ([1]) hold (0: none).  The projection depends on t and the weights only, so a call at the
  // tagged t skips its GEMM (decided on the device: a recorded pass stays right whatever t a later
  // call leaves there).
  int *pos_tag = nullptr;
  const void *pos16_cur = nullptr;  // its rows of this call
  int *valid_dev = nullptr;
  float *sub2 = nullptr;   // Parakeet conv3 output (the subsampling's second buffer)
  // Parakeet: every block's position rows in attention's packed layout for one window,
  // [layer · head][prows][hd] f16, zero where no call writes.
  _Float16 *ppk = nullptr;
  float *rope = nullptr;   // GigaAM rope table for `cap` frames
  const float *pos_cur = nullptr;  // Parakeet: the positions of this call (rows from cap - t)
  // Recorded encoder calls (HIP graphs), keyed by the call's arguments and the generations of the
  // buffers they were recorded on; replayed instead of re-issuing their ~500 launches.
  struct Graph {
    std::vector<intptr_t> key;
    hipGraphExec_t exec = nullptr;
    hipGraph_t graph = nullptr;  // kept for the life of its exec (as a recorded pass keeps it)
  };
  std::vector<Graph> graphs;
  std::vector<intptr_t> pending;  // the arguments of the last eager call
  bool use_graph = true;
  long epoch = 0;  // arena generation
  // Whisper decoding state.
  float *dx = nullptr, *dy = nullptr, *dqkv = nullptr, *dh = nullptr, *datt = nullptr, *dpart = nullptr,
        *dscratch = nullptr;
  uint32_t *ids = nullptr;
  std::vector<uint32_t *> own, cross;
  int cross_frames = 0;
  // Whisper's special ids and suppression lists (src/whisper/mod.rs:131-141, :177), and the device
  // logits of the window search's steps.
  int eot = -1, no_timestamps = -1, sot = -1;
  std::vector<int> suppress, begin_suppress;
  float *dlogits = nullptr;
  // The device window search: [WhisperState | generated ids (WHISPER_MAX_NEW) | partials | suppression mask].
  float *wsearch = nullptr;
};

namespace {

int fail(wh_model *m, const std::string &msg, int code = WH_EARG) { return wh_fail(m->ctx, code, "%s", msg.c_str()); }

#define CK(expr)             \
  do {                       \
    int rc_ = (expr);        \
    if (rc_) return rc_;     \
  } while (0)

float *dev_alloc(wh_model *m, size_t n) {
  float *p = nullptr;
  if (wh_alloc(m->ctx, n, &p)) return nullptr;
  m->owned.push_back(p);
  return p;
}

// Conformer config (src/conformer.rs:34-61).
bool conformer_config(const Gguf &g, wh_model *m, const std::string &arch, std::string &err) {
  auto u = [&](const char *name) { return (int)g.integer("stt." + arch + ".encoder." + name, -1); };
  m->layers = u("n_layers");
  m->d = u("d_model");
  m->heads = u("n_heads");
  m->d_ff = u("d_ff");
  m->kernel = u("conv_kernel");
  std::string cn = g.string("stt." + arch + ".encoder.conv_norm_type");
  if (cn != "layer_norm" && cn != "batch_norm") return err = "unsupported conv_norm_type \"" + cn + "\"", false;
  m->layer_norm_conv = cn == "layer_norm";
  int d = m->d, heads = m->heads;
  if (m->layers <= 0 || d <= 0 || heads <= 0 || d % heads || d > 1024 || d / heads > 128 || (d / heads) % 2) {
    err = "unsupported attention shape: d_model " + std::to_string(d) + ", " + std::to_string(heads) + " heads";
    return false;
  }
  if (m->kernel <= 0 || m->kernel % 2 == 0) return err = "conv kernel " + std::to_string(m->kernel) + ": only odd kernels are supported", false;
  if ((d / heads) % 4) return err = "head_dim must be a multiple of 4 on this backend", false;
  return true;
}

// Block::load (src/conformer.rs:180-229).
void load_block(Loader &L, wh_model *m, int i, Block &k) {
  int d = m->d, hd = d / m->heads;
  std::string p = "enc.blocks." + std::to_string(i) + ".";
  bool bias = !m->relative;  // GigaAM has layer biases, Parakeet none
  k.norm_ff1 = L.norm(p + "norm_ff1", d, true);
  k.ff1[0] = L.linear({p + "ff1.linear1"}, bias);
  k.ff1[1] = L.linear({p + "ff1.linear2"}, bias);
  k.norm_attn = L.norm(p + "norm_attn", d, true);
  if (!m->relative) {
    k.qk = L.linear({p + "attn.linear_q", p + "attn.linear_k"}, bias);
    k.v = L.linear({p + "attn.linear_v"}, bias);
  } else {
    // [q | k | v] with biases [pos_bias_u | 0 | 0], and q again with pos_bias_v (dual outputs).
    auto u = L.f32s(p + "attn.pos_bias_u", (size_t)hd * m->heads);
    auto v = L.f32s(p + "attn.pos_bias_v", (size_t)hd * m->heads);
    std::vector<float> b(u);
    b.insert(b.end(), 2 * (size_t)d, 0.0f);
    b.insert(b.end(), v.begin(), v.end());
    k.qkv = L.linear({p + "attn.linear_q", p + "attn.linear_k", p + "attn.linear_v"}, false, -1, b);
    // linear_pos: loaded for all blocks at once (the model's pos_all).
  }
  k.out = L.linear({p + "attn.linear_out"}, bias);
  k.norm_conv = L.norm(p + "norm_conv", d, true);
  k.pw1 = L.glu_groups(p + "conv.pointwise1", bias, &k.pw1_groups);
  if (m->layer_norm_conv) {
    k.conv_norm = L.norm(p + "conv.ln", d, true);
  } else {
    // batch_norm (src/conformer.rs:132-139): x·scale + shift.
    auto w = L.f32s(p + "conv.bn.weight", d), b = L.f32s(p + "conv.bn.bias", d);
    auto mean = L.f32s(p + "conv.bn.running_mean", d), var = L.f32s(p + "conv.bn.running_var", d);
    std::vector<float> scale(d), shift(d);
    for (int c = 0; c < d; c++) {
      scale[c] = w[c] / std::sqrt(var[c] + 1e-5f);
      shift[c] = b[c] - mean[c] * scale[c];
    }
    k.conv_norm.w = L.upload(scale);
    k.conv_norm.b = L.upload(shift);
  }
  // Depthwise taps [d][kernel] as the file stores them (the GPU layout).
  k.dw.w = L.upload(L.f32s(p + "conv.depthwise.weight", (size_t)d * m->kernel));
  k.dw.b = L.upload(bias ? L.f32s(p + "conv.depthwise.bias", d) : std::vector<float>(d, 0.0f));
  k.pw2 = L.linear({p + "conv.pointwise2"}, bias);
  k.norm_ff2 = L.norm(p + "norm_ff2", d, true);
  k.ff2[0] = L.linear({p + "ff2.linear1"}, bias);
  k.ff2[1] = L.linear({p + "ff2.linear2"}, bias);
  k.norm_out = L.norm(p + "norm_out", d, true);
}

HostMat host_mat(Loader &L, const std::string &name) {
  HostMat h;
  const Tensor *t = L.need(name);
  if (!t) return h;
  h.k = (int)t->dims[0];
  h.rows = (int)(t->count() / h.k);
  h.w = to_f32(*t);
  return h;
}

bool load_parakeet(const Gguf &g, Loader &L, wh_model *m, std::string &err) {
  m->relative = true;
  if (!conformer_config(g, m, "parakeet", err)) return false;
  m->mels = (int)g.integer("stt.frontend.num_mels", -1);
  m->ch = (int)g.integer("stt.parakeet.encoder.subsampling_channels", -1);
  if (m->mels <= 0 || m->ch <= 0 || m->ch > 4096) return err = "bad Parakeet subsampling metadata", false;
  // 3×3 taps [ch][time tap][freq tap] → [tap][ch] (src/parakeet/encoder.rs:54-59).
  auto taps = [&](int i) {
    std::string p = "enc.pre_encode.conv." + std::to_string(i);
    auto w = L.f32s(p + ".weight", (size_t)9 * m->ch);
    std::vector<float> t(9 * (size_t)m->ch);
    for (size_t e = 0; e < t.size(); e++) t[e] = w[(e % m->ch) * 9 + e / m->ch];
    Chan c;
    c.w = L.upload(t);
    c.b = L.upload(L.f32s(p + ".bias", m->ch));
    return c;
  };
  m->sc0 = taps(0);
  m->sc2 = taps(2);
  m->sc5 = taps(5);
  m->conv3 = L.linear({"enc.pre_encode.conv.3"}, true);
  m->conv6 = L.linear({"enc.pre_encode.conv.6"}, true);
  m->pre_out = L.linear({"enc.pre_encode.out"}, true);
  m->joint_enc = L.linear({"joint.enc"}, true);
  m->blocks.resize(m->layers);
  for (int i = 0; i < m->layers && L.err.empty(); i++) load_block(L, m, i, m->blocks[i]);
  {
    // The position rows do not depend on the input: one GEMM per call projects them for every block
    // (rows of the blocks' linear_pos stacked), instead of one per block.
    std::vector<std::string> names;
    for (int i = 0; i < m->layers; i++) names.push_back("enc.blocks." + std::to_string(i) + ".attn.linear_pos");
    m->pos_all = L.linear(names, false);
  }
  // TDT decoder (src/parakeet/decoder.rs:46-89), kept on the host as the reference keeps it.
  m->blank = (int)g.integer("tokenizer.ggml.blank_token_id", -1);
  m->hidden = (int)g.integer("stt.parakeet.predictor.hidden", -1);
  m->joint = (int)g.integer("stt.parakeet.joint.hidden", -1);
  m->max_symbols = (int)g.integer("stt.parakeet.tdt.max_symbols", 10);
  m->global = g.string("stt.parakeet.tdt.symbol_budget") == "global";
  for (long v : g.ints("stt.parakeet.tdt.durations")) m->durations.push_back((int)v);
  m->lstm_layers = (int)g.integer("stt.parakeet.predictor.n_layers", 1);
  if (g.tensor("pred.embed.weight") && !m->durations.empty()) {
    m->embed_h = host_mat(L, "pred.embed.weight");
    m->classes = m->embed_h.rows;
    for (int l = 0; l < m->lstm_layers; l++) {
      std::string p = "pred.lstm." + std::to_string(l);
      m->wx.push_back(host_mat(L, p + ".Wx"));
      m->wh.push_back(host_mat(L, p + ".Wh"));
      m->lstm_b.push_back(L.f32s(p + ".bias", (size_t)4 * m->hidden));
    }
    m->pred_w = host_mat(L, "joint.pred.weight");
    m->pred_b = L.f32s("joint.pred.bias", m->joint);
    m->out_w = host_mat(L, "joint.out.weight");
    m->out_b = L.f32s("joint.out.bias", (size_t)(m->classes + m->durations.size()));
    // The device copy; the joined LSTM layers need whole blocks of the hidden size.
    if (m->hidden % 32 == 0 && m->embed_h.k == m->hidden && m->durations.size() <= 16) {
      for (int l = 0; l < m->lstm_layers; l++) {
        std::string p = "pred.lstm." + std::to_string(l);
        m->tdt_lstm.push_back(L.joined({p + ".Wx", p + ".Wh"}, m->lstm_b[l]));
      }
      m->tdt_pred = L.linear({"joint.pred"}, true);
      m->tdt_out = L.linear({"joint.out"}, true);
      m->tdt_embed = L.upload(m->embed_h.w);
    }
  }
  return L.err.empty();
}

bool load_gigaam(const Gguf &g, Loader &L, wh_model *m, std::string &err) {
  if (g.string("stt.gigaam.encoder.self_attention_model") != "rotary")
    return err = "stt.gigaam.encoder.self_attention_model must be \"rotary\"", false;
  m->relative = false;
  if (!conformer_config(g, m, "gigaam", err)) return false;
  m->mels = (int)g.integer("stt.frontend.num_mels", -1);
  if (g.tensor("frontend.window") && g.tensor("frontend.mel_filterbank") && m->mels > 0) {
    m->fe_window = L.f32s("frontend.window", 320);
    m->fe_filters = L.f32s("frontend.mel_filterbank", (size_t)161 * m->mels);
  }
  m->theta = (double)g.integer("stt.gigaam.encoder.pos_emb_max_len", 5000);
  m->conv0 = L.linear({"enc.pre_encode.conv.0"}, true);
  m->conv2 = L.linear({"enc.pre_encode.conv.2"}, true);
  bool rnnt = g.string("stt.gigaam.head_kind") == "rnnt";
  m->head = L.linear({rnnt ? "joint.enc" : "head.ctc"}, true);
  const Tensor *ht = g.tensor(rnnt ? "joint.enc.weight" : "head.ctc.weight");
  m->outputs = ht ? (int)ht->dims.back() : 0;
  m->blank = (int)g.integer("tokenizer.ggml.blank_token_id", -1);
  m->blocks.resize(m->layers);
  for (int i = 0; i < m->layers && L.err.empty(); i++) load_block(L, m, i, m->blocks[i]);
  return L.err.empty();
}

bool load_whisper(const Gguf &g, Loader &L, wh_model *m, std::string &err) {
  auto u = [&](const char *k) { return (int)g.integer(std::string("stt.whisper.") + k, -1); };
  m->d = u("encoder.d_model");
  m->heads = u("encoder.n_heads");
  m->layers = u("encoder.n_layers");
  m->d_ff = u("encoder.ffn_dim");
  m->dec_heads = u("decoder.n_heads");
  m->dec_layers = u("decoder.n_layers");
  m->dec_ff = u("decoder.ffn_dim");
  m->vocab = u("decoder.vocab_size");
  m->context = u("decoder.max_target_positions");
  m->mels = u("encoder.num_mel_bins");
  m->frames = u("encoder.max_source_positions");
  int d = m->d;
  for (int heads : {m->heads, m->dec_heads}) {
    if (d <= 0 || heads <= 0 || d % heads || d / heads > 64 || (d / heads) % 8)
      return err = "unsupported shape: d_model " + std::to_string(d) + ", " + std::to_string(heads) + " heads", false;
  }
  if (m->frames <= 0 || m->mels <= 0 || m->vocab <= 0 || m->context <= 0) return err = "bad Whisper metadata", false;
  if (g.tensor("frontend.window") && g.tensor("frontend.mel_filterbank")) {
    m->fe_window = L.f32s("frontend.window", 400);
    m->fe_filters = L.f32s("frontend.mel_filterbank", (size_t)201 * m->mels);
  }
  m->wconv0 = L.linear({"enc.conv.0"}, true, -1, {}, 1);
  m->wconv1 = L.linear({"enc.conv.1"}, true, -1, {}, 1);
  m->enc_pos = L.upload(L.f32s("enc.pos_emb.weight", (size_t)d * m->frames));
  m->wblocks.resize(m->layers);
  for (int i = 0; i < m->layers && L.err.empty(); i++) {
    std::string p = "enc.blocks." + std::to_string(i) + ".";
    WBlock &b = m->wblocks[i];
    b.norm_attn = L.norm(p + "norm_attn", d, true);
    b.qkv = L.linear({p + "attn.q", p + "attn.k", p + "attn.v"}, true, 1);
    b.out = L.linear({p + "attn.out"}, true);
    b.norm_ffn = L.norm(p + "norm_ffn", d, true);
    b.fc1 = L.linear({p + "ffn.fc1"}, true);
    b.fc2 = L.linear({p + "ffn.fc2"}, true);
  }
  m->enc_norm = L.norm("enc.final_norm", d, true);
  m->dl.resize(m->dec_layers);
  for (int i = 0; i < m->dec_layers && L.err.empty(); i++) {
    std::string p = "dec.blocks." + std::to_string(i) + ".";
    DLayer &l = m->dl[i];
    l.norm_self = L.norm(p + "norm_self", d, true);
    l.qkv = L.linear({p + "self_attn.q", p + "self_attn.k", p + "self_attn.v"}, true, 1);
    l.self_out = L.linear({p + "self_attn.out"}, true);
    l.norm_cross = L.norm(p + "norm_cross", d, true);
    l.cross_q = L.linear({p + "cross_attn.q"}, true);
    l.cross_kv = L.linear({p + "cross_attn.k", p + "cross_attn.v"}, true, 0);
    l.cross_out = L.linear({p + "cross_attn.out"}, true);
    l.norm_ffn = L.norm(p + "norm_ffn", d, true);
    l.fc1 = L.linear({p + "ffn.fc1"}, true);
    l.fc2 = L.linear({p + "ffn.fc2"}, true);
  }
  m->dec_norm = L.norm("dec.final_norm", d, true);
  m->eot = (int)g.integer("tokenizer.ggml.eos_token_id", -1);
  m->no_timestamps = (int)g.integer("stt.whisper.no_timestamps_token_id", -1);
  m->sot = (int)g.integer("stt.whisper.sot_token_id", -1);
  // The converter writes a suppress list only when it is not empty (src/whisper/mod.rs:131-133).
  for (long v : g.ints("stt.whisper.suppress_tokens")) m->suppress.push_back((int)v);
  for (long v : g.ints("stt.whisper.begin_suppress_tokens")) m->begin_suppress.push_back((int)v);
  {
    bool ok = m->eot >= 0 && m->eot < m->vocab && m->no_timestamps >= 0 && m->no_timestamps + 1 < m->vocab &&
              m->sot >= 0 && m->sot < m->vocab;
    for (int id : m->suppress) ok = ok && id >= 0 && id < m->vocab;
    for (int id : m->begin_suppress) ok = ok && id >= 0 && id < m->vocab;
    if (!ok) return err = "special token ids out of the vocabulary", false;
  }
  m->token_embd = L.linear({"dec.token_embd"}, false);
  m->dec_pos = L.upload(L.f32s("dec.pos_emb.weight", (size_t)d * m->context));
  return L.err.empty();
}

// rel_positions (src/conformer.rs:144-153): rows of [sin, cos] pairs from position `first` down.
std::vector<float> rel_positions(int d, long first, int rows) {
  std::vector<float> div(d / 2), out((size_t)rows * d);
  for (int k = 0; k < d / 2; k++) div[k] = std::exp((float)(2 * k) * (-std::log(10000.0f) / (float)d));
  for (int r = 0; r < rows; r++) {
    float p = (float)(first - r);
    for (int k = 0; k < d / 2; k++) {
      out[(size_t)r * d + 2 * k] = std::sin(p * div[k]);
      out[(size_t)r * d + 2 * k + 1] = std::cos(p * div[k]);
    }
  }
  return out;
}

// The GigaAM rope table (src/gigaam/mod.rs:86-97), f64 then f32.
std::vector<float> rope_table(int frames, int hd, double theta) {
  std::vector<float> out((size_t)frames * hd);
  for (int t = 0; t < frames; t++)
    for (int i = 0; i < hd / 2; i++) {
      double a = (double)t * std::pow(theta, -2.0 * i / hd);
      out[(size_t)t * hd + i] = (float)std::cos(a);
      out[(size_t)t * hd + hd / 2 + i] = (float)std::sin(a);
    }
  return out;
}

int parakeet_frames(int mel_frames) { return half_len(half_len(half_len(mel_frames - 1))); }

// Grows the arena to `frames` encoder frames × `batch` windows (rounded up to 64 frames).
// A recorded graph is destroyed only once the stream has drained: a launch of it may still be queued
// (replays are asynchronous), and destroying an exec with a pending launch leaves the runtime (and
// any tool that follows the launch, such as a kernel tracer) holding freed state.
// The graph the exec was instantiated from lives as long as the exec: a launch tracer can refer back
// to the graph's nodes when the exec is launched (a kernel trace of the replayed TDT loop and window
// search read freed memory when the graph was destroyed right after instantiation).
void destroy_graph(wh_model *m, hipGraphExec_t exec, hipGraph_t graph, bool &drained) {
  if (!drained) {
    (void)hipStreamSynchronize(m->ctx->stream);
    drained = true;
  }
  (void)hipGraphExecDestroy(exec);
  if (graph) (void)hipGraphDestroy(graph);
}

void drop_graphs(wh_model *m) {
  bool drained = false;
  for (auto &g : m->graphs) destroy_graph(m, g.exec, g.graph, drained);
  m->graphs.clear();
  m->pending.clear();
}

int arena(wh_model *m, int frames, int batch) {
  if (frames <= m->cap && batch <= m->cap_batch) return WH_OK;
  drop_graphs(m);
  m->epoch++;
  int F = (std::max(frames, m->cap) + 63) / 64 * 64, B = std::max(batch, std::max(m->cap_batch, 1));
  for (float *p : {m->x, m->y, m->h, m->qk, m->yr, m->pos, m->sub, m->sub2, m->rope, (float *)m->pos16, (float *)m->posp,
                   (float *)m->ppk, (float *)m->pos_tag})
    if (p) {
      wh_free(m->ctx, p);
      for (auto &o : m->owned)
        if (o == p) o = nullptr;
    }
  if (m->valid_dev) wh_free(m->ctx, m->valid_dev);
  m->x = m->y = m->h = m->qk = m->yr = m->pos = m->sub = m->sub2 = m->rope = nullptr;
  m->pos16 = m->posp = m->ppk = nullptr;
  m->pos_tag = nullptr;
  m->valid_dev = nullptr;
  const int d = m->d;
  const size_t rows = (size_t)F * B;
  // yr: the projected positions (2F + 15 rows), rotary rows or the next block's first norm (f16).
  size_t hsz = rows * std::max(m->d_ff, d), qsz = rows * 4 * d,
         ysz = std::max((size_t)(2 * F + 15 + 64) * d, (rows * d + 1) / 2), sub = 0;
  if (m->arch == PARAKEET) {
    // The subsampling unchunked: conv2/conv3 outputs (2F + 1) rows of [MELS / 4][ch] per window, and
    // conv5's [F][MELS / 8][ch].
    int f2 = half_len(half_len(m->mels)), f = half_len(f2);
    sub = (size_t)(2 * F + 1) * f2 * m->ch * B;
    hsz = std::max(hsz, rows * f * m->ch);
    qsz = std::max(qsz, rows * f * m->ch);
  } else if (m->arch == GIGAAM) {
    hsz = std::max(hsz, (size_t)2 * rows * ((5 * m->mels + 31) / 32 * 32));
    hsz = std::max(hsz, rows * 5 * d);
    qsz = std::max(qsz, 2 * rows * d);
  } else {
    // Whisper: conv columns (2F rows of 3·mels, F rows of 3·d) in qk, conv0's output 2F × d in h.
    qsz = std::max(qsz, (size_t)2 * F * ((3 * m->mels + 31) / 32 * 32));
    qsz = std::max(qsz, (size_t)F * 3 * d);
    hsz = std::max(hsz, (size_t)2 * F * d);
  }
  m->x = dev_alloc(m, rows * d);
  m->y = dev_alloc(m, rows * d);
  m->h = dev_alloc(m, hsz);
  m->qk = dev_alloc(m, qsz);
  m->yr = dev_alloc(m, ysz);
  m->pos = dev_alloc(m, ysz);
  if (sub) {
    m->sub = dev_alloc(m, sub);
    m->sub2 = dev_alloc(m, sub);
  }
  if (wh_alloc(m->ctx, B, (float **)&m->valid_dev)) return WH_EOOM;
  if (!m->x || !m->y || !m->h || !m->qk || !m->yr || !m->pos || (sub && (!m->sub || !m->sub2)))
    return wh_fail(m->ctx, WH_EOOM, "arena of %d frames x %d windows: out of device memory", F, B);
  // Attention's split operands for the largest call, so that encoding allocates nothing.
  if (!wh_scratch(m->ctx, attention_scratch_bytes(m->ctx, F, m->heads, d / m->heads, B, m->arch == PARAKEET)))
    return WH_EOOM;
  if (m->arch == PARAKEET) {
    // The sinusoidal table for F frames stays on the device; a call over t frames reads its
    // pos_rows(t) rows from row F − t (src/parakeet/encoder.rs:93, :129-131).
    auto table = rel_positions(d, (long)F + 15, 2 * F + 15);
    CK(wh_write(m->ctx, m->pos, table.data(), table.size() * 4));
    m->pos16 = dev_alloc(m, (table.size() + 1) / 2);
    m->posp = dev_alloc(m, ((size_t)(2 * F + 15) * m->layers * d + 1) / 2);
    m->pos_tag = (int *)dev_alloc(m, 2);
    if (!m->pos16 || !m->posp || !m->pos_tag) return WH_EOOM;
    CK(launch_zero(m->ctx, m->pos_tag, 2 * sizeof(int)));  // no projection held yet
    const int hd = d / m->heads;
    if (hd == 32 || hd == 64 || hd == 128) {
      int most = 0, tk, pfront, prows;
      for (int t = 1; t <= F; t++) attention_layout(t, m->heads, hd, 1, &tk, &pfront, &prows), most = std::max(most, prows);
      const size_t n = (size_t)m->layers * d * most;  // halves
      m->ppk = (_Float16 *)dev_alloc(m, (n + 1) / 2);
      if (!m->ppk) return WH_EOOM;
      CK(launch_zero(m->ctx, m->ppk, n * 2));  // a fill kernel on the context's stream
    }
    CK(launch_to_half(m->ctx, m->pos, m->pos16, table.size()));
  } else if (m->arch == GIGAAM) {
    int hd = d / m->heads;
    auto t = rope_table(F, hd, m->theta);
    m->rope = dev_alloc(m, t.size());
    if (!m->rope) return WH_EOOM;
    CK(wh_write(m->ctx, m->rope, t.data(), t.size() * 4));
  }
  m->cap = F;
  m->cap_batch = B;
  return WH_OK;
}

// Conformer Block::record (src/conformer.rs:232-265) over `batch` windows of t frames in x; the
// block's output goes to y.  `valid_dev` (or none) masks keys and conv inputs per window.  The
// residual stream x stays f32; every activation whose only consumer is a GEMM (the norms' outputs,
// the first FFN projections, attention and the conv module) is written as f16, the rounding that
// GEMM applies to its input anyway (src/cpu/gemm.rs:163-176), into f16 views of the arena buffers.
// One block from x into y (y = norm_out(x), x is spent).  pre: the block's first norm (norm_ff1 of x)
// is already in m->yr as f16 (the previous block's last kernel wrote it); next: the following
// block's norm_ff1, which this block's last kernel then writes into m->yr.
// Whether a Parakeet call's attention takes its operands packed by the projections themselves: one
// window (padded batches pack per call), head dims the packed layout holds unpadded.
bool packed_attention(const wh_model *m, int batch, const int *valid_dev) {
  const int hd = m->d / m->heads;
  return m->relative && m->ppk && batch == 1 && !valid_dev && (hd == 32 || hd == 64 || hd == 128) && !m->ctx->unfused;
}

int record_block(wh_model *m, int layer, const Block &k, float *x, float *y, int t, int batch, const int *valid_dev,
                 bool pre, const Chan *next, bool out16) {
  wh_ctx *c = m->ctx;
  const int d = m->d, hd = d / m->heads, rows = t * batch;
  void *y16 = y, *h16 = m->h;
  auto g16 = [&](const void *a, const wh_linear *l, void *out, int r, int epi, float alpha, int o16) {
    return launch_gemm_h(c, a, l, out, r, l->cols + l->dual, epi, alpha, o16);
  };
  auto ln16 = [&](const Chan &n) { return launch_layer_norm(c, x, n.w, n.b, y16, rows, d, nullptr, nullptr, 0, 1); };
  if (!pre) CK(ln16(k.norm_ff1));
  CK(g16(pre ? (const void *)m->yr : y16, k.ff1[0], h16, rows, WH_SILU, 0.0f, 1));
  if (!m->relative) {
    CK(g16(h16, k.ff1[1], x, rows, WH_RESIDUAL, 0.5f, 0));
    void *yr16 = m->yr;
    CK(launch_layer_norm(c, x, k.norm_attn.w, k.norm_attn.b, y16, rows, d, m->rope, yr16, hd, 1));
    CK(g16(yr16, k.qk, m->qk, rows, WH_BIAS, 0.0f, 1));
    CK(g16(y16, k.v, m->h, rows, WH_BIAS, 0.0f, 1));
    CK(launch_attention(c, m->qk, m->h, nullptr, y16, t, m->heads, hd, valid_dev, t, batch, 1, 1));
  } else {
    // The FFN's residual projection and the attention norm (one kernel after a k-split GEMM).
    CK(launch_gemm_h_ln(c, h16, k.ff1[1], x, rows, 0.5f, k.norm_attn.w, k.norm_attn.b, y16, 1));
    // This block's projected position rows (record_blocks projected every block's).
    const int ps = m->pos_all->cols;
    const _Float16 *pos = (const _Float16 *)m->posp + (size_t)layer * d;
    if (packed_attention(m, batch, valid_dev)) {
      // One window: the projection writes K and Vᵀ in attention's packed layout (after its f16 rows
      // in qk) and record_blocks wrote every block's position rows packed: no packing launch.
      int tk, pfront, prows;
      attention_layout(t, m->heads, hd, 1, &tk, &pfront, &prows);
      _Float16 *q16 = (_Float16 *)m->qk, *kp = q16 + (size_t)m->cap * 4 * d, *vt = kp + (size_t)m->cap * d;
      const HeadsOut outs[2] = {{kp, d, d, hd, tk, 0, false}, {vt, 2 * d, d, hd, tk, 0, true}};
      CK(launch_gemm_h_heads(c, y16, k.qkv, m->qk, rows, k.qkv->cols + k.qkv->dual, WH_BIAS, outs, 2));
      CK(launch_attention_packed(c, q16, 4 * d, q16 + 3 * d, kp, vt, m->ppk + (size_t)layer * d * prows, y16, t,
                                 m->heads, hd, 1));
    } else {
      CK(g16(y16, k.qkv, m->qk, rows, WH_BIAS, 0.0f, 1));
      CK(launch_attention(c, m->qk, nullptr, pos, y16, t, m->heads, hd, valid_dev, t, batch, 1, 1, ps));
    }
  }
  // The residual projections and the norm after them: one fused finish + LayerNorm kernel when the
  // GEMM's plan splits k, else the GEMM's residual epilogue and a LayerNorm launch.
  CK(launch_gemm_h_ln(c, y16, k.out, x, rows, 1.0f, k.norm_conv.w, k.norm_conv.b, y16, 1));
  // The conv module: pw1 and its GLU in one GEMM (its epilogue) when pw1's rows are in GLU groups,
  // then the depthwise conv, norm and SiLU.
  int glu = 0;  // the layout of pw1's output for launch_conv_glu
  if (k.pw1_groups && !c->unfused && gemm_glu_ok(k.pw1, m->qk)) {
    CK(launch_gemm_h(c, y16, k.pw1, m->qk, rows, k.pw1->cols / 2, EPI_GLU, 0.0f, 0));
    glu = 2;
  } else {
    CK(g16(y16, k.pw1, m->qk, rows, WH_BIAS, 0.0f, 0));
    glu = k.pw1_groups ? 1 : 0;
  }
  CK(launch_conv_glu(c, m->qk, k.dw.w, k.dw.b, m->kernel, k.conv_norm.w, k.conv_norm.b, m->layer_norm_conv, y16, t, d,
                     valid_dev, t, batch, 1, glu));
  CK(launch_gemm_h_ln(c, y16, k.pw2, x, rows, 1.0f, k.norm_ff2.w, k.norm_ff2.b, y16, 1));
  CK(g16(y16, k.ff2[0], h16, rows, WH_SILU, 0.0f, 1));
  // The block output is norm_out(x), not the residual stream (x is not stored again); f16 (out16) when
  // its only reader is the GEMM after the last block.
  return launch_gemm_h_ln(c, h16, k.ff2[1], x, rows, 0.5f, k.norm_out.w, k.norm_out.b, y, out16 ? 1 : 0, 0,
                          next ? next->w : nullptr, next ? next->b : nullptr, next ? m->yr : nullptr);
}

}  // namespace

namespace {

// The position projection of a t-frame call into output `which` (0: posp, 1: ppk) by gemm(): tagged
// with t on the device, so that the GEMM skips while its output holds t's projection.  A call over
// fewer than all blocks (whole: false) packs only theirs: it runs untagged and clears the tag.
template <class F>
int position_projection(wh_model *m, int t, int which, bool whole, F &&gemm) {
  if (m->ctx->no_position_cache || !whole) {
    if (int rc = gemm()) return rc;
    return launch_set_int(m->ctx, m->pos_tag + which, 0);
  }
  m->ctx->gemm_skip = m->pos_tag + which;
  m->ctx->gemm_skip_val = t;
  const int rc = gemm();
  m->ctx->gemm_skip = nullptr;
  if (rc) return rc;
  return launch_set_int(m->ctx, m->pos_tag + which, t);
}

// Conformer::record (src/conformer.rs:107-116): `layers` blocks from m->x, output in m->x — f32, or
// with out16 f16 (the f32 values rounded, RNE, as the GEMM reading them would round them).  pre: the
// first block's norm_ff1 of m->x is already in m->yr (f16).
int record_blocks(wh_model *m, int t, int batch, const int *valid_dev, int layers, bool out16 = false,
                  bool pre = false) {
  if (m->relative && layers > 0) {  // every block's linear_pos(P) in one GEMM: [2t + 15][layers · d] f16
    if (packed_attention(m, batch, valid_dev)) {
      // One window: written as attention's packed position rows, [layer · head][prows][hd] from row
      // pfront (the rows around them stay zero from the arena's allocation).
      const int hd = m->d / m->heads;
      int tk, pfront, prows;
      attention_layout(t, m->heads, hd, 1, &tk, &pfront, &prows);
      const HeadsOut out{m->ppk, 0, layers * m->d, hd, prows, pfront, false};
      CK(position_projection(m, t, 1, layers == m->layers, [&] {
        return launch_gemm_h_heads(m->ctx, m->pos16_cur, m->pos_all, m->posp, 2 * t + 15, m->pos_all->cols, WH_BIAS,
                                   &out, 1);
      }));
    } else {
      CK(position_projection(m, t, 0, layers == m->layers, [&] {
        return launch_gemm_h(m->ctx, m->pos16_cur, m->pos_all, m->posp, 2 * t + 15, m->pos_all->cols, WH_BIAS, 0.0f, 1);
      }));
    }
  }
  for (int i = 0; i < layers; i++) {
    const Chan *next = i + 1 < layers ? &m->blocks[i + 1].norm_ff1 : nullptr;
    CK(record_block(m, i, m->blocks[i], m->x, m->y, t, batch, valid_dev, i > 0 || pre, next, out16 && !next));
    std::swap(m->x, m->y);
  }
  return WH_OK;
}

int lin(wh_model *m, const float *a, const wh_linear *l, float *c, int rows, int epi, float alpha = 0.0f) {
  return launch_gemm(m->ctx, a, l, c, rows, l->cols + l->dual, epi, alpha);
}

// The same with `a` already f16, the output f32 or (out16) f16.
int lin_h(wh_model *m, const _Float16 *a, const wh_linear *l, void *c, int rows, int epi, int out16) {
  return launch_gemm_h(m->ctx, a, l, c, rows, l->cols + l->dual, epi, 0.0f, out16);
}

// Parakeet Encoder::record (src/parakeet/encoder.rs:103-124) over `batch` windows of mel_frames
// [batch][mel_frames][mels]; window b's first valid[b] mel frames are real.  One window: kestrel
// masking as the reference (conv0/conv2 see the valid frames, conv5 the whole image).  Several
// windows: each is subsampled as if alone (conv5 sees its own valid image rows), and its keys and
// conv inputs past its own encoder frames are masked.
// The window's encoder frames for Parakeet, and for batched windows each window's valid ones.
std::vector<int> parakeet_valid(int batch, int mel_frames, int t, const int *valid) {
  std::vector<int> enc_valid(batch);
  for (int b = 0; b < batch; b++) {
    int v = std::min(std::max(valid[b], 1), mel_frames);
    enc_valid[b] = batch == 1 ? t : std::min(t, parakeet_frames(std::max(v, 3)));
  }
  return enc_valid;
}

int parakeet_record(wh_model *m, const float *mel, int batch, int mel_frames, const int *valid, float *out) {
  const int mels = m->mels, ch = m->ch;
  const int t2 = half_len(half_len(mel_frames)), f2 = half_len(half_len(mels));
  const int t = parakeet_frames(mel_frames), f = half_len(f2);
  wh_ctx *c = m->ctx;
  const int rows1 = 2 * t + 1;  // conv2's output rows from −1 on
  const size_t per = (size_t)rows1 * f2 * ch;
  // The outputs whose only reader is a GEMM (which rounds its input to f16, RNE, as these kernels
  // round their stores) are f16: conv2's (into sub), conv5's (into h), conv6's and the flattened rows.
  // conv3's output stays f32: the depthwise conv5 reads it at full precision.
  _Float16 *sub16 = (_Float16 *)m->sub, *h16 = (_Float16 *)m->h, *qk16 = (_Float16 *)m->qk;
  for (int b = 0; b < batch; b++) {
    int v = std::min(std::max(valid[b], 1), mel_frames);
    CK(launch_depthwise(c, mel + (size_t)b * mel_frames * mels, m->sc0.w, m->sc0.b, m->sc2.w, m->sc2.b,
                        sub16 + per * b, v, mels, ch, 0, rows1, 1));
  }
  CK(lin_h(m, sub16, m->conv3, m->sub2, rows1 * f2 * batch, WH_RELU, 0));
  for (int b = 0; b < batch; b++) {
    int img = batch == 1 ? t2 : half_len(half_len(std::min(std::max(valid[b], 1), mel_frames)));
    CK(launch_depthwise(c, m->sub2 + per * b, nullptr, nullptr, m->sc5.w, m->sc5.b, h16 + (size_t)b * t * f * ch,
                        img, f2, ch, 0, t, 1));
  }
  // conv6, then its [t][f][ch] image flattened to [t][ch·f] rows: by the GEMM's epilogue (rows in
  // blocks of f, into qk) when every tile plan's width divides ch, else by a launch of its own (into h).
  const _Float16 *flat = h16;
  if (ch % 256 == 0 && f % 8 == 0 && !c->unfused) {
    const int rows = t * f * batch;
    const HeadsOut out{qk16, 0, ch, ch, rows, 0, true, f};
    CK(launch_gemm_h_heads(c, h16, m->conv6, qk16, rows, m->conv6->cols, WH_RELU, &out, 1));
    flat = qk16;
  } else {
    CK(lin_h(m, h16, m->conv6, qk16, t * f * batch, WH_RELU, 1));
    CK(launch_flatten(c, qk16, h16, t * batch, f, ch, 1));
  }
  // The projection's output (the residual stream) and the first block's norm_ff1 of it (f16, into yr):
  // one kernel after a k-split GEMM.
  if (m->layers > 0) {
    const Chan &n1 = m->blocks[0].norm_ff1;
    CK(launch_gemm_h_ln(c, flat, m->pre_out, m->x, t * batch, 1.0f, n1.w, n1.b, m->yr, 1, 1, nullptr, nullptr, nullptr, 0));
  } else {
    CK(lin_h(m, flat, m->pre_out, m->x, t * batch, WH_BIAS, 0));
  }
  CK(record_blocks(m, t, batch, batch > 1 ? m->valid_dev : nullptr, m->layers, true, m->layers > 0));
  return lin_h(m, (const _Float16 *)m->x, m->joint_enc, out, t * batch, WH_BIAS, 0);
}

// Runs `record` (a function queuing kernels only) for the call identified by `key`: eagerly the first
// time, recorded into a HIP graph the second time, replayed from then on.  Buffers the graph names
// must not move: the key carries the arena's and the scratch's generations (and the context's tuning
// generation: a recording made under other launch plans is not replayed).
template <typename F>
int run_recorded(wh_model *m, std::vector<intptr_t> key, F &&record) {
  wh_ctx *c = m->ctx;
  key.push_back(c->tune_epoch);
  key.push_back(m->epoch);
  key.push_back(c->scratch_epoch);
  if (!m->use_graph || c->prof) return record();
  for (auto &g : m->graphs)
    if (g.key == key) {
      hipError_t e = hipGraphLaunch(g.exec, c->stream);
      if (e != hipSuccess) return wh_fail(c, WH_EGPU, "graph launch: %s", hipGetErrorString(e));
      return WH_OK;
    }
  if (m->pending != key) {
    m->pending = key;
    return record();
  }
  hipGraph_t graph = nullptr;
  if (hipStreamBeginCapture(c->stream, hipStreamCaptureModeThreadLocal) != hipSuccess) {
    (void)hipGetLastError();
    return record();
  }
  const int rc = record();
  hipError_t e = hipStreamEndCapture(c->stream, &graph);
  hipGraphExec_t exec = nullptr;
  if (rc == WH_OK && e == hipSuccess && graph) e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
  if (rc != WH_OK || e != hipSuccess || !exec) {
    if (exec) (void)hipGraphExecDestroy(exec);
    if (graph) (void)hipGraphDestroy(graph);
  }
  if (rc != WH_OK) return rc;
  if (e != hipSuccess || !exec) {  // recording failed: stay eager for this model
    (void)hipGetLastError();
    m->use_graph = false;
    return record();
  }
  // Stale generations are never matched again: drop them, and keep at most 8 recordings (each
  // destroyed once its queued launches are done).
  bool drained = false;
  for (size_t i = 0; i < m->graphs.size();)
    if (m->graphs[i].key[m->graphs[i].key.size() - 3] != c->tune_epoch ||
        m->graphs[i].key[m->graphs[i].key.size() - 2] != m->epoch || m->graphs[i].key.back() != c->scratch_epoch ||
        m->graphs.size() >= 8) {
      destroy_graph(m, m->graphs[i].exec, m->graphs[i].graph, drained);
      m->graphs.erase(m->graphs.begin() + i);
    } else {
      i++;
    }
  m->graphs.push_back({key, exec, graph});
  e = hipGraphLaunch(exec, c->stream);
  if (e != hipSuccess) return wh_fail(c, WH_EGPU, "graph launch: %s", hipGetErrorString(e));
  return WH_OK;
}

// Parakeet Encoder::record (src/parakeet/encoder.rs:103-124) over `batch` windows of mel_frames
// [batch][mel_frames][mels]; window b's first valid[b] mel frames are real.  One window: kestrel
// masking as the reference (conv0/conv2 see the valid frames, conv5 the whole image).  Several
// windows: each is subsampled as if alone (conv5 sees its own valid image rows), and its keys and
// conv inputs past its own encoder frames are masked.
int parakeet_encode(wh_model *m, const float *mel, int batch, int mel_frames, const int *valid, float *out) {
  const int t = parakeet_frames(mel_frames), d = m->d;
  if (mel_frames < 3 || t < 1) return fail(m, "too few mel frames");
  CK(arena(m, t, batch));
  m->pos_cur = m->pos + (size_t)(m->cap - t) * d;
  m->pos16_cur = (const _Float16 *)m->pos16 + (size_t)(m->cap - t) * d;
  wh_ctx *c = m->ctx;
  if (batch > 1) {
    // The windows' valid encoder frames, read by the kernels (uploaded before the recorded part).
    const std::vector<int> enc_valid = parakeet_valid(batch, mel_frames, t, valid);
    hipError_t e = hipMemcpyAsync(m->valid_dev, enc_valid.data(), sizeof(int) * batch, hipMemcpyHostToDevice, c->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(c->stream);
    if (e != hipSuccess) return wh_fail(c, WH_EGPU, "valid lengths: %s", hipGetErrorString(e));
  }
  std::vector<intptr_t> key = {PARAKEET, (intptr_t)mel, (intptr_t)out, batch, mel_frames};
  for (int b = 0; b < batch; b++) key.push_back(valid[b]);
  return run_recorded(m, std::move(key), [&] { return parakeet_record(m, mel, batch, mel_frames, valid, out); });
}

// GigaAM Encoder::record (src/gigaam/encoder.rs:83-93).
int gigaam_encode(wh_model *m, const float *mel, int mel_frames, float *out) {
  const int t1 = half_len(mel_frames), t = half_len(t1), d = m->d;
  if (mel_frames < 5) return fail(m, "too few mel frames");
  CK(arena(m, t1, 1));
  wh_ctx *c = m->ctx;
  return run_recorded(m, {GIGAAM, (intptr_t)mel, (intptr_t)out, mel_frames}, [&] {
    CK(launch_im2col(c, mel, m->h, mel_frames, m->mels, 5, 2, 2, 1, 0, 0));
    CK(lin(m, m->h, m->conv0, m->qk, t1, WH_RELU));
    CK(launch_im2col(c, m->qk, m->h, t1, d, 5, 2, 2, 1, 0, 0));
    CK(lin(m, m->h, m->conv2, m->x, t, WH_RELU));
    CK(record_blocks(m, t, 1, nullptr, m->layers, true));
    return lin_h(m, (const _Float16 *)m->x, m->head, out, t, WH_BIAS, 0);
  });
}

// Whisper Encoder::record (src/whisper/encoder.rs:67-74; transformer.rs:122-138) into out [t][d].
int whisper_encode(wh_model *m, const float *mel, int mel_frames, float *out) {
  const int t = m->frames, d = m->d, hd = d / m->heads;
  if (mel_frames != 2 * t) return fail(m, "Whisper takes windows of " + std::to_string(2 * t) + " mel frames");
  CK(arena(m, t, 1));
  wh_ctx *c = m->ctx;
  return run_recorded(m, {WHISPER, (intptr_t)mel, (intptr_t)out, mel_frames}, [&] {
    CK(launch_im2col(c, mel, m->qk, 2 * t, m->mels, 3, 1, 1, 1, 0, 0));
    CK(lin(m, m->qk, m->wconv0, m->h, 2 * t, WH_GELU));
    CK(launch_im2col(c, m->h, m->qk, 2 * t, d, 3, 2, 1, 1, 0, 0));
    CK(launch_copy(c, m->x, m->enc_pos, (size_t)t * d * 4));
    CK(lin(m, m->qk, m->wconv1, m->x, t, WH_GELU_RESIDUAL));
    // Pre-LN blocks; the GEMMs' inputs as f16 (see record_block).  Each residual projection runs with
    // the norm that follows it (a k-split GEMM's finish, the residual add and the norm in one kernel):
    // the attention output's with norm_ffn, the FFN's with the next block's norm_attn or, last, the
    // encoder's final norm into `out`.
    void *y16 = m->y, *h16 = m->h;
    if (m->wblocks.empty()) return launch_layer_norm(c, m->x, m->enc_norm.w, m->enc_norm.b, out, t, d, nullptr, nullptr, 0);
    CK(launch_layer_norm(c, m->x, m->wblocks[0].norm_attn.w, m->wblocks[0].norm_attn.b, y16, t, d, nullptr, nullptr, 0, 1));
    for (size_t i = 0; i < m->wblocks.size(); i++) {
      const WBlock &b = m->wblocks[i];
      CK(launch_gemm_h(c, y16, b.qkv, m->qk, t, b.qkv->cols + b.qkv->dual, WH_BIAS, 0.0f, 1));
      CK(launch_attention(c, m->qk, nullptr, nullptr, y16, t, m->heads, hd, nullptr, t, 1, 1, 1));
      CK(launch_gemm_h_ln(c, y16, b.out, m->x, t, 1.0f, b.norm_ffn.w, b.norm_ffn.b, y16, 1));
      CK(launch_gemm_h(c, y16, b.fc1, h16, t, b.fc1->cols + b.fc1->dual, WH_GELU, 0.0f, 1));
      const bool last = i + 1 == m->wblocks.size();
      const Chan &nn = last ? m->enc_norm : m->wblocks[i + 1].norm_attn;
      CK(launch_gemm_h_ln(c, h16, b.fc2, m->x, t, 1.0f, nn.w, nn.b, last ? (void *)out : y16, last ? 0 : 1));
    }
    return WH_OK;
  });
}

// dot (src/cpu/mod.rs:20-43): 16 fused lanes summed pairwise, then the tail.
float dot16(const float *a, const float *b, int n) {
  float acc[16] = {0};
  int n16 = n / 16 * 16;
  for (int i = 0; i < n16; i += 16)
    for (int l = 0; l < 16; l++) acc[l] = std::fma(a[i + l], b[i + l], acc[l]);
  for (int w = 8; w >= 1; w >>= 1)
    for (int l = 0; l < w; l++) acc[l] += acc[l + w];
  float tail = 0.0f;
  for (int i = n16; i < n; i++) tail += a[i] * b[i];
  return acc[0] + tail;
}

void matvec(const HostMat &w, const float *x, float *out) {
  for (int r = 0; r < w.rows; r++) out[r] = dot16(&w.w[(size_t)r * w.k], x, w.k);
}

int argmax_first(const float *v, int n) {
  int best = 0;
  for (int i = 1; i < n; i++)
    if (v[i] > v[best]) best = i;
  return best;
}

// Decoder::predict (src/parakeet/decoder.rs:111-133).
void predict(const wh_model *m, int token, const std::vector<float> &state, std::vector<float> &next,
             std::vector<float> &pred) {
  const int n = m->hidden;
  std::vector<float> x(n, 0.0f), gx(4 * n), gh(4 * n);
  if (token >= 0) x.assign(m->embed_h.w.begin() + (size_t)token * m->embed_h.k,
                           m->embed_h.w.begin() + (size_t)(token + 1) * m->embed_h.k);
  for (int l = 0; l < m->lstm_layers; l++) {
    const float *h = &state[(size_t)2 * n * l], *cc = h + n;
    float *nh = &next[(size_t)2 * n * l], *nc = nh + n;
    matvec(m->wx[l], x.data(), gx.data());
    matvec(m->wh[l], h, gh.data());
    const float *bb = m->lstm_b[l].data();
    auto sig = [](float v) { return 1.0f / (1.0f + std::exp(-v)); };
    for (int k = 0; k < n; k++) {
      float ig = gx[k] + gh[k] + bb[k], fg = gx[n + k] + gh[n + k] + bb[n + k];
      float gg = gx[2 * n + k] + gh[2 * n + k] + bb[2 * n + k], og = gx[3 * n + k] + gh[3 * n + k] + bb[3 * n + k];
      nc[k] = sig(fg) * cc[k] + sig(ig) * std::tanh(gg);
      nh[k] = sig(og) * std::tanh(nc[k]);
    }
    x.assign(nh, nh + n);
  }
  pred.resize(m->joint);
  matvec(m->pred_w, x.data(), pred.data());
  for (int j = 0; j < m->joint; j++) pred[j] = pred[j] + m->pred_b[j];
}

// TDT greedy (src/parakeet/decoder.rs:91-103, loop :158-191).
int tdt_greedy(const wh_model *m, const float *enc, int frames, int width, uint32_t *out, int cap) {
  const int S = 2 * m->lstm_layers * m->hidden, nd = (int)m->durations.size(), outs = m->classes + nd;
  std::vector<float> state(S, 0.0f), next(S, 0.0f), pred, z(m->joint), logits(outs);
  predict(m, -1, state, next, pred);
  int count = 0, t = 0, symbols = 0, emitted = -1;
  long left = m->global ? (long)m->max_symbols * frames : -1;
  while (t < frames && left != 0) {
    if (emitted >= 0) {
      state = next;
      predict(m, emitted, state, next, pred);
    }
    const float *e = enc + (size_t)t * width;
    for (int j = 0; j < m->joint; j++) z[j] = std::max(e[j] + pred[j], 0.0f);
    matvec(m->out_w, z.data(), logits.data());
    for (int i = 0; i < outs; i++) logits[i] = logits[i] + m->out_b[i];
    int token = argmax_first(logits.data(), m->classes), di = argmax_first(logits.data() + m->classes, nd);
    emitted = -1;
    if (token != m->blank) {
      if (count < cap) {
        out[2 * count] = (uint32_t)token;
        out[2 * count + 1] = (uint32_t)t;
      }
      count++;
      emitted = token;
    }
    int dur = m->durations[di];
    if (m->global) {
      left--;
      t += token == m->blank ? std::max(dur, 1) : dur;
      continue;
    }
    t += dur;
    symbols++;
    if (dur != 0) symbols = 0;
    else if (symbols >= m->max_symbols || token == m->blank) {
      t++;
      symbols = 0;
    }
  }
  return count;
}

// ---- greedy decoding on the device

// The TDT loop's device buffers in tdt_buf: [h_old | h_new | c] ([layers][hidden] each), the joint's
// predictor projection, the next frame's encoder row and the next joint input ([joint] each), the
// joint's partial maxima [parts][4], and the two state records; each part on a 64-float boundary.
constexpr int TDT_PARTS = 1024;  // the most the joint's launch may have (16384 output rows)

struct TdtBufs {
  float *h_old, *h_new, *c, *pred, *erow, *z, *part;
  TdtState *st, *nx;
  size_t total;  // floats
};

TdtBufs tdt_bufs(const wh_model *m, float *base) {
  auto up = [](size_t n) { return (n + 63) / 64 * 64; };
  const size_t ln = (size_t)m->lstm_layers * m->hidden, sw = up((sizeof(TdtState) + 3) / 4);
  size_t at = 0;
  TdtBufs b;
  b.h_old = base + at, at += up(ln);
  b.h_new = base + at, at += up(ln);
  b.c = base + at, at += up(ln);
  b.pred = base + at, at += up(m->joint);
  b.erow = base + at, at += up(m->joint);
  b.z = base + at, at += up(m->joint);
  b.part = base + at, at += up((size_t)4 * TDT_PARTS);
  b.st = (TdtState *)(base + at), at += sw;
  b.nx = (TdtState *)(base + at), at += sw;
  b.total = at;
  return b;
}

TdtConfig tdt_config(const wh_model *m) {
  TdtConfig cfg{};
  cfg.classes = m->classes;
  cfg.ndur = (int)m->durations.size();
  cfg.blank = m->blank;
  cfg.max_symbols = m->max_symbols;
  cfg.global = m->global;
  for (int i = 0; i < cfg.ndur; i++) cfg.durations[i] = m->durations[i];
  return cfg;
}

TdtArgs tdt_args(const wh_model *m) {
  const TdtBufs b = tdt_bufs(m, m->tdt_buf);
  TdtArgs a{};
  a.out_w = m->tdt_out->w, a.out_b = m->tdt_out->bias, a.out_rb = m->tdt_out->row_bytes;
  a.pred_w = m->tdt_pred->w, a.pred_b = m->tdt_pred->bias, a.pred_rb = m->tdt_pred->row_bytes;
  for (int l = 0; l < m->lstm_layers; l++) a.lstm_w[l] = m->tdt_lstm[l]->w, a.lstm_b[l] = m->tdt_lstm[l]->bias;
  a.lstm_rb = m->tdt_lstm[0]->row_bytes;
  a.type = m->tdt_out->type;
  a.n = m->hidden, a.joint = m->joint, a.layers = m->lstm_layers;
  a.out_rows = m->tdt_out->rows;
  a.parts = tdt_parts(a.type, a.out_rows);
  a.embed = m->tdt_embed;
  a.st = b.st, a.nx = b.nx;
  a.h_old = b.h_old, a.h_new = b.h_new, a.c = b.c, a.pred = b.pred, a.part = b.part;
  a.erow = b.erow, a.z = b.z;
  a.cfg = tdt_config(m);
  return a;
}

// `count` decisions of the TDT loop (src/parakeet/decoder.rs:158-191), three launches each (and one
// per further LSTM layer).
int tdt_decisions(wh_model *m, int count) {
  const TdtArgs a = tdt_args(m);
  for (int i = 0; i < count; i++) {
    CK(launch_tdt(m->ctx, a, TDT_JOINT));
    CK(launch_tdt(m->ctx, a, TDT_STEP));
    CK(launch_tdt(m->ctx, a, TDT_PRED));
  }
  return WH_OK;
}

// Decoder::decode (src/parakeet/decoder.rs:91-103) over an encoder output in device memory.
int tdt_greedy_device(wh_model *m, const float *enc, int frames, int width, uint32_t *out, int cap) {
  wh_ctx *c = m->ctx;
  if (m->tdt_lstm.empty() || !m->tdt_pred || !m->tdt_out || !m->tdt_embed)
    return wh_fail(c, WH_EARG, "model has no device TDT decoder");
  if (width < m->joint) return wh_fail(c, WH_EARG, "encoder width %d is below the joint's %d", width, m->joint);
  if (m->lstm_layers > 4) return wh_fail(c, WH_EARG, "tdt: %d LSTM layers (the device decoder takes up to 4)", m->lstm_layers);
  for (const wh_linear *l : m->tdt_lstm)
    if (l->type != m->tdt_out->type || l->row_bytes != m->tdt_lstm[0]->row_bytes)
      return wh_fail(c, WH_EARG, "tdt: the decoder's weights differ in type");
  if (m->tdt_pred->type != m->tdt_out->type) return wh_fail(c, WH_EARG, "tdt: the decoder's weights differ in type");
  if (tdt_parts(m->tdt_out->type, m->tdt_out->rows) > TDT_PARTS || m->hidden > 1024 || m->joint > 1024)
    return wh_fail(c, WH_EARG, "tdt: the decoder is larger than the device decoder takes");
  if (frames == 0) return 0;
  if (!m->tdt_buf) CK(wh_alloc(c, tdt_bufs(m, nullptr).total, &m->tdt_buf));
  // At most max_symbols decisions per frame (and the global budget is as many), so no more tokens.
  const long most = (long)frames * m->max_symbols;
  if (most > INT_MAX / 2) return wh_fail(c, WH_EARG, "tdt: %d frames is too many", frames);
  const int need = (int)std::max(1L, std::min((long)cap, most));
  if (need > m->tdt_list_cap) {
    if (m->tdt_list) CK(wh_free(c, m->tdt_list));
    m->tdt_list = nullptr, m->tdt_list_cap = 0;
    float *p = nullptr;
    CK(wh_alloc(c, (size_t)2 * need, &p));
    m->tdt_list = (uint32_t *)p, m->tdt_list_cap = need;
  }
  const TdtArgs a = tdt_args(m);
  TdtState init{};
  init.left = m->global ? (int)most : -1;
  init.idle = 1;
  init.frames = frames;
  init.width = width;
  init.cap = need;
  init.enc = enc;
  init.out = m->tdt_list;
  CK(launch_tdt_init(c, a.st, a.nx, init));
  // The first predict(None): a zero input and state.
  CK(launch_zero(c, a.h_old, (size_t)(a.pred - a.h_old) * 4));
  CK(launch_tdt(c, a, TDT_INIT));
  CK(launch_tdt(c, a, TDT_PRED));
  TdtState s{};
  for (;;) {
    CK(run_recorded(m, {TDT_CHUNK}, [&] { return tdt_decisions(m, TDT_DECISIONS); }));
    CK(wh_read(c, &s, a.st, sizeof s));
    if (s.done) break;
    if (s.decisions > most) return wh_fail(c, WH_EGPU, "tdt: %d decisions without reaching the end", s.decisions);
  }
  const int k = std::min(s.count, cap);
  if (k > 0) CK(wh_read(c, out, m->tdt_list, (size_t)k * 8));
  return s.count;
}

// Greedy CTC (src/gigaam/decoder.rs:135-151) over logits in device memory.
int ctc_greedy_device(wh_model *m, const float *logits, int frames, int width, uint32_t *out, int cap) {
  wh_ctx *c = m->ctx;
  if (width < m->outputs || m->outputs <= 0) return WH_EARG;
  if (frames == 0) return 0;
  if (frames > m->ctc_cap) {
    if (m->ctc_buf) CK(wh_free(c, m->ctc_buf));
    m->ctc_buf = nullptr, m->ctc_cap = 0;
    float *p = nullptr;
    CK(wh_alloc(c, (size_t)3 * frames + 1, &p));
    m->ctc_buf = (int *)p, m->ctc_cap = frames;
  }
  int *ids = m->ctc_buf, *count = ids + frames;
  uint32_t *pairs = (uint32_t *)(count + 1);
  CK(launch_ctc(c, logits, frames, width, m->outputs, m->blank, ids, pairs, frames, count));
  int n = 0;
  CK(wh_read(c, &n, count, 4));
  const int k = std::min(n, cap);
  if (k > 0) CK(wh_read(c, out, pairs, (size_t)k * 8));
  return n;
}

// ---- the log-mel frontend on the device

// Fft::new's tables (src/fft.rs:47-70): the input permutation, the leaves' cos and sin [j][k] and per
// radix-2 stage the twiddle of each output i < n / 2, from cos and sin of 2πi/n in f64.
void fft_tables(int n, std::vector<int> &perm, std::vector<double> &lc, std::vector<double> &ls,
                std::vector<double> &tc, std::vector<double> &ts, int &leaf, int &stages) {
  leaf = n;
  while (leaf % 2 == 0) leaf /= 2;
  const int blocks = n / leaf;
  std::vector<int> starts{0};
  while ((int)starts.size() < blocks) {
    std::vector<int> next;
    for (int s : starts) next.push_back(2 * s);
    for (int s : starts) next.push_back(2 * s + 1);
    starts.swap(next);
  }
  perm.resize(n);
  for (int i = 0; i < n; i++) perm[i] = starts[i % blocks] + i / blocks * blocks;
  auto trig = [n](long i, double &c, double &s) {
    const double phase = 6.283185307179586 * (double)i / (double)n;
    c = std::cos(phase), s = std::sin(phase);
  };
  lc.resize((size_t)leaf * leaf), ls.resize((size_t)leaf * leaf);
  for (int i = 0; i < leaf * leaf; i++) trig((long)(i / leaf) * (i % leaf) * blocks % n, lc[i], ls[i]);
  stages = 0;
  tc.clear(), ts.clear();
  for (int size = 2 * leaf; size <= n; size *= 2, stages++)
    for (int i = 0; i < n / 2; i++) {
      double c, s;
      trig((long)(i / (n / size)) * (n / size), c, s);
      tc.push_back(c), ts.push_back(s);
    }
}

// Parakeet's symmetric Hann(400) centred in 512 and Slaney filterbank [128][257] (src/parakeet/
// frontend.rs:31-40, :113-141), in f64 and rounded to f32 as the reference builds them.
void parakeet_tables(std::vector<double> &window, std::vector<float> &filters) {
  window.assign(512, 0.0);
  for (int i = 0; i < 512; i++) {
    const int k = i - 56;
    if (k >= 0 && k < 400) window[i] = 0.5 - 0.5 * std::cos(2.0 * 3.141592653589793 * (double)k / 399.0);
  }
  const double fsp = 200.0 / 3.0, min_log_hz = 1000.0, min_log_mel = min_log_hz / fsp;
  const double log_step = std::log(6.4) / 27.0;
  const double mel_max = min_log_mel + std::log(8000.0 / min_log_hz) / log_step;
  double hz[130];
  for (int m = 0; m < 130; m++) {
    const double mel = mel_max * (double)m / 129.0;
    hz[m] = mel < min_log_mel ? mel * fsp : min_log_hz * std::exp(log_step * (mel - min_log_mel));
  }
  filters.assign((size_t)128 * 257, 0.0f);
  for (int m = 0; m < 128; m++) {
    const double enorm = 2.0 / (hz[m + 2] - hz[m]);
    for (int k = 0; k < 257; k++) {
      const double f = 16000.0 * (double)k / 512.0;
      const double lower = (f - hz[m]) / (hz[m + 1] - hz[m]), upper = (hz[m + 2] - f) / (hz[m + 2] - hz[m + 1]);
      double v = std::min(lower, upper);
      v = v > 0.0 ? v : 0.0;
      filters[(size_t)m * 257 + k] = (float)(v * enorm);
    }
  }
}

// Per filter, the range its sum covers: Parakeet the nonzero bins (src/parakeet/frontend.rs:41-47),
// GigaAM those widened to dot's 16-bin chunks (src/gigaam/frontend.rs:31-38), Whisper the 4-bin
// groups below the last bin (src/whisper/frontend.rs:34-39).
std::vector<int> mel_spans(const std::vector<float> &filters, int mels, int bins, int kind) {
  std::vector<int> span(2 * (size_t)mels);
  for (int m = 0; m < mels; m++) {
    const float *f = filters.data() + (size_t)m * bins;
    int first = -1, last = -1;
    for (int k = 0; k < bins; k++)
      if (f[k] != 0.0f) {
        if (first < 0) first = k;
        last = k;
      }
    int lo, hi;
    if (kind == 0) {
      lo = first < 0 ? 0 : first;
      hi = last < 0 ? lo : last + 1;
    } else if (kind == 1) {
      lo = (first < 0 ? 0 : first) / 16 * 16;
      hi = last < 0 ? 0 : last + 1;
      hi = hi > bins / 16 * 16 ? bins : (hi + 15) / 16 * 16;
      hi = std::max(hi, lo);
    } else {
      lo = (first < 0 ? 0 : first) / 4;
      hi = last < 0 ? 0 : last / 4 + 1;
      hi = std::min(std::max(hi, lo), (bins - 1) / 4);
    }
    span[2 * m] = lo, span[2 * m + 1] = hi;
  }
  return span;
}

int mel_frames(const wh_model *m, int samples) {
  switch (m->arch) {
    case PARAKEET: return samples / 160 + 1 >= 3 ? samples / 160 + 1 : 0;
    case GIGAAM: return samples >= 320 ? (samples - 320) / 160 + 1 : 0;
    default: return std::max(samples, 480000) / 160;
  }
}

// The device tables of the model's frontend, in one allocation.
int mel_plan(wh_model *m) {
  auto &d = m->mel;
  if (d.ready) return WH_OK;
  wh_ctx *c = m->ctx;
  const int kind = m->arch == PARAKEET ? 0 : m->arch == GIGAAM ? 1 : 2;
  const int n = kind == 0 ? 512 : kind == 1 ? 320 : 400, bins = n / 2 + 1;
  std::vector<double> window;
  std::vector<float> filters;
  int mels = m->mels;
  if (kind == 0) {
    if (mels != 128) return wh_fail(c, WH_EARG, "the Parakeet frontend makes 128 bins; the model takes %d", mels);
    parakeet_tables(window, filters);
  } else {
    if (m->fe_window.size() != (size_t)n || m->fe_filters.size() != (size_t)bins * mels)
      return wh_fail(c, WH_EARG, "the model file has no frontend.window / frontend.mel_filterbank");
    window.assign(m->fe_window.begin(), m->fe_window.end());
    filters = m->fe_filters;
  }
  std::vector<int> perm;
  std::vector<double> lc, ls, tc, ts;
  int leaf = 0, stages = 0;
  fft_tables(n, perm, lc, ls, tc, ts, leaf, stages);
  const std::vector<int> span = mel_spans(filters, mels, bins, kind);
  // Layout: perm | leaf cos | leaf sin | twiddle cos | twiddle sin | window | filters | spans | scratch.
  const size_t es = kind == 0 ? 8 : 4;
  std::vector<size_t> sizes = {4 * perm.size(), es * lc.size(), es * ls.size(), es * tc.size(), es * ts.size(),
                               es * window.size(), 4 * filters.size(), 4 * span.size(), 256};
  std::vector<size_t> at;
  size_t total = 0;
  for (size_t b : sizes) at.push_back(total), total += (b + 255) / 256 * 256;
  std::vector<uint8_t> host(total, 0);
  auto put_t = [&](size_t off, const std::vector<double> &v) {
    for (size_t i = 0; i < v.size(); i++) {
      if (kind == 0) memcpy(host.data() + off + 8 * i, &v[i], 8);
      else {
        const float f = (float)v[i];
        memcpy(host.data() + off + 4 * i, &f, 4);
      }
    }
  };
  memcpy(host.data() + at[0], perm.data(), sizes[0]);
  put_t(at[1], lc), put_t(at[2], ls), put_t(at[3], tc), put_t(at[4], ts);
  if (kind == 0) put_t(at[5], window);
  else memcpy(host.data() + at[5], m->fe_window.data(), 4 * m->fe_window.size());  // the GGUF's f32 window
  memcpy(host.data() + at[6], filters.data(), sizes[6]);
  memcpy(host.data() + at[7], span.data(), sizes[7]);
  float *buf = nullptr;
  CK(wh_alloc(c, (total + 3) / 4, &buf));
  d.buf = (uint8_t *)buf;
  CK(wh_write(c, d.buf, host.data(), total));
  MelArgs &a = d.args;
  a.perm = (const int *)(d.buf + at[0]);
  a.leaf_cos = d.buf + at[1], a.leaf_sin = d.buf + at[2];
  a.tw_cos = d.buf + at[3], a.tw_sin = d.buf + at[4];
  a.window = d.buf + at[5];
  a.filters = (const float *)(d.buf + at[6]);
  a.span = (const int *)(d.buf + at[7]);
  a.hop = 160, a.mels = mels, a.leaf = leaf, a.stages = stages;
  a.silent = (float)std::log10(1e-10);
  d.scratch = (float *)(d.buf + at[8]);
  d.kind = kind, d.n = n, d.mels = mels, d.leaf = leaf, d.stages = stages;
  d.ready = true;
  return WH_OK;
}

// Decoder::record_step (src/transformer.rs:254-290) for the token and position held at m->ids[0..1]:
// kernels only, so that a recording replays it for every position.
int whisper_step_kernels(wh_model *m, float *logits) {
  const int d = m->d, heads = m->dec_heads, hd = d / heads;
  wh_ctx *c = m->ctx;
  const int *dpos = (const int *)(m->ids + 1);
  CK(launch_embed(c, m->token_embd, m->dec_pos, m->dx, m->ids, 0, 0, dpos, d));
  // Each LayerNorm runs inside the GEMV that consumes it (its only reader).
  for (int i = 0; i < m->dec_layers; i++) {
    const DLayer &l = m->dl[i];
    // q, k, v, with k and v also written into the self-attention cache's column (Decoder::pack).
    const GemvPack kv{m->own[i], d, d, m->context, 0, dpos};
    CK(launch_gemv(c, m->dx, l.qkv, m->dqkv, WH_BIAS, 0.0f, 0, l.norm_self.w, l.norm_self.b, m->dy, &kv));
    CK(launch_attend(c, m->dqkv, m->own[i], m->dpart, m->datt, 1, m->context, heads, hd, dpos));
    CK(launch_gemv(c, m->datt, l.self_out, m->dx, WH_RESIDUAL, 1.0f, 0));
    CK(launch_gemv(c, m->dx, l.cross_q, m->dqkv, WH_BIAS, 0.0f, 0, l.norm_cross.w, l.norm_cross.b, m->dy));
    CK(launch_attend(c, m->dqkv, m->cross[i], m->dpart, m->datt, m->cross_frames, m->cross_frames, heads, hd));
    CK(launch_gemv(c, m->datt, l.cross_out, m->dx, WH_RESIDUAL, 1.0f, 0));
    CK(launch_gemv(c, m->dx, l.fc1, m->dh, WH_GELU, 0.0f, 0, l.norm_ffn.w, l.norm_ffn.b, m->dy));
    CK(launch_gemv(c, m->dh, l.fc2, m->dx, WH_RESIDUAL, 1.0f, 0));
  }
  return launch_gemv(c, m->dx, m->token_embd, logits, WH_BIAS, 0.0f, 0, m->dec_norm.w, m->dec_norm.b, m->dy);
}

// The window search's loop (src/whisper/search.rs:35-71) on the device, from the logits of the
// prompt's last step in m->dlogits: a pick, then recorded runs of WHISPER_PICKS (step, pick) pairs
// until the state says done.  A pair after the end repeats the last step on the same token and
// position (same cache column, same values) and its pick returns at once.  Returns the number of
// ids picked, the first `cap` of them in `out`, and the mean log-probability when `logprobs`.
int whisper_search_device(wh_model *m, int np, int limit, bool logprobs, uint32_t *out, int cap, float *avg) {
  wh_ctx *c = m->ctx;
  const int vocab = m->vocab;
  // [state | generated ids | a partial per 1024 ids (64) | suppression mask, padded to whole quads]
  constexpr size_t state = 16, parts = 64 * sizeof(WhisperPart) / 4;
  static_assert(sizeof(WhisperState) <= state * 4 && sizeof(WhisperPart) % 8 == 0, "search buffer slots");
  const size_t mask = ((size_t)vocab + 3) / 4, at_mask = state + WHISPER_MAX_NEW + parts;
  if (!m->wsearch) {
    float *p = dev_alloc(m, at_mask + mask);
    if (!p) return WH_EOOM;
    // Bit 0: suppressed (src/whisper/search.rs:47-49); bit 1: suppressed at the window's first pick (:50-54).
    std::vector<uint8_t> bits((size_t)mask * 4, 0);
    for (int id : m->suppress) bits[id] |= 1;
    for (int id : m->begin_suppress) bits[id] |= 2;
    CK(wh_write(c, p + at_mask, bits.data(), bits.size()));
    m->wsearch = p;
  }
  WhisperPickArgs a{};
  a.logits = m->dlogits;
  a.vocab = vocab;
  a.eot = m->eot;
  a.no_ts = m->no_timestamps;
  a.begin = m->no_timestamps + 1;
  a.max_initial = 50;  // src/whisper/search.rs:13
  a.mask = (const uint8_t *)(m->wsearch + at_mask);
  a.st = (WhisperState *)m->wsearch;
  a.gen = (uint32_t *)(m->wsearch + state);
  a.part = (WhisperPart *)(m->wsearch + state + WHISPER_MAX_NEW);
  a.ids = m->ids;
  WhisperState init{};
  init.pos = np;
  init.np = np;
  init.limit = limit;
  init.max_new = WHISPER_MAX_NEW;
  init.logprobs = logprobs;
  init.last_ts = -1;
  CK(launch_whisper_init(c, a.st, init));
  CK(launch_whisper_pick(c, a));
  WhisperState s{};
  CK(wh_read(c, &s, a.st, sizeof s));
  for (int runs = 0; !s.done; runs++) {
    if (runs > WHISPER_MAX_NEW / WHISPER_PICKS + 1) return wh_fail(c, WH_EGPU, "whisper search: no end after %d picks", s.picks);
    CK(run_recorded(m, {WHISPER_LOOP, (intptr_t)m->dlogits, m->cross_frames}, [&] {
      for (int i = 0; i < WHISPER_PICKS; i++) {
        CK(whisper_step_kernels(m, m->dlogits));
        CK(launch_whisper_pick(c, a));
      }
      return WH_OK;
    }));
    CK(wh_read(c, &s, a.st, sizeof s));
  }
  if (s.n < 0 || s.n > WHISPER_MAX_NEW || s.picks <= 0) return wh_fail(c, WH_EGPU, "whisper search: bad state");
  const int k = std::min(s.n, cap);
  if (k > 0) CK(wh_read(c, out, a.gen, (size_t)k * 4));
  if (avg) *avg = logprobs ? (float)(s.sum / s.picks) : 0.0f;
  return s.n;
}

}  // namespace

extern "C" {

int wh_model_load(wh_ctx *ctx, const char *path, wh_model **out) {
  if (!ctx || !path || !out) return wh_fail(ctx, WH_EARG, "wh_model_load: bad arguments");
  *out = nullptr;
  auto m = std::make_unique<wh_model>();
  m->ctx = ctx;
  m->g = std::make_unique<Gguf>();
  std::string err;
  if (!m->g->open(path, err)) return wh_fail(ctx, WH_EARG, "%s", err.c_str());
  const Gguf &g = *m->g;
  Loader L(ctx, g);
  std::string arch = g.string("general.architecture");
  bool ok;
  if (arch == "gigaam") m->arch = GIGAAM, ok = load_gigaam(g, L, m.get(), err);
  else if (arch == "parakeet") m->arch = PARAKEET, ok = load_parakeet(g, L, m.get(), err);
  else if (arch == "whisper") m->arch = WHISPER, ok = load_whisper(g, L, m.get(), err);
  else ok = false, err = "unsupported general.architecture \"" + arch + "\"";
  m->owned = L.owned;
  m->linears = L.linears;
  // Every staged upload done (and its errors seen) before the model is handed out.
  if (ok && L.err.empty() && (stage_fence(ctx) || stage_wait(ctx))) L.fail(ctx->error);
  if (!ok || !L.err.empty()) {
    std::string msg = err.empty() ? L.err : err;
    wh_model_free(m.release());
    return wh_fail(ctx, msg.find("memory") != std::string::npos ? WH_EOOM : WH_EARG, "%s", msg.c_str());
  }
  *out = m.release();
  return WH_OK;
}

void wh_model_free(wh_model *m) {
  if (!m) return;
  (void)hipStreamSynchronize(m->ctx->stream);
  drop_graphs(m);
  for (float *p : m->owned)
    if (p) wh_free(m->ctx, p);
  if (m->valid_dev) wh_free(m->ctx, m->valid_dev);
  for (wh_linear *l : m->linears) wh_linear_free(m->ctx, l);
  for (uint32_t *p : m->own) wh_free(m->ctx, p);
  for (uint32_t *p : m->cross) wh_free(m->ctx, p);
  if (m->ids) wh_free(m->ctx, m->ids);
  for (void *p : {(void *)m->tdt_buf, (void *)m->tdt_list, (void *)m->ctc_buf, (void *)m->mel.buf})
    if (p) wh_free(m->ctx, p);
  delete m;
}

int wh_model_info(const wh_model *m, int *arch, int *d, int *layers, int *mels, int *width) {
  if (!m) return WH_EARG;
  if (arch) *arch = (int)m->arch;
  if (d) *d = m->d;
  if (layers) *layers = m->layers;
  if (mels) *mels = m->mels;
  if (width) {
    switch (m->arch) {
      case GIGAAM: *width = wh_linear_width(m->head); break;
      case PARAKEET: *width = wh_linear_width(m->joint_enc); break;
      default: *width = m->d;
    }
  }
  return WH_OK;
}

int wh_model_frames(const wh_model *m, int mel_frames, int *frames, int *width) {
  if (!m || mel_frames <= 0) return WH_EARG;
  int f = 0;
  switch (m->arch) {
    case GIGAAM: f = half_len(half_len(mel_frames)); break;
    case PARAKEET: f = mel_frames >= 3 ? parakeet_frames(mel_frames) : 0; break;
    default: f = m->frames;
  }
  if (frames) *frames = f;
  return wh_model_info(m, nullptr, nullptr, nullptr, nullptr, width);
}

int wh_model_encode(wh_model *m, const float *mel, int mel_frames, int valid, float *out) {
  if (!m || !mel || !out || mel_frames <= 0) return WH_EARG;
  (void)hipSetDevice(m->ctx->device);
  switch (m->arch) {
    case GIGAAM: return gigaam_encode(m, mel, mel_frames, out);
    case PARAKEET: {
      int v = valid <= 0 || valid > mel_frames ? mel_frames : valid;
      return parakeet_encode(m, mel, 1, mel_frames, &v, out);
    }
    default: return whisper_encode(m, mel, mel_frames, out);
  }
}

int wh_model_encode_batch(wh_model *m, const float *mel, int batch, int mel_frames, const int *valid, float *out) {
  if (!m || !mel || !out || !valid || batch <= 0 || mel_frames <= 0) return WH_EARG;
  if (m->arch != PARAKEET) return wh_fail(m->ctx, WH_EARG, "batched windows are built for the Parakeet encoder");
  (void)hipSetDevice(m->ctx->device);
  return parakeet_encode(m, mel, batch, mel_frames, valid, out);
}

int wh_model_graphs(wh_model *m, int on) {
  if (!m) return WH_EARG;
  (void)hipStreamSynchronize(m->ctx->stream);
  drop_graphs(m);
  m->use_graph = on != 0;
  return WH_OK;
}

int wh_model_blocks(wh_model *m, float *x, int t, int layers) {
  if (!m || !x || t <= 0 || layers < 0 || layers > m->layers || m->arch == WHISPER) return WH_EARG;
  CK(arena(m, t, 1));
  if (m->arch == PARAKEET) {
    m->pos_cur = m->pos + (size_t)(m->cap - t) * m->d;
    m->pos16_cur = (const _Float16 *)m->pos16 + (size_t)(m->cap - t) * m->d;
  }
  CK(wh_copy(m->ctx, m->x, x, (size_t)t * m->d * 4));
  CK(record_blocks(m, t, 1, nullptr, layers));
  return wh_copy(m->ctx, x, m->x, (size_t)t * m->d * 4);
}

int wh_model_greedy(wh_model *m, const float *enc, int frames, int width, uint32_t *out, int cap) {
  if (!m || !enc || frames < 0 || width <= 0 || !out || cap < 0) return WH_EARG;
  if (m->arch == GIGAAM) {
    if (width < m->outputs) return WH_EARG;
    // Greedy CTC (src/gigaam/decoder.rs:135-151) over the first `outputs` columns.
    int count = 0, prev = -1;
    for (int t = 0; t < frames; t++) {
      int best = argmax_first(enc + (size_t)t * width, m->outputs);
      if (prev != best && best != m->blank) {
        if (count < cap) {
          out[2 * count] = (uint32_t)best;
          out[2 * count + 1] = (uint32_t)t;
        }
        count++;
      }
      prev = best;
    }
    return count;
  }
  if (m->arch == PARAKEET) {
    if (m->embed_h.rows == 0 || width < m->joint) return wh_fail(m->ctx, WH_EARG, "model has no TDT decoder");
    return tdt_greedy(m, enc, frames, width, out, cap);
  }
  return wh_fail(m->ctx, WH_EARG, "Whisper decodes through wh_whisper_step");
}

int wh_model_mel(wh_model *m, const float *pcm_dev, int samples, float *mel_dev, int *frames) {
  if (!m || samples < 0 || !frames) return WH_EARG;
  const int f = mel_frames(m, samples);
  *frames = f;
  if (!mel_dev || f == 0) return WH_OK;
  if (!pcm_dev) return wh_fail(m->ctx, WH_EARG, "wh_model_mel: no audio");
  (void)hipSetDevice(m->ctx->device);
  CK(mel_plan(m));
  MelArgs a = m->mel.args;
  a.pcm = pcm_dev;
  a.samples = samples;
  a.len = std::max(samples, 480000);
  a.out = mel_dev;
  a.raw = m->ctx->mel_raw;
  return launch_mel(m->ctx, a, m->mel.kind, f, m->mel.scratch);
}

int wh_model_greedy_device(wh_model *m, const float *enc_dev, int frames, int width, uint32_t *out, int cap) {
  if (!m || !enc_dev || frames < 0 || width <= 0 || !out || cap < 0) return WH_EARG;
  (void)hipSetDevice(m->ctx->device);
  if (m->arch == GIGAAM) return ctc_greedy_device(m, enc_dev, frames, width, out, cap);
  if (m->arch == PARAKEET) return tdt_greedy_device(m, enc_dev, frames, width, out, cap);
  return wh_fail(m->ctx, WH_EARG, "Whisper decodes through wh_whisper_decode");
}

int wh_whisper_begin(wh_model *m, const float *enc, int frames) {
  if (!m || !enc || frames <= 0 || m->arch != WHISPER) return WH_EARG;
  const int d = m->d;
  wh_ctx *c = m->ctx;
  if (frames > m->frames)  // before anything is allocated
    return wh_fail(c, WH_EARG, "wh_whisper_begin: %d encoder frames, more than the model's window of %d", frames,
                   m->frames);
  if (m->own.empty()) {
    for (int i = 0; i < m->dec_layers; i++) {
      float *a = nullptr, *b = nullptr;
      CK(wh_alloc(c, (size_t)m->context * d, &a));
      CK(wh_alloc(c, (size_t)m->frames * d, &b));
      m->own.push_back((uint32_t *)a);
      m->cross.push_back((uint32_t *)b);
    }
    size_t vp = (size_t)(m->vocab % 32 == 0 ? m->vocab : (m->vocab + 63) / 64 * 64);
    m->dx = dev_alloc(m, d);
    m->dy = dev_alloc(m, d);
    m->dqkv = dev_alloc(m, 3 * (size_t)d);
    m->dh = dev_alloc(m, (size_t)m->dec_ff);
    m->datt = dev_alloc(m, d);
    m->dpart = dev_alloc(m, wh_attend_len(std::max(m->frames, m->context), m->dec_heads, d / m->dec_heads));
    m->dscratch = dev_alloc(m, (size_t)m->frames * 2 * d);
    float *ids = nullptr;  // the step's token and position
    CK(wh_alloc(c, 2, &ids));
    m->ids = (uint32_t *)ids;
    (void)vp;
    if (!m->dx || !m->dy || !m->dqkv || !m->dh || !m->datt || !m->dpart || !m->dscratch) return WH_EOOM;
  }
  // Decoder::record_cross (src/transformer.rs:243-248).
  for (int i = 0; i < m->dec_layers; i++) {
    CK(lin(m, enc, m->dl[i].cross_kv, m->dscratch, frames, WH_BIAS));
    CK(launch_pack(c, m->dscratch, 0, 2 * d, m->cross[i], frames, d, frames, 0));
  }
  m->cross_frames = frames;
  return WH_OK;
}

int wh_whisper_step(wh_model *m, int token, int pos, float *logits) {
  if (!m || m->arch != WHISPER || !logits || m->own.empty() || pos < 0 || pos >= m->context || token < 0 ||
      token >= m->vocab)
    return WH_EARG;
  // The token and position go to device memory; the step itself reads them there, so one recording
  // serves every position.
  CK(launch_step_args(m->ctx, m->ids, token, pos));
  return run_recorded(m, {WHISPER_STEP, (intptr_t)logits, m->cross_frames}, [&] { return whisper_step_kernels(m, logits); });
}


int wh_whisper_ids_of(const wh_model *m, wh_whisper_ids *out) {
  if (!m || !out || m->arch != WHISPER) return WH_EARG;
  out->eot = m->eot;
  out->no_timestamps = m->no_timestamps;
  out->begin = m->no_timestamps + 1;
  out->sot = m->sot;
  out->suppress = m->suppress.data();
  out->n_suppress = (int)m->suppress.size();
  out->begin_suppress = m->begin_suppress.data();
  out->n_begin_suppress = (int)m->begin_suppress.size();
  return WH_OK;
}

int wh_whisper_decode(wh_model *m, const float *enc, int frames, const uint32_t *prompt, int n_prompt, uint32_t *out,
                      int cap, float *no_speech, float *avg_logprob) {
  if (!m || m->arch != WHISPER || !enc || frames <= 0 || n_prompt < 0 || (n_prompt && !prompt) || cap < 0 ||
      (cap && !out))
    return WH_EARG;
  if (n_prompt && (int)prompt[0] != m->sot) return wh_fail(m->ctx, WH_EARG, "wh_whisper_decode: the prompt starts with SOT");
  for (int i = 0; i < n_prompt; i++)
    if ((int)prompt[i] >= m->vocab) return wh_fail(m->ctx, WH_EARG, "wh_whisper_decode: prompt id out of the vocabulary");
  constexpr float NO_SPEECH = 0.6f;  // src/whisper/mod.rs:31
  wh_ctx *c = m->ctx;
  (void)hipSetDevice(c->device);
  const int vocab = m->vocab, vp = vocab % 32 == 0 ? vocab : (vocab + 63) / 64 * 64;
  if (!m->dlogits && !(m->dlogits = dev_alloc(m, (size_t)vp))) return WH_EOOM;
  CK(wh_whisper_begin(m, enc, frames));
  const uint32_t sot_only = (uint32_t)m->sot;
  const uint32_t *pr = n_prompt ? prompt : &sot_only;
  const int np = n_prompt ? n_prompt : 1;
  const int limit = std::min(WHISPER_CONTEXT, m->context);
  if (np > limit) return wh_fail(c, WH_EARG, "wh_whisper_decode: prompt longer than the context");
  std::vector<float> logits((size_t)vocab);
  // Whisper::window: the decoder on SOT at position 0; its logits give the no-speech probability
  // (src/whisper/mod.rs:226-227), then the rest of the prompt (:235).
  CK(wh_whisper_step(m, (int)pr[0], 0, m->dlogits));
  CK(wh_read(c, logits.data(), m->dlogits, sizeof(float) * (size_t)vocab));
  const float ns = wh_whisper_probability(logits.data(), vocab, m->no_timestamps - 1);
  if (no_speech) *no_speech = ns;
  for (int i = 1; i < np; i++) CK(wh_whisper_step(m, (int)pr[i], i, m->dlogits));
  const bool logprobs = ns > NO_SPEECH || c->whisper_logprobs;
  if (!c->whisper_host) return whisper_search_device(m, np, limit, logprobs, out, cap, avg_logprob);
  // The same loop with each pick on the host (wh_whisper_pick), one read of the logits per step.
  if (np > 1) CK(wh_read(c, logits.data(), m->dlogits, sizeof(float) * (size_t)vocab));
  wh_whisper_ids ids;
  CK(wh_whisper_ids_of(m, &ids));
  std::vector<uint32_t> gen;
  double sum = 0.0;
  int picks = 0;
  float lp = 0.0f;
  auto pick = [&]() {
    const int id = wh_whisper_pick(&ids, logits.data(), vocab, gen.data(), (int)gen.size(), logprobs ? &lp : nullptr);
    sum += logprobs ? lp : 0.0f;
    picks++;
    return id;
  };
  int next = pick();
  if (next < 0) return wh_fail(c, WH_EARG, "wh_whisper_decode: bad token ids");
  for (int pos = np; pos < np + WHISPER_MAX_NEW; pos++) {
    if (next == m->eot) break;
    gen.push_back((uint32_t)next);
    if (pos + 1 > limit) break;
    CK(wh_whisper_step(m, (int)next, pos, m->dlogits));
    CK(wh_read(c, logits.data(), m->dlogits, sizeof(float) * (size_t)vocab));
    next = pick();
  }
  if (avg_logprob) *avg_logprob = logprobs ? (float)(sum / picks) : 0.0f;
  for (size_t i = 0; i < gen.size() && (int)i < cap; i++) out[i] = gen[i];
  return (int)gen.size();
}

}  // extern "C"
