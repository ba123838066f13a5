// Device, memory and weight management behind the C ABI (include/wavo_hip.h), and the thin
// entry points of the Pass ops.  The reference's counterparts are in src/gpu/mod.rs: Gpu::new
// (:461-577), buffer/readback/upload/write (:675-750), upload_linear (:770-834), run/complete
// (:906-1002).  One HIP stream per context replaces wgpu's queue; errors that wgpu reports through
// callbacks (:508-512, :995-1000) surface here as HIP status codes at the next wh_sync/wh_read.
#include <unistd.h>

#include <algorithm>
#include <cstdarg>
#include <cstdlib>
#include <cstdio>
#include <cstring>
#include <thread>
#include <vector>

#include "internal.h"

static thread_local std::string g_open_error;

int wh_fail(wh_ctx *ctx, int code, const char *fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  if (ctx) ctx->error = buf;
  else g_open_error = buf;
  return code;
}

int wh_launched(wh_ctx *ctx, const char *what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return wh_fail(ctx, WH_EGPU, "%s: %s", what, hipGetErrorString(e));
  return WH_OK;
}

static int prof_event(wh_ctx *ctx) {
  if (ctx->next_event == ctx->events.size()) {
    hipEvent_t e;
    if (hipEventCreate(&e) != hipSuccess) return -1;
    ctx->events.push_back(e);
  }
  return (int)ctx->next_event++;
}

ProfScope::ProfScope(wh_ctx *c, const char *kernel, double flops, double bytes) : ctx(c) {
  if (!ctx || ctx->prof != 1) return;
  wh_prof_rec r;
  r.kernel = kernel;
  r.flops = flops;
  r.bytes = bytes;
  r.ev0 = prof_event(ctx);
  r.ev1 = prof_event(ctx);
  if (r.ev0 < 0 || r.ev1 < 0) return;
  rec = (int)ctx->recs.size();
  ctx->recs.push_back(r);
  ctx->prof_pending = rec;
}

ProfScope::~ProfScope() {
  if (rec >= 0 && ctx->prof_pending == rec) ctx->prof_pending = -1;  // no launch took the events
}

void wh_prof_take(wh_ctx *ctx, hipEvent_t *start, hipEvent_t *stop) {
  *start = *stop = nullptr;
  if (ctx->prof_pending < 0) return;
  wh_prof_rec &r = ctx->recs[ctx->prof_pending];
  *start = ctx->events[r.ev0];
  *stop = ctx->events[r.ev1];
  r.used = true;
  ctx->prof_pending = -1;
}

void *wh_scratch(wh_ctx *ctx, size_t bytes) {
  if (bytes <= ctx->scratch_bytes) return ctx->scratch;
  if (ctx->recording) {  // no allocation inside a capture: the op has to run once before recording
    wh_fail(ctx, WH_EARG, "recording: an op needs %zu bytes of scratch (run it once before recording)", bytes);
    return nullptr;
  }
  hipError_t e = hipStreamSynchronize(ctx->stream);
  if (e == hipSuccess && ctx->scratch) e = hipFree(ctx->scratch);
  ctx->scratch = nullptr;
  ctx->scratch_bytes = 0;
  if (e == hipSuccess) e = hipMalloc(&ctx->scratch, bytes);
  if (e != hipSuccess) {
    ctx->scratch = nullptr;
    (void)hipGetLastError();
    wh_fail(ctx, e == hipErrorOutOfMemory ? WH_EOOM : WH_EGPU, "scratch of %zu bytes: %s", bytes, hipGetErrorString(e));
    return nullptr;
  }
  ctx->scratch_bytes = bytes;
  ctx->scratch_epoch++;
  return ctx->scratch;
}

size_t wh_type_bytes(int type, size_t n) {
  switch (type) {
    case WH_F32: return n * 4;
    case WH_F16: return n * 2;
    case WH_Q8_0: return n / 32 * 34;
    case WH_Q4_0: return n / 32 * 18;
  }
  return 0;
}

extern "C" {

int wh_open(int device_index, wh_ctx **out) {
  if (!out) return wh_fail(nullptr, WH_EARG, "wh_open: out is NULL");
  *out = nullptr;
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess || n == 0)
    return wh_fail(nullptr, WH_EGPU, "no GPU: %s", e != hipSuccess ? hipGetErrorString(e) : "none");
  int dev = device_index < 0 ? 0 : device_index;
  if (dev >= n) return wh_fail(nullptr, WH_EGPU, "no GPU at index %d: %d listed", dev, n);
  hipDeviceProp_t p;
  if ((e = hipGetDeviceProperties(&p, dev)) != hipSuccess)
    return wh_fail(nullptr, WH_EGPU, "hipGetDeviceProperties: %s", hipGetErrorString(e));
  if (strncmp(p.gcnArchName, "gfx950", 6) != 0)
    return wh_fail(nullptr, WH_EGPU, "device %d is %s; this build runs on gfx950 (MI355X) only",
                   dev, p.gcnArchName);
  if ((e = hipSetDevice(dev)) != hipSuccess)
    return wh_fail(nullptr, WH_EGPU, "hipSetDevice: %s", hipGetErrorString(e));
  wh_ctx *ctx = new wh_ctx;
  ctx->device = dev;
  ctx->cus = p.multiProcessorCount;
  ctx->name = p.name;
  if ((e = hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking)) != hipSuccess) {
    delete ctx;
    return wh_fail(nullptr, WH_EGPU, "hipStreamCreate: %s", hipGetErrorString(e));
  }
  if ((e = hipMalloc((void **)&ctx->attend_count, sizeof(int) * ATTEND_HEADS)) != hipSuccess ||
      (e = hipMemset(ctx->attend_count, 0, sizeof(int) * ATTEND_HEADS)) != hipSuccess) {
    if (ctx->attend_count) (void)hipFree(ctx->attend_count);
    (void)hipStreamDestroy(ctx->stream);
    delete ctx;
    return wh_fail(nullptr, WH_EGPU, "attend counters: %s", hipGetErrorString(e));
  }
  // The workspace address of wh_gemm_noalloc on this device; a failed lookup only disables that
  // entry point (it reports the error), every other one works without it.
  (void)gemm_noalloc_init(ctx);
  *out = ctx;
  return WH_OK;
}

void wh_close(wh_ctx *ctx) {
  if (!ctx) return;
  (void)hipSetDevice(ctx->device);
  (void)hipStreamSynchronize(ctx->stream);
  if (ctx->upload) {
    (void)hipStreamSynchronize(ctx->upload);
    for (int i = 0; i < wh_ctx::STAGE_SLOTS; i++) {
      if (ctx->pinned[i]) (void)hipHostFree(ctx->pinned[i]);
      if (ctx->pinned_done[i]) (void)hipEventDestroy(ctx->pinned_done[i]);
    }
    if (ctx->upload_fence) (void)hipEventDestroy(ctx->upload_fence);
    (void)hipStreamDestroy(ctx->upload);
  }
  for (hipEvent_t e : ctx->events) (void)hipEventDestroy(e);
  if (ctx->scratch) (void)hipFree(ctx->scratch);
  if (ctx->attend_count) (void)hipFree(ctx->attend_count);
  (void)hipStreamDestroy(ctx->stream);
  delete ctx;
}

}  // extern "C"

// ------------------------------------------------------------------------------ staged uploads
// Weights reach the device through a ring of pinned host buffers and a second stream: the host fills
// one slot (memcpy, or pread from the model file: no page faults on its mapping) while the DMA
// engine drains the others, and several host threads fill a large piece together.  Small pieces
// share a slot (each copy is queued at once; the slot's event marks its last copy).

constexpr size_t STAGE_BYTES = (size_t)16 << 20;
constexpr size_t STAGE_SPLIT = (size_t)2 << 20;  // pieces at least this large are filled by threads
constexpr int STAGE_THREADS = 8;

static int stage_init(wh_ctx *ctx) {
  if (ctx->upload) return WH_OK;
  hipError_t e = hipStreamCreateWithFlags(&ctx->upload, hipStreamNonBlocking);
  if (e == hipSuccess) e = hipEventCreateWithFlags(&ctx->upload_fence, hipEventDisableTiming);
  for (int i = 0; i < wh_ctx::STAGE_SLOTS && e == hipSuccess; i++) {
    e = hipHostMalloc(&ctx->pinned[i], STAGE_BYTES, hipHostMallocDefault);
    if (e == hipSuccess) e = hipEventCreateWithFlags(&ctx->pinned_done[i], hipEventDisableTiming);
  }
  if (e != hipSuccess) {
    (void)hipGetLastError();
    return wh_fail(ctx, e == hipErrorOutOfMemory ? WH_EOOM : WH_EGPU, "upload staging: %s", hipGetErrorString(e));
  }
  return WH_OK;
}

// dst[0..n) = src[0..n), read from the file where src lies in its mapping.
static bool fill_part(uint8_t *dst, const uint8_t *src, size_t n, const StageFile *f) {
  if (f && src >= f->base && src + n <= f->base + f->size) {
    off_t at = (off_t)(src - f->base);
    while (n) {
      ssize_t r = pread(f->fd, dst, n, at);
      if (r <= 0) return false;
      dst += r, at += r, n -= (size_t)r;
    }
    return true;
  }
  memcpy(dst, src, n);
  return true;
}

static bool fill(uint8_t *dst, const uint8_t *src, size_t n, const StageFile *f) {
  if (n < STAGE_SPLIT) return fill_part(dst, src, n, f);
  const int parts = STAGE_THREADS;
  const size_t per = (n / parts + 4095) / 4096 * 4096;
  bool ok[STAGE_THREADS];
  std::vector<std::thread> th;
  for (int i = 0; i < parts; i++) {
    const size_t lo = std::min(n, i * per), hi = std::min(n, lo + per);
    ok[i] = true;
    if (hi > lo) th.emplace_back([&, i, lo, hi] { ok[i] = fill_part(dst + lo, src + lo, hi - lo, f); });
  }
  for (auto &t : th) t.join();
  for (int i = 0; i < parts; i++)
    if (!ok[i]) return false;
  return true;
}

int stage_upload(wh_ctx *ctx, void *dst, const void *src, size_t bytes, const StageFile *file) {
  if (!bytes) return WH_OK;
  if (int rc = stage_init(ctx)) return rc;
  const uint8_t *s = (const uint8_t *)src;
  uint8_t *d = (uint8_t *)dst;
  for (size_t off = 0; off < bytes;) {
    const size_t n = std::min(STAGE_BYTES, bytes - off);
    if (ctx->pinned_fill + n > STAGE_BYTES) {  // the next slot, once its last copy is done
      ctx->pinned_slot = (ctx->pinned_slot + 1) % wh_ctx::STAGE_SLOTS;
      ctx->pinned_fill = 0;
    }
    const int k = ctx->pinned_slot;
    if (ctx->pinned_fill == 0 && ctx->pinned_used[k]) {
      hipError_t e = hipEventSynchronize(ctx->pinned_done[k]);
      if (e != hipSuccess) return wh_fail(ctx, WH_EGPU, "upload: %s", hipGetErrorString(e));
    }
    uint8_t *p = (uint8_t *)ctx->pinned[k] + ctx->pinned_fill;
    if (!fill(p, s + off, n, file)) return wh_fail(ctx, WH_EARG, "upload: reading the model file failed");
    hipError_t e = hipMemcpyAsync(d + off, p, n, hipMemcpyHostToDevice, ctx->upload);
    if (e == hipSuccess) e = hipEventRecord(ctx->pinned_done[k], ctx->upload);
    if (e != hipSuccess) return wh_fail(ctx, WH_EGPU, "upload: %s", hipGetErrorString(e));
    ctx->pinned_used[k] = true;
    ctx->pinned_fill += (n + 255) / 256 * 256;
    off += n;
  }
  return WH_OK;
}

int stage_fence(wh_ctx *ctx) {
  if (!ctx->upload) return WH_OK;
  hipError_t e = hipEventRecord(ctx->upload_fence, ctx->upload);
  if (e == hipSuccess) e = hipStreamWaitEvent(ctx->stream, ctx->upload_fence, 0);
  if (e != hipSuccess) return wh_fail(ctx, WH_EGPU, "upload fence: %s", hipGetErrorString(e));
  return WH_OK;
}

int stage_wait(wh_ctx *ctx) {
  if (!ctx->upload) return WH_OK;
  hipError_t e = hipStreamSynchronize(ctx->upload);
  if (e != hipSuccess) return wh_fail(ctx, WH_EGPU, "upload: %s", hipGetErrorString(e));
  return WH_OK;
}

extern "C" {

const char *wh_last_error(const wh_ctx *ctx) {
  return ctx ? ctx->error.c_str() : g_open_error.c_str();
}

int wh_device_info(wh_ctx *ctx, char *name, size_t name_len, int *cus, int *wave) {
  if (!ctx) return WH_EARG;
  if (name && name_len) snprintf(name, name_len, "%s", ctx->name.c_str());
  if (cus) *cus = ctx->cus;
  if (wave) *wave = 64;
  return WH_OK;
}

int wh_alloc(wh_ctx *ctx, size_t n_f32, float **dptr) {
  if (!ctx || !dptr) return WH_EARG;
  (void)hipSetDevice(ctx->device);
  void *p = nullptr;
  hipError_t e = hipMalloc(&p, (n_f32 ? n_f32 : 1) * sizeof(float));
  if (e != hipSuccess) {
    (void)hipGetLastError();
    return wh_fail(ctx, e == hipErrorOutOfMemory ? WH_EOOM : WH_EGPU, "hipMalloc of %zu floats: %s",
                   n_f32, hipGetErrorString(e));
  }
  *dptr = (float *)p;
  return WH_OK;
}

int wh_free(wh_ctx *ctx, void *dptr) {
  if (!ctx) return WH_EARG;
  if (!dptr) return WH_OK;
  (void)hipSetDevice(ctx->device);
  if (ctx->upload) (void)hipStreamSynchronize(ctx->upload);  // no staged copy into it still queued
  hipError_t e = hipFree(dptr);
  if (e != hipSuccess) return wh_fail(ctx, WH_EGPU, "hipFree: %s", hipGetErrorString(e));
  return WH_OK;
}

int wh_host_alloc(wh_ctx *ctx, size_t bytes, void **host) {
  if (!ctx || !host) return WH_EARG;
  (void)hipSetDevice(ctx->device);
  void *p = nullptr;
  hipError_t e = hipHostMalloc(&p, bytes ? bytes : 1, hipHostMallocDefault);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    return wh_fail(ctx, e == hipErrorOutOfMemory ? WH_EOOM : WH_EGPU, "hipHostMalloc of %zu bytes: %s", bytes,
                   hipGetErrorString(e));
  }
  *host = p;
  return WH_OK;
}

int wh_host_free(wh_ctx *ctx, void *host) {
  if (!ctx) return WH_EARG;
  if (!host) return WH_OK;
  (void)hipSetDevice(ctx->device);
  (void)hipStreamSynchronize(ctx->stream);  // no queued copy from or into it
  hipError_t e = hipHostFree(host);
  if (e != hipSuccess) return wh_fail(ctx, WH_EGPU, "hipHostFree: %s", hipGetErrorString(e));
  return WH_OK;
}

int wh_write(wh_ctx *ctx, void *dst, const void *src, size_t bytes) {
  if (!ctx || (!dst && bytes) || (!src && bytes)) return WH_EARG;
  if (!bytes) return WH_OK;
  (void)hipSetDevice(ctx->device);
  hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
  if (e != hipSuccess) return wh_fail(ctx, WH_EGPU, "write of %zu bytes: %s", bytes, hipGetErrorString(e));
  return WH_OK;
}

int wh_copy(wh_ctx *ctx, void *dst, const void *src, size_t bytes) {
  if (!ctx || (!bytes)) return ctx ? WH_OK : WH_EARG;
  return launch_copy(ctx, dst, src, bytes);
}

int wh_zero(wh_ctx *ctx, void *dst, size_t bytes) {
  if (!ctx) return WH_EARG;
  return launch_zero(ctx, dst, bytes);
}

int wh_sync(wh_ctx *ctx) {
  if (!ctx) return WH_EARG;
  (void)hipSetDevice(ctx->device);
  hipError_t e = hipStreamSynchronize(ctx->stream);
  if (e != hipSuccess) return wh_fail(ctx, WH_EGPU, "device error: %s", hipGetErrorString(e));
  return WH_OK;
}

int wh_read(wh_ctx *ctx, void *host, const void *dptr, size_t bytes) {
  if (!ctx || (bytes && (!host || !dptr))) return WH_EARG;
  int rc = wh_sync(ctx);
  if (rc) return rc;
  if (!bytes) return WH_OK;
  hipError_t e = hipMemcpy(host, dptr, bytes, hipMemcpyDeviceToHost);
  if (e != hipSuccess) return wh_fail(ctx, WH_EGPU, "read of %zu bytes: %s", bytes, hipGetErrorString(e));
  return WH_OK;
}

void *wh_stream(wh_ctx *ctx) { return ctx ? (void *)ctx->stream : nullptr; }

int wh_tune(wh_ctx *ctx, const char *key, const char *value) {
  if (!ctx || !key) return WH_EARG;
  ctx->tune_epoch++;
  const char *v = value ? value : "";
  if (!strcmp(key, "gemm_plan")) {
    int o[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    if (*v && (sscanf(v, "%d,%d,%d,%d,%d,%d,%d,%d", &o[0], &o[1], &o[2], &o[3], &o[4], &o[5], &o[6], &o[7]) < 6 ||
               o[5] < 1 || o[5] > 4 || o[7] < 0 || o[7] > 2))
      return wh_fail(ctx, WH_EARG,
                     "wh_tune gemm_plan: \"bm,bn,wm,wn,stages,split[,pipeline[,kgroups]]\" (split 1..4, kgroups 1..2) or \"\"");
    memcpy(ctx->gemm_plan, o, sizeof o);
  } else if (!strcmp(key, "gemm_shape_plans")) {
    ctx->gemm_shape_plans.clear();
    for (const char *q = v; *q;) {
      std::array<int, 11> o{};
      if (sscanf(q, "%d,%d,%d:%d,%d,%d,%d,%d,%d,%d,%d", &o[0], &o[1], &o[2], &o[3], &o[4], &o[5], &o[6], &o[7], &o[8],
                 &o[9], &o[10]) < 9 ||
          o[8] < 1 || o[8] > 4 || o[10] < 0 || o[10] > 2)
        return wh_fail(ctx, WH_EARG,
                       "wh_tune gemm_shape_plans: \"m,cols,k:bm,bn,wm,wn,stages,split[,pipeline[,kgroups]];...\"");
      ctx->gemm_shape_plans.push_back(o);
      const char *n = strchr(q, ';');
      if (!n) break;
      q = n + 1;
    }
  } else if (!strcmp(key, "gemm_kernel_only")) {
    ctx->gemm_kernel_only = atoi(v) != 0;
  } else if (!strcmp(key, "position_cache")) {
    ctx->no_position_cache = atoi(v) == 0;
  } else if (!strcmp(key, "gemm_group")) {
    ctx->gemm_group = std::max(0, atoi(v));
  } else if (!strcmp(key, "attn_split")) {
    ctx->attn_split = std::max(0, std::min(atoi(v), 64));
  } else if (!strcmp(key, "mel_raw")) {
    ctx->mel_raw = atoi(v) != 0;
  } else if (!strcmp(key, "whisper_host")) {
    ctx->whisper_host = atoi(v) != 0;
  } else if (!strcmp(key, "whisper_logprobs")) {
    ctx->whisper_logprobs = atoi(v) != 0;
  } else if (!strcmp(key, "epilogue_fusion")) {
    ctx->unfused = atoi(v) == 0;
  } else if (!strcmp(key, "attend_merge")) {
    ctx->attend_merge = atoi(v) != 0;
  } else {
    return wh_fail(ctx, WH_EARG, "wh_tune: unknown key \"%s\"", key);
  }
  return WH_OK;
}

// ------------------------------------------------------------------------------ recorded passes

struct wh_pass {
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
  wh_ctx *ctx = nullptr;
  long scratch_epoch = 0;
};

int wh_record_begin(wh_ctx *ctx) {
  if (!ctx) return WH_EARG;
  if (ctx->recording) return wh_fail(ctx, WH_EARG, "wh_record_begin: already recording");
  if (ctx->prof) return wh_fail(ctx, WH_EARG, "wh_record_begin: profiling is on (its events are per launch)");
  (void)hipSetDevice(ctx->device);
  hipError_t e = hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeThreadLocal);
  if (e != hipSuccess) return wh_fail(ctx, WH_EGPU, "wh_record_begin: %s", hipGetErrorString(e));
  ctx->recording = 1;
  return WH_OK;
}

int wh_record_end(wh_ctx *ctx, wh_pass **out) {
  if (!ctx || !out) return WH_EARG;
  *out = nullptr;
  if (!ctx->recording) return wh_fail(ctx, WH_EARG, "wh_record_end: not recording");
  ctx->recording = 0;
  hipGraph_t graph = nullptr;
  hipError_t e = hipStreamEndCapture(ctx->stream, &graph);
  if (e != hipSuccess || !graph) {
    (void)hipGetLastError();
    if (graph) (void)hipGraphDestroy(graph);
    return wh_fail(ctx, WH_EGPU, "wh_record_end: capture failed (%s)", hipGetErrorString(e));
  }
  hipGraphExec_t exec = nullptr;
  e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    (void)hipGraphDestroy(graph);
    return wh_fail(ctx, WH_EGPU, "wh_record_end: %s", hipGetErrorString(e));
  }
  wh_pass *p = new wh_pass;
  p->graph = graph;
  p->exec = exec;
  p->ctx = ctx;
  p->scratch_epoch = ctx->scratch_epoch;
  *out = p;
  return WH_OK;
}

int wh_replay(wh_ctx *ctx, const wh_pass *p) {
  if (!ctx || !p || p->ctx != ctx) return wh_fail(ctx, WH_EARG, "wh_replay: a pass of another context");
  if (ctx->recording) return wh_fail(ctx, WH_EARG, "wh_replay: recording");
  if (p->scratch_epoch != ctx->scratch_epoch)
    return wh_fail(ctx, WH_EARG, "wh_replay: the context's scratch moved since the pass was recorded; record it again");
  (void)hipSetDevice(ctx->device);
  hipError_t e = hipGraphLaunch(p->exec, ctx->stream);
  if (e != hipSuccess) return wh_fail(ctx, WH_EGPU, "wh_replay: %s", hipGetErrorString(e));
  return WH_OK;
}

void wh_pass_free(wh_pass *p) {
  if (!p) return;
  if (p->ctx) (void)hipStreamSynchronize(p->ctx->stream);
  if (p->exec) (void)hipGraphExecDestroy(p->exec);
  if (p->graph) (void)hipGraphDestroy(p->graph);
  delete p;
}

int wh_profile(wh_ctx *ctx, int mode) {
  if (!ctx || mode < 0 || mode > 2) return WH_EARG;
  if (ctx->recording) return wh_fail(ctx, WH_EARG, "wh_profile: recording");
  int rc = wh_sync(ctx);
  if (rc) return rc;
  ctx->prof = mode;
  ctx->recs.clear();
  ctx->next_event = 0;
  ctx->open_region = -1;
  ctx->prof_pending = -1;
  return WH_OK;
}

int wh_region(wh_ctx *ctx, const char *name, double flops, double bytes) {
  if (!ctx || !ctx->prof) return ctx ? WH_OK : WH_EARG;
  if (name) {  // begin
    if (ctx->open_region >= 0) return wh_fail(ctx, WH_EARG, "wh_region: a region is open");
    wh_prof_rec r;
    r.kernel = name;
    r.ev0 = prof_event(ctx);
    r.ev1 = prof_event(ctx);
    if (r.ev0 < 0 || r.ev1 < 0) return wh_fail(ctx, WH_EGPU, "wh_region: event creation failed");
    if (hipEventRecord(ctx->events[r.ev0], ctx->stream) != hipSuccess) return wh_fail(ctx, WH_EGPU, "wh_region: event record failed");
    r.used = true;
    ctx->open_region = (int)ctx->recs.size();
    ctx->recs.push_back(r);
    return WH_OK;
  }
  if (ctx->open_region < 0) return wh_fail(ctx, WH_EARG, "wh_region: no open region");
  wh_prof_rec &r = ctx->recs[ctx->open_region];
  r.flops = flops;
  r.bytes = bytes;
  ctx->open_region = -1;
  if (hipEventRecord(ctx->events[r.ev1], ctx->stream) != hipSuccess) return wh_fail(ctx, WH_EGPU, "wh_region: event record failed");
  return WH_OK;
}

int wh_profile_read(wh_ctx *ctx, char *out, size_t len) {
  if (!ctx || !out || !len) return WH_EARG;
  int rc = wh_sync(ctx);
  if (rc) return rc;
  // Per kernel: launches, total milliseconds, algorithmic flops and bytes, in first-seen order.
  std::vector<std::string> order;
  std::vector<double> ms, fl, by;
  std::vector<long> n;
  for (const wh_prof_rec &r : ctx->recs) {
    if (!r.used) continue;
    float t = 0.0f;
    if (hipEventElapsedTime(&t, ctx->events[r.ev0], ctx->events[r.ev1]) != hipSuccess) t = 0.0f;
    size_t i = 0;
    while (i < order.size() && order[i] != r.kernel) i++;
    if (i == order.size()) {
      order.push_back(r.kernel);
      ms.push_back(0), fl.push_back(0), by.push_back(0), n.push_back(0);
    }
    ms[i] += t, fl[i] += r.flops, by[i] += r.bytes, n[i]++;
  }
  std::string s = "[";
  for (size_t i = 0; i < order.size(); i++) {
    char buf[512];
    snprintf(buf, sizeof buf, "%s{\"kernel\": \"%s\", \"launches\": %ld, \"ms\": %.6f, \"flops\": %.6g, \"bytes\": %.6g}",
             i ? ", " : "", order[i].c_str(), n[i], ms[i], fl[i], by[i]);
    s += buf;
  }
  s += "]";
  snprintf(out, len, "%s", s.c_str());
  return s.size() < len ? WH_OK : wh_fail(ctx, WH_EARG, "profile text needs %zu bytes", s.size() + 1);
}

// ------------------------------------------------------------------------------------ weights

int wh_linear_new(wh_ctx *ctx, const wh_tensor *ws, int count, const float *bias, int n_bias,
                  int pad_k, wh_linear **out) {
  return linear_new(ctx, ws, count, bias, n_bias, pad_k, out, nullptr);
}

}  // extern "C"

int linear_new(wh_ctx *ctx, const wh_tensor *ws, int count, const float *bias, int n_bias, int pad_k,
               wh_linear **out, const StageFile *file) {
  if (!ctx || !ws || count <= 0 || !out || n_bias < 0) return wh_fail(ctx, WH_EARG, "wh_linear_new: bad arguments");
  if (ctx->recording) return wh_fail(ctx, WH_EARG, "wh_linear_new: weights cannot be created while recording");
  *out = nullptr;
  int type = ws[0].type, k = ws[0].k, rows = 0;
  for (int i = 0; i < count; i++) {
    if (ws[i].type != type || ws[i].k != k || ws[i].rows <= 0 || !ws[i].data)
      return wh_fail(ctx, WH_EARG, "stacked weights differ in type or shape");
    rows += ws[i].rows;
  }
  if (type != WH_F32 && type != WH_F16 && type != WH_Q8_0 && type != WH_Q4_0)
    return wh_fail(ctx, WH_EARG, "unsupported weight type %d", type);
  if (k <= 0) return wh_fail(ctx, WH_EARG, "linear layer with k = %d", k);
  if ((type == WH_Q8_0 || type == WH_Q4_0) && k % 32)
    return wh_fail(ctx, WH_EARG, "linear layer %d→%d: quantized rows need k %% 32 == 0", k, rows);
  if (!pad_k && k % 32) return wh_fail(ctx, WH_EARG, "linear layer %d→%d: needs k %% 32 == 0", k, rows);
  int dual = n_bias > rows ? n_bias - rows : 0;
  if ((n_bias && n_bias < rows) || dual > rows)
    return wh_fail(ctx, WH_EARG, "linear layer %d→%d: bias has %d values", k, rows, n_bias);
  int n = (rows + 63) / 64 * 64;
  int cols = rows % 32 == 0 ? rows : n;
  int kp = (k + 31) / 32 * 32;
  std::vector<uint8_t> host;
  int dtype = type;
  if (kp != k) {
    // Padded k (Gpu::conv, src/gpu/mod.rs:787-796): the rows in F32 with zero columns.
    dtype = WH_F32;
    host.assign((size_t)rows * kp * 4, 0);
    std::vector<float> row(k);
    int at = 0;
    for (int i = 0; i < count; i++) {
      const uint8_t *src = (const uint8_t *)ws[i].data;
      for (int r = 0; r < ws[i].rows; r++, at++) {
        if (type == WH_F32) {
          memcpy(host.data() + (size_t)at * kp * 4, src + (size_t)r * k * 4, (size_t)k * 4);
        } else {  // F16 rows
          const uint16_t *h = (const uint16_t *)(src + (size_t)r * k * 2);
          float *o = (float *)(host.data() + (size_t)at * kp * 4);
          for (int c = 0; c < k; c++) {
            uint32_t x = h[c], s = (x & 0x8000u) << 16, e = (x >> 10) & 31, mnt = x & 0x3ff, u;
            if (e == 0) {
              float v = (float)mnt * 5.9604644775390625e-8f;
              o[c] = s ? -v : v;
              continue;
            }
            u = e == 31 ? (s | 0x7f800000u | (mnt << 13)) : (s | ((e + 112) << 23) | (mnt << 13));
            memcpy(&o[c], &u, 4);
          }
        }
      }
    }
  }
  wh_linear *l = new wh_linear;
  l->rows = rows;
  l->cols = cols;
  l->dual = dual;
  l->k = kp;
  l->type = dtype;
  l->row_bytes = wh_type_bytes(dtype, (size_t)kp);
  (void)hipSetDevice(ctx->device);
  size_t wbytes = l->row_bytes * rows;
  // 256 bytes of slack: the GEMM's loaders read whole dwords of the last row.
  hipError_t e = hipMalloc(&l->w, wbytes + 256);
  if (e == hipSuccess) e = hipMalloc(&l->bias, sizeof(float) * (size_t)(n > cols + dual ? n : cols + dual));
  if (e != hipSuccess) {
    (void)hipGetLastError();
    int rc = wh_fail(ctx, e == hipErrorOutOfMemory ? WH_EOOM : WH_EGPU, "weights: %s", hipGetErrorString(e));
    wh_linear_free(ctx, l);
    return rc;
  }
  // The weights and the bias through the staged uploads; the 256 bytes of slack are zeros.
  std::vector<float> pb((size_t)(n > cols + dual ? n : cols + dual), 0.0f);
  if (n_bias) {
    memcpy(pb.data(), bias, sizeof(float) * rows);
    if (dual) memcpy(pb.data() + cols, bias + rows, sizeof(float) * dual);
  }
  static const uint8_t zeros[256] = {};
  int rc = WH_OK;
  if (!host.empty()) {
    rc = stage_upload(ctx, l->w, host.data(), wbytes);
  } else {
    size_t at = 0;
    for (int i = 0; i < count && rc == WH_OK; i++) {
      size_t b = l->row_bytes * ws[i].rows;
      rc = stage_upload(ctx, l->w + at, ws[i].data, b, file);
      at += b;
    }
  }
  if (rc == WH_OK) rc = stage_upload(ctx, l->w + wbytes, zeros, sizeof zeros);
  if (rc == WH_OK) rc = stage_upload(ctx, l->bias, pb.data(), sizeof(float) * pb.size());
  if (rc == WH_OK) rc = stage_fence(ctx);
  if (rc != WH_OK) {
    (void)stage_wait(ctx);
    wh_linear_free(ctx, l);
    return rc;
  }
  *out = l;
  return WH_OK;
}

extern "C" {

int wh_linear_width(const wh_linear *l) { return l ? l->cols + l->dual : 0; }
int wh_linear_k(const wh_linear *l) { return l ? l->k : 0; }
int wh_linear_type(const wh_linear *l) { return l ? l->type : -1; }

void wh_linear_free(wh_ctx *ctx, wh_linear *l) {
  if (!l) return;
  if (ctx) (void)hipSetDevice(ctx->device);
  if (ctx && ctx->upload) (void)hipStreamSynchronize(ctx->upload);  // no copy into it still queued
  if (l->w) (void)hipFree(l->w);
  if (l->bias) (void)hipFree(l->bias);
  delete l;
}

// ------------------------------------------------------------------------------------ Pass ops

int wh_gemm(wh_ctx *ctx, const float *a, const wh_linear *l, float *c, int m, int epi, float alpha) {
  if (!ctx || !l) return WH_EARG;
  return launch_gemm(ctx, a, l, c, m, l->cols + l->dual, epi, alpha);
}

int wh_gemm_h(wh_ctx *ctx, const void *a16, const wh_linear *l, void *c, int m, int epi, float alpha, int out16) {
  if (!ctx || !l) return WH_EARG;
  // (the library's internal epilogues, past WH_TANH, are not part of the interface)
  if (epi < WH_BIAS || epi > WH_TANH) return wh_fail(ctx, WH_EARG, "gemm: epilogue %d", epi);
  return launch_gemm_h(ctx, a16, l, c, m, l->cols + l->dual, epi, alpha, out16);
}

int wh_gemv(wh_ctx *ctx, const float *a, const wh_linear *l, float *c, int epi, float alpha,
            int offset) {
  if (!ctx || !l) return WH_EARG;
  return launch_gemv(ctx, a, l, c, epi, alpha, offset);
}

int wh_embed(wh_ctx *ctx, const wh_linear *l, const float *pos, float *c, const uint32_t *ids, int i,
             int offset) {
  if (!ctx || !l) return WH_EARG;
  return launch_embed(ctx, l, pos, c, ids, i, offset);
}

int wh_layer_norm(wh_ctx *ctx, const float *x, const float *g, const float *b, float *y, int rows,
                  int cols, const float *table, float *yr, int head_dim) {
  if (!ctx) return WH_EARG;
  return launch_layer_norm(ctx, x, g, b, y, rows, cols, table, yr, head_dim);
}

size_t wh_attend_len(int n, int heads, int hd) {
  return (size_t)((n + 255) / 256) * heads * (hd + 2);
}

int wh_attend(wh_ctx *ctx, const float *q, const uint32_t *kv, float *part, float *o, int n, int cols,
              int heads, int hd) {
  if (!ctx) return WH_EARG;
  return launch_attend(ctx, q, kv, part, o, n, cols, heads, hd);
}

int wh_pack(wh_ctx *ctx, const float *x, int src, int stride, uint32_t *y, int rows, int d, int cols,
            int col) {
  if (!ctx) return WH_EARG;
  return launch_pack(ctx, x, src, stride, y, rows, d, cols, col);
}

int wh_im2col(wh_ctx *ctx, const float *x, float *col, int t, int ch, int kernel, int stride, int pad) {
  if (!ctx) return WH_EARG;
  return launch_im2col(ctx, x, col, t, ch, kernel, stride, pad, 1, 0, 0);
}

int wh_conv_glu(wh_ctx *ctx, const float *h, const float *dw_w, const float *dw_b, int kernel,
                const float *g, const float *b, int layer_norm, float *y, int t, int ch, int valid) {
  if (!ctx) return WH_EARG;
  return launch_conv_glu(ctx, h, dw_w, dw_b, kernel, g, b, layer_norm, y, t, ch, nullptr, valid, 1);
}

int wh_attention(wh_ctx *ctx, const float *qk, const float *v, const float *pos, float *o, int t,
                 int heads, int hd, int valid) {
  if (!ctx) return WH_EARG;
  return launch_attention(ctx, qk, v, pos, o, t, heads, hd, nullptr, valid, 1);
}

int wh_depthwise(wh_ctx *ctx, const float *x, const float *first_w, const float *first_b,
                 const float *w, const float *b, float *y, int t, int f, int ch, int t0, int rows) {
  if (!ctx) return WH_EARG;
  return launch_depthwise(ctx, x, first_w, first_b, w, b, y, t, f, ch, t0, rows);
}

int wh_flatten(wh_ctx *ctx, const float *x, float *y, int t, int f, int ch) {
  if (!ctx) return WH_EARG;
  return launch_flatten(ctx, x, y, t, f, ch);
}

int wh_argmax(wh_ctx *ctx, const float *x, uint32_t *out, int n) {
  if (!ctx) return WH_EARG;
  return launch_argmax(ctx, x, out, n);
}

}  // extern "C"
