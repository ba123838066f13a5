// The quantized GEMM of Pass::gemm (src/gpu/mod.rs:1394-1426) on gfx950 matrix cores:
//   c[m][j] = epi(Σ_k h(a[m][k]) · h(W[j][k]) + bias[j]),  h = round to f16 (RNE), f32 accumulate,
// as gemm.wgsl:170-242 and the CPU backend (src/cpu/gemm.rs:126-177) define it.  W stays in HBM as
// the GGUF stores it (src/gguf.rs:14-38): Q8_0 34-byte blocks (f16 scale + 32 int8), Q4_0 18-byte
// blocks (f16 scale + 16 bytes of nibbles), F16 or F32 rows.
//
// Main kernel (gemm_lds_kernel; k % 64 == 0, W in Q8_0 / Q4_0 / F16, `a` in f16): two LDS stages
// fed by the LDS DMA of gfx950 — per 64- or 128-wide k step, the a tile (16-byte
// global_load_lds_dwordx4) and each W row's GGUF blocks as stored (68 or 36 bytes per block pair,
// 4-byte global_load_lds_dword; F16 rows like a) — so the next step's bytes land while the MFMAs
// work on the current one.  Each lane dequantizes one block of its W row from LDS into the f16
// operand of v_mfma_f32_32x32x16_f16: int8 q becomes the f16 1024 + (q + 128) by byte placement, an
// exact subtraction gives q, and one packed f16 multiply by the block scale rounds q·d once to
// nearest even — f16(q·d), the reference's exact rounding (products q·d have at most 19 significant
// bits, so f32 and the f16 multiply round the same value).  The epilogues of Epilogue::params
// (src/gpu/mod.rs:445-455; gemm.wgsl:72-94) and the dual outputs are fused into the store, in f32
// or, for a consumer that rounds its input to f16 anyway (another GEMM), in f16.  Shapes with too
// few output tiles for the 256 CUs split k 2 or 4 ways into f32 partial sums that a second kernel
// adds in a fixed order before the epilogue.
//
// Fallback kernel (gemm_reg_kernel; any k % 32 == 0 and F32 weights): a double-buffered a tile in
// LDS and W blocks loaded straight into registers.
#include <algorithm>
#include <cstdio>
#include <mutex>
#include <type_traits>
#include <utility>

#include "internal.h"
#include "gemm_impl.h"

// Chosen per GEMM shape from measurements on MI355X (random operands, inside the encoder step, or
// replayed back to back for m ≥ 1024): many output tiles → 256×256, 192×128 or 128×128 tiles; fewer
// → 64×64 tiles of 4 wavefronts, and when even those leave CUs idle, k split 2 or 4 ways.  Ring slots
// of 64-wide k steps (a slot is refilled NS steps ahead, so NS − 1 steps hide the DMA's latency).
GemmPlan gemm_plan_for(const wh_ctx *ctx, int m, int cols, int k) {
  const int cus = ctx->cus > 0 ? ctx->cus : 256;
  const long t128 = (long)((cols + 127) / 128) * ((m + 127) / 128), t64 = (long)((cols + 63) / 64) * ((m + 63) / 64);
  GemmPlan p{64, 64, 2, 2, 3, 1};
  const long t256 = (long)((cols + 255) / 256) * ((m + 255) / 256);
  if (t128 >= 2L * cus && m >= 4096 && k >= 1024) {
    // Two or more rounds of 128×128 tiles over many rows and a long k (batched windows, m ≈ 12000):
    // wide outputs with at least two rounds of 256×256 tiles take those (8 wavefronts of 128×64, one
    // workgroup per CU: the least a and W traffic per output — 12000×4096×1024 154 µs against 172 for
    // 192×128 and 189 for 128×128); the others 192×128 tiles of 4 wavefronts, two workgroups per CU
    // (12000×3072×1024 119 µs, 12000×1024×1024 44, 12000×1024×4096 152, against 131, 56 and 162 for
    // 256×256 and 124, 47 and 162 for 128×128 tiles of 8).  (The batched position projection,
    // 1515×24576×1024, streams its 27 MB of W from HBM in the step: 128×128 tiles, 2304 of them,
    // run it in 128 µs there, 256×256 tiles in 189.)
    if (cols >= 4096 && t256 >= 2L * cus) p = {256, 256, 2, 4, 2, 1};
    else p = {192, 128, 2, 2, 2, 1};
  } else if (t128 >= 4L * cus) p = {128, 128, 2, 4, 2, 1};
  else if (t128 > cus && t128 <= 2L * cus && k < 4096)
    // Between one and two 128×128 tiles per CU (a 1500-frame window's wide projections): 256×128
    // tiles of 8 wavefronts with 64×64 wave tiles, one per CU, read each a fragment for twice the
    // columns (measured in the Whisper encoder: 6.05 against 6.16 ms per call, fc1 1.28 against
    // 1.35 ms, than 4-wave 128×128 tiles two per CU; at m = 12000 they are slower).
    p = {256, 128, 4, 2, 2, 1};
  else if (t128 > cus && (t128 <= 2L * cus || k >= 4096))
    // More tiles than CUs with a long k (16 windows' FFN down projection): 4-wave workgroups in
    // two slots, two per CU, take them in one round or fewer (measured in the encoder: 16 × 60 s
    // FFN down 8.0 against 8.6 ms per call; the 16 windows' 1024 × 1024 projections stay with 8-wave
    // workgroups, 3.13 against 3.22).
    p = {128, 128, 2, 2, 2, 1};
  else if (t128 * 4 >= 3L * cus)
    // Three quarters of a tile per CU or more (the FFN's first projection at 750 frames): 96×128 tiles
    // of one row of 4 wavefronts (96×32 each: every W fragment dequantized once per workgroup and fed
    // to three MFMAs; 256 workgroups, one per CU) for k ≥ 1024 (60 s step 4.285 against 4.324 ms for
    // 128×128 tiles of 2×4), in two k groups (15.7 against 16.0 µs in the step), else 128×128 tiles;
    // fewer tiles (the qkv projection, 144) run faster as 64×64 tiles (4.96 against 4.98 ms per 60 s
    // call; 96×128 tiles for it: 4.51 against 4.32).
    p = k >= 1024 ? GemmPlan{96, 128, 1, 4, 3, 1, 0, 2} : GemmPlan{128, 128, 2, 4, 3, 1};
  else if (t128 * 4 <= cus && k % (4 * 64) == 0 && k / (4 * 64) >= 16)
    // Long k over few tiles (the FFN's down projection, 750 × 1024 × 4096): k split 4 ways over
    // 96×64 tiles of 2 wavefronts (96×32 per wavefront: each dequantized W fragment feeds three
    // MFMAs) in two slots: 512 workgroups, two per CU, whose barriers do not align (measured in
    // the encoder step, 60 s: 4.64 ms, against 4.68 for 128×64 tiles of 4 wavefronts, 4.75 for
    // 128×128 tiles of 8 wavefronts, 4.92 for 128×64 tiles in three slots, one per CU); in two k
    // groups where they divide every split (14.3 against 15.0 µs in the step, the groups' sums in
    // LDS planes of their own).
    p = {96, 64, 1, 2, 2, 4, 0, k % (4 * 128) == 0 ? 2 : 1};
  else if (t128 * 4 <= 2L * cus && k % (4 * 64) == 0 && k / (4 * 64) >= 16)
    // The same with up to two workgroups per CU (Whisper's fc2, 1500 × 1280 × 5120: 1.18 + its
    // finish against 1.82 ms per call for 64×64 tiles whole).
    p = {128, 128, 2, 2, 2, 4};
  else if (t64 < cus) {
    // Split only while every split keeps at least 16 k steps: shorter ones spend more on the
    // pipeline's fill and the partial sums than the extra workgroups win (k = 1024 runs faster whole).
    while (p.split < 4 && t64 * p.split < 2L * cus && k % (2 * p.split * 64) == 0 && k / (2 * p.split * 64) >= 16)
      p.split *= 2;
    // Unsplit: two k groups of 4 wavefronts over a 4-slot ring (one workgroup per CU; the 750-frame
    // 1024 × 1024 projections 9.5 against 10.0 µs in the step; deeper rings alone are slower there:
    // 10.8 for 5 slots, 11.4 for 8).
    if (p.split == 1 && k % 128 == 0) p = {64, 64, 2, 2, 4, 1, 0, 2};
  } else if (t64 < 2L * cus)
    // One to two 64×64 tiles per CU (the 750-frame pointwise projection, 750 × 2048 × 1024): 96×64
    // tiles of one row of 2 wavefronts in two k groups, one workgroup per CU (11.7 against 12.7 µs
    // in the step for 64×64 tiles; 12.2 with 4 slots).
    p = {96, 64, 1, 2, 2, 1, 0, 2};
  if (ctx->gemm_plan[0]) {  // tuning override (wh_tune "gemm_plan"): bm, bn, wm, wn, stages, split, pipeline, kgroups
    const int *o = ctx->gemm_plan;
    p = {o[0], o[1], o[2], o[3], o[4], o[5], o[6], std::max(1, o[7])};
  }
  for (const auto &o : ctx->gemm_shape_plans)  // tuning override for one shape (wh_tune "gemm_shape_plans")
    if (o[0] == m && o[1] == cols && o[2] == k) p = {o[3], o[4], o[5], o[6], o[7], o[8], o[9], std::max(1, o[10])};
  // Whole k steps per split and k group.
  if (k % (64 * p.wk)) p.wk = 1;
  if (k % (64 * p.wk * p.split)) p.split = 1;
  return p;
}

namespace {

// a (f32) rounded to f16 (RNE; h of the reference), for the GEMMs whose producer wrote f32.
__global__ __launch_bounds__(256) void to_half_kernel(const float4 *__restrict__ x, half4 *__restrict__ y, size_t n4) {
  for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n4; i += (size_t)gridDim.x * 256) {
    const float4 v = x[i];
    y[i] = half4{(_Float16)v.x, (_Float16)v.y, (_Float16)v.z, (_Float16)v.w};
  }
}

// The main kernel's conditions: 64-wide k steps over Q8_0 / Q4_0 / F16 rows, and an output whose
// rows start on 16 bytes (its epilogue stores 8 columns at a time).
bool lds_path(const wh_linear *l, const void *c, int ldc) {
  return l->k % 64 == 0 && (l->type == WH_Q8_0 || l->type == WH_Q4_0 || l->type == WH_F16) && l->row_bytes % 4 == 0 &&
         ldc % 8 == 0 && (uintptr_t)c % 16 == 0;
}


// Scratch bytes for the split-k partial sums of an m-row GEMM (0 when it does not split).
size_t split_bytes(const wh_ctx *ctx, const wh_linear *l, int m) {
  const GemmPlan p = gemm_plan_for(ctx, m, l->cols, l->k);
  return p.split > 1 ? (size_t)p.split * m * l->cols * 4 : 0;
}

// a16: f16 rows; part: scratch for split-k partial sums (or NULL: no split).  With `splits`, a split
// GEMM stops after writing its partial sums (the caller finishes them) and *splits is the count
// (1: c was written whole).
int launch_lds(wh_ctx *ctx, const _Float16 *a, const wh_linear *l, void *c, int m, int ldc, int epi, float alpha,
               bool out16, float *part, int *splits = nullptr, const HeadsOut *ho = nullptr, int nho = 0) {
  switch (l->type) {
    case WH_Q8_0: return gemm_lds_q8_0(ctx, a, l, c, m, ldc, epi, alpha, out16, part, splits, ho, nho);
    case WH_Q4_0: return gemm_lds_q4_0(ctx, a, l, c, m, ldc, epi, alpha, out16, part, splits, ho, nho);
    default: return gemm_lds_f16(ctx, a, l, c, m, ldc, epi, alpha, out16, part, splits, ho, nho);
  }
}

template <int WT, bool ALIGNED, bool A16, bool OUT16>
int launch_t(wh_ctx *ctx, const void *a, const wh_linear *l, void *c, int m, int ldc, int epi, float alpha) {
  // Tile: the largest whose grid still gives every CU a workgroup, else the smallest.
  const int cus = ctx->cus > 0 ? ctx->cus : 256;
  auto tiles = [&](int bm, int bn) { return (long)((l->cols + bn - 1) / bn) * ((m + bm - 1) / bm); };
  int bm = 64, bn = 64;
  if (tiles(128, 128) >= cus) bm = 128, bn = 128;
  else if (tiles(64, 128) >= cus) bm = 64, bn = 128;
  dim3 grid((l->cols + bn - 1) / bn, (m + bm - 1) / bm);
  // Algorithmic work: 2·m·rows·k flops over the real rows; bytes of W as stored, a, c (and c read
  // back by the residual epilogues).
  static const char *tn = WT == WH_F32 ? "f32" : WT == WH_F16 ? "f16" : WT == WH_Q8_0 ? "q8_0" : "q4_0";
  char name[64];
  snprintf(name, sizeof name, "gemm_reg_%s%s_%dx%d", tn, A16 ? "_a16" : "", bm, bn);
  double width = l->cols + l->dual;
  double bytes = (double)l->rows * l->row_bytes + (A16 ? 2.0 : 4.0) * m * l->k +
                 (OUT16 ? 2.0 : 4.0) * m * width * (epi == WH_RESIDUAL || epi == WH_GELU_RESIDUAL ? 2 : 1);
  ProfScope prof(ctx, name, 2.0 * m * l->rows * l->k, bytes);
  if (bm == 128)
    wh_launch(ctx, gemm_reg_kernel<WT, 128, 128, ALIGNED, A16, OUT16>, grid, 256, 0, a, l->w, l->bias, c, m, l->rows, l->cols, l->k, l->dual, ldc, epi, alpha, l->row_bytes);
  else if (bn == 128)
    wh_launch(ctx, gemm_reg_kernel<WT, 64, 128, ALIGNED, A16, OUT16>, grid, 256, 0, a, l->w, l->bias, c, m, l->rows, l->cols, l->k, l->dual, ldc, epi, alpha, l->row_bytes);
  else
    wh_launch(ctx, gemm_reg_kernel<WT, 64, 64, ALIGNED, A16, OUT16>, grid, 256, 0, a, l->w, l->bias, c, m, l->rows, l->cols, l->k, l->dual, ldc, epi, alpha, l->row_bytes);
  return wh_launched(ctx, "gemm");
}

template <bool A16, bool OUT16>
int launch_typed(wh_ctx *ctx, const void *a, const wh_linear *l, void *c, int m, int ldc, int epi, float alpha) {
  const bool aligned = l->k % 64 == 0;
  switch (l->type) {
    case WH_F32: return launch_t<WH_F32, true, A16, OUT16>(ctx, a, l, c, m, ldc, epi, alpha);
    case WH_F16: return launch_t<WH_F16, true, A16, OUT16>(ctx, a, l, c, m, ldc, epi, alpha);
    case WH_Q8_0:
      return aligned ? launch_t<WH_Q8_0, true, A16, OUT16>(ctx, a, l, c, m, ldc, epi, alpha)
                     : launch_t<WH_Q8_0, false, A16, OUT16>(ctx, a, l, c, m, ldc, epi, alpha);
    case WH_Q4_0:
      return aligned ? launch_t<WH_Q4_0, true, A16, OUT16>(ctx, a, l, c, m, ldc, epi, alpha)
                     : launch_t<WH_Q4_0, false, A16, OUT16>(ctx, a, l, c, m, ldc, epi, alpha);
  }
  return wh_fail(ctx, WH_EARG, "gemm: weight type %d", l->type);
}

}  // namespace

bool gemm_glu_ok(const wh_linear *l, const void *c) {
  return l && !l->dual && l->rows == l->cols && l->cols % 16 == 0 && lds_path(l, c, l->cols / 2);
}

// glu: the caller takes EPI_GLU (launch_gemm_h only; the public entry points take WH_BIAS .. WH_TANH).
static int check(wh_ctx *ctx, const void *a, const wh_linear *l, const void *c, int m, int epi, bool glu = false) {
  if (m < 0 || !l || (m && (!a || !c))) return wh_fail(ctx, WH_EARG, "gemm: bad arguments (m %d)", m);
  if ((epi < WH_BIAS || epi > WH_TANH) && !(glu && epi == EPI_GLU))
    return wh_fail(ctx, WH_EARG, "gemm: epilogue %d", epi);
  if (epi == EPI_GLU && !gemm_glu_ok(l, c)) return wh_fail(ctx, WH_EARG, "gemm: GLU epilogue off its layout");
  if ((uintptr_t)a % 16) return wh_fail(ctx, WH_EARG, "gemm: a must be 16-byte aligned");
  return WH_OK;
}

// Workspace of an f32-input GEMM on the main kernel: the f16 copy of `a`, then the split-k partial sums.
static size_t f32_gemm_abytes(const wh_linear *l, int m) { return ((size_t)m * l->k * 2 + 255) / 256 * 256; }

// The f32-input GEMM on the main kernel with its workspace at ws (f32_gemm_abytes + split_bytes).
static int gemm_f32_ws(wh_ctx *ctx, const float *a, const wh_linear *l, float *c, int m, int ldc, int epi, float alpha,
                       uint8_t *ws) {
  const size_t n = (size_t)m * l->k, abytes = f32_gemm_abytes(l, m);
  _Float16 *a16 = (_Float16 *)ws;
  {
    ProfScope prof(ctx, "to_half", 0.0, 6.0 * n);
    const size_t n4 = n / 4;
    const int blocks = (int)std::min<size_t>((n4 + 255) / 256, 4096);
    wh_launch(ctx, to_half_kernel, blocks, 256, 0, (const float4 *)a, (half4 *)a16, n4);
    if (int rc = wh_launched(ctx, "gemm: rounding a")) return rc;
  }
  return launch_lds(ctx, a16, l, c, m, ldc, epi, alpha, false, (float *)(ws + abytes));
}

int launch_gemm(wh_ctx *ctx, const float *a, const wh_linear *l, float *c, int m, int ldc, int epi, float alpha) {
  if (int rc = check(ctx, a, l, c, m, epi)) return rc;
  if (m == 0) return WH_OK;
  if (!lds_path(l, c, ldc)) return launch_typed<false, false>(ctx, a, l, c, m, ldc, epi, alpha);
  // The main kernel takes a in f16: round it once into scratch (followed by the split partials).
  uint8_t *ws = (uint8_t *)wh_scratch(ctx, f32_gemm_abytes(l, m) + split_bytes(ctx, l, m));
  if (!ws) return WH_EOOM;
  return gemm_f32_ws(ctx, a, l, c, m, ldc, epi, alpha, ws);
}

// ------------------------------------------------------------------ the GEMM that allocates nothing
// wh_gemm_noalloc's workspace (the f16 copy of `a` and the split-k partial sums): a file-scope device
// array, which every device the library runs on holds until the process ends.  In host code its name
// is not a device address: the address comes from hipGetSymbolAddress, once per device with that
// device current (gemm_noalloc_init, from wh_open), and only that address is used.  Every call on a
// device shares the array, so calls that overlap on one device (other streams or contexts) race; a
// call writes all of the workspace it reads (the rounded `a` and every split's partial plane), so
// nothing in it has to start at zero.
constexpr size_t NOALLOC_BYTES = (size_t)32 << 20;
static __device__ __align__(256) uint8_t scratch[NOALLOC_BYTES];

namespace {
constexpr int NOALLOC_DEVICES = 64;
// Per device: the workspace address, the failed lookup's error, and the last call's stream with an
// event recorded after its kernels (created at set-up, with the address).
struct NoallocDevice {
  void *addr = nullptr;
  hipError_t err = hipSuccess;
  hipEvent_t done = nullptr;
  hipStream_t last = nullptr;
};
std::mutex noalloc_mu;
NoallocDevice noalloc_dev[NOALLOC_DEVICES];
}  // namespace

int gemm_noalloc_init(wh_ctx *ctx) {
  std::lock_guard<std::mutex> lock(noalloc_mu);
  ctx->noalloc = nullptr;
  if (ctx->device < 0 || ctx->device >= NOALLOC_DEVICES) return WH_EGPU;
  NoallocDevice &d = noalloc_dev[ctx->device];
  if (!d.addr && d.err == hipSuccess) {
    void *p = nullptr;
    hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e == hipSuccess && p) e = hipEventCreateWithFlags(&d.done, hipEventDisableTiming);
    if (e != hipSuccess || !p) {
      (void)hipGetLastError();
      d.err = e != hipSuccess ? e : hipErrorInvalidSymbol;
    } else {
      d.addr = p;
    }
  }
  ctx->noalloc = d.addr;
  ctx->noalloc_error = ctx->noalloc ? hipSuccess : d.err;
  return ctx->noalloc ? WH_OK : WH_EGPU;
}

size_t wh_gemm_noalloc_limit(void) { return NOALLOC_BYTES; }

int wh_gemm_noalloc(wh_ctx *ctx, const float *a, const wh_linear *l, float *c, int m, int epi, float alpha) {
  if (!ctx || !l) return WH_EARG;
  if (int rc = check(ctx, a, l, c, m, epi)) return rc;
  if (!ctx->noalloc)
    return wh_fail(ctx, WH_EGPU, "wh_gemm_noalloc: no workspace address on device %d (%s)", ctx->device,
                   hipGetErrorString(ctx->noalloc_error));
  if (ctx->prof == 1) return wh_fail(ctx, WH_EARG, "wh_gemm_noalloc: per-launch profiling creates events; turn it off");
  if (m == 0) return WH_OK;
  const int ldc = l->cols + l->dual;
  if (!lds_path(l, c, ldc)) return launch_typed<false, false>(ctx, a, l, c, m, ldc, epi, alpha);  // no workspace
  const size_t need = f32_gemm_abytes(l, m) + split_bytes(ctx, l, m);
  if (need > NOALLOC_BYTES)
    return wh_fail(ctx, WH_EARG, "wh_gemm_noalloc: %d x %d x %d needs %zu bytes of workspace, more than its %zu", m,
                   l->rows, l->k, need, NOALLOC_BYTES);
  // The workspace is shared by every call on the device: a call from another stream while the last
  // call's kernels may still run would corrupt both, so it is refused (calls must be serialized).  A
  // stream under capture is neither checked nor remembered (its kernels run at replay).
  std::lock_guard<std::mutex> lock(noalloc_mu);
  NoallocDevice &d = noalloc_dev[ctx->device];
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(ctx->stream, &cs) != hipSuccess) {
    (void)hipGetLastError();
    cs = hipStreamCaptureStatusNone;
  }
  const bool capturing = cs != hipStreamCaptureStatusNone;
  if (!capturing && d.last && d.last != ctx->stream) {
    const hipError_t q = hipEventQuery(d.done);
    if (q != hipSuccess) {
      (void)hipGetLastError();
      if (q == hipErrorNotReady)
        return wh_fail(ctx, WH_EARG,
                       "wh_gemm_noalloc: the last call on device %d (another stream) may still be running; its "
                       "workspace is shared, so calls on one device must not overlap", ctx->device);
    }
  }
  const int rc = gemm_f32_ws(ctx, a, l, c, m, ldc, epi, alpha, (uint8_t *)ctx->noalloc);
  if (rc == WH_OK && !capturing) {
    if (hipEventRecord(d.done, ctx->stream) == hipSuccess) d.last = ctx->stream;
    else (void)hipGetLastError();
  }
  return rc;
}

int launch_to_half(wh_ctx *ctx, const float *x, void *y, size_t n) {
  if (n % 4 || (uintptr_t)x % 16 || (uintptr_t)y % 8) return wh_fail(ctx, WH_EARG, "to_half: n %% 4 == 0 and aligned buffers");
  if (!n) return WH_OK;
  ProfScope prof(ctx, "to_half", 0.0, 6.0 * n);
  const size_t n4 = n / 4;
  const int blocks = (int)std::min<size_t>((n4 + 255) / 256, 4096);
  wh_launch(ctx, to_half_kernel, blocks, 256, 0, (const float4 *)x, (half4 *)y, n4);
  return wh_launched(ctx, "to_half");
}

int launch_gemm_h(wh_ctx *ctx, const void *a16, const wh_linear *l, void *c, int m, int ldc, int epi, float alpha,
                  int out16) {
  if (int rc = check(ctx, a16, l, c, m, epi, true)) return rc;
  if (out16 && (epi == WH_RESIDUAL || epi == WH_GELU_RESIDUAL))
    return wh_fail(ctx, WH_EARG, "gemm: residual epilogues accumulate into f32 outputs");
  if (epi == EPI_GLU && (out16 || ldc != l->cols / 2))
    return wh_fail(ctx, WH_EARG, "gemm: the GLU epilogue writes f32 rows of cols / 2");
  if (m == 0) return WH_OK;
  // (no split-k partials for the GLU epilogue: the main kernel finishes its own tiles)
  if (epi == EPI_GLU) return launch_lds(ctx, (const _Float16 *)a16, l, c, m, ldc, epi, alpha, false, nullptr);
  if (lds_path(l, c, ldc)) {
    const size_t pb = split_bytes(ctx, l, m);
    float *part = nullptr;
    if (pb && !(part = (float *)wh_scratch(ctx, pb))) return WH_EOOM;
    return launch_lds(ctx, (const _Float16 *)a16, l, c, m, ldc, epi, alpha, out16 != 0, part);
  }
  if (out16) return launch_typed<true, true>(ctx, a16, l, c, m, ldc, epi, alpha);
  return launch_typed<true, false>(ctx, a16, l, c, m, ldc, epi, alpha);
}

int launch_gemm_h_heads(wh_ctx *ctx, const void *a16, const wh_linear *l, void *c, int m, int ldc, int epi,
                        const HeadsOut *outs, int n) {
  if (int rc = check(ctx, a16, l, c, m, epi)) return rc;
  if (epi == WH_RESIDUAL || epi == WH_GELU_RESIDUAL) return wh_fail(ctx, WH_EARG, "gemm: packed output with a residual epilogue");
  if (!lds_path(l, c, ldc) || !outs || n <= 0) return wh_fail(ctx, WH_EARG, "gemm: packed output needs the main kernel");
  for (int i = 0; i < n; i++)
    if (!outs[i].dst || outs[i].hd <= 0) return wh_fail(ctx, WH_EARG, "gemm: packed output %d", i);
  if (m == 0) return WH_OK;
  return launch_lds(ctx, (const _Float16 *)a16, l, c, m, ldc, epi, 0.0f, true, nullptr, nullptr, outs, n);
}

int launch_gemm_h_ln(wh_ctx *ctx, const void *a16, const wh_linear *l, float *x, int m, float alpha, const float *g,
                     const float *b, void *y, int out16, int keep_x, const float *g2, const float *b2, void *y2,
                     int residual) {
  const int epi = residual ? WH_RESIDUAL : WH_BIAS;
  if (int rc = check(ctx, a16, l, x, m, epi)) return rc;
  if (m == 0) return WH_OK;
  if (g2 && (out16 || !b2 || !y2)) return wh_fail(ctx, WH_EARG, "gemm_h_ln: the second norm takes an f32 y");
  const int cols = l->cols;
  // The GEMM adds the residual into x, then one or two LayerNorm launches (one pass for both norms,
  // the fused finish kernel without partial sums, measured slower at 11616 rows: 51 against ~24 µs).
  auto unfused = [&](int rc) {
    if (rc) return rc;
    if ((rc = launch_layer_norm(ctx, x, g, b, y, m, cols, nullptr, nullptr, 0, out16))) return rc;
    return g2 ? launch_layer_norm(ctx, (const float *)y, g2, b2, y2, m, cols, nullptr, nullptr, 0, 1) : WH_OK;
  };
  if (l->dual || !lds_path(l, x, cols)) return unfused(launch_gemm_h(ctx, a16, l, x, m, cols, epi, alpha, 0));
  const size_t pb = split_bytes(ctx, l, m);
  float *part = nullptr;
  if (pb && !(part = (float *)wh_scratch(ctx, pb))) return WH_EOOM;
  int splits = 1;
  if (int rc = launch_lds(ctx, (const _Float16 *)a16, l, x, m, cols, epi, alpha, false, part, &splits)) return rc;
  if (splits > 1)
    return launch_split_residual_ln(ctx, part, splits, l->bias, l->rows, residual ? alpha : 1.0f, x, g, b, y, m, cols,
                                    out16, keep_x, g2, b2, y2, residual);
  return unfused(WH_OK);
}
