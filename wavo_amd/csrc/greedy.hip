// Greedy decoders of an encoder output on the device: CTC (src/gigaam/decoder.rs:135-151) and the
// TDT loop with its LSTM predictor and joint (src/parakeet/decoder.rs:91-191).  The reference runs
// both on the host; here the encoder output never leaves the device and only the (token, frame)
// pairs come back.
//
// TDT: the loop's control state lives in device memory (TdtState), so one decision is a fixed
// sequence of three launches that a caller records once and replays until the state says done.
// tdt_joint_kernel builds z = ReLU(enc[t] + pred) in LDS and takes its share of the output layer's
// rows, keeping the first maximum of its token rows and of its duration rows; tdt_step_kernel
// reduces those in every workgroup to the same decision (workgroup 0 applies the frame / symbol
// rules to the next state and appends the emission) and, after an emission, runs the first LSTM
// layer on the token's embedding row, a wavefront per cell (its four gate rows of [Wx | Wh], the
// gates and the cell); tdt_pred_kernel projects the last layer's h for the joint and makes the next
// state current.  Further LSTM layers take one launch each.  The decoder's weights (the C1 shape:
// 9.5 MB) stay in the L2 caches between decisions, so each product is a wavefront per row reading
// the blocks as stored.
#include <cfloat>

#include "internal.h"
#include "xlane.h"

namespace {

__device__ __forceinline__ bool better(float v, int i, float bv, int bi) {
  // The first maximum: a larger value, or an equal one at a smaller index.
  return v > bv || (v == bv && i < bi);
}

// (value, index) of the first maximum of x[0..n) over a workgroup of 256 threads; every thread gets it.
__device__ __forceinline__ void wg_argmax(const float *__restrict__ x, int n, float *sv, int *si, float &v, int &i) {
  const int tid = threadIdx.x;
  float bv = -FLT_MAX;
  int bi = n;
  for (int j = tid; j < n; j += 256) {
    const float y = x[j];
    if (bi == n || better(y, j, bv, bi)) bv = y, bi = j;
  }
  xlane::wave_first_max(bv, bi, [n](float ov, int oi, float v, int i) { return oi < n && (i == n || better(ov, oi, v, i)); });
  if ((tid & 63) == 0) sv[tid >> 6] = bv, si[tid >> 6] = bi;
  __syncthreads();
  v = sv[0], i = si[0];
  for (int w = 1; w < 4; w++)
    if (si[w] < n && (i == n || better(sv[w], si[w], v, i))) v = sv[w], i = si[w];
  __syncthreads();
}

__device__ __forceinline__ float half_to_f(uint32_t h) { return (float)__builtin_bit_cast(_Float16, (uint16_t)h); }

// 16 weights of a row as the file stores them (half of a 32-weight block: weights 16·hb .. 16·hb + 15),
// loaded into registers first and multiplied with x (in LDS) later, so that a wavefront issues every
// load of its rows before it waits for any.  Q8_0 / Q4_0: the block's scale and the 16 bytes (Q4_0: the
// block's 16 bytes, whose low or high nibbles are these weights), as 2-byte words (blocks start on 2
// bytes); F16: 32 bytes; F32: 64 bytes.
template <int WT>
struct Half {
  static constexpr int R = WT == WH_F32 ? 16 : WT == WH_F16 ? 8 : 9;
  uint32_t r[R];

  __device__ __forceinline__ void load(const uint8_t *__restrict__ row, int hb) {
    if constexpr (WT == WH_F32 || WT == WH_F16) {
      const uint4 *p = (const uint4 *)(row + (size_t)hb * R * 4);
#pragma unroll
      for (int i = 0; i < R / 4; i++) {
        const uint4 v = p[i];
        r[4 * i] = v.x, r[4 * i + 1] = v.y, r[4 * i + 2] = v.z, r[4 * i + 3] = v.w;
      }
    } else {
      // Aligned dword loads (blocks start on 2 bytes; wide loads at 2 bytes past a dword are split by
      // the hardware): the dword holding the scale, and the 5 dwords covering these 16 weights'
      // bytes, whose 2-byte words start at bit 0 or 16 of the first (a select, not an indexed register).
      const size_t at = (size_t)(hb >> 1) * (WT == WH_Q8_0 ? 34 : 18);
      const size_t data = at + 2 + (WT == WH_Q8_0 ? 16 * (hb & 1) : 0);
      const uint32_t sc = *(const uint32_t *)(row + (at & ~(size_t)3));
      const uint32_t *p = (const uint32_t *)(row + (data & ~(size_t)3));
      uint32_t d[5];
#pragma unroll
      for (int i = 0; i < 5; i++) d[i] = p[i];
      r[0] = (sc >> ((at & 3) * 8)) & 0xffffu;
      const bool odd = data & 3;  // the words start at bit 16
#pragma unroll
      for (int e = 0; e < 8; e++) {
        const uint32_t even = (d[e >> 1] >> (16 * (e & 1))) & 0xffffu;
        const uint32_t shifted = (d[(e + 1) >> 1] >> (16 * ((e + 1) & 1))) & 0xffffu;
        r[1 + e] = odd ? shifted : even;
      }
    }
  }

  __device__ __forceinline__ float dot(int hb, const float *x) const {
    const float *xv = x + 16 * hb;
    float s = 0.0f;
    if constexpr (WT == WH_F32) {
#pragma unroll
      for (int e = 0; e < 16; e++) s += __builtin_bit_cast(float, r[e]) * xv[e];
      return s;
    } else if constexpr (WT == WH_F16) {
#pragma unroll
      for (int e = 0; e < 8; e++) s += half_to_f(r[e] & 0xffffu) * xv[2 * e] + half_to_f(r[e] >> 16) * xv[2 * e + 1];
      return s;
    } else if constexpr (WT == WH_Q8_0) {
#pragma unroll
      for (int e = 0; e < 8; e++)
        s += (float)(int8_t)(r[1 + e] & 0xffu) * xv[2 * e] + (float)(int8_t)(r[1 + e] >> 8) * xv[2 * e + 1];
      return s * half_to_f(r[0]);
    } else {
      const int sh = 4 * (hb & 1);
#pragma unroll
      for (int e = 0; e < 8; e++)
        s += (float)((int)((r[1 + e] >> sh) & 15u) - 8) * xv[2 * e] +
             (float)((int)((r[1 + e] >> (8 + sh)) & 15u) - 8) * xv[2 * e + 1];
      return s * half_to_f(r[0]);
    }
  }
};

// Rows per wavefront in the joint's output layer (8198 rows of the C1 shape over 513 workgroups: two
// per CU, so each wavefront's chain of products is half as long as with 8 rows).
template <int WT>
constexpr int rows_per_wave() { return 4; }
// Rows per wavefront of the predictor's projection (joint outputs: 640 rows over 80 workgroups).
template <int WT>
constexpr int pred_rows_per_wave() { return 2; }

// Sums each of the N = 2, 4 or 8 values of every lane over the wavefront; afterwards lanes 64·v/N ..
// 64·(v + 1)/N − 1 hold value v's sum.  Each halving step pairs a lane with the one that differs in
// a lane bit (5, 4, then 3 for N = 8) and leaves it half its values (the upper half where the bit is
// set) plus the partner's of the same half; then the lanes that hold the same value sum it.
template <int N>
__device__ __forceinline__ float wave_sums(float (&v)[N]) {
  static_assert(N == 2 || N == 4 || N == 8, "2, 4 or 8 values");
  float c[N];
#pragma unroll
  for (int i = 0; i < N; i++) c[i] = v[i];
#pragma unroll
  for (int i = 0; i < N / 2; i++) {
    float x = c[i], y = c[N / 2 + i];
    xlane::swap32(x, y);
    c[i] = x + y;
  }
#pragma unroll
  for (int i = 0; i < N / 4; i++) {
    float x = c[i], y = c[N / 4 + i];
    xlane::swap16(x, y);
    c[i] = x + y;
  }
  float s;
  if constexpr (N == 8) {
    const bool up = threadIdx.x & 8;
    s = (up ? c[1] : c[0]) + xlane::dpp<xlane::ROR8>(up ? c[0] : c[1]);
  } else {
    s = c[0];
  }
  // The lanes that share the value: 8 (N = 8), 16 (N = 4) or 32 (N = 2) consecutive ones.
  s += xlane::dpp<xlane::XOR1>(s);
  s += xlane::dpp<xlane::XOR2>(s);
  s += xlane::dpp<xlane::HALF_MIRROR>(s);
  if constexpr (N <= 4) s += xlane::dpp<xlane::MIRROR>(s);
  if constexpr (N == 2) s = xlane::bit4(s, xlane::Add{});
  return s;
}

// The first maximum of every lane's (v, i) over the wavefront, in every lane; index −1 is none.
__device__ __forceinline__ void wave_first_max(float &v, int &i) {
  xlane::wave_first_max(v, i, [](float ov, int oi, float bv, int bi) { return oi >= 0 && (bi < 0 || better(ov, oi, bv, bi)); });
}

// ------------------------------------------------------------------ weight rows staged through LDS
// A workgroup's weight rows are one run of contiguous bytes (the joint's or the predictor's 4·RW
// consecutive rows) or four (an LSTM workgroup's four cells: rows g·n + 4·blockIdx.x .. + 3 of gate
// g).  They go into LDS in whole 16-byte chunks, a coalesced 16-byte load per lane and chunk with
// every load of a round issued before any store, and the products read them from LDS: one memory
// round trip for all of a wavefront's rows.  (Each lane loading its 2-byte-aligned half blocks as a
// few dwords straight from global memory took ~5 µs for a wavefront's 8 rows: many small requests
// per row.)  A run starts `lead` = its offset & 15 bytes into its first chunk.  The chunks copied
// cover the run's bytes and stay inside the layer's allocation, which is 256-byte aligned (so offsets
// and addresses agree mod 16) with 256 bytes of zeros after its last row.
constexpr int STAGE_P = 8;  // chunks per thread and round: 32 KiB per workgroup and round

// LDS chunks given to a run of `bytes` bytes (its lead is a multiple of 4: rows of whole dwords).
__host__ __device__ constexpr int run_chunks(size_t bytes) { return (int)((bytes + 12 + 15) / 16); }

template <int RUNS>
struct Runs {
  const uint8_t *w;
  size_t start[RUNS];  // byte offsets of the runs in w
  int len;             // chunks copied per run (≤ cpr)
  int cpr;             // LDS chunks per run

  __device__ __forceinline__ const uint4 *base(int g) const { return (const uint4 *)(w + (start[g] & ~(size_t)15)); }
  // Where run g's first byte lands in LDS.
  __device__ __forceinline__ const uint8_t *at(const uint4 *lds, int g) const {
    return (const uint8_t *)(lds + g * cpr) + (start[g] & 15);
  }
};

// One run of `nrows` rows of rb bytes from row `first` (fewer than the run's LDS room at a layer's end:
// only the chunks of the rows that exist are copied).
__device__ __forceinline__ Runs<1> one_run(const uint8_t *w, size_t rb, int first, int nrows, int cpr) {
  Runs<1> r;
  r.w = w, r.start[0] = (size_t)first * rb, r.cpr = cpr;
  r.len = (int)(((r.start[0] & 15) + (size_t)nrows * rb + 15) / 16);
  return r;
}

// One round of a staging copy: chunks j0 + tid + 256·i (i < STAGE_P / RUNS) of every run.
template <int RUNS>
struct StageRound {
  static constexpr int PR = STAGE_P / RUNS;
  uint4 v[STAGE_P];

  __device__ __forceinline__ void load(const Runs<RUNS> &r, int j0) {
#pragma unroll
    for (int g = 0; g < RUNS; g++)
#pragma unroll
      for (int i = 0; i < PR; i++) v[g * PR + i] = r.base(g)[min(j0 + (int)threadIdx.x + 256 * i, r.len - 1)];  // clamped
  }
  // Unconditional (lanes past the end write the last chunk again, the same bytes): a store behind a
  // branch lets the compiler sink its load there, after the waits that precede it.
  __device__ __forceinline__ void store(uint4 *lds, const Runs<RUNS> &r, int j0) const {
#pragma unroll
    for (int g = 0; g < RUNS; g++)
#pragma unroll
      for (int i = 0; i < PR; i++) lds[g * r.cpr + min(j0 + (int)threadIdx.x + 256 * i, r.len - 1)] = v[g * PR + i];
  }
};

// The rounds after the first (runs longer than 256·STAGE_P / RUNS chunks), a round trip each.
template <int RUNS>
__device__ __forceinline__ void stage_rest(uint4 *lds, const Runs<RUNS> &r) {
  constexpr int STEP = 256 * StageRound<RUNS>::PR;
  for (int j0 = STEP; j0 < r.len; j0 += STEP) {
    StageRound<RUNS> s;
    s.load(r, j0);
    s.store(lds, r, j0);
  }
}

// RW consecutive rows from r0 (those below `rows`) of a layer with k ≤ 1024 inputs, held by one
// wavefront and staged in LDS (row r at run + (r − rr0)·rb, rr0 the run's first row); lane 64·i/RW
// gets row i's value (plus bias).
template <int WT, int RW>
struct Rows {
  float b;
  int r0, rows, k;

  // The bias load, issued with the kernel's other loads.
  __device__ __forceinline__ void init(const float *__restrict__ bias, int first, int nrows, int kk) {
    r0 = first, rows = nrows, k = kk;
    b = bias[min(r0 + (int)(threadIdx.x & 63) * RW / 64, rows - 1)];
  }

  // The value of row r0 + lane·RW/64 (0 past the rows).
  __device__ __forceinline__ float finish(const uint8_t *run, int rr0, size_t rb, const float *x) const {
    const int lane = threadIdx.x & 63, hb = min(lane, k / 16 - 1);
    const bool on = lane < k / 16;
    Half<WT> h[RW];
#pragma unroll
    for (int i = 0; i < RW; i++) h[i].load(run + (size_t)(min(r0 + i, rows - 1) - rr0) * rb, hb);
    float v[RW];
#pragma unroll
    for (int i = 0; i < RW; i++) v[i] = on && r0 + i < rows ? h[i].dot(hb, x) : 0.0f;
    return wave_sums<RW>(v) + b;
  }
};

// LDS of the joint's and the predictor's weight rows (4·RW rows per workgroup).
template <int WT>
__host__ __device__ constexpr int rows_cpr(size_t rb) { return run_chunks(4 * rows_per_wave<WT>() * rb); }
template <int WT>
__host__ __device__ constexpr int pred_rows_cpr(size_t rb) { return run_chunks(4 * pred_rows_per_wave<WT>() * rb); }

// Stages n ≤ 256·P values into LDS: every load into registers first (one round trip), then the stores,
// unconditional as the staged rows' (lanes past n write value n − 1 again).
template <int P, typename F>
__device__ __forceinline__ void stage(float *dst, int n, F value) {
  float v[P];
#pragma unroll
  for (int i = 0; i < P; i++) v[i] = value(min((int)threadIdx.x + 256 * i, n - 1));  // clamped: no branch
#pragma unroll
  for (int i = 0; i < P; i++) dst[min((int)threadIdx.x + 256 * i, n - 1)] = v[i];
}

// Keeps a loaded value's load where it is: the compiler would otherwise sink it into the branch that
// uses it, behind the decision's own round trip.
__device__ __forceinline__ void pin(float v) { asm volatile("" : : "v"(v)); }

__device__ __forceinline__ float sigm(float v) { return 1.0f / (1.0f + expf(-v)); }

// One TDT decision, first part (Decoder::joint, src/parakeet/decoder.rs:135-149): the joint's input
// z = ReLU(enc[t] + pred) (made by the previous decision's last kernel) in LDS, this workgroup's rows
// of the output layer (RW per wavefront), and the first maximum of its token rows and of its duration
// rows into part[blockIdx.x] (value, index, value, index; index −1 when it has none).
template <int WT>
__global__ __launch_bounds__(256) void tdt_joint_kernel(TdtArgs a) {
  constexpr int RW = rows_per_wave<WT>();
  extern __shared__ uint4 lds[];
  __shared__ float bv[2][4];
  __shared__ int bi[2][4];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  // The workgroup's rows and z (written by the previous decision's last kernel) in one round trip.
  const int g0 = blockIdx.x * 4 * RW, r0 = g0 + wave * RW;
  const Runs<1> run = one_run(a.out_w, a.out_rb, g0, min(4 * RW, a.out_rows - g0), rows_cpr<WT>(a.out_rb));
  StageRound<1> w0;
  w0.load(run, 0);
  Rows<WT, RW> rows;
  rows.init(a.out_b, r0, a.out_rows, a.joint);
  float *z = (float *)(lds + run.cpr);
  const float *zg = a.z;
  const int done = a.st->done;
  stage<4>(z, a.joint, [&](int j) { return zg[j]; });
  w0.store(lds, run, 0);
  pin(rows.b);
  if (done) return;
  stage_rest(lds, run);
  __syncthreads();
  // Row r0 + i's value is in lane 64·i/RW: the first maximum over those lanes, in row order.
  const float val = rows.finish(run.at(lds, 0), g0, a.out_rb, z);
  const int r = r0 + lane * RW / 64;
  const bool mine = lane % (64 / RW) == 0 && r < a.out_rows;
  float tv = -FLT_MAX, dv = -FLT_MAX;
  int ti = -1, di = -1;
  if (mine) {
    if (r < a.cfg.classes) tv = val, ti = r;
    else dv = val, di = r - a.cfg.classes;
  }
  wave_first_max(tv, ti);
  wave_first_max(dv, di);
  if (lane == 0) bv[0][wave] = tv, bi[0][wave] = ti, bv[1][wave] = dv, bi[1][wave] = di;
  __syncthreads();
  if (tid == 0) {
    float out[4];
    for (int k = 0; k < 2; k++) {
      float bvv = -FLT_MAX;
      int bii = -1;
      for (int w = 0; w < 4; w++)
        if (bi[k][w] >= 0 && (bii < 0 || better(bv[k][w], bi[k][w], bvv, bii))) bvv = bv[k][w], bii = bi[k][w];
      out[2 * k] = bvv, out[2 * k + 1] = (float)bii;
    }
    *(float4 *)(a.part + 4 * blockIdx.x) = float4{out[0], out[1], out[2], out[3]};
  }
}

// LDS chunks per gate run of an LSTM workgroup (four cells' rows of one gate).
__host__ __device__ constexpr int lstm_cpr(size_t rb) { return run_chunks(4 * rb); }

// One LSTM layer's cell k (one per wavefront) over [x | h_old] (2n ≤ 2048 values in LDS): the four gate
// rows k, n + k, 2n + k, 3n + k of the joined [Wx | Wh] (staged in LDS with the workgroup's other
// cells') with the bias, c' = σ(f)·c + σ(i)·tanh(g), h' = σ(o)·tanh(c').
template <int WT>
struct Cell {
  float b[4], cold;
  int k, hbs;

  // The workgroup's four gate runs (n % 16 == 0: every workgroup has four cells).
  __device__ __forceinline__ static Runs<4> runs(const TdtArgs &a, int layer) {
    Runs<4> r;
    r.w = a.lstm_w[layer], r.cpr = r.len = lstm_cpr(a.lstm_rb);
#pragma unroll
    for (int g = 0; g < 4; g++) r.start[g] = (size_t)(g * a.n + 4 * (int)blockIdx.x) * a.lstm_rb;
    return r;
  }

  // The biases and the cell's c, issued with the kernel's other loads.
  __device__ __forceinline__ void init(const TdtArgs &a, int layer) {
    const int n = a.n;
    hbs = 2 * n / 16;
    k = blockIdx.x * 4 + (threadIdx.x >> 6);
    const int kk = min(k, n - 1);
    const float *bias = a.lstm_b[layer];
#pragma unroll
    for (int g = 0; g < 4; g++) b[g] = bias[g * n + kk];
    cold = a.c[(size_t)layer * n + kk];
  }
  __device__ __forceinline__ void pin_loads() const {
#pragma unroll
    for (int g = 0; g < 4; g++) pin(b[g]);
    pin(cold);
  }

  __device__ __forceinline__ void finish(const TdtArgs &a, int layer, const Runs<4> &run, const uint4 *lds,
                                         const float *xin, float *h_new) const {
    const int n = a.n, lane = threadIdx.x & 63, cell = threadIdx.x >> 6;
    Half<WT> h[4][2];
#pragma unroll
    for (int g = 0; g < 4; g++) {
      const uint8_t *row = run.at(lds, g) + (size_t)cell * a.lstm_rb;
#pragma unroll
      for (int i = 0; i < 2; i++) h[g][i].load(row, min(lane + 64 * i, hbs - 1));
    }
    float acc[4];
#pragma unroll
    for (int g = 0; g < 4; g++) {
      float s = 0.0f;
#pragma unroll
      for (int i = 0; i < 2; i++)
        if (lane + 64 * i < hbs) s += h[g][i].dot(lane + 64 * i, xin);
      acc[g] = s;
    }
    // Gate g's sum lands in lanes 16g..16g + 15: lane 0 gathers all four.
    const float own = wave_sums<4>(acc);
    float gate[4];
#pragma unroll
    for (int g = 0; g < 4; g++) gate[g] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, own), 16 * g)) + b[g];
    if (lane == 0 && k < n) {
      const float cc = sigm(gate[1]) * cold + sigm(gate[0]) * tanhf(gate[2]);
      a.c[(size_t)layer * n + k] = cc;
      h_new[k] = sigm(gate[3]) * tanhf(cc);
    }
  }
};

// One TDT decision, second part: every workgroup reduces the joint's partial maxima to the same
// decision (the token and duration argmaxes, src/parakeet/decoder.rs:158-191) and workgroup 0 writes
// the next state and appends the emission; then, after an emission, the first LSTM layer over the
// token's embedding row (Decoder::predict, :107-133).  INIT: the first predict(None): no decision,
// a zero input.
template <int WT, bool INIT>
__global__ __launch_bounds__(256) void tdt_step_kernel(TdtArgs a) {
  extern __shared__ uint4 lds[];
  __shared__ float sv[2][4];
  __shared__ int si[2][4];
  const int tid = threadIdx.x, n = a.n;
  // The cells' weight rows, biases and c and the old h do not depend on the decision: their loads go
  // out first.
  Cell<WT> cell;
  const Runs<4> run = Cell<WT>::runs(a, 0);
  StageRound<4> w0;
  w0.load(run, 0);
  cell.init(a, 0);
  float *xin = (float *)(lds + 4 * run.cpr);
  float hv[4];
#pragma unroll
  for (int i = 0; i < 4; i++) hv[i] = a.h_old[min(tid + 256 * i, n - 1)];
  // The parts' first maxima (token rows, duration rows): every part loaded with the rest, and the
  // state (one round trip for all).
  float4 q[4];
  if constexpr (!INIT) {
#pragma unroll
    for (int i = 0; i < 4; i++) q[i] = *(const float4 *)(a.part + 4 * min(tid + 256 * i, a.parts - 1));  // clamped: no branch
  }
  const int done0 = INIT ? 0 : a.st->done;
  w0.store(lds, run, 0);
#pragma unroll
  for (int i = 0; i < 4; i++) xin[n + min(tid + 256 * i, n - 1)] = hv[i];  // the old h: layer 0's input's second half
  cell.pin_loads();
  if (done0) return;
  int token = 0;
  float ev[4] = {0.0f, 0.0f, 0.0f, 0.0f};  // the emitted token's embedding row (zero for the first predict)
  if constexpr (!INIT) {
    const TdtState *st = a.st;
#pragma unroll
    for (int k = 0; k < 2; k++) {
      float v = -FLT_MAX;
      int i = -1;
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const float pv = k ? q[j].z : q[j].x;
        const int pi = tid + 256 * j < a.parts ? (int)(k ? q[j].w : q[j].y) : -1;  // clamped copies: none
        if (pi >= 0 && (i < 0 || better(pv, pi, v, i))) v = pv, i = pi;
      }
      wave_first_max(v, i);
      if ((tid & 63) == 0) sv[k][tid >> 6] = v, si[k][tid >> 6] = i;
    }
    __syncthreads();
    int dec[2];
#pragma unroll
    for (int k = 0; k < 2; k++) {
      float bvv = -FLT_MAX;
      int bii = -1;
      for (int w = 0; w < 4; w++)
        if (si[k][w] >= 0 && (bii < 0 || better(sv[k][w], si[k][w], bvv, bii))) bvv = sv[k][w], bii = si[k][w];
      dec[k] = bii;
    }
    token = dec[0];
    const int dur = a.cfg.durations[dec[1]], t = st->t;
    const bool emit = token != a.cfg.blank;
    int nt = t, symbols = st->symbols, left = st->left;
    if (a.cfg.global) {
      left--;
      nt = t + (token == a.cfg.blank ? max(dur, 1) : dur);
    } else {
      nt = t + dur;
      symbols++;
      if (dur != 0) {
        symbols = 0;
      } else if (symbols >= a.cfg.max_symbols || token == a.cfg.blank) {
        nt++;
        symbols = 0;
      }
    }
    const int done = nt >= st->frames || (a.cfg.global && left <= 0);
    const int idle = (!emit || done) ? 1 : 0;
    // The decision's dependent loads go out together: the token's embedding row (layer 0's input)
    // and, below, the next frame's encoder row.
    {
      const float *row = a.embed + (size_t)min(max(token, 0), a.cfg.classes - 1) * n;
#pragma unroll
      for (int i = 0; i < 4; i++) ev[i] = row[min(tid + 256 * i, n - 1)];  // clamped: no branch
    }
    // The next frame's encoder row, for the next joint input: each workgroup its slice.
    if (!done) {
      const float *e = st->enc + (size_t)nt * st->width;
      for (int j = blockIdx.x * 256 + tid; j < a.joint; j += gridDim.x * 256) a.erow[j] = e[j];
    }
    if (blockIdx.x == 0 && tid == 0) {
      TdtState nx = *st;
      if (emit) {
        if (nx.count < nx.cap) {
          nx.out[2 * nx.count] = (uint32_t)token;
          nx.out[2 * nx.count + 1] = (uint32_t)t;
        }
        nx.count++;
        nx.token = token;
      }
      nx.t = nt, nx.symbols = symbols, nx.left = left, nx.decisions++;
      nx.done = done, nx.idle = idle;
      *a.nx = nx;
    }
    if (idle) return;
  }
  if constexpr (INIT) {  // the first frame's encoder row
    const float *e = a.st->enc;
    for (int j = blockIdx.x * 256 + tid; j < a.joint; j += gridDim.x * 256) a.erow[j] = e[j];
  }
  stage_rest(lds, run);
  // Layer 0's input [embedding row of the token | h]: the first predict has a zero input.
#pragma unroll
  for (int i = 0; i < 4; i++) xin[min(tid + 256 * i, n - 1)] = ev[i];
  __syncthreads();
  cell.finish(a, 0, run, lds, xin, a.h_new);
}

// LSTM layer l ≥ 1 over [layer l − 1's new h | its own h]; nothing while idle.
template <int WT>
__global__ __launch_bounds__(256) void tdt_layer_kernel(TdtArgs a, int layer) {
  extern __shared__ uint4 lds[];
  Cell<WT> cell;
  const Runs<4> run = Cell<WT>::runs(a, layer);
  StageRound<4> w0;
  w0.load(run, 0);
  cell.init(a, layer);
  const int n = a.n;
  float *xin = (float *)(lds + 4 * run.cpr);
  const float *x = a.h_new + (size_t)(layer - 1) * n, *h = a.h_old + (size_t)layer * n;
  float xv[8];
#pragma unroll
  for (int i = 0; i < 8; i++) {
    const int j = min((int)threadIdx.x + 256 * i, 2 * n - 1);  // clamped: no branch
    xv[i] = j < n ? x[j] : h[j - n];
  }
  const int idle = a.nx->idle;
  w0.store(lds, run, 0);
#pragma unroll
  for (int i = 0; i < 8; i++) xin[min((int)threadIdx.x + 256 * i, 2 * n - 1)] = xv[i];
  cell.pin_loads();
  if (idle) return;
  stage_rest(lds, run);
  __syncthreads();
  cell.finish(a, layer, run, lds, xin, a.h_new + (size_t)layer * n);
}

// One TDT decision, last part: after an emission the joint's predictor projection of the last layer's
// new h (Decoder::predict's pred, src/parakeet/decoder.rs:129-133), RW rows per wavefront, and the new
// h as the old; then the next decision's joint input z = ReLU(enc[t] + pred) from the encoder row the
// step kernel copied, and the next state becomes the current one.
template <int WT>
__global__ __launch_bounds__(256) void tdt_pred_kernel(TdtArgs a) {
  constexpr int RW = pred_rows_per_wave<WT>();
  extern __shared__ uint4 lds[];
  const TdtState *nx = a.nx;
  const int n = a.n, tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  // Everything this kernel reads goes out before the wait for the state: the weights, the new h,
  // and for this wavefront's rows the next encoder row and the current projection.
  const int g0 = blockIdx.x * 4 * RW, r0 = g0 + wave * RW, r = r0 + lane * RW / 64, rc = min(r, a.joint - 1);
  const Runs<1> run = one_run(a.pred_w, a.pred_rb, g0, min(4 * RW, a.joint - g0), pred_rows_cpr<WT>(a.pred_rb));
  StageRound<1> w0;
  w0.load(run, 0);
  Rows<WT, RW> rows;
  rows.init(a.pred_b, r0, a.joint, n);
  float *hin = (float *)(lds + run.cpr);
  const float *h = a.h_new + (size_t)(a.layers - 1) * n;
  float hv[4];
#pragma unroll
  for (int i = 0; i < 4; i++) hv[i] = h[min(tid + 256 * i, n - 1)];
  const float erow = a.erow[rc];
  float pv = a.pred[rc];
  const bool mine = lane % (64 / RW) == 0 && r < a.joint;
  const int idle = nx->idle;
  w0.store(lds, run, 0);
#pragma unroll
  for (int i = 0; i < 4; i++) hin[min(tid + 256 * i, n - 1)] = hv[i];
  pin(rows.b), pin(erow), pin(pv);
  if (!idle) {
    stage_rest(lds, run);
    __syncthreads();
    pv = rows.finish(run.at(lds, 0), g0, a.pred_rb, hin);
    if (mine) a.pred[r] = pv;
    for (int j = blockIdx.x * 256 + tid; j < a.layers * n; j += gridDim.x * 256) a.h_old[j] = a.h_new[j];
  }
  // The next decision's joint input (src/parakeet/decoder.rs:135-142).
  if (mine && !nx->done) a.z[r] = fmaxf(erow + pv, 0.0f);
  if (blockIdx.x == 0 && tid == 0) *a.st = *nx;
}

__global__ void tdt_init_kernel(TdtState *st, TdtState *nx, TdtState init) {
  if (threadIdx.x == 0) {
    *st = init;
    TdtState next = init;
    next.idle = 0;  // the first predict runs
    *nx = next;
  }
}

// Greedy CTC, step 1: the first maximum of each frame's first `classes` logits.
__global__ __launch_bounds__(256) void ctc_argmax_kernel(const float *__restrict__ logits, int width, int classes,
                                                         int *__restrict__ ids) {
  __shared__ float sv[4];
  __shared__ int si[4];
  float v;
  int i;
  wg_argmax(logits + (size_t)blockIdx.x * width, classes, sv, si, v, i);
  if (threadIdx.x == 0) ids[blockIdx.x] = i;
}

// Greedy CTC, step 2 (src/gigaam/decoder.rs:135-151): a frame's id is emitted when it is not blank and
// differs from the previous frame's; (token, frame) pairs in order, the count in out_count.  One
// workgroup: each thread flags its frames, a prefix sum over the flags places the pairs.
__global__ __launch_bounds__(256) void ctc_collapse_kernel(const int *__restrict__ ids, int frames, int blank,
                                                           uint32_t *__restrict__ out, int cap, int *__restrict__ count) {
  __shared__ int part[256];
  const int tid = threadIdx.x, per = (frames + 255) / 256, f0 = tid * per, f1 = min(f0 + per, frames);
  int n = 0;
  for (int f = f0; f < f1; f++) n += ids[f] != blank && (f == 0 || ids[f] != ids[f - 1]);
  part[tid] = n;
  __syncthreads();
  for (int o = 1; o < 256; o <<= 1) {  // inclusive prefix sum
    const int add = tid >= o ? part[tid - o] : 0;
    __syncthreads();
    part[tid] += add;
    __syncthreads();
  }
  int at = part[tid] - n;
  for (int f = f0; f < f1; f++)
    if (ids[f] != blank && (f == 0 || ids[f] != ids[f - 1])) {
      if (at < cap) out[2 * at] = (uint32_t)ids[f], out[2 * at + 1] = (uint32_t)f;
      at++;
    }
  if (tid == 255) *count = part[255];
}

}  // namespace

int launch_tdt_init(wh_ctx *ctx, TdtState *st, TdtState *nx, const TdtState &init) {
  wh_launch(ctx, tdt_init_kernel, 1, 64, 0, st, nx, init);
  return wh_launched(ctx, "tdt init");
}

template <int WT>
static int tdt_launch_t(wh_ctx *ctx, const TdtArgs &a, int what) {
  const int cells = (a.n + 3) / 4;
  const size_t cell_lds = 64 * (size_t)lstm_cpr(a.lstm_rb) + 8 * a.n;
  switch (what) {
    case TDT_JOINT: {
      ProfScope prof(ctx, "tdt_joint", 2.0 * a.out_rows * a.joint, (double)a.out_rb * a.out_rows + 8.0 * a.joint);
      wh_launch(ctx, tdt_joint_kernel<WT>, a.parts, 256, 16 * (size_t)rows_cpr<WT>(a.out_rb) + 4 * a.joint, a);
      return wh_launched(ctx, "tdt joint");
    }
    case TDT_STEP:
    case TDT_INIT: {
      ProfScope prof(ctx, what == TDT_INIT ? "tdt_init_step" : "tdt_step", 16.0 * a.n * a.n,
                     (double)a.lstm_rb * 4 * a.n + 16.0 * a.parts);
      if (what == TDT_INIT) wh_launch(ctx, tdt_step_kernel<WT, true>, cells, 256, cell_lds, a);
      else wh_launch(ctx, tdt_step_kernel<WT, false>, cells, 256, cell_lds, a);
      if (int rc = wh_launched(ctx, "tdt step")) return rc;
      for (int l = 1; l < a.layers; l++) {
        ProfScope pl(ctx, "tdt_layer", 16.0 * a.n * a.n, (double)a.lstm_rb * 4 * a.n);
        wh_launch(ctx, tdt_layer_kernel<WT>, cells, 256, cell_lds, a, l);
        if (int rc = wh_launched(ctx, "tdt layer")) return rc;
      }
      return WH_OK;
    }
    default: {
      ProfScope prof(ctx, "tdt_pred", 2.0 * a.joint * a.n, (double)a.pred_rb * a.joint);
      const int rows = 4 * pred_rows_per_wave<WT>();
      wh_launch(ctx, tdt_pred_kernel<WT>, (a.joint + rows - 1) / rows, 256, 16 * (size_t)pred_rows_cpr<WT>(a.pred_rb) + 4 * a.n, a);
      return wh_launched(ctx, "tdt pred");
    }
  }
}

int tdt_parts(int type, int out_rows) {
  const int rows = 4 * rows_per_wave<WH_Q8_0>();  // the same for every type
  return (out_rows + rows - 1) / rows;
}

int launch_tdt(wh_ctx *ctx, const TdtArgs &a, int what) {
  const TdtConfig &c = a.cfg;
  if (c.classes <= 0 || c.ndur <= 0 || c.ndur > 16 || c.blank < 0 || c.blank >= c.classes || c.max_symbols <= 0 ||
      a.n <= 0 || a.n % 16 || a.n > 1024 || a.joint <= 0 || a.joint % 16 || a.joint > 1024 || a.layers < 1 ||
      a.layers > 4 || a.parts != tdt_parts(a.type, a.out_rows) || a.parts > 1024 || a.out_rows != c.classes + c.ndur)
    return wh_fail(ctx, WH_EARG, "tdt: bad decoder configuration");
  // The products read the rows from LDS as whole dwords (quantized rows: k % 64 == 0); with k ≤ 1024
  // a workgroup's rows take at most 128 KiB of LDS (four F32 gate runs of four 8 KiB rows).
  if ((a.out_rb | a.pred_rb | a.lstm_rb) % 4)
    return wh_fail(ctx, WH_EARG, "tdt: rows of %zu / %zu / %zu bytes (the device decoder takes whole dwords)", a.out_rb,
                   a.pred_rb, a.lstm_rb);
  switch (a.type) {
    case WH_F32: return tdt_launch_t<WH_F32>(ctx, a, what);
    case WH_F16: return tdt_launch_t<WH_F16>(ctx, a, what);
    case WH_Q8_0: return tdt_launch_t<WH_Q8_0>(ctx, a, what);
    case WH_Q4_0: return tdt_launch_t<WH_Q4_0>(ctx, a, what);
  }
  return wh_fail(ctx, WH_EARG, "tdt: weight type %d", a.type);
}

int launch_ctc(wh_ctx *ctx, const float *logits, int frames, int width, int classes, int blank, int *ids,
               uint32_t *out, int cap, int *count) {
  if (frames <= 0 || classes <= 0 || classes > width || blank < 0 || blank >= classes)
    return wh_fail(ctx, WH_EARG, "ctc: bad arguments");
  {
    ProfScope prof(ctx, "ctc_argmax", 0.0, 4.0 * frames * classes);
    wh_launch(ctx, ctc_argmax_kernel, frames, 256, 0, logits, width, classes, ids);
    if (int rc = wh_launched(ctx, "ctc argmax")) return rc;
  }
  ProfScope prof(ctx, "ctc_collapse", 0.0, 4.0 * frames);
  wh_launch(ctx, ctc_collapse_kernel, 1, 256, 0, ids, frames, blank, out, cap, count);
  return wh_launched(ctx, "ctc collapse");
}

// ------------------------------------------------------------------------- Whisper's window search
// search::decode's pick (src/whisper/search.rs:46-127) on the device in two launches, then the loop's
// bookkeeping (src/whisper/search.rs:35-71): the picked id appended, the next step's token and
// position written where the recorded step reads them.
//
//   whisper_rules_kernel: 1024 ids per workgroup (a float4 of logits and a word of suppression bits
//     per thread).  The rules only set logits to −∞, so they apply per id: the suppression lists (a
//     per-id mask), then the timestamp rules as id ranges.  Each workgroup writes its partial: the
//     maxima of its timestamps, its text and its finite logits, the first maximum over all its ids
//     and over its timestamps, and the f64 sums of exp(v − its maximum) over its timestamps and
//     (with log-probabilities) over all its finite logits.
//   whisper_pick_kernel: one wave merges the partials (sums rescaled to the common maximum): the
//     timestamps' mass against the best text, the first maximum (over the timestamps when the mass
//     wins), its log-softmax, and the bookkeeping.
//
// The host sums exp(v − max) in id order against the global maximum; here each term is taken against
// its workgroup's maximum and the sums are rescaled, which changes only the rounding.

namespace {

constexpr int WR_THREADS = 256, WR_IDS = 4 * WR_THREADS, WP_PARTS = 64;  // vocabularies up to 65536 ids

__device__ __forceinline__ float lane4(const float4 &v, int e) { return e == 0 ? v.x : e == 1 ? v.y : e == 2 ? v.z : v.w; }

// (value, id) pairs: the greater value, the lower id among equals (the first maximum).
__device__ __forceinline__ bool first_max_better(float ov, int oi, float v, int i) { return ov > v || (ov == v && oi < i); }
__device__ __forceinline__ void first_max(float &v, int &i, float ov, int oi) {
  if (first_max_better(ov, oi, v, i)) v = ov, i = oi;
}

// The state's view of the rules: which ids die.
struct Rules {
  int ts_lo, ts_hi, text_floor, no_ts, begin;
  uint32_t mbits;
};

__device__ __forceinline__ Rules rules_of(const WhisperPickArgs &a, int n, int lts, int g1, int g2) {
  const int begin = a.begin, vocab = a.vocab;
  const bool last = n > 0 && g1 >= begin, pen = n < 2 || g2 >= begin, n0 = n == 0;
  Rules r;
  // A text id dies below text_floor (every text id before the first pick, the ids below EOT after a
  // lone timestamp); a timestamp outside [ts_lo, ts_hi): timestamps never decrease (ids below the last
  // one, or below it + 1 when it closed a pair), none after a pair, none past MAX_INITIAL first.
  r.ts_lo = lts < 0 ? begin : min(last && !pen ? lts : lts + 1, vocab);
  r.ts_hi = last && pen ? begin : n0 ? min(begin + a.max_initial + 1, vocab) : vocab;
  r.text_floor = n0 ? begin : last && !pen ? a.eot : 0;
  r.mbits = n0 ? 0x03030303u : 0x01010101u;  // suppressed; suppressed at the first pick
  r.no_ts = a.no_ts;
  r.begin = begin;
  return r;
}

template <int N>
__device__ __forceinline__ void block_max(float (&v)[N], float *red) {
#pragma unroll
  for (int t = 0; t < N; t++) v[t] = xlane::wave_max(v[t]);
  __syncthreads();
  if ((threadIdx.x & 63) == 0)
#pragma unroll
    for (int t = 0; t < N; t++) red[4 * t + (threadIdx.x >> 6)] = v[t];
  __syncthreads();
#pragma unroll
  for (int t = 0; t < N; t++) v[t] = fmaxf(fmaxf(red[4 * t], red[4 * t + 1]), fmaxf(red[4 * t + 2], red[4 * t + 3]));
}

__global__ __launch_bounds__(WR_THREADS) void whisper_rules_kernel(WhisperPickArgs a) {
  __shared__ float redf[4 * 4];
  __shared__ double redd[2 * 4];
  __shared__ float redv[2 * 4];
  __shared__ int redi[2 * 4];
  const int tid = threadIdx.x, vocab = a.vocab, quads = (vocab + 3) / 4;
  const int q = min((int)blockIdx.x * WR_THREADS + tid, quads - 1);  // clamped: ids past vocab die below
  const float4 lg = reinterpret_cast<const float4 *>(a.logits)[q];
  const uint32_t mk = reinterpret_cast<const uint32_t *>(a.mask)[q];
  const WhisperState *st = a.st;
  const int done = st->done, n = st->n, lts = st->last_ts, logprobs = st->logprobs;
  const int g1 = (int)a.gen[max(n - 1, 0)], g2 = (int)a.gen[max(n - 2, 0)];
  if (done) return;
  const Rules r = rules_of(a, n, lts, g1, g2);
  const int i0 = 4 * ((int)blockIdx.x * WR_THREADS + tid);
  float v[4];
  // mx: the maxima of the timestamps, the text and the finite logits.
  float mx[3] = {-INFINITY, -INFINITY, -INFINITY};
  float bv = -INFINITY, tv = -INFINITY;  // first maxima over all ids and over the timestamps
  int bi = i0, ti = INT_MAX;
  const uint32_t m = mk & r.mbits;
#pragma unroll
  for (int e = 0; e < 4; e++) {
    const int i = i0 + e;
    const bool ts = i >= r.begin;
    const bool kill = ((m >> (8 * e)) & 0xffu) != 0 || i == r.no_ts || i < r.text_floor || (ts && i < r.ts_lo) ||
                      i >= r.ts_hi || i >= vocab;
    v[e] = kill ? -INFINITY : lane4(lg, e);
    if (ts) mx[0] = fmaxf(mx[0], v[e]);
    else mx[1] = fmaxf(mx[1], v[e]);
    if (isfinite(v[e])) mx[2] = fmaxf(mx[2], v[e]);
    if (v[e] > bv) bv = v[e], bi = i;
    if (ts && i < vocab && (ti == INT_MAX || v[e] > tv)) tv = v[e], ti = i;
  }
  xlane::wave_first_max(bv, bi, first_max_better);
  xlane::wave_first_max(tv, ti, first_max_better);
  if ((tid & 63) == 0) redv[tid >> 6] = bv, redi[tid >> 6] = bi, redv[4 + (tid >> 6)] = tv, redi[4 + (tid >> 6)] = ti;
  block_max(mx, redf);
  // The sums against this workgroup's maxima.
  double s[2] = {0.0, 0.0};
#pragma unroll
  for (int e = 0; e < 4; e++) {
    if (i0 + e >= r.begin && isfinite(v[e])) s[0] += exp((double)(v[e] - mx[0]));
    if (logprobs && isfinite(v[e])) s[1] += exp((double)(v[e] - mx[2]));
  }
  s[0] = xlane::wave_sum(s[0]), s[1] = xlane::wave_sum(s[1]);
  if ((tid & 63) == 0) redd[tid >> 6] = s[0], redd[4 + (tid >> 6)] = s[1];
  __syncthreads();
  if (tid != 0) return;
  WhisperPart p;
  p.s_ts = redd[0] + redd[1] + redd[2] + redd[3];
  p.s_all = redd[4] + redd[5] + redd[6] + redd[7];
  p.tmax = mx[0], p.text = mx[1], p.fmax = mx[2];
  p.best_v = redv[0], p.best_i = redi[0], p.ts_v = redv[4], p.ts_i = redi[4];
  for (int w = 1; w < 4; w++) first_max(p.best_v, p.best_i, redv[w], redi[w]), first_max(p.ts_v, p.ts_i, redv[4 + w], redi[4 + w]);
  a.part[blockIdx.x] = p;
}

__global__ __launch_bounds__(64) void whisper_pick_kernel(WhisperPickArgs a, int parts) {
  const int lane = threadIdx.x;
  WhisperState *st = a.st;
  const WhisperPart p = a.part[min(lane, parts - 1)];
  if (st->done) return;
  const bool mine = lane < parts;
  // The common maxima, then the sums rescaled to them.
  float tmax = mine ? p.tmax : -INFINITY, text = mine ? p.text : -INFINITY, fmx = mine ? p.fmax : -INFINITY;
  tmax = xlane::wave_max(tmax), text = xlane::wave_max(text), fmx = xlane::wave_max(fmx);
  double s_ts = mine && isfinite(p.tmax) ? p.s_ts * exp((double)p.tmax - (double)tmax) : 0.0;
  double s_all = mine && isfinite(p.fmax) ? p.s_all * exp((double)p.fmax - (double)fmx) : 0.0;
  float bv = mine ? p.best_v : -INFINITY, tv = mine ? p.ts_v : -INFINITY;
  int bi = mine ? p.best_i : INT_MAX, ti = mine ? p.ts_i : INT_MAX;
  s_ts = xlane::wave_sum(s_ts), s_all = xlane::wave_sum(s_all);
  xlane::wave_first_max(bv, bi, first_max_better);
  xlane::wave_first_max(tv, ti, first_max_better);
  if (lane != 0) return;
  // The timestamps' total probability against the best text token (src/whisper/search.rs:99-110);
  // when it wins, the text dies and the first maximum is over the timestamps.
  float mass = -INFINITY;
  if (isfinite(tmax) && s_ts > 0.0) mass = tmax + (float)log(s_ts);
  const bool no_text = mass > text;
  const int best = no_text ? ti : bi;
  const float best_v = no_text ? tv : bv;
  float lp = 0.0f;
  if (st->logprobs) lp = no_text ? best_v - (tmax + (float)log(s_ts)) : best_v - (fmx + (float)log(s_all));
  // The loop (src/whisper/search.rs:35-71): every pick counts; the id is kept unless it is EOT or the
  // window's new-token budget is spent, and a step follows unless the context is full.
  const int n = st->n, pos = st->pos;
  st->picks++;
  st->sum += (double)lp;
  if (pos >= st->np + st->max_new || best == a.eot) {
    st->done = 1;
    return;
  }
  a.gen[n] = (uint32_t)best;
  st->n = n + 1;
  if (best >= a.begin) st->last_ts = best;
  if (pos + 1 > st->limit) {
    st->done = 1;
    return;
  }
  a.ids[0] = (uint32_t)best;
  a.ids[1] = (uint32_t)pos;
  st->pos = pos + 1;
}

}  // namespace

__global__ void whisper_init_kernel(WhisperState *st, WhisperState init) {
  if (threadIdx.x == 0) *st = init;
}

int launch_whisper_init(wh_ctx *ctx, WhisperState *st, const WhisperState &init) {
  wh_launch(ctx, whisper_init_kernel, 1, 64, 0, st, init);
  return wh_launched(ctx, "whisper init");
}

int launch_whisper_pick(wh_ctx *ctx, const WhisperPickArgs &a) {
  // The logits and the mask are read in whole quads of ids (both buffers are padded to them).
  const int parts = (a.vocab + WR_IDS - 1) / WR_IDS;
  if (a.vocab <= 0 || parts > WP_PARTS || a.begin <= 0 || a.begin > a.vocab || a.eot < 0 || a.eot >= a.vocab ||
      ((uintptr_t)a.logits | (uintptr_t)a.mask) % 16 || !a.part)
    return wh_fail(ctx, WH_EARG, "whisper pick: bad ids, vocabulary above %d or unaligned buffers", WP_PARTS * WR_IDS);
  {
    ProfScope prof(ctx, "whisper_rules", 0.0, 5.0 * a.vocab);
    wh_launch(ctx, whisper_rules_kernel, parts, WR_THREADS, 0, a);
    if (int rc = wh_launched(ctx, "whisper rules")) return rc;
  }
  ProfScope prof(ctx, "whisper_pick", 0.0, (double)sizeof(WhisperPart) * parts);
  wh_launch(ctx, whisper_pick_kernel, 1, 64, 0, a, parts);
  return wh_launched(ctx, "whisper pick");
}
