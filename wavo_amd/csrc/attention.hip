// Flash attention of Pass::attention (src/gpu/mod.rs:1559-1601) on gfx950 matrix cores: plain
// (GigaAM's rotary layout, Whisper's [q | k | v]) and Transformer-XL relative positions (Parakeet's
// [q + u | k | v | q + v] with the projected positions), with an optional key mask for padded
// windows.  softmax_j(s·q_i·k_j (+ s·(q+v)_i·P[j − i + t + 15]))·v_j with an online softmax over
// key blocks and the exact running maximum (as flash_f16.wgsl:8-9 requires).
//
// Arithmetic: every product runs on v_mfma_f32_16x16x32_f16 with each f32 operand split into a
// high half h = f16(x) and a low half l = f16((x − h)·2¹²): x·y ≈ h_x·h_y + 2⁻¹²(h_x·l_y + l_x·h_y),
// three MFMAs summed in f32, about 2⁻²¹ relative per product — close to the f32 attention of the
// reference's CPU backend (src/cpu/ops.rs:190-273) at a sixth of the cost of f32 MFMA.
//
// Two kernels per call.  attention_split writes K, V (transposed) and the position rows once as
// split f16 in the layouts the MFMAs read, zero-padded to whole 32-key blocks, into the context's
// scratch.  The flash kernel then streams them with the LDS DMA of gfx950 (global_load_lds_dwordx4:
// 64 lanes copy 16 bytes each straight into LDS), double-buffered: the next key block's K and V and
// the 32 new position rows of the band land while the MFMAs work on the current block, so the loop
// waits on memory once per block only if a block's math is shorter than the load latency.
//
// Layout in the flash kernel: a wavefront owns 16 queries and computes the transposed scores
// Sᵀ = K·Qᵀ and output Oᵀ = Vᵀ·Pᵀ, so a query's softmax state lives in one lane column (lane % 16) of
// every MFMA result.  The waves of a workgroup (2 or 4: 32 or 64 queries) share the staged key block.
// The relative term is a band GEMM Tᵀ[r][i] = P[r]·(q+v)_i over the 47 position rows a wave's 16×32
// block needs, read from a 128-row LDS ring that holds the workgroup's band (16·waves + 32 rows)
// and the next block's 32 rows, skewed through LDS: S_pos(i, j) = Tᵀ[j − i + 15][i].  LDS rows are
// stored with their 16-byte chunks rotated by the row index, so the 16 lanes that read one chunk
// column of 16 rows hit distinct banks.
#include "internal.h"

namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr float LO = 4096.0f;        // scale of the low halves
constexpr float LO_INV = 1.0f / 4096.0f;
constexpr int KB = 32;               // keys per block
constexpr int RING = 128;            // position rows held in LDS

// Scratch layout of one call: the split operands, each array 256-byte aligned.
struct Split {
  int tk = 0;      // keys padded to whole blocks
  int dp = 0;      // head dims padded to the MFMA's k (32)
  int pfront = 0;  // position row r is stored at row r + pfront
  int prows = 0;   // stored position rows
  size_t kv = 0;   // halves of each K/V array: batch·heads·tk·dp
  size_t p = 0;    // halves of each position array: heads·prows·dp
  size_t bytes() const { return 4 * ((kv * 2 + 255) / 256 * 256) + 2 * ((p * 2 + 255) / 256 * 256); }
};

Split split_shape(int t, int heads, int hd, int batch, bool rel) {
  Split s;
  s.tk = (t + KB - 1) / KB * KB;
  s.dp = (hd + 31) / 32 * 32;
  s.kv = (size_t)batch * heads * s.tk * s.dp;
  if (rel) {
    // The band of key block j0 for queries q0.. starts at stored row j0 − q0 − 16·QW + 16 + t +
    // pfront: pfront ≥ 64 keeps it ≥ 0, and (t + pfront + 16) % 32 == 0 puts every band and every
    // 32-row group of new rows on a 32-row boundary of the ring.
    s.pfront = 64 + (32 - (t + 80) % 32) % 32;
    s.prows = (s.tk + t + s.pfront + 16 + 31) / 32 * 32;
    s.p = (size_t)heads * s.prows * s.dp;
  }
  return s;
}

struct Args {
  const float *q, *qv;   // f32 queries (q or q + u) and q + v rows
  void *o;               // f32, or f16 with o16 (for the output projection, which rounds it)
  int o16;
  int qs, os;            // row strides in floats (q/qv, o)
  long bq, bo;           // batch strides in floats
  const _Float16 *kh, *kl, *vh, *vl, *ph, *pl;
  int t, hd, heads;
  int tk, pfront, prows;
  float scale;
  const int *valid_dev;
  int valid;
};

__device__ __forceinline__ void load8(const float *p, int n, float x[8]) {
  // Up to 8 consecutive floats, zeros past n.
#pragma unroll
  for (int e = 0; e < 8; e++) x[e] = e < n ? p[e] : 0.0f;
}

__device__ __forceinline__ void split8(const float x[8], half8 &hi, half8 &lo) {
#pragma unroll
  for (int e = 0; e < 8; e++) {
    _Float16 h = (_Float16)x[e];
    hi[e] = h;
    lo[e] = (_Float16)((x[e] - (float)h) * LO);
  }
}

__device__ __forceinline__ floatx4 mfma(half8 a, half8 b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// LDS byte address of a __shared__ object.
__device__ __forceinline__ uint32_t lds_addr(const void *p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)p;
}

// LDS DMA: each lane copies the 16 bytes at `src` to LDS byte lds + 16·lane.  `lds` is wave-uniform.
// The copy is counted by vmcnt; the caller waits with dma_wait() before the data is read.
__device__ __forceinline__ void dma16(const void *src, uint32_t lds) {
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(src), "{m0}"(__builtin_amdgcn_readfirstlane(lds))
               : "memory");
}

__device__ __forceinline__ void dma_wait() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// The DMA of a tile of ROWS rows of CH 16-byte chunks (global rows `stride` halves apart) into LDS
// rows of CH chunks, chunk c of LDS row r stored at position (c + r) % CH.  ROWS·CH/64 instructions
// of 64 chunks each, shared round-robin by the QW wavefronts; each lane's source offsets are the
// same for every tile of a call, so they are planned once.
template <int CH, int ROWS, int QW>
struct Dma {
  static constexpr int NI = ROWS * CH / 64;
  static constexpr int PER = (NI + QW - 1) / QW;
  static_assert(ROWS * CH % 64 == 0, "whole instructions");
  int off[PER];  // halves from the tile's first global row
  __device__ __forceinline__ void plan(int stride, int wave, int lane) {
#pragma unroll
    for (int i = 0; i < PER; i++) {
      const int n = wave + QW * i, s = 64 * n + lane, r = s / CH, pc = s % CH;
      const int lc = (pc - r % CH + CH) % CH;
      off[i] = n < NI ? r * stride + 8 * lc : 0;
    }
  }
  __device__ __forceinline__ void issue(const _Float16 *g, uint32_t lds, int wave) const {
#pragma unroll
    for (int i = 0; i < PER; i++) {
      const int n = wave + QW * i;
      if (n < NI) dma16(g + off[i], lds + 1024 * n);
    }
  }
};

// ---------------------------------------------------------------------------------- split pass

// K rows [batch][head][tk][dp] and V transposed [batch][head][dp][tk] as split f16, zeros past t
// and hd.  One workgroup per 32 keys of one head.
template <int DP>
__global__ __launch_bounds__(256) void split_kv_kernel(const float *__restrict__ k, int ks, long kbs,
                                                       const float *__restrict__ v, int vs, long vbs, int t,
                                                       int heads, int hd, int tk, _Float16 *__restrict__ kh,
                                                       _Float16 *__restrict__ kl, _Float16 *__restrict__ vh,
                                                       _Float16 *__restrict__ vl) {
  __shared__ float vt[KB][DP + 1];
  const int j0 = blockIdx.x * KB, head = blockIdx.y, b = blockIdx.z;
  const size_t off = ((size_t)b * heads + head) * tk * DP;
  for (int e = threadIdx.x; e < KB * DP / 4; e += 256) {
    const int key = e / (DP / 4), d = 4 * (e % (DP / 4)), j = j0 + key;
    float4 kx = make_float4(0, 0, 0, 0), vx = kx;
    if (j < t && d < hd) {
      kx = *(const float4 *)(k + kbs * b + (long)j * ks + head * hd + d);
      vx = *(const float4 *)(v + vbs * b + (long)j * vs + head * hd + d);
    }
    const float a[4] = {kx.x, kx.y, kx.z, kx.w};
    half4 h, l;
#pragma unroll
    for (int q = 0; q < 4; q++) {
      h[q] = (_Float16)a[q];
      l[q] = (_Float16)((a[q] - (float)h[q]) * LO);
    }
    *(half4 *)(kh + off + (size_t)j * DP + d) = h;
    *(half4 *)(kl + off + (size_t)j * DP + d) = l;
    vt[key][d] = vx.x, vt[key][d + 1] = vx.y, vt[key][d + 2] = vx.z, vt[key][d + 3] = vx.w;
  }
  __syncthreads();
  for (int e = threadIdx.x; e < DP * (KB / 8); e += 256) {
    const int d = e / (KB / 8), q = e % (KB / 8);
    half8 h, l;
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const float x = vt[8 * q + i][d];
      h[i] = (_Float16)x;
      l[i] = (_Float16)((x - (float)h[i]) * LO);
    }
    *(half8 *)(vh + off + (size_t)d * tk + j0 + 8 * q) = h;
    *(half8 *)(vl + off + (size_t)d * tk + j0 + 8 * q) = l;
  }
}

// Position rows [head][prows][dp] as split f16: stored row sr holds position row sr − pfront of the
// projected table (zeros outside 0 .. prow).  One workgroup per 32 stored rows of one head.
template <int DP>
__global__ __launch_bounds__(256) void split_pos_kernel(const float *__restrict__ pos, int ps, int prow, int hd,
                                                        int pfront, int prows, _Float16 *__restrict__ ph,
                                                        _Float16 *__restrict__ pl) {
  const int head = blockIdx.y;
  const size_t off = (size_t)head * prows * DP;
  for (int e = threadIdx.x; e < 32 * DP / 4; e += 256) {
    const int sr = blockIdx.x * 32 + e / (DP / 4), d = 4 * (e % (DP / 4)), r = sr - pfront;
    float4 x = make_float4(0, 0, 0, 0);
    if (r >= 0 && r < prow && d < hd) x = *(const float4 *)(pos + (long)r * ps + head * hd + d);
    const float a[4] = {x.x, x.y, x.z, x.w};
    half4 h, l;
#pragma unroll
    for (int q = 0; q < 4; q++) {
      h[q] = (_Float16)a[q];
      l[q] = (_Float16)((a[q] - (float)h[q]) * LO);
    }
    *(half4 *)(ph + off + (size_t)sr * DP + d) = h;
    *(half4 *)(pl + off + (size_t)sr * DP + d) = l;
  }
}

// ---------------------------------------------------------------------------------- flash kernel

template <int NC, bool REL, int QW>
__global__ __launch_bounds__(64 * QW) void flash_kernel(Args A) {
  static_assert(QW % 2 == 0, "bands sit on 32-row boundaries only for an even number of waves");
  constexpr int DP = NC * 32;          // head dims padded to the MFMA's k
  constexpr int CH = DP / 8;           // 16-byte chunks per K / position row
  constexpr int OT = NC * 2;           // 16-dim output tiles (upper bound)
  constexpr int PR = 16 * QW + 32;     // position rows of a key block's band
  static_assert(PR + 32 <= RING, "the ring holds the band and the next block's rows");
  __shared__ __attribute__((aligned(16))) _Float16 kbuf[2][2][KB * DP];   // [stage][hi, lo][key][dim]
  __shared__ __attribute__((aligned(16))) _Float16 vbuf[2][2][DP * KB];   // [stage][hi, lo][dim][key]
  __shared__ __attribute__((aligned(16))) _Float16 pring[REL ? 2 : 1][REL ? RING * DP : 8];
  __shared__ float tt[REL ? QW * 48 * 17 : 1];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int li = lane & 15, g = lane >> 4;
  // Work item of this workgroup.  Workgroups go to the 8 XCDs round-robin by linear id; the items
  // are renumbered so that each XCD takes a contiguous run of (window, head, query tile) — the
  // query tiles of one head — and its L2 holds that head's operands.
  int qt = blockIdx.x, head = blockIdx.y, b = blockIdx.z;
  {
    const int nq = gridDim.x, total = nq * gridDim.y * gridDim.z;
    if (total % 8 == 0) {
      const int lin = blockIdx.x + nq * (blockIdx.y + gridDim.y * blockIdx.z);
      const int w = (lin % 8) * (total / 8) + lin / 8;
      qt = w % nq;
      head = (w / nq) % gridDim.y;
      b = w / (nq * gridDim.y);
    }
  }
  const int t = A.t, hd = A.hd;
  const int kv_len = A.valid_dev ? min(A.valid_dev[b], t) : min(A.valid, t);
  const int nkb = (kv_len + KB - 1) / KB;
  const int q0 = qt * 16 * QW;           // the workgroup's first query
  const int qi0 = q0 + wave * 16;        // the wave's
  const int qi = qi0 + li;               // this lane's query
  const int hoff = head * hd;
  const size_t kvoff = ((size_t)b * A.heads + head) * A.tk * DP;
  const _Float16 *kh = A.kh + kvoff, *kl = A.kl + kvoff, *vh = A.vh + kvoff, *vl = A.vl + kvoff;
  const size_t poff = (size_t)head * A.prows * DP;
  // Stored position row where key block kb's band starts (a multiple of 32).
  const int rb0 = -q0 - 16 * QW + 16 + t + A.pfront;

  Dma<CH, KB, QW> dk;
  Dma<KB / 8, DP, QW> dv;
  Dma<CH, 32, QW> dp;
  dk.plan(DP, wave, lane);
  dv.plan(A.tk, wave, lane);
  if constexpr (REL) dp.plan(DP, wave, lane);
  auto stage_kv = [&](int kb, int st) {
    const size_t j0 = (size_t)kb * KB;
    dk.issue(kh + j0 * DP, lds_addr(kbuf[st][0]), wave);
    dk.issue(kl + j0 * DP, lds_addr(kbuf[st][1]), wave);
    dv.issue(vh + j0, lds_addr(vbuf[st][0]), wave);
    dv.issue(vl + j0, lds_addr(vbuf[st][1]), wave);
  };
  // 32 stored position rows from sr (a multiple of 32) into ring rows sr % RING .. (a 32-row group:
  // chunks rotated by the row within the group).
  auto stage_pos = [&](int sr) {
    const uint32_t at = (sr % RING) * DP * 2;
    dp.issue(A.ph + poff + (size_t)sr * DP, lds_addr(pring[0]) + at, wave);
    dp.issue(A.pl + poff + (size_t)sr * DP, lds_addr(pring[REL ? 1 : 0]) + at, wave);
  };

  if (nkb > 0) {
    stage_kv(0, 0);
    if constexpr (REL)
      for (int i = 0; i < PR / 32; i++) stage_pos(rb0 + 32 * i);
  }

  // The wave's queries (and (q + v) rows) as split fragments: lane (li, g) holds dims 32c + 8g..
  half8 qh[NC], ql[NC], wh[REL ? NC : 1], wl[REL ? NC : 1];
  const float *qb = A.q + A.bq * b + hoff;
#pragma unroll
  for (int c = 0; c < NC; c++) {
    float x[8];
    int d0 = 32 * c + 8 * g;
    load8(qb + (size_t)qi * A.qs + d0, qi < t ? min(8, hd - d0) : 0, x);
    split8(x, qh[c], ql[c]);
    if constexpr (REL) {
      load8(A.qv + A.bq * b + hoff + (size_t)qi * A.qs + d0, qi < t ? min(8, hd - d0) : 0, x);
      split8(x, wh[c], wl[c]);
    }
  }

  floatx4 om[OT], oc[OT];
#pragma unroll
  for (int i = 0; i < OT; i++) om[i] = oc[i] = floatx4{};
  float m = -INFINITY, l = 0.0f;
  float *tw = tt + wave * 48 * 17;
  dma_wait();
  __syncthreads();

  for (int kb = 0; kb < nkb; kb++) {
    const int st = kb & 1, j0 = kb * KB, rb = rb0 + j0;
    if (kb + 1 < nkb) {
      stage_kv(kb + 1, st ^ 1);
      if constexpr (REL) stage_pos(rb + PR);
    }
    const _Float16 *kt = kbuf[st][0], *ktl = kbuf[st][1], *vt = vbuf[st][0], *vtl = vbuf[st][1];

    // Scores Sᵀ for the two 16-key tiles: lane holds keys 16·jt + 4g + v of query li.
    float s[2][4];
#pragma unroll
    for (int jt = 0; jt < 2; jt++) {
      floatx4 am = floatx4{}, ac = floatx4{};
      const int row = 16 * jt + li;
#pragma unroll
      for (int c = 0; c < NC; c++) {
        const int off = row * DP + 8 * ((4 * c + g + row) % CH);
        half8 ah = *(const half8 *)(kt + off), al = *(const half8 *)(ktl + off);
        am = mfma(ah, qh[c], am);
        ac = mfma(ah, ql[c], ac);
        ac = mfma(al, qh[c], ac);
      }
#pragma unroll
      for (int v = 0; v < 4; v++) s[jt][v] = am[v] + ac[v] * LO_INV;
    }

    if constexpr (REL) {
      // Band Tᵀ[r][i] = P[rb + base + r]·(q+v)_i for the wave's queries, r in 0..47 (local r =
      // jj − ii + 15); the wave's rows start 16·(QW − 1 − wave) into the band.
      const int base = rb + 16 * (QW - 1 - wave);
#pragma unroll
      for (int rt = 0; rt < 3; rt++) {
        floatx4 am = floatx4{}, ac = floatx4{};
        const int slot = (base + 16 * rt + li) % RING;
#pragma unroll
        for (int c = 0; c < NC; c++) {
          const int off = slot * DP + 8 * ((4 * c + g + (slot & 31)) % CH);
          half8 ph = *(const half8 *)(pring[0] + off), pl = *(const half8 *)(pring[REL ? 1 : 0] + off);
          am = mfma(ph, wh[c], am);
          ac = mfma(ph, wl[c], ac);
          ac = mfma(pl, wh[c], ac);
        }
#pragma unroll
        for (int v = 0; v < 4; v++) tw[(16 * rt + 4 * g + v) * 17 + li] = am[v] + ac[v] * LO_INV;
      }
      // tw is the wave's own: its LDS writes complete before its reads, in order.
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
      for (int jt = 0; jt < 2; jt++)
#pragma unroll
        for (int v = 0; v < 4; v++) s[jt][v] += tw[(16 * jt + 4 * g + v - li + 15) * 17 + li];
    }

    // Online softmax over this block (per query li: 8 scores per lane, 4 lanes).
    float bm = -INFINITY;
#pragma unroll
    for (int jt = 0; jt < 2; jt++)
#pragma unroll
      for (int v = 0; v < 4; v++) {
        int j = j0 + 16 * jt + 4 * g + v;
        s[jt][v] = j < kv_len ? s[jt][v] * A.scale : -INFINITY;
        bm = fmaxf(bm, s[jt][v]);
      }
    bm = fmaxf(bm, __shfl_xor(bm, 16, 64));
    bm = fmaxf(bm, __shfl_xor(bm, 32, 64));
    const float mn = fmaxf(m, bm);
    const float alpha = __expf(m - mn);
    m = mn;
    half8 ph, pl;
    float ps = 0.0f;
#pragma unroll
    for (int jt = 0; jt < 2; jt++)
#pragma unroll
      for (int v = 0; v < 4; v++) {
        float p = __expf(s[jt][v] - mn);
        ps += p;
        _Float16 h = (_Float16)p;
        ph[4 * jt + v] = h;
        pl[4 * jt + v] = (_Float16)((p - (float)h) * LO);
      }
    l = l * alpha + ps;

    // Oᵀ += Vᵀ·Pᵀ: the lane's 8 k-slots are keys 4g + v and 16 + 4g + v, as its P values.  A Vᵀ row
    // (one dim) has 4 chunks of 8 keys, rotated by the row.
#pragma unroll
    for (int ot = 0; ot < OT; ot++) {
      if (16 * ot >= hd) break;
      om[ot] *= alpha;
      oc[ot] *= alpha;
      const int row = 16 * ot + li;
      const int o0 = row * KB + 8 * ((g / 2 + row) % 4) + 4 * (g & 1);
      const int o1 = row * KB + 8 * ((2 + g / 2 + row) % 4) + 4 * (g & 1);
      half4 a0 = *(const half4 *)(vt + o0), a1 = *(const half4 *)(vt + o1);
      half4 b0 = *(const half4 *)(vtl + o0), b1 = *(const half4 *)(vtl + o1);
      half8 vhh = {a0[0], a0[1], a0[2], a0[3], a1[0], a1[1], a1[2], a1[3]};
      half8 vll = {b0[0], b0[1], b0[2], b0[3], b1[0], b1[1], b1[2], b1[3]};
      om[ot] = mfma(vhh, ph, om[ot]);
      oc[ot] = mfma(vhh, pl, oc[ot]);
      oc[ot] = mfma(vll, ph, oc[ot]);
    }
    dma_wait();
    __syncthreads();
  }

  // The row sums over the 4 lanes of each query, then Oᵀ tile ot holds dims 16·ot + 4g + v.
  l += __shfl_xor(l, 16, 64);
  l += __shfl_xor(l, 32, 64);
  if (qi >= t) return;
  const float inv = l > 0.0f ? 1.0f / l : 0.0f;  // a window with no valid key outputs zeros
  const size_t obase = A.bo * b + (size_t)qi * A.os + hoff;
#pragma unroll
  for (int ot = 0; ot < OT; ot++) {
    const int d = 16 * ot + 4 * g;
    if (d >= hd) break;
    float4 r;
    r.x = (om[ot][0] + oc[ot][0] * LO_INV) * inv;
    r.y = (om[ot][1] + oc[ot][1] * LO_INV) * inv;
    r.z = (om[ot][2] + oc[ot][2] * LO_INV) * inv;
    r.w = (om[ot][3] + oc[ot][3] * LO_INV) * inv;
    // hd % 4 == 0: a quad is inside or past the head
    if (A.o16) *(half4 *)((_Float16 *)A.o + obase + d) = half4{(_Float16)r.x, (_Float16)r.y, (_Float16)r.z, (_Float16)r.w};
    else *(float4 *)((float *)A.o + obase + d) = r;
  }
}

template <int NC>
void launch_split(wh_ctx *ctx, const Split &sp, const float *k, int ks, long kbs, const float *v, int vs, long vbs,
                  const float *pos, int t, int heads, int hd, int batch, _Float16 *const arr[6]) {
  constexpr int DP = NC * 32;
  split_kv_kernel<DP><<<dim3(sp.tk / KB, heads, batch), 256, 0, ctx->stream>>>(k, ks, kbs, v, vs, vbs, t, heads, hd,
                                                                                 sp.tk, arr[0], arr[1], arr[2], arr[3]);
  if (pos)
    split_pos_kernel<DP><<<dim3(sp.prows / 32, heads), 256, 0, ctx->stream>>>(pos, heads * hd, 2 * t + 15, hd,
                                                                               sp.pfront, sp.prows, arr[4], arr[5]);
}

template <bool REL, int QW>
void launch_qw(wh_ctx *ctx, const Args &a, dim3 grid, int nc) {
  switch (nc) {
    case 1: flash_kernel<1, REL, QW><<<grid, 64 * QW, 0, ctx->stream>>>(a); break;
    case 2: flash_kernel<2, REL, QW><<<grid, 64 * QW, 0, ctx->stream>>>(a); break;
    case 3: flash_kernel<3, REL, QW><<<grid, 64 * QW, 0, ctx->stream>>>(a); break;
    default: flash_kernel<4, REL, QW><<<grid, 64 * QW, 0, ctx->stream>>>(a); break;
  }
}

template <bool REL>
int launch_nc(wh_ctx *ctx, const Args &a, int heads, int batch) {
  int nc = (a.hd + 31) / 32;
  // Algorithmic flops: 4·H·T²·hd (QKᵀ and PV), plus 2·H·T²·hd for the relative term, per window.
  double tt = (double)a.t * a.t * heads * a.hd * batch;
  double bytes = 4.0 * batch * a.t * heads * a.hd * (REL ? 5 : 4);
  // 64 queries per workgroup, or 32 when that leaves CUs without a workgroup (one fits per CU).
  const long wg64 = (long)((a.t + 63) / 64) * heads * batch;
  const bool narrow = wg64 < (ctx->cus > 0 ? ctx->cus : 256);
  ProfScope prof(ctx, REL ? (narrow ? "attention_rel_q32" : "attention_rel_q64") : (narrow ? "attention_q32" : "attention_q64"),
                 (REL ? 6.0 : 4.0) * tt, bytes);
  if (narrow) launch_qw<REL, 2>(ctx, a, dim3((a.t + 31) / 32, heads, batch), nc);
  else launch_qw<REL, 4>(ctx, a, dim3((a.t + 63) / 64, heads, batch), nc);
  return wh_launched(ctx, "attention");
}

}  // namespace

size_t attention_scratch_bytes(int t, int heads, int hd, int batch, int rel) {
  return split_shape(t, heads, hd, batch, rel != 0).bytes();
}

int launch_attention(wh_ctx *ctx, const float *qk, const float *v, const float *pos, void *o, int t, int heads,
                     int hd, const int *valid_dev, int valid, int batch, int out16) {
  if (t <= 0 || heads <= 0 || hd <= 0 || hd > 128 || hd % 4 || batch <= 0 || !qk || !o)
    return wh_fail(ctx, WH_EARG, "attention: bad shape (t %d, heads %d, head_dim %d)", t, heads, hd);
  if (v && pos) return wh_fail(ctx, WH_EARG, "attention: relative positions take [q+u | k | v | q+v] rows");
  const int ch = heads * hd;
  Args a{};
  a.t = t;
  a.hd = hd;
  a.heads = heads;
  a.scale = 1.0f / sqrtf((float)hd);
  a.valid_dev = valid_dev;
  a.valid = valid < 0 || valid > t ? t : valid;
  if (!valid_dev && a.valid == 0) return wh_fail(ctx, WH_EARG, "attention: no valid keys");
  a.o = o;
  a.o16 = out16 != 0;
  a.os = ch;
  a.bo = (long)t * ch;
  a.q = qk;
  const float *k = qk + ch, *vv;
  int vs;
  if (v) {  // [t][q | k] and v [t][ch]
    a.qs = 2 * ch;
    vv = v;
    vs = ch;
  } else if (!pos) {  // [t][q | k | v]
    a.qs = 3 * ch;
    vv = qk + 2 * ch;
    vs = 3 * ch;
  } else {  // [t][q + u | k | v | q + v]
    a.qs = 4 * ch;
    vv = qk + 2 * ch;
    vs = 4 * ch;
    a.qv = qk + 3 * ch;
  }
  a.bq = (long)t * a.qs;
  const long bv = (long)t * vs;
  if ((uintptr_t)qk % 16 || (v && (uintptr_t)v % 16) || (pos && (uintptr_t)pos % 16) || (uintptr_t)o % 16)
    return wh_fail(ctx, WH_EARG, "attention: buffers must be 16-byte aligned");

  const Split sp = split_shape(t, heads, hd, batch, pos != nullptr);
  uint8_t *ws = (uint8_t *)wh_scratch(ctx, sp.bytes());
  if (!ws) return WH_EOOM;
  _Float16 *arr[6];
  size_t at = 0;
  for (int i = 0; i < 6; i++) {
    arr[i] = (_Float16 *)(ws + at);
    at += ((i < 4 ? sp.kv : sp.p) * 2 + 255) / 256 * 256;
  }
  a.kh = arr[0], a.kl = arr[1], a.vh = arr[2], a.vl = arr[3], a.ph = arr[4], a.pl = arr[5];
  a.tk = sp.tk, a.pfront = sp.pfront, a.prows = sp.prows;
  {
    ProfScope prof(ctx, "attention_split", 0.0, 4.0 * batch * t * ch * 2 * 2 + (pos ? 4.0 * (2 * t + 15) * ch * 2 : 0.0));
    switch ((hd + 31) / 32) {
      case 1: launch_split<1>(ctx, sp, k, a.qs, a.bq, vv, vs, bv, pos, t, heads, hd, batch, arr); break;
      case 2: launch_split<2>(ctx, sp, k, a.qs, a.bq, vv, vs, bv, pos, t, heads, hd, batch, arr); break;
      case 3: launch_split<3>(ctx, sp, k, a.qs, a.bq, vv, vs, bv, pos, t, heads, hd, batch, arr); break;
      default: launch_split<4>(ctx, sp, k, a.qs, a.bq, vv, vs, bv, pos, t, heads, hd, batch, arr); break;
    }
    int rc = wh_launched(ctx, "attention split");
    if (rc) return rc;
  }
  return pos ? launch_nc<true>(ctx, a, heads, batch) : launch_nc<false>(ctx, a, heads, batch);
}
