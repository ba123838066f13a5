// Flash attention of Pass::attention (src/gpu/mod.rs:1559-1601) on gfx950 matrix cores: plain
// (GigaAM's rotary layout, Whisper's [q | k | v]) and Transformer-XL relative positions (Parakeet's
// [q + u | k | v | q + v] with the projected positions), with an optional key mask for padded
// windows.  softmax_j(s·q_i·k_j (+ s·(q+v)_i·P[j − i + t + 15]))·v_j with an online softmax over
// key blocks and the exact running maximum (as flash_f16.wgsl:8-9 requires).
//
// Arithmetic: the products run on v_mfma_f32_16x16x32_f16 with f16 operands and f32 accumulation,
// the precision of the reference's own f16 flash tier (src/gpu/flash_f16.wgsl, held to 1e-3 by
// src/gpu/mod.rs:2197-2198); the softmax is f32.
//
// Two kernels per call.  pack_kernel writes K ([key][dim]), Vᵀ ([dim][key]) and the position rows as
// f16 into the context's scratch, zero-padded to whole 32-key blocks and to a head dim of 32·NC, so
// that the flash kernel's loads are whole aligned blocks.  flash_kernel gives each wavefront 16
// queries and each workgroup 4 wavefronts (64 queries) that share the key blocks: two LDS stages of
// K and Vᵀ and a ring of 32-row position groups, filled by the LDS DMA of gfx950 one block ahead of
// the MFMAs, with one barrier per block; under 80 KiB of LDS, so that two workgroups share a CU.
//
// Layout in the flash kernel: a wavefront computes the transposed scores Sᵀ = K·Qᵀ and output
// Oᵀ = Vᵀ·Pᵀ, so a query's softmax state lives in one lane column (lane % 16) of every MFMA result.
// The relative term is a band GEMM Tᵀ[r][i] = P[r]·(q+v)_i over the 47 position rows a wavefront's
// 16×32 block needs (3 tiles of 16 rows), skewed through LDS: S_pos(i, j) = Tᵀ[j − i + 15][i].  The
// band of a key block starts 32 rows after the previous one's, so each stage brings one new 32-row
// group and a block reads the groups of its own stage and the two before.  K and position rows are
// stored in LDS with their 16-byte chunks permuted by an XOR of the row index (swz), so that the
// fragment reads of 16 rows × 4 lane groups are free of bank conflicts.
#include <algorithm>
#include <type_traits>

#include "internal.h"
#include "xlane.h"

namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int KB = 32;  // keys per block
constexpr int QW = 4;   // wavefronts (16 queries each) per workgroup
// Key blocks whose DMA runs ahead of the MFMAs (measured: two or three, at one workgroup per CU
// for their LDS, are slower than one at two per CU).
constexpr int PD = 1;
constexpr int TS = 20;  // floats per row of the band skew buffer: its writes and reads hit distinct banks

// Scratch layout of one call: the packed operands, each array 256-byte aligned.
struct Pack {
  int tk = 0;      // keys padded to whole blocks
  int dp = 0;      // head dims padded to the MFMA's k (32)
  int pfront = 0;  // position row r is stored at row r + pfront
  int prows = 0;   // stored position rows
  size_t kv = 0;   // halves of the K and of the Vᵀ array: batch·heads·tk·dp
  size_t p = 0;    // halves of the position array: heads·prows·dp
  size_t bytes() const { return 2 * ((kv * 2 + 255) / 256 * 256) + (p * 2 + 255) / 256 * 256; }
};

Pack pack_shape(int t, int heads, int hd, int batch, bool rel) {
  Pack s;
  s.tk = (t + KB - 1) / KB * KB;
  s.dp = hd <= 32 ? 32 : hd <= 64 ? 64 : 128;
  s.kv = (size_t)batch * heads * s.tk * s.dp;
  if (rel) {
    // The band of key block kb for queries q0.. starts at stored row t − q0 − 48 + pfront + 32·kb:
    // pfront ≥ 64 keeps it ≥ 0 (q0 ≤ t − 1), and (t + pfront + 16) % 32 == 0 with q0 % 64 == 0 puts
    // every band on a 32-row boundary.  The last block reads up to 96 + 32 rows past its start.
    s.pfront = 64 + (32 - (t + 80) % 32) % 32;
    s.prows = (s.tk + t + s.pfront + 128 + 31) / 32 * 32;
    s.p = (size_t)heads * s.prows * s.dp;
  }
  return s;
}

struct Args {
  const _Float16 *q, *qv;  // queries (q or q + u) and q + v rows, f16
  int qs;                  // their row stride in halves
  long bq;                 // batch stride in halves
  void *o;                 // output [t][heads·hd], f32 or f16 (o16)
  int os, o16;
  long bo;
  const _Float16 *kp, *vt, *pp;  // packed K, Vᵀ, positions
  int t, hd, heads;
  int tk, pfront, prows;
  float scale;
  const int *valid_dev;
  int valid;
  // Key split: nsplit > 1 workgroups share a query tile, each over its own run of key blocks, and
  // write unnormalized partial outputs po [split][batch][t][heads·hd] and (max, sum) pairs pml
  // [split][batch][heads][t] for combine_kernel.
  int nsplit;
  float *po, *pml;
};

__device__ __forceinline__ floatx4 mfma(half8 a, half8 b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// LDS byte address of a __shared__ object.
__device__ __forceinline__ uint32_t lds_addr(const void *p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void *)p;
}

// LDS DMA: each lane copies the 16 bytes at base + off to LDS byte lds + 16·lane; base and lds are
// wave-uniform.  The copy is counted by vmcnt.
__device__ __forceinline__ void dma16s(const void *base, uint32_t off, uint32_t lds) {
  asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(base), "{m0}"(lds) : "memory");
}
__device__ __forceinline__ void dma_wait() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// f(integral_constant<I>, kb0 + I) for I = S .. N − 1 while kb0 + I < nkb: a loop body unrolled with its
// position in the period known at compile time.
template <int S, int N, class F>
__device__ __forceinline__ void unrolled_blocks(F &f, int kb0, int nkb) {
  if constexpr (S < N) {
    if (kb0 + S < nkb) {
      f(std::integral_constant<int, S>{}, kb0 + S);
      unrolled_blocks<S + 1, N>(f, kb0, nkb);
    }
  }
}

// Chunk permutation of LDS rows of CH 16-byte chunks (rows of 256, 128 or 64 bytes): logical chunk x
// of row r is stored at chunk x ^ swz<CH>(r).  gfx950 serves a 16-byte LDS read of a wavefront in
// four passes of 16 lanes — the two half-waves, each split by a parity of lane bits 2-4 (measured:
// bank-conflict counters over lane → address tables) — so a pass holds 8 rows of one lane group and 8
// of the next.  The MFMA fragment reads here (lane 16g + i: row i of a 16-row tile, logical chunk
// 4c + g) then hit 16 distinct 4-bank groups in every pass with these masks (a rotation by the row,
// (x + r) % CH, gives each pass a two-way conflict).
template <int CH>
__device__ __forceinline__ int swz(int row) {
  return CH >= 16 ? row & 15 : CH == 8 ? row & 6 : (row >> 1) & 2;
}

// ---------------------------------------------------------------------------------- pack pass

// K rows [batch][head][tk][DP] and Vᵀ [batch][head][DP][tk] as f16, zeros past t and hd.  One
// workgroup per 32 keys of one head.  T = float or _Float16 input.
template <int DP, typename T>
__device__ __forceinline__ void pack_kv(const T *__restrict__ k, int ks, long kbs, const T *__restrict__ v, int vs,
                                        long vbs, int t, int heads, int hd, int tk, _Float16 *__restrict__ kp,
                                        _Float16 *__restrict__ vt, int j0, int head, int b) {
  __shared__ _Float16 tr[KB][DP + 2];
  const size_t off = ((size_t)b * heads + head) * tk * DP;
  for (int e = threadIdx.x; e < KB * DP / 4; e += 256) {
    const int key = e / (DP / 4), d = 4 * (e % (DP / 4)), j = j0 + key;
    half4 kx = {}, vx = {};
    if (j < t && d < hd) {
      const T *kr = k + kbs * b + (long)j * ks + head * hd + d, *vr = v + vbs * b + (long)j * vs + head * hd + d;
#pragma unroll
      for (int q = 0; q < 4; q++) kx[q] = (_Float16)kr[q], vx[q] = (_Float16)vr[q];
    }
    *(half4 *)(kp + off + (size_t)j * DP + d) = kx;
#pragma unroll
    for (int q = 0; q < 4; q++) tr[key][d + q] = vx[q];
  }
  __syncthreads();
  for (int e = threadIdx.x; e < DP * (KB / 8); e += 256) {
    const int d = e / (KB / 8), q = e % (KB / 8);
    half8 h;
#pragma unroll
    for (int i = 0; i < 8; i++) h[i] = tr[8 * q + i][d];
    *(half8 *)(vt + off + (size_t)d * tk + j0 + 8 * q) = h;
  }
}

// Position rows [head][prows][DP] as f16: stored row sr holds position row sr − pfront of the
// projected table (zeros outside 0 .. prow).  One workgroup per 32 stored rows of one head.
template <int DP, typename T>
__device__ __forceinline__ void pack_pos(const T *__restrict__ pos, int ps, int prow, int hd, int pfront, int prows,
                                         _Float16 *__restrict__ pp, int x, int head) {
  const size_t off = (size_t)head * prows * DP;
  for (int e = threadIdx.x; e < 32 * DP / 4; e += 256) {
    const int sr = x * 32 + e / (DP / 4), d = 4 * (e % (DP / 4)), r = sr - pfront;
    half4 x = {};
    if (r >= 0 && r < prow && d < hd) {
      const T *pr = pos + (long)r * ps + head * hd + d;
#pragma unroll
      for (int q = 0; q < 4; q++) x[q] = (_Float16)pr[q];
    }
    *(half4 *)(pp + off + (size_t)sr * DP + d) = x;
  }
}

// Both packs in one launch: workgroups x < tk / KB pack K/Vᵀ (window z), the next prows / 32 (window
// 0 only) the position rows.
template <int DP, typename T>
__global__ __launch_bounds__(256) void pack_kernel(const T *__restrict__ k, int ks, long kbs, const T *__restrict__ v,
                                                   int vs, long vbs, int t, int heads, int hd, int tk,
                                                   _Float16 *__restrict__ kp, _Float16 *__restrict__ vt,
                                                   const T *__restrict__ pos, int ps, int prow, int pfront, int prows,
                                                   _Float16 *__restrict__ pp) {
  const int nkv = tk / KB;
  if ((int)blockIdx.x < nkv) pack_kv<DP, T>(k, ks, kbs, v, vs, vbs, t, heads, hd, tk, kp, vt, blockIdx.x * KB, blockIdx.y, blockIdx.z);
  else if (blockIdx.z == 0) pack_pos<DP, T>(pos, ps, prow, hd, pfront, prows, pp, blockIdx.x - nkv, blockIdx.y);
}

// ---------------------------------------------------------------------------------- flash kernel

template <int NC, bool REL, int PD>
__global__ __launch_bounds__(64 * QW) void flash_kernel(Args A) {
  constexpr int DP = NC * 32;          // head dims padded to the MFMA's k
  constexpr int CH = DP / 8;           // 16-byte chunks per K / position row (a power of 2)
  static_assert((CH & (CH - 1)) == 0, "chunk permutation masks");
  constexpr int OT = DP / 16;          // 16-dim output tiles
  constexpr int KBYTES = KB * DP * 2;  // one block's K, its Vᵀ, and one group of 32 position rows
  // A block's band spans NG position groups: its own and the NG − 1 before.  Rings: NKV K/V stages
  // (blocks kb .. kb + PD) and NP position groups (kb − NG + 1 .. kb + PD).
  constexpr int NG = REL ? QW / 2 + 1 : 0;
  constexpr int NKV = PD + 1, NP = REL ? NG + PD : 0;
  constexpr int P_RG = NKV * 2 * KBYTES;  // the position ring follows the K/V ring
  // DMA instructions (1 KiB each) per block and per wavefront (each issues the same count).
  constexpr int NI = (REL ? 3 : 2) * KBYTES / 1024, PER = (NI + QW - 1) / QW;
  static_assert(PER * PD < 64, "vmcnt range");
  __shared__ __attribute__((aligned(16))) uint8_t lds[P_RG + (REL ? NP * KBYTES : 0)];
  __shared__ float tt[REL ? QW * 48 * TS : 1];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int li = lane & 15, g = lane >> 4;
  // Work item of this workgroup.  Workgroups go to the 8 XCDs round-robin by linear id; the items
  // are renumbered so that each XCD takes a contiguous run of (window, head, query tile) — the
  // query tiles of one head — and its L2 holds that head's operands.
  // Items are ordered query tile fastest, then key split, head and window.
  const int nq = gridDim.x, ns = A.nsplit, total = nq * gridDim.y * gridDim.z;
  int w = blockIdx.x + nq * (blockIdx.y + gridDim.y * blockIdx.z);
  if (total % 8 == 0) w = (w % 8) * (total / 8) + w / 8;
  const int qt = w % nq, split = (w / nq) % ns, head = (w / (nq * ns)) % A.heads, b = w / (nq * ns * A.heads);
  const int t = A.t, hd = A.hd;
  const int kv_len = A.valid_dev ? min(A.valid_dev[b], t) : min(A.valid, t);
  const int nkb_all = (kv_len + KB - 1) / KB;
  // This workgroup's key blocks kb0 .. nkb − 1.
  const int kb0 = nkb_all * split / ns, nkb = nkb_all * (split + 1) / ns;
  const int q0 = qt * 16 * QW;      // the workgroup's first query
  const int qi = q0 + 16 * wave + li;  // this lane's query
  const int hoff = head * hd;
  const size_t kvoff = ((size_t)b * A.heads + head) * A.tk * DP;
  const _Float16 *kp = A.kp + kvoff, *vt = A.vt + kvoff;
  const _Float16 *pp = REL ? A.pp + (size_t)head * A.prows * DP : nullptr;
  // Stored position row where key block kb's band starts (a multiple of 32): the wave's band
  // starts 16·(QW − 1 − wave) rows into it, so stored row sb0 + 32kb + 16(QW−1−wave) + jj − ii + 15
  // is P[j − i + t + 15] (+ pfront) for key j = 32kb + jj and query i = q0 + 16·wave + ii.
  const int sb0 = A.t - q0 - 16 * (QW - 1) + A.pfront;

  // Per lane and DMA instruction: byte offset of its 16 bytes from the block's base and the
  // instruction's LDS offset in its stage or group.  A K/V stage is [K: 32 rows of CH chunks]
  // [Vᵀ: DP rows of 4 chunks], a group [positions: 32 rows of CH chunks]; K and position rows
  // permuted by swz<CH>, Vᵀ rows rotated by row / 4 (64-byte rows).
  uint32_t soff[PER], sdst[PER];
  int skind[PER];
#pragma unroll
  for (int i = 0; i < PER; i++) {
    const int n = (wave + QW * i) % NI, at = 1024 * n + 16 * lane;  // byte in the block's K|Vᵀ|positions
    if (at < KBYTES) {  // K row r, stored chunk position pc
      const int r = at / (DP * 2), pc = (at / 16) % CH, c = pc ^ swz<CH>(r);
      skind[i] = 0;
      soff[i] = (uint32_t)((r * DP + 8 * c) * 2);
      sdst[i] = 1024 * n;
    } else if (at < 2 * KBYTES) {  // Vᵀ row d (keys j0 .. j0 + 31)
      const int x = at - KBYTES, d = x / 64, pc = (x / 16) % 4, c = (pc - (d >> 2)) & 3;
      skind[i] = 1;
      soff[i] = (uint32_t)(((size_t)d * A.tk + 8 * c) * 2);
      sdst[i] = 1024 * n;
    } else {  // position row r of the group
      const int x = at - 2 * KBYTES, r = x / (DP * 2), pc = (x / 16) % CH, c = pc ^ swz<CH>(r);
      skind[i] = 2;
      soff[i] = (uint32_t)((r * DP + 8 * c) * 2);
      sdst[i] = 1024 * n - 2 * KBYTES;
    }
  }
  // Instructions are whole-kind: KBYTES is a multiple of 1 KiB, so a wave-uniform kind per i.
  const uint32_t lds0 = lds_addr(lds);
  // Block kb's K and Vᵀ into K/V slot kvs and its position group (rows sb0 + 32(kb + NG − 1) ..)
  // into group slot ps; pos_only: the group alone (the groups before the first block's).
  auto issue = [&](int kb, int kvs, int ps, bool pos_only) {
    const _Float16 *kb_k = kp + (size_t)kb * KB * DP, *kb_v = vt + (size_t)kb * KB;
    const _Float16 *kb_p = REL ? pp + (size_t)(sb0 + 32 * (kb + NG - 1)) * DP : nullptr;
#pragma unroll
    for (int i = 0; i < PER; i++) {
      const int kind = __builtin_amdgcn_readfirstlane(skind[i]);
      if (kind == 2) dma16s(kb_p, soff[i], lds0 + P_RG + ps * KBYTES + sdst[i]);
      else if (!pos_only) dma16s(kind == 0 ? kb_k : kb_v, soff[i], lds0 + kvs * 2 * KBYTES + sdst[i]);
    }
  };

  // The wave's queries (and (q + v) rows) as B fragments: lane (li, g) holds dims 32c + 8g ..+8.
  half8 qf[NC], wf[REL ? NC : 1];
  {
    const size_t row = (size_t)min(qi, t - 1) * A.qs;
    const _Float16 *qb = A.q + A.bq * b + hoff + row;
    const _Float16 *wb = REL ? A.qv + A.bq * b + hoff + row : nullptr;
#pragma unroll
    for (int c = 0; c < NC; c++) {
      const int d = 32 * c + 8 * g;
      if (qi < t && d + 8 <= hd) {  // rows and heads start on 16 bytes (hd % 4 == 0, aligned buffers)
        qf[c] = *(const half8 *)(qb + d);
        if constexpr (REL) wf[c] = *(const half8 *)(wb + d);
      } else {
#pragma unroll
        for (int e = 0; e < 8; e++) {
          const bool ok = qi < t && d + e < hd;
          qf[c][e] = ok ? qb[d + e] : (_Float16)0.0f;
          if constexpr (REL) wf[c][e] = ok ? wb[d + e] : (_Float16)0.0f;
        }
      }
    }
  }

  floatx4 om[OT];
#pragma unroll
  for (int i = 0; i < OT; i++) om[i] = floatx4{};
  // Softmax state in the log2 domain: scores s·scale·log2(e), running maximum m, row sum l.
  const float sc2 = A.scale * 1.44269504088896341f;
  float m = -INFINITY, l = 0.0f;
  float *tw = tt + wave * 48 * TS;

  if (nkb > kb0) {
    if constexpr (REL)
      for (int x = 0; x < NG - 1; x++) issue(kb0 - NG + 1 + x, 0, x, true);
#pragma unroll
    for (int x = 0; x < PD; x++)
      if (kb0 + x < nkb) issue(kb0 + x, x, NG - 1 + x, false);
  }
  // Block kb's K/V slot and its band's first group slot repeat with period PERIOD: the loop is
  // unrolled by it, so that every slot offset is a compile-time constant (no per-block address
  // arithmetic).
  constexpr int PERIOD = REL ? (NP % NKV == 0 ? NP : NKV * NP) : NKV;
  auto block = [&](auto I_c, int kb) {
    constexpr int kvs = decltype(I_c)::value % NKV, ps0 = REL ? decltype(I_c)::value % (REL ? NP : 1) : 0;
    // Block kb has landed (blocks after it may still be in flight); every wave is done with kb − 1,
    // whose K/V slot and first band group take block kb + PD.
    if (kb + PD - 1 < nkb) wait_vm<(PD - 1) * PER>();
    else dma_wait();
    __syncthreads();
    if (kb + PD < nkb) issue(kb + PD, kvs == 0 ? NKV - 1 : kvs - 1, REL ? (ps0 == 0 ? NP - 1 : ps0 - 1) : 0, false);
    const int j0 = kb * KB;
    const _Float16 *kt = (const _Float16 *)(lds + kvs * 2 * KBYTES);
    const _Float16 *vtl = kt + KB * DP;
    // The block's Vᵀ fragments are read now, ahead of the scores: their LDS latency overlaps the
    // QKᵀ and band MFMAs instead of the PV ones (the band's wave fence would keep them after it).
    // A Vᵀ row (one dim) has 4 chunks of 8 keys, rotated by row / 4; the lane's 8 k-slots are keys
    // 4g + v and 16 + 4g + v, as its P values.
    half8 vf[OT];
#pragma unroll
    for (int ot = 0; ot < OT; ot++) {
      const int row = 16 * ot + li, rr = row >> 2;
      const _Float16 *vr = vtl + row * KB;
      const half4 a0 = *(const half4 *)(vr + 8 * (((g >> 1) + rr) & 3) + 4 * (g & 1));
      const half4 a1 = *(const half4 *)(vr + 8 * ((2 + (g >> 1) + rr) & 3) + 4 * (g & 1));
      vf[ot] = half8{a0[0], a0[1], a0[2], a0[3], a1[0], a1[1], a1[2], a1[3]};
    }

    // Scores Sᵀ for the two 16-key tiles: lane holds keys 16·jt + 4g + v of query li.
    float s[2][4];
#pragma unroll
    for (int jt = 0; jt < 2; jt++) {
      floatx4 acc = floatx4{};
      const int row = 16 * jt + li;
#pragma unroll
      for (int c = 0; c < NC; c++) {
        const half8 a = *(const half8 *)(kt + row * DP + 8 * ((4 * c + g) ^ swz<CH>(row)));
        acc = mfma(a, qf[c], acc);
      }
#pragma unroll
      for (int v = 0; v < 4; v++) s[jt][v] = acc[v];
    }

    if constexpr (REL) {
      // Band Tᵀ[r][i] = P[band row r]·(q+v)_i, r in 0..47 (r = jj − ii + 15): rows base + r of the
      // block's band, whose 32-row groups are ring slots ps0 .. ps0 + NG − 1.
      const int base = 16 * (QW - 1 - wave);
#pragma unroll
      for (int rt = 0; rt < 3; rt++) {
        floatx4 acc = floatx4{};
        const int br0 = base + 16 * rt, grp = br0 >> 5;  // a 16-row tile lies in one group
        const int slot = ps0 + grp >= NP ? ps0 + grp - NP : ps0 + grp;
        const int gr = (br0 & 31) + li;
        const _Float16 *prow = (const _Float16 *)(lds + P_RG + slot * KBYTES) + gr * DP;
#pragma unroll
        for (int c = 0; c < NC; c++) {
          const half8 a = *(const half8 *)(prow + 8 * ((4 * c + g) ^ swz<CH>(gr)));
          acc = mfma(a, wf[c], acc);
        }
#pragma unroll
        for (int v = 0; v < 4; v++) tw[(16 * rt + 4 * g + v) * TS + li] = acc[v];
      }
      // tw is the wave's own: its LDS writes complete before its reads, in order.
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
      for (int jt = 0; jt < 2; jt++)
#pragma unroll
        for (int v = 0; v < 4; v++) s[jt][v] += tw[(16 * jt + 4 * g + v - li + 15) * TS + li];
      __builtin_amdgcn_wave_barrier();
    }

    // Online softmax over this block (per query li: 8 scores per lane, 4 lanes); keys past kv_len
    // only in a window's last block.
    if (j0 + KB <= kv_len) {
#pragma unroll
      for (int jt = 0; jt < 2; jt++)
#pragma unroll
        for (int v = 0; v < 4; v++) s[jt][v] *= sc2;
    } else {
#pragma unroll
      for (int jt = 0; jt < 2; jt++)
#pragma unroll
        for (int v = 0; v < 4; v++) s[jt][v] = j0 + 16 * jt + 4 * g + v < kv_len ? s[jt][v] * sc2 : -INFINITY;
    }
    float bm = fmaxf(fmaxf(fmaxf(s[0][0], s[0][1]), fmaxf(s[0][2], s[0][3])),
                     fmaxf(fmaxf(s[1][0], s[1][1]), fmaxf(s[1][2], s[1][3])));
    bm = xlane::bit5(xlane::bit4(bm, xlane::Max{}), xlane::Max{});  // the query's 4 lanes (l ^ 16, l ^ 32)
    const float mn = fmaxf(m, bm);
    const float alpha = __builtin_amdgcn_exp2f(m - mn);
    m = mn;
    half8 pf;
    float ps = 0.0f;
#pragma unroll
    for (int jt = 0; jt < 2; jt++)
#pragma unroll
      for (int v = 0; v < 4; v++) {
        const float p = __builtin_amdgcn_exp2f(s[jt][v] - mn);
        ps += p;
        pf[4 * jt + v] = (_Float16)p;
      }
    l = l * alpha + ps;

    // Oᵀ += Vᵀ·Pᵀ, the accumulators first rescaled when some query's maximum rose (α = 1 for the
    // others: the same values; after the first blocks the maximum seldom moves).
    if (__builtin_amdgcn_ballot_w64(alpha != 1.0f)) {
#pragma unroll
      for (int ot = 0; ot < OT; ot++) om[ot] *= alpha;
    }
#pragma unroll
    for (int ot = 0; ot < OT; ot++) om[ot] = mfma(vf[ot], pf, om[ot]);
  };
  for (int kb = kb0; kb < nkb; kb += PERIOD) unrolled_blocks<0, PERIOD>(block, kb, nkb);

  // The row sums over the 4 lanes of each query, then Oᵀ tile ot holds dims 16·ot + 4g + v.
  l = xlane::bit5(xlane::bit4(l, xlane::Add{}), xlane::Add{});
  if (qi >= t) return;
  if (ns > 1) {  // partial output: unnormalized O, and (m, l) of this key run (m in natural-log units)
    const int batch = gridDim.z / ns;
    const size_t prow = (((size_t)split * batch + b) * t + qi) * (size_t)A.heads * hd + hoff;
#pragma unroll
    for (int ot = 0; ot < OT; ot++) {
      const int d = 16 * ot + 4 * g;
      if (d >= hd) break;
      *(float4 *)(A.po + prow + d) = make_float4(om[ot][0], om[ot][1], om[ot][2], om[ot][3]);
    }
    if (g == 0) {
      float *ml = A.pml + 2 * ((((size_t)split * batch + b) * A.heads + head) * t + qi);
      ml[0] = m * 0.69314718055994531f, ml[1] = l;
    }
    return;
  }
  const float inv = l > 0.0f ? 1.0f / l : 0.0f;  // a window with no valid key outputs zeros
  const size_t obase = A.bo * b + (size_t)qi * A.os + hoff;
#pragma unroll
  for (int ot = 0; ot < OT; ot++) {
    const int d = 16 * ot + 4 * g;
    if (d >= hd) break;
    const float4 r = make_float4(om[ot][0] * inv, om[ot][1] * inv, om[ot][2] * inv, om[ot][3] * inv);
    // hd % 4 == 0: a quad is inside or past the head
    if (A.o16) *(half4 *)((_Float16 *)A.o + obase + d) = half4{(_Float16)r.x, (_Float16)r.y, (_Float16)r.z, (_Float16)r.w};
    else *(float4 *)((float *)A.o + obase + d) = r;
  }
}

// Key-split combine: o = Σ_s e^(m_s − M)·Õ_s / Σ_s e^(m_s − M)·l_s over the splits' unnormalized
// outputs Õ_s and (max, sum) pairs, M = max_s m_s; zeros where no split saw a valid key.  One thread
// per 4 dims.
__global__ __launch_bounds__(256) void combine_kernel(const float *__restrict__ po, const float *__restrict__ pml, int ns,
                                                      int batch, int t, int heads, int hd, void *__restrict__ o, int os,
                                                      long bo, int o16) {
  const int q4 = hd / 4;
  // With (window, head) pairs a multiple of 8, the flash kernel ran pair run x of 8 on XCD x (its
  // items in contiguous runs per XCD, the query tiles and key splits of a pair together); workgroup
  // g runs on XCD g % 8, so it takes that XCD's pairs, where their partial outputs were written.
  const int pairs = batch * heads;
  const bool runs = pairs % 8 == 0 && gridDim.x % 8 == 0;
  const int per = runs ? pairs / 8 : pairs, x = runs ? blockIdx.x % 8 : 0;
  const size_t n = (size_t)per * t * q4, first = runs ? blockIdx.x / 8 : blockIdx.x,
               stride = runs ? gridDim.x / 8 : gridDim.x;
  for (size_t e = first * 256 + threadIdx.x; e < n; e += stride * 256) {
    const int d = 4 * (int)(e % q4);
    const size_t r = e / q4;
    int head, i, b;
    if (runs) {  // the run's pairs one after another, query rows in order inside a pair
      const int pr = x * per + (int)(r / t);
      i = (int)(r % t), head = pr % heads, b = pr / heads;
    } else {
      head = (int)(r % heads), i = (int)((r / heads) % t), b = (int)(r / ((size_t)heads * t));
    }
    // Splits in groups of four, each group's loads in flight at once; a running maximum rescales
    // the sums when a later group raises it (one group: the plain two-pass merge, same order).
    float mx = -INFINITY, den = 0.0f;
    float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    for (int s0 = 0; s0 < ns; s0 += 4) {
      float2 ml[4];
      float4 x[4];
#pragma unroll
      for (int q = 0; q < 4; q++)
        if (s0 + q < ns) {
          const size_t sp = s0 + q;
          ml[q] = *(const float2 *)(pml + 2 * (((sp * batch + b) * heads + head) * t + i));
          x[q] = *(const float4 *)(po + ((sp * batch + b) * t + i) * (size_t)heads * hd + head * hd + d);
        }
      float cm = mx;
#pragma unroll
      for (int q = 0; q < 4; q++)
        if (s0 + q < ns) cm = fmaxf(cm, ml[q].x);
      if (cm == -INFINITY) continue;  // no split so far saw a valid key
      const float rs = __expf(mx - cm);
      den *= rs, acc.x *= rs, acc.y *= rs, acc.z *= rs, acc.w *= rs;
#pragma unroll
      for (int q = 0; q < 4; q++)
        if (s0 + q < ns) {
          const float w = __expf(ml[q].x - cm);
          den += w * ml[q].y;
          acc.x += w * x[q].x, acc.y += w * x[q].y, acc.z += w * x[q].z, acc.w += w * x[q].w;
        }
      mx = cm;
    }
    const float inv = den > 0.0f ? 1.0f / den : 0.0f;
    const float4 y = make_float4(acc.x * inv, acc.y * inv, acc.z * inv, acc.w * inv);
    const size_t at = bo * b + (size_t)i * os + head * hd + d;
    if (o16) *(half4 *)((_Float16 *)o + at) = half4{(_Float16)y.x, (_Float16)y.y, (_Float16)y.z, (_Float16)y.w};
    else *(float4 *)((float *)o + at) = y;
  }
}

// LDS bytes of one flash workgroup (as flash_kernel declares them).
int flash_lds(int dp, bool rel, int pd) {
  const int kbytes = KB * dp * 2, ng = rel ? QW / 2 + 1 : 0;
  return (pd + 1) * 2 * kbytes + (rel ? (ng + pd) * kbytes + QW * 48 * TS * 4 : 4);
}


// Key splits per query tile: workgroups for every slot the CUs hold at once (LDS-bound: two per CU
// for 128-dim relative attention) while every split keeps ≥ 3 key blocks.
int kv_splits(const wh_ctx *ctx, int t, int heads, int hd, int batch, bool rel) {
  const int nkb = (t + KB - 1) / KB;
  if (ctx->attn_split > 0) return std::min(ctx->attn_split, std::max(nkb, 1));
  const int cus = ctx->cus > 0 ? ctx->cus : 256;
  const int dp = hd <= 32 ? 32 : hd <= 64 ? 64 : 128;
  const long slots = (long)cus * std::max(1, std::min(2, 160 * 1024 / flash_lds(dp, rel, PD)));
  const long items = (long)((t + 16 * QW - 1) / (16 * QW)) * heads * batch;
  int ns = 1;
  while (ns < 4 && items * ns * 2 <= slots && nkb / (2 * ns) >= 3) ns *= 2;
  return ns;
}

// Scratch bytes of the key-split partials (after the packed operands).
size_t split_bytes(int ns, int t, int heads, int hd, int batch) {
  return ns > 1 ? ((size_t)ns * batch * t * heads * hd * 4 + 255) / 256 * 256 + (size_t)ns * batch * heads * t * 8 : 0;
}

template <int DP, typename T>
void launch_pack(wh_ctx *ctx, const Pack &sp, const T *k, int ks, long kbs, const T *v, int vs, long vbs, const T *pos,
                 int ps, int t, int heads, int hd, int batch, _Float16 *kp, _Float16 *vt, _Float16 *pp) {
  const int gx = sp.tk / KB + (pos ? sp.prows / 32 : 0);
  wh_launch(ctx, pack_kernel<DP, T>, dim3(gx, heads, batch), 256, 0, k, ks, kbs, v, vs, vbs, t, heads, hd, sp.tk, kp, vt,
                                                                       pos, ps, 2 * t + 15, sp.pfront, sp.prows, pp);
}

template <bool REL>
int launch_flash(wh_ctx *ctx, const Args &a, int heads, int batch, int dp) {
  // Algorithmic flops: 4·H·T²·hd (QKᵀ and PV), plus 2·H·T²·hd for the relative term, per window.
  const double tt = (double)a.t * a.t * heads * a.hd * batch;
  const double bytes = 2.0 * batch * a.t * heads * a.hd * (REL ? 6 : 4) + (a.o16 ? 2.0 : 4.0) * batch * a.t * heads * a.hd;
  ProfScope prof(ctx, REL ? "attention_rel" : "attention", (REL ? 6.0 : 4.0) * tt, bytes);
  const dim3 grid((a.t + 16 * QW - 1) / (16 * QW), heads, batch * a.nsplit);
  switch (dp) {
    case 32: wh_launch(ctx, flash_kernel<1, REL, PD>, grid, 64 * QW, 0, a); break;
    case 64: wh_launch(ctx, flash_kernel<2, REL, PD>, grid, 64 * QW, 0, a); break;
    default: wh_launch(ctx, flash_kernel<4, REL, PD>, grid, 64 * QW, 0, a); break;
  }
  if (int rc = wh_launched(ctx, "attention")) return rc;
  if (a.nsplit > 1) {
    const size_t n = (size_t)batch * a.t * heads * (a.hd / 4);
    const int blocks = (int)std::min<size_t>((n + 255) / 256 + 7, 4096) / 8 * 8;  // whole runs of 8 (per XCD)
    ProfScope pc(ctx, "attention_combine", 0.0, 4.0 * a.nsplit * batch * a.t * heads * (a.hd + 2.0) +
                                                    (a.o16 ? 2.0 : 4.0) * batch * a.t * heads * a.hd);
    wh_launch(ctx, combine_kernel, blocks, 256, 0, a.po, a.pml, a.nsplit, batch, a.t, heads, a.hd, a.o, a.os, a.bo, a.o16);
    return wh_launched(ctx, "attention combine");
  }
  return WH_OK;
}

template <typename T>
int attention_t(wh_ctx *ctx, const T *qk, const T *v, const T *pos, int ps, void *o, int t, int heads, int hd,
                const int *valid_dev, int valid, int batch, int out16) {
  const int ch = heads * hd;
  Args a{};
  a.t = t;
  a.hd = hd;
  a.heads = heads;
  a.scale = 1.0f / sqrtf((float)hd);
  a.valid_dev = valid_dev;
  a.valid = valid < 0 || valid > t ? t : valid;
  a.o = o;
  a.o16 = out16 != 0;
  a.os = ch;
  a.bo = (long)t * ch;
  const T *k = qk + ch, *vv;
  const T *q = qk, *qv = nullptr;
  int qs, vs;
  if (v) {  // [t][q | k] and v [t][ch]
    qs = 2 * ch;
    vv = v;
    vs = ch;
  } else if (!pos) {  // [t][q | k | v]
    qs = 3 * ch;
    vv = qk + 2 * ch;
    vs = 3 * ch;
  } else {  // [t][q + u | k | v | q + v]
    qs = 4 * ch;
    vv = qk + 2 * ch;
    vs = 4 * ch;
    qv = qk + 3 * ch;
  }
  const long bq = (long)t * qs, bv = (long)t * vs;
  const Pack sp = pack_shape(t, heads, hd, batch, pos != nullptr);
  // Queries: f16 rows read by the flash kernel directly (f32 input: converted first, after the
  // packed arrays in scratch).
  const size_t qbytes = std::is_same<T, float>::value ? ((size_t)batch * t * qs * 2 + 255) / 256 * 256 : 0;
  a.nsplit = kv_splits(ctx, t, heads, hd, batch, pos != nullptr);
  uint8_t *ws = (uint8_t *)wh_scratch(ctx, sp.bytes() + qbytes + split_bytes(a.nsplit, t, heads, hd, batch));
  if (!ws) return WH_EOOM;
  if (a.nsplit > 1) {
    a.po = (float *)(ws + sp.bytes() + qbytes);
    a.pml = a.po + ((size_t)a.nsplit * batch * t * heads * hd + 63) / 64 * 64;
  }
  _Float16 *kp = (_Float16 *)ws, *vt = (_Float16 *)(ws + (sp.kv * 2 + 255) / 256 * 256);
  _Float16 *pp = (_Float16 *)(ws + 2 * ((sp.kv * 2 + 255) / 256 * 256));
  {
    ProfScope prof(ctx, "attention_pack", 0.0,
                   (sizeof(T) + 2.0) * batch * t * ch * 2 + (pos ? (sizeof(T) + 2.0) * (2 * t + 15) * ch : 0.0));
    switch (sp.dp) {
      case 32: launch_pack<32, T>(ctx, sp, k, qs, bq, vv, vs, bv, pos, ps, t, heads, hd, batch, kp, vt, pp); break;
      case 64: launch_pack<64, T>(ctx, sp, k, qs, bq, vv, vs, bv, pos, ps, t, heads, hd, batch, kp, vt, pp); break;
      default: launch_pack<128, T>(ctx, sp, k, qs, bq, vv, vs, bv, pos, ps, t, heads, hd, batch, kp, vt, pp); break;
    }
    if (int rc = wh_launched(ctx, "attention pack")) return rc;
  }
  if constexpr (std::is_same<T, float>::value) {
    _Float16 *q16 = (_Float16 *)(ws + sp.bytes());
    if (int rc = launch_to_half(ctx, qk, q16, (size_t)batch * t * qs)) return rc;
    a.q = q16;
    a.qv = qv ? q16 + 3 * ch : nullptr;
  } else {
    a.q = q;
    a.qv = qv;
  }
  a.qs = qs;
  a.bq = bq;
  a.kp = kp, a.vt = vt, a.pp = pp;
  a.tk = sp.tk, a.pfront = sp.pfront, a.prows = sp.prows;
  return pos ? launch_flash<true>(ctx, a, heads, batch, sp.dp) : launch_flash<false>(ctx, a, heads, batch, sp.dp);
}

}  // namespace

void attention_layout(int t, int heads, int hd, int rel, int *tk, int *pfront, int *prows) {
  const Pack sp = pack_shape(t, heads, hd, 1, rel != 0);
  *tk = sp.tk, *pfront = sp.pfront, *prows = sp.prows;
}

// Attention over one window whose operands the projections already wrote in the packed layout
// (launch_gemm_h_heads): K [head][tk][hd], Vᵀ [head][hd][tk] and, with relative positions, the
// position rows [head][prows][hd] from row pfront; queries (and q + v rows) read from `q` rows of
// qs halves.  No packing launch.  Head dims of 32, 64 or 128.
int launch_attention_packed(wh_ctx *ctx, const _Float16 *q, int qs, const _Float16 *qv, const _Float16 *kp,
                            const _Float16 *vt, const _Float16 *pp, void *o, int t, int heads, int hd, int out16) {
  if (t <= 0 || heads <= 0 || (hd != 32 && hd != 64 && hd != 128) || !q || !kp || !vt || !o || qs < heads * hd)
    return wh_fail(ctx, WH_EARG, "attention: bad packed call (t %d, heads %d, head_dim %d)", t, heads, hd);
  if ((uintptr_t)q % 16 || (qv && (uintptr_t)qv % 16) || (uintptr_t)kp % 16 || (uintptr_t)vt % 16 ||
      (pp && (uintptr_t)pp % 16) || (uintptr_t)o % 16 || qs % 8)
    return wh_fail(ctx, WH_EARG, "attention: buffers must be 16-byte aligned");
  const bool rel = pp != nullptr;
  if (rel != (qv != nullptr)) return wh_fail(ctx, WH_EARG, "attention: relative positions take q + v rows");
  const int ch = heads * hd;
  Args a{};
  a.t = t;
  a.hd = hd;
  a.heads = heads;
  a.scale = 1.0f / sqrtf((float)hd);
  a.valid = t;
  a.o = o;
  a.o16 = out16 != 0;
  a.os = ch;
  a.bo = (long)t * ch;
  a.q = q, a.qv = qv, a.qs = qs, a.bq = (long)t * qs;
  a.kp = kp, a.vt = vt, a.pp = pp;
  const Pack sp = pack_shape(t, heads, hd, 1, rel);
  a.tk = sp.tk, a.pfront = sp.pfront, a.prows = sp.prows;
  a.nsplit = kv_splits(ctx, t, heads, hd, 1, rel);
  if (a.nsplit > 1) {
    uint8_t *ws = (uint8_t *)wh_scratch(ctx, split_bytes(a.nsplit, t, heads, hd, 1));
    if (!ws) return WH_EOOM;
    a.po = (float *)ws;
    a.pml = a.po + ((size_t)a.nsplit * t * heads * hd + 63) / 64 * 64;
  }
  return rel ? launch_flash<true>(ctx, a, heads, 1, hd) : launch_flash<false>(ctx, a, heads, 1, hd);
}

size_t attention_scratch_bytes(const wh_ctx *ctx, int t, int heads, int hd, int batch, int rel) {
  return pack_shape(t, heads, hd, batch, rel != 0).bytes() +
         split_bytes(kv_splits(ctx, t, heads, hd, batch, rel != 0), t, heads, hd, batch);
}

int launch_attention(wh_ctx *ctx, const void *qk, const void *v, const void *pos, void *o, int t, int heads,
                     int hd, const int *valid_dev, int valid, int batch, int out16, int in16, int pos_stride) {
  if (t <= 0 || heads <= 0 || hd <= 0 || hd > 128 || hd % 4 || batch <= 0 || !qk || !o)
    return wh_fail(ctx, WH_EARG, "attention: bad shape (t %d, heads %d, head_dim %d)", t, heads, hd);
  if (v && pos) return wh_fail(ctx, WH_EARG, "attention: relative positions take [q+u | k | v | q+v] rows");
  const int vvalid = valid < 0 || valid > t ? t : valid;
  if (!valid_dev && vvalid == 0) return wh_fail(ctx, WH_EARG, "attention: no valid keys");
  if ((uintptr_t)qk % 16 || (v && (uintptr_t)v % 16) || (pos && (uintptr_t)pos % 16) || (uintptr_t)o % 16)
    return wh_fail(ctx, WH_EARG, "attention: buffers must be 16-byte aligned");
  const int ps = pos_stride > 0 ? pos_stride : heads * hd;
  if (pos && ps < heads * hd)
    return wh_fail(ctx, WH_EARG, "attention: position row stride %d below heads·hd %d", ps, heads * hd);
  if (in16)
    return attention_t<_Float16>(ctx, (const _Float16 *)qk, (const _Float16 *)v, (const _Float16 *)pos, ps, o, t,
                                 heads, hd, valid_dev, valid, batch, out16);
  return attention_t<float>(ctx, (const float *)qk, (const float *)v, (const float *)pos, ps, o, t, heads, hd,
                            valid_dev, valid, batch, out16);
}
