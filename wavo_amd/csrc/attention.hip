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
// Layout: a wavefront owns 16 queries and computes the transposed scores Sᵀ = K·Qᵀ and output
// Oᵀ = Vᵀ·Pᵀ, so a query's softmax state lives in one lane column (lane % 16) of every MFMA
// result.  The waves of a workgroup (4 or 2: 64 or 32 queries) share key blocks of 32 staged in
// LDS (K as [key][dim], V transposed as [dim][key], both split).  The relative term is a band GEMM
// Tᵀ[r][i] = P[r]·(q+v)_i over the 47 position rows a wave's 16×32 block needs, out of the band of
// 16·waves + 32 rows the workgroup stages in LDS, skewed through LDS: S_pos(i, j) = Tᵀ[j − i + 15][i].
#include "internal.h"

namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr float LO = 4096.0f;        // scale of the low halves
constexpr float LO_INV = 1.0f / 4096.0f;
constexpr int KB = 32;               // keys per LDS stage
constexpr int KPAD = 8;              // halves of padding per K row
constexpr int VROW = KB + 8;         // halves per transposed-V row

struct Args {
  const float *q, *k, *v, *qv, *pos;
  float *o;
  int qs, vs, os;        // row strides in floats (q/k/qv, v, o)
  long bq, bv, bo;       // batch strides in floats
  int t, hd;
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

template <int NC, bool REL, int QW>
__global__ __launch_bounds__(64 * QW) void flash_kernel(Args A) {
  constexpr int NT = 64 * QW;          // threads
  constexpr int DP = NC * 32;          // head dims padded to the MFMA's k
  constexpr int KROW = DP + KPAD;      // halves per K / P row in LDS
  constexpr int OT = NC * 2;           // 16-dim output tiles (upper bound)
  constexpr int PR = REL ? 16 * QW + 32 : 1;  // position rows of a key block's band
  __shared__ __attribute__((aligned(16))) _Float16 khi[KB * KROW], klo[KB * KROW];
  __shared__ __attribute__((aligned(16))) _Float16 vhi[DP * VROW], vlo[DP * VROW];
  __shared__ __attribute__((aligned(16))) _Float16 phi[PR * KROW], plo[PR * KROW];
  __shared__ float tt[REL ? QW * 48 * 17 : 1];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int li = lane & 15, g = lane >> 4;
  const int b = blockIdx.z, head = blockIdx.y;
  const int t = A.t, hd = A.hd;
  const int kv_len = A.valid_dev ? min(A.valid_dev[b], t) : min(A.valid, t);
  const int q0 = blockIdx.x * 16 * QW;   // the workgroup's first query
  const int qi0 = q0 + wave * 16;        // the wave's
  const int qi = qi0 + li;               // this lane's query
  const int hoff = head * hd;

  const float *qb = A.q + A.bq * b + hoff;
  const float *kb = A.k + A.bq * b + hoff;
  const float *vb = A.v + A.bv * b + hoff;

  // The wave's queries (and (q + v) rows) as split fragments: lane (li, g) holds dims 32c + 8g..
  half8 qh[NC], ql[NC], wh[REL ? NC : 1], wl[REL ? NC : 1];
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

  for (int j0 = 0; j0 < kv_len; j0 += KB) {
    // Stage K [key][dim] and V transposed [dim][key] (two keys per 32-bit store), split.
    for (int e = tid; e < KB * (DP / 4); e += NT) {
      int key = e / (DP / 4), d = 4 * (e % (DP / 4));
      int j = j0 + key;
      float4 k4 = make_float4(0, 0, 0, 0);
      if (j < kv_len && d < hd) k4 = *(const float4 *)(kb + (size_t)j * A.qs + d);
      const float kx[4] = {k4.x, k4.y, k4.z, k4.w};
      half4 h, lo;
#pragma unroll
      for (int q = 0; q < 4; q++) {
        h[q] = (_Float16)kx[q];
        lo[q] = (_Float16)((kx[q] - (float)h[q]) * LO);
      }
      *(half4 *)(khi + key * KROW + d) = h;
      *(half4 *)(klo + key * KROW + d) = lo;
    }
    for (int e = tid; e < (KB / 2) * (DP / 4); e += NT) {
      int kp = e / (DP / 4), d = 4 * (e % (DP / 4));
      int j = j0 + 2 * kp;
      float4 v0 = make_float4(0, 0, 0, 0), v1 = v0;
      if (d < hd) {
        if (j < kv_len) v0 = *(const float4 *)(vb + (size_t)j * A.vs + d);
        if (j + 1 < kv_len) v1 = *(const float4 *)(vb + (size_t)(j + 1) * A.vs + d);
      }
      const float a0[4] = {v0.x, v0.y, v0.z, v0.w}, a1[4] = {v1.x, v1.y, v1.z, v1.w};
#pragma unroll
      for (int q = 0; q < 4; q++) {
        _Float16 h0 = (_Float16)a0[q], h1 = (_Float16)a1[q];
        typedef _Float16 half2v __attribute__((ext_vector_type(2)));
        half2v hh = {h0, h1};
        half2v ll = {(_Float16)((a0[q] - (float)h0) * LO), (_Float16)((a1[q] - (float)h1) * LO)};
        *(half2v *)(vhi + (d + q) * VROW + 2 * kp) = hh;
        *(half2v *)(vlo + (d + q) * VROW + 2 * kp) = ll;
      }
    }
    if constexpr (REL) {
      // The band of position rows this key block needs for the workgroup's queries: rows
      // r0 .. r0 + PR, r0 = j0 − q0 − 16·(QW − 1) + t (position row of key j and query i is
      // j − i + t + 15).  Rows outside the table are zeros.
      const int r0 = j0 - q0 - 16 * (QW - 1) + t, prow = 2 * t + 15;
      for (int e = tid; e < PR * (DP / 4); e += NT) {
        int rr = e / (DP / 4), d = 4 * (e % (DP / 4));
        int r = r0 + rr;
        float4 p4 = make_float4(0, 0, 0, 0);
        if (r >= 0 && r < prow && d < hd) p4 = *(const float4 *)(A.pos + (size_t)r * A.os + hoff + d);
        const float px[4] = {p4.x, p4.y, p4.z, p4.w};
        half4 h, lo;
#pragma unroll
        for (int q = 0; q < 4; q++) {
          h[q] = (_Float16)px[q];
          lo[q] = (_Float16)((px[q] - (float)h[q]) * LO);
        }
        *(half4 *)(phi + rr * KROW + d) = h;
        *(half4 *)(plo + rr * KROW + d) = lo;
      }
    }
    __syncthreads();

    // Scores Sᵀ for the two 16-key tiles: lane holds keys 16·jt + 4g + v of query li.
    float s[2][4];
#pragma unroll
    for (int jt = 0; jt < 2; jt++) {
      floatx4 am = floatx4{}, ac = floatx4{};
#pragma unroll
      for (int c = 0; c < NC; c++) {
        const int off = (16 * jt + li) * KROW + 32 * c + 8 * g;
        half8 ah = *(const half8 *)(khi + off), al = *(const half8 *)(klo + off);
        am = mfma(ah, qh[c], am);
        ac = mfma(ah, ql[c], ac);
        ac = mfma(al, qh[c], ac);
      }
#pragma unroll
      for (int v = 0; v < 4; v++) s[jt][v] = am[v] + ac[v] * LO_INV;
    }

    if constexpr (REL) {
      // Band Tᵀ[r][i] = P[rbase + r]·(q+v)_i for the wave's queries, r in 0..47 (local r =
      // jj − ii + 15); the wave's rows start 16·(QW − 1 − wave) into the staged band.
      const int base = 16 * (QW - 1 - wave);
#pragma unroll
      for (int rt = 0; rt < 3; rt++) {
        floatx4 am = floatx4{}, ac = floatx4{};
#pragma unroll
        for (int c = 0; c < NC; c++) {
          const int off = (base + 16 * rt + li) * KROW + 32 * c + 8 * g;
          half8 ph = *(const half8 *)(phi + off), pl = *(const half8 *)(plo + off);
          am = mfma(ph, wh[c], am);
          ac = mfma(ph, wl[c], ac);
          ac = mfma(pl, wh[c], ac);
        }
#pragma unroll
        for (int v = 0; v < 4; v++) tw[(16 * rt + 4 * g + v) * 17 + li] = am[v] + ac[v] * LO_INV;
      }
      __syncthreads();
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

    // Oᵀ += Vᵀ·Pᵀ: the lane's 8 k-slots are keys 4g + v and 16 + 4g + v, as its P values.
#pragma unroll
    for (int ot = 0; ot < OT; ot++) {
      if (16 * ot >= hd) break;
      om[ot] *= alpha;
      oc[ot] *= alpha;
      const int row = (16 * ot + li) * VROW;
      half4 a0 = *(const half4 *)(vhi + row + 4 * g), a1 = *(const half4 *)(vhi + row + 16 + 4 * g);
      half4 b0 = *(const half4 *)(vlo + row + 4 * g), b1 = *(const half4 *)(vlo + row + 16 + 4 * g);
      half8 vh = {a0[0], a0[1], a0[2], a0[3], a1[0], a1[1], a1[2], a1[3]};
      half8 vl = {b0[0], b0[1], b0[2], b0[3], b1[0], b1[1], b1[2], b1[3]};
      om[ot] = mfma(vh, ph, om[ot]);
      oc[ot] = mfma(vh, pl, oc[ot]);
      oc[ot] = mfma(vl, ph, oc[ot]);
    }
    __syncthreads();
  }

  // The row sums over the 4 lanes of each query, then Oᵀ tile ot holds dims 16·ot + 4g + v.
  l += __shfl_xor(l, 16, 64);
  l += __shfl_xor(l, 32, 64);
  if (qi >= t) return;
  const float inv = l > 0.0f ? 1.0f / l : 0.0f;  // a window with no valid key outputs zeros
  float *ob = A.o + A.bo * b + (size_t)qi * A.os + hoff;
#pragma unroll
  for (int ot = 0; ot < OT; ot++) {
    const int d = 16 * ot + 4 * g;
    if (d >= hd) break;
    float4 r;
    r.x = (om[ot][0] + oc[ot][0] * LO_INV) * inv;
    r.y = (om[ot][1] + oc[ot][1] * LO_INV) * inv;
    r.z = (om[ot][2] + oc[ot][2] * LO_INV) * inv;
    r.w = (om[ot][3] + oc[ot][3] * LO_INV) * inv;
    *(float4 *)(ob + d) = r;  // hd % 4 == 0: a quad is inside or past the head
  }
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
  // 64 queries per workgroup, or 32 when that leaves fewer workgroups than two per CU.
  const long wg64 = (long)((a.t + 63) / 64) * heads * batch;
  const bool narrow = wg64 < 2L * (ctx->cus > 0 ? ctx->cus : 256);
  ProfScope prof(ctx, REL ? (narrow ? "attention_rel_q32" : "attention_rel_q64") : (narrow ? "attention_q32" : "attention_q64"),
                 (REL ? 6.0 : 4.0) * tt, bytes);
  if (narrow) launch_qw<REL, 2>(ctx, a, dim3((a.t + 31) / 32, heads, batch), nc);
  else launch_qw<REL, 4>(ctx, a, dim3((a.t + 63) / 64, heads, batch), nc);
  return wh_launched(ctx, "attention");
}

}  // namespace

int launch_attention(wh_ctx *ctx, const float *qk, const float *v, const float *pos, float *o, int t, int heads,
                     int hd, const int *valid_dev, int valid, int batch) {
  if (t <= 0 || heads <= 0 || hd <= 0 || hd > 128 || hd % 4 || batch <= 0 || !qk || !o)
    return wh_fail(ctx, WH_EARG, "attention: bad shape (t %d, heads %d, head_dim %d)", t, heads, hd);
  if (v && pos) return wh_fail(ctx, WH_EARG, "attention: relative positions take [q+u | k | v | q+v] rows");
  const int ch = heads * hd;
  Args a{};
  a.t = t;
  a.hd = hd;
  a.scale = 1.0f / sqrtf((float)hd);
  a.valid_dev = valid_dev;
  a.valid = valid < 0 || valid > t ? t : valid;
  if (!valid_dev && a.valid == 0) return wh_fail(ctx, WH_EARG, "attention: no valid keys");
  a.o = o;
  a.os = ch;
  a.bo = (long)t * ch;
  a.q = qk;
  if (v) {  // [t][q | k] and v [t][ch]
    a.qs = 2 * ch;
    a.k = qk + ch;
    a.v = v;
    a.vs = ch;
  } else if (!pos) {  // [t][q | k | v]
    a.qs = 3 * ch;
    a.k = qk + ch;
    a.v = qk + 2 * ch;
    a.vs = 3 * ch;
  } else {  // [t][q + u | k | v | q + v]
    a.qs = 4 * ch;
    a.k = qk + ch;
    a.v = qk + 2 * ch;
    a.vs = 4 * ch;
    a.qv = qk + 3 * ch;
    a.pos = pos;
  }
  a.bq = (long)t * a.qs;
  a.bv = (long)t * a.vs;
  return pos ? launch_nc<true>(ctx, a, heads, batch) : launch_nc<false>(ctx, a, heads, batch);
}
