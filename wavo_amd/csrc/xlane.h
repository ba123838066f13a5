// Cross-lane reductions of a wavefront on the VALU: DPP moves within rows of 16 lanes and gfx950's
// row swaps (v_permlane16_swap / v_permlane32_swap) across them, instead of __shfl_xor, which is a
// ds_bpermute through the LDS crossbar (~100 cycles of latency per dependent step).  The butterflies
// combine lanes in the order of the __shfl_xor loops they replace (lane bit 5, 4, ..., 0, each a lane's
// own value with its partner's), so their results equal those loops' bit for bit.  Every lane of the
// wavefront must be active.
#pragma once

#include <hip/hip_runtime.h>

namespace xlane {

constexpr int XOR1 = 0xB1;         // quad_perm [1, 0, 3, 2]: lane ^ 1
constexpr int XOR2 = 0x4E;         // quad_perm [2, 3, 0, 1]: lane ^ 2
constexpr int ROR4 = 0x124;        // row_ror:4: lane + 4 within the row
constexpr int ROR8 = 0x128;        // row_ror:8: lane ^ 8
constexpr int HALF_MIRROR = 0x141; // lane i of 8 from lane 7 − i
constexpr int MIRROR = 0x140;      // lane i of 16 from lane 15 − i

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
template <int CTRL>
__device__ __forceinline__ int dpp(int v) { return __builtin_amdgcn_mov_dpp(v, CTRL, 0xF, 0xF, false); }
template <int CTRL>
__device__ __forceinline__ double dpp(double v) {  // both halves
  const unsigned long long u = __builtin_bit_cast(unsigned long long, v);
  const int lo = __builtin_amdgcn_mov_dpp((int)(unsigned)u, CTRL, 0xF, 0xF, false);
  const int hi = __builtin_amdgcn_mov_dpp((int)(unsigned)(u >> 32), CTRL, 0xF, 0xF, false);
  return __builtin_bit_cast(double, (unsigned long long)(unsigned)lo | ((unsigned long long)(unsigned)hi << 32));
}

// v_permlane32_swap: x becomes (x of lanes 0..31 | y of lanes 0..31), y (x of lanes 32..63 | y of
// lanes 32..63).  With x = y = a lane's value, every lane then holds its own value and that of lane
// l ^ 32, one in each register; with two values (x, y), x + y is in lanes 0..31 x plus the partner's x
// and in lanes 32..63 y plus the partner's y.
template <typename T>
__device__ __forceinline__ void swap32(T &x, T &y) {
  const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(unsigned, x), __builtin_bit_cast(unsigned, y), false, false);
  x = __builtin_bit_cast(T, (unsigned)r[0]), y = __builtin_bit_cast(T, (unsigned)r[1]);
}
// v_permlane16_swap: x becomes rows (x0, y0, x2, y2), y rows (x1, y1, x3, y3): the same for lane bit 4.
template <typename T>
__device__ __forceinline__ void swap16(T &x, T &y) {
  const auto r = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(unsigned, x), __builtin_bit_cast(unsigned, y), false, false);
  x = __builtin_bit_cast(T, (unsigned)r[0]), y = __builtin_bit_cast(T, (unsigned)r[1]);
}
// The same for 64-bit values, half by half.
__device__ __forceinline__ void swap32(double &x, double &y) {
  unsigned long long u = __builtin_bit_cast(unsigned long long, x), w = __builtin_bit_cast(unsigned long long, y);
  unsigned xl = (unsigned)u, xh = (unsigned)(u >> 32), yl = (unsigned)w, yh = (unsigned)(w >> 32);
  swap32(xl, yl), swap32(xh, yh);
  x = __builtin_bit_cast(double, (unsigned long long)xl | ((unsigned long long)xh << 32));
  y = __builtin_bit_cast(double, (unsigned long long)yl | ((unsigned long long)yh << 32));
}
__device__ __forceinline__ void swap16(double &x, double &y) {
  unsigned long long u = __builtin_bit_cast(unsigned long long, x), w = __builtin_bit_cast(unsigned long long, y);
  unsigned xl = (unsigned)u, xh = (unsigned)(u >> 32), yl = (unsigned)w, yh = (unsigned)(w >> 32);
  swap16(xl, yl), swap16(xh, yh);
  x = __builtin_bit_cast(double, (unsigned long long)xl | ((unsigned long long)xh << 32));
  y = __builtin_bit_cast(double, (unsigned long long)yl | ((unsigned long long)yh << 32));
}

// op(v, v of lane l ^ 32) and op(v, v of lane l ^ 16), for a commutative op.
template <typename T, class Op>
__device__ __forceinline__ T bit5(T v, Op op) {
  T x = v, y = v;
  swap32(x, y);
  return op(x, y);
}
template <typename T, class Op>
__device__ __forceinline__ T bit4(T v, Op op) {
  T x = v, y = v;
  swap16(x, y);
  return op(x, y);
}

// The xor butterfly over all six lane bits.  Bits 2 .. 0 after bits 5 .. 3: lane + 4 within the row
// differs from lane ^ 4 only in bit 3, whose lanes hold equal values by then.
template <typename T, class Op>
__device__ __forceinline__ T butterfly(T v, Op op) {
  v = bit5(v, op);
  v = bit4(v, op);
  v = op(v, dpp<ROR8>(v));
  v = op(v, dpp<ROR4>(v));
  v = op(v, dpp<XOR2>(v));
  return op(v, dpp<XOR1>(v));
}

struct Add {
  template <typename T>
  __device__ __forceinline__ T operator()(T a, T b) const { return a + b; }
};
struct Max {
  __device__ __forceinline__ float operator()(float a, float b) const { return fmaxf(a, b); }
};

// The sum and the maximum over the wavefront, in every lane.
__device__ __forceinline__ float wave_sum(float v) { return butterfly(v, Add{}); }
__device__ __forceinline__ double wave_sum(double v) { return butterfly(v, Add{}); }
__device__ __forceinline__ float wave_max(float v) { return butterfly(v, Max{}); }

// The first maximum of every lane's (v, i) (the greater value, or an equal one at the smaller index;
// i < 0 or better() false: none) over the wavefront, in every lane.  A selection by a total order: the
// result does not depend on the order in which lanes meet (values that are NaN aside).
template <class Better>
__device__ __forceinline__ void wave_first_max(float &v, int &i, Better better) {
  auto take = [&](float ov, int oi) {
    if (better(ov, oi, v, i)) v = ov, i = oi;
  };
  take(dpp<XOR1>(v), dpp<XOR1>(i));
  take(dpp<XOR2>(v), dpp<XOR2>(i));
  take(dpp<HALF_MIRROR>(v), dpp<HALF_MIRROR>(i));
  take(dpp<MIRROR>(v), dpp<MIRROR>(i));
  // Rows: after a swap both registers hold a pair of row results, the same pair for both rows.
  float x = v, y = v;
  int a = i, b = i;
  swap16(x, y), swap16(a, b);
  v = x, i = a;
  take(y, b);
  x = v, y = v, a = i, b = i;
  swap32(x, y), swap32(a, b);
  v = x, i = a;
  take(y, b);
}

}  // namespace xlane
