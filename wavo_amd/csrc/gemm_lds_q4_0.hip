// The LDS-DMA GEMM kernels instantiated for q4_0 weights (kernels and plans: gemm.hip, gemm_impl.h).
#include "gemm_impl.h"

int gemm_lds_q4_0(wh_ctx *ctx, const _Float16 *a, const wh_linear *l, void *c, int m, int ldc, int epi, float alpha,
                bool out16, float *part, int *splits, const HeadsOut *ho, int nho) {
  return launch_lds_t<WH_Q4_0>(ctx, a, l, c, m, ldc, epi, alpha, out16, part, splits, ho, nho);
}
