// gemv_inst.hip -- the standalone GEMV kernel instances for one (weight type,
// x type) pair, chosen at compile time by GEMV_WT / GEMV_XD; the build
// compiles this file once per pair (twelve translation units in parallel
// instead of one unit holding every instance).  GEMV_PICK names the pair's
// picker, which gemv.hip's launcher calls.
#include "gemv_core.h"

#if !defined(GEMV_WT) || !defined(GEMV_XD) || !defined(GEMV_PICK)
#error "gemv_inst.hip is compiled with -DGEMV_WT=<0..3> -DGEMV_XD=<0..3> -DGEMV_PICK=<name>"
#endif

// The standalone kernel: waves own row groups blockIdx*nw + wave, grid-stride.
// blockIdx.y selects a chunk of M batch rows (x, y and res advance by M rows
// per chunk): batches above 4 rows whose operands the MFMA GEMM does not take
// run as chunks of 4, each output row computed exactly as at M <= 4.
template <int WT, int XD, int M, int R, int U>
__global__ __launch_bounds__(1024) void k_gemv(ThvmGemvArgs a) {
  extern __shared__ __align__(16) unsigned char xs_raw[];
  __shared__ __align__(16) float red[GEMV_MAX_WAVES];
  const int nw = blockDim.x >> 6;
  const uint32_t g = blockIdx.x * nw + (threadIdx.x >> 6);
  if (blockIdx.y) {
    const uint64_t m0 = (uint64_t)blockIdx.y * M, ys = a.ydt == THVM_DT_FP32 ? 4 : 2;
    a.x = (const char *)a.x + m0 * a.ldx * XDr<XD>::B;
    a.y = (char *)a.y + m0 * a.ldy * ys;
    if (a.res) a.res = (const char *)a.res + m0 * a.ldy * ys;
  }
  // a fused norm reduces over the first 512 threads whatever the block size,
  // so its summation order (and the rounded row it stages) is the same at 8
  // and 16 waves per block, and the same as the persistent step's
  const uint32_t nthr = blockDim.x < 512 ? blockDim.x : 512;
  gemv_core<WT, XD, M, R, U, false>(
      a, xs_raw, red, g, gridDim.x * nw, nthr, (int)(nthr >> 6), [] { return true; },
      [&](int m) { return (const void *)((const char *)a.x + (uint64_t)m * a.ldx * XDr<XD>::B); },
      [](uint32_t, const float (&)[R][M]) {}, (uint32_t)blockDim.x);
  pclk_end(a.clk, a.clk_cap);
}

// -------------------------------------------------------------------------
typedef void (*gemv_fn)(ThvmGemvArgs);

template <int WT, int XD, int R, int U>
static gemv_fn pick_m(uint32_t M) {
  if constexpr (XD == XD_SUM4) {
    return M == 1 ? k_gemv<WT, XD, 1, R, U> : nullptr;   // one row only
  } else {
    switch (M) {
      case 1: return k_gemv<WT, XD, 1, R, U>;
      case 2: return k_gemv<WT, XD, 2, R, U>;
      case 3: return k_gemv<WT, XD, 3, R, U>;
      case 4: return k_gemv<WT, XD, 4, R, U>;
      default: return nullptr;
    }
  }
}
template <int WT, int XD>
static gemv_fn pick_ru(uint32_t M, int R, int U) {
  if (R == 1) return U == 8 ? pick_m<WT, XD, 1, 8>(M) : pick_m<WT, XD, 1, 4>(M);
  return U == 8 ? pick_m<WT, XD, 2, 8>(M) : pick_m<WT, XD, 2, 4>(M);
}
gemv_fn GEMV_PICK(uint32_t M, int R, int U) { return pick_ru<GEMV_WT, GEMV_XD>(M, R, U); }
