// gemm.hip -- small-M GEMM y[m,n] = sum_k x[m,k] W[n,k] on gfx950 MFMA, for
// decode batches M = 5..64 (the M <= 4 case runs the GEMV).  W is [N, K]
// (K contiguous) in fp16 / bf16 / fp8-e4m3 (+ per-row f32 scale), x is
// [M, K] bf16 or fp16, accumulation f32, and the output stage is the GEMV's
// (store / residual / GELU / SwiGLU / q,k RoPE + KV append).
//
// Replaces the reference's tensor-core small-M matmul
// (src/codegen/render_uop.c:1690-1986 rmu_emit_matmul_tc_tiled_cuda, launch
// shape src/backend/cuda/jit.c:724-787), which is fp16/bf16 WMMA only and
// decodes fp8 to float first.  Design for gfx950:
//   * the weights are the MFMA A operand: a 16-row tile of W against a
//     16-row tile of x (B operand) per v_mfma_f32_16x16x32_{bf16,f16}, so the
//     f32 result rows are weight rows and the columns are batch rows;
//   * each lane streams 16 consecutive k of one weight row per 64-k step
//     (lanes 0-15 rows, lanes 16-63 the next k quarters): a wave's load
//     instruction covers 16 rows x 64 k, nontemporal 16-byte loads;
//   * fp8 decodes exactly into the x operand type (e4m3 values are exact in
//     bf16 and fp16) with v_cvt_pk_f32_fp8; the row scale multiplies the
//     finished sum, as in the dequantised reference computation;
//   * the 8 waves of a block split K into contiguous slices; partial tiles
//     meet in LDS and are summed in wave order (deterministic), then each
//     thread finishes one row pair of one batch row through the shared
//     epilogue;
//   * x tiles are read from L2 (x is a few hundred KB at most and every
//     block reads it), weights once from HBM.
// MFMA operand k order: both operands give lane group g the same 8 k values
// per instruction (k = 16g + j, then 16g + 8 + j), so the sum over k is the
// full dot product whatever order the unit consumes them in.
#include "dev_common.h"
#include "../kern_api.h"
#include "launch.h"
#include "epilogue.h"
#include <stdio.h>

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

enum { GW_F16 = 0, GW_BF16 = 1, GW_FP8 = 2 };   // weight storage
enum { GX_BF16 = 0, GX_F16 = 1 };               // x storage = MFMA operand type

#define GEMM_WAVES 8
#define GEMM_THREADS (64 * GEMM_WAVES)

// four e4m3 bytes -> four 16-bit operand values (two u32), exact
template <int XT>
__device__ __forceinline__ void fp8x4_op(uint32_t w, uint32_t &lo, uint32_t &hi) {
  typedef float f2_t __attribute__((ext_vector_type(2)));
  f2_t a = __builtin_amdgcn_cvt_pk_f32_fp8(w, false);
  f2_t b = __builtin_amdgcn_cvt_pk_f32_fp8(w, true);
  if (XT == GX_BF16) {   // an e4m3 value has <= 4 significant bits: truncation is exact
    lo = (__float_as_uint(a[0]) >> 16) | (__float_as_uint(a[1]) & 0xffff0000u);
    hi = (__float_as_uint(b[0]) >> 16) | (__float_as_uint(b[1]) & 0xffff0000u);
  } else {               // and is exact in fp16 (normal range 2^-14..2^15)
    lo = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(a[0], a[1]));
    hi = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(b[0], b[1]));
  }
}

template <int XT>
__device__ __forceinline__ f32x4_t mfma16(const uint4 &A, const uint4 &B, f32x4_t c) {
  if (XT == GX_BF16)
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, A),
                                                   __builtin_bit_cast(bf16x8_t, B), c, 0, 0, 0);
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, A),
                                                __builtin_bit_cast(f16x8_t, B), c, 0, 0, 0);
}

// MT 16-row tiles of x, NT 16-row tiles of W per block, U 64-k steps in flight
template <int WT, int XT, int MT, int NT, int U>
__global__ __launch_bounds__(GEMM_THREADS) void k_gemm(ThvmGemvArgs a) {
  extern __shared__ float4 red[];                 // [GEMM_WAVES][NT*MT][64]
  constexpr int WB = WT == GW_FP8 ? 1 : 2;        // uint4 per lane per step per W tile
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int li = lane & 15, lg = lane >> 4;
  const uint32_t N = a.N, K = a.K, M = a.M;
  const uint32_t n0 = blockIdx.x * (16u * NT);
  const uint32_t S = K / 64;
  const uint32_t s0 = (uint32_t)(((uint64_t)S * wv) / GEMM_WAVES);
  const uint32_t s1 = (uint32_t)(((uint64_t)S * (wv + 1)) / GEMM_WAVES);
  const uint64_t wrow_b = (uint64_t)K * (WT == GW_FP8 ? 1 : 2);

  const char *wp[NT];
  bool wok[NT];
#pragma unroll
  for (int t = 0; t < NT; t++) {
    const uint32_t n = n0 + 16u * t + li;
    wok[t] = n < N;
    wp[t] = (const char *)a.w + (uint64_t)(wok[t] ? n : 0) * wrow_b + (uint64_t)lg * 16 * WB;
  }
  const char *xp[MT];
  bool xok[MT];
#pragma unroll
  for (int mt = 0; mt < MT; mt++) {
    const uint32_t m = 16u * mt + li;
    xok[mt] = m < M;
    xp[mt] = (const char *)a.x + (uint64_t)(xok[mt] ? m : 0) * a.ldx * 2 + (uint64_t)lg * 32;
  }

  f32x4_t acc[NT][MT];
#pragma unroll
  for (int t = 0; t < NT; t++)
#pragma unroll
    for (int mt = 0; mt < MT; mt++) acc[t][mt] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  uint4 wr[U][NT][WB];
  uint4 xr[U][MT][2];
  const uint4 z4 = make_uint4(0, 0, 0, 0);
  auto load = [&](int u, uint32_t s) {
    const bool live = s < s1;
#pragma unroll
    for (int t = 0; t < NT; t++)
#pragma unroll
      for (int j = 0; j < WB; j++)
        wr[u][t][j] = (live && wok[t]) ? ld_stream16(wp[t] + (uint64_t)s * 64 * WB + j * 16) : z4;
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
      for (int j = 0; j < 2; j++)
        xr[u][mt][j] = (live && xok[mt]) ? ld16(xp[mt] + (uint64_t)s * 128 + j * 16) : z4;
  };
  auto compute = [&](int u) {
#pragma unroll
    for (int t = 0; t < NT; t++) {
      uint4 A0, A1;
      if (WT == GW_FP8) {
        const uint4 q = wr[u][t][0];
        fp8x4_op<XT>(q.x, A0.x, A0.y);
        fp8x4_op<XT>(q.y, A0.z, A0.w);
        fp8x4_op<XT>(q.z, A1.x, A1.y);
        fp8x4_op<XT>(q.w, A1.z, A1.w);
      } else {
        A0 = wr[u][t][0];
        A1 = wr[u][t][WB - 1];
      }
#pragma unroll
      for (int mt = 0; mt < MT; mt++) {
        acc[t][mt] = mfma16<XT>(A0, xr[u][mt][0], acc[t][mt]);
        acc[t][mt] = mfma16<XT>(A1, xr[u][mt][1], acc[t][mt]);
      }
    }
  };

#pragma unroll
  for (int u = 0; u < U; u++) load(u, s0 + u);
  for (uint32_t s = s0; s < s1; s += U) {
#pragma unroll
    for (int u = 0; u < U; u++) {
      if (s + u < s1) compute(u);
      load(u, s + u + U);
    }
  }

  // partial tiles -> LDS, summed in wave order
#pragma unroll
  for (int t = 0; t < NT; t++)
#pragma unroll
    for (int mt = 0; mt < MT; mt++) {
      const f32x4_t v = acc[t][mt];
      red[((size_t)wv * (NT * MT) + t * MT + mt) * 64 + lane] = make_float4(v[0], v[1], v[2], v[3]);
    }
  __syncthreads();
  constexpr int PAIRS = 8 * NT, COLS = 16 * MT;
  for (int task = threadIdx.x; task < PAIRS * COLS; task += GEMM_THREADS) {
    const int p = task % PAIRS, m = task / PAIRS;
    if ((uint32_t)m >= M) continue;
    const int i0 = 2 * p, t = i0 / 16, ii = i0 % 16, mt = m / 16;
    const int ln = (ii / 4) * 16 + (m % 16), r = ii % 4;     // r is 0 or 2
    float s0v = 0.f, s1v = 0.f;
#pragma unroll
    for (int w = 0; w < GEMM_WAVES; w++) {
      const float4 q = red[((size_t)w * (NT * MT) + t * MT + mt) * 64 + ln];
      s0v += r == 0 ? q.x : q.z;
      s1v += r == 0 ? q.y : q.w;
    }
    const float tot[2][1] = {{s0v}, {s1v}};
    gemv_epilogue<2, 1>(a, n0 + i0, tot, (uint32_t)m);
  }
}

// -------------------------------------------------------------------------
typedef void (*gemm_fn)(ThvmGemvArgs);

template <int WT, int XT, int MT>
static gemm_fn pick_nt(int NT) {
  constexpr int U = MT >= 4 ? 2 : 4;
  switch (NT) {
    case 1: return k_gemm<WT, XT, MT, 1, U>;
    case 2: return k_gemm<WT, XT, MT, 2, U>;
    case 4: return k_gemm<WT, XT, MT, 4, (MT >= 2 ? 2 : U)>;
    default: return nullptr;
  }
}
template <int WT, int XT>
static gemm_fn pick_mt(int MT, int NT) {
  switch (MT) {
    case 1: return pick_nt<WT, XT, 1>(NT);
    case 2: return pick_nt<WT, XT, 2>(NT);
    case 4: return pick_nt<WT, XT, 4>(NT);
    default: return nullptr;
  }
}

// Called by thvm_k_gemv after its common argument checks (dtypes, strides,
// epilogue geometry); validates what only the MFMA path needs.
extern "C" int thvm_k_gemm_mfma(const ThvmGemvArgs *a, hipStream_t s, char *err, int errlen) {
  gemm_fn f = nullptr;
  if (a->norm) { snprintf(err, errlen, "gemm: no fused norm on the MFMA path (run the norm kernel first)"); return -1; }
  if (a->M == 0 || a->M > 64) { snprintf(err, errlen, "gemm: M=%u out of range 1..64", a->M); return -1; }
  if (a->K % 64) { snprintf(err, errlen, "gemm: K=%u not a multiple of 64", a->K); return -1; }
  if (((uint64_t)a->ldx * 2) % 16 || ((uintptr_t)a->x & 15) || ((uintptr_t)a->w & 15)) {
    snprintf(err, errlen, "gemm: x rows and W must be 16-byte aligned");
    return -1;
  }
  const int MT = a->M <= 16 ? 1 : a->M <= 32 ? 2 : 4;
  // 16-row weight tiles per block, from the gfx950 sweep over the C4 shapes at
  // M=16: more tiles amortise the x tile reads over more weight rows (wide N),
  // fewer keep enough blocks in flight (N <= 4096)
  int NT = a->tune_r ? (int)a->tune_r : (a->N >= 16384 ? 4 : a->N <= 4096 ? 1 : 2);
  if (NT != 1 && NT != 2 && NT != 4) { snprintf(err, errlen, "gemm: n tiles per block must be 1, 2 or 4"); return -1; }
  const int xbf = a->xdt == THVM_DT_BF16, xf16 = a->xdt == THVM_DT_FP16;
  if (a->wdt == THVM_DT_FP8E4M3) {
    f = xbf ? pick_mt<GW_FP8, GX_BF16>(MT, NT) : xf16 ? pick_mt<GW_FP8, GX_F16>(MT, NT) : nullptr;
  } else if (a->wdt == THVM_DT_BF16 && xbf) {
    f = pick_mt<GW_BF16, GX_BF16>(MT, NT);
  } else if (a->wdt == THVM_DT_FP16 && xf16) {
    f = pick_mt<GW_F16, GX_F16>(MT, NT);
  }
  if (!f) {
    snprintf(err, errlen, "gemm: no MFMA kernel for w=%u x=%u (fp16 W needs fp16 x, bf16 W bf16 x, "
             "fp8 W bf16/fp16 x)", a->wdt, a->xdt);
    return -1;
  }
  const uint32_t lds = (uint32_t)(GEMM_WAVES * NT * MT * 64 * sizeof(float4));
  if (lds > 64 * 1024) {
    hipError_t e = hipFuncSetAttribute((const void *)f, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) { snprintf(err, errlen, "gemm: hipFuncSetAttribute: %s", hipGetErrorString(e)); return -1; }
  }
  const uint32_t grid = (a->N + 16u * NT - 1) / (16u * NT);
  thvm_launch(true, true, f, dim3(grid), dim3(GEMM_THREADS), lds, s, *a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) { snprintf(err, errlen, "gemm launch: %s", hipGetErrorString(e)); return -1; }
  return 0;
}
