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
//     bf16 and fp16): v_cvt_scalef32_pk_bf16_fp8 for bf16, v_cvt_pk_f32_fp8
//     then a pack for fp16; the row scale multiplies the
//     finished sum, as in the dequantised reference computation;
//   * the 8 waves of a block split K into contiguous slices; partial tiles
//     meet in LDS and are summed in wave order (deterministic), then each
//     thread finishes one row pair of one batch row through the shared
//     epilogue;
//   * x tiles are read from L2 (x is a few hundred KB at most and every
//     block reads it), weights once from HBM;
//   * RMSNorm on x fused (NM = 1, bf16 x): the staging stores rnd(x * g[k])
//     and sums x^2 over the wave's k slice; the slices' sums meet in LDS
//     (wave order) and inv = 1/sqrtf(ss * (1/K) + eps) scales the finished
//     row sums.  Each product x*g*w therefore carries one bf16 rounding, as
//     with the norm kernel's rnd((x * inv) * g), at a different point; bf16
//     keeps f32's exponent range, so x*g cannot overflow where x*inv*g would
//     not.  The batched decode step then needs no separate norm launch.
// MFMA operand k order: both operands give lane group g the same 8 k values
// per instruction (k = 16g + j, then 16g + 8 + j), so the sum over k is the
// full dot product whatever order the unit consumes them in.
#include "dev_common.h"
#include "../kern_api.h"
#include "launch.h"
#include "epilogue.h"
#include "mfma_ops.h"
#include <stdio.h>

#define GEMM_WAVES 8
#define GEMM_THREADS (64 * GEMM_WAVES)

// MT 16-row tiles of x, NT 16-row tiles of W per block, U 64-k steps in flight.
// Each wave stages its own slice of x into a private LDS region, GEMM_SC(MT)
// 64-k steps of its 16*MT rows at a time, with row-contiguous 16-byte loads
// (8*SC lanes per row); the MFMA B operand is then read from LDS, rows padded
// by 16 bytes so the 16 rows of one read fall in different banks.
// GEMM_XSTAGE = 4 keeps a block's x staging at 66 KB, so two blocks share a
// CU: measured on gfx950 against 8 (133 KB, one block per CU, the gate/up
// grid of 448 blocks in 1.75 rounds), C4 batch 16 4.78 -> 4.57 ms per step,
// C3 batch 8 3.30 -> 3.09 ms (4 is the least the 64-row tile takes).
#ifndef GEMM_XSTAGE
#define GEMM_XSTAGE 4                              // 64-k steps x 16-row tiles staged
#endif
#define GEMM_SC(MT) (GEMM_XSTAGE / (MT))
#define GEMM_XROW(MT) (GEMM_SC(MT) * 128 + 16)
template <int WT, int XT, int MT, int NT, int U, int NM>
__global__ __launch_bounds__(GEMM_THREADS) void k_gemm(ThvmGemvArgs a) {
  extern __shared__ float4 red[];                 // x staging, then [GEMM_WAVES][NT*MT][64]
  __shared__ float ssw[NM ? GEMM_WAVES : 1][NM ? 64 : 1];   // per-wave sums of x^2 per x row
  static_assert(!NM || XT == GX_BF16, "the fused norm stages bf16 x");
  constexpr int WB = WT == GW_FP8 ? 1 : 2;        // uint4 per lane per step per W tile
  constexpr int SC = GEMM_SC(MT), XROW = GEMM_XROW(MT);
  static_assert(SC % U == 0, "sub-chunks hold whole prefetch rounds");
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int li = lane & 15, lg = lane >> 4;
  const uint32_t N = a.N, K = a.K, M = a.M;
  const uint32_t n0 = blockIdx.x * (16u * NT);
  const uint32_t S = K / 64;
  const uint32_t s0 = (uint32_t)(((uint64_t)S * wv) / GEMM_WAVES);
  const uint32_t s1 = (uint32_t)(((uint64_t)S * (wv + 1)) / GEMM_WAVES);
  const uint64_t wrow_b = (uint64_t)K * (WT == GW_FP8 ? 1 : 2);
  char *xs = (char *)red + (size_t)wv * (16 * MT * XROW);

  // this block's weight rows; rows past N read zero (row-major: the range
  // ends at row N; tiled: the padded rows of the last group are zeros)
  const bool tl = a.wtiled != 0;
  const uint32_t nrow = tl ? (((N + 15u) & ~15u) - n0) : (N - n0);
  const buf_t wrs = buf_rsrc((const char *)a.w + (uint64_t)n0 * wrow_b,
                             (uint32_t)(min(nrow, 16u * NT) * wrow_b));
  const buf_t xrs = buf_rsrc(a.x, (uint32_t)(((uint64_t)(M - 1) * a.ldx + K) * 2));
  // per step: row-major, lane l reads 16*WB bytes of row li at k quarter lg
  // (an instruction covers 16 rows x 64 bytes); tiled, the same bytes sit at
  // lane*16 of the step's 1 KB pieces (an instruction reads 1 KB contiguous)
  const uint32_t sstep = tl ? 1024u * WB : 64u * WB, jstep = tl ? 1024u : 16u;
  uint32_t wo[NT];
#pragma unroll
  for (int t = 0; t < NT; t++)
    wo[t] = tl ? (uint32_t)(t * S * WB * 1024u) + lane * 16u
               : (uint32_t)((16u * t + li) * wrow_b) + lg * 16 * WB;

  f32x4_t acc[NT][MT];
#pragma unroll
  for (int t = 0; t < NT; t++)
#pragma unroll
    for (int mt = 0; mt < MT; mt++) acc[t][mt] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  uint4 wr[U][NT][WB];
  auto load = [&](int u, uint32_t s) {
    const uint32_t so = s < s1 ? s * sstep : BUF_OOB;
#pragma unroll
    for (int t = 0; t < NT; t++)
#pragma unroll
      for (int j = 0; j < WB; j++) wr[u][t][j] = buf_ld_stream16(wrs, wo[t] + so + j * jstep);
  };
  // x rows [0, 16*MT) x steps [sc0, sc0 + SC), RPI rows per load instruction,
  // 8*SC lanes per row (16 bytes each), held in registers until stored to
  // LDS: the next sub-chunk is loaded while this one is consumed, so waiting
  // for it never waits for the weight loads issued after it.  Rows >= M and
  // k >= K read zero (out of range); steps past the wave's slice are real x
  // values that meet zero weights.
  constexpr int RPI = 8 / SC, NI = 16 * MT / RPI;
  static_assert(SC <= 8 && RPI * SC == 8 && NI * RPI == 16 * MT, "staging shape");
  const uint32_t sr = lane / (8 * SC), sl = lane % (8 * SC);
  uint4 xv[NI];
  // fused norm: the gains of the lane's 8 k, whether its step lies in the
  // wave's slice (steps past s1 are staged for zero weights and must not
  // count twice), and the lane's running sums of x^2, one per staged row
  const buf_t grs = buf_rsrc(NM ? (const void *)a.norm_w : (const void *)a.x, NM ? K * 4u : 0u);
  uint4 gv[2];
  bool xok = false;
  float ss[NI];
#pragma unroll
  for (int i = 0; i < NI; i++) ss[i] = 0.f;
  auto xload = [&](uint32_t sc0, bool live) {
    const uint32_t k = sc0 * 64 + sl * 8;
    const uint32_t base = live && k < K ? (sr * a.ldx + k) * 2 : BUF_OOB;
#pragma unroll
    for (int i = 0; i < NI; i++) xv[i] = buf_ld16(xrs, base + i * RPI * a.ldx * 2);
    if (NM) {
      const uint32_t go = live && k < K ? k * 4 : BUF_OOB;
      gv[0] = buf_ld16(grs, go);
      gv[1] = buf_ld16(grs, go + 16);
      xok = live && sc0 + sl / 8 < s1;
    }
  };
  auto xstore = [&]() {
    if (NM) {
      const uint32_t gw[8] = {gv[0].x, gv[0].y, gv[0].z, gv[0].w, gv[1].x, gv[1].y, gv[1].z, gv[1].w};
#pragma unroll
      for (int i = 0; i < NI; i++) {
        const uint32_t q[4] = {xv[i].x, xv[i].y, xv[i].z, xv[i].w};
        uint32_t o[4];
        float s = ss[i];
#pragma unroll
        for (int j = 0; j < 4; j++) {
          const float lo = __uint_as_float(q[j] << 16), hi = __uint_as_float(q[j] & 0xffff0000u);
          s = fmaf(lo, lo, s);
          s = fmaf(hi, hi, s);
          o[j] = pk_bf16(lo * __uint_as_float(gw[2 * j]), hi * __uint_as_float(gw[2 * j + 1]));
        }
        if (xok) ss[i] = s;
        xv[i] = make_uint4(o[0], o[1], o[2], o[3]);
      }
    }
#pragma unroll
    for (int i = 0; i < NI; i++) *(uint4 *)(xs + (i * RPI + sr) * XROW + sl * 16) = xv[i];
    // one wave writes and reads its region, and a wave's LDS operations
    // complete in order: only the compiler must keep the order
    __builtin_amdgcn_wave_barrier();
    asm volatile("" ::: "memory");
  };
  auto compute = [&](int u, uint32_t so) {
    uint4 B[MT][2];
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
      for (int j = 0; j < 2; j++)
        B[mt][j] = *(const uint4 *)(xs + (16 * mt + li) * XROW + so * 128 + lg * 32 + j * 16);
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
        acc[t][mt] = mfma16<XT>(A0, B[mt][0], acc[t][mt]);
        acc[t][mt] = mfma16<XT>(A1, B[mt][1], acc[t][mt]);
      }
    }
  };

  // whole sub-chunks, also past s1 (zero weights), so the step loop is
  // straight-line code and every wait counts only the loads it needs
  // phase clock (measurement build): 0 entry, 1 first loads issued, 2 first
  // x sub-chunk staged, 3 first sub-chunk's MFMAs done, 4 K slice done, 5
  // partial tiles summed, 7 drained
  pclk(a.clk, a.clk_cap, 0);
  const uint32_t nsub = (s1 - s0 + SC - 1) / SC;
  xload(s0, true);
#pragma unroll
  for (int u = 0; u < U; u++) load(u, s0 + u);
  pclk(a.clk, a.clk_cap, 1);
  for (uint32_t c = 0; c < nsub; c++) {
    const uint32_t sb = s0 + c * SC;
    xstore();
    if (c == 0) pclk(a.clk, a.clk_cap, 2);
    if (c == 1) pclk(a.clk, a.clk_cap, 3);
    xload(sb + SC, c + 1 < nsub);
    __builtin_amdgcn_sched_barrier(0);            // issue them before this sub-chunk's weight loads
#pragma unroll
    for (int g = 0; g < SC / U; g++)
#pragma unroll
      for (int u = 0; u < U; u++) {
        compute(u, g * U + u);
        load(u, sb + g * U + u + U);
      }
  }
  if (NM) {   // a row's sum over the wave's slice: its 8*SC lanes, then LDS
#pragma unroll
    for (int i = 0; i < NI; i++) {
      float s = ss[i];
#pragma unroll
      for (int o = 1; o < 8 * SC; o <<= 1) s += __shfl_xor(s, o);
      if (sl == 0) ssw[wv][i * RPI + sr] = s;
    }
  }
  pclk(a.clk, a.clk_cap, 4);
  __syncthreads();                                // the staging area becomes the reduction buffer

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
    if (NM) {
      float t = 0.f;
#pragma unroll
      for (int w = 0; w < GEMM_WAVES; w++) t += ssw[w][m];
      const float inv = 1.0f / sqrtf(t * (1.0f / (float)K) + a.norm_eps);
      s0v *= inv;
      s1v *= inv;
    }
    const float tot[2][1] = {{s0v}, {s1v}};
    if (task == (int)threadIdx.x) pclk(a.clk, a.clk_cap, 5);
    gemv_epilogue<2, 1>(a, n0 + i0, tot, (uint32_t)m);
  }
  pclk_end(a.clk, a.clk_cap);
}

// -------------------------------------------------------------------------
typedef void (*gemm_fn)(ThvmGemvArgs);

template <int WT, int XT, int MT, int NM>
static gemm_fn pick_nt(int NT) {
  constexpr int SC = GEMM_SC(MT);
  constexpr int U = (MT >= 4 ? 2 : 4) < SC ? (MT >= 4 ? 2 : 4) : SC;
  constexpr int U4 = MT >= 2 && U > 2 ? 2 : U;
  switch (NT) {
    case 1: return k_gemm<WT, XT, MT, 1, U, NM>;
    case 2: return k_gemm<WT, XT, MT, 2, U, NM>;
    case 4: return k_gemm<WT, XT, MT, 4, U4, NM>;
    // 7 or 8 tiles: one x tile and fp8 weights only (more accumulators or
    // 16-bit weight registers would spill)
    case 7: return MT == 1 && WT == GW_FP8 ? k_gemm<GW_FP8, XT, 1, 7, 2, NM> : nullptr;
    case 8: return MT == 1 && WT == GW_FP8 ? k_gemm<GW_FP8, XT, 1, 8, 2, NM> : nullptr;
    default: return nullptr;
  }
}
template <int WT, int XT, int NM = 0>
static gemm_fn pick_mt(int MT, int NT) {
  switch (MT) {
    case 1: return pick_nt<WT, XT, 1, NM>(NT);
    case 2: return pick_nt<WT, XT, 2, NM>(NT);
    case 4: return pick_nt<WT, XT, 4, NM>(NT);
    default: return nullptr;
  }
}

// Called by thvm_k_gemv after its common argument checks (dtypes, strides,
// epilogue geometry); validates what only the MFMA path needs.
extern "C" int thvm_k_gemm_mfma(const ThvmGemvArgs *a, hipStream_t s, char *err, int errlen) {
  gemm_fn f = nullptr;
  if (a->norm && (a->norm != 1 || a->xdt != THVM_DT_BF16 || a->norm_w == nullptr)) {
    snprintf(err, errlen, "gemm: the MFMA path fuses RMSNorm with a gain over bf16 x only (norm=1, xt=bf16)");
    return -1;
  }
  if (a->M == 0 || a->M > 64) { snprintf(err, errlen, "gemm: M=%u out of range 1..64", a->M); return -1; }
  if (a->K % 64) { snprintf(err, errlen, "gemm: K=%u not a multiple of 64", a->K); return -1; }
  if (((uint64_t)a->ldx * 2) % 16 || ((uintptr_t)a->x & 15) || ((uintptr_t)a->w & 15)) {
    snprintf(err, errlen, "gemm: x rows and W must be 16-byte aligned");
    return -1;
  }
  // buffer-resource ranges (x whole, W per block) and offsets are 31-bit
  if (64ull * a->ldx * 2 >= (1ull << 31) ||
      64ull * a->K * (a->wdt == THVM_DT_FP8E4M3 ? 1 : 2) >= (1ull << 30)) {
    snprintf(err, errlen, "gemm: x or a 64-row weight panel exceeds 1 GiB");
    return -1;
  }
  const int MT = a->M <= 16 ? 1 : a->M <= 32 ? 2 : 4;
  // 16-row weight tiles per block, from the gfx950 sweep over the C4 shapes at
  // M=16: more tiles amortise the x tile reads over more weight rows (wide N),
  // fewer keep enough blocks in flight (N <= 4096)
  // At one x tile (M <= 16) the block count is sized to one block per CU:
  // these kernels hold more than 128 VGPRs (8 waves: one block per CU), so a
  // grid of more than 256 blocks runs in rounds -- measured on gfx950, the
  // C4 batch-16 gate/up at 4 tiles (448 blocks) ran as a first round of 256
  // blocks and a second of 192, ~15 us each.  Tiles per block: the fewest of
  // 1, 2, 4, 7, 8 that cover ceil(N/16) tiles in 256 blocks (gate/up 7, the
  // LM head 8 in several rounds); 7 and 8 with fp8 weights only.
  const uint32_t tiles = (a->N + 15u) / 16u, need = (tiles + 255u) / 256u;
  const bool wide = MT == 1 && a->wdt == THVM_DT_FP8E4M3;
  int NT = a->tune_r ? (int)a->tune_r
         : MT == 1 ? (need <= 1 ? 1 : need == 2 ? 2 : need <= 4 || !wide ? 4 : need <= 7 ? 7 : 8)
                   : (a->N >= 16384 ? 4 : a->N <= 4096 ? 1 : 2);
  if (NT != 1 && NT != 2 && NT != 4 && !(wide && (NT == 7 || NT == 8))) {
    snprintf(err, errlen, "gemm: n tiles per block must be 1, 2 or 4 (7 or 8 with fp8 weights at M <= 16)");
    return -1;
  }
  const int xbf = a->xdt == THVM_DT_BF16, xf16 = a->xdt == THVM_DT_FP16;
  if (a->norm) {
    f = a->wdt == THVM_DT_FP8E4M3 ? pick_mt<GW_FP8, GX_BF16, 1>(MT, NT)
      : a->wdt == THVM_DT_BF16 ? pick_mt<GW_BF16, GX_BF16, 1>(MT, NT) : nullptr;
  } else if (a->wdt == THVM_DT_FP8E4M3) {
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
  uint32_t lds = (uint32_t)(GEMM_WAVES * NT * MT * 64 * sizeof(float4));
  const uint32_t xlds = (uint32_t)(GEMM_WAVES * 16 * MT * (GEMM_XSTAGE / MT * 128 + 16));
  if (xlds > lds) lds = xlds;
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

// ---- the MFMA tile layout of a weight matrix ------------------------------
// One thread per 16-byte piece of the tiled matrix (the layout is described
// at thvm_k_tile_w in kern_api.h).
__global__ __launch_bounds__(256) void k_tile_w(uint4 *y, const unsigned char *w, uint32_t N, uint64_t RB,
                                                 uint32_t lb, uint64_t nchunks) {
  const uint64_t c = (uint64_t)blockIdx.x * 256 + threadIdx.x;
  if (c >= nchunks) return;
  const uint32_t per = 4u * lb;                        // 16-byte pieces per (group, step) block
  const uint64_t blk = c / per;
  const uint32_t within = (uint32_t)(c % per), jj = within / 64, l = within % 64;
  const uint64_t S = RB / (4u * lb);
  const uint64_t g = blk / S, st = blk % S;
  const uint64_t n = g * 16 + (l % 16);
  const uint64_t b0 = st * 4u * lb + (l / 16) * lb + jj * 16;
  y[c] = n < N ? *(const uint4 *)(w + n * RB + b0) : make_uint4(0, 0, 0, 0);
}

extern "C" int thvm_k_tile_w(void *y, const void *w, uint32_t N, uint32_t K, uint32_t es, uint32_t lb,
                             hipStream_t s, char *err, int errlen) {
  if (lb == 0) lb = 16 * es;
  const uint64_t RB = (uint64_t)K * es;
  if ((es != 1 && es != 2) || (lb != 16 && lb != 32) || N == 0 || K == 0 || RB % (4 * lb) ||
      ((uintptr_t)w & 15) || ((uintptr_t)y & 15)) {
    snprintf(err, errlen, "tile_w: need es 1 or 2, 16 or 32 bytes per lane dividing a quarter row, "
             "16-byte aligned buffers (N=%u K=%u es=%u lb=%u)", N, K, es, lb);
    return -1;
  }
  const uint64_t npad = ((uint64_t)N + 15) / 16 * 16;
  const uint64_t nchunks = npad * RB / 16;
  thvm_launch(true, true, k_tile_w, dim3((unsigned)((nchunks + 255) / 256)), dim3(256), 0, s, (uint4 *)y,
              (const unsigned char *)w, N, RB, lb, nchunks);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) { snprintf(err, errlen, "tile_w launch: %s", hipGetErrorString(e)); return -1; }
  return 0;
}
