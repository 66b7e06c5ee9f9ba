// gemv.hip -- bandwidth-bound decode projection y[m,n] = sum_k x[m,k] W[n,k]
// for small M (1..4), W in f32 / fp16 / bf16 / fp8-e4m3 (+ per-row f32 scale),
// fp32 accumulation, with an optional fused RMSNorm / LayerNorm prologue on x
// and fused epilogues (residual, SwiGLU, GELU, q/k RoPE + KV-cache append).
//
// Replaces the reference's two-phase split-K GEMV + fold kernels
// (bench/dsv2_decode_bench.c:1043-1125 src_gemv/src_gred, and the folds fused
// into gred_q :435-485, kv_prep :487-556, gred_o_rms :558-611, gred_down
// :613-636), its fused RMSNorm (src_rms :397-433) and the renderer's
// GROUP_REDUCE matvec (src/codegen/hand_opts.c:413-470).  The kernel body is
// gemv_core (gemv_core.h), shared with the persistent decode step; this file
// holds the standalone kernel and its launcher (shape checks, the MFMA GEMM
// path for M > 4, launch geometry).
#include "gemv_core.h"
#include "launch.h"
#include <stdio.h>

typedef void (*gemv_fn)(ThvmGemvArgs);

// one picker per (weight type, x type), each in its own gemv_inst.hip unit
#define GEMV_PICKERS(X) \
  X(0, 0) X(0, 1) X(0, 2) X(1, 0) X(1, 1) X(1, 2) X(2, 0) X(2, 1) X(2, 2) X(3, 0) X(3, 1) X(3, 2) \
  X(2, 3) X(3, 3)
#define GEMV_DECL(w, x) gemv_fn gemv_pick_##w##_##x(uint32_t M, int R, int U);
GEMV_PICKERS(GEMV_DECL)
#undef GEMV_DECL

template <int WT>
static gemv_fn pick_x(uint32_t xdt, uint32_t M, int R, int U, bool xsum = false) {
  static_assert(WT_F32 == 0 && WT_FP8 == 3 && XD_BF16 == 0 && XD_F32 == 2 && XD_SUM4 == 3, "picker numbering");
  const int xd = xsum ? XD_SUM4
               : xdt == THVM_DT_BF16 ? XD_BF16 : xdt == THVM_DT_FP16 ? XD_F16 : xdt == THVM_DT_FP32 ? XD_F32 : -1;
#define GEMV_CASE(w, x) if (WT == w && xd == x) return gemv_pick_##w##_##x(M, R, U);
  GEMV_PICKERS(GEMV_CASE)
#undef GEMV_CASE
  return nullptr;
}

static int dt_size(uint32_t dt) {
  switch (dt) {
    case THVM_DT_FP32: return 4;
    case THVM_DT_FP16: case THVM_DT_BF16: return 2;
    case THVM_DT_FP8E4M3: return 1;
    default: return 0;
  }
}
static int act_ok(uint32_t dt) {
  return dt == THVM_DT_FP32 || dt == THVM_DT_FP16 || dt == THVM_DT_BF16;
}

extern "C" int thvm_k_gemv(const ThvmGemvArgs *a, hipStream_t s, char *err, int errlen) {
  int wsz = dt_size(a->wdt);
  if (wsz == 0 || !act_ok(a->xdt) || !act_ok(a->ydt)) {
    snprintf(err, errlen, "gemv: unsupported dtypes w=%u x=%u y=%u", a->wdt, a->xdt, a->ydt);
    return -1;
  }
  if (a->M < 1 || a->M > 64 || a->N == 0 || a->K == 0) {
    snprintf(err, errlen, "gemv: M=%u N=%u K=%u out of range (M in 1..64)", a->M, a->N, a->K);
    return -1;
  }
  if (((uint64_t)a->K * wsz) % 16 != 0) {
    snprintf(err, errlen, "gemv: K*sizeof(w)=%llu not a multiple of 16 bytes",
             (unsigned long long)a->K * wsz);
    return -1;
  }
  if (((uintptr_t)a->w & 15) != 0) {
    snprintf(err, errlen, "gemv: weight pointer not 16-byte aligned");
    return -1;
  }
  if (a->wdt == THVM_DT_FP8E4M3 && a->scale == nullptr) {
    snprintf(err, errlen, "gemv: fp8 weights need a scale vector");
    return -1;
  }
  if (a->ldx < a->K) { snprintf(err, errlen, "gemv: ldx < K"); return -1; }
  const bool xsum = a->norm == 3;
  if (xsum) {
    // x = bf16(norm_w * ((x0 + x1) + (x2 + x3))) from four f32 vectors
    if (a->M != 1 || a->xdt != THVM_DT_BF16 || (a->wdt != THVM_DT_FP8E4M3 && a->wdt != THVM_DT_BF16) ||
        a->K % 8 || a->xqs < a->K || ((uintptr_t)a->x & 7) || ((uintptr_t)a->norm_w & 7) ||
        a->tune_path == 2 || (3ull * a->xqs + a->K) * 4ull >= (1ull << 31)) {
      snprintf(err, errlen, "gemv: norm=3 (summed x) takes one bf16 x row over fp8/bf16 weights, "
               "K a multiple of 8, xqs >= K, 8-byte aligned x and gains");
      return -1;
    }
  }
  if (!xsum) {
    const uint32_t xs = a->xdt == THVM_DT_FP32 ? 4 : 2, ve = 16 / xs;
    if (a->K % ve || ((uint64_t)a->ldx * xs) % 16 || ((uintptr_t)a->x & 15) ||
        ((uintptr_t)a->norm_w & 15) || ((uintptr_t)a->norm_b & 15)) {
      snprintf(err, errlen, "gemv: x rows and norm vectors must be 16-byte aligned and K a multiple of %u", ve);
      return -1;
    }
  }
  if (a->norm > 3) { snprintf(err, errlen, "gemv: unknown norm %u", a->norm); return -1; }
  // defaults from the gfx950 sweep over the C4 projection shapes (8 waves per
  // block, one row per wave unless the epilogue pairs rows, U=4, <= 512 blocks)
  uint32_t waves = a->tune_waves ? a->tune_waves : 8;
  if (waves < 1 || waves > 16) {
    snprintf(err, errlen, "gemv: waves per block must be 1..16");
    return -1;
  }
  int R = 1;
  int pairs = 0;
  switch (a->epi) {
    case THVM_EPI_STORE: case THVM_EPI_GELU: case THVM_EPI_RESID:
      if (a->epi == THVM_EPI_RESID && a->res == nullptr) {
        snprintf(err, errlen, "gemv: residual epilogue without res");
        return -1;
      }
      R = 1;
      break;
    case THVM_EPI_SWIGLU:
      if (a->N % 2) { snprintf(err, errlen, "gemv: swiglu needs even N"); return -1; }
      R = 2; pairs = 1;
      break;
    case THVM_EPI_QKV_ROPE: case THVM_EPI_QKV: {
      uint32_t hd = a->head_dim;
      if (hd == 0 || hd % 2 || a->n_heads == 0 || a->n_kv_heads == 0 ||
          a->N != (a->n_heads + 2 * a->n_kv_heads) * hd || a->kcache == nullptr ||
          a->vcache == nullptr || a->len == nullptr || a->max_seq == 0 ||
          (a->epi == THVM_EPI_QKV_ROPE && (a->rope_cos == nullptr || a->rope_sin == nullptr))) {
        snprintf(err, errlen, "gemv: bad qkv epilogue geometry");
        return -1;
      }
      R = 2; pairs = 1;
    } break;
    default:
      snprintf(err, errlen, "gemv: unknown epilogue %u", a->epi);
      return -1;
  }
  // path: the MFMA GEMM for batches above 4 rows (or x too large for LDS
  // staging), the GEMV otherwise; tune_path 1/2 forces GEMV/MFMA
  if (a->tune_path > 2) { snprintf(err, errlen, "gemv: path must be 0, 1 or 2"); return -1; }
  // row chunks: M > 4 with operands the MFMA GEMM does not take (f32 weights
  // or x, mixed 16-bit types, a fused LayerNorm or a norm over 16-bit x
  // other than bf16) runs as M/4 chunks of 4 rows
  uint32_t Mk = a->M, chunks = 1;
  {
    const uint64_t xlds = (uint64_t)a->M * a->K * ((a->xdt == THVM_DT_FP32 || a->wdt == THVM_DT_FP32) ? 4 : 2);
    const bool mfma_norm = !a->norm || (a->norm == 1 && a->xdt == THVM_DT_BF16 && a->norm_w);
    const bool mfma_types = mfma_norm && a->K % 64 == 0 &&
        ((a->wdt == THVM_DT_FP16 && a->xdt == THVM_DT_FP16) || (a->wdt == THVM_DT_BF16 && a->xdt == THVM_DT_BF16) ||
         (a->wdt == THVM_DT_FP8E4M3 && (a->xdt == THVM_DT_BF16 || a->xdt == THVM_DT_FP16)));
    const bool mfma = a->tune_path == 2 || (a->tune_path == 0 && mfma_types && (a->M > 4 || xlds > 160 * 1024));
    if (mfma) return thvm_k_gemm_mfma(a, s, err, errlen);
    if (a->wtiled) {
      snprintf(err, errlen, "gemv: tiled weights run on the MFMA path only (M > 4, 16-bit x, K %% 64 == 0)");
      return -1;
    }
    const uint32_t nw_norm = waves < 8 ? waves : 8;   // the norm runs on at most 512 threads
    if (a->norm && !xsum && a->K > (uint64_t)XREG * 64 * nw_norm) {
      snprintf(err, errlen, "gemv: fused norm needs K <= %u for %u waves", XREG * 64 * nw_norm, waves);
      return -1;
    }
    if (a->M > 4) {
      if (a->M % 4 || a->epi == THVM_EPI_QKV || a->epi == THVM_EPI_QKV_ROPE) {
        snprintf(err, errlen, "gemv: M=%u rows of these dtypes run in chunks of 4: M must be a multiple "
                 "of 4 and the epilogue not a KV append", a->M);
        return -1;
      }
      Mk = 4;
      chunks = a->M / 4;
    }
  }
  // two rows per wave where a row fills at most half a batch of chunks (half
  // the lanes would idle) over many rows per wave: measured on gfx950 at the
  // C5 LM head (102400 x 2048 fp8), 53.5 -> 38.9 us.  A row's lanes and chunk
  // order are unchanged, so the sums are bit-identical.  (One-shot GEMVs of
  // the same rows measured no gain.)
  if (!a->tune_r && R == 1 && a->N % 2 == 0 && a->N >= 32768 && a->M <= 4 &&
      (uint64_t)a->K * wsz / 16 <= 128) {
    R = 2;
  }
  // four x rows over long weight rows (>= 768 chunks): two rows per wave share
  // each x read from LDS, which binds at M = 4 (measured on gfx950 at the C4
  // down shape, 14336-wide fp8 rows: 24.7 -> 22.6 us); bit-identical sums
  if (!a->tune_r && R == 1 && Mk == 4 && a->N % 2 == 0 && (uint64_t)a->K * wsz / 16 >= 768) R = 2;
  if (a->tune_r) {
    if (a->tune_r != 1 && a->tune_r != 2) { snprintf(err, errlen, "gemv: r must be 1 or 2"); return -1; }
    if ((pairs && a->tune_r == 1) || a->N % a->tune_r) { snprintf(err, errlen, "gemv: r=%u does not tile N/epilogue", a->tune_r); return -1; }
    R = (int)a->tune_r;
  }
  // 16-byte chunks per lane in flight: 4 (tune_u = 8 doubles them).  With
  // the weight loads unguarded, so that a wave waits only for the batch it
  // consumes while the next one is in flight, 4 beats 8 also on long rows
  // (measured on gfx950 at the C4 down projection, K = 14336 fp8: 12.0
  // against 12.6 us; before, when every wait drained all loads, 8 had won,
  // 13.9 against 14.4); 8 would leave half the lanes idle on 256-chunk rows
  int U = a->tune_u ? (int)a->tune_u : 4;
  if (U != 4 && U != 8) { snprintf(err, errlen, "gemv: u must be 4 or 8"); return -1; }
  uint32_t xsz = (a->xdt == THVM_DT_FP32 || a->wdt == THVM_DT_FP32) ? 4 : 2;
  uint64_t lds = (uint64_t)Mk * a->K * xsz + (xsum ? 16 : 0);   // (summed x: a spare word after the row)
  if (lds > 160 * 1024) {
    snprintf(err, errlen, "gemv: M*K=%llu x elements exceed LDS (use the MFMA GEMM)",
             (unsigned long long)Mk * a->K);
    return -1;
  }
  gemv_fn f = nullptr;
  switch (a->wdt) {
    case THVM_DT_FP32: f = pick_x<WT_F32>(a->xdt, Mk, R, U); break;
    case THVM_DT_FP16: f = pick_x<WT_F16>(a->xdt, Mk, R, U); break;
    case THVM_DT_BF16: f = pick_x<WT_BF16>(a->xdt, Mk, R, U, xsum); break;
    case THVM_DT_FP8E4M3: f = pick_x<WT_FP8>(a->xdt, Mk, R, U, xsum); break;
  }
  if (!f) { snprintf(err, errlen, "gemv: no kernel instance (R=%d U=%d)", R, U); return -1; }
  uint32_t Gr = (a->N + R - 1) / R;
  // 16 waves per block for a single x row whose weight rows are exactly one
  // batch of chunks (every lane busy), when 8-wave blocks would put more than
  // one block on some CUs and 16-wave blocks fit one per CU: the x staging
  // (and a fused norm) then runs once per 16 waves, on every CU alike.
  // Measured on gfx950 at the C4 shapes (K = 4096 fp8): qkv 10.6 -> 9.6 us,
  // o 6.8 -> 6.6 us.  Long rows (C4 down, U = 8: 14.0 -> 15.3 us) and rows
  // that leave lanes idle (C3 K = 1600 fp16, C1 K = 768 f32: slower steps)
  // keep 8.
  // The wave count is the one that makes the grid exactly one block per CU
  // (ceil(Gr / 256), 9..16 waves): C4 qkv's 3072 row pairs take 12-wave
  // blocks, 256 of them, where 16-wave blocks had left 64 CUs idle (192
  // blocks) and so read a third more bytes per busy CU.
  if (!a->tune_waves && Mk == 1 && chunks == 1 && (uint64_t)a->K * wsz / 16 == 64u * (uint32_t)U &&
      (Gr + 7) / 8 > 256 && (Gr + 15) / 16 <= 256) {
    waves = (Gr + 255) / 256;
  }
  if (xsum && a->K > 2u * GEMV_SQ * 64u * waves) {   // the staging's element pairs per thread
    snprintf(err, errlen, "gemv: norm=3 needs K <= %u at %u waves per block", 2u * GEMV_SQ * 64u * waves, waves);
    return -1;
  }
  uint32_t need = (Gr + waves - 1) / waves;
  uint32_t grid = need;
  if (a->tune_blocks) {
    grid = a->tune_blocks < need ? a->tune_blocks : need;
  } else {
    // blocks resident per CU bounded by LDS (160 KiB) and 32 waves; beyond
    // 2 blocks of 8 waves per CU the grid-stride loop is as fast
    uint32_t per_cu = (uint32_t)((160u * 1024u) / (lds ? lds : 1));
    uint32_t wcap = 32u / waves;
    if (per_cu > wcap) per_cu = wcap;
    if (per_cu > 2) per_cu = 2;
    if (per_cu < 1) per_cu = 1;
    uint32_t cap = 256u * per_cu;
    if (grid > cap) grid = cap;
  }
  if (lds > 64 * 1024) {
    hipError_t e = hipFuncSetAttribute((const void *)f,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) {
      snprintf(err, errlen, "gemv: hipFuncSetAttribute: %s", hipGetErrorString(e));
      return -1;
    }
  }
  thvm_launch(true, true, f, dim3(grid, chunks), dim3(64 * waves), (uint32_t)lds, s, *a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    snprintf(err, errlen, "gemv launch: %s", hipGetErrorString(e));
    return -1;
  }
  return 0;
}
