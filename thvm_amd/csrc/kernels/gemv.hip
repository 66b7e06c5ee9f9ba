// gemv.hip -- bandwidth-bound decode projection y[m,n] = sum_k x[m,k] W[n,k]
// for small M (1..4), W in f32 / fp16 / bf16 / fp8-e4m3 (+ per-row f32 scale),
// fp32 accumulation, with fused epilogues (residual, SwiGLU, GELU, q/k RoPE +
// KV-cache append).
//
// Replaces the reference's two-phase split-K GEMV + fold kernels
// (bench/dsv2_decode_bench.c:1043-1125 src_gemv/src_gred, and the folds fused
// into gred_q :435-485, kv_prep :487-556, gred_o_rms :558-611, gred_down
// :613-636) and the renderer's GROUP_REDUCE matvec (src/codegen/hand_opts.c:
// 413-470).  Design for gfx950 instead of a translation:
//   * W is [N, K] with K contiguous; one wave64 owns R consecutive rows and
//     streams them with 128-bit loads (lane l takes 16-byte chunks l, l+64, ..),
//     U chunks per row in flight per lane before any arithmetic;
//   * x (M rows) is staged once per block into LDS as f32, quad-swizzled so the
//     64 lanes' 16-byte reads hit distinct banks;
//   * fp8 decodes with v_cvt_pk_f32_fp8 (OCP e4m3, exact), scale applied once
//     per row after the reduction;
//   * the K-reduction ends in a DPP wave reduction (fixed order, deterministic),
//     so no partial buffer and no second fold kernel exist.
#include "dev_common.h"
#include "../kern_api.h"
#include <stdio.h>

enum { WT_F32 = 0, WT_F16 = 1, WT_BF16 = 2, WT_FP8 = 3 };

template <int WT> struct WTr;
template <> struct WTr<WT_F32>  { static constexpr int E = 4;  };
template <> struct WTr<WT_F16>  { static constexpr int E = 8;  };
template <> struct WTr<WT_BF16> { static constexpr int E = 8;  };
template <> struct WTr<WT_FP8>  { static constexpr int E = 16; };

// decode the 4 elements of quad j of a 16-byte chunk
template <int WT>
__device__ __forceinline__ void quad_decode(const uint4 &q, int j, float o[4]);

template <>
__device__ __forceinline__ void quad_decode<WT_FP8>(const uint4 &q, int j, float o[4]) {
  uint32_t w = j == 0 ? q.x : j == 1 ? q.y : j == 2 ? q.z : q.w;
  fp8x4_to_f32(w, o);
}
template <>
__device__ __forceinline__ void quad_decode<WT_F16>(const uint4 &q, int j, float o[4]) {
  uint32_t a = j == 0 ? q.x : q.z, b = j == 0 ? q.y : q.w;
  o[0] = h2f((f16_t)(a & 0xffffu)); o[1] = h2f((f16_t)(a >> 16));
  o[2] = h2f((f16_t)(b & 0xffffu)); o[3] = h2f((f16_t)(b >> 16));
}
template <>
__device__ __forceinline__ void quad_decode<WT_BF16>(const uint4 &q, int j, float o[4]) {
  uint32_t a = j == 0 ? q.x : q.z, b = j == 0 ? q.y : q.w;
  o[0] = __uint_as_float(a << 16); o[1] = __uint_as_float(a & 0xffff0000u);
  o[2] = __uint_as_float(b << 16); o[3] = __uint_as_float(b & 0xffff0000u);
}
template <>
__device__ __forceinline__ void quad_decode<WT_F32>(const uint4 &q, int j, float o[4]) {
  (void)j;
  o[0] = __uint_as_float(q.x); o[1] = __uint_as_float(q.y);
  o[2] = __uint_as_float(q.z); o[3] = __uint_as_float(q.w);
}

__device__ __forceinline__ float ld_any(const void *p, uint64_t i, uint32_t dt) {
  switch (dt) {
    case THVM_DT_FP32: return ((const float *)p)[i];
    case THVM_DT_BF16: return bf2f(((const bf16_t *)p)[i]);
    case THVM_DT_FP16: return h2f(((const f16_t *)p)[i]);
    default: return 0.0f;
  }
}
__device__ __forceinline__ void st_any(void *p, uint64_t i, uint32_t dt, float v) {
  switch (dt) {
    case THVM_DT_FP32: ((float *)p)[i] = v; break;
    case THVM_DT_BF16: ((bf16_t *)p)[i] = f2bf(v); break;
    case THVM_DT_FP16: ((f16_t *)p)[i] = f2h(v); break;
    default: break;
  }
}
__device__ __forceinline__ float rnd_any(float v, uint32_t dt) {
  return dt == THVM_DT_BF16 ? rbf(v) : dt == THVM_DT_FP16 ? rh(v) : v;
}

#define GEMV_WAVES 4
#define GEMV_THREADS (GEMV_WAVES * 64)

template <int WT, int M, int R, int U>
__global__ __launch_bounds__(GEMV_THREADS) void k_gemv(ThvmGemvArgs a) {
  constexpr int E = WTr<WT>::E;
  extern __shared__ float xs[];          // [M][K] f32, quad-swizzled
  const uint32_t K = a.K, N = a.N;
  const uint32_t C = K / E;              // 16-byte chunks per row
  const int lane = lane_id();
  const int wv = threadIdx.x >> 6;

  // ---- stage x into LDS: element k of row m at m*K + ((k%E)/4*C + k/E)*4 + k%4
  for (uint32_t e = threadIdx.x; e < (uint32_t)M * K; e += GEMV_THREADS) {
    uint32_t m = e / K, k = e - m * K;
    uint32_t c = k / E, r = k - c * E;
    float v = ld_any(a.x, (uint64_t)m * a.ldx + k, a.xdt);
    xs[m * K + ((r >> 2) * C + c) * 4 + (r & 3)] = v;
  }
  __syncthreads();

  const uint32_t G = (N + R - 1) / R;
  const uint64_t rowbytes = (uint64_t)K * (16 / E);
  const char *wb = (const char *)a.w;

  for (uint32_t g = blockIdx.x * GEMV_WAVES + wv; g < G; g += gridDim.x * GEMV_WAVES) {
    const uint32_t n0 = g * R;
    float acc[R][M];
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
      for (int m = 0; m < M; m++) acc[r][m] = 0.0f;

    for (uint32_t c0 = 0; c0 < C; c0 += 64 * U) {
      uint4 wq[R][U];
#pragma unroll
      for (int r = 0; r < R; r++) {
        const bool rok = (n0 + r) < N;
        const char *rp = wb + (uint64_t)(n0 + r) * rowbytes;
#pragma unroll
        for (int u = 0; u < U; u++) {
          uint32_t c = c0 + u * 64 + lane;
          if (rok && c < C) wq[r][u] = ld_stream16(rp + (uint64_t)c * 16);
          else wq[r][u] = make_uint4(0, 0, 0, 0);
        }
      }
#pragma unroll
      for (int u = 0; u < U; u++) {
        uint32_t c = c0 + u * 64 + lane;
        if (c < C) {
#pragma unroll
          for (int j = 0; j < E / 4; j++) {
            float4 xv[M];
#pragma unroll
            for (int m = 0; m < M; m++)
              xv[m] = *(const float4 *)&xs[m * K + (j * C + c) * 4];
#pragma unroll
            for (int r = 0; r < R; r++) {
              float wf[4];
              quad_decode<WT>(wq[r][u], j, wf);
#pragma unroll
              for (int m = 0; m < M; m++) {
                acc[r][m] += xv[m].x * wf[0];
                acc[r][m] += xv[m].y * wf[1];
                acc[r][m] += xv[m].z * wf[2];
                acc[r][m] += xv[m].w * wf[3];
              }
            }
          }
        }
      }
    }

    float tot[R][M];
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
      for (int m = 0; m < M; m++) tot[r][m] = wave_sum(acc[r][m]);

    if (lane != 0) continue;
    // ---- epilogue (one lane, wave-uniform values) ----
    float v[R][M];
#pragma unroll
    for (int r = 0; r < R; r++) {
      uint32_t n = n0 + r;
      float s = (a.scale != nullptr && n < N) ? a.scale[n] : 1.0f;
      float bv = (a.bias != nullptr && n < N) ? ld_any(a.bias, n, a.ydt) : 0.0f;
#pragma unroll
      for (int m = 0; m < M; m++) v[r][m] = tot[r][m] * s + bv;
    }
    const uint32_t ydt = a.ydt;
    switch (a.epi) {
      case THVM_EPI_STORE:
#pragma unroll
        for (int r = 0; r < R; r++)
          if (n0 + r < N)
#pragma unroll
            for (int m = 0; m < M; m++)
              st_any(a.y, (uint64_t)m * a.ldy + n0 + r, ydt, v[r][m]);
        break;
      case THVM_EPI_RESID:
#pragma unroll
        for (int r = 0; r < R; r++)
          if (n0 + r < N)
#pragma unroll
            for (int m = 0; m < M; m++) {
              uint64_t i = (uint64_t)m * a.ldy + n0 + r;
              float rv = ld_any(a.res, i, ydt);
              st_any(a.y, i, ydt, rv + rnd_any(v[r][m], ydt));
            }
        break;
      case THVM_EPI_GELU:
#pragma unroll
        for (int r = 0; r < R; r++)
          if (n0 + r < N)
#pragma unroll
            for (int m = 0; m < M; m++)
              st_any(a.y, (uint64_t)m * a.ldy + n0 + r, ydt,
                     gelu_tanh_f(rnd_any(v[r][m], ydt)));
        break;
      case THVM_EPI_SWIGLU:
        if (R == 2 && n0 + 1 < N) {
#pragma unroll
          for (int m = 0; m < M; m++) {
            float gg = rnd_any(v[0][m], ydt), uu = rnd_any(v[R - 1][m], ydt);
            st_any(a.y, (uint64_t)m * a.ldy + n0 / 2, ydt, silu_f(gg) * uu);
          }
        }
        break;
      case THVM_EPI_QKV_ROPE:
      case THVM_EPI_QKV: {
        if (R != 2 || n0 + 1 >= N) break;
        const uint32_t hd = a.head_dim;
        const uint32_t Hq = a.n_heads * hd, Hk = a.n_kv_heads * hd;
        const int32_t pos = a.len[0] - 1;
        if (pos < 0 || (uint32_t)pos >= a.max_seq) break;   // no live row to write
        const bool rope = a.epi == THVM_EPI_QKV_ROPE;
        const uint32_t d = n0 % hd;
        float c = 1.0f, sn = 0.0f;
        if (rope && n0 < Hq + Hk) {
          c = a.rope_cos[(uint64_t)pos * (hd / 2) + d / 2];
          sn = a.rope_sin[(uint64_t)pos * (hd / 2) + d / 2];
        }
#pragma unroll
        for (int m = 0; m < M; m++) {
          float xe = rnd_any(v[0][m], ydt), xo = rnd_any(v[R - 1][m], ydt);
          float oe = xe, oo = xo;
          if (rope && n0 < Hq + Hk) { oe = xe * c - xo * sn; oo = xo * c + xe * sn; }
          if (n0 < Hq) {
            st_any(a.y, (uint64_t)m * a.ldy + n0, ydt, oe);
            st_any(a.y, (uint64_t)m * a.ldy + n0 + 1, ydt, oo);
          } else {
            const bool isk = n0 < Hq + Hk;
            const uint32_t off = isk ? n0 - Hq : n0 - Hq - Hk;
            const uint32_t h = off / hd;
            uint64_t ci = (((uint64_t)m * a.n_kv_heads + h) * a.max_seq + (uint32_t)pos) * hd + d;
            void *cache = isk ? a.kcache : a.vcache;
            st_any(cache, ci, ydt, oe);
            st_any(cache, ci + 1, ydt, oo);
          }
        }
      } break;
      default: break;
    }
  }
}

// -------------------------------------------------------------------------
typedef void (*gemv_fn)(ThvmGemvArgs);

template <int WT, int R>
static gemv_fn pick_m(uint32_t M) {
  switch (M) {
    case 1: return k_gemv<WT, 1, R, 4>;
    case 2: return k_gemv<WT, 2, R, 4>;
    case 3: return k_gemv<WT, 3, R, 4>;
    case 4: return k_gemv<WT, 4, R, 4>;
    default: return nullptr;
  }
}
template <int WT>
static gemv_fn pick_r(uint32_t M, int R) {
  return R == 1 ? pick_m<WT, 1>(M) : pick_m<WT, 2>(M);
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
  if (a->M < 1 || a->M > 4 || a->N == 0 || a->K == 0) {
    snprintf(err, errlen, "gemv: M=%u N=%u K=%u out of range (M in 1..4)", a->M, a->N, a->K);
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
  int R = 1;
  switch (a->epi) {
    case THVM_EPI_STORE: case THVM_EPI_GELU:
      R = (a->N % 2 == 0) ? 2 : 1;
      if (a->ldy < a->N && a->M > 1) { snprintf(err, errlen, "gemv: ldy < N"); return -1; }
      break;
    case THVM_EPI_RESID:
      if (a->res == nullptr) { snprintf(err, errlen, "gemv: residual epilogue without res"); return -1; }
      R = (a->N % 2 == 0) ? 2 : 1;
      break;
    case THVM_EPI_SWIGLU:
      if (a->N % 2) { snprintf(err, errlen, "gemv: swiglu needs even N"); return -1; }
      R = 2;
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
      R = 2;
    } break;
    default:
      snprintf(err, errlen, "gemv: unknown epilogue %u", a->epi);
      return -1;
  }
  uint64_t lds = (uint64_t)a->M * a->K * 4;
  if (lds > 160 * 1024) {
    snprintf(err, errlen, "gemv: M*K=%llu floats exceed LDS (use the MFMA GEMM)",
             (unsigned long long)a->M * a->K);
    return -1;
  }
  gemv_fn f = nullptr;
  switch (a->wdt) {
    case THVM_DT_FP32: f = pick_r<WT_F32>(a->M, R); break;
    case THVM_DT_FP16: f = pick_r<WT_F16>(a->M, R); break;
    case THVM_DT_BF16: f = pick_r<WT_BF16>(a->M, R); break;
    case THVM_DT_FP8E4M3: f = pick_r<WT_FP8>(a->M, R); break;
  }
  if (!f) { snprintf(err, errlen, "gemv: no kernel instance"); return -1; }
  uint32_t G = (a->N + R - 1) / R;
  uint32_t need = (G + GEMV_WAVES - 1) / GEMV_WAVES;
  // blocks resident per CU bounded by LDS (160 KiB) and 8 blocks of 4 waves
  uint32_t per_cu = (uint32_t)((160u * 1024u) / (lds ? lds : 1));
  if (per_cu > 8) per_cu = 8;
  if (per_cu < 1) per_cu = 1;
  uint32_t cap = 256u * per_cu;
  uint32_t grid = need < cap ? need : cap;
  if (lds > 64 * 1024) {
    hipError_t e = hipFuncSetAttribute((const void *)f,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) {
      snprintf(err, errlen, "gemv: hipFuncSetAttribute: %s", hipGetErrorString(e));
      return -1;
    }
  }
  hipLaunchKernelGGL(f, dim3(grid), dim3(GEMV_THREADS), (size_t)lds, s, *a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    snprintf(err, errlen, "gemv launch: %s", hipGetErrorString(e));
    return -1;
  }
  return 0;
}
