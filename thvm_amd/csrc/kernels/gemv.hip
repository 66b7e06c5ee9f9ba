// gemv.hip -- bandwidth-bound decode projection y[m,n] = sum_k x[m,k] W[n,k]
// for small M (1..4), W in f32 / fp16 / bf16 / fp8-e4m3 (+ per-row f32 scale),
// fp32 accumulation, with an optional fused RMSNorm / LayerNorm prologue on x
// and fused epilogues (residual, SwiGLU, GELU, q/k RoPE + KV-cache append).
//
// Replaces the reference's two-phase split-K GEMV + fold kernels
// (bench/dsv2_decode_bench.c:1043-1125 src_gemv/src_gred, and the folds fused
// into gred_q :435-485, kv_prep :487-556, gred_o_rms :558-611, gred_down
// :613-636), its fused RMSNorm (src_rms :397-433) and the renderer's
// GROUP_REDUCE matvec (src/codegen/hand_opts.c:413-470).  Design for gfx950:
//   * W is [N, K] with K contiguous; one wave64 owns R consecutive rows and
//     streams them with 128-bit loads (lane l takes 16-byte chunks l, l+64, ..),
//     U chunks per row in flight per lane before any arithmetic;
//   * the first batch of weight loads is issued BEFORE x is staged, so the x
//     staging (and the fused norm's block reduction) hides under HBM latency,
//     and the next batch is prefetched while the current one is consumed;
//   * x (M rows) is staged once per block into LDS in its storage type
//     (bf16/fp16 as 16-bit, f32 as f32), chunk-swizzled so the 64 lanes'
//     16-byte LDS reads hit distinct banks; a fused norm writes the normalised
//     row there already rounded to the activation dtype, exactly as the
//     separate norm kernel would store it;
//   * fp8 decodes with v_cvt_pk_f32_fp8 (OCP e4m3, exact), the per-row scale
//     is applied once after the reduction;
//   * the K reduction ends in a DPP wave reduction (fixed order,
//     deterministic): no partial buffer and no second fold kernel.
#include "dev_common.h"
#include "../kern_api.h"
#include "launch.h"
#include "epilogue.h"
#include <stdio.h>

enum { WT_F32 = 0, WT_F16 = 1, WT_BF16 = 2, WT_FP8 = 3 };
enum { XT_BF16 = 0, XT_F16 = 1, XT_F32 = 2 };

template <int WT> struct WTr;
template <> struct WTr<WT_F32>  { static constexpr int E = 4;  };
template <> struct WTr<WT_F16>  { static constexpr int E = 8;  };
template <> struct WTr<WT_BF16> { static constexpr int E = 8;  };
template <> struct WTr<WT_FP8>  { static constexpr int E = 16; };

// decode the 4 elements of quad j of a 16-byte weight chunk
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

// ---- LDS x layout -----------------------------------------------------------
// 16-bit x: element e of row m lives at halfword  m*K + ((e%E)/8 * C + e/E)*8 + e%8
// f32 x:    element e of row m lives at float     m*K + ((e%E)/4 * C + e/E)*4 + e%4
// (C = K/E chunks per row): the 8 (or 4) elements a lane needs for one quad
// pair are one aligned 16-byte LDS word, and lanes c, c+1 read adjacent words.
template <int XT> struct XTr;
template <> struct XTr<XT_BF16> { static constexpr int B = 2, G = 8; };
template <> struct XTr<XT_F16>  { static constexpr int B = 2, G = 8; };
template <> struct XTr<XT_F32>  { static constexpr int B = 4, G = 4; };

template <int XT, int E>
__device__ __forceinline__ uint32_t xs_index(uint32_t K, uint32_t C, uint32_t m, uint32_t e) {
  constexpr int G = XTr<XT>::G;
  const uint32_t c = e / E, r = e - c * E;
  return m * K + ((r / G) * C + c) * G + (r % G);
}

// 8 x elements of a 16-bit group -> floats
template <int XT>
__device__ __forceinline__ void x8_decode(const uint4 &q, float o[8]) {
  uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
  for (int i = 0; i < 4; i++) {
    if (XT == XT_BF16) {
      o[2 * i] = __uint_as_float(w[i] << 16);
      o[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    } else {
      o[2 * i] = h2f((f16_t)(w[i] & 0xffffu));
      o[2 * i + 1] = h2f((f16_t)(w[i] >> 16));
    }
  }
}

template <int XT>
__device__ __forceinline__ void xs_store(void *xs, uint32_t idx, float v) {
  if (XT == XT_BF16) ((bf16_t *)xs)[idx] = f2bf(v);
  else if (XT == XT_F16) ((f16_t *)xs)[idx] = f2h(v);
  else ((float *)xs)[idx] = v;
}

__device__ __forceinline__ float block_sum_g(float v, float *red, int nwaves) {
  float w = wave_sum(v);
  __syncthreads();
  if (lane_id() == 0) red[threadIdx.x >> 6] = w;
  __syncthreads();
  float t = 0.0f;
  for (int i = 0; i < nwaves; i++) t += red[i];
  return t;
}

#define GEMV_MAX_WAVES 16
#define XREG 16   /* x elements per thread kept in registers by the staging */

// the output stage of one row group (one lane, wave-uniform values)
// input x dtype (compile time): vector loads of 16 bytes
enum { XD_BF16 = 0, XD_F16 = 1, XD_F32 = 2 };
template <int XD> struct XDr { static constexpr int VE = XD == XD_F32 ? 4 : 8, B = XD == XD_F32 ? 4 : 2; };

template <int XD>
__device__ __forceinline__ void xvec(const void *x, uint64_t e, float *o) {
  const uint4 q = ld16((const char *)x + e * XDr<XD>::B);
  const uint32_t w[4] = {q.x, q.y, q.z, q.w};
  if (XD == XD_F32) {
#pragma unroll
    for (int i = 0; i < 4; i++) o[i] = __uint_as_float(w[i]);
  } else {
#pragma unroll
    for (int i = 0; i < 4; i++) {
      if (XD == XD_BF16) {
        o[2 * i] = __uint_as_float(w[i] << 16);
        o[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
      } else {
        o[2 * i] = h2f((f16_t)(w[i] & 0xffffu));
        o[2 * i + 1] = h2f((f16_t)(w[i] >> 16));
      }
    }
  }
}
template <int XD>
__device__ __forceinline__ float rnd_x(float v) {
  return XD == XD_BF16 ? rbf(v) : XD == XD_F16 ? rh(v) : v;
}

template <int WT, int XD, int M, int R, int U>
__global__ __launch_bounds__(1024) void k_gemv(ThvmGemvArgs a) {
  constexpr int E = WTr<WT>::E;
  // LDS keeps x in its 16-bit storage type unless weights or x are f32
  constexpr int XT = (WT == WT_F32 || XD == XD_F32) ? XT_F32 : (XD == XD_BF16 ? XT_BF16 : XT_F16);
  constexpr int VE = XDr<XD>::VE;
  extern __shared__ __align__(16) unsigned char xs_raw[];
  __shared__ float red[GEMV_MAX_WAVES];
  const uint32_t K = a.K, N = a.N;
  const uint32_t C = K / E;              // 16-byte weight chunks per row
  const int lane = lane_id();
  const int wv = threadIdx.x >> 6;
  const int nw = blockDim.x >> 6;
  const uint32_t G = (N + R - 1) / R;
  const uint64_t rowbytes = (uint64_t)K * (16 / E);
  const char *wb = (const char *)a.w;

  // ---- 1. first weight batch in flight before anything else ----
  uint32_t g = blockIdx.x * nw + wv;
  uint4 wq[R][U];
  auto load_batch = [&](uint32_t gg, uint32_t c0) {
    const uint32_t n0 = gg * R;
#pragma unroll
    for (int r = 0; r < R; r++) {
      const bool rok = gg < G && (n0 + r) < N;
      const char *rp = wb + (uint64_t)(n0 + r) * rowbytes;
#pragma unroll
      for (int u = 0; u < U; u++) {
        const uint32_t c = c0 + u * 64 + lane;
        if (rok && c < C) wq[r][u] = ld_stream16(rp + (uint64_t)c * 16);
        else wq[r][u] = make_uint4(0, 0, 0, 0);
      }
    }
  };
  load_batch(g, 0);

  // ---- 2. stage x into LDS (16-byte loads), with the fused norm if asked ----
  const uint32_t nthr = blockDim.x;
  const uint32_t NVt = K / VE;           // x vectors per row
  for (int m = 0; m < M; m++) {
    const uint64_t xo = (uint64_t)m * a.ldx;
    if (a.norm == 0) {
      for (uint32_t v = threadIdx.x; v < NVt; v += nthr) {
        float f[VE];
        xvec<XD>(a.x, xo + (uint64_t)v * VE, f);
#pragma unroll
        for (int i = 0; i < VE; i++) xs_store<XT>(xs_raw, xs_index<XT, E>(K, C, m, v * VE + i), f[i]);
      }
    } else {
      constexpr int NV = XREG / VE;
      float xv[NV][VE];
#pragma unroll
      for (int j = 0; j < NV; j++) {
        const uint32_t v = threadIdx.x + j * nthr;
        if (v < NVt) xvec<XD>(a.x, xo + (uint64_t)v * VE, xv[j]);
        else {
#pragma unroll
          for (int i = 0; i < VE; i++) xv[j][i] = 0.0f;
        }
      }
      const float invK = 1.0f / (float)K;
      float mean = 0.0f, s1 = 0.0f, s2 = 0.0f;
      if (a.norm == 2) {
#pragma unroll
        for (int j = 0; j < NV; j++)
#pragma unroll
          for (int i = 0; i < VE; i++) s1 += xv[j][i];
        mean = block_sum_g(s1, red, nw) * invK;
      }
#pragma unroll
      for (int j = 0; j < NV; j++) {
        const bool vok = threadIdx.x + j * nthr < NVt;
#pragma unroll
        for (int i = 0; i < VE; i++) {
          const float d = xv[j][i] - mean;
          s2 += vok ? d * d : 0.0f;
        }
      }
      const float inv = 1.0f / sqrtf(block_sum_g(s2, red, nw) * invK + a.norm_eps);
#pragma unroll
      for (int j = 0; j < NV; j++) {
        const uint32_t v = threadIdx.x + j * nthr;
        if (v < NVt) {
          float gw[VE], gb[VE];
#pragma unroll
          for (int i = 0; i < VE; i += 4) {
            float4 t = a.norm_w ? *(const float4 *)(a.norm_w + v * VE + i) : make_float4(1.f, 1.f, 1.f, 1.f);
            gw[i] = t.x; gw[i + 1] = t.y; gw[i + 2] = t.z; gw[i + 3] = t.w;
            float4 u = (a.norm == 2 && a.norm_b) ? *(const float4 *)(a.norm_b + v * VE + i)
                                                 : make_float4(0.f, 0.f, 0.f, 0.f);
            gb[i] = u.x; gb[i + 1] = u.y; gb[i + 2] = u.z; gb[i + 3] = u.w;
          }
#pragma unroll
          for (int i = 0; i < VE; i++) {
            // (x - mean) * inv * w (+ b), the norm kernel's own formula
            float val = (xv[j][i] - mean) * inv;
            if (a.norm_w) val = val * gw[i];
            if (a.norm == 2 && a.norm_b) val = val + gb[i];
            xs_store<XT>(xs_raw, xs_index<XT, E>(K, C, m, v * VE + i), rnd_x<XD>(val));
          }
        }
      }
    }
  }
  __syncthreads();

  // ---- 3. stream the weight rows ----
  // A flat sequence of (row group, chunk batch) steps per wave; two register
  // sets ping-pong so the next batch is in flight while one is consumed (the
  // wait before a consume covers only the older batch's loads).
  const uint32_t NB = (C + 64 * U - 1) / (64 * U);      // batches per row group
  const uint32_t gstride = gridDim.x * nw;
  const uint32_t g0 = g;
  const uint32_t ngw = g0 < G ? (G - 1 - g0) / gstride + 1 : 0;
  const uint32_t T = ngw * NB;
  float acc[R][M];
#pragma unroll
  for (int r = 0; r < R; r++)
#pragma unroll
    for (int m = 0; m < M; m++) acc[r][m] = 0.0f;

  auto consume = [&](const uint4 (&X)[R][U], uint32_t t) {
    const uint32_t gi = t / NB, bi = t - gi * NB;
    const uint32_t c0 = bi * 64 * U;
#pragma unroll
    for (int u = 0; u < U; u++) {
      const uint32_t c = c0 + u * 64 + lane;
      if (c < C) {
        if (XT == XT_F32) {
#pragma unroll
          for (int j = 0; j < E / 4; j++) {
            float4 xv[M];
#pragma unroll
            for (int m = 0; m < M; m++)
              xv[m] = *(const float4 *)((const float *)xs_raw + m * K + (j * C + c) * 4);
#pragma unroll
            for (int r = 0; r < R; r++) {
              float wf[4];
              quad_decode<WT>(X[r][u], j, wf);
#pragma unroll
              for (int m = 0; m < M; m++) {
                acc[r][m] += xv[m].x * wf[0];
                acc[r][m] += xv[m].y * wf[1];
                acc[r][m] += xv[m].z * wf[2];
                acc[r][m] += xv[m].w * wf[3];
              }
            }
          }
        } else {
#pragma unroll
          for (int h = 0; h < (E + 7) / 8; h++) {     // 8-element x groups
            float xf[M][8];
#pragma unroll
            for (int m = 0; m < M; m++) {
              uint4 q = *(const uint4 *)((const uint16_t *)xs_raw + m * K + (h * C + c) * 8);
              x8_decode<XT>(q, xf[m]);
            }
#pragma unroll
            for (int jj = 0; jj < 2 && (h * 2 + jj) < E / 4; jj++) {
              const int j = h * 2 + jj;
#pragma unroll
              for (int r = 0; r < R; r++) {
                float wf[4];
                quad_decode<WT>(X[r][u], j, wf);
#pragma unroll
                for (int m = 0; m < M; m++) {
                  acc[r][m] += xf[m][jj * 4 + 0] * wf[0];
                  acc[r][m] += xf[m][jj * 4 + 1] * wf[1];
                  acc[r][m] += xf[m][jj * 4 + 2] * wf[2];
                  acc[r][m] += xf[m][jj * 4 + 3] * wf[3];
                }
              }
            }
          }
        }
      }
    }
    if (bi == NB - 1) {
      float tot[R][M];
#pragma unroll
      for (int r = 0; r < R; r++)
#pragma unroll
        for (int m = 0; m < M; m++) {
          tot[r][m] = wave_sum(acc[r][m]);
          acc[r][m] = 0.0f;
        }
      if (lane == 0) gemv_epilogue<R, M>(a, (g0 + gi * gstride) * R, tot);
    }
  };
  auto load_step = [&](uint4 (&X)[R][U], uint32_t t) {
    const uint32_t gi = t / NB, bi = t - gi * NB;
    const uint32_t gg = g0 + gi * gstride, n0 = gg * R, c0 = bi * 64 * U;
#pragma unroll
    for (int r = 0; r < R; r++) {
      const bool rok = gg < G && (n0 + r) < N;
      const char *rp = wb + (uint64_t)(n0 + r) * rowbytes;
#pragma unroll
      for (int u = 0; u < U; u++) {
        const uint32_t c = c0 + u * 64 + lane;
        if (rok && c < C) X[r][u] = ld_stream16(rp + (uint64_t)c * 16);
        else X[r][u] = make_uint4(0, 0, 0, 0);
      }
    }
  };
  uint4 wq2[R][U];
  for (uint32_t t = 0; t < T; t += 2) {          // step 0 is already in wq
    if (t + 1 < T) load_step(wq2, t + 1);
    consume(wq, t);
    if (t + 1 >= T) break;
    if (t + 2 < T) load_step(wq, t + 2);
    consume(wq2, t + 1);
  }
}

// -------------------------------------------------------------------------
typedef void (*gemv_fn)(ThvmGemvArgs);

template <int WT, int XD, int R, int U>
static gemv_fn pick_m(uint32_t M) {
  switch (M) {
    case 1: return k_gemv<WT, XD, 1, R, U>;
    case 2: return k_gemv<WT, XD, 2, R, U>;
    case 3: return k_gemv<WT, XD, 3, R, U>;
    case 4: return k_gemv<WT, XD, 4, R, U>;
    default: return nullptr;
  }
}
template <int WT, int XD>
static gemv_fn pick_ru(uint32_t M, int R, int U) {
  if (R == 1) return U == 8 ? pick_m<WT, XD, 1, 8>(M) : pick_m<WT, XD, 1, 4>(M);
  return U == 8 ? pick_m<WT, XD, 2, 8>(M) : pick_m<WT, XD, 2, 4>(M);
}
template <int WT>
static gemv_fn pick_x(uint32_t xdt, uint32_t M, int R, int U) {
  switch (xdt) {
    case THVM_DT_BF16: return pick_ru<WT, XD_BF16>(M, R, U);
    case THVM_DT_FP16: return pick_ru<WT, XD_F16>(M, R, U);
    case THVM_DT_FP32: return pick_ru<WT, XD_F32>(M, R, U);
    default: return nullptr;
  }
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
  {
    const uint32_t xs = a->xdt == THVM_DT_FP32 ? 4 : 2, ve = 16 / xs;
    if (a->K % ve || ((uint64_t)a->ldx * xs) % 16 || ((uintptr_t)a->x & 15) ||
        ((uintptr_t)a->norm_w & 15) || ((uintptr_t)a->norm_b & 15)) {
      snprintf(err, errlen, "gemv: x rows and norm vectors must be 16-byte aligned and K a multiple of %u", ve);
      return -1;
    }
  }
  if (a->norm > 2) { snprintf(err, errlen, "gemv: unknown norm %u", a->norm); return -1; }
  // defaults from the gfx950 sweep over the C4 projection shapes (8 waves per
  // block, one row per wave unless the epilogue pairs rows, U=4, <= 512 blocks)
  uint32_t waves = a->tune_waves ? a->tune_waves : 8;
  if (waves != 1 && waves != 2 && waves != 4 && waves != 8 && waves != 16) {
    snprintf(err, errlen, "gemv: waves per block must be 1,2,4,8 or 16");
    return -1;
  }
  if (a->norm && a->K > (uint64_t)XREG * 64 * waves) {
    snprintf(err, errlen, "gemv: fused norm needs K <= %u for %u waves", XREG * 64 * waves, waves);
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
  {
    const uint64_t xlds = (uint64_t)a->M * a->K * ((a->xdt == THVM_DT_FP32 || a->wdt == THVM_DT_FP32) ? 4 : 2);
    const bool mfma = a->tune_path == 2 || (a->tune_path == 0 && (a->M > 4 || xlds > 160 * 1024));
    if (mfma) return thvm_k_gemm_mfma(a, s, err, errlen);
    if (a->M > 4) { snprintf(err, errlen, "gemv: the GEMV path takes M <= 4 (M=%u)", a->M); return -1; }
  }
  if (a->tune_r) {
    if (a->tune_r != 1 && a->tune_r != 2) { snprintf(err, errlen, "gemv: r must be 1 or 2"); return -1; }
    if ((pairs && a->tune_r == 1) || a->N % a->tune_r) { snprintf(err, errlen, "gemv: r=%u does not tile N/epilogue", a->tune_r); return -1; }
    R = (int)a->tune_r;
  }
  int U = a->tune_u ? (int)a->tune_u : 4;
  if (U != 4 && U != 8) { snprintf(err, errlen, "gemv: u must be 4 or 8"); return -1; }
  uint32_t xsz = (a->xdt == THVM_DT_FP32 || a->wdt == THVM_DT_FP32) ? 4 : 2;
  uint64_t lds = (uint64_t)a->M * a->K * xsz;
  if (lds > 160 * 1024) {
    snprintf(err, errlen, "gemv: M*K=%llu x elements exceed LDS (use the MFMA GEMM)",
             (unsigned long long)a->M * a->K);
    return -1;
  }
  gemv_fn f = nullptr;
  switch (a->wdt) {
    case THVM_DT_FP32: f = pick_x<WT_F32>(a->xdt, a->M, R, U); break;
    case THVM_DT_FP16: f = pick_x<WT_F16>(a->xdt, a->M, R, U); break;
    case THVM_DT_BF16: f = pick_x<WT_BF16>(a->xdt, a->M, R, U); break;
    case THVM_DT_FP8E4M3: f = pick_x<WT_FP8>(a->xdt, a->M, R, U); break;
  }
  if (!f) { snprintf(err, errlen, "gemv: no kernel instance (R=%d U=%d)", R, U); return -1; }
  uint32_t Gr = (a->N + R - 1) / R;
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
  thvm_launch(true, true, f, dim3(grid), dim3(64 * waves), (uint32_t)lds, s, *a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    snprintf(err, errlen, "gemv launch: %s", hipGetErrorString(e));
    return -1;
  }
  return 0;
}
