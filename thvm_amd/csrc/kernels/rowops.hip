// rowops.hip -- row-wise decode ops on gfx950: RMSNorm / LayerNorm, softmax,
// RoPE, embedding gather, greedy argmax, the device position bump, and casts.
//
// Semantics (reference file:line):
//   RMSNorm    y = rnd((x * inv) * w), inv = 1/sqrtf(ss * (1/K) + eps)
//              (bench/dsv2_decode_bench.c:397-433 src_rms; py/thvm/nn.py:211-224)
//   LayerNorm  (x - mean) * rsqrt(var + eps) * w + b, biased variance
//              (src/nn/layernorm.c:1-7)
//   softmax    exp(x - max) * (1 / sum)   (src/nn/softmax.c:1-16)
//   RoPE       interleaved pairs (2j, 2j+1) rotated by cos/sin[pos][j]
//              (bench/dsv2_decode_bench.c:435-485 gred_q pe slice)
//   embed      x = emb[tok] (+ pos_emb[pos])  (:377-395; thvm_gpt2.py:92-95)
//   argmax     lowest index on ties, two passes (:967-1022)
//   len_bump   L += 1 (:1024-1041)
// The reductions are block-wide trees (DPP inside each wave, LDS across the
// 4-16 waves): a fixed order, so results are reproducible run to run, but not
// the reference's serial order -- parity is held to the stated tolerances.
#include "dev_common.h"
#include "../kern_api.h"
#include "launch.h"
#include <stdio.h>

__device__ __forceinline__ float ld_a(const void *p, uint64_t i, uint32_t dt) {
  switch (dt) {
    case THVM_DT_FP32: return ((const float *)p)[i];
    case THVM_DT_BF16: return bf2f(((const bf16_t *)p)[i]);
    case THVM_DT_FP16: return h2f(((const f16_t *)p)[i]);
    case THVM_DT_FP8E4M3: return fp82f(((const uint8_t *)p)[i]);
    default: return 0.0f;
  }
}
__device__ __forceinline__ void st_a(void *p, uint64_t i, uint32_t dt, float v) {
  switch (dt) {
    case THVM_DT_FP32: ((float *)p)[i] = v; break;
    case THVM_DT_BF16: ((bf16_t *)p)[i] = f2bf(v); break;
    case THVM_DT_FP16: ((f16_t *)p)[i] = f2h(v); break;
    case THVM_DT_FP8E4M3: ((uint8_t *)p)[i] = f2fp8_sat(v); break;
    default: break;
  }
}

#define ROW_THREADS 256
#define ROW_WAVES (ROW_THREADS / 64)

// block-wide sum of one float per thread (all threads get the result)
__device__ __forceinline__ float block_sum(float v, float *red) {
  float w = wave_sum(v);
  const int wv = threadIdx.x >> 6;
  __syncthreads();
  if (lane_id() == 0) red[wv] = w;
  __syncthreads();
  float t = 0.0f;
#pragma unroll
  for (int i = 0; i < ROW_WAVES; i++) t += red[i];
  return t;
}
__device__ __forceinline__ float block_max(float v, float *red) {
  float w = wave_max(v);
  const int wv = threadIdx.x >> 6;
  __syncthreads();
  if (lane_id() == 0) red[wv] = w;
  __syncthreads();
  float t = red[0];
#pragma unroll
  for (int i = 1; i < ROW_WAVES; i++) t = fmaxf(t, red[i]);
  return t;
}

// rows of K <= 16*256: every element loaded once into registers, all loads
// issued together
#define NORM_REG 16
// compile-time element access (the runtime switch of ld_a / st_a put every
// load of a thread in its own branch, each waiting for the one before)
template <uint32_t DT>
__device__ __forceinline__ float ld_t(const void *p, uint64_t i) {
  if (DT == THVM_DT_FP32) return ((const float *)p)[i];
  if (DT == THVM_DT_BF16) return bf2f(((const bf16_t *)p)[i]);
  return h2f(((const f16_t *)p)[i]);
}
template <uint32_t DT>
__device__ __forceinline__ void st_t(void *p, uint64_t i, float v) {
  if (DT == THVM_DT_FP32) ((float *)p)[i] = v;
  else if (DT == THVM_DT_BF16) ((bf16_t *)p)[i] = f2bf(v);
  else ((f16_t *)p)[i] = f2h(v);
}
// one row per block, thread t holding elements t, t + 256, ... (up to 16):
// every x, gain and bias load of the thread is issued before any arithmetic
// (clamped indices, the values past K masked afterwards); the sum of squares
// (or of deviations) in element order, then the four-wave block sum
template <uint32_t XT, uint32_t YT>
__global__ __launch_bounds__(ROW_THREADS) void k_norm_reg(ThvmNormArgs a) {
  __shared__ float red[ROW_WAVES];
  const uint32_t m = blockIdx.x;
  const uint64_t xo = (uint64_t)m * a.ldx, yo = (uint64_t)m * a.ldy;
  const float invK = 1.0f / (float)a.K;
  float xv[NORM_REG], wv[NORM_REG], bv[NORM_REG];
#pragma unroll
  for (int i = 0; i < NORM_REG; i++) {
    const uint32_t e = threadIdx.x + i * ROW_THREADS, ec = e < a.K ? e : 0;
    const float x = ld_t<XT>(a.x, xo + ec);
    xv[i] = e < a.K ? x : 0.0f;
    wv[i] = a.w ? a.w[ec] : 1.0f;
    bv[i] = a.layernorm && a.b ? a.b[ec] : 0.0f;
  }
  float mean = 0.0f, s2 = 0.0f;
  if (a.layernorm) {
    float s1 = 0.0f;
#pragma unroll
    for (int i = 0; i < NORM_REG; i++) s1 += xv[i];
    mean = block_sum(s1, red) * invK;
#pragma unroll
    for (int i = 0; i < NORM_REG; i++) {
      const float d = xv[i] - mean;
      s2 += (threadIdx.x + i * ROW_THREADS) < a.K ? d * d : 0.0f;
    }
  } else {
#pragma unroll
    for (int i = 0; i < NORM_REG; i++) s2 += xv[i] * xv[i];
  }
  const float inv = 1.0f / sqrtf(block_sum(s2, red) * invK + a.eps);
#pragma unroll
  for (int i = 0; i < NORM_REG; i++) {
    const uint32_t e = threadIdx.x + i * ROW_THREADS;
    if (e < a.K) {
      float v = (xv[i] - mean) * inv;
      if (a.w) v = v * wv[i];
      if (a.layernorm && a.b) v = v + bv[i];
      st_t<YT>(a.y, yo + e, v);
    }
  }
}
typedef void (*norm_fn)(ThvmNormArgs);
template <uint32_t XT>
static norm_fn norm_pick_y(uint32_t ydt) {
  return ydt == THVM_DT_FP32 ? k_norm_reg<XT, THVM_DT_FP32>
       : ydt == THVM_DT_BF16 ? k_norm_reg<XT, THVM_DT_BF16> : k_norm_reg<XT, THVM_DT_FP16>;
}
static norm_fn norm_pick(uint32_t xdt, uint32_t ydt) {
  return xdt == THVM_DT_FP32 ? norm_pick_y<THVM_DT_FP32>(ydt)
       : xdt == THVM_DT_BF16 ? norm_pick_y<THVM_DT_BF16>(ydt) : norm_pick_y<THVM_DT_FP16>(ydt);
}

__global__ __launch_bounds__(ROW_THREADS) void k_norm(ThvmNormArgs a) {
  __shared__ float red[ROW_WAVES];
  const uint32_t m = blockIdx.x;
  const uint64_t xo = (uint64_t)m * a.ldx, yo = (uint64_t)m * a.ldy;
  const float invK = 1.0f / (float)a.K;
  if (!a.layernorm) {
    float ss = 0.0f;
    for (uint32_t i = threadIdx.x; i < a.K; i += ROW_THREADS) {
      float v = ld_a(a.x, xo + i, a.xdt);
      ss += v * v;
    }
    ss = block_sum(ss, red);
    float inv = 1.0f / sqrtf(ss * invK + a.eps);
    for (uint32_t i = threadIdx.x; i < a.K; i += ROW_THREADS) {
      float v = ld_a(a.x, xo + i, a.xdt) * inv;
      if (a.w) v = v * a.w[i];
      st_a(a.y, yo + i, a.ydt, v);
    }
  } else {
    float s = 0.0f;
    for (uint32_t i = threadIdx.x; i < a.K; i += ROW_THREADS) s += ld_a(a.x, xo + i, a.xdt);
    float mean = block_sum(s, red) * invK;
    float vs = 0.0f;
    for (uint32_t i = threadIdx.x; i < a.K; i += ROW_THREADS) {
      float d = ld_a(a.x, xo + i, a.xdt) - mean;
      vs += d * d;
    }
    float var = block_sum(vs, red) * invK;
    float r = 1.0f / sqrtf(var + a.eps);
    for (uint32_t i = threadIdx.x; i < a.K; i += ROW_THREADS) {
      float v = (ld_a(a.x, xo + i, a.xdt) - mean) * r;
      if (a.w) v = v * a.w[i];
      if (a.b) v = v + a.b[i];
      st_a(a.y, yo + i, a.ydt, v);
    }
  }
}

static int act_dt(uint32_t dt) {
  return dt == THVM_DT_FP32 || dt == THVM_DT_FP16 || dt == THVM_DT_BF16;
}

extern "C" int thvm_k_norm(const ThvmNormArgs *a, hipStream_t s, char *err, int errlen) {
  if (!act_dt(a->xdt) || !act_dt(a->ydt) || a->M == 0 || a->K == 0 || a->ldx < a->K ||
      a->ldy < a->K) {
    snprintf(err, errlen, "norm: bad args M=%u K=%u", a->M, a->K);
    return -1;
  }
  if (a->K <= NORM_REG * ROW_THREADS)
    thvm_launch(true, true, norm_pick(a->xdt, a->ydt), dim3(a->M), dim3(ROW_THREADS), 0, s, *a);
  else
    thvm_launch(true, true, k_norm, dim3(a->M), dim3(ROW_THREADS), 0, s, *a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) { snprintf(err, errlen, "norm launch: %s", hipGetErrorString(e)); return -1; }
  return 0;
}

__global__ __launch_bounds__(ROW_THREADS) void k_softmax(ThvmSoftmaxArgs a) {
  __shared__ float red[ROW_WAVES];
  const uint64_t o = (uint64_t)blockIdx.x * a.K;
  float mx = -INFINITY;
  for (uint32_t i = threadIdx.x; i < a.K; i += ROW_THREADS) mx = fmaxf(mx, ld_a(a.x, o + i, a.xdt));
  mx = block_max(mx, red);
  float s = 0.0f;
  for (uint32_t i = threadIdx.x; i < a.K; i += ROW_THREADS) s += expf(ld_a(a.x, o + i, a.xdt) - mx);
  s = block_sum(s, red);
  float r = 1.0f / s;
  for (uint32_t i = threadIdx.x; i < a.K; i += ROW_THREADS)
    st_a(a.y, o + i, a.ydt, expf(ld_a(a.x, o + i, a.xdt) - mx) * r);
}

// the same softmax with the dtypes at compile time and the row in registers
// (K <= 16 * 256): thread t's elements t, t + 256, ... loaded once, all
// loads issued together, then the max, the sum (element order, the same
// block sum) and the outputs -- the same bits as k_softmax, whose runtime
// dtype switch put each of its 3 K / 256 loads in a branch of its own,
// waiting for the one before (13 us for one 4096-element row)
template <uint32_t XT, uint32_t YT>
__global__ __launch_bounds__(ROW_THREADS) void k_softmax_reg(ThvmSoftmaxArgs a) {
  __shared__ float red[ROW_WAVES];
  const uint64_t o = (uint64_t)blockIdx.x * a.K;
  float xv[NORM_REG];
#pragma unroll
  for (int i = 0; i < NORM_REG; i++) {
    const uint32_t e = threadIdx.x + i * ROW_THREADS, ec = e < a.K ? e : 0;
    const float x = ld_t<XT>(a.x, o + ec);
    xv[i] = e < a.K ? x : -INFINITY;
  }
  float mx = -INFINITY;
#pragma unroll
  for (int i = 0; i < NORM_REG; i++) mx = fmaxf(mx, xv[i]);
  mx = block_max(mx, red);
  float sm = 0.0f;                 // +0 plus the masked +0 terms: the same bits
#pragma unroll
  for (int i = 0; i < NORM_REG; i++) sm += (threadIdx.x + i * ROW_THREADS) < a.K ? expf(xv[i] - mx) : 0.0f;
  sm = block_sum(sm, red);
  const float r = 1.0f / sm;
#pragma unroll
  for (int i = 0; i < NORM_REG; i++) {
    const uint32_t e = threadIdx.x + i * ROW_THREADS;
    if (e < a.K) st_t<YT>(a.y, o + e, expf(xv[i] - mx) * r);
  }
}
typedef void (*softmax_fn)(ThvmSoftmaxArgs);
template <uint32_t XT>
static softmax_fn softmax_pick_y(uint32_t ydt) {
  return ydt == THVM_DT_FP32 ? k_softmax_reg<XT, THVM_DT_FP32>
       : ydt == THVM_DT_BF16 ? k_softmax_reg<XT, THVM_DT_BF16> : k_softmax_reg<XT, THVM_DT_FP16>;
}

extern "C" int thvm_k_softmax(const ThvmSoftmaxArgs *a, hipStream_t s, char *err, int errlen) {
  if (!act_dt(a->xdt) || !act_dt(a->ydt) || a->M == 0 || a->K == 0) {
    snprintf(err, errlen, "softmax: bad args");
    return -1;
  }
  if (a->K <= NORM_REG * ROW_THREADS) {
    const softmax_fn f = a->xdt == THVM_DT_FP32 ? softmax_pick_y<THVM_DT_FP32>(a->ydt)
                       : a->xdt == THVM_DT_BF16 ? softmax_pick_y<THVM_DT_BF16>(a->ydt)
                                                : softmax_pick_y<THVM_DT_FP16>(a->ydt);
    thvm_launch(true, true, f, dim3(a->M), dim3(ROW_THREADS), 0, s, *a);
  } else {
    thvm_launch(true, true, k_softmax, dim3(a->M), dim3(ROW_THREADS), 0, s, *a);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) { snprintf(err, errlen, "softmax launch: %s", hipGetErrorString(e)); return -1; }
  return 0;
}

// ---- RoPE (in place) --------------------------------------------------------
__global__ void k_rope(ThvmRopeArgs a) {
  const uint32_t half = a.hd / 2;
  const uint64_t n = (uint64_t)a.B * a.nh * half;
  const uint64_t t = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= n) return;
  const uint32_t j = (uint32_t)(t % half);
  const uint64_t row = t / half;
  const int32_t pos = a.len[0] - 1;
  if (pos < 0 || (uint32_t)pos >= a.max_seq) return;
  const float c = a.cos_t[(uint64_t)pos * half + j], sn = a.sin_t[(uint64_t)pos * half + j];
  const uint64_t base = row * a.hd + 2 * j;
  float xe = ld_a(a.x, base, a.dt), xo = ld_a(a.x, base + 1, a.dt);
  st_a(a.x, base, a.dt, xe * c - xo * sn);
  st_a(a.x, base + 1, a.dt, xo * c + xe * sn);
}

extern "C" int thvm_k_rope(const ThvmRopeArgs *a, hipStream_t s, char *err, int errlen) {
  if (!act_dt(a->dt) || a->hd == 0 || a->hd % 2) { snprintf(err, errlen, "rope: bad args"); return -1; }
  uint64_t n = (uint64_t)a->B * a->nh * (a->hd / 2);
  if (n == 0) return 0;
  thvm_launch(true, true, k_rope, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, *a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) { snprintf(err, errlen, "rope launch: %s", hipGetErrorString(e)); return -1; }
  return 0;
}

// ---- embedding --------------------------------------------------------------
__global__ void k_embed(ThvmEmbedArgs a) {
  const uint32_t b = blockIdx.y;
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= a.D) return;
  const int32_t t = a.tok[b];
  float v = 0.0f;
  if (t >= 0 && (uint32_t)t < a.V) v = ld_a(a.emb, (uint64_t)t * a.D + i, a.edt);
  if (a.pos_emb) {
    const int32_t p = a.len[0] - 1;
    if (p >= 0 && (uint32_t)p < a.max_seq) v = v + ld_a(a.pos_emb, (uint64_t)p * a.D + i, a.edt);
  }
  st_a(a.x, (uint64_t)b * a.D + i, a.xdt, v);
}

extern "C" int thvm_k_embed(const ThvmEmbedArgs *a, hipStream_t s, char *err, int errlen) {
  if (a->D == 0 || a->B == 0 || !act_dt(a->xdt) || !act_dt(a->edt) ||
      (a->pos_emb && a->len == nullptr)) {
    snprintf(err, errlen, "embed: bad args");
    return -1;
  }
  thvm_launch(true, true, k_embed, dim3((a->D + 255) / 256, a->B), dim3(256), 0, s, *a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) { snprintf(err, errlen, "embed launch: %s", hipGetErrorString(e)); return -1; }
  return 0;
}

// ---- argmax -----------------------------------------------------------------
__device__ __forceinline__ bool am_better(float v, int32_t i, float bv, int32_t bi) {
  return v > bv || (v == bv && i < bi);
}

__global__ __launch_bounds__(256) void k_argmax_part(ThvmArgmaxArgs a) {
  __shared__ float sv[256];
  __shared__ int32_t si[256];
  const uint32_t b = blockIdx.y, blk = blockIdx.x, t = threadIdx.x;
  const uint32_t chunk = (a.V + a.nb - 1) / a.nb;
  const uint64_t lo = (uint64_t)blk * chunk;
  uint64_t hi = lo + chunk;
  if (hi > a.V) hi = a.V;
  const float *lg = a.logits + (uint64_t)b * a.V;
  float bv = -INFINITY;
  int32_t bi = 0x7fffffff;
  for (uint64_t i = lo + t; i < hi; i += 256) {
    float x = lg[i];
    if (am_better(x, (int32_t)i, bv, bi)) { bv = x; bi = (int32_t)i; }
  }
  sv[t] = bv; si[t] = bi;
  __syncthreads();
  for (uint32_t st = 128; st > 0; st >>= 1) {
    if (t < st && am_better(sv[t + st], si[t + st], sv[t], si[t])) {
      sv[t] = sv[t + st]; si[t] = si[t + st];
    }
    __syncthreads();
  }
  if (t == 0) { a.pv[b * a.nb + blk] = sv[0]; a.pi[b * a.nb + blk] = si[0]; }
}

// one wave per batch row: lanes scan the block partials, then a shuffle
// reduction keeps (max value, lowest index)
__global__ void k_argmax_fin(ThvmArgmaxArgs a) {
  const uint32_t b = blockIdx.x;
  const int lane = lane_id();
  float bv = -INFINITY;
  int32_t bi = 0x7fffffff;
  for (uint32_t k = lane; k < a.nb; k += 64) {
    float v = a.pv[b * a.nb + k];
    int32_t i = a.pi[b * a.nb + k];
    if (am_better(v, i, bv, bi)) { bv = v; bi = i; }
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    float ov = __shfl_xor(bv, off);
    int32_t oi = __shfl_xor(bi, off);
    if (am_better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
  }
  if (lane != 0) return;
  a.tok[b] = bi;
  if (a.hist) {
    int32_t L = a.len[0];
    if (L >= 0 && (uint32_t)L < a.hist_stride) a.hist[(uint64_t)b * a.hist_stride + L] = bi;
  }
}

// ---- temperature sampling: id ~ softmax(logits / T), replacing argmax ----
// The draw is exactly specified so that a CPU restatement reproduces every
// id bit for bit (the oracle's or_sample):
//  * sexpf: exp by Cody-Waite reduction (x = k ln2 + r, ln2 split into a
//    20-bit head and a tail) and the degree-8 Taylor polynomial of e^r in
//    Horner form with fused multiply-adds, scaled by ldexpf -- only
//    correctly rounded IEEE operations, so any IEEE machine gets the same
//    bits; arguments below -80 give 0;
//  * z = l * (1/T); chunk k of C = ceil(V/nb) logits: m_k = max z, s_k =
//    the 256 thread sums (stride 256) folded 128, 64, ..., 1 of sexpf(z - m_k);
//  * w_k = s_k * sexpf(m_k - M), M = max m_k; lane j of 64 owns chunks
//    [jP, (j+1)P), P = ceil(nb/64), q_j their sequential sum, S = sum_j q_j;
//  * u in [0,1) from a counter hash of (seed, row, L) -- L the device-resident
//    position, so every replay of a captured step draws afresh; t = u S;
//  * select: the first lane j with q_j > 0 and A_j + q_j > t (A_j the
//    sequential sum before it; else the last lane with q_j > 0), then the
//    same rule over its own chunks; then, inside the chosen chunk, with the
//    threshold (t - base) / sexpf(m_k - M), the same two levels over lanes
//    owning E = ceil(C/64) consecutive logits each.
// No contraction anywhere in this section: every product and sum rounds.
#pragma clang fp contract(off)
__device__ __forceinline__ uint64_t mix64(uint64_t z);
__device__ __forceinline__ float sexpf(float x) {
  if (!(x >= -80.0f)) return 0.0f;
  const float k = rintf(x * 0x1.715476p+0f);
  float r = fmaf(-k, 0x1.62e000p-1f, x);
  r = fmaf(-k, 0x1.0bfbe8p-15f, r);
  float p = 0x1.a01a02p-16f;
  p = fmaf(p, r, 0x1.a01a02p-13f);
  p = fmaf(p, r, 0x1.6c16c2p-10f);
  p = fmaf(p, r, 0x1.111112p-7f);
  p = fmaf(p, r, 0x1.555556p-5f);
  p = fmaf(p, r, 0x1.555556p-3f);
  p = fmaf(p, r, 0x1.0p-1f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  return ldexpf(p, (int)k);
}

__device__ __forceinline__ float sample_u01(uint64_t seed, uint32_t row, int32_t L) {
  const uint64_t h = mix64(mix64(seed ^ mix64((uint64_t)row + 1)) + (uint64_t)(uint32_t)L);
  return (float)(uint32_t)(h >> 40) * (1.0f / 16777216.0f);
}

__global__ __launch_bounds__(256) void k_sample_part(ThvmArgmaxArgs a) {
  __shared__ float sv[256];
  const uint32_t b = blockIdx.y, blk = blockIdx.x, t = threadIdx.x;
  const uint32_t chunk = (a.V + a.nb - 1) / a.nb;
  const uint64_t lo = (uint64_t)blk * chunk;
  uint64_t hi = lo + chunk;
  if (hi > a.V) hi = a.V;
  const float *lg = a.logits + (uint64_t)b * a.V;
  float m = -INFINITY;
  for (uint64_t i = lo + t; i < hi; i += 256) m = fmaxf(m, lg[i] * a.inv_temp);
  sv[t] = m;
  __syncthreads();
  for (uint32_t st = 128; st > 0; st >>= 1) {
    if (t < st) sv[t] = fmaxf(sv[t], sv[t + st]);
    __syncthreads();
  }
  m = sv[0];
  __syncthreads();
  float acc = 0.0f;
  if (m != -INFINITY)
    for (uint64_t i = lo + t; i < hi; i += 256) acc += sexpf(lg[i] * a.inv_temp - m);
  sv[t] = acc;
  __syncthreads();
  for (uint32_t st = 128; st > 0; st >>= 1) {
    if (t < st) sv[t] += sv[t + st];
    __syncthreads();
  }
  if (t == 0) {
    a.pv[b * a.nb + blk] = m;
    ((float *)a.pi)[b * a.nb + blk] = sv[0];
  }
}

__device__ __forceinline__ float rlane(float v, int j) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), j));
}

// The two-level choice over n weights held as lane j's range [jP, (j+1)P):
// q = this lane's sequential sum; returns the chosen index and, in *base,
// the sequential sum of the weights before it.  Every lane returns the same.
template <typename W>
__device__ __forceinline__ int64_t pick2(const W &wt, float q, uint32_t n, uint32_t P, float t,
                                         float *base) {
  float A = 0.0f, Astar = 0.0f;
  int js = -1, jl = -1;
  float Al = 0.0f;
  for (int j = 0; j < 64; j++) {
    const float qj = rlane(q, j);
    if (qj > 0.0f) {
      if (js < 0 && A + qj > t) { js = j; Astar = A; }
      jl = j; Al = A;
    }
    A += qj;
  }
  if (js < 0) { js = jl; Astar = Al; }
  if (js < 0) { *base = 0.0f; return -1; }
  float c = Astar;
  int64_t ks = -1, kl = -1;
  float cl = 0.0f, cs = 0.0f;
  const uint32_t k0 = (uint32_t)js * P, k1 = k0 + P < n ? k0 + P : n;
  for (uint32_t k = k0; k < k1; k++) {
    const float w = wt(k);
    if (w > 0.0f) {
      if (ks < 0 && c + w > t) { ks = k; cs = c; }
      kl = k; cl = c;
    }
    c += w;
  }
  if (ks < 0) { ks = kl; cs = cl; }
  *base = cs;
  return ks;
}

__global__ __launch_bounds__(64) void k_sample_fin(ThvmArgmaxArgs a) {
  const uint32_t b = blockIdx.x, nb = a.nb;
  const int lane = threadIdx.x;
  const float *pv = a.pv + (uint64_t)b * nb;
  const float *ps = (const float *)a.pi + (uint64_t)b * nb;
  float M = -INFINITY;
  for (uint32_t k = lane; k < nb; k += 64) M = fmaxf(M, pv[k]);
  for (int j = 0; j < 64; j++) M = fmaxf(M, rlane(M, j));
  auto wk = [&](uint32_t k) { return pv[k] == -INFINITY ? 0.0f : ps[k] * sexpf(pv[k] - M); };
  const uint32_t P = (nb + 63) / 64;
  float q = 0.0f;
  for (uint32_t k = (uint32_t)lane * P; k < (uint32_t)(lane + 1) * P && k < nb; k++) q += wk(k);
  float S = 0.0f;
  for (int j = 0; j < 64; j++) S += rlane(q, j);
  const int32_t L = a.len ? a.len[0] : 0;
  const float tgt = sample_u01(a.seed, b, L) * S;
  float base;
  const int64_t ks = pick2(wk, q, nb, P, tgt, &base);
  if (ks < 0) return;                              // every weight zero: no finite logit
  const float r = (tgt - base) / sexpf(pv[ks] - M);
  const float mk = pv[ks];
  const uint32_t C = (a.V + nb - 1) / nb;
  const uint64_t lo = (uint64_t)ks * C;
  const uint32_t n = (uint32_t)((lo + C <= a.V ? lo + C : a.V) - lo);
  const float *lg = a.logits + (uint64_t)b * a.V + lo;
  auto ek = [&](uint32_t i) { return sexpf(lg[i] * a.inv_temp - mk); };
  const uint32_t E = (C + 63) / 64;
  float qe = 0.0f;
  for (uint32_t i = (uint32_t)lane * E; i < (uint32_t)(lane + 1) * E && i < n; i++) qe += ek(i);
  float base2;
  const int64_t is = pick2(ek, qe, n, E, r, &base2);
  if (lane != 0 || is < 0) return;
  const int32_t id = (int32_t)(lo + is);
  a.tok[b] = id;
  if (a.hist) {
    if (L >= 0 && (uint32_t)L < a.hist_stride) a.hist[(uint64_t)b * a.hist_stride + L] = id;
  }
}
#pragma clang fp contract(fast)   // back to the HIP default for the rest of the file

extern "C" int thvm_k_argmax(const ThvmArgmaxArgs *a, hipStream_t s, char *err, int errlen) {
  if (a->B == 0 || a->V == 0 || a->nb == 0 || a->nb > a->V || (a->hist && !a->len)) {
    snprintf(err, errlen, "argmax: bad args");
    return -1;
  }
  if (a->inv_temp > 0.0f) {          // temperature sampling
    if (a->nb > 4096 || (a->V + a->nb - 1) / a->nb > 64u * 4096u) {
      snprintf(err, errlen, "sample: nb %u / chunk out of range", a->nb);
      return -1;
    }
    thvm_launch(true, false, k_sample_part, dim3(a->nb, a->B), dim3(256), 0, s, *a);
    thvm_launch(false, true, k_sample_fin, dim3(a->B), dim3(64), 0, s, *a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) { snprintf(err, errlen, "sample launch: %s", hipGetErrorString(e)); return -1; }
    return 0;
  }
  thvm_launch(true, false, k_argmax_part, dim3(a->nb, a->B), dim3(256), 0, s, *a);
  thvm_launch(false, true, k_argmax_fin, dim3(a->B), dim3(64), 0, s, *a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) { snprintf(err, errlen, "argmax launch: %s", hipGetErrorString(e)); return -1; }
  return 0;
}

// ---- pending kernel-timing events of the next launcher call (the backend
// dispatches from one host thread) ----
static hipEvent_t TN_START = nullptr, TN_STOP = nullptr;
extern "C" void thvm_k_time_next(hipEvent_t start, hipEvent_t stop) {
  TN_START = start;
  TN_STOP = stop;
}
extern "C" hipEvent_t thvm_k_take_start(void) {
  hipEvent_t e = TN_START;
  TN_START = nullptr;
  return e;
}
extern "C" hipEvent_t thvm_k_take_stop(void) {
  hipEvent_t e = TN_STOP;
  TN_STOP = nullptr;
  return e;
}

__global__ void k_len_bump(int32_t *len, int32_t d) {
  if (threadIdx.x == 0 && blockIdx.x == 0) len[0] = len[0] + d;
}
extern "C" int thvm_k_len_bump(int32_t *len, int32_t delta, hipStream_t s, char *err, int errlen) {
  thvm_launch(true, true, k_len_bump, dim3(1), dim3(64), 0, s, len, delta);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) { snprintf(err, errlen, "len_bump launch: %s", hipGetErrorString(e)); return -1; }
  return 0;
}

// ---- blind speculative draft / accept (reference draft_prep and
// accept_commit, bench/dsv2_decode_bench.c:1110-1170) ----
// draft: one block; the bigram search over hist[0..P-1] runs strided over
// the 256 threads, each keeping its last (largest) match, then a block max.
__global__ __launch_bounds__(256) void k_spec_draft(int32_t *ca, int32_t *ce, const int32_t *hist,
                                                    const int32_t *len, uint32_t S, uint32_t V,
                                                    uint32_t cap, uint32_t forced) {
  __shared__ int32_t wbest[4];
  const int tid = threadIdx.x;
  const int32_t P = len[0] - 1;
  if (P < 0 || P >= (int32_t)cap) {                // no pending token: all holes
    if (tid < (int)S) { ca[tid] = -1; ce[tid] = 0; }
    return;
  }
  const int32_t pend = hist[P];
  const int32_t ok_pend = pend >= 0 && (uint32_t)pend < V ? pend : 0;
  int32_t best = -1;
  if (!forced && P >= 1) {
    const int32_t a0 = hist[P - 1];
    for (int32_t j = tid; j + 1 < P; j += 256)
      if (hist[j] == a0 && hist[j + 1] == pend) best = j;
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) best = max(best, __shfl_xor(best, off));
  if ((tid & 63) == 0) wbest[tid >> 6] = best;
  __syncthreads();
  best = max(max(wbest[0], wbest[1]), max(wbest[2], wbest[3]));
  if (tid < (int)S) {
    int32_t v;
    if (tid == 0) {
      v = pend;
    } else if (forced) {
      const int32_t i = P + tid;
      v = i < (int32_t)cap ? hist[i] : -1;
    } else {
      const int32_t i = best + 1 + tid;             // best + 2 + t, t = tid - 1
      v = (best >= 0 && i <= P) ? hist[i] : -1;
    }
    if (v < 0 || (uint32_t)v >= V) v = -1;
    ca[tid] = tid == 0 ? pend : v;
    ce[tid] = v >= 0 ? v : ok_pend;
  }
}
// accept: one lane (the commit is a handful of serial compares)
__global__ void k_spec_accept(int32_t *hist, int32_t *len, int32_t *tok, const int32_t *ca,
                              const int32_t *am, uint32_t S, uint32_t cap) {
  if (threadIdx.x != 0 || blockIdx.x != 0) return;
  const int32_t P = len[0] - 1;
  if (P < 0 || P + (int32_t)S >= (int32_t)cap) return;
  uint32_t k = 0;
  while (k + 1 < S && ca[k + 1] >= 0 && ca[k + 1] == am[k]) k++;
  for (uint32_t i = 0; i < k; i++) hist[P + 1 + i] = ca[1 + i];
  hist[P + 1 + k] = am[k];
  if (tok) tok[0] = am[k];
  len[0] = P + (int32_t)k + 2;
}
extern "C" int thvm_k_spec_draft(int32_t *cand_acc, int32_t *cand_emb, const int32_t *hist,
                                 const int32_t *len, uint32_t S, uint32_t V, uint32_t hist_cap,
                                 uint32_t forced, hipStream_t s, char *err, int errlen) {
  if (S < 2 || S > 256 || V == 0 || hist_cap == 0) {
    snprintf(err, errlen, "spec_draft: S=%u must be 2..256, V and hist_cap nonzero", S);
    return -1;
  }
  thvm_launch(true, true, k_spec_draft, dim3(1), dim3(256), 0, s, cand_acc, cand_emb, hist, len, S,
              V, hist_cap, forced);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) { snprintf(err, errlen, "spec_draft launch: %s", hipGetErrorString(e)); return -1; }
  return 0;
}
extern "C" int thvm_k_spec_accept(int32_t *hist, int32_t *len, int32_t *tok, const int32_t *cand_acc,
                                  const int32_t *am, uint32_t S, uint32_t hist_cap, hipStream_t s,
                                  char *err, int errlen) {
  if (S < 2 || hist_cap == 0) {
    snprintf(err, errlen, "spec_accept: S=%u must be >= 2, hist_cap nonzero", S);
    return -1;
  }
  thvm_launch(true, true, k_spec_accept, dim3(1), dim3(64), 0, s, hist, len, tok, cand_acc, am, S,
              hist_cap);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) { snprintf(err, errlen, "spec_accept launch: %s", hipGetErrorString(e)); return -1; }
  return 0;
}

// ---- delay: one wave sleeps a fixed number of s_sleep(127) periods (~8k
// cycles each), so a host can enqueue work behind it; the trip count is the
// only exit condition and is bounded by the launcher ----
__global__ void k_delay(uint32_t n) {
  for (uint32_t i = 0; i < n; i++) __builtin_amdgcn_s_sleep(127);
}
extern "C" int thvm_k_delay(uint32_t n, hipStream_t s, char *err, int errlen) {
  if (n > 200000) { snprintf(err, errlen, "delay: %u periods exceed the 200000 cap", n); return -1; }
  (void)hipGetLastError();   // drop a stale, already handled error
  hipLaunchKernelGGL(k_delay, dim3(1), dim3(64), 0, s, n);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) { snprintf(err, errlen, "delay launch: %s", hipGetErrorString(e)); return -1; }
  return 0;
}

// ---- casts ------------------------------------------------------------------
__global__ void k_cast(void *y, uint32_t ydt, const void *x, uint32_t xdt, uint64_t n) {
  uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  st_a(y, i, ydt, ld_a(x, i, xdt));
}
extern "C" int thvm_k_cast(void *y, uint32_t ydt, const void *x, uint32_t xdt, uint64_t n,
                           hipStream_t s, char *err, int errlen) {
  bool okx = act_dt(xdt) || xdt == THVM_DT_FP8E4M3, oky = act_dt(ydt) || ydt == THVM_DT_FP8E4M3;
  if (!okx || !oky) { snprintf(err, errlen, "cast: unsupported dtypes"); return -1; }
  if (n == 0) return 0;
  (void)hipGetLastError();   // drop a stale, already handled error
  hipLaunchKernelGGL(k_cast, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, y, ydt, x, xdt, n);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) { snprintf(err, errlen, "cast launch: %s", hipGetErrorString(e)); return -1; }
  return 0;
}

// ---- plain copy: n16 16-byte units, read once and written once (the
// reference for HBM traffic counters: FETCH = WRITE = 16*n16 bytes) ----
__global__ __launch_bounds__(256) void k_copy16(uint4 *y, const uint4 *x, uint64_t n16) {
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += stride)
    y[i] = ld_stream16(x + i);
}
extern "C" int thvm_k_copy(void *y, const void *x, uint64_t nbytes, hipStream_t s, char *err,
                           int errlen) {
  if ((nbytes & 15u) || ((uintptr_t)y & 15u) || ((uintptr_t)x & 15u)) {
    snprintf(err, errlen, "copy: pointers and size must be 16-byte aligned");
    return -1;
  }
  uint64_t n16 = nbytes / 16;
  if (n16 == 0) return 0;
  uint64_t blocks = (n16 + 255) / 256;
  if (blocks > 256 * 16) blocks = 256 * 16;
  thvm_launch(true, true, k_copy16, dim3((unsigned)blocks), dim3(256), 0, s, (uint4 *)y,
              (const uint4 *)x, n16);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) { snprintf(err, errlen, "copy launch: %s", hipGetErrorString(e)); return -1; }
  return 0;
}

// ---- zero fill and byte copies usable inside a stream capture ----------------
// (a kernel node instead of a memset / memcpy node).  The 16-byte-aligned
// middle of the range is moved with 16-byte accesses, the unaligned head and
// tail bytewise by the first wave of block 0.
__global__ __launch_bounds__(256) void k_zero_bytes(uint8_t *y, uint64_t n) {
  const uintptr_t p = (uintptr_t)y;
  const uint64_t head = ((16 - (p & 15)) & 15) < n ? ((16 - (p & 15)) & 15) : n;
  const uint64_t n16 = (n - head) / 16, tail0 = head + n16 * 16;
  uint4 *y16 = (uint4 *)(y + head);
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += stride)
    y16[i] = make_uint4(0u, 0u, 0u, 0u);
  if (blockIdx.x == 0 && threadIdx.x < 64) {
    for (uint64_t i = threadIdx.x; i < head; i += 64) y[i] = 0;
    for (uint64_t i = tail0 + threadIdx.x; i < n; i += 64) y[i] = 0;
  }
}
extern "C" int thvm_k_zero(void *y, uint64_t nbytes, hipStream_t s, char *err, int errlen) {
  if (nbytes == 0) return 0;
  uint64_t blocks = (nbytes / 16 + 255) / 256;
  if (blocks < 1) blocks = 1;
  if (blocks > 256 * 16) blocks = 256 * 16;
  thvm_launch(true, true, k_zero_bytes, dim3((unsigned)blocks), dim3(256), 0, s, (uint8_t *)y,
              nbytes);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) { snprintf(err, errlen, "zero launch: %s", hipGetErrorString(e)); return -1; }
  return 0;
}

// Read nbytes (16-byte aligned, a multiple of 16) and fold them into one word
// per block: a read-only sweep that evicts L2 and the Infinity Cache with
// clean lines (the timing of a kernel on cold caches); a fold that hits a
// fixed word lands in sink[blockIdx.x], so the loads are not dead.
__global__ __launch_bounds__(256) void k_touch(const uint4 *x, uint64_t n16, uint32_t *sink) {
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  uint32_t acc = 0;
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += stride) {
    const uint4 v = x[i];                  // plain loads: the lines are allocated in the caches
    acc ^= v.x ^ v.y ^ v.z ^ v.w;
  }
  if (acc == 0x9e3779b9u) sink[blockIdx.x] = acc;   // (keeps the loads live; rarely stores)
}
extern "C" int thvm_k_touch(const void *x, uint64_t nbytes, uint32_t *sink, uint32_t nsink, hipStream_t s,
                            char *err, int errlen) {
  if (((uintptr_t)x & 15) || (nbytes & 15) || nsink == 0) {
    snprintf(err, errlen, "touch: 16-byte aligned range and a sink needed");
    return -1;
  }
  uint64_t blocks = (nbytes / 16 + 255) / 256;
  if (blocks < 1) blocks = 1;
  if (blocks > nsink) blocks = nsink;
  thvm_launch(true, true, k_touch, dim3((unsigned)blocks), dim3(256), 0, s, (const uint4 *)x, nbytes / 16,
              sink);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) { snprintf(err, errlen, "touch launch: %s", hipGetErrorString(e)); return -1; }
  return 0;
}

// y[off + i] = x[i], i < n, with off = base + stride * idx[0] read on the
// device (idx == nullptr: off = base).  An offset whose range does not fit
// in cap bytes writes nothing.  Bytewise: this serves row appends (a few KB)
// and arbitrary alignment; bulk aligned copies use k_copy16.
__global__ __launch_bounds__(256) void k_copy_at(uint8_t *y, uint64_t cap, uint64_t base,
                                                  uint64_t stride, const int32_t *idx,
                                                  const uint8_t *x, uint64_t n) {
  int64_t r = idx ? (int64_t)idx[0] : 0;
  if (r < 0) return;
  const uint64_t off = base + stride * (uint64_t)r;
  if (off > cap || n > cap - off) return;
  const uint64_t step = (uint64_t)gridDim.x * blockDim.x;
  for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += step)
    y[off + i] = x[i];
}
extern "C" int thvm_k_copy_at(void *y, uint64_t cap, uint64_t base, uint64_t stride,
                              const int32_t *idx, const void *x, uint64_t n, hipStream_t s,
                              char *err, int errlen) {
  if (n == 0) return 0;
  if (idx == nullptr && !((base | n | (uintptr_t)y | (uintptr_t)x) & 15) && base + n <= cap)
    return thvm_k_copy((uint8_t *)y + base, x, n, s, err, errlen);
  uint64_t blocks = (n + 255) / 256;
  if (blocks > 1024) blocks = 1024;
  thvm_launch(true, true, k_copy_at, dim3((unsigned)blocks), dim3(256), 0, s, (uint8_t *)y, cap,
              base, stride, idx, (const uint8_t *)x, n);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) { snprintf(err, errlen, "copy_at launch: %s", hipGetErrorString(e)); return -1; }
  return 0;
}

// ---- synthetic data ---------------------------------------------------------
// splitmix64 finaliser over (seed, tag, counter): a counter-based generator,
// so any element is reproducible alone.  Box-Muller on a pair of 24-bit
// uniforms gives N(0, 1).
__device__ __forceinline__ uint64_t mix64(uint64_t z) {
  z += 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}
__device__ __forceinline__ float normal_at(uint64_t seed, uint64_t tag, uint64_t idx) {
  uint64_t h = mix64(mix64(seed ^ mix64(tag)) + (idx >> 1));
  float u1 = ((float)(uint32_t)(h >> 40) + 1.0f) * (1.0f / 16777216.0f);   // (0,1]
  float u2 = (float)(uint32_t)(h & 0xffffffu) * (1.0f / 16777216.0f);      // [0,1)
  float r = sqrtf(-2.0f * logf(u1));
  float th = 6.283185307179586f * u2;
  return r * ((idx & 1) ? sinf(th) : cosf(th));
}

__global__ void k_fill_normal(void *dst, uint32_t dt, uint64_t n, uint64_t seed, uint64_t tag,
                              float mean, float std) {
  uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (; i < n; i += stride) st_a(dst, i, dt, mean + std * normal_at(seed, tag, i));
}
extern "C" int thvm_k_fill_normal(void *dst, uint32_t dt, uint64_t n, uint64_t seed, uint64_t tag,
                                  float mean, float std, hipStream_t s, char *err, int errlen) {
  if (!act_dt(dt)) { snprintf(err, errlen, "fill_normal: unsupported dtype %u", dt); return -1; }
  if (n == 0) return 0;
  uint64_t blocks = (n + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  (void)hipGetLastError();   // drop a stale, already handled error
  hipLaunchKernelGGL(k_fill_normal, dim3((unsigned)blocks), dim3(256), 0, s, dst, dt, n, seed, tag,
                     mean, std);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) { snprintf(err, errlen, "fill launch: %s", hipGetErrorString(e)); return -1; }
  return 0;
}

__global__ __launch_bounds__(256) void k_fill_fp8_rows(uint8_t *q, float *scale, uint32_t rows,
                                                       uint32_t cols, uint64_t seed, uint64_t tag,
                                                       float std) {
  __shared__ float red[4];
  for (uint32_t r = blockIdx.x; r < rows; r += gridDim.x) {
    const uint64_t base = (uint64_t)r * cols;
    float mx = 0.0f;
    for (uint32_t c = threadIdx.x; c < cols; c += 256)
      mx = fmaxf(mx, fabsf(std * normal_at(seed, tag, base + c)));
    // block max
    float w = wave_max(mx);
    __syncthreads();
    if (lane_id() == 0) red[threadIdx.x >> 6] = w;
    __syncthreads();
    float am = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    float sc = am > 0.0f ? am / 448.0f : 1.0f;
    if (threadIdx.x == 0) scale[r] = sc;
    for (uint32_t c = threadIdx.x; c < cols; c += 256)
      q[base + c] = f2fp8_sat((std * normal_at(seed, tag, base + c)) / sc);
    __syncthreads();
  }
}
extern "C" int thvm_k_fill_fp8_rows(uint8_t *q, float *scale, uint32_t rows, uint32_t cols,
                                    uint64_t seed, uint64_t tag, float std, hipStream_t s,
                                    char *err, int errlen) {
  if (rows == 0 || cols == 0) return 0;
  uint32_t blocks = rows < 8192 ? rows : 8192;
  (void)hipGetLastError();   // drop a stale, already handled error
  hipLaunchKernelGGL(k_fill_fp8_rows, dim3(blocks), dim3(256), 0, s, q, scale, rows, cols, seed,
                     tag, std);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) { snprintf(err, errlen, "fill_fp8 launch: %s", hipGetErrorString(e)); return -1; }
  return 0;
}

// Per-row weight-only fp8 quantisation of a loaded checkpoint matrix x
// [rows][cols] (f32 / bf16 / fp16): scale[r] = absmax_r / 448 (1 for an
// all-zero row), q = e4m3_sat(x / scale) -- the scheme the synthetic fp8
// weights use, so a converted checkpoint feeds the same kernels.
__global__ __launch_bounds__(256) void k_quant_fp8_rows(uint8_t *q, float *scale, const void *x,
                                                        uint32_t xdt, uint32_t rows, uint32_t cols) {
  __shared__ float red[4];
  for (uint32_t r = blockIdx.x; r < rows; r += gridDim.x) {
    const uint64_t base = (uint64_t)r * cols;
    float mx = 0.0f;
    for (uint32_t c = threadIdx.x; c < cols; c += 256) mx = fmaxf(mx, fabsf(ld_a(x, base + c, xdt)));
    float w = wave_max(mx);
    __syncthreads();
    if (lane_id() == 0) red[threadIdx.x >> 6] = w;
    __syncthreads();
    const float am = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    const float sc = am > 0.0f ? am / 448.0f : 1.0f;
    if (threadIdx.x == 0) scale[r] = sc;
    for (uint32_t c = threadIdx.x; c < cols; c += 256) q[base + c] = f2fp8_sat(ld_a(x, base + c, xdt) / sc);
    __syncthreads();
  }
}
extern "C" int thvm_k_quant_fp8_rows(uint8_t *q, float *scale, const void *x, uint32_t xdt,
                                     uint32_t rows, uint32_t cols, hipStream_t s, char *err,
                                     int errlen) {
  if (xdt != THVM_DT_FP32 && xdt != THVM_DT_BF16 && xdt != THVM_DT_FP16) {
    snprintf(err, errlen, "quant_fp8: source dtype must be f32 / bf16 / fp16");
    return -1;
  }
  if (rows == 0 || cols == 0) return 0;
  const uint32_t blocks = rows < 8192 ? rows : 8192;
  thvm_launch(true, true, k_quant_fp8_rows, dim3(blocks), dim3(256), 0, s, q, scale, x, xdt, rows, cols);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) { snprintf(err, errlen, "quant_fp8 launch: %s", hipGetErrorString(e)); return -1; }
  return 0;
}

__global__ void k_fill_cache(void *cache, uint32_t dt, uint32_t B, uint32_t Hkv, uint32_t max_seq,
                             uint32_t hd, uint32_t ctx, uint64_t seed, uint64_t tag) {
  // element (b, h, p, d) with p < ctx; the counter is the flat cache index
  const uint64_t n = (uint64_t)B * Hkv * ctx * hd;
  const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
  for (uint64_t t = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; t < n; t += stride) {
    uint32_t d = (uint32_t)(t % hd);
    uint64_t r = t / hd;
    uint32_t p = (uint32_t)(r % ctx);
    uint64_t bh = r / ctx;
    uint64_t idx = (bh * max_seq + p) * hd + d;
    st_a(cache, idx, dt, normal_at(seed, tag, idx));
  }
}
extern "C" int thvm_k_fill_cache(void *cache, uint32_t dt, uint32_t B, uint32_t Hkv,
                                 uint32_t max_seq, uint32_t hd, uint32_t ctx, uint64_t seed,
                                 uint64_t tag, hipStream_t s, char *err, int errlen) {
  if (!act_dt(dt) || ctx > max_seq) { snprintf(err, errlen, "fill_cache: bad args"); return -1; }
  uint64_t n = (uint64_t)B * Hkv * ctx * hd;
  if (n == 0) return 0;
  uint64_t blocks = (n + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  (void)hipGetLastError();   // drop a stale, already handled error
  hipLaunchKernelGGL(k_fill_cache, dim3((unsigned)blocks), dim3(256), 0, s, cache, dt, B, Hkv,
                     max_seq, hd, ctx, seed, tag);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) { snprintf(err, errlen, "fill_cache launch: %s", hipGetErrorString(e)); return -1; }
  return 0;
}
