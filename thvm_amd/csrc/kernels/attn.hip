// attn.hip -- split-sequence flash-decode attention over a KV cache of
// symbolic (device-resident) length, MHA and GQA.
//
// Replaces the reference decode attention: nn_scaled_dot_product_attention
// (src/nn/scaled_dot_product_attention.c:4-30) rendered as separate matmul /
// softmax / matmul kernels over kvar loops (src/codegen/render_uop.c:5055-5064),
// and the one-block-per-head score kernel that holds a whole row in shared
// memory (bench/dsv2_decode_bench.c:665-725).  Semantics: out[h] = softmax(q_h .
// K^T * scale) V over cache rows [0, L), L read from device memory at run time
// so a captured graph replays at every length (the symbolic-length finding of
// the reference's graph replay, src/jit/capture.c:2715-2731).
//
// gfx950 design:
//   phase 1: grid (Hkv, n_split, B), 256 threads.  A block owns one KV head and
//            CHUNK=64 positions; its 4 waves take 16 positions each.  A K or V
//            row of hd bf16 is hd/8 lanes x 16 bytes, so one wave-wide load
//            covers 64*8/hd rows; every K and V load of the wave is issued
//            before any arithmetic.  All G = H/Hkv query heads of the group reuse
//            the same K/V registers (GQA reuse), scores reduce inside the
//            row-lane group with DPP, each wave keeps (m, l, acc) and the block
//            merges its 4 waves through LDS.  Writes (acc[hd], m, l) per split.
//   phase 2: one block per (b, h) merges the live splits (ceil(L/CHUNK)).
#include "dev_common.h"
#include "../kern_api.h"
#include <stdio.h>

#define ATT_THREADS 256
#define ATT_WAVES 4
#define ATT_CHUNK 64

__device__ __forceinline__ float ldq(const void *p, uint64_t i, uint32_t dt) {
  return dt == THVM_DT_BF16 ? bf2f(((const bf16_t *)p)[i])
       : dt == THVM_DT_FP16 ? h2f(((const f16_t *)p)[i])
       : ((const float *)p)[i];
}

// one 16-byte chunk of cache elements -> floats (ES = element bytes: 2 or 4)
template <int ES>
__device__ __forceinline__ void chunk_f(const uint4 &q, uint32_t dt, float *o) {
  uint32_t w[4] = {q.x, q.y, q.z, q.w};
  if (ES == 4) {
#pragma unroll
    for (int i = 0; i < 4; i++) o[i] = __uint_as_float(w[i]);
  } else {
#pragma unroll
    for (int i = 0; i < 4; i++) {
      if (dt == THVM_DT_BF16) {
        o[2 * i] = __uint_as_float(w[i] << 16);
        o[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
      } else {
        o[2 * i] = h2f((f16_t)(w[i] & 0xffffu));
        o[2 * i + 1] = h2f((f16_t)(w[i] >> 16));
      }
    }
  }
}

// sum over the LPR lanes of a row group (LPR in {8, 16, 32}); all lanes get it
template <int LPR>
__device__ __forceinline__ float group_sum(float v) {
  v += dpp_f<0xB1>(v);
  v += dpp_f<0x4E>(v);
  v += dpp_f<0x141>(v);
  if (LPR >= 16) v += dpp_f<0x140>(v);
  if (LPR == 32) v += __shfl_xor(v, 16);
  return v;
}

template <int HD, int G, int ES>
__global__ __launch_bounds__(ATT_THREADS) void k_attn_split(ThvmAttnArgs a) {
  constexpr int EPL = 16 / ES;           // elements per lane chunk
  constexpr int LPR = HD / EPL;          // lanes per cache row
  constexpr int RPW = 64 / LPR;          // rows per wave-wide load
  constexpr int PPW = ATT_CHUNK / ATT_WAVES;
  constexpr int IT = PPW / RPW;          // loads per wave
  static_assert(LPR >= 8 && LPR <= 32 && IT >= 1, "attention geometry");
  __shared__ float wm[ATT_WAVES][G], wl[ATT_WAVES][G];
  __shared__ float wacc[ATT_WAVES][G][HD];

  const uint32_t kvh = blockIdx.x, split = blockIdx.y, b = blockIdx.z;
  const int32_t L = a.len[0];
  const uint32_t p0 = split * ATT_CHUNK;
  if ((int32_t)p0 >= L) return;          // phase 2 reads only live splits

  const int lane = lane_id(), wv = threadIdx.x >> 6;
  const int rg = lane / LPR, li = lane % LPR;
  const uint32_t d0 = li * EPL;
  const uint64_t cbase = ((uint64_t)b * a.Hkv + kvh) * a.max_seq;
  const char *kb = (const char *)a.kcache, *vb = (const char *)a.vcache;

  // issue every K/V load of this wave first
  uint4 kq[IT], vq[IT];
  bool ok[IT];
#pragma unroll
  for (int it = 0; it < IT; it++) {
    uint32_t j = p0 + wv * PPW + it * RPW + rg;
    ok[it] = (int32_t)j < L && j < a.max_seq;
    uint64_t off = ((cbase + (ok[it] ? j : 0)) * HD + d0) * ES;
    kq[it] = ld_stream16(kb + off);
    vq[it] = ld_stream16(vb + off);
  }
  // query fragment: G heads x EPL dims
  float qf[G][EPL];
#pragma unroll
  for (int g = 0; g < G; g++) {
    uint64_t qo = ((uint64_t)b * a.H + kvh * G + g) * HD + d0;
#pragma unroll
    for (int i = 0; i < EPL; i++) qf[g][i] = ldq(a.q, qo + i, a.qdt);
  }

  float sc[IT][G];
#pragma unroll
  for (int it = 0; it < IT; it++) {
    float kf[EPL];
    chunk_f<ES>(kq[it], a.cdt, kf);
#pragma unroll
    for (int g = 0; g < G; g++) {
      float s = 0.0f;
#pragma unroll
      for (int i = 0; i < EPL; i++) s += qf[g][i] * kf[i];
      s = group_sum<LPR>(s) * a.scale;
      sc[it][g] = ok[it] ? s : -INFINITY;
    }
  }
  float mw[G], lw[G];
#pragma unroll
  for (int g = 0; g < G; g++) {
    float m = sc[0][g];
#pragma unroll
    for (int it = 1; it < IT; it++) m = fmaxf(m, sc[it][g]);
#pragma unroll
    for (int off = LPR; off < 64; off *= 2) m = fmaxf(m, __shfl_xor(m, off));
    mw[g] = m;
  }
  float acc[G][EPL];
#pragma unroll
  for (int g = 0; g < G; g++) {
    lw[g] = 0.0f;
#pragma unroll
    for (int i = 0; i < EPL; i++) acc[g][i] = 0.0f;
  }
#pragma unroll
  for (int it = 0; it < IT; it++) {
    float vf[EPL];
    chunk_f<ES>(vq[it], a.cdt, vf);
#pragma unroll
    for (int g = 0; g < G; g++) {
      float p = (ok[it] && mw[g] != -INFINITY) ? expf(sc[it][g] - mw[g]) : 0.0f;
      lw[g] += p;
#pragma unroll
      for (int i = 0; i < EPL; i++) acc[g][i] += p * vf[i];
    }
  }
  // combine the row groups of the wave (lanes li, li+LPR, ...)
#pragma unroll
  for (int g = 0; g < G; g++) {
#pragma unroll
    for (int off = LPR; off < 64; off *= 2) {
      lw[g] += __shfl_xor(lw[g], off);
#pragma unroll
      for (int i = 0; i < EPL; i++) acc[g][i] += __shfl_xor(acc[g][i], off);
    }
  }
  if (rg == 0) {
#pragma unroll
    for (int g = 0; g < G; g++) {
#pragma unroll
      for (int i = 0; i < EPL; i++) wacc[wv][g][d0 + i] = acc[g][i];
      if (li == 0) { wm[wv][g] = mw[g]; wl[wv][g] = lw[g]; }
    }
  }
  __syncthreads();
  // block merge: thread t handles outputs t, t+256, ... of the G*HD block
  for (int o = threadIdx.x; o < G * HD; o += ATT_THREADS) {
    const int g = o / HD, d = o % HD;
    float M = wm[0][g];
#pragma unroll
    for (int w = 1; w < ATT_WAVES; w++) M = fmaxf(M, wm[w][g]);
    float l = 0.0f, s = 0.0f;
#pragma unroll
    for (int w = 0; w < ATT_WAVES; w++) {
      float f = wm[w][g] == -INFINITY ? 0.0f : expf(wm[w][g] - M);
      l += f * wl[w][g];
      s += f * wacc[w][g][d];
    }
    float *pp = a.part + (((uint64_t)b * a.H + kvh * G + g) * a.n_split + split) * (HD + 2);
    pp[d] = s;
    if (d == 0) { pp[HD] = M; pp[HD + 1] = l; }
  }
}

__global__ void k_attn_combine(ThvmAttnArgs a) {
  const uint32_t bh = blockIdx.x;            // b*H + h
  const int32_t L = a.len[0];
  uint32_t ns = (uint32_t)((L + ATT_CHUNK - 1) / ATT_CHUNK);
  if (ns > a.n_split) ns = a.n_split;
  const float *pp = a.part + (uint64_t)bh * a.n_split * (a.hd + 2);
  for (uint32_t d = threadIdx.x; d < a.hd; d += blockDim.x) {
    float M = -INFINITY;
    for (uint32_t s = 0; s < ns; s++) M = fmaxf(M, pp[s * (a.hd + 2) + a.hd]);
    float l = 0.0f, acc = 0.0f;
    for (uint32_t s = 0; s < ns; s++) {
      const float *q = pp + s * (a.hd + 2);
      float f = q[a.hd] == -INFINITY ? 0.0f : expf(q[a.hd] - M);
      l += f * q[a.hd + 1];
      acc += f * q[d];
    }
    float v = l > 0.0f ? acc / l : 0.0f;
    uint64_t oi = (uint64_t)bh * a.hd + d;
    if (a.odt == THVM_DT_BF16) ((bf16_t *)a.out)[oi] = f2bf(v);
    else if (a.odt == THVM_DT_FP16) ((f16_t *)a.out)[oi] = f2h(v);
    else ((float *)a.out)[oi] = v;
  }
}

typedef void (*attn_fn)(ThvmAttnArgs);
template <int HD, int ES>
static attn_fn attn_pick(uint32_t G) {
  switch (G) {
    case 1: return k_attn_split<HD, 1, ES>;
    case 2: return k_attn_split<HD, 2, ES>;
    case 4: return k_attn_split<HD, 4, ES>;
    case 8: return k_attn_split<HD, 8, ES>;
    default: return nullptr;
  }
}

extern "C" uint64_t thvm_k_attn_part_bytes(uint32_t B, uint32_t H, uint32_t hd, uint32_t n_split) {
  return (uint64_t)B * H * n_split * (hd + 2) * 4;
}

extern "C" int thvm_k_attn_decode(const ThvmAttnArgs *a, hipStream_t s, char *err, int errlen) {
  if (a->H == 0 || a->Hkv == 0 || a->H % a->Hkv || a->B == 0 || a->max_seq == 0) {
    snprintf(err, errlen, "attn: bad head geometry H=%u Hkv=%u", a->H, a->Hkv);
    return -1;
  }
  if (a->cdt != THVM_DT_BF16 && a->cdt != THVM_DT_FP16 && a->cdt != THVM_DT_FP32) {
    snprintf(err, errlen, "attn: cache dtype must be bf16/fp16/f32");
    return -1;
  }
  if (a->chunk != ATT_CHUNK || a->n_split * ATT_CHUNK < a->max_seq) {
    snprintf(err, errlen, "attn: chunk must be %d and n_split*chunk >= max_seq", ATT_CHUNK);
    return -1;
  }
  attn_fn f = nullptr;
  uint32_t G = a->H / a->Hkv;
  const bool f32 = a->cdt == THVM_DT_FP32;
  if (a->hd == 128) f = f32 ? attn_pick<128, 4>(G) : attn_pick<128, 2>(G);
  else if (a->hd == 64) f = f32 ? attn_pick<64, 4>(G) : attn_pick<64, 2>(G);
  if (!f) {
    snprintf(err, errlen, "attn: no kernel for hd=%u G=%u", a->hd, G);
    return -1;
  }
  hipLaunchKernelGGL(f, dim3(a->Hkv, a->n_split, a->B), dim3(ATT_THREADS), 0, s, *a);
  hipLaunchKernelGGL(k_attn_combine, dim3(a->B * a->H), dim3(a->hd), 0, s, *a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) { snprintf(err, errlen, "attn launch: %s", hipGetErrorString(e)); return -1; }
  return 0;
}
