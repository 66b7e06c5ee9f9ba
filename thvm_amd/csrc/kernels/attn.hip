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
// gfx950 design, one kernel:
//   split phase: grid (Hkv, n_split, B), 8 waves.  A block owns one KV head and
//     CHUNK=64 cache rows; each wave takes 8 rows.  A cache row of hd elements
//     is hd*esize/16 lanes x 16 bytes, so one wave-wide load covers several
//     rows; every K and V load of the wave is issued before any arithmetic.  All
//     G = H/Hkv query heads of the group reuse the same K/V registers (GQA
//     reuse).  Scores live in the log2 domain (q pre-scaled by scale*log2 e) so
//     the softmax uses the hardware exp2.  Row-group sums use DPP, the 8 waves
//     merge through LDS with one rescale per wave, and the block writes
//     (acc[hd], m, l) for its split.
//   merge kernel: one block per (b, q head) merges the ceil(L/CHUNK) live
//     splits in a fixed order (deterministic) and writes out [B][H*hd].  (An
//     in-kernel "last block merges" variant with device-scope fences measured
//     3x slower on gfx950: the fences write back / invalidate L2 across XCDs.)
#include "dev_common.h"
#include "../kern_api.h"
#include "launch.h"
#include <stdio.h>

#define ATT_WAVES 8
#define ATT_THREADS (ATT_WAVES * 64)
#define ATT_CHUNK 64
#define ATT_MAX_SPLITS 128   /* max_seq <= 8192 */
#define LOG2E 1.4426950408889634f

// activation dtype of q, the caches and the output (one compile-time type)
enum { AT_BF16 = 0, AT_F16 = 1, AT_F32 = 2 };
template <int AT> struct ATr { static constexpr int ES = AT == AT_F32 ? 4 : 2; };

// one 16-byte chunk of elements -> floats
template <int AT>
__device__ __forceinline__ void chunk_f(const uint4 &q, float *o) {
  uint32_t w[4] = {q.x, q.y, q.z, q.w};
  if (AT == AT_F32) {
#pragma unroll
    for (int i = 0; i < 4; i++) o[i] = __uint_as_float(w[i]);
  } else {
#pragma unroll
    for (int i = 0; i < 4; i++) {
      if (AT == AT_BF16) {
        o[2 * i] = __uint_as_float(w[i] << 16);
        o[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
      } else {
        o[2 * i] = h2f((f16_t)(w[i] & 0xffffu));
        o[2 * i + 1] = h2f((f16_t)(w[i] >> 16));
      }
    }
  }
}

template <int AT>
__device__ __forceinline__ void st_act(void *p, uint64_t i, float v) {
  if (AT == AT_BF16) ((bf16_t *)p)[i] = f2bf(v);
  else if (AT == AT_F16) ((f16_t *)p)[i] = f2h(v);
  else ((float *)p)[i] = v;
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

__device__ __forceinline__ float fexp2(float x) { return exp2f(x); }

template <int HD, int G, int AT>
__global__ __launch_bounds__(ATT_THREADS) void k_attn(ThvmAttnArgs a) {
  constexpr int ES = ATr<AT>::ES;
  constexpr int EPL = 16 / ES;           // elements per lane chunk
  constexpr int LPR = HD / EPL;          // lanes per cache row
  constexpr int RPW = 64 / LPR;          // rows per wave-wide load
  constexpr int PPW = ATT_CHUNK / ATT_WAVES;
  constexpr int IT = PPW / RPW;          // loads per wave
  static_assert(LPR >= 8 && LPR <= 32 && IT >= 1 && PPW % RPW == 0, "attention geometry");
  __shared__ float wm[ATT_WAVES][G], wl[ATT_WAVES][G], wf[ATT_WAVES][G];
  __shared__ __align__(16) float wacc[ATT_WAVES][G][HD];

  const uint32_t kvh = blockIdx.x, split = blockIdx.y, b = blockIdx.z;
  const int32_t L = a.len[0];
  const uint32_t p0 = split * ATT_CHUNK;
  if ((int32_t)p0 >= L) return;          // the merge reads only live splits

  const int lane = lane_id(), wv = threadIdx.x >> 6;
  const int rg = lane / LPR, li = lane % LPR;
  const uint32_t d0 = li * EPL;
  const uint64_t cbase = ((uint64_t)b * a.Hkv + kvh) * a.max_seq;
  const char *kb = (const char *)a.kcache, *vb = (const char *)a.vcache;

  // every K / V load of the wave in flight first
  uint4 kq[IT], vq[IT];
  bool ok[IT];
#pragma unroll
  for (int it = 0; it < IT; it++) {
    const uint32_t j = p0 + wv * PPW + it * RPW + rg;
    ok[it] = (int32_t)j < L && j < a.max_seq;
    const uint64_t off = ((cbase + (ok[it] ? j : 0)) * HD + d0) * ES;
    kq[it] = ld_stream16(kb + off);
    vq[it] = ld_stream16(vb + off);
  }
  // query fragment (one 16-byte load per head), pre-scaled into log2 domain
  const float qs = a.scale * LOG2E;
  float qf[G][EPL];
#pragma unroll
  for (int g = 0; g < G; g++) {
    const uint64_t qo = ((uint64_t)b * a.H + kvh * G + g) * HD + d0;
    chunk_f<AT>(ld16((const char *)a.q + qo * ES), qf[g]);
#pragma unroll
    for (int i = 0; i < EPL; i++) qf[g][i] *= qs;
  }

  float sc[IT][G];
#pragma unroll
  for (int it = 0; it < IT; it++) {
    float kf[EPL];
    chunk_f<AT>(kq[it], kf);
#pragma unroll
    for (int g = 0; g < G; g++) {
      float s = 0.0f;
#pragma unroll
      for (int i = 0; i < EPL; i++) s += qf[g][i] * kf[i];
      s = group_sum<LPR>(s);
      sc[it][g] = ok[it] ? s : -INFINITY;
    }
  }
  float mw[G], lw[G], acc[G][EPL];
#pragma unroll
  for (int g = 0; g < G; g++) {
    float m = sc[0][g];
#pragma unroll
    for (int it = 1; it < IT; it++) m = fmaxf(m, sc[it][g]);
#pragma unroll
    for (int off = LPR; off < 64; off *= 2) m = fmaxf(m, __shfl_xor(m, off));
    mw[g] = m;
    lw[g] = 0.0f;
#pragma unroll
    for (int i = 0; i < EPL; i++) acc[g][i] = 0.0f;
  }
#pragma unroll
  for (int it = 0; it < IT; it++) {
    float vf[EPL];
    chunk_f<AT>(vq[it], vf);
#pragma unroll
    for (int g = 0; g < G; g++) {
      const float p = (ok[it] && mw[g] != -INFINITY) ? fexp2(sc[it][g] - mw[g]) : 0.0f;
      lw[g] += p;
#pragma unroll
      for (int i = 0; i < EPL; i++) acc[g][i] += p * vf[i];
    }
  }
  // the row groups of the wave hold disjoint rows: sum them (all lanes)
#pragma unroll
  for (int g = 0; g < G; g++) {
#pragma unroll
    for (int off = LPR; off < 64; off *= 2) {
      lw[g] += __shfl_xor(lw[g], off);
#pragma unroll
      for (int i = 0; i < EPL; i++) acc[g][i] += __shfl_xor(acc[g][i], off);
    }
  }
  if (lane == 0) {
#pragma unroll
    for (int g = 0; g < G; g++) { wm[wv][g] = mw[g]; wl[wv][g] = lw[g]; }
  }
  __syncthreads();
  // rescale factor of this wave against the block max, then publish acc
  {
    float f[G];
#pragma unroll
    for (int g = 0; g < G; g++) {
      float M = wm[0][g];
#pragma unroll
      for (int w = 1; w < ATT_WAVES; w++) M = fmaxf(M, wm[w][g]);
      f[g] = mw[g] == -INFINITY ? 0.0f : fexp2(mw[g] - M);
      if (lane == 0) wf[wv][g] = f[g];
    }
    if (rg == 0) {
#pragma unroll
      for (int g = 0; g < G; g++)
#pragma unroll
        for (int i = 0; i < EPL; i++) wacc[wv][g][d0 + i] = acc[g][i] * f[g];
    }
  }
  __syncthreads();
  for (int o = threadIdx.x; o < G * HD; o += ATT_THREADS) {
    const int g = o / HD, d = o % HD;
    float s = 0.0f, l = 0.0f, M = wm[0][g];
#pragma unroll
    for (int w = 0; w < ATT_WAVES; w++) {
      s += wacc[w][g][d];
      l += wf[w][g] * wl[w][g];
      M = fmaxf(M, wm[w][g]);
    }
    float *pp = a.part + (((uint64_t)b * a.H + kvh * G + g) * a.n_split + split) * (HD + 2);
    pp[d] = s;
    if (d == 0) { pp[HD] = M; pp[HD + 1] = l; }
  }

}

// Merge of the live splits of one (b, q head): split weights w_s = exp2(m_s -
// M) and the denominator from one wave, then SQ threads per float4 of the
// head's output each sum a strided subset of splits, folded in a fixed order.
// Every load of a phase is issued before its first use.
template <int HD, int AT>
__global__ __launch_bounds__(256) void k_attn_merge(ThvmAttnArgs a) {
  constexpr int U4 = HD / 4;
  constexpr int SQ = 256 / U4;
  __shared__ float sm_w[ATT_MAX_SPLITS];
  __shared__ float sm_L;
  __shared__ __align__(16) float4 red4[256];
  const uint32_t bh = blockIdx.x;                      // b*H + h
  const int32_t L = a.len[0];
  uint32_t n_live = L > 0 ? (uint32_t)((L + ATT_CHUNK - 1) / ATT_CHUNK) : 0u;
  if (n_live > a.n_split) n_live = a.n_split;
  const float *pb = a.part + (uint64_t)bh * a.n_split * (HD + 2);
  const int lane = lane_id();
  if (threadIdx.x < 64) {
    const float mv0 = lane < (int)n_live ? pb[(uint64_t)lane * (HD + 2) + HD] : -INFINITY;
    const float lv0 = lane < (int)n_live ? pb[(uint64_t)lane * (HD + 2) + HD + 1] : 0.0f;
    const float mv1 = lane + 64 < (int)n_live ? pb[(uint64_t)(lane + 64) * (HD + 2) + HD] : -INFINITY;
    const float lv1 = lane + 64 < (int)n_live ? pb[(uint64_t)(lane + 64) * (HD + 2) + HD + 1] : 0.0f;
    const float M = wave_max(fmaxf(mv0, mv1));
    const float w0 = mv0 == -INFINITY ? 0.0f : fexp2(mv0 - M);
    const float w1 = mv1 == -INFINITY ? 0.0f : fexp2(mv1 - M);
    const float Ls = wave_sum(w0 * lv0 + w1 * lv1);
    if (lane < (int)n_live) sm_w[lane] = w0;
    if (lane + 64 < (int)n_live) sm_w[lane + 64] = w1;
    if (lane == 0) sm_L = Ls;
  }
  __syncthreads();
  {
    const int dq = threadIdx.x % U4, sq = threadIdx.x / U4;
    const float *pg = pb + dq * 4;
    float4 s4 = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll 8
    for (uint32_t s = sq; s < n_live; s += SQ) {
      const float w = sm_w[s];
      const float *q = pg + (uint64_t)s * (HD + 2);
      // HD + 2 floats per split: a split's row is 8-byte aligned only
      const float2 v0 = *(const float2 *)q, v1 = *(const float2 *)(q + 2);
      s4.x += w * v0.x; s4.y += w * v0.y; s4.z += w * v1.x; s4.w += w * v1.y;
    }
    red4[threadIdx.x] = s4;
  }
  __syncthreads();
  if (threadIdx.x < U4) {
    float4 s4 = red4[threadIdx.x];
#pragma unroll
    for (int sq = 1; sq < SQ; sq++) {
      const float4 r = red4[sq * U4 + threadIdx.x];
      s4.x += r.x; s4.y += r.y; s4.z += r.z; s4.w += r.w;
    }
    const float inv = sm_L > 0.0f ? 1.0f / sm_L : 0.0f;
    const uint64_t oi = (uint64_t)bh * HD + threadIdx.x * 4;
    st_act<AT>(a.out, oi, s4.x * inv);
    st_act<AT>(a.out, oi + 1, s4.y * inv);
    st_act<AT>(a.out, oi + 2, s4.z * inv);
    st_act<AT>(a.out, oi + 3, s4.w * inv);
  }
}

typedef void (*attn_fn)(ThvmAttnArgs);
template <int HD, int AT>
static attn_fn attn_pick(uint32_t G) {
  switch (G) {
    case 1: return k_attn<HD, 1, AT>;
    case 2: return k_attn<HD, 2, AT>;
    case 4: return k_attn<HD, 4, AT>;
    case 8: return k_attn<HD, 8, AT>;
    default: return nullptr;
  }
}

// partials [B][H][n_split][hd + 2] f32 (the Hkv argument keeps room for
// per-kv-head state; none is used)
extern "C" uint64_t thvm_k_attn_part_bytes(uint32_t B, uint32_t H, uint32_t Hkv, uint32_t hd,
                                           uint32_t n_split) {
  return (uint64_t)B * H * n_split * (hd + 2) * 4 + (uint64_t)B * Hkv * 4;
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
  if (a->chunk != ATT_CHUNK || a->n_split * ATT_CHUNK < a->max_seq || a->n_split > ATT_MAX_SPLITS) {
    snprintf(err, errlen, "attn: chunk must be %d, n_split*chunk >= max_seq, n_split <= %d",
             ATT_CHUNK, ATT_MAX_SPLITS);
    return -1;
  }
  if (a->qdt != a->cdt || a->odt != a->cdt) {
    snprintf(err, errlen, "attn: q, cache and out must share one dtype");
    return -1;
  }
  attn_fn f = nullptr, fm = nullptr;
  const uint32_t G = a->H / a->Hkv;
  const int at = a->cdt == THVM_DT_BF16 ? AT_BF16 : a->cdt == THVM_DT_FP16 ? AT_F16 : AT_F32;
  if (a->hd == 128) {
    f = at == AT_BF16 ? attn_pick<128, AT_BF16>(G) : at == AT_F16 ? attn_pick<128, AT_F16>(G) : attn_pick<128, AT_F32>(G);
    fm = at == AT_BF16 ? k_attn_merge<128, AT_BF16> : at == AT_F16 ? k_attn_merge<128, AT_F16> : k_attn_merge<128, AT_F32>;
  } else if (a->hd == 64) {
    f = at == AT_BF16 ? attn_pick<64, AT_BF16>(G) : at == AT_F16 ? attn_pick<64, AT_F16>(G) : attn_pick<64, AT_F32>(G);
    fm = at == AT_BF16 ? k_attn_merge<64, AT_BF16> : at == AT_F16 ? k_attn_merge<64, AT_F16> : k_attn_merge<64, AT_F32>;
  }
  if (!f) {
    snprintf(err, errlen, "attn: no kernel for hd=%u G=%u", a->hd, G);
    return -1;
  }
  thvm_launch(true, false, f, dim3(a->Hkv, a->n_split, a->B), dim3(ATT_THREADS), 0, s, *a);
  thvm_launch(false, true, fm, dim3(a->B * a->H), dim3(256), 0, s, *a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) { snprintf(err, errlen, "attn launch: %s", hipGetErrorString(e)); return -1; }
  return 0;
}
