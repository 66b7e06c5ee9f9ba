// attn_core.h -- split-sequence flash-decode attention as block-level device
// functions, shared by the standalone kernels (attn.hip) and the persistent
// decode step (step.hip), so both compute every split and every merge with
// the same instructions in the same order.
//
// Semantics: out[h] = softmax(q_h . K^T * scale) V over cache rows [0, L), L
// read from device memory, MHA and GQA (G = H / Hkv query heads per KV head).
//
// Split unit (kv head, split, row b), 8 waves = 512 threads: the unit owns
// CHUNK=64 cache rows, each wave 8 of them.  A cache row of hd elements is
// hd*esize/16 lanes x 16 bytes, so one wave-wide load covers several rows;
// every K and V load of the wave is issued before any arithmetic (issue()),
// and the arithmetic runs in finish().  All G query heads of the group reuse
// the same K/V registers.  Scores live in the log2 domain (q pre-scaled by
// scale*log2 e) so the softmax uses the hardware exp2.  Row-group sums use
// DPP, the 8 waves merge through LDS with one rescale per wave, and the unit
// writes (acc[hd], m, l) for its split.
// Merge (batch row b, q head h), 256 threads: the ceil(L/(CHUNK*cpb)) live
// partials in a fixed order (deterministic).
//
// COH (persistent kernel): q, the partials and the output are read/written
// with system-scope accesses, and the cache row L-1 -- appended by another
// block of the same launch -- is excluded from issue() and loaded with a
// system-scope load in finish(), after the caller's grid barrier.
#pragma once
#include "dev_common.h"
#include "coh.h"
#include "../kern_api.h"

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
__device__ __forceinline__ uint16_t act_bits(float v) {
  return AT == AT_BF16 ? f2bf(v) : f2h(v);
}
template <int AT, bool COH>
__device__ __forceinline__ void st_act(void *p, uint64_t i, float v) {
  if (COH) {
    if (AT == AT_F32) coh_stf(p, (uint32_t)(i * 4), v);
    else coh_st2(p, (uint32_t)(i * 2), act_bits<AT>(v));
    return;
  }
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

// Query row b's cache length and cache row.  Plain decode: L = len[0] over
// cache row b.  Speculative verify (a.spec): the B query rows are the
// consecutive positions L-1 .. L-1+B-1 of one sequence, so row b attends
// causally over the L+b rows of cache row 0.
__device__ __forceinline__ int32_t attn_row_len(const ThvmAttnArgs &a, uint32_t b) {
  return a.len[0] + (a.spec ? (int32_t)b : 0);
}
__device__ __forceinline__ uint32_t attn_cache_row(const ThvmAttnArgs &a, uint32_t b) {
  return a.spec ? 0u : b;
}

// LDS of one split unit
template <int HD, int G>
struct AttnLds {
  float wm[ATT_WAVES][G], wl[ATT_WAVES][G], wf[ATT_WAVES][G];
  __align__(16) float wacc[ATT_WAVES][G][HD];
};
// LDS of one 256-thread merge group
struct MergeLds {
  float w[ATT_MAX_SPLITS];
  float L;
  __align__(16) float4 red4[256];
};

// COH: q, the partials (and, in attn_merge, the output) use system-scope
// accesses; LATE: the cache row L-1 is written by another block of the same
// launch and is loaded in finish() with a system-scope load.
template <int HD, int G, int AT, bool COH, bool LATE = COH>
struct AttnSplit {
  static constexpr int ES = ATr<AT>::ES;
  static constexpr int EPL = 16 / ES;           // elements per lane chunk
  static constexpr int LPR = HD / EPL;          // lanes per cache row
  static constexpr int RPW = 64 / LPR;          // rows per wave-wide load
  static constexpr int PPW = ATT_CHUNK / ATT_WAVES;
  static constexpr int IT = PPW / RPW;          // loads per wave
  static_assert(LPR >= 8 && LPR <= 32 && IT >= 1 && PPW % RPW == 0, "attention geometry");

  uint4 kq[IT], vq[IT];
  bool ok[IT];

  __device__ __forceinline__ uint64_t row_off(const ThvmAttnArgs &a, uint32_t b, uint32_t kvh,
                                              uint32_t j) const {
    const uint64_t cbase = ((uint64_t)attn_cache_row(a, b) * a.Hkv + kvh) * a.max_seq;
    return ((cbase + j) * HD + (lane_id() % LPR) * EPL) * ES;
  }
  // Issue every K / V load of wave wv (0..7) of the unit (kvh, split, b).
  __device__ __forceinline__ void issue(const ThvmAttnArgs &a, uint32_t kvh, uint32_t split,
                                        uint32_t b, int wv, int32_t L) {
    const int rg = lane_id() / LPR;
    const uint32_t p0 = split * ATT_CHUNK;
    const char *kb = (const char *)a.kcache, *vb = (const char *)a.vcache;
#pragma unroll
    for (int it = 0; it < IT; it++) {
      const uint32_t j = p0 + wv * PPW + it * RPW + rg;
      ok[it] = (int32_t)j < L && j < a.max_seq;
      const bool early = ok[it] && !(LATE && (int32_t)j == L - 1);
      const uint64_t off = row_off(a, b, kvh, early ? j : 0);
      kq[it] = ld_stream16(kb + off);
      vq[it] = ld_stream16(vb + off);
    }
  }
  // Scores, softmax and the V mix of the unit; writes the split's partial.
  // Every thread of the block calls it (the two block barriers inside are
  // block-wide); `active` false skips the work.
  __device__ __forceinline__ void finish(const ThvmAttnArgs &a, uint32_t kvh, uint32_t split,
                                         uint32_t b, int wv, int tid, int32_t L, bool active,
                                         AttnLds<HD, G> &s) {
    const int lane = lane_id();
    const int rg = lane / LPR, li = lane % LPR;
    const uint32_t d0 = li * EPL;
    float mw[G], lw[G], acc[G][EPL];
    if (active) {
      if (LATE) {   // the row appended at L-1 by another block of this launch
        const uint32_t p0 = split * ATT_CHUNK;
#pragma unroll
        for (int it = 0; it < IT; it++) {
          const uint32_t j = p0 + wv * PPW + it * RPW + rg;
          if (ok[it] && (int32_t)j == L - 1) {
            const uint32_t off = (uint32_t)row_off(a, b, kvh, j);
            kq[it] = coh_ld16(a.kcache, off);
            vq[it] = coh_ld16(a.vcache, off);
          }
        }
      }
      // query fragments (one 16-byte load per head, all in flight), kept
      // packed; each use decodes and pre-scales them into the log2 domain
      const float qs = a.scale * LOG2E;
      uint4 qr[G];
#pragma unroll
      for (int g = 0; g < G; g++) {
        const uint64_t qo = ((uint64_t)b * a.H + kvh * G + g) * HD + d0;
        qr[g] = COH ? coh_ld16(a.q, (uint32_t)(qo * ES)) : ld16((const char *)a.q + qo * ES);
      }
      float sc[IT][G];
#pragma unroll
      for (int it = 0; it < IT; it++) {
        float kf[EPL];
        chunk_f<AT>(kq[it], kf);
#pragma unroll
        for (int g = 0; g < G; g++) {
          float qf[EPL];
          chunk_f<AT>(qr[g], qf);
          float sv = 0.0f;
#pragma unroll
          for (int i = 0; i < EPL; i++) sv += (qf[i] * qs) * kf[i];
          sv = group_sum<LPR>(sv);
          sc[it][g] = ok[it] ? sv : -INFINITY;
        }
      }
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
        for (int g = 0; g < G; g++) { s.wm[wv][g] = mw[g]; s.wl[wv][g] = lw[g]; }
      }
    }
    __syncthreads();
    // rescale factor of this wave against the unit max, then publish acc
    if (active) {
      float f[G];
#pragma unroll
      for (int g = 0; g < G; g++) {
        float M = s.wm[0][g];
#pragma unroll
        for (int w = 1; w < ATT_WAVES; w++) M = fmaxf(M, s.wm[w][g]);
        f[g] = mw[g] == -INFINITY ? 0.0f : fexp2(mw[g] - M);
        if (lane == 0) s.wf[wv][g] = f[g];
      }
      if (rg == 0) {
#pragma unroll
        for (int g = 0; g < G; g++)
#pragma unroll
          for (int i = 0; i < EPL; i++) s.wacc[wv][g][d0 + i] = acc[g][i] * f[g];
      }
    }
    __syncthreads();
    if (active) {
      for (int o = tid; o < G * HD; o += ATT_THREADS) {
        const int g = o / HD, d = o % HD;
        float sv = 0.0f, l = 0.0f, M = s.wm[0][g];
#pragma unroll
        for (int w = 0; w < ATT_WAVES; w++) {
          sv += s.wacc[w][g][d];
          l += s.wf[w][g] * s.wl[w][g];
          M = fmaxf(M, s.wm[w][g]);
        }
        const uint64_t pi = (((uint64_t)b * a.H + kvh * G + g) * a.n_split + split) * (HD + 2);
        if (COH) {
          coh_stf(a.part, (uint32_t)((pi + d) * 4), sv);
          if (d == 0) {
            coh_stf(a.part, (uint32_t)((pi + HD) * 4), M);
            coh_stf(a.part, (uint32_t)((pi + HD + 1) * 4), l);
          }
        } else {
          float *pp = a.part + pi;
          pp[d] = sv;
          if (d == 0) { pp[HD] = M; pp[HD + 1] = l; }
        }
      }
    }
  }
};

// Merge of the live splits of one (b, q head) bh = b*H + h by 256 threads
// (tid 0..255): split weights w_s = exp2(m_s - M) and the denominator from one
// wave, then SQ threads per float4 of the head's output each sum a strided
// subset of splits, folded in a fixed order.  Every thread of the block calls
// it (two block barriers inside); `active` false skips the work.
template <int HD, int AT, bool COH>
__device__ __forceinline__ void attn_merge(const ThvmAttnArgs &a, uint32_t bh, int tid, int32_t L,
                                           bool active, MergeLds &s) {
  constexpr int U4 = HD / 4;
  constexpr int SQ = 256 / U4;
  const int32_t span = ATT_CHUNK * (a.cpb > 1 ? (int32_t)a.cpb : 1);   // cache rows per partial
  uint32_t n_live = L > 0 ? (uint32_t)((L + span - 1) / span) : 0u;
  if (n_live > a.n_split) n_live = a.n_split;
  const uint64_t pbi = (uint64_t)bh * a.n_split * (HD + 2);
  const float *pb = a.part + pbi;
  auto ldp = [&](uint64_t i) -> float {
    return COH ? coh_ldf(a.part, (uint32_t)((pbi + i) * 4)) : pb[i];
  };
  const int lane = lane_id();
  // this thread's first MP splits' partial vectors, loaded with wave 0's
  // (m, l) loads (clamped indices, unconditional): they do not depend on the
  // split weights, so the merge waits for one memory round trip, not two
  constexpr int U4P = HD / 4, SQP = 256 / U4P, MP = 4;
  const int dqp = tid % U4P, sqp = tid / U4P;
  float2 pv[MP][2];
  if (active) {
#pragma unroll
    for (int j = 0; j < MP; j++) {
      const uint32_t sp = sqp + j * SQP, spc = sp < n_live ? sp : 0;
      const uint64_t q = (uint64_t)spc * (HD + 2) + dqp * 4;
      if (COH) {
        const uint2 r0 = coh_ld8(a.part, (uint32_t)((pbi + q) * 4));
        const uint2 r1 = coh_ld8(a.part, (uint32_t)((pbi + q + 2) * 4));
        pv[j][0] = make_float2(__uint_as_float(r0.x), __uint_as_float(r0.y));
        pv[j][1] = make_float2(__uint_as_float(r1.x), __uint_as_float(r1.y));
      } else {
        pv[j][0] = *(const float2 *)(pb + q);
        pv[j][1] = *(const float2 *)(pb + q + 2);
      }
    }
  }
  if (active && tid < 64) {
    const float mv0 = lane < (int)n_live ? ldp((uint64_t)lane * (HD + 2) + HD) : -INFINITY;
    const float lv0 = lane < (int)n_live ? ldp((uint64_t)lane * (HD + 2) + HD + 1) : 0.0f;
    const float mv1 = lane + 64 < (int)n_live ? ldp((uint64_t)(lane + 64) * (HD + 2) + HD) : -INFINITY;
    const float lv1 = lane + 64 < (int)n_live ? ldp((uint64_t)(lane + 64) * (HD + 2) + HD + 1) : 0.0f;
    const float M = wave_max(fmaxf(mv0, mv1));
    const float w0 = mv0 == -INFINITY ? 0.0f : fexp2(mv0 - M);
    const float w1 = mv1 == -INFINITY ? 0.0f : fexp2(mv1 - M);
    const float Ls = wave_sum(w0 * lv0 + w1 * lv1);
    if (lane < (int)n_live) s.w[lane] = w0;
    if (lane + 64 < (int)n_live) s.w[lane + 64] = w1;
    if (lane == 0) s.L = Ls;
  }
  __syncthreads();
  if (active) {
    const int dq = tid % U4, sq = tid / U4;
    float4 s4 = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int j = 0; j < MP; j++) {                 // the prefetched splits, in order
      const uint32_t sp = sq + j * SQ;
      if (sp < n_live) {
        const float w = s.w[sp];
        s4.x += w * pv[j][0].x; s4.y += w * pv[j][0].y; s4.z += w * pv[j][1].x; s4.w += w * pv[j][1].y;
      }
    }
#pragma unroll 8
    for (uint32_t sp = sq + MP * SQ; sp < n_live; sp += SQ) {
      const float w = s.w[sp];
      const uint64_t q = (uint64_t)sp * (HD + 2) + dq * 4;
      // HD + 2 floats per split: a split's row is 8-byte aligned only
      float2 v0, v1;
      if (COH) {
        const uint2 r0 = coh_ld8(a.part, (uint32_t)((pbi + q) * 4));
        const uint2 r1 = coh_ld8(a.part, (uint32_t)((pbi + q + 2) * 4));
        v0 = make_float2(__uint_as_float(r0.x), __uint_as_float(r0.y));
        v1 = make_float2(__uint_as_float(r1.x), __uint_as_float(r1.y));
      } else {
        v0 = *(const float2 *)(pb + q);
        v1 = *(const float2 *)(pb + q + 2);
      }
      s4.x += w * v0.x; s4.y += w * v0.y; s4.z += w * v1.x; s4.w += w * v1.y;
    }
    s.red4[tid] = s4;
  }
  __syncthreads();
  if (active && tid < U4) {
    float4 s4 = s.red4[tid];
#pragma unroll
    for (int sq = 1; sq < SQ; sq++) {
      const float4 r = s.red4[sq * U4 + tid];
      s4.x += r.x; s4.y += r.y; s4.z += r.z; s4.w += r.w;
    }
    const float inv = s.L > 0.0f ? 1.0f / s.L : 0.0f;
    const uint64_t oi = (uint64_t)bh * HD + tid * 4;
    st_act<AT, COH>(a.out, oi, s4.x * inv);
    st_act<AT, COH>(a.out, oi + 1, s4.y * inv);
    st_act<AT, COH>(a.out, oi + 2, s4.z * inv);
    st_act<AT, COH>(a.out, oi + 3, s4.w * inv);
  }
}
