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
// Merge (batch row b, kv head), 512 threads: the G heads' ceil(L/(CHUNK*cpb))
// live partials in a fixed order (deterministic), one memory round trip.
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
#define ATT_MAX_SPLITS 2048  /* max_seq <= 131072 (the merge folds any number of partials) */
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
  if (LPR == 32) v += xor16_f(v);
  return v;
}

__device__ __forceinline__ float fexp2(float x) { return exp2f(x); }

// v of lane (lane ^ off), off in {8, 16, 32} (a compile-time constant where
// it is used): the row groups of a wave meet without an LDS round trip -- a
// DPP row rotation by 8 (row_ror:8) or a permlane swap across 16 / 32 lanes
// (a ds_bpermute shuffle costs one LDS round trip each)
__device__ __forceinline__ float attn_xor(float v, int off) {
  return off == 8 ? dpp_f<0x128>(v) : off == 16 ? xor16_f(v) : xor32_f(v);
}

// Query row b's cache length and cache row.  Plain decode: L = len[0] over
// cache row b.  Speculative verify (a.spec): the B query rows are the
// consecutive positions L-1 .. L-1+B-1 of one sequence, so row b attends
// causally over the L+b rows of cache row 0.  A length past the cache (a
// replay pushed beyond max_seq) is clamped to max_seq, so the live-split
// count never exceeds the split blocks the grid holds.
__device__ __forceinline__ int32_t attn_row_len(const ThvmAttnArgs &a, uint32_t b) {
  const int32_t L = a.len[0] + (a.spec ? (int32_t)b : 0);
  return L < (int32_t)a.max_seq ? L : (int32_t)a.max_seq;
}
__device__ __forceinline__ uint32_t attn_cache_row(const ThvmAttnArgs &a, uint32_t b) {
  return a.spec ? 0u : b;
}

// LDS of one split unit
template <int HD, int G>
struct AttnLds {
  float wm[ATT_WAVES][G], wl[ATT_WAVES][G];
  __align__(16) float wacc[ATT_WAVES][G][HD];
};

// COH: q and the partials use system-scope
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
        for (int off = LPR; off < 64; off *= 2) m = fmaxf(m, attn_xor(m, off));
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
          lw[g] += attn_xor(lw[g], off);
#pragma unroll
          for (int i = 0; i < EPL; i++) acc[g][i] += attn_xor(acc[g][i], off);
        }
      }
      // each wave publishes its (m, l) and its accumulator relative to its
      // own max; one barrier, then each output thread rescales the 8 waves'
      // terms to the unit max and sums them in wave order (the products and
      // the order of rescaling before publishing, so the same values)
      if (lane == 0) {
#pragma unroll
        for (int g = 0; g < G; g++) { s.wm[wv][g] = mw[g]; s.wl[wv][g] = lw[g]; }
      }
      if (rg == 0) {
#pragma unroll
        for (int g = 0; g < G; g++)
#pragma unroll
          for (int i = 0; i < EPL; i++) s.wacc[wv][g][d0 + i] = acc[g][i];
      }
    }
    __syncthreads();
    if (active) {
      for (int o = tid; o < G * HD; o += ATT_THREADS) {
        const int g = o / HD, d = o % HD;
        float M = s.wm[0][g];
#pragma unroll
        for (int w = 1; w < ATT_WAVES; w++) M = fmaxf(M, s.wm[w][g]);
        float sv = 0.0f, l = 0.0f;
#pragma unroll
        for (int w = 0; w < ATT_WAVES; w++) {
          const float mwv = s.wm[w][g];
          const float f = mwv == -INFINITY ? 0.0f : fexp2(mwv - M);
          sv += s.wacc[w][g][d] * f;
          l += f * s.wl[w][g];
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
// ---- one-round-trip merge of a (row, kv head) group ----------------------
// The G heads of query row b and kv head kvh, by 512 threads: thread t owns
// the output pair (g, d) = (e / (HD/2), 2 (e % (HD/2))), e = t % PAIRS, and
// folds the live partials s = p, p + NP, p + 2 NP, ... of its partition
// p = t / PAIRS (NP = 512 / PAIRS partitions), loading up to MC of them
// before any arithmetic (one memory round trip for up to NP * MC partials;
// MC only batches the loads, the fold order is the same for every MC);
// partition 0 then folds partitions 1 .. NP-1 in order.  The fold of (m, l,
// acc) into (mp, lp, ap): mn = max(mp, m), lp = lp 2^(mp-mn) + l 2^(m-mn),
// likewise ap; out = ap / lp.  Every caller (the merge kernel, the one-launch
// forms, the persistent step) runs this function, so all that group the heads
// alike give the same bits (the VALU forms merge a kv head's G heads as one
// group, the MFMA forms each head as a group of one: NP differs, and so does
// the fold order).
// COH: system-scope loads of the partials and stores of the output.
#define MERGE_THREADS 512
#define MCH 16
template <int HD, int G>
struct MergeFlatLds {
  static constexpr int PAIRS = G * HD / 2, NP = MERGE_THREADS / PAIRS;
  float m[NP][PAIRS], l[NP][PAIRS];
  float2 a[NP][PAIRS];
};
#define MERGE_LDS_BYTES (MERGE_THREADS * 16)   /* sizeof(MergeFlatLds<HD, G>), every HD and G */

__device__ __forceinline__ void merge_fold(float &mp, float &lp, float &a0, float &a1, float m,
                                           float l, float x0, float x1) {
  const float mn = fmaxf(mp, m);
  const float fo = mp == -INFINITY ? 0.0f : fexp2(mp - mn);
  const float fn = m == -INFINITY ? 0.0f : fexp2(m - mn);
  lp = lp * fo + l * fn;
  a0 = a0 * fo + x0 * fn;
  a1 = a1 * fo + x1 * fn;
  mp = mn;
}

// n_live partials of the (row, kv head) are folded; nl() gives n_live.
// n_max >= n_live bounds the slots the first batch of loads may touch (0:
// n_live): with a bound known at launch those loads go out first and nl()
// is called only after them, so a row length read from memory there costs
// no round trip of its own (it arrives with the partials); slots past
// n_live are read but never folded.
template <int HD, int G, int AT, bool COH, int MC = MCH, class NLive>
__device__ __forceinline__ void attn_merge_flat_d(const ThvmAttnArgs &a, uint32_t b, uint32_t kvh,
                                                  NLive &&nl, int tid, bool active,
                                                  MergeFlatLds<HD, G> &s, uint32_t n_max = 0,
                                                  uint64_t *clk = nullptr, uint32_t clk_cap = 0) {
  typedef MergeFlatLds<HD, G> FL;
  constexpr int PAIRS = FL::PAIRS, NP = FL::NP;
  static_assert(NP >= 1 && MERGE_THREADS % PAIRS == 0, "merge geometry");
  const int e = tid % PAIRS, p = tid / PAIRS;
  const int g = e / (HD / 2), d = (e % (HD / 2)) * 2;
  const uint64_t bh = (uint64_t)b * a.H + kvh * G + g;
  const uint64_t pbi = bh * a.n_split * (HD + 2);
  float mp = -INFINITY, lp = 0.0f, a0 = 0.0f, a1 = 0.0f;
  if (active && p < NP) {
    float mv[MC], lv[MC];
    float2 av[MC];
    // loads of slots s0 + j NP (slots at or past `bound` read slot s0
    // again: every load stays inside the group's partials; those are never
    // folded)
    auto load = [&](uint32_t s0, uint32_t bound) {
#pragma unroll
      for (int j = 0; j < MC; j++) {
        const uint32_t sp = s0 + j * NP, spc = sp < bound ? sp : s0;
        const uint64_t q = pbi + (uint64_t)spc * (HD + 2);
        if (COH) {
          const uint2 r = coh_ld8(a.part, (uint32_t)((q + d) * 4));
          const uint2 ml = coh_ld8(a.part, (uint32_t)((q + HD) * 4));
          av[j] = make_float2(__uint_as_float(r.x), __uint_as_float(r.y));
          mv[j] = __uint_as_float(ml.x);
          lv[j] = __uint_as_float(ml.y);
        } else {
          av[j] = *(const float2 *)(a.part + q + d);
          const float2 ml = *(const float2 *)(a.part + q + HD);
          mv[j] = ml.x;
          lv[j] = ml.y;
        }
      }
    };
    // (a partition with no slot issues no load: the clamped loads of empty
    // partitions, 2 MC per thread, had taken the one-launch VALU attention
    // of a 12-head GPT-2 step from 5.7 to 7.2 us per layer)
    const uint32_t nmax = n_max ? n_max : nl();
    if ((uint32_t)p < nmax) load((uint32_t)p, nmax);
    __builtin_amdgcn_sched_barrier(0);
    const uint32_t n_live = nl();
#pragma unroll
    for (int j = 0; j < MC; j++)
      if (p + j * NP < n_live) merge_fold(mp, lp, a0, a1, mv[j], lv[j], av[j].x, av[j].y);
    for (uint32_t s0 = p + NP * MC; s0 < n_live; s0 += NP * MC) {
      load(s0, n_live);
#pragma unroll
      for (int j = 0; j < MC; j++)
        if (s0 + j * NP < n_live) merge_fold(mp, lp, a0, a1, mv[j], lv[j], av[j].x, av[j].y);
    }
  }
  pclk(clk, clk_cap, 1);
  if (NP > 1) {
    if (active) { s.m[p][e] = mp; s.l[p][e] = lp; s.a[p][e] = make_float2(a0, a1); }
    __syncthreads();
    pclk(clk, clk_cap, 2);
    if (active && p == 0)
#pragma unroll
      for (int q = 1; q < NP; q++) merge_fold(mp, lp, a0, a1, s.m[q][e], s.l[q][e], s.a[q][e].x, s.a[q][e].y);
  }
  if (active && p == 0) {
    const float inv = lp > 0.0f ? 1.0f / lp : 0.0f;
    const uint64_t oi = bh * HD + d;
    st_act<AT, COH>(a.out, oi, a0 * inv);
    st_act<AT, COH>(a.out, oi + 1, a1 * inv);
  }
}
// NH heads at once, each merged as a group of one (the per-head merge's
// fold: the same partitions, slot order and partition order, so the same
// bits as attn_merge_flat<HD, 1> run head by head): every thread takes its
// (pair, partition) of all NH heads, all their first-batch loads in flight
// together, then one LDS round for all the heads.  Heads kvh * NH + gi of
// row b; n_live partials; s holds NH per-head LDS areas.
template <int HD, int NH, int AT, bool COH, int MC>
__device__ __forceinline__ void attn_merge_heads(const ThvmAttnArgs &a, uint32_t b, uint32_t kvh,
                                                 uint32_t n_live, int tid, MergeFlatLds<HD, 1> *s) {
  typedef MergeFlatLds<HD, 1> FL;
  constexpr int PAIRS = FL::PAIRS, NP = FL::NP;
  static_assert(NP >= 1 && MERGE_THREADS % PAIRS == 0, "merge geometry");
  const int e = tid % PAIRS, p = tid / PAIRS, d = e * 2;
  float mp[NH], lp[NH], a0[NH], a1[NH];
#pragma unroll
  for (int gi = 0; gi < NH; gi++) { mp[gi] = -INFINITY; lp[gi] = 0.0f; a0[gi] = 0.0f; a1[gi] = 0.0f; }
  if (p < NP) {
    for (uint32_t s0 = p; s0 < n_live; s0 += NP * MC) {
      float mv[NH][MC], lv[NH][MC];
      float2 av[NH][MC];
#pragma unroll
      for (int gi = 0; gi < NH; gi++) {
        const uint64_t pbi = ((uint64_t)b * a.H + kvh * NH + gi) * a.n_split * (HD + 2);
#pragma unroll
        for (int j = 0; j < MC; j++) {             // slots past n_live read slot s0, never folded
          const uint32_t sp = s0 + j * NP, spc = sp < n_live ? sp : s0;
          const uint64_t q = pbi + (uint64_t)spc * (HD + 2);
          if (COH) {
            const uint2 r = coh_ld8(a.part, (uint32_t)((q + d) * 4));
            const uint2 ml = coh_ld8(a.part, (uint32_t)((q + HD) * 4));
            av[gi][j] = make_float2(__uint_as_float(r.x), __uint_as_float(r.y));
            mv[gi][j] = __uint_as_float(ml.x);
            lv[gi][j] = __uint_as_float(ml.y);
          } else {
            av[gi][j] = *(const float2 *)(a.part + q + d);
            const float2 ml = *(const float2 *)(a.part + q + HD);
            mv[gi][j] = ml.x;
            lv[gi][j] = ml.y;
          }
        }
      }
#pragma unroll
      for (int gi = 0; gi < NH; gi++)
#pragma unroll
        for (int j = 0; j < MC; j++)
          if (s0 + j * NP < n_live)
            merge_fold(mp[gi], lp[gi], a0[gi], a1[gi], mv[gi][j], lv[gi][j], av[gi][j].x, av[gi][j].y);
    }
  }
  if (NP > 1) {
    if (p < NP)
#pragma unroll
      for (int gi = 0; gi < NH; gi++) {
        s[gi].m[p][e] = mp[gi];
        s[gi].l[p][e] = lp[gi];
        s[gi].a[p][e] = make_float2(a0[gi], a1[gi]);
      }
    __syncthreads();
    if (p == 0)
#pragma unroll
      for (int gi = 0; gi < NH; gi++)
#pragma unroll
        for (int q = 1; q < NP; q++)
          merge_fold(mp[gi], lp[gi], a0[gi], a1[gi], s[gi].m[q][e], s[gi].l[q][e], s[gi].a[q][e].x,
                     s[gi].a[q][e].y);
  }
  if (p == 0) {
#pragma unroll
    for (int gi = 0; gi < NH; gi++) {
      const float inv = lp[gi] > 0.0f ? 1.0f / lp[gi] : 0.0f;
      const uint64_t oi = ((uint64_t)b * a.H + kvh * NH + gi) * HD + d;
      st_act<AT, COH>(a.out, oi, a0[gi] * inv);
      st_act<AT, COH>(a.out, oi + 1, a1[gi] * inv);
    }
  }
}
// the same with n_live known at the call
template <int HD, int G, int AT, bool COH>
__device__ __forceinline__ void attn_merge_flat(const ThvmAttnArgs &a, uint32_t b, uint32_t kvh,
                                                uint32_t n_live, int tid, bool active,
                                                MergeFlatLds<HD, G> &s, uint32_t n_max = 0,
                                                uint64_t *clk = nullptr, uint32_t clk_cap = 0) {
  attn_merge_flat_d<HD, G, AT, COH>(a, b, kvh, [n_live] { return n_live; }, tid, active, s, n_max, clk,
                                    clk_cap);
}
