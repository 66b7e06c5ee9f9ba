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
// gfx950 design (the unit and merge bodies are in attn_core.h, shared with the
// persistent decode step):
//   split kernel: grid (Hkv, n_split, B), 8 waves; a block is one split unit
//     (one KV head, CHUNK=64 cache rows, all G = H/Hkv query heads of the
//     group on the same K/V registers) and writes (acc[hd], m, l).
//   merge kernel: one block per (b, q head) merges the ceil(L/CHUNK) live
//     splits in a fixed order (deterministic) and writes out [B][H*hd].  (An
//     in-kernel "last block merges" variant with device-scope fences measured
//     3x slower on gfx950: the fences write back / invalidate L2 across XCDs.)
#include "attn_core.h"
#include "mfma_ops.h"
#include "launch.h"
#include <stdio.h>

template <int HD, int G, int AT>
__global__ __launch_bounds__(ATT_THREADS) void k_attn(ThvmAttnArgs a) {
  __shared__ AttnLds<HD, G> s;
  const uint32_t kvh = blockIdx.x, split = blockIdx.y, b = blockIdx.z;
  const int32_t L = attn_row_len(a, b);
  if ((int32_t)(split * ATT_CHUNK) >= L) return;   // the merge reads only live splits
  const int wv = threadIdx.x >> 6;
  AttnSplit<HD, G, AT, false> u;
  u.issue(a, kvh, split, b, wv, L);
  u.finish(a, kvh, split, b, wv, threadIdx.x, L, true, s);
}

// live partials of a row of length L: one per cpb chunks, at most the
// number of split blocks in the grid (ceil(n_split / cpb))
__device__ __forceinline__ uint32_t attn_live(const ThvmAttnArgs &a, int32_t L) {
  const uint32_t cpb = a.cpb > 1 ? a.cpb : 1u;
  const int32_t span = ATT_CHUNK * (int32_t)cpb;
  const uint32_t n = L > 0 ? (uint32_t)((L + span - 1) / span) : 0u, nb = (a.n_split + cpb - 1) / cpb;
  return n < nb ? n : nb;
}

// one block per (row, kv head): the group's G heads
template <int HD, int G, int AT, int MC>
__global__ __launch_bounds__(MERGE_THREADS) void k_attn_merge(ThvmAttnArgs a) {
  __shared__ MergeFlatLds<HD, G> s;
  const uint32_t b = blockIdx.x / a.Hkv, kvh = blockIdx.x % a.Hkv;
  // phase clock: the merge's blocks follow the split's in the clock buffer;
  // 0 entry, 1 partials folded, 2 partition partials combined, 7 drained
  uint64_t *const clk = a.clk ? a.clk + (uint64_t)a.clk_cap * PCLK_MARKS : nullptr;
  pclk(clk, a.clk_cap, 0);
  const uint32_t cpb = a.cpb > 1 ? a.cpb : 1u;
  // (the row length is read after the first partial loads are out)
  attn_merge_flat_d<HD, G, AT, false, MC>(a, b, kvh, [&] { return attn_live(a, attn_row_len(a, b)); },
                                      threadIdx.x, true, s, (a.n_split + cpb - 1) / cpb, clk, a.clk_cap);
  pclk_end(clk, a.clk_cap);
}

// The one-launch forms' hand-off: publish this block's partial (written
// with system-scope stores), count it on the (row, kv head) counter -- one
// agent-scope atomic, B*Hkv words after the partials, zero between launches
// -- and merge the group when this block brings the count to n_live (then
// reset the counter).  No fence: the partials never sit in an L2.
// PH: the group's heads merged together, each as a group of one (the
// per-head merge kernel's fold; ms is then G MergeFlatLds<HD, 1>).
template <int HD, int G, int AT, bool PH = false>
__device__ __forceinline__ void attn_handoff_merge(const ThvmAttnArgs &a, uint32_t b, uint32_t kvh,
                                                   uint32_t n_live, uint32_t *last,
                                                   MergeFlatLds<HD, PH ? 1 : G> *ms) {
  vm_drain();
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t *ctr = (uint32_t *)(a.part + (uint64_t)a.B * a.H * a.n_split * (HD + 2)) + b * a.Hkv + kvh;
    const uint32_t old = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *last = old == n_live - 1 ? 1u : 0u;
    if (*last) __hip_atomic_exchange(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  if (!*last) return;                              // block-uniform
  if constexpr (PH) {
    attn_merge_heads<HD, G, AT, true, 4>(a, b, kvh, n_live, threadIdx.x, ms);
  } else {
    attn_merge_flat<HD, G, AT, true>(a, b, kvh, n_live, threadIdx.x, true, *ms);
  }
}

// Split and merge in one launch, one chunk per block: each split unit
// publishes its partial and the last one merges (attn_handoff_merge).  Same
// split and merge code as the two-kernel form, so the same outputs.
template <int HD, int G, int AT>
__global__ __launch_bounds__(ATT_THREADS) void k_attn_fused(ThvmAttnArgs a) {
  __shared__ AttnLds<HD, G> s;
  __shared__ MergeFlatLds<HD, G> ms;
  __shared__ uint32_t last;
  const uint32_t kvh = blockIdx.x, split = blockIdx.y, b = blockIdx.z;
  const int32_t L = attn_row_len(a, b);
  if ((int32_t)(split * ATT_CHUNK) >= L) return;   // dead splits are not counted
  uint32_t n_live = (uint32_t)((L + ATT_CHUNK - 1) / ATT_CHUNK);
  if (n_live > a.n_split) n_live = a.n_split;
  const int wv = threadIdx.x >> 6;
  AttnSplit<HD, G, AT, true, false> u;
  u.issue(a, kvh, split, b, wv, L);
  u.finish(a, kvh, split, b, wv, threadIdx.x, L, true, s);
  attn_handoff_merge<HD, G, AT>(a, b, kvh, n_live, &last, &ms);
}

// Batched split: one block runs cpb (a.cpb) consecutive chunks of a (kv head, row),
// the next chunk's K/V loads in flight while the current one is consumed.
// The per-chunk work of the one-chunk unit is dominated by its fixed part at
// large unit counts (the q decode, the wave-wide max and the row-group
// shuffles, the LDS merge of the 8 waves): here q is decoded once, each row
// group (LPR lanes holding one cache row) keeps its own running max, sum and
// accumulator across the block's chunks (online softmax: rescaled by
// exp2(m_old - m_new) when the max grows), and the row groups and waves are
// combined once per block.  The block writes one partial (acc, m, l) at slot
// blockIdx.y of the merge's [n_split] rows; the merge reads ceil(L/(64 cpb))
// of them.  FUSE: the partial is published with system-scope stores and the
// last block of the (row, kv head) merges in the same launch.
template <int HD, int G, int AT, bool FUSE>
__global__ __launch_bounds__(ATT_THREADS, 4) void k_attn_multi(ThvmAttnArgs a) {   // 2 blocks per CU
  __shared__ AttnLds<HD, G> s;
  __shared__ MergeFlatLds<HD, G> ms;
  __shared__ uint32_t last;
  typedef AttnSplit<HD, G, AT, false> SU;
  constexpr int EPL = SU::EPL, LPR = SU::LPR, RPW = SU::RPW, PPW = SU::PPW, IT = SU::IT, ES = SU::ES;
  const uint32_t kvh = blockIdx.x, grp = blockIdx.y, b = blockIdx.z;
  const int32_t L = attn_row_len(a, b);
  const uint32_t cpb = a.cpb, c0 = grp * cpb;
  if ((int32_t)(c0 * ATT_CHUNK) >= L) return;      // the merge reads only live partials
  // phase clock: 0 entry, 1 first chunk's loads issued and q decoded, 2 first
  // chunk consumed, 3 chunks done, 4 row groups combined, 5 wave maxima in
  // LDS, 6 wave accumulators in LDS, 7 partial stored (drained)
  pclk(a.clk, a.clk_cap, 0);
  const int tid = threadIdx.x, wv = tid >> 6, lane = lane_id();
  const int rg = lane / LPR, li = lane % LPR;
  const uint32_t d0 = li * EPL;
  // this (row, kv head)'s cache rows as buffer resources: rows past L read
  // zero through an out-of-range offset, with no memory access, so the loads
  // of a chunk past the block's last are issued unconditionally
  const uint64_t cbase = ((uint64_t)attn_cache_row(a, b) * a.Hkv + kvh) * a.max_seq * HD * ES;
  const buf_t krs = buf_rsrc((const char *)a.kcache + cbase, a.max_seq * HD * ES);
  const buf_t vrs = buf_rsrc((const char *)a.vcache + cbase, a.max_seq * HD * ES);
  // the block's chunks c0 .. c0+nc-1; the ping-pong below issues one chunk
  // ahead unconditionally, and a row at or past jend takes the no-access
  // offset (past the block's last chunk it would re-read the next block's)
  const uint32_t nlive = (uint32_t)((L + ATT_CHUNK - 1) / ATT_CHUNK);
  const uint32_t nc = min(cpb, nlive - c0);            // block-uniform
  const int32_t jend = min(L, (int32_t)((c0 + nc) * ATT_CHUNK));
  uint4 kq[2][IT], vq[2][IT];
  bool ok[2][IT];
  auto issue = [&](int buf, uint32_t c) {
#pragma unroll
    for (int it = 0; it < IT; it++) {
      const uint32_t j = c * ATT_CHUNK + wv * PPW + it * RPW + rg;
      ok[buf][it] = (int32_t)j < jend && j < a.max_seq;
      const uint32_t off = ok[buf][it] ? (j * HD + d0) * ES : BUF_OOB;
      kq[buf][it] = buf_ld_stream16(krs, off);
      vq[buf][it] = buf_ld_stream16(vrs, off);
    }
  };
  // q's raw bytes requested ahead of the first chunk, so that decoding q waits
  // for q alone and the second chunk is issued while the first is in flight
  uint4 qraw[G];
#pragma unroll
  for (int g = 0; g < G; g++) {
    const uint64_t qo = ((uint64_t)b * a.H + kvh * G + g) * HD + d0;
    qraw[g] = ld16((const char *)a.q + qo * ES);
  }
  issue(0, c0);
  // q, decoded and pre-scaled into the log2 domain once
  const float qs = a.scale * LOG2E;
  float qf[G][EPL];
#pragma unroll
  for (int g = 0; g < G; g++) {
    chunk_f<AT>(qraw[g], qf[g]);
#pragma unroll
    for (int i = 0; i < EPL; i++) qf[g][i] *= qs;
  }
  pclk(a.clk, a.clk_cap, 1);
  float m[G], l[G], acc[G][EPL];
#pragma unroll
  for (int g = 0; g < G; g++) {
    m[g] = -INFINITY;
    l[g] = 0.0f;
#pragma unroll
    for (int i = 0; i < EPL; i++) acc[g][i] = 0.0f;
  }
  auto consume = [&](int buf) {
    float sc[IT][G];
#pragma unroll
    for (int it = 0; it < IT; it++) {
      float kf[EPL];
      chunk_f<AT>(kq[buf][it], kf);
#pragma unroll
      for (int g = 0; g < G; g++) {
        float sv = 0.0f;
#pragma unroll
        for (int i = 0; i < EPL; i++) sv += qf[g][i] * kf[i];
        sv = group_sum<LPR>(sv);
        sc[it][g] = ok[buf][it] ? sv : -INFINITY;
      }
    }
#pragma unroll
    for (int g = 0; g < G; g++) {
      float mn = m[g];
#pragma unroll
      for (int it = 0; it < IT; it++) mn = fmaxf(mn, sc[it][g]);
      const float f = m[g] == -INFINITY ? 0.0f : fexp2(m[g] - mn);
      l[g] *= f;
#pragma unroll
      for (int i = 0; i < EPL; i++) acc[g][i] *= f;
      m[g] = mn;
    }
#pragma unroll
    for (int it = 0; it < IT; it++) {
      float vf[EPL];
      chunk_f<AT>(vq[buf][it], vf);
#pragma unroll
      for (int g = 0; g < G; g++) {
        const float p = (ok[buf][it] && m[g] != -INFINITY) ? fexp2(sc[it][g] - m[g]) : 0.0f;
        l[g] += p;
#pragma unroll
        for (int i = 0; i < EPL; i++) acc[g][i] += p * vf[i];
      }
    }
  };
  for (uint32_t c = 0; c < nc; c += 2) {               // two register sets, ping-pong
    issue(1, c0 + c + 1);
    consume(0);
    if (c == 0) pclk(a.clk, a.clk_cap, 2);
    if (c + 1 >= nc) break;
    issue(0, c0 + c + 2);
    consume(1);
  }
  pclk(a.clk, a.clk_cap, 3);
  // row groups of the wave -> one (m, l, acc) per head: rescale to the wave
  // max, then sum (all lanes).  A row group is LPR lanes, so the groups of a
  // wave meet across lanes LPR, 2 LPR, .. 32 apart: a butterfly in that order,
  // 8 apart by a DPP row rotation, 16 and 32 apart by permlane swaps.
  static_assert(LPR == 8 || LPR == 16 || LPR == 32, "row groups of 8, 16 or 32 lanes");
  float mw[G];
#pragma unroll
  for (int g = 0; g < G; g++) {
    float M = m[g];
#pragma unroll
    for (int off = LPR; off < 64; off *= 2) M = fmaxf(M, attn_xor(M, off));
    const float f = m[g] == -INFINITY ? 0.0f : fexp2(m[g] - M);
    l[g] *= f;
#pragma unroll
    for (int i = 0; i < EPL; i++) acc[g][i] *= f;
#pragma unroll
    for (int off = LPR; off < 64; off *= 2) {
      l[g] += attn_xor(l[g], off);
#pragma unroll
      for (int i = 0; i < EPL; i++) acc[g][i] += attn_xor(acc[g][i], off);
    }
    mw[g] = M;
  }
  pclk(a.clk, a.clk_cap, 4);
  // waves -> the block's partial in one LDS round: each wave stores its (m, l)
  // and its accumulator relative to its own max; each output thread rescales
  // the 8 waves' terms to the block max and sums them in wave order (the same
  // products and the same order as rescaling first, so the same values)
  if (lane == 0) {
#pragma unroll
    for (int g = 0; g < G; g++) { s.wm[wv][g] = mw[g]; s.wl[wv][g] = l[g]; }
  }
  if (rg == 0) {
#pragma unroll
    for (int g = 0; g < G; g++)
#pragma unroll
      for (int i = 0; i < EPL; i++) s.wacc[wv][g][d0 + i] = acc[g][i];
  }
  __syncthreads();
  pclk(a.clk, a.clk_cap, 5);
  for (int o = tid; o < G * HD; o += ATT_THREADS) {
    const int g = o / HD, d = o % HD;
    float M = s.wm[0][g];
#pragma unroll
    for (int w = 1; w < ATT_WAVES; w++) M = fmaxf(M, s.wm[w][g]);
    float sv = 0.0f, lt = 0.0f;
#pragma unroll
    for (int w = 0; w < ATT_WAVES; w++) {
      const float mwv = s.wm[w][g];
      const float f = mwv == -INFINITY ? 0.0f : fexp2(mwv - M);
      sv += s.wacc[w][g][d] * f;
      lt += f * s.wl[w][g];
    }
    const uint64_t pi = (((uint64_t)b * a.H + kvh * G + g) * a.n_split + grp) * (HD + 2);
    if (FUSE) {
      coh_stf(a.part, (uint32_t)((pi + d) * 4), sv);
      if (d == 0) { coh_stf(a.part, (uint32_t)((pi + HD) * 4), M); coh_stf(a.part, (uint32_t)((pi + HD + 1) * 4), lt); }
    } else {
      float *pp = a.part + pi;
      pp[d] = sv;
      if (d == 0) { pp[HD] = M; pp[HD + 1] = lt; }
    }
  }
  if (FUSE) attn_handoff_merge<HD, G, AT>(a, b, kvh, attn_live(a, L), &last, &ms);
  pclk_end(a.clk, a.clk_cap);
}

// ---- the split on MFMA (batched decode, 16-bit caches) -------------------
// Where many split blocks run at once (batched decode) the VALU split is
// bound by its arithmetic, not by HBM: ~400 VALU instructions per 8 cache
// rows per wave for the dot products, the row-group DPP sums, the exp2s and
// the accumulator FMAs.  Here both products run on MFMA, a wave per 16-row
// tile of the cache (v_mfma_f32_16x16x32 for the scores, 16x16x16 for the
// weighted sum), with no LDS in the tile loop:
//   scores  S^T[row][head] = K[row][:] . q[head][:]: A = the K rows (lane l
//           holds row l%16, d = 8 (l/16) + 32 ks + j: one 16-byte load
//           straight from the cache), B = q^T (lane l holds head l%16, the
//           same d; heads past G are zero).  The result puts rows 4 (l/16)
//           + i and head l%16 in lane l;
//   softmax online per head over the block's tiles: the tile max over a
//           lane's 4 rows and the lanes 16 and 32 apart (permlane swaps),
//           p = exp2(s - m) in the log2 domain, the lane's own row sums;
//   mix     O^T[d][head] += V^T[d][rows] P^T[rows][head]: B = P^T is the
//           score layout itself (lane l: rows 4 (l/16) + j, head l%16), so
//           p needs no shuffle; A = V^T wants 4 rows of one column per lane,
//           so lane l loads rows 4 (l/16) + j, d 8 (l%16) .. +8 (four 16-byte
//           loads) and instruction e (0..7) takes column 8 (l%16) + e of its
//           4 rows (v_perm_b32 pairs): instruction e yields O^T[8 m + e]
//           [head] for m = 0..15 -- d permuted across the 8 instructions, and
//           the accumulator of head l%16 stays in lane l's group, so the
//           rescale by exp2(m_old - m_new) is lane-local (skipped when no
//           max of the wave moved).
// p enters as 16-bit hi + lo pairs (two MFMAs), so each weight keeps ~16
// significant bits against the exact 16-bit V value.  A block runs cpb
// chunks of 64 rows of one (row, kv head) as in the VALU form, tiles
// round-robin over its 8 waves with the next tile's K and V in flight; the
// waves meet once through LDS and the block writes the same partial (acc, m,
// l) the merge kernel folds.  Rows at or past the block's end read zero
// through the no-access offset (a stale cache row times a zero weight could
// still be a NaN).  GF > 0 (the one-launch form, G = GF heads per kv head):
// the partial goes out with system-scope stores and the last split block of
// the (row, kv head) merges the group's heads in the same launch, all at
// once (attn_handoff_merge: the per-head merge kernel's fold, so the same
// outputs as the two-launch form).
#define MF_GMAX 8
template <int HD, int AT, int GF = 0>
__global__ __launch_bounds__(ATT_THREADS) void k_attn_mf(ThvmAttnArgs a) {
  static_assert(AT == AT_BF16 || AT == AT_F16, "16-bit caches");
  constexpr int XT = AT == AT_BF16 ? GX_BF16 : GX_F16;
  constexpr int KS = HD / 32;                    // score k-steps
  constexpr int NC = HD / 8;                     // lane columns of the mix (8 d each)
  static_assert(HD == 64 || HD == 128, "head dim 64 or 128");
  __shared__ float wm[ATT_WAVES][MF_GMAX], wl[ATT_WAVES][MF_GMAX];
  __shared__ __align__(16) float wacc[ATT_WAVES][MF_GMAX][HD + 4];
  const uint32_t kvh = blockIdx.x, grp = blockIdx.y, b = blockIdx.z;
  const uint32_t G = a.H / a.Hkv;
  const int32_t L = attn_row_len(a, b);
  const uint32_t c0 = grp * a.cpb;
  if ((int32_t)(c0 * ATT_CHUNK) >= L) return;     // the merge reads only live partials
  pclk(a.clk, a.clk_cap, 0);
  // wv through readfirstlane: the compiler then knows it is wave-uniform, so
  // the tile loop below is a scalar loop rather than an exec-masked one
  const int tid = threadIdx.x, wv = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63, lc = lane & 15,
            lg = lane >> 4;
  const int32_t r0 = (int32_t)(c0 * ATT_CHUNK);
  const int32_t r1 = min(L, (int32_t)((c0 + a.cpb) * ATT_CHUNK));
  const int nt = (r1 - r0 + 15) / 16;             // 16-row tiles of the block
  const uint64_t cbase = ((uint64_t)attn_cache_row(a, b) * a.Hkv + kvh) * a.max_seq * HD * 2;
  const buf_t krs = buf_rsrc((const char *)a.kcache + cbase, a.max_seq * HD * 2);
  const buf_t vrs = buf_rsrc((const char *)a.vcache + cbase, a.max_seq * HD * 2);
  // q^T operands (head lc; heads past G read zero)
  const buf_t qrs = buf_rsrc((const char *)a.q + ((uint64_t)b * a.H + kvh * G) * HD * 2, G * HD * 2);
  uint4 qb[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ks++)
    qb[ks] = buf_ld16(qrs, (uint32_t)lc < G ? (uint32_t)(lc * HD + 8 * lg + 32 * ks) * 2 : BUF_OOB);
  uint4 kb[2][KS], vb[2][4];
  auto issue = [&](int buf, int t) {
    const int32_t rk = r0 + 16 * t + lc, rv = r0 + 16 * t + 4 * lg;
#pragma unroll
    for (int ks = 0; ks < KS; ks++)
      kb[buf][ks] = buf_ld_stream16(krs, rk < r1 ? (uint32_t)(rk * HD + 8 * lg + 32 * ks) * 2 : BUF_OOB);
#pragma unroll
    for (int j = 0; j < 4; j++)
      vb[buf][j] = buf_ld_stream16(vrs, rv + j < r1 && lc < NC ? (uint32_t)((rv + j) * HD + 8 * lc) * 2 : BUF_OOB);
  };
  const float qs = a.scale * LOG2E;
  float m = -INFINITY, l = 0.0f;
  f32x4_t acc[8];
#pragma unroll
  for (int e = 0; e < 8; e++) acc[e] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  auto tile = [&](int buf, int t) {
    f32x4_t sc = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < KS; ks++) sc = mfma16<XT>(kb[buf][ks], qb[ks], sc);
    const int32_t rb = r0 + 16 * t + 4 * lg;
    float sv[4];
#pragma unroll
    for (int i = 0; i < 4; i++) sv[i] = rb + i < r1 ? sc[i] * qs : -INFINITY;
    float mx = fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3]));
    mx = fmaxf(mx, xor16_f(mx));
    mx = fmaxf(mx, xor32_f(mx));
    const float mn = fmaxf(m, mx);
    const float f = m == -INFINITY ? 0.0f : fexp2(m - mn);
    float p[4];
#pragma unroll
    for (int i = 0; i < 4; i++) p[i] = sv[i] == -INFINITY ? 0.0f : fexp2(sv[i] - mn);
    l = l * f + ((p[0] + p[1]) + (p[2] + p[3]));
    m = mn;
    if (__builtin_amdgcn_ballot_w64(f != 1.0f)) {
#pragma unroll
      for (int e = 0; e < 8; e++)
#pragma unroll
        for (int i = 0; i < 4; i++) acc[e][i] *= f;
    }
    // P^T operands: hi = rnd(p), lo = rnd(p - hi) (p - hi exact in f32)
    uint32_t ph[2], pl[2];
#pragma unroll
    for (int h = 0; h < 2; h++) {
      if (AT == AT_BF16) {
        ph[h] = pk_bf16(p[2 * h], p[2 * h + 1]);
        pl[h] = pk_bf16(p[2 * h] - __uint_as_float(ph[h] << 16), p[2 * h + 1] - __uint_as_float(ph[h] & 0xffff0000u));
      } else {
        ph[h] = pk_f16(p[2 * h], p[2 * h + 1]);
        pl[h] = pk_f16(p[2 * h] - h2f((f16_t)(ph[h] & 0xffffu)), p[2 * h + 1] - h2f((f16_t)(ph[h] >> 16)));
      }
    }
    const uint32_t w[4][4] = {{vb[buf][0].x, vb[buf][0].y, vb[buf][0].z, vb[buf][0].w},
                              {vb[buf][1].x, vb[buf][1].y, vb[buf][1].z, vb[buf][1].w},
                              {vb[buf][2].x, vb[buf][2].y, vb[buf][2].z, vb[buf][2].w},
                              {vb[buf][3].x, vb[buf][3].y, vb[buf][3].z, vb[buf][3].w}};
#pragma unroll
    for (int e = 0; e < 8; e++) {
      // column 8 lc + e of rows 0..3: the low (e even) or high half of dword e/2
      const uint32_t sel = (e & 1) ? 0x07060302u : 0x05040100u;
      const uint32_t a01 = __builtin_amdgcn_perm(w[1][e >> 1], w[0][e >> 1], sel);
      const uint32_t a23 = __builtin_amdgcn_perm(w[3][e >> 1], w[2][e >> 1], sel);
      acc[e] = mfma16x16<XT>(a01, a23, ph[0], ph[1], acc[e]);
      acc[e] = mfma16x16<XT>(a01, a23, pl[0], pl[1], acc[e]);
    }
  };
  if (nt <= ATT_WAVES) {                          // at most one tile per wave (block-uniform)
    issue(0, wv);
    if (wv < nt) tile(0, wv);
  } else {
    // q, then the two register sets, in this issue order (scheduling
    // barriers: with q scheduled after the rows, the wait for q at the loop
    // head drained every load in flight, in every iteration)
    __builtin_amdgcn_sched_barrier(0);
    issue(0, wv);
    __builtin_amdgcn_sched_barrier(0);
    issue(1, wv + ATT_WAVES);
    __builtin_amdgcn_sched_barrier(0);
    // two register sets, ping-pong: each tile waits only for its own rows,
    // the other set's stay in flight.  Past the block's rows the second tile
    // is skipped but the loop goes on to its end (the loads then read
    // zeros): an early exit there split the loop state so that the loop head
    // waited for every load in flight.
    for (int t = wv; t < nt; t += 2 * ATT_WAVES) {
      tile(0, t);
      __builtin_amdgcn_sched_barrier(0);
      issue(0, t + 2 * ATT_WAVES);
      __builtin_amdgcn_sched_barrier(0);
      if (t + ATT_WAVES < nt) tile(1, t + ATT_WAVES);   // wave-uniform
      __builtin_amdgcn_sched_barrier(0);
      issue(1, t + 3 * ATT_WAVES);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  pclk(a.clk, a.clk_cap, 3);
  // a head's rows are spread over the lanes 16 and 32 apart
  l += xor16_f(l);
  l += xor32_f(l);
  if (lg == 0 && (uint32_t)lc < G) { wm[wv][lc] = m; wl[wv][lc] = l; }
  if ((uint32_t)lc < G) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int mm = 4 * lg + i;                    // d = 8 mm + e
      if (mm < NC) {
        *(float4 *)&wacc[wv][lc][8 * mm] = make_float4(acc[0][i], acc[1][i], acc[2][i], acc[3][i]);
        *(float4 *)&wacc[wv][lc][8 * mm + 4] = make_float4(acc[4][i], acc[5][i], acc[6][i], acc[7][i]);
      }
    }
  }
  __syncthreads();
  pclk(a.clk, a.clk_cap, 5);
  for (int o = tid; o < (int)(G * HD); o += ATT_THREADS) {
    const int g = o / HD, d = o % HD;
    float M = wm[0][g];
#pragma unroll
    for (int w = 1; w < ATT_WAVES; w++) M = fmaxf(M, wm[w][g]);
    float sv = 0.0f, lt = 0.0f;
#pragma unroll
    for (int w = 0; w < ATT_WAVES; w++) {
      const float mw = wm[w][g];
      const float f = mw == -INFINITY ? 0.0f : fexp2(mw - M);
      sv += wacc[w][g][d] * f;
      lt += f * wl[w][g];
    }
    const uint64_t pi = (((uint64_t)b * a.H + kvh * G + g) * a.n_split + grp) * (HD + 2);
    if (GF) {
      coh_stf(a.part, (uint32_t)((pi + d) * 4), sv);
      if (d == 0) {
        coh_stf(a.part, (uint32_t)((pi + HD) * 4), M);
        coh_stf(a.part, (uint32_t)((pi + HD + 1) * 4), lt);
      }
    } else {
      float *pp = a.part + pi;
      pp[d] = sv;
      if (d == 0) { pp[HD] = M; pp[HD + 1] = lt; }
    }
  }
  if (GF) {
    __shared__ MergeFlatLds<HD, 1> ms[GF ? GF : 1];
    __shared__ uint32_t last;
    attn_handoff_merge<HD, (GF ? GF : 1), AT, true>(a, b, kvh, attn_live(a, L), &last, ms);
  }
  pclk_end(a.clk, a.clk_cap);
}

typedef void (*attn_fn)(ThvmAttnArgs);
// (G = 8 heads per kv head would spill its accumulators: one chunk per block)
template <int HD, int AT>
static attn_fn attn_pick_multi(uint32_t G, bool fused) {
  switch (G) {
    case 1: return fused ? k_attn_multi<HD, 1, AT, true> : k_attn_multi<HD, 1, AT, false>;
    case 2: return fused ? k_attn_multi<HD, 2, AT, true> : k_attn_multi<HD, 2, AT, false>;
    case 4: return fused ? k_attn_multi<HD, 4, AT, true> : k_attn_multi<HD, 4, AT, false>;
    default: return nullptr;
  }
}
template <int HD, int G, int AT>
static attn_fn attn_pick_merge_mc(uint32_t mc) {
  return mc <= 4 ? k_attn_merge<HD, G, AT, 4> : mc <= 8 ? k_attn_merge<HD, G, AT, 8> : k_attn_merge<HD, G, AT, MCH>;
}
// the merge for G heads per group and nmax partials: the load batch MC just
// covers a partition's share of the partials (the loads past it would read
// slot 0 again for nothing -- at 8 blocks the merge is bound by its load
// instructions, not by bytes), at most MCH
template <int HD, int AT>
static attn_fn attn_pick_merge(uint32_t G, uint32_t nmax) {
  const uint32_t np = MERGE_THREADS / (G * HD / 2), mc = (nmax + np - 1) / np;
  switch (G) {
    case 1: return attn_pick_merge_mc<HD, 1, AT>(mc);
    case 2: return attn_pick_merge_mc<HD, 2, AT>(mc);
    case 4: return attn_pick_merge_mc<HD, 4, AT>(mc);
    case 8: return attn_pick_merge_mc<HD, 8, AT>(mc);
    default: return nullptr;
  }
}
template <int HD, int AT>
static attn_fn attn_pick(uint32_t G, bool fused) {
  switch (G) {
    case 1: return fused ? k_attn_fused<HD, 1, AT> : k_attn<HD, 1, AT>;
    case 2: return fused ? k_attn_fused<HD, 2, AT> : k_attn<HD, 2, AT>;
    case 4: return fused ? k_attn_fused<HD, 4, AT> : k_attn<HD, 4, AT>;
    case 8: return fused ? k_attn_fused<HD, 8, AT> : k_attn<HD, 8, AT>;
    default: return nullptr;
  }
}

// partials [B][H][n_split][hd + 2] f32, then the fused form's B*Hkv merge
// counters (zero-filled with the buffer; each merge resets its own)
extern "C" uint64_t thvm_k_attn_part_bytes(uint32_t B, uint32_t H, uint32_t Hkv, uint32_t hd,
                                           uint32_t n_split) {
  return (uint64_t)B * H * n_split * (hd + 2) * 4 + (uint64_t)B * Hkv * 4;
}

// chunks per split block for cpb = 0: one at small unit counts (every CU
// needs a block); at batched shapes 2 or more, so each block's fixed work is
// shared by more cache rows.  (Measured on gfx950 at the C4 shapes: two
// chunks per block beat one at every unit count -- 11.3 against 12.9 us per
// launch at batch 1, where the merge also reads half the partials.  Above
// 1024 units the chunk count keeps the grid within one round of 2 blocks per
// CU, so no tail round of a few blocks is left: 9 chunks at C4 batch 16.
// With at most 4 chunks per head and a grid of at most one such round, the
// merge has little to save and one chunk per block runs the chunks side by
// side: C3 batch 1 (4 chunks, 100 units) 1.818 -> 1.785 ms per step.)  A
// speculative verify passes its base step's value explicitly, so that its
// rows fold the same partials in the same order as the base step.
extern "C" uint32_t thvm_k_attn_auto_cpb(uint32_t B, uint32_t H, uint32_t Hkv, uint32_t n_split,
                                         uint32_t fused) {
  if (Hkv == 0 || n_split == 0) return 1;
  const uint64_t units = (uint64_t)B * Hkv * n_split;
  const uint32_t bh = B * Hkv, groups = bh >= 512 ? 1u : 512u / bh;   // split blocks per (row, kv head)
  (void)fused;
  uint32_t cpb = (H / Hkv > 4 || (n_split <= 4 && units <= 512)) ? 1
               : units > 1024 ? (n_split + groups - 1) / groups : 2;
  return cpb > n_split ? n_split : cpb;
}

// shapes the MFMA split takes
static bool attn_mf_can(const ThvmAttnArgs *a) {
  const uint32_t G = a->Hkv ? a->H / a->Hkv : 0;
  return a->cdt != THVM_DT_FP32 && (a->hd == 64 || a->hd == 128) && G >= 1 && G <= MF_GMAX &&
         (G & (G - 1)) == 0;
}

// chunks per block of the MFMA split for cpb = 0: the grid one round of
// blocks per CU where the rows allow (at most 256 blocks of 8 waves)
static uint32_t attn_mf_cpb(const ThvmAttnArgs *a) {
  const uint32_t bh = a->B * a->Hkv, groups = bh >= 256 ? 1u : 256u / bh;
  const uint32_t cpb = (a->n_split + groups - 1) / groups;
  return cpb < 1 ? 1 : cpb;
}

// The split a launch with these arguments runs (*mf: 1 the MFMA split, 0
// the VALU forms) and its chunks per block.  The MFMA split is picked
// wherever it applies (measured on gfx950 at the C4 head shape, split +
// merge per launch in a graph: batch 1 10.3 against 12.3 us, batch 4 15.1
// against 20.3, batch 16 31.5 against 38.4), except where the VALU split
// runs as one launch by default (at most 8 chunks: the kernel boundary it
// saves outweighs its arithmetic, C3 and C1) and in a speculative verify,
// whose rows follow the base step's plan, passed explicitly (mf, cpb).
extern "C" void thvm_k_attn_plan(const ThvmAttnArgs *a, uint32_t *mf, uint32_t *cpb) {
  const bool one_launch = a->fused == 1 || (a->fused == 2 && a->n_split <= 8);
  const bool use = a->mf == 1 || (a->mf == 0 && !a->spec && !one_launch && attn_mf_can(a));
  uint32_t c = a->cpb;
  if (c > a->n_split) c = a->n_split;
  if (c == 0) c = use ? attn_mf_cpb(a) : thvm_k_attn_auto_cpb(a->B, a->H, a->Hkv, a->n_split, one_launch);
  *mf = use ? 1u : 0u;
  *cpb = c;
}

// the one-launch MFMA split for G heads per kv head
template <int HD, int AT>
static attn_fn attn_pick_mf_fused(uint32_t G) {
  switch (G) {
    case 1: return k_attn_mf<HD, AT, 1>;
    case 2: return k_attn_mf<HD, AT, 2>;
    case 4: return k_attn_mf<HD, AT, 4>;
    case 8: return k_attn_mf<HD, AT, 8>;
    default: return nullptr;
  }
}

static int attn_mf_launch(const ThvmAttnArgs *a, hipStream_t s, char *err, int errlen) {
  const uint32_t G = a->H / a->Hkv;
  const int at = a->cdt == THVM_DT_BF16 ? AT_BF16 : AT_F16;
  if (a->fused == 1) {                            // split and merge in one launch
    attn_fn ff = a->hd == 128 ? (at == AT_BF16 ? attn_pick_mf_fused<128, AT_BF16>(G) : attn_pick_mf_fused<128, AT_F16>(G))
                              : (at == AT_BF16 ? attn_pick_mf_fused<64, AT_BF16>(G) : attn_pick_mf_fused<64, AT_F16>(G));
    if (!ff) { snprintf(err, errlen, "attn: no one-launch MFMA split for G=%u", G); return -1; }
    if ((uint64_t)a->B * a->H * a->n_split * (a->hd + 2) * 4 >= (1ull << 31)) {
      snprintf(err, errlen, "attn: partials of 2 GiB or more");
      return -1;
    }
    ThvmAttnArgs ak = *a;
    uint32_t mf = 0;
    thvm_k_attn_plan(a, &mf, &ak.cpb);
    thvm_launch(true, true, ff, dim3(a->Hkv, (a->n_split + ak.cpb - 1) / ak.cpb, a->B), dim3(ATT_THREADS), 0, s, ak);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) { snprintf(err, errlen, "attn launch: %s", hipGetErrorString(e)); return -1; }
    return 0;
  }
  attn_fn f = a->hd == 128 ? (at == AT_BF16 ? k_attn_mf<128, AT_BF16> : k_attn_mf<128, AT_F16>)
                           : (at == AT_BF16 ? k_attn_mf<64, AT_BF16> : k_attn_mf<64, AT_F16>);
  // the merge: one block per (row, query head) -- the G = 1 merge over the
  // per-head partials, each query head taken as its own group, with a load
  // batch sized to the partials (C4 batch 16: 2.990 -> 2.981 ms per step;
  // batch 1, against one block per (row, kv head): 1.984 -> 1.936 ms, the 8
  // group blocks were bound by their load instructions).  Every MFMA form
  // (the one-launch form and a speculative verify included) folds this way.
  ThvmAttnArgs ak = *a;
  uint32_t mf = 0;
  thvm_k_attn_plan(a, &mf, &ak.cpb);
  const uint32_t nmax = (a->n_split + ak.cpb - 1) / ak.cpb;
  attn_fn fm = a->hd == 128 ? (at == AT_BF16 ? attn_pick_merge<128, AT_BF16>(1, nmax) : attn_pick_merge<128, AT_F16>(1, nmax))
                            : (at == AT_BF16 ? attn_pick_merge<64, AT_BF16>(1, nmax) : attn_pick_merge<64, AT_F16>(1, nmax));
  if (!fm) { snprintf(err, errlen, "attn: no merge kernel for G=%u", G); return -1; }
  if ((uint64_t)a->B * a->H * a->n_split * (a->hd + 2) * 4 >= (1ull << 31)) {
    snprintf(err, errlen, "attn: partials of 2 GiB or more");
    return -1;
  }
  thvm_launch(true, false, f, dim3(a->Hkv, (a->n_split + ak.cpb - 1) / ak.cpb, a->B), dim3(ATT_THREADS), 0, s, ak);
  ThvmAttnArgs am = ak;
  am.Hkv = a->H;                                  // groups of one head
  thvm_launch(false, true, fm, dim3(a->B * am.Hkv), dim3(MERGE_THREADS), 0, s, am);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) { snprintf(err, errlen, "attn launch: %s", hipGetErrorString(e)); return -1; }
  return 0;
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
  // fused = 1: the last split block of a (row, kv head) merges in the same
  // launch; 0: a second launch merges; 2 (the shape's pick): one launch for
  // caches of at most 8 chunks (512 rows), two above.  Measured in a graph on
  // gfx950: one launch wins at short caches (C3 B=1 1.809 -> 1.767 ms, C3 B=8
  // 2.372 -> 2.285, C1 0.396 -> 0.390 ms per step), two launches at long ones
  // (C4: 11.1 against 11.9 us at L = 2051; B=16 3.50 against 3.59 ms).
  if (a->fused > 2) { snprintf(err, errlen, "attn: fused must be 0, 1 or 2"); return -1; }
  if (a->mf > 2) { snprintf(err, errlen, "attn: mf must be 0, 1 or 2"); return -1; }
  {
    const uint32_t G = a->H / a->Hkv;
    if (a->mf == 1 && !attn_mf_can(a)) {
      snprintf(err, errlen, "attn: the MFMA split takes 16-bit caches, hd 64 or 128, G in 1, 2, 4, 8 "
               "(hd=%u G=%u)", a->hd, G);
      return -1;
    }
    uint32_t mf = 0, cpb = 0;
    thvm_k_attn_plan(a, &mf, &cpb);
    if (mf) return attn_mf_launch(a, s, err, errlen);
  }
  const bool fused = a->fused == 1 || (a->fused == 2 && a->n_split <= 8);
  uint32_t cpb = a->cpb;
  if (cpb > a->n_split) cpb = a->n_split;          // one block takes every chunk
  if (cpb == 0) cpb = thvm_k_attn_auto_cpb(a->B, a->H, a->Hkv, a->n_split, fused);
  attn_fn f = nullptr, fm = nullptr;
  const uint32_t G = a->H / a->Hkv;
  const int at = a->cdt == THVM_DT_BF16 ? AT_BF16 : a->cdt == THVM_DT_FP16 ? AT_F16 : AT_F32;
  const uint32_t nmax = (a->n_split + cpb - 1) / cpb;     // the merge's partial slots
  if (a->hd == 128) {
    f = cpb > 1 ? (at == AT_BF16 ? attn_pick_multi<128, AT_BF16>(G, fused) : at == AT_F16 ? attn_pick_multi<128, AT_F16>(G, fused) : attn_pick_multi<128, AT_F32>(G, fused))
        : at == AT_BF16 ? attn_pick<128, AT_BF16>(G, fused) : at == AT_F16 ? attn_pick<128, AT_F16>(G, fused) : attn_pick<128, AT_F32>(G, fused);
    fm = at == AT_BF16 ? attn_pick_merge<128, AT_BF16>(G, nmax) : at == AT_F16 ? attn_pick_merge<128, AT_F16>(G, nmax) : attn_pick_merge<128, AT_F32>(G, nmax);
  } else if (a->hd == 64) {
    f = cpb > 1 ? (at == AT_BF16 ? attn_pick_multi<64, AT_BF16>(G, fused) : at == AT_F16 ? attn_pick_multi<64, AT_F16>(G, fused) : attn_pick_multi<64, AT_F32>(G, fused))
        : at == AT_BF16 ? attn_pick<64, AT_BF16>(G, fused) : at == AT_F16 ? attn_pick<64, AT_F16>(G, fused) : attn_pick<64, AT_F32>(G, fused);
    fm = at == AT_BF16 ? attn_pick_merge<64, AT_BF16>(G, nmax) : at == AT_F16 ? attn_pick_merge<64, AT_F16>(G, nmax) : attn_pick_merge<64, AT_F32>(G, nmax);
  }
  if (!f || !fm) {
    snprintf(err, errlen, "attn: no kernel for hd=%u G=%u cpb=%u", a->hd, G, cpb);
    return -1;
  }
  if ((uint64_t)a->B * a->H * a->n_split * (a->hd + 2) * 4 >= (1ull << 31)) {
    snprintf(err, errlen, "attn: partials of 2 GiB or more");
    return -1;
  }
  ThvmAttnArgs ak = *a;
  ak.cpb = cpb;
  thvm_launch(true, fused, f, dim3(a->Hkv, (a->n_split + cpb - 1) / cpb, a->B), dim3(ATT_THREADS), 0, s, ak);
  if (!fused) thvm_launch(false, true, fm, dim3(a->B * a->Hkv), dim3(MERGE_THREADS), 0, s, ak);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) { snprintf(err, errlen, "attn launch: %s", hipGetErrorString(e)); return -1; }
  return 0;
}

// ---- attention without a caller-provided workspace --------------------------
// For callers that cannot allocate device memory (code under graph capture,
// serving loops, harnesses that forbid hipMalloc): the partials and merge
// counters live in a file-scope device array of THVM_ATTN_SCRATCH_BYTES, one
// copy per GPU, held until the process ends.  Its device address comes from
// hipGetSymbolAddress, taken once per device at set-up with that device
// current; host code never passes the array's name to a kernel (in host code
// it is a stand-in symbol, not a device address).  Every call on a GPU shares
// that GPU's array: calls that overlap on one GPU race.
#define THVM_K_MAX_DEVICES 16
static __device__ __align__(256) unsigned char scratch[THVM_ATTN_SCRATCH_BYTES];
static void *SCRATCH_PTR[THVM_K_MAX_DEVICES];

extern "C" int thvm_k_attn_scratch_setup(char *err, int errlen) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess || dev < 0 || dev >= THVM_K_MAX_DEVICES) {
    snprintf(err, errlen, "attn scratch: current device %d: %s", dev, hipGetErrorString(e));
    return -1;
  }
  if (SCRATCH_PTR[dev]) return 0;
  void *p = nullptr;
  e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (e != hipSuccess || p == nullptr) {
    snprintf(err, errlen, "attn scratch: hipGetSymbolAddress: %s", hipGetErrorString(e));
    return -1;
  }
  SCRATCH_PTR[dev] = p;
  return 0;
}

extern "C" int thvm_k_attn_decode_scratch(const ThvmAttnArgs *a, hipStream_t s, char *err,
                                          int errlen) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= THVM_K_MAX_DEVICES ||
      SCRATCH_PTR[dev] == nullptr) {
    snprintf(err, errlen, "attn (no-alloc): scratch not set up on device %d (thvm_hip_init)", dev);
    return -1;
  }
  const uint64_t need = thvm_k_attn_part_bytes(a->B, a->H, a->Hkv, a->hd, a->n_split);
  if (need > (uint64_t)THVM_ATTN_SCRATCH_BYTES) {
    snprintf(err, errlen,
             "attn (no-alloc): needs %llu bytes of partials (B=%u H=%u hd=%u n_split=%u), the "
             "static scratch holds %u",
             (unsigned long long)need, a->B, a->H, a->hd, a->n_split, THVM_ATTN_SCRATCH_BYTES);
    return -1;
  }
  ThvmAttnArgs ak = *a;
  ak.part = (float *)SCRATCH_PTR[dev];
  // the one-launch form's merge counters (after the partials) must start at
  // zero; the two-launch form's merge reads only partials this call writes
  if (ak.fused) {
    const uint64_t cnt = (uint64_t)a->B * a->Hkv * 4;
    if (thvm_k_zero((char *)SCRATCH_PTR[dev] + (need - cnt), cnt, s, err, errlen)) return -1;
  }
  return thvm_k_attn_decode(&ak, s, err, errlen);
}
