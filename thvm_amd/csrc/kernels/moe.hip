// moe.hip -- DeepSeek-V2 mixture-of-experts decode on gfx950: router top-K
// and the routed + shared expert FFN with an index gather on the weights.
//
// Replaces the reference's route (bench/dsv2_decode_bench.c :787-863),
// moe_full_h (:865-910) and moe_full_out (:912-965).  Design for gfx950:
//   * k_route: one wave per batch row; lane e holds gate logit e, the max and
//     the softmax denominator are DPP wave reductions, each of the K rounds is
//     a butterfly arg-max over (value desc, index asc) -- the same winner as
//     the reference's serial scan (ties to the lowest expert id);
//   * k_moe_gateup: one wave per (gate_i, up_i) row pair of a selected (or
//     shared) expert; the expert id is read from sel on the device, so the
//     gather is an address computation, not a copy; the row loads are issued
//     before x is staged into LDS (x rounded to bf16, the experts' input
//     dtype), 16-byte nontemporal loads, fp8 decoded with v_cvt_pk_f32_fp8,
//     h = silu(g)*u kept in f32 as the reference keeps it;
//   * k_moe_down: one wave per output row d; the K routed segments (row d of
//     each selected expert's down matrix) and the shared segment are all in
//     flight before any arithmetic, h sits in LDS, the weighted sum follows
//     the reference's order (routed slots ascending, then shared) and the
//     residual add rounds like the reference's mm-out + add chain.
#include "dev_common.h"
#include "mfma_ops.h"
#include "../kern_api.h"
#include "launch.h"
#include <stdio.h>
#include <limits.h>

#define MOE_WAVES 8
#define MOE_THREADS (64 * MOE_WAVES)
#define MOE_MAXC 4      /* 16-byte chunks per lane per row: rows up to 4 KiB */
#define MOE_MAXCS 8     /* the shared-expert down row: up to 8 KiB */
#define MOE_MAXK 8      /* routed experts per token */

// ---- router ---------------------------------------------------------------
// top-K of one row's E <= 64 logits by one wave (lane e holds logit e):
// every lane ends with the K ids and probabilities.  The order is the
// reference's serial scan: value descending, ties to the lowest expert id
// (finite logits; NaN ones are put after every number, by id).  Each lane
// builds a 64-bit key that orders its logit that way -- class (number 2,
// NaN 1, lane past E 0), the order-preserving bits of the value (-0 taken
// as +0, so the two tie), 63 - lane -- and counts the keys above its own
// through LDS, 16 keys per batch of reads (all distinct: the rank of its
// logit); slot k is the lane of rank k (a ballot).  (K rounds of a wave max
// and a ballot each were a dependent chain of DPP steps on one wave.)
__device__ __forceinline__ void route_wave(float g, uint32_t lane, uint32_t E, uint32_t K,
                                           int32_t (&ids)[MOE_MAXK], float (&pr)[MOE_MAXK]) {
  __shared__ __align__(16) uint64_t rkey[64];
  const float mx = wave_max(g);
  const float pe = lane < E ? expf(g - mx) : 0.0f;   // each lane's numerator, computed once
  const float sum = wave_sum(pe);
  const uint32_t gb = __float_as_uint(g + 0.0f);       // -0 -> +0
  const uint32_t ord = (gb & 0x80000000u) ? ~gb : (gb | 0x80000000u);
  const uint64_t cls = lane >= E ? 0ull : (g != g) ? 1ull : 2ull;
  const uint64_t key = (cls << 38) | ((cls == 2ull ? (uint64_t)ord : 0ull) << 6) | (63u - lane);
  rkey[lane] = key;
  // one wave writes and reads the keys, and its LDS operations complete in
  // order: only the compiler must keep the order
  __builtin_amdgcn_wave_barrier();
  asm volatile("" ::: "memory");
  uint32_t rank = 0;
#pragma unroll 1
  for (int jb = 0; jb < 64; jb += 16) {
    uint4 kv[8];
#pragma unroll
    for (int i = 0; i < 8; i++) kv[i] = *(const uint4 *)&rkey[jb + 2 * i];
#pragma unroll
    for (int i = 0; i < 8; i++)
      rank += (((uint64_t)kv[i].y << 32 | kv[i].x) > key ? 1u : 0u) +
              (((uint64_t)kv[i].w << 32 | kv[i].z) > key ? 1u : 0u);
  }
  const float pl = pe / sum;                           // every lane's probability, in parallel
#pragma unroll
  for (uint32_t kk = 0; kk < MOE_MAXK; kk++) {
    if (kk >= K) break;
    const uint64_t m = __ballot(rank == kk);           // exactly one lane
    const int bi = m ? (int)__builtin_ctzll(m) : 0;
    ids[kk] = bi;
    pr[kk] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(pl), bi));   // expf(g_bi - mx) / sum
  }
  __builtin_amdgcn_wave_barrier();                     // rkey is rewritten by the next call
  asm volatile("" ::: "memory");
}

__global__ __launch_bounds__(64) void k_route(ThvmRouteArgs a) {
  const uint32_t b = blockIdx.x, lane = threadIdx.x, E = a.E;
  const float g = lane < E ? a.logits[(uint64_t)b * E + lane] : -INFINITY;
  int32_t ids[MOE_MAXK];
  float pr[MOE_MAXK];
  route_wave(g, lane, E, a.K, ids, pr);
  if (lane == 0)
#pragma unroll
    for (uint32_t kk = 0; kk < MOE_MAXK; kk++)
      if (kk < a.K) { a.sel[(uint64_t)b * a.K + kk] = ids[kk]; a.probs[(uint64_t)b * a.K + kk] = pr[kk]; }
}

// The post-attention RMSNorm (f32 out) and the f32 router GEMV in one
// launch: grid (ceil(E / EPB), B), 512 threads (256 at EPB = 1); each block renormalises its
// row (the first 256 threads exactly as the norm kernel: the same elements
// per thread, the same block sum over four waves, the same formula) and its
// first EPB waves take one expert each, lane l folding 16-byte chunks l,
// l + 64, ... in order (four FMAs each) with one wave sum -- the GEMV's f32
// path -- so xn and the logits are those kernels' bits.  The expert row is
// in flight before the norm starts.  EPB = 1 for a few rows (64 blocks at
// batch 1, each reading 8 KiB of router row and ~12 KiB of x and gains;
// eight experts per block left 8 CUs pulling 76 KiB each: 2.87 -> 2.71 us
// per launch in the phase clock), else 8.
#define RT_THREADS 512
#define RT_WAVES (RT_THREADS / 64)
#define RT_NORM_THREADS 256
#define RT_NREG 16       /* x elements per norm thread: D <= 4096 */
template <int NCH, int EPB>   /* 16-byte router chunks per lane: D <= 256 * NCH; experts per block */
__global__ __launch_bounds__(RT_THREADS) void k_moe_gate(ThvmGateArgs a) {
  __shared__ __align__(16) float xs[RT_NREG * RT_NORM_THREADS];
  __shared__ float red[RT_NORM_THREADS / 64];
  const uint32_t b = blockIdx.y, tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const uint32_t D = a.D, E = a.E, C = D / 4;
  const bool ew = wv < (uint32_t)EPB;                 // a wave with an expert
  const uint32_t e = blockIdx.x * EPB + (ew ? wv : 0u);
  // phase clock: 0 entry, 1 loads issued, 2 x normalised in LDS, 7 drained
  pclk(a.clk, a.clk_cap, 0);
  const float4 *W = (const float4 *)a.gate;
  const uint64_t xo = (uint64_t)b * D;
  const float invK = 1.0f / (float)D;
  // x and the gains first: the loads return in issue order, so the norm
  // runs while the expert rows are in flight.  Every load is an unguarded
  // buffer load (out-of-range offsets read zero with no access: threads past
  // the norm's 256, elements past D, experts past E), so no load is branched
  // around and each wait counts only the loads it needs.
  const buf_t xr = buf_rsrc((const bf16_t *)a.x + xo, D * 2u);
  const buf_t gr = buf_rsrc(a.w, a.w ? D * 4u : 0u);
  const buf_t wr = buf_rsrc(W, E * C * 16u);
  uint32_t xb[RT_NREG], gb[RT_NREG];
#pragma unroll
  for (int i = 0; i < RT_NREG; i++) {
    const uint32_t k = tid + i * RT_NORM_THREADS;
    const bool ok = tid < RT_NORM_THREADS && k < D;
    xb[i] = buf_ld2(xr, ok ? k * 2u : BUF_OOB);
    gb[i] = buf_ld4(gr, ok ? k * 4u : BUF_OOB);
  }
  uint4 wq[NCH];
#pragma unroll
  for (int t = 0; t < NCH; t++) {
    const uint32_t c = lane + 64u * t;
    wq[t] = buf_ld_stream16(wr, ew && e < E && c < C ? (e * C + c) * 16u : BUF_OOB);
  }
  pclk(a.clk, a.clk_cap, 1);
  float xv[RT_NREG], gw[RT_NREG];
#pragma unroll
  for (int i = 0; i < RT_NREG; i++) {
    xv[i] = bf2f((bf16_t)xb[i]);               // 0 past D
    gw[i] = a.w ? __uint_as_float(gb[i]) : 1.0f;
  }
  if (tid < RT_NORM_THREADS) {
    float s2 = 0.0f;
#pragma unroll
    for (int i = 0; i < RT_NREG; i++) s2 += xv[i] * xv[i];
    const float w = wave_sum(s2);
    if (lane == 0) red[wv] = w;
  }
  __syncthreads();
  if (tid < RT_NORM_THREADS) {
    float t = 0.0f;
#pragma unroll
    for (int i = 0; i < RT_NORM_THREADS / 64; i++) t += red[i];
    const float inv = 1.0f / sqrtf(t * invK + a.eps);
#pragma unroll
    for (int i = 0; i < RT_NREG; i++) {
      const uint32_t k = tid + i * RT_NORM_THREADS;
      if (k < D) {
        float v = (xv[i] - 0.0f) * inv;
        if (a.w) v = v * gw[i];
        xs[k] = v;
        if (blockIdx.x == 0) a.xn[xo + k] = v;
      }
    }
  }
  __syncthreads();
  pclk(a.clk, a.clk_cap, 2);
  const float4 *x4 = (const float4 *)xs;
  float acc = 0.0f;
#pragma unroll
  for (int t = 0; t < NCH; t++) {
    const uint32_t c = lane + 64u * t;
    if (c < C) {
      const float4 v4 = x4[c];
      acc += v4.x * __uint_as_float(wq[t].x);
      acc += v4.y * __uint_as_float(wq[t].y);
      acc += v4.z * __uint_as_float(wq[t].z);
      acc += v4.w * __uint_as_float(wq[t].w);
    }
  }
  const float tot = wave_sum(acc);
  if (ew && e < E && lane == 0) a.logits[(uint64_t)b * E + e] = tot * 1.0f + 0.0f;   // the GEMV epilogue's scale, bias
  pclk_end(a.clk, a.clk_cap);
}

// decode one 16-byte chunk: 16 fp8 or 8 bf16 weights
template <bool FP8>
__device__ __forceinline__ void chunk_f32(const uint4 &q, float o[16]) {
  if (FP8) {
    fp8x4_to_f32(q.x, o); fp8x4_to_f32(q.y, o + 4);
    fp8x4_to_f32(q.z, o + 8); fp8x4_to_f32(q.w, o + 12);
  } else {
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int i = 0; i < 4; i++) {
      o[2 * i] = __uint_as_float(w[i] << 16);
      o[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
  }
}

// dot of one row's chunks held by this lane with the chunk-swizzled LDS
// vector v of nch chunks (chunk_swz layout)
template <bool FP8, int NC>
__device__ __forceinline__ float chunk_dot(const uint4 (&q)[NC], const float *v,
                                           uint32_t lane, uint32_t nch) {
  constexpr uint32_t EPC = FP8 ? 16 : 8;
  const float4 *v4 = (const float4 *)v;
  float acc = 0.0f;
#pragma unroll
  for (int c = 0; c < NC; c++) {
    const uint32_t ch = lane + 64u * c;
    if (ch < nch) {
      float w[16];
      chunk_f32<FP8>(q[c], w);
#pragma unroll
      for (uint32_t qd = 0; qd < EPC / 4; qd++) {
        const float4 x = v4[qd * nch + ch];
        acc += x.x * w[4 * qd] + x.y * w[4 * qd + 1] + x.z * w[4 * qd + 2] + x.w * w[4 * qd + 3];
      }
    }
  }
  return acc;
}

// one row's NC chunks per lane: unguarded buffer loads over the row (an
// empty range when !ok, chunks past nch out of range: zeros, no access), so
// the loads are never branched around and later waits count only what they
// need; the row address is wave-uniform
template <int NC>
__device__ __forceinline__ void load_row(uint4 (&q)[NC], const char *row, uint32_t lane,
                                         uint32_t nch, bool ok) {
  const buf_t r = buf_rsrc_u(row, ok ? nch * 16u : 0u);
#pragma unroll
  for (int c = 0; c < NC; c++) {
    const uint32_t ch = lane + 64u * c;
    q[c] = buf_ld_stream16(r, ch < nch ? ch * 16u : BUF_OOB);
  }
}

// LDS <- f32 vector of n elements (optionally rounded through bf16), laid
// out in chunk_swz order per segment: elements [0, nseg*seg) form nseg
// segments of seg elements (chunk count seg/EPC each), the rest one tail
// segment.  Four 16-byte loads are in flight per thread before any store.
template <bool RBF, int EPC>
__device__ __forceinline__ void stage_swz(float *dst, const float *src, uint32_t n, uint32_t nseg,
                                          uint32_t seg) {
  const uint32_t tid = threadIdx.x, nt = blockDim.x, n4 = n / 4, head = nseg * seg;
  const float4 *s4 = (const float4 *)src;
  float4 *d4 = (float4 *)dst;
  for (uint32_t i = tid; i < n4; i += 4 * nt) {
    float4 v[4];
#pragma unroll
    for (int u = 0; u < 4; u++) {
      const uint32_t j = i + u * nt;
      v[u] = j < n4 ? s4[j] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
#pragma unroll
    for (int u = 0; u < 4; u++) {
      const uint32_t j = i + u * nt;
      if (j >= n4) continue;
      float4 w = v[u];
      if (RBF) { w.x = rbf(w.x); w.y = rbf(w.y); w.z = rbf(w.z); w.w = rbf(w.w); }
      const uint32_t k = 4 * j;
      uint32_t base, kk, nch;
      if (k < head) { base = (k / seg) * seg; kk = k - base; nch = seg / EPC; }
      else { base = head; kk = k - head; nch = (n - head) / EPC; }
      d4[(base + chunk_swz<EPC>(kk, nch)) / 4] = w;
    }
  }
}

// stage_swz in two halves: the loads into NV float4 registers per thread
// (n/4 <= NV * blockDim.x), issued early, and the LDS stores, run later --
// the same elements to the same places
template <int NV>
__device__ __forceinline__ void stage_load(float4 (&v)[NV], const float *src, uint32_t n) {
  const uint32_t tid = threadIdx.x, nt = blockDim.x, n4 = n / 4;
  const buf_t r = buf_rsrc_u(src, n4 * 16u);      // unguarded: past n reads zero
#pragma unroll
  for (int u = 0; u < NV; u++) {
    const uint32_t j = tid + u * nt;
    const uint4 w = buf_ld16(r, j < n4 ? j * 16u : BUF_OOB);
    v[u] = make_float4(__uint_as_float(w.x), __uint_as_float(w.y), __uint_as_float(w.z), __uint_as_float(w.w));
  }
}
template <bool RBF, int EPC, int NV>
__device__ __forceinline__ void stage_store(float *dst, const float4 (&v)[NV], uint32_t n, uint32_t nseg,
                                            uint32_t seg) {
  const uint32_t tid = threadIdx.x, nt = blockDim.x, n4 = n / 4, head = nseg * seg;
  float4 *d4 = (float4 *)dst;
#pragma unroll
  for (int u = 0; u < NV; u++) {
    const uint32_t j = tid + u * nt;
    if (j >= n4) continue;
    float4 w = v[u];
    if (RBF) { w.x = rbf(w.x); w.y = rbf(w.y); w.z = rbf(w.z); w.w = rbf(w.w); }
    const uint32_t k = 4 * j;
    uint32_t base, kk, nch;
    if (k < head) { base = (k / seg) * seg; kk = k - base; nch = seg / EPC; }
    else { base = head; kk = k - head; nch = (n - head) / EPC; }
    d4[(base + chunk_swz<EPC>(kk, nch)) / 4] = w;
  }
}
#define MOE_XPRE 2      /* gate/up: x float4 per thread loaded early (D <= 4096) */

// ---- gate/up --------------------------------------------------------------
// grid (ceil(P / (8 * PPW)), B) with P = K*I + S row pairs per batch row;
// each wave owns PPW consecutive pairs, NC 16-byte chunks per lane per row,
// all its rows in flight before x is staged
template <bool FP8, int NC, int PPW>
__global__ __launch_bounds__(MOE_THREADS) void k_moe_gateup(ThvmMoeArgs a) {
  extern __shared__ float xs[];
  const uint32_t b = blockIdx.y, D = a.D, I = a.I, K = a.K;
  const uint32_t P = K * I + a.S;
  const uint32_t lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  // phase clock: 0 entry, 1 top-K picked, 2 rows and scales issued, 3 x
  // staged, 7 drained
  pclk(a.clk, a.clk_cap, 0);
  // the row's router logits first (the top-K waits for them only), then x
  // (staged into LDS while the rows are in flight)
  const buf_t lrs = buf_rsrc(a.logits ? a.logits + (uint64_t)b * a.E : nullptr, a.logits ? a.E * 4u : 0u);
  const uint32_t lgv = buf_ld4(lrs, lane < a.E ? lane * 4u : BUF_OOB);
  __builtin_amdgcn_sched_barrier(0);              // keep the logits ahead of x in issue order
  const bool xpre = D / 4 <= MOE_XPRE * blockDim.x;
  float4 xv[MOE_XPRE];
  stage_load(xv, a.x + (uint64_t)b * D, D);      // unconditional: no branch around the loads
  // the row's top-K, as the route kernel picks it, by wave 0 of a block
  // with a routed pair and handed to the others through LDS (every wave
  // routing for itself put four waves per SIMD on the same serial VALU
  // chain); block 0 publishes it for the down kernel
  __shared__ int32_t rsh[MOE_MAXK];
  int32_t rids[MOE_MAXK] = {};
  float rpr[MOE_MAXK] = {};
  pclk_after(a.clk, a.clk_cap, 4, lgv);
  if (a.logits && (blockIdx.x * MOE_WAVES * PPW < K * I || blockIdx.x == 0)) {   // block-uniform
    if (wv == 0) {
      route_wave(lane < a.E ? __uint_as_float(lgv) : -INFINITY, lane, a.E, K, rids, rpr);
      if (lane < MOE_MAXK) {
        int32_t v = 0;
#pragma unroll
        for (uint32_t kk = 0; kk < MOE_MAXK; kk++) v = kk == lane ? rids[kk] : v;
        rsh[lane] = v;
      }
      if (blockIdx.x == 0 && lane == 0)
#pragma unroll
        for (uint32_t kk = 0; kk < MOE_MAXK; kk++)
          if (kk < K) { a.sel_out[(uint64_t)b * K + kk] = rids[kk]; a.probs_out[(uint64_t)b * K + kk] = rpr[kk]; }
      pclk(a.clk, a.clk_cap, 6);
    }
    __syncthreads();
#pragma unroll
    for (uint32_t kk = 0; kk < MOE_MAXK; kk++) rids[kk] = rsh[kk];
  }
  pclk(a.clk, a.clk_cap, 1);
  const uint32_t p0 = (blockIdx.x * MOE_WAVES + wv) * PPW;
  const uint64_t rowb = (uint64_t)D * (FP8 ? 1 : 2);
  const uint32_t nch = (uint32_t)(rowb / 16);
  // every pair's expert first (routed slots from the route picked above, or
  // from sel in one round of unconditional loads), then all the pairs' row
  // loads: buffer loads through a resource over the pair's (gate, up) rows,
  // empty for a pair past P, so no load is branched around and each wait
  // counts only the loads it needs (a guarded load made every wait drain all
  // of them: the pairs' rows were requested one pair at a time)
  const buf_t srs = buf_rsrc(a.sel, a.logits ? 0u : a.B * K * 4u);
  uint32_t selv[PPW];
#pragma unroll
  for (int i = 0; i < PPW; i++) {
    const uint32_t p = p0 + i, e = p < K * I ? p / I : 0u;
    selv[i] = buf_ld4(srs, (b * K + e) * 4u);
  }
  uint4 gq[PPW][NC], uq[PPW][NC];
  uint64_t row0[PPW];
  const float *scp[PPW];
#pragma unroll
  for (int i = 0; i < PPW; i++) {
    const uint32_t p = p0 + i;
    const bool live = p < P;
    const char *base;
    if (live && p < K * I) {
      const uint32_t e = p / I, r = p % I;
      int32_t id = 0;
      if (a.logits) {
#pragma unroll
        for (uint32_t kk = 0; kk < MOE_MAXK; kk++) id = kk == e ? rids[kk] : id;
      } else {
        id = (int32_t)selv[i];
      }
      id = id < 0 ? 0 : id >= (int32_t)a.E ? (int32_t)a.E - 1 : id;   // a valid expert row
      row0[i] = (uint64_t)id * 2 * I + 2 * r;
      base = (const char *)a.wgu_e;
      scp[i] = a.sgu_e;
    } else {
      row0[i] = live ? 2ull * (p - K * I) : 0;
      base = (const char *)a.wgu_s;
      scp[i] = a.sgu_s;
    }
    const uint64_t rp = (uint64_t)(uintptr_t)base + row0[i] * rowb;
    const uint32_t plo = __builtin_amdgcn_readfirstlane((uint32_t)rp);
    const uint32_t phi = __builtin_amdgcn_readfirstlane((uint32_t)(rp >> 32));
    const buf_t rrs = buf_rsrc((const void *)(uintptr_t)(((uint64_t)phi << 32) | plo),
                              __builtin_amdgcn_readfirstlane(live ? 2u * (uint32_t)rowb : 0u));
#pragma unroll
    for (int c = 0; c < NC; c++) {
      const uint32_t ch = lane + 64u * c;
      gq[i][c] = buf_ld_stream16(rrs, ch < nch ? ch * 16u : BUF_OOB);
      uq[i][c] = buf_ld_stream16(rrs, ch < nch ? (uint32_t)rowb + ch * 16u : BUF_OOB);
    }
  }
  // the pairs' row scales with the rows (an empty range without scales)
  uint32_t scg[PPW], scu[PPW];
#pragma unroll
  for (int i = 0; i < PPW; i++) {
    const bool live = p0 + i < P;
    const uint64_t sp = (uint64_t)(uintptr_t)scp[i];
    const uint32_t slo = __builtin_amdgcn_readfirstlane((uint32_t)sp);
    const uint32_t shi = __builtin_amdgcn_readfirstlane((uint32_t)(sp >> 32));
    const buf_t crs = buf_rsrc((const void *)(uintptr_t)(((uint64_t)shi << 32) | slo),
                               __builtin_amdgcn_readfirstlane(live && scp[i] ? 0x7fffffffu : 0u));
    const uint64_t so = row0[i] * 4u;
    scg[i] = buf_ld4(crs, so < 0x7ffffff0ull ? (uint32_t)so : BUF_OOB);
    scu[i] = buf_ld4(crs, so < 0x7ffffff0ull ? (uint32_t)so + 4u : BUF_OOB);
  }
  pclk(a.clk, a.clk_cap, 2);
  if (xpre) stage_store<true, FP8 ? 16 : 8>(xs, xv, D, 0, 1);
  else stage_swz<true, FP8 ? 16 : 8>(xs, a.x + (uint64_t)b * D, D, 0, 1);
  __syncthreads();
  pclk(a.clk, a.clk_cap, 3);
  pclk_after(a.clk, a.clk_cap, 5, uq[PPW - 1][NC - 1].x);
#pragma unroll
  for (int i = 0; i < PPW; i++) {
    const uint32_t p = p0 + i;
    if (p >= P) break;                                   // wave-uniform
    float G = wave_sum(chunk_dot<FP8>(gq[i], xs, lane, nch));
    float U = wave_sum(chunk_dot<FP8>(uq[i], xs, lane, nch));
    if (lane == 0) {
      if (scp[i]) { G *= __uint_as_float(scg[i]); U *= __uint_as_float(scu[i]); }
      a.h[(uint64_t)b * P + p] = silu_f(G) * U;
    }
  }
  pclk_end(a.clk, a.clk_cap);
}

// ---- down + residual ------------------------------------------------------
// grid (ceil(D / (DW / 2)), B), DW waves: two waves per output row d.  (Every
// block stages the whole h row in LDS, 45 KiB at C5; 16 waves per block
// halved those reads but ended no sooner than 8: 8.23 against 8.08 us in the
// phase clock, the wider block waiting on its slowest wave's rows.)  The row's segments are
// split at routed slot c: wave half 0 takes slots [0, c), half 1 slots
// [c, K) and the shared segment (c balances their bytes, each half at most
// MOE_HALFK slots), so each wave holds half the rows in flight and a CU runs
// twice the waves.  Half 0 folds its slots in order from 0 and hands the
// partial sum to half 1 through LDS; half 1 continues the same sequence --
// routed slots ascending, then shared -- so every output has the one-wave
// fold's bits.
#define MOE_HALFK 4
__device__ __forceinline__ uint32_t moe_down_split(uint32_t K, uint32_t I, uint32_t S) {
  uint32_t c = (K * I + S) / (2 * I);
  if (c + MOE_HALFK < K) c = K - MOE_HALFK;
  if (c > MOE_HALFK) c = MOE_HALFK;
  if (c > K) c = K;
  return c;
}
template <bool FP8, int NC, int NCS, int DW>   /* 16-byte chunks per lane: routed rows, shared row; waves */
__global__ __launch_bounds__(64 * DW, 4) void k_moe_down(ThvmMoeArgs a) {
  extern __shared__ float hs[];
  __shared__ float part[DW / 2];
  const uint32_t b = blockIdx.y, D = a.D, I = a.I, K = a.K, S = a.S;
  const uint32_t P = K * I + S;
  const uint32_t lane = threadIdx.x & 63, wv = threadIdx.x >> 6, hf = wv & 1, rw = wv >> 1;
  const uint32_t d = blockIdx.x * (DW / 2) + rw;
  // phase clock: 0 entry, 1 rows issued, 2 h staged, 3 half sums done, 7
  // drained
  pclk(a.clk, a.clk_cap, 0);
  const bool live = d < D;
  const uint32_t c = moe_down_split(K, I, S);
  const uint32_t e0 = hf ? c : 0, e1 = hf ? K : c;          // this half's routed slots
  const uint64_t rI = (uint64_t)I * (FP8 ? 1 : 2), rS = (uint64_t)S * (FP8 ? 1 : 2);
  const uint32_t nI = (uint32_t)(rI / 16), nS = (uint32_t)(rS / 16);
  uint4 q[MOE_HALFK][NC], qs[NCS];
  int32_t ids[MOE_HALFK];
  // this half's routing ids requested at once (clamped, unconditional loads:
  // one round trip); the shared row, which needs no routing, goes out before
  // the routed rows, the rows' scales and the slots' probabilities after
  // them (unguarded buffer loads: no wait after the dot products), and h is
  // staged into LDS behind them (its registers would cost the second block
  // per CU)
#pragma unroll
  for (int j = 0; j < MOE_HALFK; j++) {
    const uint32_t e = e0 + j;
    ids[j] = a.sel[(uint64_t)b * K + (e < e1 ? e : 0u)];
  }
  load_row(qs, (const char *)a.wd_s + (uint64_t)(live ? d : 0) * rS, lane, nS, live && hf && S > 0);
  pclk_after(a.clk, a.clk_cap, 4, (uint32_t)ids[0]);
#pragma unroll
  for (int j = 0; j < MOE_HALFK; j++) {
    const bool ok = live && e0 + j < e1;
    int32_t id = ok ? ids[j] : 0;
    id = id < 0 ? 0 : id >= (int32_t)a.E ? (int32_t)a.E - 1 : id;
    ids[j] = id;
    const uint64_t row = (uint64_t)id * D + (live ? d : 0);
    load_row(q[j], (const char *)a.wd_e + row * rI, lane, nI, ok);
  }
  uint32_t scv[MOE_HALFK], pbv[MOE_HALFK], scs;
  {
    const buf_t srs = buf_rsrc_u(a.sd_e, a.sd_e ? 0x7fffffffu : 0u);
    const buf_t prs = buf_rsrc(a.probs, a.B * K * 4u);
#pragma unroll
    for (int j = 0; j < MOE_HALFK; j++) {
      const uint32_t e = e0 + j;
      const uint64_t so = ((uint64_t)ids[j] * D + (live ? d : 0)) * 4u;
      scv[j] = buf_ld4(srs, live && e < e1 && so < 0x7ffffff0ull ? (uint32_t)so : BUF_OOB);
      pbv[j] = buf_ld4(prs, e < e1 ? (b * K + e) * 4u : BUF_OOB);
    }
    const buf_t ssr = buf_rsrc(a.sd_s, a.sd_s ? D * 4u : 0u);
    scs = buf_ld4(ssr, live && hf ? d * 4u : BUF_OOB);
  }
  pclk(a.clk, a.clk_cap, 1);
  stage_swz<false, FP8 ? 16 : 8>(hs, a.h + (uint64_t)b * P, P, K, I);
  __syncthreads();
  pclk(a.clk, a.clk_cap, 2);
  pclk_after(a.clk, a.clk_cap, 5, q[MOE_HALFK - 1][NC - 1].x);
  // this half's segment values, in slot order
  float sv[MOE_HALFK];
#pragma unroll
  for (int j = 0; j < MOE_HALFK; j++) {
    const uint32_t e = e0 + j;
    sv[j] = 0.0f;
    if (e >= e1) continue;                               // wave-uniform
    float t = wave_sum(chunk_dot<FP8>(q[j], hs + e * I, lane, nI));
    if (a.sd_e) t *= __uint_as_float(scv[j]);
    sv[j] = t;
  }
  float acc = 0.0f;
  if (hf == 0) {
#pragma unroll
    for (int j = 0; j < MOE_HALFK; j++) {
      const uint32_t e = j;
      if (e >= e1) break;
      acc += __uint_as_float(pbv[j]) * sv[j];
    }
    if (lane == 0) part[rw] = acc;
  }
  float ssh = 0.0f;
  if (hf == 1 && S > 0) {
    ssh = wave_sum(chunk_dot<FP8>(qs, hs + K * I, lane, nS));
    if (a.sd_s) ssh *= __uint_as_float(scs);
  }
  __syncthreads();
  pclk(a.clk, a.clk_cap, 3);
  if (hf == 1 && live) {                               // wave-uniform
    acc = part[rw];
#pragma unroll
    for (int j = 0; j < MOE_HALFK; j++) {
      const uint32_t e = e0 + j;
      if (e >= e1) break;
      acc += __uint_as_float(pbv[j]) * sv[j];
    }
    if (S > 0) acc += ssh;
    if (lane == 0) {
      bf16_t *r = (bf16_t *)a.res + (uint64_t)b * D + d;
      r[0] = f2bf(bf2f(r[0]) + rbf(acc));
    }
  }
  pclk_end(a.clk, a.clk_cap);
}

// ---- expert-grouped form (batches above 4 rows) ---------------------------
// Rows routed to each expert, in ascending (b, slot) order.  One wave per
// expert (grid E): the wave reads the B*K routing entries 64 at a time (four
// chunks' loads in flight) and compacts its expert's entries with a ballot --
// position = that expert's entries in earlier chunks and lower lanes -- so
// every expert's list is built in parallel with no serial scan.
#define MOE_PLAN_MAX 4096   /* B*K routing entries */
__global__ __launch_bounds__(64) void k_moe_plan(ThvmMoeArgs a) {
  const uint32_t e = blockIdx.x, lane = threadIdx.x, n = a.B * a.K;
  int32_t *lst = a.plan + a.E + (uint64_t)e * n;
  const uint64_t below = (1ull << lane) - 1ull;
  uint32_t base = 0;
  for (uint32_t c0 = 0; c0 < n; c0 += 4 * 64) {
    int32_t v[4];
#pragma unroll
    for (int u = 0; u < 4; u++) {            // clamped indices: unconditional loads
      const uint32_t i = c0 + u * 64 + lane, ic = i < n ? i : 0;
      v[u] = a.sel[ic];
    }
#pragma unroll
    for (int u = 0; u < 4; u++) {
      const uint32_t i = c0 + u * 64 + lane;
      const bool hit = i < n && v[u] == (int32_t)e;
      const uint64_t m = __ballot(hit);
      if (hit) lst[base + __popcll(m & below)] = (int32_t)i;
      base += (uint32_t)__popcll(m);
    }
  }
  if (lane == 0) {
    a.plan[e] = (int32_t)base;
    if (a.live && base > 0) atomicAdd(a.live, 1);     // experts streamed (measurement)
  }
}

#define MOE_RG 4        /* x / h rows staged in LDS per pass */

// Stage ng <= MOE_RG rows of n f32 each (row j from src(j)) into dst + j*n,
// each row in stage_swz's single-segment layout (chunk_swz over n/EPC
// chunks); every row's 16-byte loads are in flight before the first store.
template <bool RBF, int EPC, class SrcF>
__device__ __forceinline__ void stage_rows(float *dst, uint32_t ng, uint32_t n, SrcF &&src) {
  const uint32_t tid = threadIdx.x, nt = blockDim.x, n4 = n / 4, nch = n / EPC;
  for (uint32_t i = tid; i < n4; i += nt) {
    float4 v[MOE_RG];
#pragma unroll
    for (int j = 0; j < MOE_RG; j++)
      v[j] = (uint32_t)j < ng ? ((const float4 *)src(j))[i] : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int j = 0; j < MOE_RG; j++) {
      if ((uint32_t)j >= ng) break;
      float4 w = v[j];
      if (RBF) { w.x = rbf(w.x); w.y = rbf(w.y); w.z = rbf(w.z); w.w = rbf(w.w); }
      ((float4 *)(dst + j * n))[chunk_swz<EPC>(4 * i, nch) / 4] = w;
    }
  }
}

// grid (ceil(max(I, S) / (8 * PPW)), E + 1): blockIdx.y < E is routed expert
// e over the rows the plan lists for it; blockIdx.y == E is the shared expert
// (S row pairs) over every batch row.  Each wave's PPW (gate, up) row pairs
// are loaded once; the rows' x are staged MOE_RG at a time.  Per (row,
// pair) the arithmetic is k_moe_gateup's.
template <bool FP8, int NC, int PPW>
__global__ __launch_bounds__(MOE_THREADS) void k_moe_gateup_g(ThvmMoeArgs a) {
  extern __shared__ float xs[];
  const uint32_t e = blockIdx.y, D = a.D, I = a.I, K = a.K;
  const bool shared = e == a.E;
  const uint32_t npair = shared ? a.S : I;
  const uint32_t nrows = shared ? a.B : (uint32_t)a.plan[e];
  const uint32_t pb = blockIdx.x * MOE_WAVES * PPW;
  if (nrows == 0 || pb >= npair) return;                   // block-uniform
  const int32_t *lst = a.plan + a.E + (uint64_t)e * a.B * K;
  const uint32_t P = K * I + a.S;
  const uint32_t lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const uint32_t p0 = pb + wv * PPW;
  const uint64_t rowb = (uint64_t)D * (FP8 ? 1 : 2);
  const uint32_t nch = (uint32_t)(rowb / 16);
  const char *base = shared ? (const char *)a.wgu_s : (const char *)a.wgu_e;
  const float *scp = shared ? a.sgu_s : a.sgu_e;
  uint4 gq[PPW][NC], uq[PPW][NC];
#pragma unroll
  for (int i = 0; i < PPW; i++) {
    const uint32_t p = p0 + i;
    const bool live = p < npair;
    const uint64_t r0 = shared ? 2ull * p : (uint64_t)e * 2 * I + 2 * p;
    load_row(gq[i], base + (live ? r0 : 0) * rowb, lane, nch, live);
    load_row(uq[i], base + (live ? r0 + 1 : 0) * rowb, lane, nch, live);
  }
  for (uint32_t g0 = 0; g0 < nrows; g0 += MOE_RG) {
    const uint32_t ng = min((uint32_t)MOE_RG, nrows - g0);
    __syncthreads();                                       // the previous pass's reads
    stage_rows<true, FP8 ? 16 : 8>(xs, ng, D, [&](uint32_t j) {
      const uint32_t b = shared ? g0 + j : (uint32_t)lst[g0 + j] / K;
      return a.x + (uint64_t)b * D;
    });
    __syncthreads();
    for (uint32_t j = 0; j < ng; j++) {
      const uint32_t ent = shared ? 0u : (uint32_t)lst[g0 + j];
      const uint32_t b = shared ? g0 + j : ent / K, slot = ent % K;
#pragma unroll
      for (int i = 0; i < PPW; i++) {
        const uint32_t p = p0 + i;
        if (p >= npair) break;                             // wave-uniform
        float G = wave_sum(chunk_dot<FP8>(gq[i], xs + j * D, lane, nch));
        float U = wave_sum(chunk_dot<FP8>(uq[i], xs + j * D, lane, nch));
        if (lane == 0) {
          const uint64_t r0 = shared ? 2ull * p : (uint64_t)e * 2 * I + 2 * p;
          if (scp) { G *= scp[r0]; U *= scp[r0 + 1]; }
          a.h[(uint64_t)b * P + (shared ? K * I : slot * I) + p] = silu_f(G) * U;
        }
      }
    }
  }
}

// grid (ceil(D / (8 * RPW)), E + 1): routed expert e (rows d of its down
// matrix, over the plan's rows) or the shared expert (every batch row); the
// weights are loaded once, the rows' h staged MOE_RG at a time, and each
// (row, d) down value -- k_moe_down's per-segment value, scale included -- is
// written to part[b][slot][d] (shared: part[B*K*D + b*D + d]).
template <bool FP8, int NC, int RPW>
__global__ __launch_bounds__(MOE_THREADS) void k_moe_down_g(ThvmMoeArgs a) {
  extern __shared__ float hs[];
  const uint32_t e = blockIdx.y, D = a.D, I = a.I, K = a.K, S = a.S;
  const bool shared = e == a.E;
  const uint32_t nrows = shared ? a.B : (uint32_t)a.plan[e];
  const uint32_t db = blockIdx.x * MOE_WAVES * RPW;
  if (nrows == 0 || db >= D) return;                       // block-uniform
  const int32_t *lst = a.plan + a.E + (uint64_t)e * a.B * K;
  const uint32_t P = K * I + S, W = shared ? S : I;
  const uint32_t lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const uint32_t d0 = db + wv * RPW;
  const uint64_t rowb = (uint64_t)W * (FP8 ? 1 : 2);
  const uint32_t nch = (uint32_t)(rowb / 16);
  uint4 q[RPW][NC];
#pragma unroll
  for (int r = 0; r < RPW; r++) {
    const uint32_t d = d0 + r;
    const bool live = d < D;
    const uint64_t row = shared ? (uint64_t)(live ? d : 0) : (uint64_t)e * D + (live ? d : 0);
    load_row(q[r], (shared ? (const char *)a.wd_s : (const char *)a.wd_e) + row * rowb, lane, nch, live);
  }
  const float *scl = shared ? a.sd_s : a.sd_e;
  for (uint32_t g0 = 0; g0 < nrows; g0 += MOE_RG) {
    const uint32_t ng = min((uint32_t)MOE_RG, nrows - g0);
    __syncthreads();
    stage_rows<false, FP8 ? 16 : 8>(hs, ng, W, [&](uint32_t j) {
      const uint32_t ent = shared ? 0u : (uint32_t)lst[g0 + j];
      const uint32_t b = shared ? g0 + j : ent / K, slot = ent % K;
      return a.h + (uint64_t)b * P + (shared ? K * I : slot * I);
    });
    __syncthreads();
    for (uint32_t j = 0; j < ng; j++) {
      const uint32_t ent = shared ? 0u : (uint32_t)lst[g0 + j];
      const uint32_t b = shared ? g0 + j : ent / K, slot = ent % K;
#pragma unroll
      for (int r = 0; r < RPW; r++) {
        const uint32_t d = d0 + r;
        if (d >= D) break;                                 // wave-uniform
        float sv = wave_sum(chunk_dot<FP8>(q[r], hs + j * W, lane, nch));
        if (scl) sv *= shared ? scl[d] : scl[(uint64_t)e * D + d];
        if (lane == 0) {
          const uint64_t o = shared ? (uint64_t)a.B * K * D + (uint64_t)b * D + d
                                    : ((uint64_t)b * K + slot) * D + d;
          a.part[o] = sv;
        }
      }
    }
  }
}

// ---- expert-grouped form on MFMA (grouped = 2) ----------------------------
// The same plan / part contract as the VALU grouped kernels, with each
// expert's rows as a small GEMM on v_mfma_f32_16x16x32_bf16: the weights are
// the A operand (NT 16-row tiles per block, fp8 decoded exactly into bf16),
// 16 of the expert's routed batch rows the B operand (blockIdx.z picks which
// 16: column j is the plan's (16 z + j)-th row; columns past the row count
// read zero through an out-of-range buffer offset and are never stored).
// Gate/up (KIND 0): B = x rounded to bf16, the experts' input dtype, one MFMA
// per 32 k.  Down (KIND 1): B = the f32 h split into bf16 hi + lo, two MFMAs
// per 32 k, so h keeps about 16 significant bits.  The MM_WAVES waves split K
// into contiguous slices and keep NU steps of loads in flight (a step
// is consumed, then the slot refilled); steps past a wave's slice read zero,
// so the loop is straight-line code.  Partial tiles are summed in wave order
// through LDS; the epilogue is the VALU kernels' (scale, silu(g)*u into h /
// the scaled down value into part).
// A lane (li = lane & 15, lg = lane >> 4) supplies row li, k in
// [KL lg, KL lg + KL) of each step to both operands (KL = LB weight bytes
// per lane as elements), 8 k per MFMA; a result tile's entry (weight row ii,
// column m) is lane (ii / 4) * 16 + m, element ii % 4.  Measured at the C5
// batch-32 shape: gate/up fastest with 32-byte lanes and one step in flight
// (whole 128-byte lines per row), down with 16-byte lanes and two steps.
#ifndef MM_WAVES
#define MM_WAVES 4
#endif
#ifndef MM_NT
#define MM_NT 4         /* 16-row weight tiles per block */
#endif
template <int KIND, bool FP8, int LB, int NU>
__global__ __launch_bounds__(64 * MM_WAVES) void k_moe_mm(ThvmMoeArgs a) {
  constexpr int NT = MM_NT;
  __shared__ float4 red[MM_WAVES * NT * 64];
  const uint32_t e = blockIdx.y, D = a.D, I = a.I, K = a.K, S = a.S;
  const bool shared = e == a.E;
  const uint32_t nrows = shared ? a.B : (uint32_t)a.plan[e];
  const uint32_t NR = KIND == 0 ? (shared ? 2 * S : 2 * I) : D;      // weight rows
  const uint32_t KK = KIND == 0 ? D : (shared ? S : I);              // reduction length
  const uint32_t n0 = blockIdx.x * 16u * NT, c0 = blockIdx.z * 16u;
  if (c0 >= nrows || n0 >= NR) return;                                // block-uniform
  const int32_t *lst = a.plan + a.E + (uint64_t)e * a.B * K;
  const uint32_t P = K * I + S;
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6, li = lane & 15, lg = lane >> 4;
  // per step a lane reads LB contiguous weight bytes of its row (k = KL lg ..
  // KL lg + KL - 1), the 4 lanes of a row 4 LB bytes; KL / 8 MFMAs per tile
  constexpr uint32_t KL = FP8 ? LB : LB / 2, KS = 4 * KL, NMF = KL / 8, NC = LB / 16;
  const uint64_t rowb = (uint64_t)KK * (FP8 ? 1 : 2);
  // this block's weight rows (rows past NR read zero)
  const char *wbase = KIND == 0 ? (shared ? (const char *)a.wgu_s : (const char *)a.wgu_e + (uint64_t)e * 2 * I * rowb)
                                : (shared ? (const char *)a.wd_s : (const char *)a.wd_e + (uint64_t)e * D * rowb);
  const buf_t wrs = buf_rsrc(wbase + n0 * rowb, (uint32_t)(min(NR - n0, 16u * NT) * rowb));
  // row-major: lane l reads LB bytes of row li at quarter lg per step; tiled
  // (a.wtiled), the same bytes are the lane's 16-byte slots of the step's
  // 64 LB-byte block, so every load instruction reads 1 KB contiguous
  const bool tl = a.wtiled != 0;
  const uint32_t sstep = tl ? 64u * LB : 4u * LB, jstep = tl ? 1024u : 16u;
  uint32_t wo[NT];
#pragma unroll
  for (int t = 0; t < NT; t++)
    wo[t] = tl ? (uint32_t)(16u * t * rowb) + lane * 16u : (uint32_t)((16u * t + li) * rowb) + lg * LB;
  // this lane's x / h row (byte offset; out of range for columns past nrows)
  const buf_t xrs = KIND == 0 ? buf_rsrc(a.x, a.B * D * 4) : buf_rsrc(a.h, a.B * P * 4);
  uint32_t xo = BUF_OOB;
  if (c0 + li < nrows) {
    const uint32_t ent = shared ? c0 + li : (uint32_t)lst[c0 + li];
    const uint32_t b = shared ? ent : ent / K, slot = shared ? 0 : ent % K;
    xo = (KIND == 0 ? b * D : b * P + (shared ? K * I : slot * I)) * 4 + lg * KL * 4;
  }
  const uint32_t NS = KK / KS;
  const uint32_t s0 = (uint32_t)(((uint64_t)NS * wv) / MM_WAVES), s1 = (uint32_t)(((uint64_t)NS * (wv + 1)) / MM_WAVES);
  f32x4_t acc[NT];
#pragma unroll
  for (int t = 0; t < NT; t++) acc[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  uint4 wq[NU][NT][NC], xq[NU][KL / 4];
  auto load = [&](int u, uint32_t st) {
    const bool in = st < s1;
    const uint32_t so = in ? st * sstep : BUF_OOB;                    // 4 LB weight bytes per row per step
#pragma unroll
    for (int t = 0; t < NT; t++)
#pragma unroll
      for (int jj = 0; jj < (int)NC; jj++) wq[u][t][jj] = buf_ld_stream16(wrs, wo[t] + so + jj * jstep);
    const uint32_t xs = in && xo != BUF_OOB ? xo + st * KS * 4 : BUF_OOB;
#pragma unroll
    for (int q = 0; q < (int)KL / 4; q++) xq[u][q] = buf_ld16(xrs, xs + 16 * q);
  };
  // the epilogue's operands, staged while the first loads are in flight:
  // each column's (row, slot) and the block's row scales
  __shared__ uint32_t col_b[16], col_slot[16];
  __shared__ float rsc[16 * NT];
  // consume step u: x converted once, then tile by tile -- each tile's
  // weight registers are refilled with step `nxt` right after their last
  // MFMA, so the next step's loads are in flight during the rest of this
  // step's arithmetic (x is refilled after the last tile)
  auto compute_refill = [&](int u, uint32_t nxt) {
    uint4 H[NMF], L[NMF];
#pragma unroll
    for (int j = 0; j < (int)NMF; j++) {
      const float *xf = (const float *)&xq[u][2 * j];
      uint32_t hb[4], lb[4];
#pragma unroll
      for (int i = 0; i < 4; i++) {
        // bf16 hi (and for down lo = v - hi, exact in f32), round to nearest
        // even.  Down rounds in hardware (76.0 -> 70.4 us per layer at C5
        // batch 32); gate/up keeps the software form, with which its
        // instance holds 148 VGPRs (3 waves per SIMD) instead of 222
        if (KIND == 1) {
          hb[i] = pk_bf16(xf[2 * i], xf[2 * i + 1]);
          lb[i] = pk_bf16(xf[2 * i] - __uint_as_float(hb[i] << 16), xf[2 * i + 1] - __uint_as_float(hb[i] & 0xffff0000u));
        } else {
          const bf16_t h0 = f2bf(xf[2 * i]), h1 = f2bf(xf[2 * i + 1]);
          hb[i] = (uint32_t)h0 | ((uint32_t)h1 << 16);
          lb[i] = 0;
        }
      }
      H[j] = make_uint4(hb[0], hb[1], hb[2], hb[3]);
      L[j] = make_uint4(lb[0], lb[1], lb[2], lb[3]);
    }
    const bool in = nxt < s1;
    const uint32_t so = in ? nxt * sstep : BUF_OOB;
#pragma unroll
    for (int t = 0; t < NT; t++) {
#pragma unroll
      for (int j = 0; j < (int)NMF; j++) {
        uint4 A;
        if (FP8) {
          const uint4 q = wq[u][t][j / 2];
          fp8x4_op<GX_BF16>(j % 2 ? q.z : q.x, A.x, A.y);
          fp8x4_op<GX_BF16>(j % 2 ? q.w : q.y, A.z, A.w);
        } else {
          A = wq[u][t][j];
        }
        acc[t] = mfma16<GX_BF16>(A, H[j], acc[t]);
        if (KIND == 1) acc[t] = mfma16<GX_BF16>(A, L[j], acc[t]);
      }
#pragma unroll
      for (int jj = 0; jj < (int)NC; jj++) wq[u][t][jj] = buf_ld_stream16(wrs, wo[t] + so + jj * jstep);
    }
    const uint32_t xs = in && xo != BUF_OOB ? xo + nxt * KS * 4 : BUF_OOB;
#pragma unroll
    for (int q = 0; q < (int)KL / 4; q++) xq[u][q] = buf_ld16(xrs, xs + 16 * q);
  };
#pragma unroll
  for (int u = 0; u < NU; u++) load(u, s0 + u);
  if (threadIdx.x < 16) {
    const uint32_t m = threadIdx.x;
    const uint32_t ent = c0 + m < nrows ? (shared ? c0 + m : (uint32_t)lst[c0 + m]) : 0u;
    col_b[m] = shared ? ent : ent / K;
    col_slot[m] = shared ? 0u : ent % K;
  } else if (threadIdx.x < 16 + 16 * NT) {
    const uint32_t i = threadIdx.x - 16, n = n0 + i;
    const float *scp = KIND == 0 ? (shared ? a.sgu_s : a.sgu_e) : (shared ? a.sd_s : a.sd_e);
    const uint64_t r = KIND == 0 ? (shared ? (uint64_t)n : (uint64_t)e * 2 * I + n)
                                 : (shared ? (uint64_t)n : (uint64_t)e * D + n);
    rsc[i] = (scp && n < NR) ? scp[r] : 1.0f;
  }
  for (uint32_t sb = s0; sb < s1; sb += NU) {
#pragma unroll
    for (int u = 0; u < NU; u++) compute_refill(u, sb + u + NU);
  }
#pragma unroll
  for (int t = 0; t < NT; t++) {
    const f32x4_t v = acc[t];
    red[((uint32_t)wv * NT + t) * 64 + lane] = make_float4(v[0], v[1], v[2], v[3]);
  }
  __syncthreads();
  const uint32_t ncols = min(nrows - c0, 16u);
  const uint32_t per = KIND == 0 ? 8 * NT : 16 * NT;                  // row pairs / rows per column
  for (uint32_t task = threadIdx.x; task < per * ncols; task += 64 * MM_WAVES) {
    const uint32_t p = task % per, m = task / per;
    const uint32_t b = col_b[m], slot = col_slot[m];
    auto tile_val = [&](uint32_t ii_all) {                            // sum over waves, in order
      const uint32_t t = ii_all / 16, ii = ii_all % 16, ln = (ii / 4) * 16 + m, r = ii % 4;
      float sum = 0.0f;
#pragma unroll
      for (int w = 0; w < MM_WAVES; w++) {
        const float4 q = red[((uint32_t)w * NT + t) * 64 + ln];
        sum += r == 0 ? q.x : r == 1 ? q.y : r == 2 ? q.z : q.w;
      }
      return sum;
    };
    if (KIND == 0) {
      const uint32_t i0 = 2 * p, n = n0 + i0;
      if (n >= NR) continue;                                          // NR is even
      float G = tile_val(i0), U = tile_val(i0 + 1);
      if (shared ? a.sgu_s : a.sgu_e) {
        G *= rsc[i0];
        U *= rsc[i0 + 1];
      }
      a.h[(uint64_t)b * P + (shared ? K * I : slot * I) + n / 2] = silu_f(G) * U;
    } else {
      const uint32_t n = n0 + p;
      if (n >= NR) continue;
      float sv = tile_val(p);
      if (shared ? a.sd_s : a.sd_e) sv *= rsc[p];
      const uint64_t o = shared ? (uint64_t)a.B * K * D + (uint64_t)b * D + n : ((uint64_t)b * K + slot) * D + n;
      a.part[o] = sv;
    }
  }
}

// res[b][d] = bf16(res + bf16(sum_slot probs * part + shared)), k_moe_down's
// sum order; grid (ceil(D / 256), B)
__global__ __launch_bounds__(256) void k_moe_combine(ThvmMoeArgs a) {
  const uint32_t b = blockIdx.y, d = blockIdx.x * 256 + threadIdx.x, D = a.D, K = a.K;
  if (d >= D) return;
  float acc = 0.0f;
  for (uint32_t e = 0; e < K; e++) acc += a.probs[(uint64_t)b * K + e] * a.part[((uint64_t)b * K + e) * D + d];
  if (a.S > 0) acc += a.part[(uint64_t)a.B * K * D + (uint64_t)b * D + d];
  bf16_t *r = (bf16_t *)a.res + (uint64_t)b * D + d;
  r[0] = f2bf(bf2f(r[0]) + rbf(acc));
}

extern "C" uint64_t thvm_k_moe_plan_bytes(uint32_t B, uint32_t E, uint32_t K) {
  return ((uint64_t)E + (uint64_t)E * B * K) * 4;
}
extern "C" uint64_t thvm_k_moe_part_bytes(uint32_t B, uint32_t K, uint32_t D) {
  return ((uint64_t)B * K * D + (uint64_t)B * D) * 4;
}

// -------------------------------------------------------------------------
extern "C" int thvm_k_route(const ThvmRouteArgs *a, hipStream_t s, char *err, int errlen) {
  if (a->B == 0 || a->E == 0 || a->E > 64 || a->K == 0 || a->K > a->E) {
    snprintf(err, errlen, "route: need 1 <= K <= E <= 64 (E=%u K=%u)", a->E, a->K);
    return -1;
  }
  thvm_launch(true, true, k_route, dim3(a->B), dim3(64), 0, s, *a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) { snprintf(err, errlen, "route launch: %s", hipGetErrorString(e)); return -1; }
  return 0;
}

extern "C" int thvm_k_moe_gate(const ThvmGateArgs *a, hipStream_t s, char *err, int errlen) {
  if (a->B == 0 || a->E == 0 || a->E > 64 || a->D == 0 || a->D % 4 || a->D > RT_NREG * RT_NORM_THREADS) {
    snprintf(err, errlen, "moe_gate: need 1 <= E <= 64, D a multiple of 4 up to %d (E=%u D=%u)",
             RT_NREG * RT_NORM_THREADS, a->E, a->D);
    return -1;
  }
  if (((uintptr_t)a->gate & 15) || !a->x || !a->xn || !a->logits) {
    snprintf(err, errlen, "moe_gate: null buffers or a router matrix not 16-byte aligned");
    return -1;
  }
  const uint32_t nch = (a->D / 4 + 63) / 64;
  const bool one = a->B <= 4;                     // one expert per block for a few rows
  void (*f)(ThvmGateArgs) = nch <= 4 ? (one ? k_moe_gate<4, 1> : k_moe_gate<4, RT_WAVES>)
                          : nch <= 8 ? (one ? k_moe_gate<8, 1> : k_moe_gate<8, RT_WAVES>)
                                     : (one ? k_moe_gate<16, 1> : k_moe_gate<16, RT_WAVES>);
  const uint32_t epb = one ? 1 : RT_WAVES;
  // (one expert per block: the norm's 256 threads only -- the other four
  // waves had nothing to do but issue their share of the no-access loads)
  thvm_launch(true, true, f, dim3((a->E + epb - 1) / epb, a->B), dim3(one ? RT_NORM_THREADS : RT_THREADS), 0, s, *a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) { snprintf(err, errlen, "moe_gate launch: %s", hipGetErrorString(e)); return -1; }
  return 0;
}

static int moe_check(const ThvmMoeArgs *a, int gateup, char *err, int errlen) {
  const uint32_t wsz = a->wdt == THVM_DT_FP8E4M3 ? 1 : a->wdt == THVM_DT_BF16 ? 2 : 0;
  if (!wsz) { snprintf(err, errlen, "moe: weights must be fp8 e4m3 or bf16"); return -1; }
  if (a->wtiled && a->grouped != 2) {
    snprintf(err, errlen, "moe: tiled expert weights are read by the MFMA grouped form (grouped=2) only");
    return -1;
  }
  if (a->B == 0 || a->D == 0 || a->E == 0 || a->K == 0 || a->K > MOE_MAXK || a->K > a->E ||
      a->I == 0) {
    snprintf(err, errlen, "moe: bad geometry (K <= %u)", MOE_MAXK);
    return -1;
  }
  const uint64_t rd = (uint64_t)a->D * wsz, ri = (uint64_t)a->I * wsz, rs = (uint64_t)a->S * wsz;
  const bool rows_ok = gateup ? (rd % 16 == 0 && rd <= 64 * 16 * MOE_MAXC)
                               : (ri % 16 == 0 && rs % 16 == 0 && ri <= 64 * 16 * MOE_MAXC &&
                                  rs <= 64 * 16 * MOE_MAXCS);
  if (!rows_ok) {
    snprintf(err, errlen, "moe: weight rows must be 16-byte multiples up to %u bytes (%u for the "
             "shared down row)", 64 * 16 * MOE_MAXC, 64 * 16 * MOE_MAXCS);
    return -1;
  }
  const void *we = gateup ? a->wgu_e : a->wd_e, *ws = gateup ? a->wgu_s : a->wd_s;
  const float *se = gateup ? a->sgu_e : a->sd_e, *ss = gateup ? a->sgu_s : a->sd_s;
  if (!we || (a->S && !ws) || (((uintptr_t)we | (uintptr_t)ws) & 15)) {
    snprintf(err, errlen, "moe: weights missing or not 16-byte aligned");
    return -1;
  }
  if (a->wdt == THVM_DT_FP8E4M3 && (!se || (a->S && !ss))) {
    snprintf(err, errlen, "moe: fp8 weights need their row scales");
    return -1;
  }
  if (a->D % 16 || a->I % 16 || a->S % 16) {
    snprintf(err, errlen, "moe: D, I and S must be multiples of 16");
    return -1;
  }
  if (((uintptr_t)a->x | (uintptr_t)a->h) & 15) {
    snprintf(err, errlen, "moe: x and h must be 16-byte aligned");
    return -1;
  }
  if (gateup ? (!a->h || !a->x || (!a->sel && !a->logits)) : (!a->h || !a->res || !a->sel || !a->probs)) {
    snprintf(err, errlen, "moe: missing operand");
    return -1;
  }
  if (a->logits && (!gateup || a->grouped || a->E > 64 || !a->sel_out || !a->probs_out)) {
    snprintf(err, errlen, "moe: routing inside the gate/up is for the per-row form, E <= 64, "
             "with sel_out and probs_out");
    return -1;
  }
  return 0;
}

typedef void (*moe_fn)(ThvmMoeArgs);
template <bool FP8>
static moe_fn pick_gateup(uint32_t nch, uint32_t *ppw) {
  if (nch <= 64) { *ppw = 8; return k_moe_gateup<FP8, 1, 8>; }
  // (3 pairs per wave at 128-chunk rows: the C5 batch-1 grid is 470 blocks,
  // one round of two per CU, against 352 with 4 -- 96 CUs with two blocks,
  // 160 with one; measured 15.0 -> 12.8 us per launch)
  if (nch <= 128) { *ppw = 3; return k_moe_gateup<FP8, 2, 3>; }
  *ppw = 2;
  return k_moe_gateup<FP8, 4, 2>;
}

template <bool FP8>
static moe_fn pick_gateup_g(uint32_t nch, uint32_t *ppw) {
  if (nch <= 64) { *ppw = 4; return k_moe_gateup_g<FP8, 1, 4>; }
  if (nch <= 128) { *ppw = 2; return k_moe_gateup_g<FP8, 2, 2>; }
  *ppw = 1;
  return k_moe_gateup_g<FP8, 4, 1>;
}

static int moe_grouped_check(const ThvmMoeArgs *a, int gateup, char *err, int errlen) {
  if (a->grouped > 2) { snprintf(err, errlen, "moe: grouped is 0, 1 (VALU) or 2 (MFMA)"); return -1; }
  if ((uint64_t)a->B * a->K > MOE_PLAN_MAX) {
    snprintf(err, errlen, "moe: grouped form takes B*K <= %d routing entries", MOE_PLAN_MAX);
    return -1;
  }
  if (!a->plan || (!gateup && !a->part)) {
    snprintf(err, errlen, "moe: the grouped form needs the plan (and, for down, the part) scratch");
    return -1;
  }
  if (a->E > 64) { snprintf(err, errlen, "moe: grouped form takes E <= 64"); return -1; }
  if (a->wtiled) {
    const uint32_t es = a->wdt == THVM_DT_FP8E4M3 ? 1 : 2;
    // whole 16-row groups per expert; a row a whole number of steps (gate/up
    // 128-byte steps over D, down 64-byte steps over I and S)
    const bool ok = a->grouped == 2 && (2 * a->I) % 16 == 0 && a->D % 16 == 0 && (2 * a->S) % 16 == 0 &&
                    (gateup ? ((uint64_t)a->D * es) % 128 == 0
                            : ((uint64_t)a->I * es) % 64 == 0 && ((uint64_t)a->S * es) % 64 == 0);
    if (!ok) {
      snprintf(err, errlen, "moe: tiled expert weights need the MFMA grouped form and 16-row-group experts");
      return -1;
    }
  }
  return 0;
}

static int moe_mm_launch(const ThvmMoeArgs *a, int gateup, hipStream_t s, char *err, int errlen) {
  const bool f8 = a->wdt == THVM_DT_FP8E4M3;
  // k per step: gate/up 32-byte lanes (128 k fp8, 64 k bf16), down 16-byte
  const uint32_t ks = gateup ? (f8 ? 128 : 64) : (f8 ? 64 : 32);
  if (gateup ? a->D % ks : (a->I % ks || a->S % ks)) {
    snprintf(err, errlen, "moe: the MFMA grouped form needs %s multiples of %u", gateup ? "D" : "I and S", ks);
    return -1;
  }
  const moe_fn f = gateup ? (f8 ? k_moe_mm<0, true, 32, 1> : k_moe_mm<0, false, 32, 1>)
                          : (f8 ? k_moe_mm<1, true, 16, 2> : k_moe_mm<1, false, 16, 2>);
  // 16 routed rows per column group (blockIdx.z): a group past an expert's
  // row count exits at once; groups beyond the first re-read that expert's
  // weights, which only experts with more than 16 rows need
  const uint32_t nr = gateup ? 2 * (a->I > a->S ? a->I : a->S) : a->D;
  const dim3 grid((nr + 16 * MM_NT - 1) / (16 * MM_NT), a->E + (a->S ? 1 : 0), (a->B + 15) / 16);
  const uint32_t lds = 0;
  if ((uint64_t)a->B * (a->K * a->I + a->S) * 4 >= BUF_OOB || (uint64_t)a->B * a->D * 4 >= BUF_OOB) {
    snprintf(err, errlen, "moe: x / h above 2 GiB");
    return -1;
  }
  if (gateup) thvm_launch(true, false, k_moe_plan, dim3(a->E), dim3(64), 0, s, *a);
  thvm_launch(!gateup, gateup, f, grid, dim3(64 * MM_WAVES), lds, s, *a);
  if (!gateup) thvm_launch(false, true, k_moe_combine, dim3((a->D + 255) / 256, a->B), dim3(256), 0, s, *a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) { snprintf(err, errlen, "moe mm launch: %s", hipGetErrorString(e)); return -1; }
  return 0;
}

extern "C" int thvm_k_moe_gateup(const ThvmMoeArgs *a, hipStream_t s, char *err, int errlen) {
  if (moe_check(a, 1, err, errlen)) return -1;
  if (a->grouped == 2) {
    if (moe_grouped_check(a, 1, err, errlen)) return -1;
    return moe_mm_launch(a, 1, s, err, errlen);
  }
  if (a->grouped) {
    if (moe_grouped_check(a, 1, err, errlen)) return -1;
    const uint32_t nch = a->D * (a->wdt == THVM_DT_FP8E4M3 ? 1 : 2) / 16;
    uint32_t ppw = 1;
    const moe_fn f = a->wdt == THVM_DT_FP8E4M3 ? pick_gateup_g<true>(nch, &ppw) : pick_gateup_g<false>(nch, &ppw);
    const uint32_t np = a->I > a->S ? a->I : a->S;
    const dim3 grid((np + MOE_WAVES * ppw - 1) / (MOE_WAVES * ppw), a->E + (a->S ? 1 : 0));
    const uint32_t lds = MOE_RG * a->D * 4;
    if (lds > 160 * 1024) { snprintf(err, errlen, "moe: D too large for the grouped form"); return -1; }
    if (lds > 64 * 1024) {
      hipError_t e = hipFuncSetAttribute((const void *)f, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
      if (e != hipSuccess) { snprintf(err, errlen, "moe_gateup: hipFuncSetAttribute: %s", hipGetErrorString(e)); return -1; }
    }
    thvm_launch(true, false, k_moe_plan, dim3(a->E), dim3(64), 0, s, *a);
    thvm_launch(false, true, f, grid, dim3(MOE_THREADS), lds, s, *a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) { snprintf(err, errlen, "moe_gateup launch: %s", hipGetErrorString(e)); return -1; }
    return 0;
  }
  const uint32_t P = a->K * a->I + a->S;
  const uint32_t nch = a->D * (a->wdt == THVM_DT_FP8E4M3 ? 1 : 2) / 16;
  uint32_t ppw = 1;
  const moe_fn f = a->wdt == THVM_DT_FP8E4M3 ? pick_gateup<true>(nch, &ppw) : pick_gateup<false>(nch, &ppw);
  const dim3 grid((P + MOE_WAVES * ppw - 1) / (MOE_WAVES * ppw), a->B);
  const uint32_t lds = a->D * 4;
  if (lds > 64 * 1024) { snprintf(err, errlen, "moe: D too large"); return -1; }
  thvm_launch(true, true, f, grid, dim3(MOE_THREADS), lds, s, *a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) { snprintf(err, errlen, "moe_gateup launch: %s", hipGetErrorString(e)); return -1; }
  return 0;
}

extern "C" int thvm_k_moe_down(const ThvmMoeArgs *a, hipStream_t s, char *err, int errlen) {
  if (moe_check(a, 0, err, errlen)) return -1;
  if (a->grouped == 2) {
    if (moe_grouped_check(a, 0, err, errlen)) return -1;
    return moe_mm_launch(a, 0, s, err, errlen);
  }
  if (a->grouped) {
    if (moe_grouped_check(a, 0, err, errlen)) return -1;
    const uint32_t wsz = a->wdt == THVM_DT_FP8E4M3 ? 1 : 2;
    const uint32_t W = a->I > a->S ? a->I : a->S, nch = W * wsz / 16;
    if (nch > 64 * 6) { snprintf(err, errlen, "moe: down rows above 6 KiB"); return -1; }
    const bool f8 = a->wdt == THVM_DT_FP8E4M3;
    // rows per wave 4 up to 4 KiB rows, 2 beyond (register budget)
    const int RPW = nch <= 256 ? 4 : 2;
    moe_fn f = nch <= 64 ? (f8 ? k_moe_down_g<true, 1, 4> : k_moe_down_g<false, 1, 4>)
             : nch <= 128 ? (f8 ? k_moe_down_g<true, 2, 4> : k_moe_down_g<false, 2, 4>)
             : nch <= 192 ? (f8 ? k_moe_down_g<true, 3, 4> : k_moe_down_g<false, 3, 4>)
             : nch <= 256 ? (f8 ? k_moe_down_g<true, 4, 4> : k_moe_down_g<false, 4, 4>)
                          : (f8 ? k_moe_down_g<true, 6, 2> : k_moe_down_g<false, 6, 2>);
    const dim3 grid((a->D + MOE_WAVES * RPW - 1) / (MOE_WAVES * RPW), a->E + (a->S ? 1 : 0));
    const uint32_t lds = MOE_RG * W * 4;
    if (lds > 160 * 1024) { snprintf(err, errlen, "moe: I / S too large for the grouped form"); return -1; }
    if (lds > 64 * 1024) {
      hipError_t e = hipFuncSetAttribute((const void *)f, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
      if (e != hipSuccess) { snprintf(err, errlen, "moe_down: hipFuncSetAttribute: %s", hipGetErrorString(e)); return -1; }
    }
    thvm_launch(true, false, f, grid, dim3(MOE_THREADS), lds, s, *a);
    thvm_launch(false, true, k_moe_combine, dim3((a->D + 255) / 256, a->B), dim3(256), 0, s, *a);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) { snprintf(err, errlen, "moe_down launch: %s", hipGetErrorString(e)); return -1; }
    return 0;
  }
  const uint32_t P = a->K * a->I + a->S;
  const uint32_t lds = P * 4;
  if (lds > 160 * 1024) { snprintf(err, errlen, "moe: K*I+S too large for LDS"); return -1; }
  constexpr int DW = 8;                           // waves per block: 4 output rows
  const dim3 grid((a->D + DW / 2 - 1) / (DW / 2), a->B);
  // chunks per lane sized to the rows (registers: 16 waves per CU)
  const uint32_t wsz = a->wdt == THVM_DT_FP8E4M3 ? 1 : 2;
  const bool nc2 = a->I * wsz / 16 <= 128, ncs4 = a->S * wsz / 16 <= 256;
  moe_fn f;
  if (a->wdt == THVM_DT_FP8E4M3)
    f = nc2 ? (ncs4 ? k_moe_down<true, 2, 4, DW> : k_moe_down<true, 2, 8, DW>)
            : (ncs4 ? k_moe_down<true, 4, 4, DW> : k_moe_down<true, 4, 8, DW>);
  else
    f = nc2 ? (ncs4 ? k_moe_down<false, 2, 4, DW> : k_moe_down<false, 2, 8, DW>)
            : (ncs4 ? k_moe_down<false, 4, 4, DW> : k_moe_down<false, 4, 8, DW>);
  if (lds > 64 * 1024) {
    hipError_t e = hipFuncSetAttribute((const void *)f, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) { snprintf(err, errlen, "moe_down: hipFuncSetAttribute: %s", hipGetErrorString(e)); return -1; }
  }
  thvm_launch(true, true, f, grid, dim3(64 * DW), lds, s, *a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) { snprintf(err, errlen, "moe_down launch: %s", hipGetErrorString(e)); return -1; }
  return 0;
}
