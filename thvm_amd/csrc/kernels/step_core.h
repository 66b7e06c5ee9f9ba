// step_core.h -- the whole LLAMA decode step as one persistent launch
// (kernel templates; instantiated by step_m{1,2,4}.hip, launched by step.hip).
//
// Replaces, for batch-small decode, the per-op dispatch of a captured step
// (reference: jit_replay re-dispatching the op list, src/jit/capture.c:2687-
// 2884, one kernel per op; bench/dsv2_decode_bench.c step_build :2328-2430,
// about 14 kernels per layer).  At batch 1 every op is HBM-bound but small
// (8-117 MB), and a kernel boundary costs its launch gap plus the ramp and
// tail of a kernel whose loads all wait on the previous one: measured, these
// fixed costs were about half of the step.  Here one block per CU runs every
// stage, and the stages are separated by grid barriers (coh.h, ~2 us) -- but
// each wave issues its first weight loads of the NEXT stage before it waits
// at the barrier (weights do not depend on the previous stage), so HBM keeps
// streaming across stage boundaries.
//
// Stages, per layer (k = barrier index):
//   QKV   RMSNorm(x) . Wqkv^T, RoPE(q, k), k/v appended at L-1  [R=2 rows/wave]
//   ATTN  split units (kv head, 64 rows, batch row), two units per block at a
//         time (8 waves each); the last unit of a (row, kv head) to finish
//         merges its G heads (an atomic counter per (row, kv head))
//   O     x += att . Wo^T                                       [R=1]
//   GU    h = silu(g) * u of RMSNorm(x) . Wgu^T                  [R=2]
//   DOWN  x += h . Wd^T                                          [R=1]
// then LM (final RMSNorm, logits, per-wave argmax) and the tail: the last
// block to finish reduces the per-block argmax, writes tok / history and
// advances L and the barrier epoch.  Layer 0's QKV stage reads x straight
// from the embedding rows (block 0 also stores them as the residual).
//
// Numerics: every row of every projection is computed by gemv_core, every
// split and merge by attn_core, with the staging of an 8-wave block -- the
// multi-kernel step's code and orders -- so the outputs are identical to it
// bit for bit.  Data handed between stages moves with system-scope accesses
// (coh.h); read-only inputs (weights, scales, gains, tables) use plain loads.
#pragma once
#include "gemv_core.h"
#include "attn_core.h"

#define STEP_THREADS 1024
#define STEP_WAVES (STEP_THREADS / 64)
#define STAGE_THREADS 512            /* x staging of an 8-wave GEMV block */
#define STEP_U 4
#define STEP_MAX_M 4

// argmax order: larger value, then lower index (rowops.hip am_better)
__device__ __forceinline__ bool st_better(float v, int32_t i, float bv, int32_t bi) {
  return v > bv || (v == bv && i < bi);
}

template <int AT> struct AtXd;
template <> struct AtXd<AT_BF16> { static constexpr int XD = XD_BF16; };
template <> struct AtXd<AT_F16>  { static constexpr int XD = XD_F16; };

// per-wave argmax of the LM stage, read by the tail (one LDS array for both)
static __shared__ float step_amv[STEP_WAVES][STEP_MAX_M];
static __shared__ int32_t step_ami[STEP_WAVES][STEP_MAX_M];

// Barrier index of stage st (0 QKV, 1 ATTN, 2 O, 3 GU, 4 DOWN) of layer l:
// the first QKV stage has no barrier before it; the LM stage takes the last.
__device__ __forceinline__ uint32_t bar_index(uint32_t l, uint32_t st) { return l * 5u + st - 1u; }

__device__ __forceinline__ GridSync step_sync(const ThvmStepArgs &a, uint32_t epoch) {
  return GridSync{a.sync, epoch * (a.n_layers * 5u), gridDim.x};
}

template <int AT>
__device__ __forceinline__ ThvmGemvArgs gemv_base(const ThvmStepArgs &a, uint32_t M) {
  ThvmGemvArgs t = {};
  t.M = M; t.wdt = a.wdt; t.xdt = a.adt; t.ydt = a.adt; t.len = a.len;
  t.max_seq = a.max_seq; t.norm_eps = a.eps;
  return t;
}

template <int AT>
__device__ __forceinline__ const void *act_row(const void *base, uint32_t ld, int m) {
  return (const void *)((const char *)base + (uint64_t)m * ld * ATr<AT>::ES);
}

// One projection stage: st in {0 QKV, 2 O, 3 GU, 4 DOWN} of layer l, or the LM
// head (st 5, with the per-wave argmax left in step_amv/step_ami).  Each stage is its
// own function so that register allocation sees one stage at a time.
template <int WT, int AT, int M, int HD, int ST>
__device__ __attribute__((noinline)) bool step_gemv(const ThvmStepArgs &a, uint32_t l, uint32_t epoch) {
  constexpr int XD = AtXd<AT>::XD;
  constexpr int R = (ST == 0 || ST == 3) ? 2 : 1;
  extern __shared__ __align__(16) unsigned char lds[];
  __shared__ __align__(16) float red[GEMV_MAX_WAVES];
  __shared__ uint32_t flag;
  const GridSync gs = step_sync(a, epoch);
  const int wv = threadIdx.x >> 6;
  const uint32_t g0 = blockIdx.x * STEP_WAVES + wv, gstride = gridDim.x * STEP_WAVES;
  const uint32_t D = a.D, HQ = a.H * HD;
  ThvmGemvArgs ga = gemv_base<AT>(a, M);
  const void *xb;
  uint32_t ldx;
  if (ST == 0) {
    const ThvmStepLayer &ly = a.layers[l];
    ga.y = a.q; ga.w = ly.wqkv; ga.scale = ly.sqkv; ga.N = (a.H + 2 * a.Hkv) * HD; ga.K = D;
    ga.ldy = HQ; ga.epi = THVM_EPI_QKV_ROPE; ga.n_heads = a.H; ga.n_kv_heads = a.Hkv;
    ga.head_dim = HD; ga.rope_cos = a.rope_cos; ga.rope_sin = a.rope_sin; ga.kcache = ly.kcache;
    ga.vcache = ly.vcache; ga.norm = 1; ga.norm_w = ly.g_attn;
    xb = a.x; ldx = D;
  } else if (ST == 2) {
    const ThvmStepLayer &ly = a.layers[l];
    ga.y = a.x; ga.res = a.x; ga.w = ly.wo; ga.scale = ly.so; ga.N = D; ga.K = HQ; ga.ldy = D;
    ga.epi = THVM_EPI_RESID;
    xb = a.att; ldx = HQ;
  } else if (ST == 3) {
    const ThvmStepLayer &ly = a.layers[l];
    ga.y = a.h; ga.w = ly.wgu; ga.scale = ly.sgu; ga.N = 2 * a.F; ga.K = D; ga.ldy = a.F;
    ga.epi = THVM_EPI_SWIGLU; ga.norm = 1; ga.norm_w = ly.g_ffn;
    xb = a.x; ldx = D;
  } else if (ST == 4) {
    const ThvmStepLayer &ly = a.layers[l];
    ga.y = a.x; ga.res = a.x; ga.w = ly.wd; ga.scale = ly.sd; ga.N = D; ga.K = a.F; ga.ldy = D;
    ga.epi = THVM_EPI_RESID;
    xb = a.h; ldx = a.F;
  } else {
    ga.y = a.logits; ga.ydt = THVM_DT_FP32; ga.w = a.lm; ga.scale = a.slm; ga.N = a.V; ga.K = D;
    ga.ldy = a.V; ga.epi = THVM_EPI_STORE; ga.norm = 1; ga.norm_w = a.norm_f;
    xb = a.x; ldx = D;
  }
  ga.ldx = ldx;
  // layer 0's QKV stage reads the embedding rows and has no barrier before it
  const bool first = ST == 0 && l == 0;
  auto xr = [&](int m) -> const void * {
    if (first) {
      const int32_t t = a.tok[m];
      const uint32_t tv = (t >= 0 && (uint32_t)t < a.V) ? (uint32_t)t : 0u;
      return (const void *)((const char *)a.emb + (uint64_t)tv * D * ATr<AT>::ES);
    }
    return act_row<AT>(xb, ldx, m);
  };
  const uint32_t kb = ST == 5 ? a.n_layers * 5u - 1u : bar_index(l, ST);
  const uint32_t sid = ST == 5 ? a.n_layers * 5u : l * 5u + ST;   // stage id (detail clock)
  gs.dclock(sid, 0);
  auto wait = [&]() {
    const bool r = first || gs.sync(kb, &flag);
    gs.dclock(sid, 1);
    return r;
  };
  bool ok;
  if (ST == 5) {
    float bv[M];
    int32_t bi[M];
#pragma unroll
    for (int m = 0; m < M; m++) { bv[m] = -INFINITY; bi[m] = 0x7fffffff; }
    auto amhook = [&](uint32_t n0, const float (&tot)[R][M]) {
      if (n0 >= ga.N) return;
      // the stored logit: the STORE epilogue's value (acc * scale + 0)
      const float sc = ga.scale != nullptr ? ga.scale[n0] : 1.0f;
#pragma unroll
      for (int m = 0; m < M; m++) {
        const float v = tot[0][m] * sc + 0.0f;
        if (st_better(v, (int32_t)n0, bv[m], bi[m])) { bv[m] = v; bi[m] = (int32_t)n0; }
      }
    };
    ok = gemv_core<WT, XD, M, R, STEP_U, true>(ga, lds, red, g0, gstride, STAGE_THREADS, 8, wait, xr, amhook,
                                               (uint32_t)blockDim.x);
    if (ok && lane_id() == 0) {
#pragma unroll
      for (int m = 0; m < M; m++) { step_amv[wv][m] = bv[m]; step_ami[wv][m] = bi[m]; }
    }
  } else {
    ok = gemv_core<WT, XD, M, R, STEP_U, true>(ga, lds, red, g0, gstride, STAGE_THREADS, 8, wait, xr,
                                               [](uint32_t, const float (&)[R][M]) {}, (uint32_t)blockDim.x);
  }
  gs.dclock(sid, 2);
  vm_drain();
  gs.dclock(sid, 3);
  return ok;
}

// Merge of the G heads of (row ub, kv head uk) by the calling 8-wave half
// (512 threads) when mg is set: the merge every attention form runs.
template <int WT, int AT, int M, int HD, int G>
__device__ __attribute__((noinline)) void step_merge(const ThvmStepArgs &a, uint32_t l, uint32_t ub,
                                                     uint32_t uk, bool mg) {
  extern __shared__ __align__(16) unsigned char lds[];
  static_assert(sizeof(MergeFlatLds<HD, G>) == MERGE_LDS_BYTES, "merge LDS");
  const int wv = threadIdx.x >> 6;
  const int half = wv >> 3, htid = threadIdx.x & 511;
  MergeFlatLds<HD, G> *ml = (MergeFlatLds<HD, G> *)(lds + 2 * sizeof(AttnLds<HD, G>)) + half;
  ThvmAttnArgs aa = {};
  aa.out = a.att; aa.part = a.part; aa.H = a.H; aa.n_split = a.n_split;
  const int32_t L = a.len[0];
  uint32_t n_live = L > 0 ? (uint32_t)((L + ATT_CHUNK - 1) / ATT_CHUNK) : 0u;
  if (n_live > a.n_split) n_live = a.n_split;
  attn_merge_flat<HD, G, AT, true>(aa, ub, uk, n_live, htid, mg, *ml);
}

// The attention stage of layer l: split units (two at a time per block, one
// per 8-wave half), each unit's K/V loads issued before the barrier; the
// last unit of a (row, kv head) merges its G heads.
template <int WT, int AT, int M, int HD, int G>
__device__ __attribute__((noinline)) bool step_attn(const ThvmStepArgs &a, uint32_t l, uint32_t epoch) {
  extern __shared__ __align__(16) unsigned char lds[];
  __shared__ uint32_t flag, mflag[2];
  const GridSync gs = step_sync(a, epoch);
  const ThvmStepLayer &ly = a.layers[l];
  const int32_t L = a.len[0];
  ThvmAttnArgs aa = {};
  aa.out = a.att; aa.q = a.q; aa.kcache = ly.kcache; aa.vcache = ly.vcache; aa.len = a.len;
  aa.part = a.part; aa.B = M; aa.H = a.H; aa.Hkv = a.Hkv; aa.hd = HD; aa.max_seq = a.max_seq;
  aa.chunk = ATT_CHUNK; aa.n_split = a.n_split; aa.qdt = a.adt; aa.cdt = a.adt; aa.odt = a.adt;
  aa.scale = a.attn_scale;
  const int wv = threadIdx.x >> 6;
  const int half = wv >> 3, hw = wv & 7, htid = threadIdx.x & 511;
  AttnLds<HD, G> *al = (AttnLds<HD, G> *)lds + half;
  uint32_t n_live = L > 0 ? (uint32_t)((L + ATT_CHUNK - 1) / ATT_CHUNK) : 0u;
  if (n_live > a.n_split) n_live = a.n_split;
  const uint32_t n_units = M * a.Hkv * n_live, nslots = gridDim.x * 2, slot = blockIdx.x * 2 + half;
  const uint32_t iters = (n_units + nslots - 1) / nslots;
  AttnSplit<HD, G, AT, true> u;
  uint32_t ub = 0, uk = 0, us = 0;
  auto unit = [&](uint32_t it) {
    const uint32_t id = it * nslots + slot;
    us = id % n_live;
    uk = (id / n_live) % a.Hkv;
    ub = id / (n_live * a.Hkv);
    return id < n_units;
  };
  const uint32_t sid = l * 5u + 1u;
  gs.dclock(sid, 0);
  bool act = iters > 0 && unit(0);
  if (act && wv != 0) u.issue(aa, uk, us, ub, hw, L);
  if (!gs.sync(bar_index(l, 1), &flag)) return false;
  gs.dclock(sid, 1);
  if (act && wv == 0) u.issue(aa, uk, us, ub, hw, L);
  for (uint32_t it = 0; it < iters; it++) {
    if (it > 0) {
      act = unit(it);
      if (act) u.issue(aa, uk, us, ub, hw, L);
    }
    u.finish(aa, uk, us, ub, hw, htid, L, act, *al);
    if (it == 0) gs.dclock(sid, 2);
    vm_drain();
    __syncthreads();
    if (htid == 0) {
      uint32_t mg = 0;
      if (act) {
        uint32_t *ctr = a.sync + SYNC_W_MERGE + (ub * a.Hkv + uk) * SYNC_STRIDE;
        const uint32_t old = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (old == n_live - 1) {
          mg = 1;
          __hip_atomic_exchange(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
      }
      mflag[half] = mg;
    }
    __syncthreads();
    step_merge<WT, AT, M, HD, G>(a, l, ub, uk, mflag[half] != 0u);
  }
  vm_drain();
  gs.dclock(sid, 3);
  return true;
}

// The tail, after the LM stage: publish the block's argmax; the last block to
// do so reduces them, writes tok / history, advances L and the epoch.
template <int M>
__device__ __attribute__((noinline)) void step_tail(const ThvmStepArgs &a, uint32_t epoch) {
  __shared__ uint32_t last;
  const uint32_t nblk = gridDim.x;
  const int lane = lane_id();
  __syncthreads();
  if (threadIdx.x < M) {
    const int m = threadIdx.x;
    float v = step_amv[0][m];
    int32_t i = step_ami[0][m];
    for (int w = 1; w < STEP_WAVES; w++)
      if (st_better(step_amv[w][m], step_ami[w][m], v, i)) { v = step_amv[w][m]; i = step_ami[w][m]; }
    coh_stf(a.am_pv, (m * nblk + blockIdx.x) * 4, v);
    coh_st4(a.am_pi, (m * nblk + blockIdx.x) * 4, (uint32_t)i);
  }
  vm_drain();
  __syncthreads();
  if (threadIdx.x == 0) {
    const uint32_t old = __hip_atomic_fetch_add(a.sync + SYNC_W_FINAL, 1u, __ATOMIC_RELAXED,
                                                __HIP_MEMORY_SCOPE_AGENT);
    last = old == nblk - 1 ? 1u : 0u;
    if (last) __hip_atomic_exchange(a.sync + SYNC_W_FINAL, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  if (!last || threadIdx.x >= 64) return;
  const int32_t L = a.len[0];
#pragma unroll
  for (int m = 0; m < M; m++) {
    float v = -INFINITY;
    int32_t i = 0x7fffffff;
    for (uint32_t b = lane; b < nblk; b += 64) {
      const float pv = coh_ldf(a.am_pv, (m * nblk + b) * 4);
      const int32_t pi = (int32_t)coh_ld4(a.am_pi, (m * nblk + b) * 4);
      if (st_better(pv, pi, v, i)) { v = pv; i = pi; }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      const float ov = __shfl_xor(v, off);
      const int32_t oi = __shfl_xor(i, off);
      if (st_better(ov, oi, v, i)) { v = ov; i = oi; }
    }
    if (lane == 0) {
      a.tok[m] = i;
      if (a.hist && L >= 0 && (uint32_t)L < a.hist_stride) a.hist[(uint64_t)m * a.hist_stride + L] = i;
    }
  }
  if (lane == 0) {
    a.len[0] = L + 1;
    const uint32_t nbar = a.n_layers * 5u;
    if (nbar + 1 < SYNC_MAX_CLOCK) step_sync(a, epoch).clock(nbar + 1);   // stage clock: end
    vm_drain();
    coh_st4(a.sync, SYNC_W_EPOCH * 4, epoch + 1u);
  }
}

template <int WT, int AT, int M, int HD, int G>
__global__ __launch_bounds__(STEP_THREADS) void k_llama_step(ThvmStepArgs a) {
  constexpr int ES = ATr<AT>::ES;
  if (coh_ld4(a.sync, SYNC_W_ERR * 4) != 0u) return;       // an earlier launch failed
  const uint32_t epoch = coh_ld4(a.sync, SYNC_W_EPOCH * 4);
  if (blockIdx.x == 0 && threadIdx.x == 0) step_sync(a, epoch).clock(0);   // stage clock: start
  // the residual stream starts as the embedding rows (read by layer 0's O stage)
  if (blockIdx.x == 0) {
    const uint32_t D = a.D;
    for (uint32_t i = threadIdx.x; i < M * D / 8; i += STEP_THREADS) {
      const uint32_t m = i / (D / 8), c = i % (D / 8);
      const int32_t t = a.tok[m];
      const uint32_t tv = (t >= 0 && (uint32_t)t < a.V) ? (uint32_t)t : 0u;
      const uint4 v = ld16((const char *)a.emb + ((uint64_t)tv * D + c * 8) * ES);
      coh_st16(a.x, (m * D + c * 8) * ES, v);
    }
  }
  for (uint32_t l = 0; l < a.n_layers; l++) {
    if (!step_gemv<WT, AT, M, HD, 0>(a, l, epoch)) return;
    if (!step_attn<WT, AT, M, HD, G>(a, l, epoch)) return;
    if (!step_gemv<WT, AT, M, HD, 2>(a, l, epoch)) return;
    if (!step_gemv<WT, AT, M, HD, 3>(a, l, epoch)) return;
    if (!step_gemv<WT, AT, M, HD, 4>(a, l, epoch)) return;
  }
  if (!step_gemv<WT, AT, M, HD, 5>(a, 0, epoch)) return;
  step_tail<M>(a, epoch);
}

typedef void (*step_fn)(ThvmStepArgs);

template <int WT, int AT, int M, int HD>
static step_fn step_pick_g(uint32_t G) {
  switch (G) {
    case 1: return k_llama_step<WT, AT, M, HD, 1>;
    case 2: return k_llama_step<WT, AT, M, HD, 2>;
    case 4: return k_llama_step<WT, AT, M, HD, 4>;
    default: return nullptr;
  }
}
// the instance for batch M (weights fp8 / bf16 with bf16 activations)
template <int M>
static step_fn step_pick(uint32_t wdt, uint32_t adt, uint32_t hd, uint32_t G) {
  if (adt != THVM_DT_BF16) return nullptr;
  if (wdt == THVM_DT_FP8E4M3)
    return hd == 128 ? step_pick_g<WT_FP8, AT_BF16, M, 128>(G) : hd == 64 ? step_pick_g<WT_FP8, AT_BF16, M, 64>(G) : nullptr;
  if (wdt == THVM_DT_BF16)
    return hd == 128 ? step_pick_g<WT_BF16, AT_BF16, M, 128>(G) : hd == 64 ? step_pick_g<WT_BF16, AT_BF16, M, 64>(G) : nullptr;
  return nullptr;
}
