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
#include "launch.h"
#include <stdio.h>

template <int HD, int G, int AT>
__global__ __launch_bounds__(ATT_THREADS) void k_attn(ThvmAttnArgs a) {
  __shared__ AttnLds<HD, G> s;
  const uint32_t kvh = blockIdx.x, split = blockIdx.y, b = blockIdx.z;
  const int32_t L = a.len[0];
  if ((int32_t)(split * ATT_CHUNK) >= L) return;   // the merge reads only live splits
  const int wv = threadIdx.x >> 6;
  AttnSplit<HD, G, AT, false> u;
  u.issue(a, kvh, split, b, wv, L);
  u.finish(a, kvh, split, b, wv, threadIdx.x, L, true, s);
}

template <int HD, int AT>
__global__ __launch_bounds__(256) void k_attn_merge(ThvmAttnArgs a) {
  __shared__ MergeLds s;
  attn_merge<HD, AT, false>(a, blockIdx.x, threadIdx.x, a.len[0], true, s);
}

// Split and merge in one launch: each split unit publishes its partial with
// system-scope stores, drains them, and counts itself on its (row, kv head)
// counter (one agent-scope atomic); the unit that brings the count to the
// number of live splits merges the group's G heads (two at a time, 256
// threads each) and resets the counter.  No fence: the partials never sit
// in an L2.  Same split and merge code as the two-kernel form, so the same
// outputs.  Counters: B*Hkv words after the partials, zero between launches.
template <int HD, int G, int AT>
__global__ __launch_bounds__(ATT_THREADS) void k_attn_fused(ThvmAttnArgs a) {
  __shared__ AttnLds<HD, G> s;
  __shared__ MergeLds ms[2];
  __shared__ uint32_t last;
  const uint32_t kvh = blockIdx.x, split = blockIdx.y, b = blockIdx.z;
  const int32_t L = a.len[0];
  if ((int32_t)(split * ATT_CHUNK) >= L) return;   // dead splits are not counted
  uint32_t n_live = (uint32_t)((L + ATT_CHUNK - 1) / ATT_CHUNK);
  if (n_live > a.n_split) n_live = a.n_split;
  const int wv = threadIdx.x >> 6;
  AttnSplit<HD, G, AT, true, false> u;
  u.issue(a, kvh, split, b, wv, L);
  u.finish(a, kvh, split, b, wv, threadIdx.x, L, true, s);
  vm_drain();
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t *ctr = (uint32_t *)(a.part + (uint64_t)a.B * a.H * a.n_split * (HD + 2)) + b * a.Hkv + kvh;
    const uint32_t old = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    last = old == n_live - 1 ? 1u : 0u;
    if (last) __hip_atomic_exchange(ctr, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  if (!last) return;                               // block-uniform
  const int half = threadIdx.x >> 8;
#pragma unroll
  for (int gb = 0; gb < G; gb += 2) {
    const int g = gb + half;
    attn_merge<HD, AT, true>(a, b * a.H + kvh * G + g, threadIdx.x & 255, L, g < G, ms[half]);
  }
}

typedef void (*attn_fn)(ThvmAttnArgs);
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
  // two launches by default; fused = 1 merges in the split launch.  At the C4
  // shape the fused form measured slower (2.40 vs 2.32 ms per step): one
  // block per kv head then runs all of its heads' merges, where the merge
  // kernel spreads one head per block.
  const bool fused = a->fused != 0;
  attn_fn f = nullptr, fm = nullptr;
  const uint32_t G = a->H / a->Hkv;
  const int at = a->cdt == THVM_DT_BF16 ? AT_BF16 : a->cdt == THVM_DT_FP16 ? AT_F16 : AT_F32;
  if (a->hd == 128) {
    f = at == AT_BF16 ? attn_pick<128, AT_BF16>(G, fused) : at == AT_F16 ? attn_pick<128, AT_F16>(G, fused) : attn_pick<128, AT_F32>(G, fused);
    fm = at == AT_BF16 ? k_attn_merge<128, AT_BF16> : at == AT_F16 ? k_attn_merge<128, AT_F16> : k_attn_merge<128, AT_F32>;
  } else if (a->hd == 64) {
    f = at == AT_BF16 ? attn_pick<64, AT_BF16>(G, fused) : at == AT_F16 ? attn_pick<64, AT_F16>(G, fused) : attn_pick<64, AT_F32>(G, fused);
    fm = at == AT_BF16 ? k_attn_merge<64, AT_BF16> : at == AT_F16 ? k_attn_merge<64, AT_F16> : k_attn_merge<64, AT_F32>;
  }
  if (!f) {
    snprintf(err, errlen, "attn: no kernel for hd=%u G=%u", a->hd, G);
    return -1;
  }
  if ((uint64_t)a->B * a->H * a->n_split * (a->hd + 2) * 4 >= (1ull << 31)) {
    snprintf(err, errlen, "attn: partials of 2 GiB or more");
    return -1;
  }
  thvm_launch(true, fused, f, dim3(a->Hkv, a->n_split, a->B), dim3(ATT_THREADS), 0, s, *a);
  if (!fused) thvm_launch(false, true, fm, dim3(a->B * a->H), dim3(256), 0, s, *a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) { snprintf(err, errlen, "attn launch: %s", hipGetErrorString(e)); return -1; }
  return 0;
}
