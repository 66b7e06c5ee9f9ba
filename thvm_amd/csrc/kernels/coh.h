// coh.h -- cross-block communication inside one launch on gfx950: coherent
// (system-scope) loads and stores, and a grid barrier for persistent kernels.
//
// The eight XCDs of an MI355X each have their own L2, and those L2s are not
// coherent with one another for ordinary device memory.  The C++ way to
// publish data across XCDs, an agent-scope release/acquire, writes back and
// invalidates the whole L2 of the issuing XCD (buffer_wbl2 + buffer_inv): a
// grid barrier built that way costs 12-35 us (measured, 256-512 blocks).  The
// data a decode stage hands to the next is small (activations, partials), so
// instead every such access carries the system-scope cache bits (sc0 sc1):
// stores write through every cache level and loads miss them, and data
// written on one XCD is read correctly on another with no cache maintenance.
// Ordering is explicit: a writer waits for its own stores (vmcnt(0)) before
// it signals, and a reader loads only after it has seen the signal.
//
// Accesses go through buffer resources over a wave-uniform base pointer (the
// buffer intrinsics take the cache-policy bits directly); offsets are in
// bytes and stay below 2 GiB (checked by the launchers).
//
// Grid barrier: block b arrives on counter (b % SYNC_GROUPS) with one
// agent-scope atomic add; the blocks of a group share one XCD (blocks are
// dispatched to XCDs round-robin), so contention is SYNC_GROUPS-fold lower
// than on one counter.  The poll is one wave: lane g < SYNC_GROUPS loads
// counter g until it reaches the barrier's target.  Targets grow
// monotonically across launches (an epoch word advanced at the end of each
// launch), so the counters are never reset.  Every wait is bounded by the
// wall clock (100 MHz): on expiry the block raises the error word and the
// kernel unwinds; every later wait sees the error word and returns at once.
#pragma once
#include "dev_common.h"

#define COH_AUX 17          /* SC0 | SC1: system scope */
#define COH_RANGE 0x7fffffff

__device__ __forceinline__ buf_t coh_rsrc(const void *base) { return buf_rsrc(base, COH_RANGE); }

__device__ __forceinline__ uint4 coh_ld16(const void *base, uint32_t off) {
  u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(coh_rsrc(base), off, 0, COH_AUX);
  return make_uint4(v[0], v[1], v[2], v[3]);
}
__device__ __forceinline__ uint2 coh_ld8(const void *base, uint32_t off) {
  auto v = __builtin_amdgcn_raw_buffer_load_b64(coh_rsrc(base), off, 0, COH_AUX);
  return make_uint2(v[0], v[1]);
}
__device__ __forceinline__ uint32_t coh_ld4(const void *base, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b32(coh_rsrc(base), off, 0, COH_AUX);
}
__device__ __forceinline__ uint16_t coh_ld2(const void *base, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b16(coh_rsrc(base), off, 0, COH_AUX);
}
__device__ __forceinline__ void coh_st16(void *base, uint32_t off, uint4 v) {
  u32x4_t w = {v.x, v.y, v.z, v.w};
  __builtin_amdgcn_raw_buffer_store_b128(w, coh_rsrc(base), off, 0, COH_AUX);
}
__device__ __forceinline__ void coh_st8(void *base, uint32_t off, uint2 v) {
  typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
  u32x2_t w = {v.x, v.y};
  __builtin_amdgcn_raw_buffer_store_b64(w, coh_rsrc(base), off, 0, COH_AUX);
}
__device__ __forceinline__ void coh_st4(void *base, uint32_t off, uint32_t v) {
  __builtin_amdgcn_raw_buffer_store_b32(v, coh_rsrc(base), off, 0, COH_AUX);
}
__device__ __forceinline__ void coh_st2(void *base, uint32_t off, uint16_t v) {
  __builtin_amdgcn_raw_buffer_store_b16(v, coh_rsrc(base), off, 0, COH_AUX);
}
__device__ __forceinline__ float coh_ldf(const void *base, uint32_t off) {
  return __uint_as_float(coh_ld4(base, off));
}
__device__ __forceinline__ void coh_stf(void *base, uint32_t off, float v) {
  coh_st4(base, off, __float_as_uint(v));
}

// wait until every vector memory access this wave issued has completed (its
// stores are visible at system scope); also a compiler barrier
__device__ __forceinline__ void vm_drain() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// ---- sync area layout (uint32 words) --------------------------------------
#define SYNC_GROUPS 32
#define SYNC_STRIDE 32                       /* one 128-byte line per counter */
#define SYNC_W_EPOCH (SYNC_GROUPS * SYNC_STRIDE)
#define SYNC_W_ERR (SYNC_W_EPOCH + SYNC_STRIDE)
#define SYNC_W_FINAL (SYNC_W_ERR + SYNC_STRIDE)        /* last-block counter of the tail */
#define SYNC_W_MERGE (SYNC_W_FINAL + SYNC_STRIDE)       /* per-(row, kv head) merge counters */
#define SYNC_MAX_MERGE 256                              /* B * Hkv <= 256 */
#define SYNC_W_CLOCK (SYNC_W_MERGE + SYNC_MAX_MERGE * SYNC_STRIDE)   /* stage clock, 64-bit */
#define SYNC_MAX_CLOCK 1024                             /* barriers + 2 recorded */
#define SYNC_W_DCLOCK (SYNC_W_CLOCK + 2 * SYNC_MAX_CLOCK)  /* per-stage detail clock */
#define SYNC_DCLOCK_EV 4                                 /* events per stage */
#define SYNC_WORDS (SYNC_W_DCLOCK + 2 * SYNC_DCLOCK_EV * SYNC_MAX_CLOCK)
#define SYNC_BYTES (SYNC_WORDS * 4)
#define SYNC_SPIN_TICKS 200000000ull                    /* 2 s at 100 MHz */

struct GridSync {
  uint32_t *w;           // sync area
  uint32_t base;         // epoch * barriers per launch
  uint32_t nblk;

  // blocks in group g
  __device__ __forceinline__ uint32_t group_count(uint32_t g) const {
    return nblk / SYNC_GROUPS + (g < nblk % SYNC_GROUPS ? 1u : 0u);
  }
  // Called by every thread of the block once each wave has drained its
  // stage's stores (vm_drain) -- and possibly issued loads of the next
  // stage, which need not complete: block barrier, one arrival, wave 0 polls
  // barrier k, block barrier.  Returns false when the wait expired or another
  // block failed (the caller unwinds).  `flag` is one LDS word.
  __device__ bool sync(uint32_t k, uint32_t *flag) const {
    __syncthreads();
    const int lane = lane_id();
    if (threadIdx.x < 64) {
      if (lane == 0)
        __hip_atomic_fetch_add(w + (blockIdx.x % SYNC_GROUPS) * SYNC_STRIDE, 1u, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
      const bool ok = wait_wave(k);
      if (lane == 0) {
        *flag = ok ? 1u : 0u;
        // stage clock: block 0 records when barrier k opened (slot k + 1)
        if (blockIdx.x == 0 && k + 1 < SYNC_MAX_CLOCK) clock(k + 1);
      }
    }
    __syncthreads();
    return *flag != 0u;
  }
  // the wall clock (100 MHz) into stage-clock slot i (one thread)
  __device__ __forceinline__ void clock(uint32_t i) const {
    const uint64_t t = wall_clock64();
    coh_st8(w, (SYNC_W_CLOCK + 2 * i) * 4, make_uint2((uint32_t)t, (uint32_t)(t >> 32)));
  }
  // block 0, thread 0: detail clock of stage st, event ev (0 entry, 1 barrier
  // open, 2 work done, 3 stores drained)
  __device__ __forceinline__ void dclock(uint32_t st, uint32_t ev) const {
    if (blockIdx.x != 0 || threadIdx.x != 0 || st >= SYNC_MAX_CLOCK) return;
    const uint64_t t = wall_clock64();
    coh_st8(w, (SYNC_W_DCLOCK + 2 * (st * SYNC_DCLOCK_EV + ev)) * 4,
            make_uint2((uint32_t)t, (uint32_t)(t >> 32)));
  }
  // wave 0 only: poll until every group reached barrier k
  __device__ bool wait_wave(uint32_t k) const {
    const int lane = lane_id();
    const uint32_t tgt = (base + k + 1u) * (lane < SYNC_GROUPS ? group_count(lane) : 0u);
    bool done = lane >= SYNC_GROUPS;
    const uint64_t t0 = wall_clock64();
    while (true) {
      if (!done) done = (int32_t)(coh_ld4(w, (uint32_t)lane * SYNC_STRIDE * 4) - tgt) >= 0;
      if (__all(done)) return true;
      if (wall_clock64() - t0 > SYNC_SPIN_TICKS || coh_ld4(w, SYNC_W_ERR * 4) != 0u) {
        coh_st4(w, SYNC_W_ERR * 4, 1u);
        return false;
      }
      __builtin_amdgcn_s_sleep(1);
    }
  }
};
