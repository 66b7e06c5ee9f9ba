/* hip_backend.c -- the DEV=hip device: lifecycle, buffer table, dispatch
 * drain, timers.  C11 over the HIP runtime C API.
 *
 * Reference counterparts (the CUDA driver-API backend):
 *   lifecycle        src/backend/cuda/init.c:110-146, _.c:12-53
 *   buffer table     src/backend/cuda/init.c:40-60 (CudaBuf), buf_alloc.c,
 *                    buf_free.c, buf_incref.c, buf_decref.c, buf_freelist.c
 *   read / write     buf_read.c:6-26, buf_write.c:7-17, buf_copy.c
 *   dispatch_end     _.c:23-27 (drain unless a graph capture is open)
 *   pool / preserve  buf_pool.c:9-183 (watermark rollback, preserve marks,
 *                    the table-wide unpreserved sweep)
 * Semantics kept: ids are u32 with 0 = none; fresh buffers read as zeros; a
 * decref to 0 parks an owning block on a best-fit freelist, and a recycled
 * block moves to a fresh id (the donor id goes dead), so a stale id can never
 * alias live storage; arena views hold a reference on their parent.
 * Unlike the reference's ever-growing table, dead slots are reused: an id is
 * the slot index (low HB_IDX_BITS bits) and the slot's generation (high
 * bits), bumped each time the slot dies, so a stale id fails the generation
 * check instead of aliasing the slot's next buffer; a slot whose generation
 * is spent is retired.  Pool watermarks are allocation sequence numbers, not
 * slot indices.  All transfers and kernels are ordered on one non-blocking
 * stream created at default priority. */
#define _GNU_SOURCE
#include "internal.h"

#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

char        HB_ERRBUF[512];
int         HB_READY = 0;
hipStream_t HB_STREAM = NULL;
int         HB_GRAPH_CAPTURING = 0;

void hb_set_error(const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(HB_ERRBUF, sizeof HB_ERRBUF, fmt, ap);
  va_end(ap);
  if (getenv("THVM_HIP_QUIET") == NULL) fprintf(stderr, "thvm-hip: %s\n", HB_ERRBUF);
}

THVM_API const char *thvm_hip_last_error(void) { return HB_ERRBUF; }
THVM_API const char *thvm_hip_version(void) { return "thvm-hip 0.1 gfx950"; }

int hb_require_ready(const char *who) {
  if (!HB_READY) {
    hb_set_error("%s: backend not initialised (thvm_hip_init)", who);
    return -1;
  }
  return 0;
}

u64 hb_hash64(const void *p, size_t n, u64 h) {
  const u8 *s = (const u8 *)p;
  if (h == 0) h = 1469598103934665603ull;
  for (size_t i = 0; i < n; i++) { h ^= s[i]; h *= 1099511628211ull; }
  return h;
}

u32 hb_dt_size(u32 dt) {
  switch (dt) {
    case THVM_DT_BOOL: case THVM_DT_INT8: case THVM_DT_UINT8:
    case THVM_DT_FP8E4M3: case THVM_DT_FP8E5M2: return 1;
    case THVM_DT_INT16: case THVM_DT_UINT16: case THVM_DT_FP16: case THVM_DT_BF16: return 2;
    case THVM_DT_INT32: case THVM_DT_UINT32: case THVM_DT_FP32: return 4;
    case THVM_DT_INT64: case THVM_DT_UINT64: case THVM_DT_FP64: return 8;
    default: return 0;
  }
}

/* ======================= buffer table ================================== */

typedef struct {
  void *dptr;          /* device address (view: parent base + offset) */
  u64   nbytes;        /* capacity of the block                       */
  u64   req;           /* requested (logical) size                    */
  u32   refcount;
  u32   parent;        /* views: parent id                            */
  u32   seq;           /* allocation sequence number (pool watermark) */
  uint16_t   gen;           /* generation of the slot's current id         */
  u8    live;
  u8    owns;          /* 1: hipFree on release                       */
  u8    parked;        /* on the freelist (refcount 0)                */
  u8    jit_pinned;
  u8    preserved;     /* survives the current pool rollback          */
  u8    arena;         /* freed outright at rollback, never parked    */
} HbBuf;

#define HB_IDX_BITS     18u
#define HB_BUFS_CAP     (1u << HB_IDX_BITS)
#define HB_IDX_MASK     (HB_BUFS_CAP - 1u)
#define HB_GEN_MAX      ((1u << (32u - HB_IDX_BITS)) - 1u)
#define HB_FREELIST_CAP 4096u

static HbBuf *BUFS = NULL;
static u32    BUFS_NEXT = 1;          /* slots [1, BUFS_NEXT) have been used */
static u32   *DEAD = NULL;            /* reusable dead slot indices          */
static u32    N_DEAD = 0;
static u32    N_RETIRED = 0;          /* slots whose ids are all spent       */
static u32    ALLOC_SEQ = 1;          /* next allocation's sequence number   */
static u32    FREELIST[HB_FREELIST_CAP];
static u32    FREELIST_LEN = 0;
static u64    MEM_LIVE = 0, MEM_PEAK = 0;
/* allocation log: (slot, sequence number) of each buffer issued, in sequence
 * order, so a pool watermark's buffers are found without scanning the table.
 * An entry whose slot has died or been reissued no longer matches its slot's
 * sequence number; compaction drops those. */
static u32   *LOG_IDX = NULL, *LOG_SEQ = NULL;
static u32    LOG_N = 0, LOG_CAP = 0;

static u32 id_of(u32 idx) { return idx | ((u32)BUFS[idx].gen << HB_IDX_BITS); }

static HbBuf *buf_get(u32 id) {
  const u32 idx = id & HB_IDX_MASK;
  if (BUFS == NULL || idx == 0 || idx >= BUFS_NEXT) return NULL;
  HbBuf *b = &BUFS[idx];
  return (b->live && b->gen == (id >> HB_IDX_BITS)) ? b : NULL;
}

void *hb_buf_ptr(u32 id) {
  HbBuf *b = buf_get(id);
  return (b && !b->parked) ? b->dptr : NULL;
}
u64 hb_buf_size(u32 id) {
  HbBuf *b = buf_get(id);
  return (b && !b->parked) ? b->req : 0;
}

/* A slot index for a new buffer: a dead slot if any, else a fresh one.
 * The caller fills the slot and marks it live. */
static u32 slot_new(void) {
  if (N_DEAD) return DEAD[--N_DEAD];
  if (BUFS_NEXT >= HB_BUFS_CAP) {
    hb_set_error("buf_alloc: out of buffer slots (cap %u live)", HB_BUFS_CAP - 1);
    return 0;
  }
  return BUFS_NEXT++;
}
/* a slot taken by slot_new but never issued goes back unchanged */
static void slot_unuse(u32 idx) { DEAD[N_DEAD++] = idx; }
/* the slot's buffer is gone: clear it, bump its generation (every id it
 * issued goes stale), and reuse it -- or retire it when the generation is
 * spent, so an id is never issued twice */
static void slot_kill(u32 idx) {
  const u32 gen = BUFS[idx].gen + 1u;
  memset(&BUFS[idx], 0, sizeof(HbBuf));
  if (gen > HB_GEN_MAX) { N_RETIRED++; return; }
  BUFS[idx].gen = (uint16_t)gen;
  DEAD[N_DEAD++] = idx;
}
static int log_live(u32 i) {
  const HbBuf *b = &BUFS[LOG_IDX[i]];
  return b->live && b->seq == LOG_SEQ[i];
}
/* keep the live entries of [start, LOG_N), in order */
static void log_compact_from(u32 start) {
  u32 w = start;
  for (u32 r = start; r < LOG_N; r++)
    if (log_live(r)) { LOG_IDX[w] = LOG_IDX[r]; LOG_SEQ[w] = LOG_SEQ[r]; w++; }
  LOG_N = w;
}
/* first entry with sequence number >= wm */
static u32 log_first(u32 wm) {
  u32 lo = 0, hi = LOG_N;
  while (lo < hi) {
    const u32 mid = lo + (hi - lo) / 2;
    if (LOG_SEQ[mid] < wm) lo = mid + 1; else hi = mid;
  }
  return lo;
}
static void log_push(u32 idx, u32 seq) {
  const u32 live = BUFS_NEXT - 1u - N_DEAD - N_RETIRED;
  if (LOG_N > 2u * live + 1024u) log_compact_from(0);
  if (LOG_N == LOG_CAP) {
    const u32 cap = LOG_CAP ? 2u * LOG_CAP : 4096u;
    u32 *a = (u32 *)realloc(LOG_IDX, cap * sizeof(u32)), *q = a ? (u32 *)realloc(LOG_SEQ, cap * sizeof(u32)) : NULL;
    if (a) LOG_IDX = a;
    if (!a || !q) return;      /* out of host memory: this buffer is simply never rolled back */
    LOG_SEQ = q;
    LOG_CAP = cap;
  }
  LOG_IDX[LOG_N] = idx;
  LOG_SEQ[LOG_N] = seq;
  LOG_N++;
}

/* fill a fresh slot as a live buffer and return its id */
static u32 slot_issue(u32 idx, void *dptr, u64 nbytes, u64 req, u8 owns, u32 parent) {
  HbBuf *b = &BUFS[idx];
  const uint16_t gen = b->gen;
  memset(b, 0, sizeof *b);
  b->gen = gen;
  b->dptr = dptr;
  b->nbytes = nbytes;
  b->req = req;
  b->refcount = 1;
  b->live = 1;
  b->owns = owns;
  b->parent = parent;
  b->seq = ALLOC_SEQ++;
  log_push(idx, b->seq);
  return id_of(idx);
}

static void freelist_drop(u32 id) {
  for (u32 i = 0; i < FREELIST_LEN; i++) {
    if (FREELIST[i] == id) {
      FREELIST[i] = FREELIST[--FREELIST_LEN];
      return;
    }
  }
}

static void real_free(u32 idx) {
  HbBuf *b = &BUFS[idx];
  if (b->owns && b->dptr) {
    hipStreamSynchronize(HB_STREAM);
    hipFree(b->dptr);
    MEM_LIVE -= b->nbytes;
  }
  slot_kill(idx);
}

/* best fit among parked blocks with capacity in [n, 2n]; moves the block to a
 * fresh slot id (reference buf_freelist.c:42-110 slot swap) */
static u32 freelist_pop(u64 n) {
  u32 best = 0, best_i = 0;
  u64 best_sz = ~0ull;
  for (u32 i = 0; i < FREELIST_LEN; i++) {
    HbBuf *b = &BUFS[FREELIST[i] & HB_IDX_MASK];
    if (b->nbytes >= n && b->nbytes <= 2 * n + 4096 && b->nbytes < best_sz) {
      best = FREELIST[i];
      best_i = i;
      best_sz = b->nbytes;
    }
  }
  if (best == 0) return 0;
  FREELIST[best_i] = FREELIST[--FREELIST_LEN];
  const u32 donor = best & HB_IDX_MASK;
  void *dptr = BUFS[donor].dptr;
  const u64 cap = BUFS[donor].nbytes;
  slot_kill(donor);                        /* donor id goes dead */
  const u32 idx = slot_new();              /* (at worst the donor's own slot, next generation) */
  if (idx == 0) {                          /* its generation was spent and no slot is left */
    hipStreamSynchronize(HB_STREAM);
    hipFree(dptr);
    MEM_LIVE -= cap;
    return 0;
  }
  const u32 nid = slot_issue(idx, dptr, cap, n, 1, 0);
  hipMemsetAsync(dptr, 0, cap, HB_STREAM);
  return nid;
}

static u32 alloc_fresh(u64 nbytes, u8 arena);

THVM_API uint32_t thvm_hip_buf_alloc(uint64_t nbytes) {
  if (hb_require_ready("buf_alloc")) return 0;
  if (hb_stream_capturing()) {       /* a memset node would enter the graph */
    hb_set_error("buf_alloc: not allowed while a graph capture is open");
    return 0;
  }
  const char *cap = getenv("THVM_MAX_BUF_BYTES");
  if (cap && cap[0]) {
    u64 c = strtoull(cap, NULL, 10);
    if (c != 0 && nbytes > c) {
      hb_set_error("buf_alloc: refusing %llu-byte allocation (> THVM_MAX_BUF_BYTES %llu)",
                   (unsigned long long)nbytes, (unsigned long long)c);
      return 0;
    }
  }
  if (nbytes == 0) nbytes = 1;
  u32 r = freelist_pop(nbytes);
  if (r) return r;
  return alloc_fresh(nbytes, 0);
}

/* hipMalloc a zero-filled block into a new slot */
static u32 alloc_fresh(u64 nbytes, u8 arena) {
  u32 idx = slot_new();
  if (idx == 0) return 0;
  u64 cap_bytes = (nbytes + 255) & ~255ull;
  void *p = NULL;
  hipError_t e = hipMalloc(&p, cap_bytes);
  if (e != hipSuccess) {
    slot_unuse(idx);
    hb_set_error("hipMalloc(%llu): %s", (unsigned long long)cap_bytes, hipGetErrorString(e));
    return 0;
  }
  e = hipMemsetAsync(p, 0, cap_bytes, HB_STREAM);
  if (e != hipSuccess) {
    hipFree(p);
    slot_unuse(idx);
    hb_set_error("hipMemsetAsync: %s", hipGetErrorString(e));
    return 0;
  }
  const u32 id = slot_issue(idx, p, cap_bytes, nbytes, 1, 0);
  BUFS[idx].arena = arena;
  MEM_LIVE += cap_bytes;
  if (MEM_LIVE > MEM_PEAK) MEM_PEAK = MEM_LIVE;
  return id;
}

/* A per-realize arena block (the reference's skip_freelist buffers): like
 * buf_alloc, never recycled from or parked on the freelist -- a pool
 * rollback or the unpreserved sweep frees it outright, so its bytes do not
 * sit parked while the next realize allocates a fresh arena. */
THVM_API uint32_t thvm_hip_buf_arena_alloc(uint64_t nbytes) {
  if (hb_require_ready("buf_arena_alloc")) return 0;
  if (hb_stream_capturing()) {
    hb_set_error("buf_arena_alloc: not allowed while a graph capture is open");
    return 0;
  }
  return alloc_fresh(nbytes ? nbytes : 1, 1);
}

THVM_API uint32_t thvm_hip_buf_view(uint32_t parent_id, uint64_t byte_off, uint64_t nbytes) {
  if (hb_require_ready("buf_view")) return 0;
  HbBuf *p = buf_get(parent_id);
  if (!p || p->parked) { hb_set_error("buf_view: parent %u not live", parent_id); return 0; }
  if (byte_off > p->nbytes || nbytes > p->nbytes - byte_off) {
    hb_set_error("buf_view: [%llu, +%llu) outside parent of %llu bytes",
                 (unsigned long long)byte_off, (unsigned long long)nbytes,
                 (unsigned long long)p->nbytes);
    return 0;
  }
  u32 idx = slot_new();
  if (idx == 0) return 0;
  const u32 id = slot_issue(idx, (char *)p->dptr + byte_off, nbytes, nbytes, 0, parent_id);
  p->refcount++;
  return id;
}

static void release(u32 id);

THVM_API void thvm_hip_buf_free(uint32_t buf_id) {
  HbBuf *b = buf_get(buf_id);
  if (!b) return;
  if (b->parked) freelist_drop(buf_id);
  u32 parent = b->owns ? 0 : b->parent;
  real_free(buf_id & HB_IDX_MASK);
  if (parent) release(parent);
}

static void release(u32 id) {
  HbBuf *b = buf_get(id);
  if (!b || b->refcount == 0) return;
  if (--b->refcount > 0) return;
  if (b->jit_pinned) { b->refcount = 1; return; }   /* held by a capture */
  if (b->owns && !b->arena && FREELIST_LEN < HB_FREELIST_CAP) {
    b->parked = 1;
    b->preserved = 0;
    FREELIST[FREELIST_LEN++] = id;
    return;
  }
  thvm_hip_buf_free(id);
}

THVM_API void thvm_hip_buf_incref(uint32_t buf_id) {
  HbBuf *b = buf_get(buf_id);
  if (b && !b->parked) b->refcount++;
}
THVM_API void thvm_hip_buf_decref(uint32_t buf_id) { release(buf_id); }

THVM_API void thvm_hip_buf_jit_pin(uint32_t buf_id) {
  HbBuf *b = buf_get(buf_id);
  if (b) b->jit_pinned = 1;
}
THVM_API void thvm_hip_buf_jit_unpin(uint32_t buf_id) {
  HbBuf *b = buf_get(buf_id);
  if (b) b->jit_pinned = 0;
}
THVM_API uint32_t thvm_hip_buf_refcount(uint32_t buf_id) {
  HbBuf *b = buf_get(buf_id);
  return (b && !b->parked) ? b->refcount : 0;
}
THVM_API void thvm_hip_buf_freelist_push(uint32_t buf_id) {
  HbBuf *b = buf_get(buf_id);
  if (!b || b->parked || !b->owns || b->arena || b->jit_pinned) return;
  if (FREELIST_LEN >= HB_FREELIST_CAP) return;
  b->refcount = 0;
  b->parked = 1;
  b->preserved = 0;
  FREELIST[FREELIST_LEN++] = buf_id;
}
THVM_API void thvm_hip_buf_freelist_remove(uint32_t buf_id) {
  HbBuf *b = buf_get(buf_id);
  if (!b || !b->parked) return;
  freelist_drop(buf_id);
  b->parked = 0;
  b->refcount = 1;
}
THVM_API uint32_t thvm_hip_buf_storage_root(uint32_t buf_id) {
  HbBuf *b = buf_get(buf_id);
  u32 id = buf_id;
  while (b && !b->owns && b->parent) {
    id = b->parent;
    b = buf_get(id);
  }
  return b ? id : 0;
}
THVM_API uint64_t thvm_hip_buf_nbytes(uint32_t buf_id) { return hb_buf_size(buf_id); }
THVM_API uint64_t thvm_hip_buf_device_ptr(uint32_t buf_id) {
  return (uint64_t)(uintptr_t)hb_buf_ptr(buf_id);
}
THVM_API uint64_t thvm_hip_mem_live_bytes(void) { return MEM_LIVE; }
THVM_API uint64_t thvm_hip_mem_peak_bytes(void) { return MEM_PEAK; }
THVM_API uint32_t thvm_hip_buf_slots_used(void) { return BUFS ? BUFS_NEXT - 1u - N_DEAD - N_RETIRED : 0u; }
THVM_API uint32_t thvm_hip_buf_slot_highwater(void) { return BUFS ? BUFS_NEXT - 1u : 0u; }

/* ---- pool watermarks and preserve marks (reference buf_pool.c) ----
 * A watermark is the sequence number the next allocation will take; "since
 * wm" means every live buffer whose sequence number is >= wm (wm 0 or 1:
 * every buffer).  Sequence numbers are 32-bit: a session of more than 2^32
 * allocations wraps them. */
static u32 wm_of(u32 wm) { return wm < 1u ? 1u : wm; }

THVM_API uint32_t thvm_hip_buf_pool_begin(void) { return ALLOC_SEQ; }

THVM_API void thvm_hip_buf_mark_preserved(uint32_t buf_id) {
  HbBuf *b = buf_get(buf_id);
  if (b && !b->parked) b->preserved = 1;
}

THVM_API void thvm_hip_buf_clear_preserved(uint32_t wm) {
  if (!BUFS) return;
  for (u32 i = log_first(wm_of(wm)); i < LOG_N; i++)
    if (log_live(i)) BUFS[LOG_IDX[i]].preserved = 0;
}

/* Arena views since wm lose their mark, and so does their parent when the
 * parent itself was allocated since wm (an older parent -- a weight a view
 * reads -- keeps its mark). */
THVM_API void thvm_hip_buf_clear_preserved_arena_views(uint32_t wm) {
  if (!BUFS) return;
  wm = wm_of(wm);
  for (u32 i = log_first(wm); i < LOG_N; i++) {
    if (!log_live(i)) continue;
    HbBuf *b = &BUFS[LOG_IDX[i]];
    if (b->owns || !b->parent) continue;
    b->preserved = 0;
    HbBuf *p = buf_get(b->parent);
    if (p && p->seq >= wm) p->preserved = 0;
  }
}

/* Every buffer allocated since wm that is not preserved, not held by a JIT
 * capture and not already parked: an arena block is freed, an owning block is
 * parked on the freelist for the next same-size allocation (freed when the
 * freelist is full), a view is freed (releasing its parent).  Refcounts are
 * not consulted: the caller's planner has established that these buffers are
 * dead. */
THVM_API void thvm_hip_buf_pool_rollback_with_preserve(uint32_t wm) {
  if (!BUFS) return;
  const u32 first = log_first(wm_of(wm));
  for (u32 i = first; i < LOG_N; i++) {
    if (!log_live(i)) continue;
    HbBuf *b = &BUFS[LOG_IDX[i]];
    if (b->preserved || b->jit_pinned || b->parked) continue;
    const u32 id = id_of(LOG_IDX[i]);
    if (b->owns && !b->arena) {
      thvm_hip_buf_freelist_push(id);
      if (!b->parked) thvm_hip_buf_free(id);
    } else {
      thvm_hip_buf_free(id);
    }
  }
  log_compact_from(first);
}

/* As the rollback, but every such buffer is freed outright (its storage
 * returned to the device rather than parked). */
THVM_API void thvm_hip_buf_pool_free_unpreserved(uint32_t wm) {
  if (!BUFS) return;
  const u32 first = log_first(wm_of(wm));
  for (u32 i = first; i < LOG_N; i++) {
    if (!log_live(i)) continue;
    HbBuf *b = &BUFS[LOG_IDX[i]];
    if (b->preserved || b->jit_pinned || b->parked) continue;
    thvm_hip_buf_free(id_of(LOG_IDX[i]));
  }
  log_compact_from(first);
}

/* The whole table: every owning buffer that is live, not preserved and not
 * held by a capture is parked (freed when the freelist is full; an arena
 * block is always freed).  Views are left alone -- their storage goes with
 * the parent's entry.  The stream is drained first so no kernel in flight
 * still reads a reclaimed block.  Returns the bytes reclaimed. */
THVM_API uint64_t thvm_hip_buf_free_unpreserved_all(void) {
  if (!HB_READY || !BUFS) return 0;
  u32 n = 0;
  for (u32 i = 1; i < BUFS_NEXT; i++) {
    const HbBuf *b = &BUFS[i];
    n += b->live && !b->parked && b->owns && !b->preserved && !b->jit_pinned;
  }
  if (n == 0) return 0;
  hipStreamSynchronize(HB_STREAM);
  u64 freed = 0;
  for (u32 i = 1; i < BUFS_NEXT; i++) {
    HbBuf *b = &BUFS[i];
    if (!b->live || b->parked || !b->owns || b->preserved || b->jit_pinned) continue;
    freed += b->nbytes;
    const u32 id = id_of(i);
    if (!b->arena) thvm_hip_buf_freelist_push(id);
    if (!b->parked) thvm_hip_buf_free(id);
  }
  log_compact_from(0);
  return freed;
}

/* 1 while work on the dispatch stream is being recorded into a graph
 * (the library's own capture or one the caller opened on the stream) */
int hb_stream_capturing(void) {
  if (HB_GRAPH_CAPTURING) return 1;
  hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
  if (!HB_STREAM || hipStreamIsCapturing(HB_STREAM, &st) != hipSuccess) return 0;
  return st != hipStreamCaptureStatusNone;
}

/* A zero-fill kernel, never a memset node: the reference's jit_replay zeroes
 * recycled outputs inside an open graph capture (src/jit/capture.c:2779-2780). */
THVM_API void thvm_hip_buf_zero(uint32_t buf_id) {
  HbBuf *b = buf_get(buf_id);
  if (!b || b->parked || !HB_READY) return;
  char err[128];
  if (thvm_k_zero(b->dptr, b->req, HB_STREAM, err, sizeof err)) hb_set_error("buf_zero: %s", err);
}

/* Host transfers are refused inside a capture; device-to-device copies are
 * recorded as copy kernels (the reference's KV ASSIGN runs buf_copy_at inside
 * the capture, src/jit/capture.c:2791-2815, src/tensor/assign.c:89-94). */
static int xfer_check_any(const char *who, u32 id, u64 off, u64 n, HbBuf **out, int in_capture_ok) {
  if (hb_require_ready(who)) return -1;
  if (!in_capture_ok && hb_stream_capturing()) {
    hb_set_error("%s: not allowed while a graph capture is open", who);
    return -1;
  }
  HbBuf *b = buf_get(id);
  if (!b || b->parked) { hb_set_error("%s: buffer %u not live", who, id); return -1; }
  if (off > b->req || n > b->req - off) {
    hb_set_error("%s: [%llu, +%llu) outside buffer %u of %llu bytes", who,
                 (unsigned long long)off, (unsigned long long)n, id, (unsigned long long)b->req);
    return -1;
  }
  *out = b;
  return 0;
}
static int xfer_check(const char *who, u32 id, u64 off, u64 n, HbBuf **out) {
  return xfer_check_any(who, id, off, n, out, 0);
}

THVM_API int thvm_hip_buf_write_at(uint32_t buf_id, uint64_t off, const void *src, uint64_t n) {
  HbBuf *b;
  if (xfer_check("buf_write", buf_id, off, n, &b)) return -1;
  if (n == 0) return 0;
  hipError_t e = hipMemcpyAsync((char *)b->dptr + off, src, n, hipMemcpyHostToDevice, HB_STREAM);
  if (e == hipSuccess) e = hipStreamSynchronize(HB_STREAM);
  if (e != hipSuccess) { hb_set_error("buf_write: %s", hipGetErrorString(e)); return -1; }
  return 0;
}
THVM_API int thvm_hip_buf_write(uint32_t buf_id, const void *src, uint64_t n) {
  return thvm_hip_buf_write_at(buf_id, 0, src, n);
}
THVM_API int thvm_hip_buf_read(uint32_t buf_id, void *dst, uint64_t n) {
  HbBuf *b;
  if (xfer_check("buf_read", buf_id, 0, n, &b)) return -1;
  if (n == 0) return 0;
  hipError_t e = hipMemcpyAsync(dst, b->dptr, n, hipMemcpyDeviceToHost, HB_STREAM);
  if (e == hipSuccess) e = hipStreamSynchronize(HB_STREAM);
  if (e != hipSuccess) { hb_set_error("buf_read: %s", hipGetErrorString(e)); return -1; }
  return 0;
}
THVM_API int thvm_hip_buf_copy_at(uint32_t dst_id, uint64_t dst_off, uint32_t src_id, uint64_t n) {
  HbBuf *d, *s;
  if (xfer_check_any("buf_copy", dst_id, dst_off, n, &d, 1)) return -1;
  if (xfer_check_any("buf_copy", src_id, 0, n, &s, 1)) return -1;
  if (n == 0) return 0;
  if (hb_stream_capturing()) {      /* a kernel node in the graph */
    char err[128];
    if (thvm_k_copy_at(d->dptr, d->req, dst_off, 0, NULL, s->dptr, n, HB_STREAM, err, sizeof err)) {
      hb_set_error("buf_copy: %s", err);
      return -1;
    }
    return 0;
  }
  hipError_t e = hipMemcpyAsync((char *)d->dptr + dst_off, s->dptr, n, hipMemcpyDeviceToDevice,
                                HB_STREAM);
  if (e != hipSuccess) { hb_set_error("buf_copy: %s", hipGetErrorString(e)); return -1; }
  return 0;
}

THVM_API int thvm_hip_buf_copy_row(uint32_t dst_id, uint64_t base_off, uint64_t row_bytes,
                                   uint32_t row_buf_id, uint64_t row_buf_off, uint32_t src_id,
                                   uint64_t n) {
  HbBuf *d, *s, *r;
  if (xfer_check_any("buf_copy_row", dst_id, base_off, n, &d, 1)) return -1;
  if (xfer_check_any("buf_copy_row", src_id, 0, n, &s, 1)) return -1;
  if (xfer_check_any("buf_copy_row", row_buf_id, row_buf_off, 4, &r, 1)) return -1;
  if (row_buf_off & 3) { hb_set_error("buf_copy_row: row index offset %llu not 4-byte aligned",
                                      (unsigned long long)row_buf_off); return -1; }
  if (n == 0) return 0;
  char err[128];
  if (thvm_k_copy_at(d->dptr, d->req, base_off, row_bytes,
                     (const int32_t *)((const char *)r->dptr + row_buf_off), s->dptr, n, HB_STREAM,
                     err, sizeof err)) {
    hb_set_error("buf_copy_row: %s", err);
    return -1;
  }
  return 0;
}
THVM_API int thvm_hip_buf_copy(uint32_t dst_id, uint32_t src_id, uint64_t n) {
  return thvm_hip_buf_copy_at(dst_id, 0, src_id, n);
}

/* ======================= lifecycle ===================================== */

THVM_API int thvm_hip_init(void) {
  if (HB_READY) return 0;
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess || n < 1) {
    hb_set_error("init: no HIP device (%s)", hipGetErrorString(e));
    return -1;
  }
  hipDeviceProp_t prop;
  e = hipGetDeviceProperties(&prop, 0);
  if (e != hipSuccess) { hb_set_error("init: hipGetDeviceProperties: %s", hipGetErrorString(e)); return -1; }
  if (strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
    hb_set_error("init: device 0 is %s, this library is built for gfx950", prop.gcnArchName);
    return -1;
  }
  e = hipSetDevice(0);
  if (e != hipSuccess) { hb_set_error("init: hipSetDevice: %s", hipGetErrorString(e)); return -1; }
  {  /* the no-allocation attention's static scratch: its address on this device */
    char err[256];
    if (thvm_k_attn_scratch_setup(err, sizeof err)) { hb_set_error("init: %s", err); return -1; }
  }
  e = hipStreamCreateWithFlags(&HB_STREAM, hipStreamNonBlocking);
  if (e != hipSuccess) { hb_set_error("init: hipStreamCreate: %s", hipGetErrorString(e)); return -1; }
  if (BUFS == NULL) {
    BUFS = (HbBuf *)calloc(HB_BUFS_CAP, sizeof(HbBuf));
    DEAD = (u32 *)malloc(HB_BUFS_CAP * sizeof(u32));
    if (!BUFS || !DEAD) { hb_set_error("init: out of host memory"); return -1; }
  }
  HB_READY = 1;
  return 0;
}

THVM_API int thvm_hip_available(void) { return HB_READY; }

THVM_API void thvm_hip_shutdown(void) {
  if (!HB_READY) return;
  hipStreamSynchronize(HB_STREAM);
  hb_decoder_reset();
  hb_jit_reset();
  hb_graph_reset();
  hb_rtc_reset();
  hb_loader_reset();
  for (u32 i = BUFS_NEXT; i-- > 1;) {
    if (BUFS[i].live && !BUFS[i].owns) memset(&BUFS[i], 0, sizeof(HbBuf));
  }
  for (u32 i = 1; i < BUFS_NEXT; i++) {
    if (BUFS[i].live && BUFS[i].owns && BUFS[i].dptr) hipFree(BUFS[i].dptr);
    memset(&BUFS[i], 0, sizeof(HbBuf));
  }
  BUFS_NEXT = 1;
  N_DEAD = 0;
  N_RETIRED = 0;
  LOG_N = 0;
  FREELIST_LEN = 0;
  MEM_LIVE = 0;
  hipStreamDestroy(HB_STREAM);
  HB_STREAM = NULL;
  HB_READY = 0;
}

/* ======================= dispatch drain ================================ */

THVM_API void thvm_hip_dispatch_begin(void) {}
THVM_API void thvm_hip_dispatch_flush(void) {}
THVM_API void thvm_hip_dispatch_end(void) {
  if (!HB_READY || HB_GRAPH_CAPTURING) return;
  hipError_t e = hipStreamSynchronize(HB_STREAM);
  if (e != hipSuccess) hb_set_error("dispatch_end: %s", hipGetErrorString(e));
}

/* ======================= timers ======================================== */

#define HB_TIMERS 64
static hipEvent_t TIMER_EV[HB_TIMERS];
static u32 TIMER_NEXT = 0;

THVM_API uint32_t thvm_hip_timer_start(void) {
  if (hb_require_ready("timer_start")) return 0;
  u32 id = (TIMER_NEXT % (HB_TIMERS - 1)) + 1;
  TIMER_NEXT++;
  if (TIMER_EV[id] == NULL && hipEventCreate(&TIMER_EV[id]) != hipSuccess) {
    hb_set_error("timer: hipEventCreate failed");
    return 0;
  }
  hipEventRecord(TIMER_EV[id], HB_STREAM);
  return id;
}
THVM_API double thvm_hip_timer_stop(uint32_t id) {
  if (!HB_READY || id == 0 || id >= HB_TIMERS || TIMER_EV[id] == NULL) return -1.0;
  hipEvent_t end;
  if (hipEventCreate(&end) != hipSuccess) return -1.0;
  hipEventRecord(end, HB_STREAM);
  hipEventSynchronize(end);
  float ms = 0.0f;
  hipEventElapsedTime(&ms, TIMER_EV[id], end);
  hipEventDestroy(end);
  return (double)ms;
}

/* ---- per-kernel profiling: an event pair around each builtin launch,
 *      resolved lazily (no per-launch synchronisation) ---- */
typedef struct { char tag[24]; hipEvent_t e0, e1; u64 bytes; } KpRec;
static KpRec *KP = NULL;
static u32 KP_N = 0, KP_CAP = 0;
static int KP_ON = 0;
static hipEvent_t *KP_POOL = NULL;
static u32 KP_POOL_N = 0, KP_POOL_CAP = 0, KP_POOL_USED = 0;

/* Each profiled builtin launch binds an event pair to its own kernels
 * (thvm_k_time_next), so a record's elapsed time is the kernels' execution
 * alone.  Launches made while the stream is being captured are not
 * profiled. */
int hb_kprof_on(void) {
  if (!KP_ON) return 0;
  hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(HB_STREAM, &st) != hipSuccess) return 0;
  return st == hipStreamCaptureStatusNone;
}

static hipEvent_t kp_event(void) {
  if (KP_POOL_USED < KP_POOL_N) return KP_POOL[KP_POOL_USED++];
  if (KP_POOL_N == KP_POOL_CAP) {
    KP_POOL_CAP = KP_POOL_CAP ? 2 * KP_POOL_CAP : 1024;
    KP_POOL = (hipEvent_t *)realloc(KP_POOL, KP_POOL_CAP * sizeof(hipEvent_t));
  }
  hipEvent_t e = NULL;
  hipEventCreate(&e);
  KP_POOL[KP_POOL_N++] = e;
  KP_POOL_USED++;
  return e;
}

void hb_kprof_begin(const char *tag, hipEvent_t *e0, hipEvent_t *e1) {
  (void)tag;
  *e0 = kp_event();
  *e1 = kp_event();
  thvm_k_time_next(*e0, *e1);
}
void hb_kprof_end(const char *tag, hipEvent_t e0, hipEvent_t e1, u64 bytes) {
  if (KP_N == KP_CAP) {
    KP_CAP = KP_CAP ? 2 * KP_CAP : 1024;
    KP = (KpRec *)realloc(KP, KP_CAP * sizeof(KpRec));
  }
  KpRec *r = &KP[KP_N++];
  snprintf(r->tag, sizeof r->tag, "%s", tag);
  r->e0 = e0;
  r->e1 = e1;
  r->bytes = bytes;
}

THVM_API void thvm_hip_kprof_enable(int on) { KP_ON = on; }
THVM_API void thvm_hip_kprof_reset(void) {
  if (HB_READY) hipStreamSynchronize(HB_STREAM);
  KP_N = 0;
  KP_POOL_USED = 0;
}
THVM_API uint64_t thvm_hip_kprof_bytes(const char *tag) {
  u64 tot = 0;
  for (u32 i = 0; i < KP_N; i++)
    if (tag == NULL || strcmp(KP[i].tag, tag) == 0) tot += KP[i].bytes;
  return tot;
}
THVM_API double thvm_hip_kprof_query(const char *tag, uint64_t *count_out) {
  if (!HB_READY) return -1.0;
  hipStreamSynchronize(HB_STREAM);
  double tot = 0.0;
  u64 cnt = 0;
  for (u32 i = 0; i < KP_N; i++) {
    if (tag != NULL && strcmp(KP[i].tag, tag) != 0) continue;
    float ms = 0.0f;
    if (hipEventElapsedTime(&ms, KP[i].e0, KP[i].e1) == hipSuccess) tot += ms;
    cnt++;
  }
  if (count_out) *count_out = cnt;
  return cnt ? tot : -1.0;
}
