/* tune.c -- device search over a rendered kernel's launch opts.
 *
 * Reference counterpart: the BEAM autotuner (src/codegen/autotune.c: propose
 * candidates, bench each on the kernel's own buffers, keep one only if its
 * output statistics match the baseline's and it is faster, cache the winner
 * on disk by a structural key) over the CUDA action space of
 * src/codegen/propose.c:382-415 (LOCAL 256/128/64/32, UPCAST 8/4/2).
 *
 * gfx950 action space (ThvmRenderOpts): group 1..1024 threads per output
 * (GROUP_REDUCE; the whole 64-lane wave and beyond, with the 160 KiB of LDS
 * holding only the group's wave partials), block 64..1024 (LOCAL) and upcast
 * 1..8 (UPCAST, one thread per output).  The search is a beam ($BEAM wide,
 * default 3; AUTOTUNE_DISABLE=1 or AUTOTUNE_CACHE=0 bypass the cache):
 * the group sizes first (each with the block the hand-coded choice would
 * give it), then the block sizes around the kept groups, then upcast for
 * one-thread-per-output kernels.  Every candidate is rendered, compiled
 * (hiprtc, code objects cached), run `reps` times between two events on the
 * dispatch stream, and its output compared with the hand-coded choice's:
 * floats within 1e-5 relative plus 1e-6 of the largest magnitude (the
 * summation order changes with the group), integers exactly.  Each timed
 * launch runs on cold caches (a 512 MiB read sweep before it), and the
 * winner must beat the hand-coded choice by 3% and 0.3 us.  The caller's
 * output buffer ends holding the winner's result.  Winners are cached in the
 * process and under $AUTOTUNE_CACHE_DIR (else $THVM_HIP_CACHE_DIR/tune/) by a
 * hash of the rows. */
#define _GNU_SOURCE
#include "internal.h"
#include "thvm_hip.h"

#include <errno.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/stat.h>

#define TUNE_SRC_CAP (1u << 20)
#define TUNE_MEM 256

typedef struct { u64 key; ThvmRenderOpts o; } TuneHit;
static TuneHit TUNE_CACHE[TUNE_MEM];
static u32 TUNE_N;

static u64 rows_key(const ThvmUop *nodes, uint32_t n) {
  return hb_hash64(nodes, (size_t)n * sizeof *nodes, 0x74756e65ull);
}

/* $AUTOTUNE_CACHE_DIR (the reference's switch) or $THVM_HIP_CACHE_DIR/tune */
static int disk_path(u64 key, char *p, size_t cap) {
  const char *a = getenv("AUTOTUNE_CACHE_DIR");
  const char *d = a && a[0] ? a : getenv("THVM_HIP_CACHE_DIR");
  if (!d || !d[0]) return -1;
  char dir[512];
  if (a && a[0]) snprintf(dir, sizeof dir, "%s", d);
  else snprintf(dir, sizeof dir, "%s/tune", d);
  if (mkdir(d, 0755) && errno != EEXIST) return -1;
  if (mkdir(dir, 0755) && errno != EEXIST) return -1;
  snprintf(p, cap, "%s/%016llx.txt", dir, (unsigned long long)key);
  return 0;
}

static int cache_get(u64 key, ThvmRenderOpts *o) {
  for (u32 i = 0; i < TUNE_N; i++)
    if (TUNE_CACHE[i].key == key) { *o = TUNE_CACHE[i].o; return 1; }
  char p[640];
  if (disk_path(key, p, sizeof p)) return 0;
  FILE *f = fopen(p, "r");
  if (!f) return 0;
  unsigned b = 0, g = 0, u = 0;
  const int ok = fscanf(f, "block=%u group=%u upcast=%u", &b, &g, &u) == 3;
  fclose(f);
  if (!ok) return 0;
  o->block = b; o->group = g; o->upcast = u; o->reserved = 0;
  return 1;
}

static void cache_put(u64 key, const ThvmRenderOpts *o) {
  if (TUNE_N < TUNE_MEM) { TUNE_CACHE[TUNE_N].key = key; TUNE_CACHE[TUNE_N].o = *o; TUNE_N++; }
  char p[640];
  if (disk_path(key, p, sizeof p)) return;
  FILE *f = fopen(p, "w");
  if (!f) return;
  fprintf(f, "block=%u group=%u upcast=%u\n", o->block, o->group, o->upcast);
  fclose(f);
}

typedef struct {
  const ThvmUop *nodes;
  uint32_t n;
  const uint32_t *ids;
  uint32_t n_args;
  uint32_t reps;
  char *src;
  u32 out_dt;
  u64 out_bytes;
  void *want, *got;
  int n_run;
  void *flush;          /* TUNE_FLUSH_BYTES swept between timed runs (NULL: warm timing) */
  uint32_t *sink;
} Tune;
/* larger than the Infinity Cache (256 MiB) and every XCD's L2 together */
#define TUNE_FLUSH_BYTES (512ull << 20)
#define TUNE_SINK 4096u

static float as_f(const void *p, u64 i, u32 dt) {
  switch (dt) {
    case THVM_DT_FP32: return ((const float *)p)[i];
    case THVM_DT_BF16: { const uint32_t u = (uint32_t)((const uint16_t *)p)[i] << 16; float f; memcpy(&f, &u, 4); return f; }
    default: return 0.0f;
  }
}

/* output of this run == the baseline's (see the header) */
static int outputs_match(const Tune *t) {
  const u32 dt = t->out_dt;
  if (dt != THVM_DT_FP32 && dt != THVM_DT_BF16) return memcmp(t->got, t->want, t->out_bytes) == 0;
  const u64 n = t->out_bytes / (dt == THVM_DT_FP32 ? 4 : 2);
  float scale = 0.0f;
  for (u64 i = 0; i < n; i++) {
    const float w = fabsf(as_f(t->want, i, dt));
    if (isfinite(w) && w > scale) scale = w;
  }
  const float rel = dt == THVM_DT_FP32 ? 1e-5f : 1.0f / 128.0f;
  for (u64 i = 0; i < n; i++) {
    const float w = as_f(t->want, i, dt), g = as_f(t->got, i, dt);
    if (w == g || (isnan(w) && isnan(g))) continue;
    if (!(fabsf(g - w) <= rel * fabsf(w) + 1e-6f * scale)) return 0;
  }
  return 1;
}

/* render + run one candidate: its mean time in us, or < 0 when it does not
 * render, launch, or match */
static double run_candidate(Tune *t, const ThvmRenderOpts *o, int baseline) {
  char name[80];
  snprintf(name, sizeof name, "tune_%016llx_%u_%u_%u", (unsigned long long)rows_key(t->nodes, t->n),
           o->block, o->group, o->upcast);
  ThvmRenderInfo info;
  if (thvm_hip_render_kernel_opts(t->nodes, t->n, name, o, t->src, TUNE_SRC_CAP, &info)) return -1.0;
  if (info.n_slots != t->n_args || info.grid_max > 0x7fffffffull) return -1.0;
  const u32 grid[3] = {(u32)info.grid_max, 1, 1}, block[3] = {info.block, 1, 1};
  if (hb_launch_op(name, t->src, grid, block, 0, t->ids, t->n_args)) return -1.0;   /* compile + warm */
  hipEvent_t e0 = NULL, e1 = NULL;
  if (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess) {
    if (e0) hipEventDestroy(e0);
    hb_set_error("autotune: hipEventCreate failed");
    return -2.0;
  }
  /* each repetition timed alone on cold caches: the flush sweep runs
   * between the event pairs, as the kernel runs in a decode step after other
   * kernels have streamed their own bytes (times taken back to back on warm
   * caches favour geometries that lose in a step) */
  int rc = 0;
  float ms = 0.0f;
  for (u32 r = 0; !rc && r < t->reps; r++) {
    if (t->flush) {
      char err[128];
      if (thvm_k_touch(t->flush, TUNE_FLUSH_BYTES, t->sink, TUNE_SINK, HB_STREAM, err, sizeof err)) {
        hb_set_error("autotune: %s", err);
        rc = 1;
        break;
      }
    }
    rc = hipEventRecord(e0, HB_STREAM) != hipSuccess;
    if (!rc) rc = hb_launch_op(name, t->src, grid, block, 0, t->ids, t->n_args);
    if (!rc) rc = hipEventRecord(e1, HB_STREAM) != hipSuccess;
    float one = 0.0f;
    if (!rc) rc = hipEventSynchronize(e1) != hipSuccess || hipEventElapsedTime(&one, e0, e1) != hipSuccess;
    ms += one;
  }
  hipEventDestroy(e0);
  hipEventDestroy(e1);
  if (rc) return -1.0;
  t->n_run++;
  if (thvm_hip_buf_read(t->ids[0], baseline ? t->want : t->got, t->out_bytes)) return -2.0;
  if (!baseline && !outputs_match(t)) return -1.0;
  return (double)ms * 1000.0 / t->reps;
}

typedef struct { ThvmRenderOpts o; double us; } Cand;
#define BEAM_MAX 16

/* beam width: $BEAM (1..16, default 3), as the reference reads it */
static int beam_width(void) {
  const char *e = getenv("BEAM");
  const int w = e && e[0] ? atoi(e) : 3;
  return w < 1 ? 3 : w > BEAM_MAX ? BEAM_MAX : w;
}
/* AUTOTUNE_DISABLE=1 or AUTOTUNE_CACHE=0: no cached winners */
static int cache_off(void) {
  const char *d = getenv("AUTOTUNE_DISABLE"), *c = getenv("AUTOTUNE_CACHE");
  return (d && d[0] == '1') || (c && c[0] == '0' && !c[1]);
}

static void keep_top(Cand *top, int *nt, int w, ThvmRenderOpts o, double us) {
  if (us < 0) return;
  for (int i = 0; i < *nt; i++)
    if (!memcmp(&top[i].o, &o, sizeof o)) return;
  int at;
  if (*nt < w) {
    at = (*nt)++;
  } else {
    if (us >= top[w - 1].us) return;
    at = w - 1;
  }
  top[at].o = o;
  top[at].us = us;
  for (int i = at; i > 0 && top[i].us < top[i - 1].us; i--) { Cand c = top[i]; top[i] = top[i - 1]; top[i - 1] = c; }
}

THVM_API int thvm_hip_render_autotune(const ThvmUop *nodes, uint32_t n, const uint32_t *buf_ids,
                                      uint32_t n_args, uint32_t reps, ThvmRenderOpts *best,
                                      double *best_us, double *base_us) {
  if (!nodes || n == 0 || !buf_ids || n_args == 0 || !best) { hb_set_error("render_autotune: bad arguments"); return -1; }
  /* an input slot bound to the output buffer is an in-place update too: every
   * repetition would read what the previous one wrote */
  for (uint32_t i = 1; i < n_args; i++)
    if (buf_ids[i] == buf_ids[0]) {
      hb_set_error("render_autotune: the kernel reads its output buffer (slot %u is the output's buffer)", i);
      return -1;
    }
  if (hb_require_ready("render_autotune")) return -1;
  if (hb_stream_capturing() || thvm_hip_jit_is_capturing()) { hb_set_error("render_autotune: not during a capture"); return -1; }
  if (reps == 0) reps = 20;
  const u64 key = rows_key(nodes, n);
  Tune t;
  memset(&t, 0, sizeof t);
  t.nodes = nodes; t.n = n; t.ids = buf_ids; t.n_args = n_args; t.reps = reps;
  t.out_bytes = hb_buf_size(buf_ids[0]);
  {
    const ThvmUop *st = &nodes[n - 1];
    if (st->op != 37 || st->src[0] < 0 || (uint32_t)st->src[0] >= n) {
      hb_set_error("render_autotune: the last row must be the STORE");
      return -1;
    }
    t.out_dt = nodes[st->src[0]].dtype;
    /* a kernel reading its own output (an in-place update) changes what the
     * next repetition computes: not searched */
    for (uint32_t i = 0; i < n; i++)
      if (nodes[i].op == 26 && nodes[i].src[0] >= 0 && nodes[nodes[i].src[0]].op == 36 &&
          nodes[nodes[i].src[0]].arg[0] == 0) {
        hb_set_error("render_autotune: the kernel reads its output buffer");
        return -1;
      }
  }
  /* the cold-cache sweep's buffer, for this search only (a device without
   * the room times warm) */
  if (hipMalloc(&t.flush, TUNE_FLUSH_BYTES + TUNE_SINK * 4) != hipSuccess) {
    (void)hipGetLastError();
    t.flush = NULL;
  } else {
    t.sink = (uint32_t *)((char *)t.flush + TUNE_FLUSH_BYTES);
    char err[128];
    if (thvm_k_zero(t.flush, TUNE_FLUSH_BYTES + TUNE_SINK * 4, HB_STREAM, err, sizeof err)) {
      hb_set_error("render_autotune: %s", err);
      (void)hipFree(t.flush);
      return -1;
    }
  }
  t.src = (char *)malloc(TUNE_SRC_CAP);
  t.want = malloc(t.out_bytes ? t.out_bytes : 1);
  t.got = malloc(t.out_bytes ? t.out_bytes : 1);
  int rc = -1;
  if (!t.src || !t.want || !t.got) { hb_set_error("render_autotune: out of host memory"); goto out; }
  /* the hand-coded choice: the baseline output and time */
  ThvmRenderInfo hi;
  if (thvm_hip_render_kernel(nodes, n, "tune_probe", t.src, TUNE_SRC_CAP, &hi)) goto out;
  ThvmRenderOpts base = {hi.block, hi.group, hi.upcast, 0};
  const double tb = run_candidate(&t, &base, 1);
  if (tb < 0) { if (tb > -2.0) hb_set_error("render_autotune: the hand-coded geometry did not run"); goto out; }
  if (base_us) *base_us = tb;
  ThvmRenderOpts hit;
  if (!cache_off() && cache_get(key, &hit)) {
    const double th = run_candidate(&t, &hit, 0);
    if (th >= 0) { *best = hit; if (best_us) *best_us = th; rc = 0; goto out; }
  }
  const int W = beam_width();
  Cand top[BEAM_MAX];
  int nt = 0;
  keep_top(top, &nt, W, base, tb);
  /* 1: groups (the reduction's thread count), block = max(group, 256) */
  static const uint32_t groups[] = {1, 4, 8, 16, 32, 64, 128, 256, 512, 1024};
  for (size_t i = 0; i < sizeof groups / sizeof groups[0]; i++) {
    ThvmRenderOpts o = {groups[i] > 256 ? groups[i] : 256, groups[i], 1, 0};
    keep_top(top, &nt, W, o, run_candidate(&t, &o, 0));
  }
  /* 2: blocks around the kept groups */
  Cand kept[BEAM_MAX];
  const int nk = nt;
  memcpy(kept, top, sizeof top);
  static const uint32_t blocks[] = {64, 128, 256, 512, 1024};
  for (int k = 0; k < nk; k++)
    for (size_t i = 0; i < sizeof blocks / sizeof blocks[0]; i++) {
      if (blocks[i] < kept[k].o.group) continue;
      ThvmRenderOpts o = kept[k].o;
      o.block = blocks[i];
      keep_top(top, &nt, W, o, run_candidate(&t, &o, 0));
    }
  /* 3: upcast where one thread owns an output */
  memcpy(kept, top, sizeof top);
  const int nk2 = nt;
  for (int k = 0; k < nk2; k++) {
    if (kept[k].o.group > 1) continue;
    for (uint32_t u = 2; u <= 8; u *= 2) {
      ThvmRenderOpts o = kept[k].o;
      o.upcast = u;
      keep_top(top, &nt, W, o, run_candidate(&t, &o, 0));
    }
  }
  /* a searched geometry replaces the hand-coded one only when it is clearly
   * faster (3% and 0.3 us): differences inside the timing noise of a
   * single launch do not carry over to a decode step */
  if (top[0].us < tb * 0.97 - 0.3) {
    *best = top[0].o;
    if (best_us) *best_us = top[0].us;
  } else {
    *best = base;
    if (best_us) *best_us = tb;
  }
  if (!cache_off()) cache_put(key, best);
  /* leave the winner's output in the caller's buffer */
  if (run_candidate(&t, best, 0) < 0) { hb_set_error("render_autotune: the winner did not rerun"); goto out; }
  rc = 0;
out:
  if (t.flush) {
    (void)hipStreamSynchronize(HB_STREAM);
    (void)hipFree(t.flush);
  }
  free(t.src);
  free(t.want);
  free(t.got);
  return rc;
}
