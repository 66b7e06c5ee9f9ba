/* hip_custom.c -- custom-kernel dispatch (hiprtc source programs and the
 * built-in hand-written gfx950 kernels), JIT capture/replay over hipGraph,
 * and the backend graph hooks.
 *
 * Reference counterparts:
 *   custom dispatch   src/backend/cuda/jit.c:802 cuda_custom_dispatch, with the
 *                     argument ABI of src/schedule/kernel_custom.c:14-35
 *   nvrtc + cache     src/backend/cuda/jit.c:20-390 (source-hash module cache
 *                     and on-disk PTX cache)        -> hiprtc + code objects
 *   graph hooks       src/backend/cuda/jit.c:444-615
 *   capture / replay  src/jit/capture.c:644-745 (begin/end/drop/op_count),
 *                     :1139 (record), :2615-2684 (input rebinding),
 *                     :2687-2884 (replay: graph hit, else capture the op loop)
 */
#define _GNU_SOURCE
#include "internal.h"

#include <hip/hiprtc.h>
#include <errno.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/stat.h>
#include <unistd.h>

#define BUILTIN_PREFIX "thvm-builtin:"

/* ======================= builtin spec parsing ========================== */

typedef struct {
  char kernel[32];
  u32  n;
  char key[40][16];
  char val[40][48];
} Spec;

static int spec_parse(const char *program, Spec *sp) {
  memset(sp, 0, sizeof *sp);
  const char *p = program + strlen(BUILTIN_PREFIX);
  while (*p == ' ') p++;
  size_t k = 0;
  while (p[k] && p[k] != ' ' && k < sizeof sp->kernel - 1) { sp->kernel[k] = p[k]; k++; }
  sp->kernel[k] = 0;
  if (k == 0) { hb_set_error("builtin: empty kernel name in \"%s\"", program); return -1; }
  p += k;
  while (*p) {
    while (*p == ' ') p++;
    if (!*p) break;
    const char *eq = strchr(p, '=');
    const char *sp_end = strchr(p, ' ');
    if (!eq || (sp_end && sp_end < eq)) { hb_set_error("builtin: malformed token near \"%s\"", p); return -1; }
    if (sp->n >= 40) { hb_set_error("builtin: too many keys"); return -1; }
    size_t kl = (size_t)(eq - p);
    if (kl >= sizeof sp->key[0]) { hb_set_error("builtin: key too long"); return -1; }
    memcpy(sp->key[sp->n], p, kl);
    sp->key[sp->n][kl] = 0;
    const char *v = eq + 1;
    size_t vl = 0;
    while (v[vl] && v[vl] != ' ') vl++;
    if (vl >= sizeof sp->val[0]) { hb_set_error("builtin: value too long"); return -1; }
    memcpy(sp->val[sp->n], v, vl);
    sp->val[sp->n][vl] = 0;
    sp->n++;
    p = v + vl;
  }
  return 0;
}

static const char *spec_get(const Spec *sp, const char *key) {
  for (u32 i = 0; i < sp->n; i++)
    if (strcmp(sp->key[i], key) == 0) return sp->val[i];
  return NULL;
}
static int spec_u32(const Spec *sp, const char *key, u32 *out, int required, u32 dflt) {
  const char *v = spec_get(sp, key);
  if (!v) {
    if (required) { hb_set_error("builtin %s: missing key '%s'", sp->kernel, key); return -1; }
    *out = dflt;
    return 0;
  }
  char *end = NULL;
  errno = 0;
  unsigned long long x = strtoull(v, &end, 0);
  if (errno || end == v || *end || x > 0xffffffffull) {
    hb_set_error("builtin %s: bad value %s=%s", sp->kernel, key, v);
    return -1;
  }
  *out = (u32)x;
  return 0;
}
static int spec_u64(const Spec *sp, const char *key, u64 *out, int required, u64 dflt) {
  const char *v = spec_get(sp, key);
  if (!v) {
    if (required) { hb_set_error("builtin %s: missing key '%s'", sp->kernel, key); return -1; }
    *out = dflt;
    return 0;
  }
  char *end = NULL;
  errno = 0;
  unsigned long long x = strtoull(v, &end, 0);
  if (errno || end == v || *end) { hb_set_error("builtin %s: bad value %s=%s", sp->kernel, key, v); return -1; }
  *out = (u64)x;
  return 0;
}
static int spec_f32(const Spec *sp, const char *key, float *out, int required, float dflt) {
  const char *v = spec_get(sp, key);
  if (!v) {
    if (required) { hb_set_error("builtin %s: missing key '%s'", sp->kernel, key); return -1; }
    *out = dflt;
    return 0;
  }
  char *end = NULL;
  float x = strtof(v, &end);
  if (end == v || *end) { hb_set_error("builtin %s: bad value %s=%s", sp->kernel, key, v); return -1; }
  *out = x;
  return 0;
}

/* argument slot i must be a live buffer of at least `bytes` */
typedef struct { const u32 *ids; u32 n; const char *k; int bad; } ArgCtx;
static void *arg(ArgCtx *c, u32 i, u64 bytes) {
  if (c->bad) return NULL;
  if (i >= c->n) {
    hb_set_error("builtin %s: needs argument slot %u, got %u arguments", c->k, i, c->n);
    c->bad = 1;
    return NULL;
  }
  void *p = hb_buf_ptr(c->ids[i]);
  if (!p) {
    hb_set_error("builtin %s: argument %u (buffer %u) is not live", c->k, i, c->ids[i]);
    c->bad = 1;
    return NULL;
  }
  u64 have = hb_buf_size(c->ids[i]);
  if (have < bytes) {
    hb_set_error("builtin %s: argument %u holds %llu bytes, needs %llu", c->k, i,
                 (unsigned long long)have, (unsigned long long)bytes);
    c->bad = 1;
    return NULL;
  }
  return p;
}

static int is_act(u32 dt) { return dt == THVM_DT_FP32 || dt == THVM_DT_FP16 || dt == THVM_DT_BF16; }

/* the attn builtin's spec and buffer slots: out, q, kcache, vcache, len and,
 * with_part, the partials workspace */
static int attn_parse(const Spec *sp, ArgCtx *c, ThvmAttnArgs *a, int with_part) {
  memset(a, 0, sizeof *a);
  if (spec_u32(sp, "b", &a->B, 1, 0) || spec_u32(sp, "h", &a->H, 1, 0) ||
      spec_u32(sp, "hkv", &a->Hkv, 1, 0) || spec_u32(sp, "hd", &a->hd, 1, 0) ||
      spec_u32(sp, "maxseq", &a->max_seq, 1, 0) || spec_u32(sp, "chunk", &a->chunk, 0, 64) ||
      spec_u32(sp, "qt", &a->qdt, 0, THVM_DT_BF16) || spec_u32(sp, "ct", &a->cdt, 0, THVM_DT_BF16) ||
      spec_u32(sp, "ot", &a->odt, 0, THVM_DT_BF16) || spec_f32(sp, "scale", &a->scale, 1, 0) ||
      spec_u32(sp, "fused", &a->fused, 0, 0) || spec_u32(sp, "cpb", &a->cpb, 0, 0) ||
      spec_u32(sp, "spec", &a->spec, 0, 0) || spec_u32(sp, "clk", &a->clk_cap, 0, 0) ||
      spec_u32(sp, "mf", &a->mf, 0, 0))
    return -1;
  if (a->chunk == 0) { hb_set_error("builtin attn: chunk=0"); return -1; }
  if (spec_u32(sp, "nsplit", &a->n_split, 0, (a->max_seq + a->chunk - 1) / a->chunk)) return -1;
  if (!is_act(a->qdt) || !is_act(a->odt)) { hb_set_error("builtin attn: bad dtypes"); return -1; }
  u64 cb = (u64)(a->spec ? 1 : a->B) * a->Hkv * a->max_seq * a->hd * hb_dt_size(a->cdt);
  a->out = arg(c, 0, (u64)a->B * a->H * a->hd * hb_dt_size(a->odt));
  a->q = arg(c, 1, (u64)a->B * a->H * a->hd * hb_dt_size(a->qdt));
  a->kcache = arg(c, 2, cb);
  a->vcache = arg(c, 3, cb);
  a->len = (const int32_t *)arg(c, 4, 4);
  if (with_part)
    a->part = (float *)arg(c, 5, thvm_k_attn_part_bytes(a->B, a->H, a->Hkv, a->hd, a->n_split));
  /* clk=<blocks>: a phase-clock buffer after the others (split blocks, then
   * merge blocks: 2 x blocks x 10 u64) */
  if (with_part && a->clk_cap) a->clk = (uint64_t *)arg(c, 6, (u64)a->clk_cap * 2 * 80);
  return c->bad ? -1 : 0;
}

/* Launch (or only validate, check_only=1) a builtin program. */
int hb_builtin_launch(const char *program, const u32 *ids, u32 n, int check_only) {
  Spec sp;
  if (spec_parse(program, &sp)) return -1;
  ArgCtx c = {ids, n, sp.kernel, 0};
  char err[256] = {0};
  int rc = -1;
  u64 bytes = 0;                     /* algorithmic bytes, for kprof */
  hipEvent_t e0 = NULL, e1 = NULL;
  int prof = !check_only && hb_kprof_on();
  const char *K = sp.kernel;

#define NEED(...) do { if (__VA_ARGS__) return -1; } while (0)
  if (strcmp(K, "gemv") == 0) {
    ThvmGemvArgs a;
    memset(&a, 0, sizeof a);
    u32 bias = 0, ngain = 1, nbias = 0;
    NEED(spec_u32(&sp, "m", &a.M, 1, 0) || spec_u32(&sp, "n", &a.N, 1, 0) ||
         spec_u32(&sp, "k", &a.K, 1, 0) || spec_u32(&sp, "wt", &a.wdt, 1, 0) ||
         spec_u32(&sp, "xt", &a.xdt, 0, THVM_DT_BF16) || spec_u32(&sp, "yt", &a.ydt, 0, THVM_DT_BF16) ||
         spec_u32(&sp, "epi", &a.epi, 0, THVM_EPI_STORE) || spec_u32(&sp, "bias", &bias, 0, 0) ||
         spec_u32(&sp, "h", &a.n_heads, 0, 0) || spec_u32(&sp, "hkv", &a.n_kv_heads, 0, 0) ||
         spec_u32(&sp, "hd", &a.head_dim, 0, 0) || spec_u32(&sp, "maxseq", &a.max_seq, 0, 0) ||
         spec_u32(&sp, "norm", &a.norm, 0, 0) || spec_f32(&sp, "eps", &a.norm_eps, 0, 1e-6f) ||
         spec_u32(&sp, "ngain", &ngain, 0, 1) || spec_u32(&sp, "nbias", &nbias, 0, a.norm == 2) ||
         spec_u32(&sp, "waves", &a.tune_waves, 0, 0) || spec_u32(&sp, "r", &a.tune_r, 0, 0) ||
         spec_u32(&sp, "u", &a.tune_u, 0, 0) || spec_u32(&sp, "blocks", &a.tune_blocks, 0, 0) ||
         spec_u32(&sp, "path", &a.tune_path, 0, 0) || spec_u32(&sp, "spec", &a.spec, 0, 0) ||
         spec_u32(&sp, "tiled", &a.wtiled, 0, 0) || spec_u32(&sp, "clk", &a.clk_cap, 0, 0) ||
         spec_u32(&sp, "xqs", &a.xqs, 0, a.K));
    {
      u32 ldy0 = a.epi == THVM_EPI_SWIGLU ? a.N / 2
               : (a.epi == THVM_EPI_QKV || a.epi == THVM_EPI_QKV_ROPE) ? a.n_heads * a.head_dim
               : a.N;
      NEED(spec_u32(&sp, "ldx", &a.ldx, 0, a.K) || spec_u32(&sp, "ldy", &a.ldy, 0, ldy0));
    }
    u32 wsz = hb_dt_size(a.wdt), xsz = hb_dt_size(a.xdt), ysz = hb_dt_size(a.ydt);
    if (!wsz || !is_act(a.xdt) || !is_act(a.ydt) || a.M == 0) {
      hb_set_error("builtin gemv: bad dtypes/shape");
      return -1;
    }
    u32 ncols_out = a.epi == THVM_EPI_SWIGLU ? a.N / 2 : a.N;
    u32 slot = 0;
    int qkv = a.epi == THVM_EPI_QKV || a.epi == THVM_EPI_QKV_ROPE;
    u64 ybytes = qkv ? ((u64)(a.M - 1) * a.ldy + (u64)a.n_heads * a.head_dim) * ysz
                     : ((u64)(a.M - 1) * a.ldy + ncols_out) * ysz;
    a.y = arg(&c, slot++, ybytes);
    /* norm=3: x is four f32 vectors xqs elements apart (the MLA quarter sums) */
    a.x = arg(&c, slot++, a.norm == 3 ? (3ull * a.xqs + a.K) * 4 : ((u64)(a.M - 1) * a.ldx + a.K) * xsz);
    a.w = arg(&c, slot++, (a.wtiled ? ((u64)a.N + 15) / 16 * 16 : (u64)a.N) * a.K * wsz);
    if (a.wdt == THVM_DT_FP8E4M3) a.scale = (const float *)arg(&c, slot++, (u64)a.N * 4);
    if (a.norm && ngain) a.norm_w = (const float *)arg(&c, slot++, (u64)a.K * 4);
    if (a.norm == 2 && nbias) a.norm_b = (const float *)arg(&c, slot++, (u64)a.K * 4);
    if (bias) a.bias = arg(&c, slot++, (u64)a.N * ysz);
    if (a.epi == THVM_EPI_RESID) a.res = arg(&c, slot++, ybytes);
    if (a.epi == THVM_EPI_QKV_ROPE) {
      a.rope_cos = (const float *)arg(&c, slot++, (u64)a.max_seq * (a.head_dim / 2) * 4);
      a.rope_sin = (const float *)arg(&c, slot++, (u64)a.max_seq * (a.head_dim / 2) * 4);
    }
    if (qkv) {
      u64 cb = (u64)(a.spec ? 1 : a.M) * a.n_kv_heads * a.max_seq * a.head_dim * ysz;
      a.len = (const int32_t *)arg(&c, slot++, 4);
      a.kcache = arg(&c, slot++, cb);
      a.vcache = arg(&c, slot++, cb);
    }
    /* clk=<blocks>: a phase-clock buffer after the others (blocks x 10 u64) */
    if (a.clk_cap) a.clk = (uint64_t *)arg(&c, slot++, (u64)a.clk_cap * 80);
    if (c.bad) return -1;
    bytes = (u64)a.N * a.K * wsz + (a.scale ? (u64)a.N * 4 : 0) + (u64)a.M * a.K * (a.norm == 3 ? 16 : xsz) +
            (u64)a.M * ncols_out * ysz * (a.res ? 2 : 1);
    if (check_only) return 0;
    if (prof) hb_kprof_begin(K, &e0, &e1);
    rc = thvm_k_gemv(&a, HB_STREAM, err, sizeof err);
  } else if (strcmp(K, "tile_w") == 0) {   /* y (tiled), w (row-major) */
    u32 n = 0, k = 0, wt = 0, lb = 0;
    NEED(spec_u32(&sp, "n", &n, 1, 0) || spec_u32(&sp, "k", &k, 1, 0) || spec_u32(&sp, "wt", &wt, 1, 0) ||
         spec_u32(&sp, "lb", &lb, 0, 0));
    const u32 es = hb_dt_size(wt);
    if (es != 1 && es != 2) { hb_set_error("builtin tile_w: wt must be a 1- or 2-byte type"); return -1; }
    void *y = arg(&c, 0, ((u64)n + 15) / 16 * 16 * k * es);
    const void *w = arg(&c, 1, (u64)n * k * es);
    if (c.bad) return -1;
    bytes = (u64)n * k * es * 2;
    if (check_only) return 0;
    if (prof) hb_kprof_begin(K, &e0, &e1);
    rc = thvm_k_tile_w(y, w, n, k, es, lb, HB_STREAM, err, sizeof err);
  } else if (strcmp(K, "norm") == 0) {
    ThvmNormArgs a;
    memset(&a, 0, sizeof a);
    u32 gain = 1, has_b = 0, ln = 0;
    NEED(spec_u32(&sp, "m", &a.M, 1, 0) || spec_u32(&sp, "k", &a.K, 1, 0) ||
         spec_u32(&sp, "xt", &a.xdt, 0, THVM_DT_BF16) || spec_u32(&sp, "yt", &a.ydt, 0, THVM_DT_BF16) ||
         spec_f32(&sp, "eps", &a.eps, 0, 1e-6f) || spec_u32(&sp, "ln", &ln, 0, 0) ||
         spec_u32(&sp, "gain", &gain, 0, 1) || spec_u32(&sp, "bias", &has_b, 0, 0));
    NEED(spec_u32(&sp, "ldx", &a.ldx, 0, a.K) || spec_u32(&sp, "ldy", &a.ldy, 0, a.K));
    a.layernorm = (int)ln;
    u32 xsz = hb_dt_size(a.xdt), ysz = hb_dt_size(a.ydt);
    if (!is_act(a.xdt) || !is_act(a.ydt) || a.M == 0) { hb_set_error("builtin norm: bad dtypes"); return -1; }
    a.y = arg(&c, 0, ((u64)(a.M - 1) * a.ldy + a.K) * ysz);
    a.x = arg(&c, 1, ((u64)(a.M - 1) * a.ldx + a.K) * xsz);
    u32 slot = 2;
    if (gain) a.w = (const float *)arg(&c, slot++, (u64)a.K * 4);
    if (has_b) a.b = (const float *)arg(&c, slot++, (u64)a.K * 4);
    if (c.bad) return -1;
    bytes = (u64)a.M * a.K * (xsz + ysz) + (gain ? (u64)a.K * 4 : 0);
    if (check_only) return 0;
    if (prof) hb_kprof_begin(K, &e0, &e1);
    rc = thvm_k_norm(&a, HB_STREAM, err, sizeof err);
  } else if (strcmp(K, "softmax") == 0) {
    ThvmSoftmaxArgs a;
    memset(&a, 0, sizeof a);
    NEED(spec_u32(&sp, "m", &a.M, 1, 0) || spec_u32(&sp, "k", &a.K, 1, 0) ||
         spec_u32(&sp, "xt", &a.xdt, 0, THVM_DT_FP32) || spec_u32(&sp, "yt", &a.ydt, 0, THVM_DT_FP32));
    if (!is_act(a.xdt) || !is_act(a.ydt)) { hb_set_error("builtin softmax: bad dtypes"); return -1; }
    u64 ne = (u64)a.M * a.K;
    a.y = arg(&c, 0, ne * hb_dt_size(a.ydt));
    a.x = arg(&c, 1, ne * hb_dt_size(a.xdt));
    if (c.bad) return -1;
    bytes = ne * (hb_dt_size(a.xdt) + hb_dt_size(a.ydt));
    if (check_only) return 0;
    if (prof) hb_kprof_begin(K, &e0, &e1);
    rc = thvm_k_softmax(&a, HB_STREAM, err, sizeof err);
  } else if (strcmp(K, "attn") == 0) {
    ThvmAttnArgs a;
    NEED(attn_parse(&sp, &c, &a, 1));
    bytes = 0; /* live-length dependent: the decoder accounts for it */
    if (check_only) return 0;
    if (prof) hb_kprof_begin(K, &e0, &e1);
    rc = thvm_k_attn_decode(&a, HB_STREAM, err, sizeof err);
  } else if (strcmp(K, "mla_prep") == 0 || strcmp(K, "mla_attn") == 0) {
    ThvmMlaArgs a;
    memset(&a, 0, sizeof a);
    const int prep = strcmp(K, "mla_prep") == 0;
    NEED(spec_u32(&sp, "b", &a.B, 1, 0) || spec_u32(&sp, "h", &a.H, 1, 0) ||
         spec_u32(&sp, "dn", &a.dn, 1, 0) || spec_u32(&sp, "dr", &a.dr, 1, 0) ||
         spec_u32(&sp, "kv", &a.kv, 1, 0) || spec_u32(&sp, "dv", &a.dv, 1, 0) ||
         spec_u32(&sp, "maxseq", &a.max_seq, 1, 0) || spec_u32(&sp, "wt", &a.wdt, 0, THVM_DT_FP8E4M3) ||
         spec_f32(&sp, "eps", &a.eps, 0, 1e-6f) || spec_f32(&sp, "scale", &a.scale, !prep, 0));
    NEED(spec_u32(&sp, "ldq", &a.ldq, 0, a.H * (a.dn + a.dr) + a.kv + a.dr) ||
         spec_u32(&sp, "nsplit", &a.n_split, 0, (a.max_seq + 63) / 64) ||
         spec_u32(&sp, "mode", &a.mode, 0, 0) || spec_u32(&sp, "cpb", &a.cpb, 0, 0) ||
         spec_u32(&sp, "clk", &a.clk_cap, 0, 0) || spec_u32(&sp, "oq", &a.oq, 0, 0));
    const u32 wsz = hb_dt_size(a.wdt);
    const int fp8 = a.wdt == THVM_DT_FP8E4M3;
    if (!wsz) { hb_set_error("builtin %s: bad weight dtype", K); return -1; }
    const u64 ckvb = (u64)a.B * a.max_seq * a.kv * 2, kpeb = (u64)a.B * a.max_seq * a.dr * 2;
    u32 slot = 0;
    if (prep) {
      a.qkv = arg(&c, slot++, (u64)a.B * a.ldq * 2);
      a.wuk = arg(&c, slot++, (u64)a.H * a.kv * a.dn * wsz);
      if (fp8) a.suk = (const float *)arg(&c, slot++, (u64)a.H * a.kv * 4);
      a.wkvn = (const float *)arg(&c, slot++, (u64)a.kv * 4);
      a.rope_cos = (const float *)arg(&c, slot++, (u64)a.max_seq * (a.dr / 2) * 4);
      a.rope_sin = (const float *)arg(&c, slot++, (u64)a.max_seq * (a.dr / 2) * 4);
      a.len = (const int32_t *)arg(&c, slot++, 4);
      a.ckv = arg(&c, slot++, ckvb);
      a.kpe = arg(&c, slot++, kpeb);
      a.qlat = (float *)arg(&c, slot++, (u64)a.B * a.H * a.kv * 4);
      a.qpe = arg(&c, slot++, (u64)a.B * a.H * a.dr * 2);
      bytes = (u64)a.H * a.kv * a.dn * wsz + (u64)a.B * a.ldq * 2;
    } else {
      /* oq=1: the four f32 quarter sums of the latent-quarter merge */
      a.o = arg(&c, slot++, (u64)a.B * a.H * a.dv * (a.oq ? 16 : 2));
      a.qlat = (float *)arg(&c, slot++, (u64)a.B * a.H * a.kv * 4);
      a.qpe = arg(&c, slot++, (u64)a.B * a.H * a.dr * 2);
      a.ckv = arg(&c, slot++, ckvb);
      a.kpe = arg(&c, slot++, kpeb);
      a.len = (const int32_t *)arg(&c, slot++, 4);
      a.part = (float *)arg(&c, slot++, thvm_k_mla_part_bytes(a.B, a.H, a.kv, a.n_split));
      a.wuv = arg(&c, slot++, (u64)a.H * a.dv * a.kv * wsz);
      if (fp8) a.suv = (const float *)arg(&c, slot++, (u64)a.H * a.dv * 4);
      bytes = 0; /* live-length dependent: the decoder accounts for it */
    }
    /* clk=<blocks>: a phase-clock buffer after the others (mla_attn: split
     * blocks, then merge blocks) */
    if (a.clk_cap) a.clk = (uint64_t *)arg(&c, slot++, (u64)a.clk_cap * (prep ? 1 : 2) * 80);
    if (c.bad) return -1;
    if (check_only) return 0;
    if (prof) hb_kprof_begin(K, &e0, &e1);
    rc = prep ? thvm_k_mla_prep(&a, HB_STREAM, err, sizeof err)
              : thvm_k_mla_attn(&a, HB_STREAM, err, sizeof err);
  } else if (strcmp(K, "route") == 0) {
    ThvmRouteArgs a;
    memset(&a, 0, sizeof a);
    NEED(spec_u32(&sp, "b", &a.B, 1, 0) || spec_u32(&sp, "e", &a.E, 1, 0) ||
         spec_u32(&sp, "k", &a.K, 1, 0));
    a.sel = (int32_t *)arg(&c, 0, (u64)a.B * a.K * 4);
    a.probs = (float *)arg(&c, 1, (u64)a.B * a.K * 4);
    a.logits = (const float *)arg(&c, 2, (u64)a.B * a.E * 4);
    if (c.bad) return -1;
    bytes = (u64)a.B * (a.E * 4 + a.K * 8);
    if (check_only) return 0;
    if (prof) hb_kprof_begin(K, &e0, &e1);
    rc = thvm_k_route(&a, HB_STREAM, err, sizeof err);
  } else if (strcmp(K, "moe_gate") == 0) {   /* xn, logits, x, gain, gate */
    ThvmGateArgs a;
    memset(&a, 0, sizeof a);
    NEED(spec_u32(&sp, "b", &a.B, 1, 0) || spec_u32(&sp, "d", &a.D, 1, 0) ||
         spec_u32(&sp, "e", &a.E, 1, 0) || spec_f32(&sp, "eps", &a.eps, 0, 1e-6f) ||
         spec_u32(&sp, "clk", &a.clk_cap, 0, 0));
    a.xn = (float *)arg(&c, 0, (u64)a.B * a.D * 4);
    a.logits = (float *)arg(&c, 1, (u64)a.B * a.E * 4);
    a.x = arg(&c, 2, (u64)a.B * a.D * 2);
    a.w = (const float *)arg(&c, 3, (u64)a.D * 4);
    a.gate = (const float *)arg(&c, 4, (u64)a.E * a.D * 4);
    if (a.clk_cap) a.clk = (uint64_t *)arg(&c, 5, (u64)a.clk_cap * 80);
    if (c.bad) return -1;
    bytes = (u64)a.E * a.D * 4 + (u64)a.B * a.D * 6 + (u64)a.B * a.E * 4;
    if (check_only) return 0;
    if (prof) hb_kprof_begin(K, &e0, &e1);
    rc = thvm_k_moe_gate(&a, HB_STREAM, err, sizeof err);
  } else if (strcmp(K, "moe_gateup") == 0 || strcmp(K, "moe_down") == 0) {
    ThvmMoeArgs a;
    memset(&a, 0, sizeof a);
    const int gu = strcmp(K, "moe_gateup") == 0;
    u32 route = 0;
    NEED(spec_u32(&sp, "b", &a.B, 1, 0) || spec_u32(&sp, "d", &a.D, 1, 0) ||
         spec_u32(&sp, "e", &a.E, 1, 0) || spec_u32(&sp, "k", &a.K, 1, 0) ||
         spec_u32(&sp, "i", &a.I, 1, 0) || spec_u32(&sp, "s", &a.S, 0, 0) ||
         spec_u32(&sp, "wt", &a.wdt, 0, THVM_DT_FP8E4M3) || spec_u32(&sp, "grouped", &a.grouped, 0, 0) ||
         spec_u32(&sp, "route", &route, 0, 0) || spec_u32(&sp, "tiled", &a.wtiled, 0, 0) ||
         spec_u32(&sp, "clk", &a.clk_cap, 0, 0));
    if (route && !gu) { hb_set_error("builtin moe_down: route=1 is a gate/up key"); return -1; }
    const u32 wsz = hb_dt_size(a.wdt);
    const int fp8 = a.wdt == THVM_DT_FP8E4M3;
    if (!wsz) { hb_set_error("builtin %s: bad weight dtype", K); return -1; }
    const u64 hb = (u64)a.B * (a.K * a.I + a.S) * 4;
    u32 slot = 0;
    if (gu) {
      a.h = (float *)arg(&c, slot++, hb);
      a.x = (const float *)arg(&c, slot++, (u64)a.B * a.D * 4);
      /* route=1: this slot receives the picked experts; logits and probs
       * come last */
      a.sel = (const int32_t *)arg(&c, slot++, (u64)a.B * a.K * 4);
      a.wgu_e = arg(&c, slot++, (u64)a.E * 2 * a.I * a.D * wsz);
      if (fp8) a.sgu_e = (const float *)arg(&c, slot++, (u64)a.E * 2 * a.I * 4);
      if (a.S) {
        a.wgu_s = arg(&c, slot++, (u64)2 * a.S * a.D * wsz);
        if (fp8) a.sgu_s = (const float *)arg(&c, slot++, (u64)2 * a.S * 4);
      }
      bytes = (u64)a.B * ((u64)a.K * 2 * a.I + 2 * a.S) * a.D * wsz + hb;
      if (a.grouped) {   /* plan scratch, then the live-expert counter it adds to */
        a.plan = (int32_t *)arg(&c, slot++, thvm_k_moe_plan_bytes(a.B, a.E, a.K));
        a.live = (int32_t *)arg(&c, slot++, 4);
        bytes = 0;       /* the experts streamed are known on the device only (live) */
      }
      if (route) {
        a.logits = (const float *)arg(&c, slot++, (u64)a.B * a.E * 4);
        a.probs_out = (float *)arg(&c, slot++, (u64)a.B * a.K * 4);
        a.sel_out = (int32_t *)a.sel;
      }
    } else {
      a.res = arg(&c, slot++, (u64)a.B * a.D * 2);
      a.h = (float *)arg(&c, slot++, hb);
      a.sel = (const int32_t *)arg(&c, slot++, (u64)a.B * a.K * 4);
      a.probs = (const float *)arg(&c, slot++, (u64)a.B * a.K * 4);
      a.wd_e = arg(&c, slot++, (u64)a.E * a.D * a.I * wsz);
      if (fp8) a.sd_e = (const float *)arg(&c, slot++, (u64)a.E * a.D * 4);
      if (a.S) {
        a.wd_s = arg(&c, slot++, (u64)a.D * a.S * wsz);
        if (fp8) a.sd_s = (const float *)arg(&c, slot++, (u64)a.D * 4);
      }
      bytes = (u64)a.B * ((u64)a.K * a.I + a.S) * a.D * wsz + hb + (u64)a.B * a.D * 4;
      if (a.grouped) {   /* the gate/up's plan, then the per-slot down outputs */
        a.plan = (int32_t *)arg(&c, slot++, thvm_k_moe_plan_bytes(a.B, a.E, a.K));
        a.part = (float *)arg(&c, slot++, thvm_k_moe_part_bytes(a.B, a.K, a.D));
        bytes = 0;
      }
    }
    if (a.clk_cap) a.clk = (uint64_t *)arg(&c, slot++, (u64)a.clk_cap * 80);
    if (c.bad) return -1;
    if (check_only) return 0;
    if (prof) hb_kprof_begin(K, &e0, &e1);
    rc = gu ? thvm_k_moe_gateup(&a, HB_STREAM, err, sizeof err)
            : thvm_k_moe_down(&a, HB_STREAM, err, sizeof err);
  } else if (strcmp(K, "embed") == 0) {
    ThvmEmbedArgs a;
    memset(&a, 0, sizeof a);
    u32 pos = 0;
    NEED(spec_u32(&sp, "b", &a.B, 1, 0) || spec_u32(&sp, "d", &a.D, 1, 0) ||
         spec_u32(&sp, "v", &a.V, 1, 0) || spec_u32(&sp, "et", &a.edt, 0, THVM_DT_BF16) ||
         spec_u32(&sp, "xt", &a.xdt, 0, THVM_DT_BF16) || spec_u32(&sp, "pos", &pos, 0, 0) ||
         spec_u32(&sp, "maxseq", &a.max_seq, 0, 0));
    if (!is_act(a.edt) || !is_act(a.xdt)) { hb_set_error("builtin embed: bad dtypes"); return -1; }
    a.x = arg(&c, 0, (u64)a.B * a.D * hb_dt_size(a.xdt));
    a.emb = arg(&c, 1, (u64)a.V * a.D * hb_dt_size(a.edt));
    a.tok = (const int32_t *)arg(&c, 2, (u64)a.B * 4);
    if (pos) {
      if (a.max_seq == 0) { hb_set_error("builtin embed: pos=1 needs maxseq"); return -1; }
      a.pos_emb = arg(&c, 3, (u64)a.max_seq * a.D * hb_dt_size(a.edt));
      a.len = (const int32_t *)arg(&c, 4, 4);
    }
    if (c.bad) return -1;
    bytes = (u64)a.B * a.D * (hb_dt_size(a.edt) * (pos ? 2 : 1) + hb_dt_size(a.xdt));
    if (check_only) return 0;
    if (prof) hb_kprof_begin(K, &e0, &e1);
    rc = thvm_k_embed(&a, HB_STREAM, err, sizeof err);
  } else if (strcmp(K, "argmax") == 0) {
    ThvmArgmaxArgs a;
    memset(&a, 0, sizeof a);
    u32 hist = 0;
    float temp = 0.0f;
    NEED(spec_u32(&sp, "b", &a.B, 1, 0) || spec_u32(&sp, "v", &a.V, 1, 0) ||
         spec_u32(&sp, "nb", &a.nb, 0, 256) || spec_u32(&sp, "hist", &hist, 0, 0) ||
         spec_u32(&sp, "hstride", &a.hist_stride, 0, 0) || spec_f32(&sp, "temp", &temp, 0, 0.0f) ||
         spec_u64(&sp, "seed", &a.seed, 0, 0));
    if (!(temp >= 0.0f) || temp > 1e30f) { hb_set_error("builtin argmax: temp must be >= 0"); return -1; }
    a.inv_temp = temp > 0.0f ? 1.0f / temp : 0.0f;
    if (a.nb > a.V) a.nb = a.V;
    a.tok = (int32_t *)arg(&c, 0, (u64)a.B * 4);
    a.logits = (const float *)arg(&c, 1, (u64)a.B * a.V * 4);
    a.pv = (float *)arg(&c, 2, (u64)a.B * a.nb * 4);
    a.pi = (int32_t *)arg(&c, 3, (u64)a.B * a.nb * 4);
    if (hist) {
      if (a.hist_stride == 0) { hb_set_error("builtin argmax: hist=1 needs hstride"); return -1; }
      a.hist = (int32_t *)arg(&c, 4, (u64)a.B * a.hist_stride * 4);
      a.len = (const int32_t *)arg(&c, 5, 4);
    } else if (temp > 0.0f) {       /* sampling keys its draw on the position */
      a.len = (const int32_t *)arg(&c, 4, 4);
    }
    if (c.bad) return -1;
    bytes = (u64)a.B * a.V * 4;
    if (check_only) return 0;
    if (prof) hb_kprof_begin(K, &e0, &e1);
    rc = thvm_k_argmax(&a, HB_STREAM, err, sizeof err);
  } else if (strcmp(K, "quant_fp8") == 0) {   /* q, scale, x */
    u32 rows = 0, cols = 0, xdt = 0;
    NEED(spec_u32(&sp, "rows", &rows, 1, 0) || spec_u32(&sp, "cols", &cols, 1, 0) ||
         spec_u32(&sp, "xt", &xdt, 1, 0));
    if (!is_act(xdt)) { hb_set_error("builtin quant_fp8: xt must be f32 / bf16 / fp16"); return -1; }
    uint8_t *q = (uint8_t *)arg(&c, 0, (u64)rows * cols);
    float *scale = (float *)arg(&c, 1, (u64)rows * 4);
    const void *x = arg(&c, 2, (u64)rows * cols * hb_dt_size(xdt));
    if (c.bad) return -1;
    bytes = (u64)rows * cols * (1 + hb_dt_size(xdt)) + (u64)rows * 4;
    if (check_only) return 0;
    if (prof) hb_kprof_begin(K, &e0, &e1);
    rc = thvm_k_quant_fp8_rows(q, scale, x, xdt, rows, cols, HB_STREAM, err, sizeof err);
  } else if (strcmp(K, "spec_draft") == 0) {   /* cand_acc, cand_emb, hist, len */
    u32 S = 0, V = 0, hcap = 0, forced = 0;
    NEED(spec_u32(&sp, "s", &S, 1, 0) || spec_u32(&sp, "v", &V, 1, 0) ||
         spec_u32(&sp, "hcap", &hcap, 1, 0) || spec_u32(&sp, "forced", &forced, 0, 0));
    int32_t *ca = (int32_t *)arg(&c, 0, (u64)S * 4), *ce = (int32_t *)arg(&c, 1, (u64)S * 4);
    const int32_t *hist = (const int32_t *)arg(&c, 2, (u64)hcap * 4);
    const int32_t *L = (const int32_t *)arg(&c, 3, 4);
    if (c.bad) return -1;
    bytes = (u64)hcap * 4;
    if (check_only) return 0;
    if (prof) hb_kprof_begin(K, &e0, &e1);
    rc = thvm_k_spec_draft(ca, ce, hist, L, S, V, hcap, forced, HB_STREAM, err, sizeof err);
  } else if (strcmp(K, "spec_accept") == 0) {  /* hist, len, cand_acc, am [, tok] */
    u32 S = 0, hcap = 0;
    NEED(spec_u32(&sp, "s", &S, 1, 0) || spec_u32(&sp, "hcap", &hcap, 1, 0));
    int32_t *hist = (int32_t *)arg(&c, 0, (u64)hcap * 4);
    int32_t *L = (int32_t *)arg(&c, 1, 4);
    const int32_t *ca = (const int32_t *)arg(&c, 2, (u64)S * 4);
    const int32_t *am = (const int32_t *)arg(&c, 3, (u64)S * 4);
    int32_t *tok = n > 4 ? (int32_t *)arg(&c, 4, 4) : NULL;
    if (c.bad) return -1;
    bytes = (u64)S * 12;
    if (check_only) return 0;
    if (prof) hb_kprof_begin(K, &e0, &e1);
    rc = thvm_k_spec_accept(hist, L, tok, ca, am, S, hcap, HB_STREAM, err, sizeof err);
  } else if (strcmp(K, "len_bump") == 0) {
    u32 d = 1;
    NEED(spec_u32(&sp, "delta", &d, 0, 1));
    int32_t *L = (int32_t *)arg(&c, 0, 4);
    if (c.bad) return -1;
    if (check_only) return 0;
    if (prof) hb_kprof_begin(K, &e0, &e1);
    rc = thvm_k_len_bump(L, (int32_t)d, HB_STREAM, err, sizeof err);
  } else if (strcmp(K, "touch") == 0) {   /* read a range into the caches */
    u64 nb = 0;
    u32 nsink = 0;
    NEED(spec_u64(&sp, "n", &nb, 1, 0) || spec_u32(&sp, "blocks", &nsink, 0, 1024));
    const void *x = arg(&c, 0, nb);
    uint32_t *sink = (uint32_t *)arg(&c, 1, (u64)nsink * 4);
    if (c.bad) return -1;
    bytes = nb;
    if (check_only) return 0;
    if (prof) hb_kprof_begin(K, &e0, &e1);
    rc = thvm_k_touch(x, nb, sink, nsink, HB_STREAM, err, sizeof err);
  } else if (strcmp(K, "delay") == 0) {
    u32 nper = 0;
    NEED(spec_u32(&sp, "n", &nper, 1, 0));
    if (!arg(&c, 0, 0)) return -1;      /* the ABI needs one argument slot */
    if (check_only) return 0;
    rc = thvm_k_delay(nper, HB_STREAM, err, sizeof err);
  } else if (strcmp(K, "rope") == 0) {
    ThvmRopeArgs a;
    memset(&a, 0, sizeof a);
    u32 maxseq = 0;
    NEED(spec_u32(&sp, "b", &a.B, 1, 0) || spec_u32(&sp, "nh", &a.nh, 1, 0) ||
         spec_u32(&sp, "hd", &a.hd, 1, 0) || spec_u32(&sp, "dt", &a.dt, 0, THVM_DT_BF16) ||
         spec_u32(&sp, "maxseq", &maxseq, 1, 0));
    a.max_seq = maxseq;
    if (!is_act(a.dt)) { hb_set_error("builtin rope: bad dtype"); return -1; }
    a.x = arg(&c, 0, (u64)a.B * a.nh * a.hd * hb_dt_size(a.dt));
    a.cos_t = (const float *)arg(&c, 1, (u64)maxseq * (a.hd / 2) * 4);
    a.sin_t = (const float *)arg(&c, 2, (u64)maxseq * (a.hd / 2) * 4);
    a.len = (const int32_t *)arg(&c, 3, 4);
    if (c.bad) return -1;
    if (check_only) return 0;
    if (prof) hb_kprof_begin(K, &e0, &e1);
    rc = thvm_k_rope(&a, HB_STREAM, err, sizeof err);
  } else if (strcmp(K, "llama_step") == 0) {
    /* the persistent LLAMA decode step; slot 0 is the per-layer table of
     * device pointers (ThvmStepLayer[l]), built by its owner from live
     * buffers, the other slots are checked against the shapes here */
    ThvmStepArgs a;
    memset(&a, 0, sizeof a);
    NEED(spec_u32(&sp, "l", &a.n_layers, 1, 0) || spec_u32(&sp, "m", &a.M, 1, 0) ||
         spec_u32(&sp, "d", &a.D, 1, 0) || spec_u32(&sp, "h", &a.H, 1, 0) ||
         spec_u32(&sp, "hkv", &a.Hkv, 1, 0) || spec_u32(&sp, "hd", &a.hd, 1, 0) ||
         spec_u32(&sp, "f", &a.F, 1, 0) || spec_u32(&sp, "v", &a.V, 1, 0) ||
         spec_u32(&sp, "maxseq", &a.max_seq, 1, 0) || spec_u32(&sp, "wt", &a.wdt, 1, 0) ||
         spec_u32(&sp, "at", &a.adt, 0, THVM_DT_BF16) || spec_f32(&sp, "eps", &a.eps, 1, 0) ||
         spec_f32(&sp, "scale", &a.attn_scale, 1, 0) || spec_u32(&sp, "hstride", &a.hist_stride, 1, 0));
    NEED(spec_u32(&sp, "nsplit", &a.n_split, 0, (a.max_seq + 63) / 64));
    const u32 wsz = hb_dt_size(a.wdt), as = hb_dt_size(a.adt), nb = thvm_k_step_blocks();
    const int fp8 = a.wdt == THVM_DT_FP8E4M3;
    if (!wsz || !is_act(a.adt) || !nb) { hb_set_error("builtin llama_step: bad dtypes or no device"); return -1; }
    const u64 hq = (u64)a.H * a.hd;
    u32 slot = 0;
    a.layers = (const ThvmStepLayer *)arg(&c, slot++, (u64)a.n_layers * sizeof(ThvmStepLayer));
    a.emb = arg(&c, slot++, (u64)a.V * a.D * as);
    a.norm_f = (const float *)arg(&c, slot++, (u64)a.D * 4);
    a.lm = arg(&c, slot++, (u64)a.V * a.D * wsz);
    if (fp8) a.slm = (const float *)arg(&c, slot++, (u64)a.V * 4);
    a.rope_cos = (const float *)arg(&c, slot++, (u64)a.max_seq * (a.hd / 2) * 4);
    a.rope_sin = (const float *)arg(&c, slot++, (u64)a.max_seq * (a.hd / 2) * 4);
    a.tok = (int32_t *)arg(&c, slot++, (u64)a.M * 4);
    a.len = (int32_t *)arg(&c, slot++, 4);
    a.hist = (int32_t *)arg(&c, slot++, (u64)a.M * a.hist_stride * 4);
    a.logits = (float *)arg(&c, slot++, (u64)a.M * a.V * 4);
    a.x = arg(&c, slot++, (u64)a.M * a.D * as);
    a.q = arg(&c, slot++, (u64)a.M * hq * as);
    a.att = arg(&c, slot++, (u64)a.M * hq * as);
    a.h = arg(&c, slot++, (u64)a.M * a.F * as);
    a.part = (float *)arg(&c, slot++, thvm_k_attn_part_bytes(a.M, a.H, a.Hkv, a.hd, a.n_split));
    a.am_pv = (float *)arg(&c, slot++, (u64)a.M * nb * 4);
    a.am_pi = (int32_t *)arg(&c, slot++, (u64)a.M * nb * 4);
    a.sync = (uint32_t *)arg(&c, slot++, thvm_k_step_sync_bytes());
    if (c.bad) return -1;
    {
      /* weight (+ row scale) bytes per step: qkv, o, gate/up, down, LM head;
       * the live KV rows are added by the caller, which knows L */
      const u64 nqkv = (u64)(a.H + 2 * a.Hkv) * a.hd;
      const u64 elems = nqkv * a.D + (u64)a.D * hq + 2ull * a.F * a.D + (u64)a.D * a.F;
      const u64 rows = nqkv + a.D + 2ull * a.F + a.D;
      bytes = (u64)a.n_layers * (elems * wsz + (fp8 ? rows * 4 : 0)) + (u64)a.V * a.D * wsz +
              (fp8 ? (u64)a.V * 4 : 0);
    }
    if (thvm_k_llama_step_check(&a, err, sizeof err)) { hb_set_error("builtin llama_step: %s", err); return -1; }
    if (check_only) return 0;
    if (prof) hb_kprof_begin(K, &e0, &e1);
    rc = thvm_k_llama_step(&a, HB_STREAM, err, sizeof err);
  } else if (strcmp(K, "cast") == 0) {
    u64 ne = 0;
    u32 xt = 0, yt = 0;
    NEED(spec_u64(&sp, "n", &ne, 1, 0) || spec_u32(&sp, "xt", &xt, 1, 0) || spec_u32(&sp, "yt", &yt, 1, 0));
    if (!hb_dt_size(xt) || !hb_dt_size(yt)) { hb_set_error("builtin cast: bad dtypes"); return -1; }
    void *y = arg(&c, 0, ne * hb_dt_size(yt));
    void *x = arg(&c, 1, ne * hb_dt_size(xt));
    if (c.bad) return -1;
    if (check_only) return 0;
    if (prof) hb_kprof_begin(K, &e0, &e1);
    rc = thvm_k_cast(y, yt, x, xt, ne, HB_STREAM, err, sizeof err);
  } else if (strcmp(K, "copy") == 0) {
    u64 nb = 0;
    NEED(spec_u64(&sp, "n", &nb, 1, 0));
    void *y = arg(&c, 0, nb);
    const void *x = arg(&c, 1, nb);
    if (c.bad) return -1;
    bytes = 2 * nb;
    if (check_only) return 0;
    if (prof) hb_kprof_begin(K, &e0, &e1);
    rc = thvm_k_copy(y, x, nb, HB_STREAM, err, sizeof err);
  } else if (strcmp(K, "fill_normal") == 0) {
    u64 ne = 0, seed = 0, tag = 0;
    u32 dt = 0;
    float mean = 0, std = 1;
    NEED(spec_u64(&sp, "n", &ne, 1, 0) || spec_u32(&sp, "dt", &dt, 1, 0) ||
         spec_u64(&sp, "seed", &seed, 0, 0) || spec_u64(&sp, "tag", &tag, 0, 0) ||
         spec_f32(&sp, "mean", &mean, 0, 0.0f) || spec_f32(&sp, "std", &std, 0, 1.0f));
    void *y = arg(&c, 0, ne * hb_dt_size(dt));
    if (c.bad) return -1;
    if (check_only) return 0;
    rc = thvm_k_fill_normal(y, dt, ne, seed, tag, mean, std, HB_STREAM, err, sizeof err);
  } else if (strcmp(K, "fill_fp8") == 0) {
    u32 rows = 0, cols = 0;
    u64 seed = 0, tag = 0;
    float std = 0.02f;
    NEED(spec_u32(&sp, "rows", &rows, 1, 0) || spec_u32(&sp, "cols", &cols, 1, 0) ||
         spec_u64(&sp, "seed", &seed, 0, 0) || spec_u64(&sp, "tag", &tag, 0, 0) ||
         spec_f32(&sp, "std", &std, 0, 0.02f));
    uint8_t *q = (uint8_t *)arg(&c, 0, (u64)rows * cols);
    float *scl = (float *)arg(&c, 1, (u64)rows * 4);
    if (c.bad) return -1;
    if (check_only) return 0;
    rc = thvm_k_fill_fp8_rows(q, scl, rows, cols, seed, tag, std, HB_STREAM, err, sizeof err);
  } else {
    hb_set_error("builtin: unknown kernel '%s'", K);
    return -1;
  }
#undef NEED
  if (rc != 0) {
    if (prof) thvm_k_time_next(NULL, NULL);
    hb_set_error("builtin %s: %s", K, err);
    return -1;
  }
  if (prof) hb_kprof_end(K, e0, e1, bytes);
  return 0;
}

/* ======================= hiprtc programs =============================== */

typedef struct {
  u64 key;
  hipModule_t mod;
  hipFunction_t fn;
} RtcEntry;
static RtcEntry *RTC = NULL;
static u32 RTC_N = 0, RTC_CAP = 0;

static const char *cache_dir(void) {
  static char dir[512];
  const char *e = getenv("THVM_HIP_CACHE_DIR");
  if (e && e[0]) return e;
  const char *home = getenv("HOME");
  snprintf(dir, sizeof dir, "%s/.cache/thvm/hip_co", home ? home : "/tmp");
  return dir;
}

static void mkdirs(const char *path) {
  char tmp[512];
  snprintf(tmp, sizeof tmp, "%s", path);
  for (char *p = tmp + 1; *p; p++) {
    if (*p == '/') { *p = 0; mkdir(tmp, 0755); *p = '/'; }
  }
  mkdir(tmp, 0755);
}

static void *read_file(const char *path, size_t *n) {
  FILE *f = fopen(path, "rb");
  if (!f) return NULL;
  fseek(f, 0, SEEK_END);
  long sz = ftell(f);
  fseek(f, 0, SEEK_SET);
  void *buf = sz > 0 ? malloc((size_t)sz) : NULL;
  if (buf && fread(buf, 1, (size_t)sz, f) != (size_t)sz) { free(buf); buf = NULL; }
  fclose(f);
  *n = buf ? (size_t)sz : 0;
  return buf;
}

static hipFunction_t rtc_get(const char *name, const char *source) {
  /* packed FP32 instructions stay off in runtime-compiled code too (as in
   * the library's own build): part of the code object's key */
  static const char *opts[] = {"--offload-arch=gfx950", "-O3", "-std=c++17", "-Xclang",
                               "-target-feature", "-Xclang", "-packed-fp32-ops"};
  u64 key = hb_hash64(source, strlen(source), 0x70667033ull);
  key = hb_hash64(name, strlen(name), key ^ 0x5bd1e995ull);
  for (u32 i = 0; i < RTC_N; i++)
    if (RTC[i].key == key) return RTC[i].fn;

  char path[640];
  snprintf(path, sizeof path, "%s/%016llx.co", cache_dir(), (unsigned long long)key);
  size_t co_n = 0;
  void *co = NULL;
  const char *nocache = getenv("THVM_HIP_NO_DISK_CACHE");
  if (!(nocache && nocache[0] == '1')) co = read_file(path, &co_n);
  if (!co) {
    hiprtcProgram prog;
    hiprtcResult r = hiprtcCreateProgram(&prog, source, name, 0, NULL, NULL);
    if (r != HIPRTC_SUCCESS) { hb_set_error("hiprtcCreateProgram(%s): %s", name, hiprtcGetErrorString(r)); return NULL; }
    r = hiprtcCompileProgram(prog, (int)(sizeof opts / sizeof opts[0]), opts);
    if (r != HIPRTC_SUCCESS) {
      size_t ln = 0;
      hiprtcGetProgramLogSize(prog, &ln);
      char *log = (char *)malloc(ln + 1);
      if (log) { hiprtcGetProgramLog(prog, log); log[ln] = 0; }
      hb_set_error("hiprtc compile of %s failed: %.400s", name, log ? log : "");
      free(log);
      hiprtcDestroyProgram(&prog);
      return NULL;
    }
    hiprtcGetCodeSize(prog, &co_n);
    co = malloc(co_n);
    if (!co) { hiprtcDestroyProgram(&prog); hb_set_error("hiprtc: out of memory"); return NULL; }
    hiprtcGetCode(prog, (char *)co);
    hiprtcDestroyProgram(&prog);
    if (!(nocache && nocache[0] == '1')) {
      mkdirs(cache_dir());
      char tmp[700];
      snprintf(tmp, sizeof tmp, "%s.%d.tmp", path, (int)getpid());
      FILE *f = fopen(tmp, "wb");
      if (f) {
        int ok = fwrite(co, 1, co_n, f) == co_n;
        fclose(f);
        if (ok) rename(tmp, path); else unlink(tmp);
      }
    }
  }
  hipModule_t mod;
  hipError_t e = hipModuleLoadData(&mod, co);
  free(co);
  if (e != hipSuccess) {
    (void)hipGetLastError();   /* handled here: do not leave it for the next launch check */
    hb_set_error("hipModuleLoadData(%s): %s", name, hipGetErrorString(e));
    return NULL;
  }
  hipFunction_t fn;
  e = hipModuleGetFunction(&fn, mod, name);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    hipModuleUnload(mod);
    hb_set_error("hipModuleGetFunction(%s): %s", name, hipGetErrorString(e));
    return NULL;
  }
  if (RTC_N == RTC_CAP) {
    RTC_CAP = RTC_CAP ? 2 * RTC_CAP : 64;
    RTC = (RtcEntry *)realloc(RTC, RTC_CAP * sizeof(RtcEntry));
  }
  RTC[RTC_N].key = key;
  RTC[RTC_N].mod = mod;
  RTC[RTC_N].fn = fn;
  RTC_N++;
  return fn;
}

void hb_rtc_reset(void) {
  for (u32 i = 0; i < RTC_N; i++) hipModuleUnload(RTC[i].mod);
  free(RTC);
  RTC = NULL;
  RTC_N = RTC_CAP = 0;
}

int hb_rtc_launch(const char *name, const char *source, const u32 grid[3], const u32 block[3],
                  u32 shared, const u32 *ids, u32 n, int check_only) {
  void *ptrs[64];
  for (u32 i = 0; i < n; i++) {
    ptrs[i] = hb_buf_ptr(ids[i]);
    if (!ptrs[i]) { hb_set_error("custom %s: argument %u (buffer %u) is not live", name, i, ids[i]); return -1; }
  }
  hipFunction_t fn = rtc_get(name, source);
  if (!fn) return -1;
  if (check_only) return 0;
  u32 g[3], b[3];
  for (int d = 0; d < 3; d++) {
    g[d] = (grid && grid[d]) ? grid[d] : 1;
    b[d] = (block && block[d]) ? block[d] : 1;
  }
  if ((u64)b[0] * b[1] * b[2] > 1024) { hb_set_error("custom %s: block of %u threads > 1024", name, b[0] * b[1] * b[2]); return -1; }
  if (shared > 160u * 1024u) { hb_set_error("custom %s: %u bytes of LDS > 160 KiB", name, shared); return -1; }
  void *params[64];
  for (u32 i = 0; i < n; i++) params[i] = &ptrs[i];
  hipError_t e = hipModuleLaunchKernel(fn, g[0], g[1], g[2], b[0], b[1], b[2], shared, HB_STREAM,
                                       params, NULL);
  if (e != hipSuccess) { hb_set_error("custom %s: launch: %s", name, hipGetErrorString(e)); return -1; }
  return 0;
}

int hb_launch_op(const char *name, const char *program, const u32 grid[3], const u32 block[3],
                 u32 shared, const u32 *ids, u32 n) {
  if (strncmp(program, BUILTIN_PREFIX, strlen(BUILTIN_PREFIX)) == 0)
    return hb_builtin_launch(program, ids, n, 0);
  return hb_rtc_launch(name, program, grid, block, shared, ids, n, 0);
}

THVM_API int thvm_hip_program_check(const char *name, const char *program) {
  if (hb_require_ready("program_check")) return -1;
  if (!name || !program || !name[0] || !program[0]) { hb_set_error("program_check: empty name or program"); return -1; }
  if (strncmp(program, BUILTIN_PREFIX, strlen(BUILTIN_PREFIX)) == 0) {
    Spec sp;
    return spec_parse(program, &sp);
  }
  return rtc_get(name, program) ? 0 : -1;
}

/* ======================= attention without a workspace ================= */

THVM_API int thvm_hip_attn_decode_noalloc(const char *program, const uint32_t *buf_ids,
                                          uint32_t n_args) {
  if (hb_require_ready("attn_decode_noalloc")) return -1;
  if (!program || !buf_ids) { hb_set_error("attn_decode_noalloc: null program or ids"); return -1; }
  Spec sp;
  if (spec_parse(program, &sp)) return -1;
  if (strcmp(sp.kernel, "attn") != 0) {
    hb_set_error("attn_decode_noalloc: program is thvm-builtin:%s, want thvm-builtin:attn", sp.kernel);
    return -1;
  }
  if (n_args != 5) {
    hb_set_error("attn_decode_noalloc: %u buffers, want 5 (out, q, kcache, vcache, len)", n_args);
    return -1;
  }
  ArgCtx c = {buf_ids, n_args, sp.kernel, 0};
  ThvmAttnArgs a;
  if (attn_parse(&sp, &c, &a, 0)) return -1;
  char err[256] = {0};
  if (thvm_k_attn_decode_scratch(&a, HB_STREAM, err, sizeof err)) {
    hb_set_error("%s", err);
    return -1;
  }
  return 0;
}

/* ======================= graph hooks =================================== */

#define HB_GRAPH_SLOTS 16
typedef struct { hipGraph_t g; hipGraphExec_t ge; int valid; } GraphSlot;
static GraphSlot GRAPHS[HB_GRAPH_SLOTS];

THVM_API int thvm_hip_graph_replay(uint32_t slot) {
  if (!HB_READY || slot >= HB_GRAPH_SLOTS || !GRAPHS[slot].valid) return -1;
  const char *off = getenv("THVM_HIP_JIT_GRAPH");
  if (off && off[0] == '0') return -1;
  hipError_t e = hipGraphLaunch(GRAPHS[slot].ge, HB_STREAM);
  if (e != hipSuccess) { hb_set_error("hipGraphLaunch: %s", hipGetErrorString(e)); return -1; }
  return 0;
}

THVM_API int thvm_hip_graph_capture_begin(void) {
  if (hb_require_ready("graph_capture_begin")) return -1;
  const char *off = getenv("THVM_HIP_JIT_GRAPH");
  if (off && off[0] == '0') return -1;
  if (HB_GRAPH_CAPTURING) { hb_set_error("graph_capture_begin: capture already open"); return -1; }
  hipError_t e = hipStreamBeginCapture(HB_STREAM, hipStreamCaptureModeThreadLocal);
  if (e != hipSuccess) { hb_set_error("hipStreamBeginCapture: %s", hipGetErrorString(e)); return -1; }
  HB_GRAPH_CAPTURING = 1;
  return 0;
}

THVM_API void thvm_hip_graph_invalidate(uint32_t slot) {
  if (slot >= HB_GRAPH_SLOTS || !GRAPHS[slot].valid) return;
  hipGraphExecDestroy(GRAPHS[slot].ge);
  hipGraphDestroy(GRAPHS[slot].g);
  memset(&GRAPHS[slot], 0, sizeof GRAPHS[slot]);
}

THVM_API int thvm_hip_graph_capture_end_and_launch(uint32_t slot) {
  if (!HB_GRAPH_CAPTURING) { hb_set_error("graph_capture_end: no capture open"); return -1; }
  hipGraph_t g = NULL;
  hipError_t e = hipStreamEndCapture(HB_STREAM, &g);
  HB_GRAPH_CAPTURING = 0;
  if (e != hipSuccess || g == NULL) { hb_set_error("hipStreamEndCapture: %s", hipGetErrorString(e)); return -1; }
  if (slot >= HB_GRAPH_SLOTS) { hipGraphDestroy(g); hb_set_error("graph slot %u out of range", slot); return -1; }
  hipGraphExec_t ge = NULL;
  e = hipGraphInstantiate(&ge, g, NULL, NULL, 0);
  if (e != hipSuccess) { hipGraphDestroy(g); hb_set_error("hipGraphInstantiate: %s", hipGetErrorString(e)); return -1; }
  thvm_hip_graph_invalidate(slot);
  GRAPHS[slot].g = g;
  GRAPHS[slot].ge = ge;
  GRAPHS[slot].valid = 1;
  e = hipGraphLaunch(ge, HB_STREAM);
  if (e != hipSuccess) { hb_set_error("hipGraphLaunch(first): %s", hipGetErrorString(e)); return -1; }
  return 0;
}

void hb_graph_reset(void) {
  if (HB_GRAPH_CAPTURING) {
    hipGraph_t g = NULL;
    hipStreamEndCapture(HB_STREAM, &g);
    if (g) hipGraphDestroy(g);
    HB_GRAPH_CAPTURING = 0;
  }
  for (u32 i = 0; i < HB_GRAPH_SLOTS; i++) thvm_hip_graph_invalidate(i);
}

/* ======================= JIT capture / replay ========================== */

typedef struct {
  int  used;
  HbOp *ops;
  u32  n_ops, cap;
  u64  addr_sig;        /* device addresses the cached graph was built on */
} JitSlot;
static JitSlot JIT[HB_GRAPH_SLOTS];
static u32 JIT_CAPTURING = 0;    /* slot being recorded, 0 = none */

THVM_API int thvm_hip_jit_is_capturing(void) { return JIT_CAPTURING != 0; }

static void op_free(HbOp *o) {
  free(o->name);
  free(o->program);
  memset(o, 0, sizeof *o);
}

THVM_API uint32_t thvm_hip_jit_capture_begin(void) {
  if (hb_require_ready("jit_capture_begin")) return 0;
  if (JIT_CAPTURING) { hb_set_error("jit_capture_begin: a capture is already open"); return 0; }
  for (u32 s = 1; s < HB_GRAPH_SLOTS; s++) {
    if (!JIT[s].used) {
      memset(&JIT[s], 0, sizeof JIT[s]);
      JIT[s].used = 1;
      JIT_CAPTURING = s;
      thvm_hip_graph_invalidate(s);
      return s;
    }
  }
  hb_set_error("jit_capture_begin: all %d slots in use", HB_GRAPH_SLOTS - 1);
  return 0;
}

THVM_API void thvm_hip_jit_capture_end(void) { JIT_CAPTURING = 0; }

THVM_API uint32_t thvm_hip_jit_capture_op_count(uint32_t slot) {
  if (slot == 0 || slot >= HB_GRAPH_SLOTS || !JIT[slot].used) return 0;
  return JIT[slot].n_ops;
}

static int jit_record(const char *name, const char *program, const u32 grid[3], const u32 block[3],
                      u32 shared, const u32 *ids, u32 n, u64 outs_mask) {
  JitSlot *js = &JIT[JIT_CAPTURING];
  if (js->n_ops == js->cap) {
    js->cap = js->cap ? 2 * js->cap : 64;
    HbOp *nops = (HbOp *)realloc(js->ops, js->cap * sizeof(HbOp));
    if (!nops) { hb_set_error("jit_record: out of memory"); return -1; }
    js->ops = nops;
  }
  HbOp *o = &js->ops[js->n_ops];
  memset(o, 0, sizeof *o);
  o->name = strdup(name);
  o->program = strdup(program);
  for (int d = 0; d < 3; d++) {
    o->grid[d] = grid ? grid[d] : 1;
    o->block[d] = block ? block[d] : 1;
  }
  o->shared = shared;
  o->n_args = n;
  memcpy(o->args, ids, n * sizeof(u32));
  o->outs_mask = outs_mask;
  for (u32 i = 0; i < n; i++) thvm_hip_buf_jit_pin(ids[i]);
  js->n_ops++;
  return 0;
}

static u64 jit_addr_sig(const JitSlot *js) {
  u64 h = 0;
  for (u32 i = 0; i < js->n_ops; i++) {
    const HbOp *o = &js->ops[i];
    for (u32 a = 0; a < o->n_args; a++) {
      void *p = hb_buf_ptr(o->args[a]);
      h = hb_hash64(&p, sizeof p, h);
    }
  }
  return h;
}

THVM_API int thvm_hip_jit_replay(uint32_t slot) {
  if (hb_require_ready("jit_replay")) return -1;
  if (slot == 0 || slot >= HB_GRAPH_SLOTS || !JIT[slot].used) { hb_set_error("jit_replay: slot %u not captured", slot); return -1; }
  if (JIT_CAPTURING) { hb_set_error("jit_replay: a capture is open"); return -1; }
  JitSlot *js = &JIT[slot];
  u64 sig = jit_addr_sig(js);
  if (sig == js->addr_sig && thvm_hip_graph_replay(slot) == 0) return 0;
  /* graph miss: capture the op loop, then launch (capture.c:2695-2760) */
  int graph = thvm_hip_graph_capture_begin() == 0;
  for (u32 i = 0; i < js->n_ops; i++) {
    HbOp *o = &js->ops[i];
    if (hb_launch_op(o->name, o->program, o->grid, o->block, o->shared, o->args, o->n_args)) {
      if (graph) {
        hipGraph_t g = NULL;
        hipStreamEndCapture(HB_STREAM, &g);
        if (g) hipGraphDestroy(g);
        HB_GRAPH_CAPTURING = 0;
      }
      return -1;
    }
  }
  if (graph) {
    if (thvm_hip_graph_capture_end_and_launch(slot)) return -1;
    js->addr_sig = sig;
  }
  return 0;
}

THVM_API int thvm_hip_jit_rebind(uint32_t slot, const uint32_t *old_ids, const uint32_t *new_ids,
                                 uint32_t n) {
  if (slot == 0 || slot >= HB_GRAPH_SLOTS || !JIT[slot].used) { hb_set_error("jit_rebind: bad slot %u", slot); return -1; }
  JitSlot *js = &JIT[slot];
  for (u32 k = 0; k < n; k++) {
    if (!hb_buf_ptr(new_ids[k])) { hb_set_error("jit_rebind: buffer %u not live", new_ids[k]); return -1; }
  }
  for (u32 i = 0; i < js->n_ops; i++) {
    HbOp *o = &js->ops[i];
    for (u32 a = 0; a < o->n_args; a++)
      for (u32 k = 0; k < n; k++)
        if (o->args[a] == old_ids[k]) { o->args[a] = new_ids[k]; break; }
  }
  for (u32 k = 0; k < n; k++) thvm_hip_buf_jit_pin(new_ids[k]);
  return 0;   /* the address signature re-captures on the next replay */
}

THVM_API void thvm_hip_jit_capture_drop(uint32_t slot) {
  if (slot == 0 || slot >= HB_GRAPH_SLOTS || !JIT[slot].used) return;
  JitSlot *js = &JIT[slot];
  for (u32 i = 0; i < js->n_ops; i++) {
    for (u32 a = 0; a < js->ops[i].n_args; a++) thvm_hip_buf_jit_unpin(js->ops[i].args[a]);
    op_free(&js->ops[i]);
  }
  free(js->ops);
  memset(js, 0, sizeof *js);
  if (JIT_CAPTURING == slot) JIT_CAPTURING = 0;
  thvm_hip_graph_invalidate(slot);
}

void hb_jit_reset(void) {
  for (u32 s = 1; s < HB_GRAPH_SLOTS; s++) thvm_hip_jit_capture_drop(s);
  JIT_CAPTURING = 0;
}

/* ======================= custom dispatch =============================== */

THVM_API int thvm_hip_dispatch_custom(const char *name, const char *program, const uint32_t grid[3],
                                      const uint32_t block[3], uint32_t shared_bytes,
                                      const uint32_t *buf_ids, uint32_t n_args, uint64_t outs_mask) {
  if (hb_require_ready("dispatch_custom")) return -1;
  if (!name || !program || !name[0] || !program[0]) { hb_set_error("dispatch_custom: empty name or program"); return -1; }
  if (n_args == 0 || n_args > 64) { hb_set_error("dispatch_custom: n_args=%u out of range [1,64]", n_args); return -1; }
  if (outs_mask == 0 || (n_args < 64 && (outs_mask >> n_args) != 0)) {
    hb_set_error("dispatch_custom: outs_mask 0x%llx does not name an argument slot",
                 (unsigned long long)outs_mask);
    return -1;
  }
  if (JIT_CAPTURING &&
      jit_record(name, program, grid, block, shared_bytes, buf_ids, n_args, outs_mask))
    return -1;
  return hb_launch_op(name, program, grid, block, shared_bytes, buf_ids, n_args);
}
