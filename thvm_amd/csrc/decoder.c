/* decoder.c -- synthetic decode drivers: the whole decode step of a
 * random-init model as a list of custom dispatches over builtin gfx950
 * kernels, captured once and replayed as one hipGraph launch per token.
 *
 * Counterpart of the reference DeepSeek-V2 decode driver
 * (bench/dsv2_decode_bench.c: model_init, step_build :2328-2430, capture +
 * replay :2898-3008) and of the GPT-2 driver (bench/gpt2/thvm_gpt2.py:96-131).
 * As there, the token and the position live in device buffers (argmax writes
 * the next token, len_bump advances L), so a replay needs no host values.
 *
 * Step (LLAMA, per layer):
 *   norm   xn = rms(x) * g_attn                       -> bf16
 *   gemv   [q|k|v] = xn Wqkv^T, RoPE(q, k) at L-1, k/v appended to the caches
 *   attn   att = softmax(q K^T / sqrt(hd)) V over rows [0, L)
 *   gemv   x = x + att Wo^T                           (residual epilogue)
 *   norm   xn = rms(x) * g_ffn
 *   gemv   h = silu(xn Wg^T) * (xn Wu^T)              (rows interleaved g/u)
 *   gemv   x = x + h Wd^T
 * then final norm, LM head (f32 logits), argmax -> tok / history, len_bump.
 * GPT2 swaps RMSNorm for LayerNorm (+bias), RoPE for learned positions,
 * SwiGLU for GELU, and ties the LM head to the token embedding.
 *
 * Numerics: activations are rounded to the activation dtype exactly where
 * the reference decode chain rounds them (matmul outputs before RoPE /
 * residual use, residual sums, norm outputs: bench/dsv2_decode_bench.c:20-34). */
#define _GNU_SOURCE
#include "internal.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

typedef struct {
  char name[40];
  u32  id;
  u32  dt;
  u64  nbytes;
} DTensor;

typedef struct {
  char *name;
  char *prog;
  u32   args[24];
  u32   n_args;
  u64   outs;
  int32_t tag;   /* 2l: layer l's attention sublayer, 2l+1: its FFN; -1 before the layers, -2 after */
} DOp;

typedef struct {
  int used;
  ThvmDecodeConfig c;
  u64 seed;
  DTensor t[2048];
  u32 nt;
  DOp *ops;
  u32 n_ops, cap_ops;
  u32 jit_slot;
  u32 n_split;
  u64 weight_bytes;       /* streamed weight + scale bytes per step */
  /* op emission: the rows of the step being built, speculative verify, and
   * the name prefix of its activation tensors ("" for the one-row step) */
  u32 rows;
  int spec;
  char pfx[4];
  int32_t cur_tag;        /* tag of the ops being added */
  DOp *sops;              /* the speculative step (spec_rows > 0) */
  u32 n_sops;
  u32 spec_slot;
  /* the MFMA GEMM's tiled copies of weight matrices (batches above 4 rows) */
  struct { u32 src, dst, n, k, wt, lb; } tiles[512];
  u32 n_tiles;
} Decoder;

#define MAX_DEC 8
static Decoder DEC[MAX_DEC];

static Decoder *dec_get(u32 h) {
  if (h == 0 || h > MAX_DEC || !DEC[h - 1].used) {
    hb_set_error("decoder %u: no such decoder", h);
    return NULL;
  }
  return &DEC[h - 1];
}

static u32 tens_find(Decoder *d, const char *name) {
  for (u32 i = 0; i < d->nt; i++)
    if (strcmp(d->t[i].name, name) == 0) return d->t[i].id;
  return 0;
}

static u32 tens_new(Decoder *d, const char *name, u32 dt, u64 nbytes) {
  if (d->nt >= sizeof d->t / sizeof d->t[0]) { hb_set_error("decoder: tensor table full"); return 0; }
  u32 id = thvm_hip_buf_alloc(nbytes);
  if (!id) return 0;
  DTensor *t = &d->t[d->nt++];
  snprintf(t->name, sizeof t->name, "%s", name);
  t->id = id;
  t->dt = dt;
  t->nbytes = nbytes;
  return id;
}

/* a per-step activation tensor of the step being built */
static u32 act(Decoder *d, const char *name) {
  char nm[48];
  snprintf(nm, sizeof nm, "%s%s", d->pfx, name);
  return tens_find(d, nm);
}

static u64 name_tag(const char *name) { return hb_hash64(name, strlen(name), 0x7468766dull); }

/* run a builtin immediately (set-up work, never recorded) */
static int run_now(const char *prog, const u32 *ids, u32 n) {
  return hb_builtin_launch(prog, ids, n, 0);
}

static u32 weight_normal(Decoder *d, const char *name, u32 dt, u64 n, float mean, float std) {
  u32 id = tens_new(d, name, dt, n * hb_dt_size(dt));
  if (!id) return 0;
  char p[256];
  snprintf(p, sizeof p, "thvm-builtin:fill_normal n=%llu dt=%u seed=%llu tag=%llu mean=%a std=%a",
           (unsigned long long)n, dt, (unsigned long long)d->seed,
           (unsigned long long)name_tag(name), mean, std);
  if (run_now(p, &id, 1)) return 0;
  return id;
}

static u32 weight_const(Decoder *d, const char *name, u64 n, float v) {
  u32 id = tens_new(d, name, THVM_DT_FP32, n * 4);
  if (!id) return 0;
  float *h = (float *)malloc(n * 4);
  if (!h) { hb_set_error("decoder: out of host memory"); return 0; }
  for (u64 i = 0; i < n; i++) h[i] = v;
  int rc = thvm_hip_buf_write(id, h, n * 4);
  free(h);
  return rc ? 0 : id;
}

/* weight matrix [rows, cols] of dtype wdt; fp8 also gets "<name>.scale" */
static int weight_matrix(Decoder *d, const char *name, u32 rows, u32 cols, u32 *w, u32 *s) {
  u32 wdt = d->c.wdtype;
  *s = 0;
  if (wdt == THVM_DT_FP8E4M3) {
    *w = tens_new(d, name, wdt, (u64)rows * cols);
    char sn[48];
    snprintf(sn, sizeof sn, "%s.scale", name);
    *s = tens_new(d, sn, THVM_DT_FP32, (u64)rows * 4);
    if (!*w || !*s) return -1;
    char p[256];
    snprintf(p, sizeof p, "thvm-builtin:fill_fp8 rows=%u cols=%u seed=%llu tag=%llu std=%a", rows,
             cols, (unsigned long long)d->seed, (unsigned long long)name_tag(name), d->c.init_std);
    u32 ids[2] = {*w, *s};
    if (run_now(p, ids, 2)) return -1;
    d->weight_bytes += (u64)rows * cols + (u64)rows * 4;
    return 0;
  }
  *w = weight_normal(d, name, wdt, (u64)rows * cols, 0.0f, d->c.init_std);
  if (!*w) return -1;
  d->weight_bytes += (u64)rows * cols * hb_dt_size(wdt);
  return 0;
}

/* The unsigned value of " key=" in a builtin spec (def when absent). */
static u32 prog_u32(const char *prog, const char *key, u32 def) {
  char k[24];
  snprintf(k, sizeof k, " %s=", key);
  const char *p = strstr(prog, k);
  return p ? (u32)strtoul(p + strlen(k), NULL, 0) : def;
}

/* Batches above 4 rows run their projections on the MFMA GEMM, which reads
 * weights in the tile layout of thvm_k_tile_w (a wave's load instruction
 * then reads 1 KB contiguous instead of 16 rows x 64 bytes): each weight
 * matrix such an op names gets a tiled copy "<name>.tiled", made here and
 * refreshed by thvm_hip_decoder_sync_weights after the row-major tensor is
 * written.  The row-major tensors stay what the decoder's tensor API reads
 * and writes.  THVM_HIP_WTILE=0 keeps the row-major reads (A/B). */
static int wtile_on(void) {
  const char *e = getenv("THVM_HIP_WTILE");
  return !(e && e[0] == '0');
}

static int tile_run(const Decoder *d, u32 i) {
  char p[128];
  snprintf(p, sizeof p, "thvm-builtin:tile_w n=%u k=%u wt=%u lb=%u", d->tiles[i].n, d->tiles[i].k,
           d->tiles[i].wt, d->tiles[i].lb);
  const u32 ids[2] = {d->tiles[i].dst, d->tiles[i].src};
  return run_now(p, ids, 2);
}

static u32 tiled_copy(Decoder *d, u32 src, u32 n, u32 k, u32 wt, u32 lb) {
  for (u32 i = 0; i < d->n_tiles; i++)
    if (d->tiles[i].src == src && d->tiles[i].n == n && d->tiles[i].k == k && d->tiles[i].lb == lb)
      return d->tiles[i].dst;
  if (d->n_tiles >= sizeof d->tiles / sizeof d->tiles[0]) { hb_set_error("decoder: tiled weight table full"); return 0; }
  const char *nm = "w";
  for (u32 i = 0; i < d->nt; i++)
    if (d->t[i].id == src) { nm = d->t[i].name; break; }
  char tn[48];
  snprintf(tn, sizeof tn, "%s.tiled", nm);
  const u32 dst = tens_new(d, tn, wt, ((u64)n + 15) / 16 * 16 * k * hb_dt_size(wt));
  if (!dst) return 0;
  const u32 i = d->n_tiles++;
  d->tiles[i].src = src; d->tiles[i].dst = dst; d->tiles[i].n = n; d->tiles[i].k = k; d->tiles[i].wt = wt;
  d->tiles[i].lb = lb;
  return tile_run(d, i) ? 0 : dst;
}

static int op_add_raw(Decoder *d, const char *name, const char *prog, const u32 *args, u32 n);

static int op_add(Decoder *d, const char *name, const char *prog, const u32 *args, u32 n) {
  if (n >= 3 && d->rows > 4 && wtile_on() && strncmp(prog, "thvm-builtin:gemv ", 18) == 0 &&
      prog_u32(prog, "path", 0) != 1 && prog_u32(prog, "m", 0) > 4) {
    const u32 wt = prog_u32(prog, "wt", 0), xt = prog_u32(prog, "xt", THVM_DT_BF16), k = prog_u32(prog, "k", 0);
    const u32 nrm = prog_u32(prog, "norm", 0);
    const int mfma = (nrm == 0 || (nrm == 1 && xt == THVM_DT_BF16)) && k % 64 == 0 &&
                     ((wt == THVM_DT_FP16 && xt == THVM_DT_FP16) ||
                                     (wt == THVM_DT_BF16 && xt == THVM_DT_BF16) ||
                                     (wt == THVM_DT_FP8E4M3 && (xt == THVM_DT_BF16 || xt == THVM_DT_FP16)));
    if (mfma && n <= 24 && strlen(prog) + 10 < 1024) {
      const u32 tw = tiled_copy(d, args[2], prog_u32(prog, "n", 0), k, wt, 16 * hb_dt_size(wt));
      if (!tw) return -1;
      u32 a2[24];
      memcpy(a2, args, n * sizeof(u32));
      a2[2] = tw;
      char p2[1024];
      snprintf(p2, sizeof p2, "%s tiled=1", prog);
      return op_add_raw(d, name, p2, a2, n);
    }
  }
  return op_add_raw(d, name, prog, args, n);
}

static int op_add_raw(Decoder *d, const char *name, const char *prog, const u32 *args, u32 n) {
  if (n > 24) { hb_set_error("decoder: op %s has too many args", name); return -1; }
  if (d->n_ops == d->cap_ops) {
    d->cap_ops = d->cap_ops ? 2 * d->cap_ops : 256;
    d->ops = (DOp *)realloc(d->ops, d->cap_ops * sizeof(DOp));
    if (!d->ops) { hb_set_error("decoder: out of memory"); return -1; }
  }
  for (u32 i = 0; i < n; i++)
    if (args[i] == 0) { hb_set_error("decoder: op %s arg %u unset", name, i); return -1; }
  DOp *o = &d->ops[d->n_ops++];
  o->name = strdup(name);
  o->prog = strdup(prog);
  memcpy(o->args, args, n * sizeof(u32));
  o->n_args = n;
  o->outs = 1;
  o->tag = d->cur_tag;
  if (hb_builtin_launch(prog, args, n, 1)) return -1;   /* validate now */
  return 0;
}

static int rope_tables(Decoder *d) {
  u32 hd = d->c.head_dim, half = hd / 2, ms = d->c.max_seq;
  u64 n = (u64)ms * half;
  float *cs = (float *)malloc(n * 4), *sn = (float *)malloc(n * 4);
  if (!cs || !sn) { free(cs); free(sn); hb_set_error("decoder: out of host memory"); return -1; }
  for (u32 p = 0; p < ms; p++)
    for (u32 j = 0; j < half; j++) {
      double f = 1.0 / pow((double)d->c.rope_theta, (double)(2 * j) / (double)hd);
      double a = (double)p * f;
      cs[(u64)p * half + j] = (float)cos(a);
      sn[(u64)p * half + j] = (float)sin(a);
    }
  u32 ci = tens_new(d, "rope.cos", THVM_DT_FP32, n * 4);
  u32 si = tens_new(d, "rope.sin", THVM_DT_FP32, n * 4);
  int rc = (!ci || !si || thvm_hip_buf_write(ci, cs, n * 4) || thvm_hip_buf_write(si, sn, n * 4)) ? -1 : 0;
  free(cs);
  free(sn);
  return rc;
}

/* the argmax op's sampling keys: "" (greedy) or " temp=<T> seed=<seed>" */
static const char *sample_keys(const ThvmDecodeConfig *c, char *buf, size_t n) {
  buf[0] = 0;
  if (c->temperature > 0.0f)
    snprintf(buf, n, " temp=%a seed=%llu", (double)c->temperature,
             (unsigned long long)(((u64)c->sample_seed_hi << 32) | c->sample_seed_lo));
  return buf;
}

static int cfg_check(const ThvmDecodeConfig *c) {
  if (c->arch != THVM_ARCH_LLAMA && c->arch != THVM_ARCH_GPT2 && c->arch != THVM_ARCH_DSV2) {
    hb_set_error("decoder: arch %u not supported by this build", c->arch);
    return -1;
  }
  if (!(c->temperature >= 0.0f) || c->temperature > 1e30f) {
    hb_set_error("decoder: temperature must be a finite value >= 0");
    return -1;
  }
  if (c->step_mode && c->temperature > 0.0f) {
    hb_set_error("decoder: the persistent step (step_mode 1) decodes greedily; temperature must be 0");
    return -1;
  }
  if (c->step_mode > 1 || (c->step_mode && c->arch != THVM_ARCH_LLAMA)) {
    hb_set_error("decoder: step_mode 1 (persistent step) is for the LLAMA architecture");
    return -1;
  }
  if (c->attn_cpb > 64) {
    hb_set_error("decoder: attn_cpb is 0 (auto) or 1..64 chunks per split block");
    return -1;
  }
  if (c->spec_rows == 1 || c->spec_rows > 4 || c->spec_forced > 1) {
    hb_set_error("decoder: spec_rows is 0 (off) or 2..4, spec_forced 0 or 1");
    return -1;
  }
  if (c->spec_rows && (c->arch != THVM_ARCH_LLAMA || c->batch != 1 || c->temperature > 0.0f ||
                       c->step_mode)) {
    hb_set_error("decoder: speculative decode is for the LLAMA op-list step at batch 1, greedy");
    return -1;
  }
  if (c->attn_fused > 2) {
    hb_set_error("decoder: attn_fused is 0 (auto), 1 (one launch) or 2 (two launches)");
    return -1;
  }
  if (c->attn_mf > 2) {
    hb_set_error("decoder: attn_mf is 0 (auto), 1 (the MFMA split) or 2 (the VALU split)");
    return -1;
  }
  if (c->moe_mode > 2) {
    hb_set_error("decoder: moe_mode is 0 (auto), 1 (VALU grouped) or 2 (MFMA grouped)");
    return -1;
  }
  if (c->arch == THVM_ARCH_DSV2) {
    if (!c->n_layers || !c->dim || !c->n_heads || !c->vocab || !c->max_seq || !c->batch ||
        !c->kv_lora || !c->d_nope || !c->d_rope || !c->d_v || !c->n_experts || !c->top_k ||
        !c->moe_inter || (c->first_dense && !c->ffn)) {
      hb_set_error("decoder: zero dimension in DSV2 config");
      return -1;
    }
    if (c->batch > 64 || (c->batch > 4 && c->batch % 4)) {
      hb_set_error("decoder: DSV2 batch %u (1..4, or a multiple of 4 up to 64)", c->batch);
      return -1;
    }
    if (c->batch > 4 && (c->dim % 64 || (c->n_heads * c->d_v) % 64 || (c->first_dense && c->ffn % 64))) {
      hb_set_error("decoder: DSV2 batch above 4 runs the MFMA GEMM: dim, heads*d_v and ffn multiples of 64");
      return -1;
    }
    if (c->wdtype != THVM_DT_FP8E4M3 && c->wdtype != THVM_DT_BF16) {
      hb_set_error("decoder: DSV2 weights must be fp8 e4m3 or bf16");
      return -1;
    }
    if (c->adtype != THVM_DT_BF16) { hb_set_error("decoder: DSV2 activations are bf16"); return -1; }
    return 0;
  }
  if (!c->n_layers || !c->dim || !c->n_heads || !c->head_dim || !c->ffn || !c->vocab ||
      !c->max_seq || !c->batch) {
    hb_set_error("decoder: zero dimension in config");
    return -1;
  }
  u32 hkv = c->n_kv_heads ? c->n_kv_heads : c->n_heads;
  if (c->n_heads % hkv) { hb_set_error("decoder: n_heads %% n_kv_heads != 0"); return -1; }
  if (c->head_dim != 64 && c->head_dim != 128) { hb_set_error("decoder: head_dim must be 64 or 128"); return -1; }
  u32 wdt = c->wdtype, adt = c->adtype;
  if (c->batch > 64) { hb_set_error("decoder: batch %u > 64", c->batch); return -1; }
  if (c->batch > 4) {   /* projections run on the MFMA GEMM */
    int ok = (wdt == THVM_DT_FP8E4M3 && (adt == THVM_DT_BF16 || adt == THVM_DT_FP16)) ||
             (wdt == THVM_DT_BF16 && adt == THVM_DT_BF16) || (wdt == THVM_DT_FP16 && adt == THVM_DT_FP16);
    if (!ok) {
      hb_set_error("decoder: batch %u > 4 runs the MFMA GEMM, which takes fp8 weights with bf16/fp16 "
                   "activations or 16-bit weights of the activation dtype", c->batch);
      return -1;
    }
    if (c->dim % 64 || (c->n_heads * c->head_dim) % 64 || c->ffn % 64) {
      hb_set_error("decoder: batch %u > 4 needs dim, heads*head_dim and ffn multiples of 64", c->batch);
      return -1;
    }
  }
  if (wdt != THVM_DT_FP32 && wdt != THVM_DT_FP16 && wdt != THVM_DT_BF16 && wdt != THVM_DT_FP8E4M3) {
    hb_set_error("decoder: weight dtype %u unsupported", wdt);
    return -1;
  }
  if (adt != THVM_DT_FP32 && adt != THVM_DT_FP16 && adt != THVM_DT_BF16) {
    hb_set_error("decoder: activation dtype %u unsupported", adt);
    return -1;
  }
  if (c->arch == THVM_ARCH_GPT2 && wdt == THVM_DT_FP8E4M3) {
    hb_set_error("decoder: GPT2 ties the LM head to the embedding; fp8 weights unsupported");
    return -1;
  }
  if (c->arch == THVM_ARCH_GPT2 && (adt == THVM_DT_FP32) != (wdt == THVM_DT_FP32)) {
    hb_set_error("decoder: GPT2 keeps weights and activations in one dtype");
    return -1;
  }
  return 0;
}

static int build_llama(Decoder *d);
static int build_gpt2(Decoder *d);
static int build_dsv2(Decoder *d);

static void ops_free(DOp *ops, u32 n) {
  for (u32 i = 0; i < n; i++) { free(ops[i].name); free(ops[i].prog); }
  free(ops);
}

static void dec_free(Decoder *d) {
  if (d->jit_slot) thvm_hip_jit_capture_drop(d->jit_slot);
  if (d->spec_slot) thvm_hip_jit_capture_drop(d->spec_slot);
  for (u32 i = 0; i < d->nt; i++) thvm_hip_buf_free(d->t[i].id);
  ops_free(d->ops, d->n_ops);
  ops_free(d->sops, d->n_sops);
  memset(d, 0, sizeof *d);
}

THVM_API uint32_t thvm_hip_decoder_create(const ThvmDecodeConfig *cfg, uint64_t seed) {
  if (hb_require_ready("decoder_create")) return 0;
  if (!cfg || cfg_check(cfg)) return 0;
  u32 h = 0;
  for (u32 i = 0; i < MAX_DEC; i++)
    if (!DEC[i].used) { h = i + 1; break; }
  if (!h) { hb_set_error("decoder_create: too many decoders"); return 0; }
  Decoder *d = &DEC[h - 1];
  memset(d, 0, sizeof *d);
  d->used = 1;
  d->c = *cfg;
  if (!d->c.n_kv_heads) d->c.n_kv_heads = d->c.n_heads;
  if (d->c.init_std == 0.0f) d->c.init_std = 0.02f;
  d->seed = seed;
  d->n_split = (d->c.max_seq + 63) / 64;
  d->rows = d->c.batch;
  d->cur_tag = -1;
  int rc = d->c.arch == THVM_ARCH_LLAMA ? build_llama(d)
         : d->c.arch == THVM_ARCH_GPT2  ? build_gpt2(d) : build_dsv2(d);
  if (rc) { dec_free(d); return 0; }
  hipError_t e = hipStreamSynchronize(HB_STREAM);
  if (e != hipSuccess) { hb_set_error("decoder_create: %s", hipGetErrorString(e)); dec_free(d); return 0; }
  return h;
}

/* shared state tensors: tok, len, hist, logits, argmax partials, acts */
static int build_state(Decoder *d) {
  const ThvmDecodeConfig *c = &d->c;
  u32 B = c->batch, adt = c->adtype, as = hb_dt_size(adt);
  u32 hq = c->n_heads * c->head_dim;
  if (!tens_new(d, "tok", THVM_DT_INT32, (u64)B * 4) || !tens_new(d, "len", THVM_DT_INT32, 4) ||
      !tens_new(d, "hist", THVM_DT_INT32, (u64)B * (c->max_seq + 1) * 4) ||
      !tens_new(d, "logits", THVM_DT_FP32, (u64)B * c->vocab * 4) ||
      !tens_new(d, "am.pv", THVM_DT_FP32, (u64)B * 256 * 4) ||
      !tens_new(d, "am.pi", THVM_DT_INT32, (u64)B * 256 * 4) ||
      !tens_new(d, "x", adt, (u64)B * c->dim * as) || !tens_new(d, "xn", adt, (u64)B * c->dim * as) ||
      !tens_new(d, "q", adt, (u64)B * hq * as) || !tens_new(d, "att", adt, (u64)B * hq * as) ||
      !tens_new(d, "h", adt, (u64)B * c->ffn * as) ||
      !tens_new(d, "attn.part", THVM_DT_FP32,
                thvm_k_attn_part_bytes(B, c->n_heads, c->n_kv_heads, c->head_dim, d->n_split)))
    return -1;
  for (u32 l = 0; l < c->n_layers; l++) {
    char kn[32], vn[32];
    snprintf(kn, sizeof kn, "l%u.kcache", l);
    snprintf(vn, sizeof vn, "l%u.vcache", l);
    u64 cb = (u64)B * c->n_kv_heads * c->max_seq * c->head_dim * as;
    if (!tens_new(d, kn, adt, cb) || !tens_new(d, vn, adt, cb)) return -1;
  }
  return 0;
}

static int op_attn(Decoder *d, u32 l) {
  const ThvmDecodeConfig *c = &d->c;
  char p[320], kn[32], vn[32];
  snprintf(kn, sizeof kn, "l%u.kcache", l);
  snprintf(vn, sizeof vn, "l%u.vcache", l);
  const u32 fused = c->attn_fused == 1 ? 1u : c->attn_fused == 2 ? 0u : 2u;
  /* a verify row folds the partials as the one-row step does: the same
   * split (MFMA or VALU) and the same split blocks, so the one-row step's
   * plan, passed explicitly */
  u32 cpb = c->attn_cpb, mf = c->attn_mf;
  if (d->spec) {
    ThvmAttnArgs base;
    memset(&base, 0, sizeof base);
    base.B = c->batch; base.H = c->n_heads; base.Hkv = c->n_kv_heads; base.hd = c->head_dim;
    base.max_seq = c->max_seq; base.chunk = 64; base.n_split = d->n_split;
    base.qdt = base.cdt = base.odt = c->adtype; base.fused = fused; base.cpb = c->attn_cpb;
    base.mf = c->attn_mf;
    u32 bmf = 0;
    thvm_k_attn_plan(&base, &bmf, &cpb);
    mf = bmf ? 1u : 2u;
  }
  snprintf(p, sizeof p,
           "thvm-builtin:attn b=%u h=%u hkv=%u hd=%u maxseq=%u chunk=64 nsplit=%u qt=%u ct=%u ot=%u scale=%a cpb=%u fused=%u mf=%u%s",
           d->rows, c->n_heads, c->n_kv_heads, c->head_dim, c->max_seq, d->n_split, c->adtype,
           c->adtype, c->adtype, (float)(1.0 / sqrt((double)c->head_dim)), cpb, fused, mf,
           d->spec ? " spec=1" : "");
  u32 a[6] = {act(d, "att"), act(d, "q"), tens_find(d, kn), tens_find(d, vn),
              tens_find(d, "len"), act(d, "attn.part")};
  return op_add(d, "attn", p, a, 6);
}

/* The norm feeding a GEMV: fused into the GEMV's x staging (default; above
 * 4 rows the MFMA GEMM's, which fuses RMSNorm over bf16 x), or as a separate
 * norm kernel writing xn (LayerNorm or fp16 x above 4 rows, or
 * THVM_HIP_UNFUSED_NORM=1 for A/B).  Above 4 rows every projection a norm
 * feeds runs on the MFMA GEMM (dim % 64 == 0 and the dtypes are checked at
 * config time).  Writes the GEMV's input id to *gin and its norm spec
 * fragment to nspec; gains are appended to the GEMV's argument list by the
 * caller via gargs. */
typedef struct { int kind; u32 g, b; } NormSpec;

static int fused_norms(const Decoder *d, const NormSpec *ns) {
  const char *e = getenv("THVM_HIP_UNFUSED_NORM");
  if (e && e[0] == '1') return 0;
  return d->rows <= 4 || (ns->kind == 1 && d->c.adtype == THVM_DT_BF16);
}

static int emit_norm(Decoder *d, const NormSpec *ns, u32 *gin, char *nspec, size_t nlen,
                     u32 *gargs, u32 *ng) {
  const ThvmDecodeConfig *c = &d->c;
  u32 x = act(d, "x"), xn = act(d, "xn");
  *ng = 0;
  if (fused_norms(d, ns)) {
    snprintf(nspec, nlen, " norm=%d eps=%a", ns->kind, c->eps);
    gargs[(*ng)++] = ns->g;
    if (ns->kind == 2) gargs[(*ng)++] = ns->b;
    *gin = x;
    return 0;
  }
  char p[200];
  nspec[0] = 0;
  snprintf(p, sizeof p, "thvm-builtin:norm m=%u k=%u xt=%u yt=%u eps=%a ln=%d bias=%d", d->rows,
           c->dim, c->adtype, c->adtype, c->eps, ns->kind == 2, ns->kind == 2);
  u32 a[4] = {xn, x, ns->g, ns->b};
  *gin = xn;
  return op_add(d, "norm", p, a, ns->kind == 2 ? 4 : 3);
}

static int op_tail(Decoder *d, u32 lm_w, u32 lm_s, const NormSpec *fn) {
  const ThvmDecodeConfig *c = &d->c;
  char p[400], nsp[96];
  u32 gin, gargs[2], ng;
  if (emit_norm(d, fn, &gin, nsp, sizeof nsp, gargs, &ng)) return -1;
  /* LM head -> f32 logits */
  snprintf(p, sizeof p, "thvm-builtin:gemv m=%u n=%u k=%u wt=%u xt=%u yt=%u epi=0%s",
           d->rows, c->vocab, c->dim, c->arch == THVM_ARCH_GPT2 ? c->adtype : c->wdtype,
           c->adtype, THVM_DT_FP32, nsp);
  u32 a[8], n = 0;
  a[n++] = act(d, "logits"); a[n++] = gin; a[n++] = lm_w;
  if (lm_s) a[n++] = lm_s;
  for (u32 i = 0; i < ng; i++) a[n++] = gargs[i];
  if (op_add(d, "lm_head", p, a, n)) return -1;
  u32 nb = c->vocab >= 256 * 64 ? 256 : (c->vocab + 63) / 64;
  if (d->spec) {   /* the verify rows' greedy ids, then the commit */
    snprintf(p, sizeof p, "thvm-builtin:argmax b=%u v=%u nb=%u", d->rows, c->vocab, nb);
    u32 b[4] = {act(d, "am"), act(d, "logits"), act(d, "am.pv"), act(d, "am.pi")};
    if (op_add(d, "argmax", p, b, 4)) return -1;
    snprintf(p, sizeof p, "thvm-builtin:spec_accept s=%u hcap=%u", d->rows, c->max_seq + 1);
    u32 e[5] = {tens_find(d, "hist"), tens_find(d, "len"), act(d, "ca"), act(d, "am"),
                tens_find(d, "tok")};
    return op_add(d, "spec_accept", p, e, 5);
  }
  char sk[96];
  snprintf(p, sizeof p, "thvm-builtin:argmax b=%u v=%u nb=%u hist=1 hstride=%u%s", c->batch,
           c->vocab, nb, c->max_seq + 1, sample_keys(c, sk, sizeof sk));
  u32 b[6] = {tens_find(d, "tok"), tens_find(d, "logits"), tens_find(d, "am.pv"),
              tens_find(d, "am.pi"), tens_find(d, "hist"), tens_find(d, "len")};
  if (op_add(d, "argmax", p, b, 6)) return -1;
  u32 L = tens_find(d, "len");
  return op_add(d, "len_bump", "thvm-builtin:len_bump delta=1", &L, 1);
}

/* The persistent step (step_mode 1): the same weights and state as the op
 * list just built, which it replaces by one llama_step dispatch.  Its first
 * slot is a device table of per-layer weight / cache pointers. */
static int build_llama_step(Decoder *d) {
  const ThvmDecodeConfig *c = &d->c;
  const u32 NL = c->n_layers, B = c->batch, nb = thvm_k_step_blocks();
  const int f8 = c->wdtype == THVM_DT_FP8E4M3;
  if (!nb) { hb_set_error("decoder: step_mode needs a device"); return -1; }
  ThvmStepLayer *tab = (ThvmStepLayer *)calloc(NL, sizeof *tab);
  if (!tab) { hb_set_error("decoder: out of host memory"); return -1; }
  char nm[48];
#define TP(fmt) (snprintf(nm, sizeof nm, fmt, l), hb_buf_ptr(tens_find(d, nm)))
  for (u32 l = 0; l < NL; l++) {
    ThvmStepLayer *t = &tab[l];
    t->wqkv = TP("l%u.wqkv"); t->wo = TP("l%u.wo"); t->wgu = TP("l%u.wgu"); t->wd = TP("l%u.wd");
    if (f8) {
      t->sqkv = (const float *)TP("l%u.wqkv.scale"); t->so = (const float *)TP("l%u.wo.scale");
      t->sgu = (const float *)TP("l%u.wgu.scale"); t->sd = (const float *)TP("l%u.wd.scale");
    }
    t->g_attn = (const float *)TP("l%u.g_attn"); t->g_ffn = (const float *)TP("l%u.g_ffn");
    t->kcache = TP("l%u.kcache"); t->vcache = TP("l%u.vcache");
    if (!t->wqkv || !t->wo || !t->wgu || !t->wd || !t->g_attn || !t->g_ffn || !t->kcache ||
        !t->vcache || (f8 && (!t->sqkv || !t->so || !t->sgu || !t->sd))) {
      free(tab);
      hb_set_error("decoder: layer %u tensors missing for the persistent step", l);
      return -1;
    }
  }
#undef TP
  const u32 tb = tens_new(d, "step.layers", THVM_DT_UINT8, (u64)NL * sizeof *tab);
  const int wrc = tb ? thvm_hip_buf_write(tb, tab, (u64)NL * sizeof *tab) : -1;
  free(tab);
  if (wrc) return -1;
  /* argmax partials per block, the grid-barrier words (zero-filled) */
  if (!tens_new(d, "step.pv", THVM_DT_FP32, (u64)B * nb * 4) ||
      !tens_new(d, "step.pi", THVM_DT_INT32, (u64)B * nb * 4) ||
      !tens_new(d, "step.sync", THVM_DT_UINT32, thvm_k_step_sync_bytes()))
    return -1;
  for (u32 i = 0; i < d->n_ops; i++) { free(d->ops[i].name); free(d->ops[i].prog); }
  d->n_ops = 0;
  char p[400];
  snprintf(p, sizeof p,
           "thvm-builtin:llama_step l=%u m=%u d=%u h=%u hkv=%u hd=%u f=%u v=%u maxseq=%u nsplit=%u "
           "wt=%u at=%u eps=%a scale=%a hstride=%u",
           NL, B, c->dim, c->n_heads, c->n_kv_heads, c->head_dim, c->ffn, c->vocab, c->max_seq,
           d->n_split, c->wdtype, c->adtype, c->eps, (float)(1.0 / sqrt((double)c->head_dim)),
           c->max_seq + 1);
  u32 a[24], n = 0;
  a[n++] = tb; a[n++] = tens_find(d, "emb"); a[n++] = tens_find(d, "norm_f"); a[n++] = tens_find(d, "lm");
  if (f8) a[n++] = tens_find(d, "lm.scale");
  a[n++] = tens_find(d, "rope.cos"); a[n++] = tens_find(d, "rope.sin"); a[n++] = tens_find(d, "tok");
  a[n++] = tens_find(d, "len"); a[n++] = tens_find(d, "hist"); a[n++] = tens_find(d, "logits");
  a[n++] = tens_find(d, "x"); a[n++] = tens_find(d, "q"); a[n++] = tens_find(d, "att");
  a[n++] = tens_find(d, "h"); a[n++] = tens_find(d, "attn.part"); a[n++] = tens_find(d, "step.pv");
  a[n++] = tens_find(d, "step.pi"); a[n++] = tens_find(d, "step.sync");
  return op_add(d, "llama_step", p, a, n);
}

/* 0, or -1 when a persistent step of this decoder failed (a grid barrier
 * expired: the step's outputs are not valid) */
static int step_status(Decoder *d) {
  const u32 sy = tens_find(d, "step.sync");
  if (!sy) return 0;
  const u64 nbytes = thvm_k_step_sync_bytes();
  uint32_t *w = (uint32_t *)malloc(nbytes);
  if (!w) { hb_set_error("decoder: out of host memory"); return -1; }
  int rc = thvm_hip_buf_read(sy, w, nbytes);
  if (!rc && w[thvm_k_step_err_word()]) {
    hb_set_error("decoder: a persistent step failed (a grid barrier expired); its outputs are invalid");
    rc = -1;
  }
  free(w);
  return rc;
}

/* The LLAMA step's op list over the weights build_llama made, for d->rows
 * rows: the one-row (batch) step, or the speculative step (d->spec: draft,
 * S verify rows of one sequence, commit). */
static int llama_ops(Decoder *d) {
  const ThvmDecodeConfig *c = &d->c;
  u32 D = c->dim, H = c->n_heads, Hkv = c->n_kv_heads, hd = c->head_dim, F = c->ffn;
  u32 adt = c->adtype, B = d->rows;
  u32 nqkv = (H + 2 * Hkv) * hd;
  const int f8 = c->wdtype == THVM_DT_FP8E4M3;
  char p[400], nm[48];
  u32 x = act(d, "x"), q = act(d, "q"), att = act(d, "att"), hb = act(d, "h"),
      L = tens_find(d, "len");

  if (d->spec) {
    snprintf(p, sizeof p, "thvm-builtin:spec_draft s=%u v=%u hcap=%u forced=%u", B, c->vocab,
             c->max_seq + 1, c->spec_forced);
    u32 da[4] = {act(d, "ca"), act(d, "ce"), tens_find(d, "hist"), L};
    if (op_add(d, "spec_draft", p, da, 4)) return -1;
  }
  snprintf(p, sizeof p, "thvm-builtin:embed b=%u d=%u v=%u et=%u xt=%u", B, D, c->vocab, adt, adt);
  u32 ea[3] = {x, tens_find(d, "emb"), d->spec ? act(d, "ce") : tens_find(d, "tok")};
  if (op_add(d, "embed", p, ea, 3)) return -1;

  for (u32 l = 0; l < c->n_layers; l++) {
    d->cur_tag = (int32_t)(2 * l);
#define LT(fmt) (snprintf(nm, sizeof nm, fmt, l), tens_find(d, nm))
    const u32 wqkv = LT("l%u.wqkv"), wo = LT("l%u.wo"), wgu = LT("l%u.wgu"), wd = LT("l%u.wd");
    const u32 sqkv = f8 ? LT("l%u.wqkv.scale") : 0, so = f8 ? LT("l%u.wo.scale") : 0,
              sgu = f8 ? LT("l%u.wgu.scale") : 0, sd = f8 ? LT("l%u.wd.scale") : 0;
    const u32 ga = LT("l%u.g_attn"), gf = LT("l%u.g_ffn"), kc = LT("l%u.kcache"), vc = LT("l%u.vcache");
#undef LT

    char nsp[96];
    u32 gin, gargs[2], ng;
    NormSpec n1 = {1, ga, 0};
    if (emit_norm(d, &n1, &gin, nsp, sizeof nsp, gargs, &ng)) return -1;
    snprintf(p, sizeof p,
             "thvm-builtin:gemv m=%u n=%u k=%u wt=%u xt=%u yt=%u epi=%u h=%u hkv=%u hd=%u maxseq=%u%s%s",
             B, nqkv, D, c->wdtype, adt, adt, THVM_EPI_QKV_ROPE, H, Hkv, hd, c->max_seq, nsp,
             d->spec ? " spec=1" : "");
    u32 qa[12], qn = 0;
    qa[qn++] = q; qa[qn++] = gin; qa[qn++] = wqkv;
    if (f8) qa[qn++] = sqkv;
    for (u32 i = 0; i < ng; i++) qa[qn++] = gargs[i];
    qa[qn++] = tens_find(d, "rope.cos"); qa[qn++] = tens_find(d, "rope.sin");
    qa[qn++] = L; qa[qn++] = kc; qa[qn++] = vc;
    if (op_add(d, "gemv_qkv", p, qa, qn)) return -1;

    if (op_attn(d, l)) return -1;

    snprintf(p, sizeof p, "thvm-builtin:gemv m=%u n=%u k=%u wt=%u xt=%u yt=%u epi=%u", B, D, H * hd,
             c->wdtype, adt, adt, THVM_EPI_RESID);
    u32 oa[6], on = 0;
    oa[on++] = x; oa[on++] = att; oa[on++] = wo;
    if (f8) oa[on++] = so;
    oa[on++] = x;
    if (op_add(d, "gemv_o", p, oa, on)) return -1;

    d->cur_tag = (int32_t)(2 * l + 1);
    NormSpec n2 = {1, gf, 0};
    if (emit_norm(d, &n2, &gin, nsp, sizeof nsp, gargs, &ng)) return -1;
    snprintf(p, sizeof p, "thvm-builtin:gemv m=%u n=%u k=%u wt=%u xt=%u yt=%u epi=%u%s", B, 2 * F,
             D, c->wdtype, adt, adt, THVM_EPI_SWIGLU, nsp);
    u32 ga2[7], gn = 0;
    ga2[gn++] = hb; ga2[gn++] = gin; ga2[gn++] = wgu;
    if (f8) ga2[gn++] = sgu;
    for (u32 i = 0; i < ng; i++) ga2[gn++] = gargs[i];
    if (op_add(d, "gemv_gateup", p, ga2, gn)) return -1;

    snprintf(p, sizeof p, "thvm-builtin:gemv m=%u n=%u k=%u wt=%u xt=%u yt=%u epi=%u", B, D, F,
             c->wdtype, adt, adt, THVM_EPI_RESID);
    u32 da[6], dn = 0;
    da[dn++] = x; da[dn++] = hb; da[dn++] = wd;
    if (f8) da[dn++] = sd;
    da[dn++] = x;
    if (op_add(d, "gemv_down", p, da, dn)) return -1;
  }
  d->cur_tag = -2;
  NormSpec nf = {1, tens_find(d, "norm_f"), 0};
  const int rc = op_tail(d, tens_find(d, "lm"), f8 ? tens_find(d, "lm.scale") : 0, &nf);
  d->cur_tag = -1;
  return rc;
}

/* The speculative step (reference step_build_spec, bench/dsv2_decode_bench.c:
 * 2419-2620): its own S-row activations ("s." tensors), the one-row step's
 * weights, caches, token history and length; built as a second op list. */
static int build_llama_spec(Decoder *d) {
  const ThvmDecodeConfig *c = &d->c;
  const u32 S = c->spec_rows, adt = c->adtype, as = hb_dt_size(adt);
  const u32 hq = c->n_heads * c->head_dim;
  if (!tens_new(d, "s.x", adt, (u64)S * c->dim * as) || !tens_new(d, "s.xn", adt, (u64)S * c->dim * as) ||
      !tens_new(d, "s.q", adt, (u64)S * hq * as) || !tens_new(d, "s.att", adt, (u64)S * hq * as) ||
      !tens_new(d, "s.h", adt, (u64)S * c->ffn * as) ||
      !tens_new(d, "s.logits", THVM_DT_FP32, (u64)S * c->vocab * 4) ||
      !tens_new(d, "s.am.pv", THVM_DT_FP32, (u64)S * 256 * 4) ||
      !tens_new(d, "s.am.pi", THVM_DT_INT32, (u64)S * 256 * 4) ||
      !tens_new(d, "s.am", THVM_DT_INT32, (u64)S * 4) || !tens_new(d, "s.ca", THVM_DT_INT32, (u64)S * 4) ||
      !tens_new(d, "s.ce", THVM_DT_INT32, (u64)S * 4) ||
      !tens_new(d, "s.attn.part", THVM_DT_FP32,
                thvm_k_attn_part_bytes(S, c->n_heads, c->n_kv_heads, c->head_dim, d->n_split)))
    return -1;
  DOp *ops = d->ops;
  const u32 n = d->n_ops, cap = d->cap_ops;
  d->ops = NULL;
  d->n_ops = d->cap_ops = 0;
  d->rows = S;
  d->spec = 1;
  snprintf(d->pfx, sizeof d->pfx, "s.");
  const int rc = llama_ops(d);
  d->sops = d->ops;
  d->n_sops = d->n_ops;
  d->ops = ops;
  d->n_ops = n;
  d->cap_ops = cap;
  d->rows = c->batch;
  d->spec = 0;
  d->pfx[0] = 0;
  return rc;
}

static int build_llama(Decoder *d) {
  const ThvmDecodeConfig *c = &d->c;
  u32 D = c->dim, H = c->n_heads, Hkv = c->n_kv_heads, hd = c->head_dim, F = c->ffn;
  u32 nqkv = (H + 2 * Hkv) * hd;
  if (build_state(d)) return -1;
  if (!weight_normal(d, "emb", c->adtype, (u64)c->vocab * D, 0.0f, c->init_std)) return -1;
  if (rope_tables(d)) return -1;
  if (!weight_const(d, "norm_f", D, 1.0f)) return -1;
  char nm[48];
  for (u32 l = 0; l < c->n_layers; l++) {
    u32 w, sc;
    snprintf(nm, sizeof nm, "l%u.wqkv", l);
    if (weight_matrix(d, nm, nqkv, D, &w, &sc)) return -1;
    snprintf(nm, sizeof nm, "l%u.wo", l);
    if (weight_matrix(d, nm, D, H * hd, &w, &sc)) return -1;
    snprintf(nm, sizeof nm, "l%u.wgu", l);
    if (weight_matrix(d, nm, 2 * F, D, &w, &sc)) return -1;
    snprintf(nm, sizeof nm, "l%u.wd", l);
    if (weight_matrix(d, nm, D, F, &w, &sc)) return -1;
    snprintf(nm, sizeof nm, "l%u.g_attn", l);
    if (!weight_const(d, nm, D, 1.0f)) return -1;
    snprintf(nm, sizeof nm, "l%u.g_ffn", l);
    if (!weight_const(d, nm, D, 1.0f)) return -1;
  }
  u32 lw, ls;
  if (weight_matrix(d, "lm", c->vocab, D, &lw, &ls)) return -1;
  if (llama_ops(d)) return -1;
  if (c->spec_rows && build_llama_spec(d)) return -1;
  return c->step_mode ? build_llama_step(d) : 0;
}

static int build_gpt2(Decoder *d) {
  const ThvmDecodeConfig *c = &d->c;
  u32 D = c->dim, H = c->n_heads, hd = c->head_dim, F = c->ffn, B = c->batch;
  u32 adt = c->adtype, wdt = c->wdtype;
  if (H * hd != D) { hb_set_error("decoder: GPT2 needs n_heads*head_dim == dim"); return -1; }
  if (build_state(d)) return -1;
  u32 wte = weight_normal(d, "wte", adt, (u64)c->vocab * D, 0.0f, c->init_std);
  u32 wpe = weight_normal(d, "wpe", adt, (u64)c->max_seq * D, 0.0f, c->init_std);
  u32 gf = weight_const(d, "lnf.g", D, 1.0f), bf = weight_const(d, "lnf.b", D, 0.0f);
  if (!wte || !wpe || !gf || !bf) return -1;
  char p[400], nm[48];
  u32 x = tens_find(d, "x"), q = tens_find(d, "q"),
      att = tens_find(d, "att"), hb = tens_find(d, "h"), L = tens_find(d, "len");

  snprintf(p, sizeof p, "thvm-builtin:embed b=%u d=%u v=%u et=%u xt=%u pos=1 maxseq=%u", B, D,
           c->vocab, adt, adt, c->max_seq);
  u32 ea[5] = {x, wte, tens_find(d, "tok"), wpe, L};
  if (op_add(d, "embed", p, ea, 5)) return -1;

  for (u32 l = 0; l < c->n_layers; l++) {
    d->cur_tag = (int32_t)(2 * l);
    u32 wqkv, wo, wfc, wpr, s_unused;
    snprintf(nm, sizeof nm, "l%u.c_attn", l);
    if (weight_matrix(d, nm, 3 * D, D, &wqkv, &s_unused)) return -1;
    snprintf(nm, sizeof nm, "l%u.c_attn.b", l);
    u32 bqkv = weight_normal(d, nm, adt, 3 * D, 0.0f, c->init_std);
    snprintf(nm, sizeof nm, "l%u.c_proj", l);
    if (weight_matrix(d, nm, D, D, &wo, &s_unused)) return -1;
    snprintf(nm, sizeof nm, "l%u.c_proj.b", l);
    u32 bo = weight_normal(d, nm, adt, D, 0.0f, c->init_std);
    snprintf(nm, sizeof nm, "l%u.c_fc", l);
    if (weight_matrix(d, nm, F, D, &wfc, &s_unused)) return -1;
    snprintf(nm, sizeof nm, "l%u.c_fc.b", l);
    u32 bfc = weight_normal(d, nm, adt, F, 0.0f, c->init_std);
    snprintf(nm, sizeof nm, "l%u.mlp_proj", l);
    if (weight_matrix(d, nm, D, F, &wpr, &s_unused)) return -1;
    snprintf(nm, sizeof nm, "l%u.mlp_proj.b", l);
    u32 bpr = weight_normal(d, nm, adt, D, 0.0f, c->init_std);
    snprintf(nm, sizeof nm, "l%u.ln1.g", l);
    u32 g1 = weight_const(d, nm, D, 1.0f);
    snprintf(nm, sizeof nm, "l%u.ln1.b", l);
    u32 b1 = weight_const(d, nm, D, 0.0f);
    snprintf(nm, sizeof nm, "l%u.ln2.g", l);
    u32 g2 = weight_const(d, nm, D, 1.0f);
    snprintf(nm, sizeof nm, "l%u.ln2.b", l);
    u32 b2 = weight_const(d, nm, D, 0.0f);
    if (!bqkv || !bo || !bfc || !bpr || !g1 || !b1 || !g2 || !b2) return -1;
    d->weight_bytes += (u64)(3 * D + D + F + D) * hb_dt_size(adt);
    char kn[32], vn[32];
    snprintf(kn, sizeof kn, "l%u.kcache", l);
    snprintf(vn, sizeof vn, "l%u.vcache", l);

    char nsp[96];
    u32 gin, gargs[2], ng;
    NormSpec n1 = {2, g1, b1};
    if (emit_norm(d, &n1, &gin, nsp, sizeof nsp, gargs, &ng)) return -1;
    snprintf(p, sizeof p,
             "thvm-builtin:gemv m=%u n=%u k=%u wt=%u xt=%u yt=%u epi=%u bias=1 h=%u hkv=%u hd=%u maxseq=%u%s",
             B, 3 * D, D, wdt, adt, adt, THVM_EPI_QKV, H, H, hd, c->max_seq, nsp);
    u32 qa[10], qn = 0;
    qa[qn++] = q; qa[qn++] = gin; qa[qn++] = wqkv;
    for (u32 i = 0; i < ng; i++) qa[qn++] = gargs[i];
    qa[qn++] = bqkv; qa[qn++] = L; qa[qn++] = tens_find(d, kn); qa[qn++] = tens_find(d, vn);
    if (op_add(d, "gemv_qkv", p, qa, qn)) return -1;
    if (op_attn(d, l)) return -1;
    snprintf(p, sizeof p, "thvm-builtin:gemv m=%u n=%u k=%u wt=%u xt=%u yt=%u epi=%u bias=1", B, D,
             D, wdt, adt, adt, THVM_EPI_RESID);
    u32 oa[5] = {x, att, wo, bo, x};
    if (op_add(d, "gemv_o", p, oa, 5)) return -1;
    d->cur_tag = (int32_t)(2 * l + 1);
    NormSpec n2 = {2, g2, b2};
    if (emit_norm(d, &n2, &gin, nsp, sizeof nsp, gargs, &ng)) return -1;
    snprintf(p, sizeof p, "thvm-builtin:gemv m=%u n=%u k=%u wt=%u xt=%u yt=%u epi=%u bias=1%s", B,
             F, D, wdt, adt, adt, THVM_EPI_GELU, nsp);
    u32 fa[6], fn = 0;
    fa[fn++] = hb; fa[fn++] = gin; fa[fn++] = wfc;
    for (u32 i = 0; i < ng; i++) fa[fn++] = gargs[i];
    fa[fn++] = bfc;
    if (op_add(d, "gemv_fc", p, fa, fn)) return -1;
    snprintf(p, sizeof p, "thvm-builtin:gemv m=%u n=%u k=%u wt=%u xt=%u yt=%u epi=%u bias=1", B, D,
             F, wdt, adt, adt, THVM_EPI_RESID);
    u32 pa[5] = {x, hb, wpr, bpr, x};
    if (op_add(d, "gemv_proj", p, pa, 5)) return -1;
  }
  d->weight_bytes += (u64)c->vocab * D * hb_dt_size(adt);   /* tied LM head */
  d->cur_tag = -2;
  NormSpec nf = {2, gf, bf};
  const int rc = op_tail(d, wte, 0, &nf);
  d->cur_tag = -1;
  return rc;
}

/* ---- DeepSeek-V2 (MLA + MoE), the C5 shape ------------------------------
 * Step (reference bench/dsv2_decode_bench.c step_build :2328-2411): embed ->
 * per layer [RMSNorm + q|kv GEMV -> mla_prep -> mla_attn (split + merge +
 * W_uv) -> o GEMV + residual -> post-attention RMSNorm -> dense SwiGLU FFN
 * (first_dense layers) or router GEMV + route + expert gate/up + expert down
 * with residual] -> final RMSNorm (f32) -> LM head -> argmax -> len_bump. */

/* YaRN-corrected RoPE tables for the pe dims, [max_seq][d_rope/2]: the
 * DeepSeek-V2-Lite rope scaling (factor 40 over an original 4096-position
 * window, beta_fast 32, beta_slow 1), as the reference builds them
 * (rope_tables :312-343). */
static int rope_tables_yarn(Decoder *d) {
  const u32 dr = d->c.d_rope, half = dr / 2, ms = d->c.max_seq;
  const double theta = d->c.rope_theta > 0.0f ? (double)d->c.rope_theta : 10000.0;
  const double factor = 40.0, orig = 4096.0, beta_fast = 32.0, beta_slow = 1.0;
  double lo = floor(dr * log(orig / (beta_fast * 2.0 * M_PI)) / (2.0 * log(theta)));
  double hi = ceil(dr * log(orig / (beta_slow * 2.0 * M_PI)) / (2.0 * log(theta)));
  if (lo < 0.0) lo = 0.0;
  if (hi > dr - 1.0) hi = dr - 1.0;
  const double span = (hi - lo) > 1e-3 ? (hi - lo) : 1e-3;
  u64 n = (u64)ms * half;
  float *cs = (float *)malloc(n * 4), *sn = (float *)malloc(n * 4);
  if (!cs || !sn) { free(cs); free(sn); hb_set_error("decoder: out of host memory"); return -1; }
  for (u32 j = 0; j < half; j++) {
    const double inv = 1.0 / pow(theta, (double)(2 * j) / (double)dr);
    double ramp = ((double)j - lo) / span;
    ramp = ramp < 0.0 ? 0.0 : ramp > 1.0 ? 1.0 : ramp;
    const double f = (inv / factor) * ramp + inv * (1.0 - ramp);
    for (u32 p = 0; p < ms; p++) {
      cs[(u64)p * half + j] = (float)cos((double)p * f);
      sn[(u64)p * half + j] = (float)sin((double)p * f);
    }
  }
  u32 ci = tens_new(d, "rope.cos", THVM_DT_FP32, n * 4);
  u32 si = tens_new(d, "rope.sin", THVM_DT_FP32, n * 4);
  int rc = (!ci || !si || thvm_hip_buf_write(ci, cs, n * 4) || thvm_hip_buf_write(si, sn, n * 4)) ? -1 : 0;
  free(cs);
  free(sn);
  return rc;
}

/* softmax scale with the YaRN mscale correction: (dn+dr)^-1/2 * mscale^2,
 * mscale = 0.1 * 0.707 * ln(40) + 1 (reference cfg_init :141-147) */
static float dsv2_scale(const ThvmDecodeConfig *c) {
  const double ms = 0.1 * 0.707 * log(40.0) + 1.0;
  return (float)(pow((double)(c->d_nope + c->d_rope), -0.5) * ms * ms);
}

static int build_dsv2(Decoder *d) {
  const ThvmDecodeConfig *c = &d->c;
  const u32 D = c->dim, H = c->n_heads, dn = c->d_nope, dr = c->d_rope, kv = c->kv_lora;
  const u32 dv = c->d_v, E = c->n_experts, K = c->top_k, I = c->moe_inter, F = c->ffn;
  const u32 S = c->n_shared * I, B = c->batch, V = c->vocab, wdt = c->wdtype;
  const u32 nqkv = H * (dn + dr) + kv + dr, P = K * I + S;
  const int f8 = wdt == THVM_DT_FP8E4M3;
  const float scale = dsv2_scale(c);
  d->n_split = (c->max_seq + 63) / 64;
  if (!tens_new(d, "tok", THVM_DT_INT32, (u64)B * 4) || !tens_new(d, "len", THVM_DT_INT32, 4) ||
      !tens_new(d, "hist", THVM_DT_INT32, (u64)B * (c->max_seq + 1) * 4) ||
      !tens_new(d, "logits", THVM_DT_FP32, (u64)B * V * 4) ||
      !tens_new(d, "am.pv", THVM_DT_FP32, (u64)B * 256 * 4) ||
      !tens_new(d, "am.pi", THVM_DT_INT32, (u64)B * 256 * 4) ||
      !tens_new(d, "x", THVM_DT_BF16, (u64)B * D * 2) || !tens_new(d, "xn", THVM_DT_BF16, (u64)B * D * 2) ||
      !tens_new(d, "qkv", THVM_DT_BF16, (u64)B * nqkv * 2) ||
      !tens_new(d, "qlat", THVM_DT_FP32, (u64)B * H * kv * 4) ||
      !tens_new(d, "qpe", THVM_DT_BF16, (u64)B * H * dr * 2) ||
      !tens_new(d, "o", THVM_DT_BF16, (u64)B * H * dv * 2) ||
      !tens_new(d, "xnf", THVM_DT_FP32, (u64)B * D * 4) ||
      !tens_new(d, "hmoe", THVM_DT_FP32, (u64)B * P * 4) ||
      !tens_new(d, "h", THVM_DT_BF16, (u64)B * (F ? F : 1) * 2) ||
      !tens_new(d, "mla.part", THVM_DT_FP32, thvm_k_mla_part_bytes(B, H, kv, d->n_split)))
    return -1;
  /* one row: the MLA merge in latent quarters (4 blocks per head instead of
   * 2, each reading a quarter of the head's partials), its four f32 quarter
   * sums added, scaled by the W_uv row scales and rounded to bf16 where the
   * o projection's GEMV stages x (norm=3); "o" then stays unwritten */
  const int oqm = B == 1 && kv % 64 == 0;
  if (oqm && !tens_new(d, "o4", THVM_DT_FP32, (u64)4 * B * H * dv * 4)) return -1;
  /* batches above 4 rows: expert-grouped MoE scratch and its live-expert
   * counter; projections on the MFMA GEMM (bf16 inputs from separate norms) */
  /* (the MFMA form takes D in multiples of 128 and I, S of 64 for fp8
   * weights, 64 and 32 for bf16; other shapes run the VALU form) */
  const u32 mk = wdt == THVM_DT_FP8E4M3 ? 128 : 64;
  const int grp = B <= 4 ? 0 : (c->moe_mode == 1 || D % mk || I % (mk / 2) || S % (mk / 2)) ? 1 : 2;
  if (grp && (!tens_new(d, "moe.plan", THVM_DT_INT32, thvm_k_moe_plan_bytes(B, E, K)) ||
              !tens_new(d, "moe.part", THVM_DT_FP32, thvm_k_moe_part_bytes(B, K, D)) ||
              !tens_new(d, "moe.live", THVM_DT_INT32, 4)))
    return -1;
  if (!weight_normal(d, "emb", THVM_DT_BF16, (u64)V * D, 0.0f, c->init_std)) return -1;
  if (rope_tables_yarn(d) || !weight_const(d, "norm_f", D, 1.0f)) return -1;
  char p[512], nm[48];
  const u32 x = tens_find(d, "x"), L = tens_find(d, "len"), qkv = tens_find(d, "qkv");
  const u32 qlat = tens_find(d, "qlat"), qpe = tens_find(d, "qpe"), o = tens_find(d, "o");
  const u32 xnf = tens_find(d, "xnf"), hmoe = tens_find(d, "hmoe"), hd = tens_find(d, "h");
  const u32 cosb = tens_find(d, "rope.cos"), sinb = tens_find(d, "rope.sin");

  snprintf(p, sizeof p, "thvm-builtin:embed b=%u d=%u v=%u et=%u xt=%u", B, D, V, THVM_DT_BF16,
           THVM_DT_BF16);
  u32 ea[3] = {x, tens_find(d, "emb"), tens_find(d, "tok")};
  if (op_add(d, "embed", p, ea, 3)) return -1;

  for (u32 l = 0; l < c->n_layers; l++) {
    d->cur_tag = (int32_t)(2 * l);
    u32 wqkv, sqkv, wuk, suk, wuv, suv, wo, so;
#define WM(nmfmt, rows, cols, w, s) \
    do { snprintf(nm, sizeof nm, nmfmt, l); if (weight_matrix(d, nm, rows, cols, w, s)) return -1; } while (0)
    WM("l%u.wqkv", nqkv, D, &wqkv, &sqkv);
    WM("l%u.wuk", H * kv, dn, &wuk, &suk);
    WM("l%u.wuv", H * dv, kv, &wuv, &suv);
    WM("l%u.wo", D, H * dv, &wo, &so);
    snprintf(nm, sizeof nm, "l%u.win", l);
    const u32 win = weight_const(d, nm, D, 1.0f);
    snprintf(nm, sizeof nm, "l%u.wkvn", l);
    const u32 wkvn = weight_const(d, nm, kv, 1.0f);
    snprintf(nm, sizeof nm, "l%u.wpost", l);
    const u32 wpost = weight_const(d, nm, D, 1.0f);
    char cn[32], pn[32];
    snprintf(cn, sizeof cn, "l%u.ckv", l);
    snprintf(pn, sizeof pn, "l%u.kpe", l);
    const u32 ckv = tens_new(d, cn, THVM_DT_BF16, (u64)B * c->max_seq * kv * 2);
    const u32 kpe = tens_new(d, pn, THVM_DT_BF16, (u64)B * c->max_seq * dr * 2);
    if (!win || !wkvn || !wpost || !ckv || !kpe) return -1;

    /* RMSNorm (rms1) fused into the q|kv projection, output rounded to bf16 */
    char nsp[96];
    u32 gin, gargs[2], ng;
    NormSpec n1 = {1, win, 0};
    if (emit_norm(d, &n1, &gin, nsp, sizeof nsp, gargs, &ng)) return -1;
    snprintf(p, sizeof p, "thvm-builtin:gemv m=%u n=%u k=%u wt=%u xt=%u yt=%u epi=0%s", B, nqkv, D,
             wdt, THVM_DT_BF16, THVM_DT_BF16, nsp);
    u32 qa[8], qn = 0;
    qa[qn++] = qkv; qa[qn++] = gin; qa[qn++] = wqkv;
    if (f8) qa[qn++] = sqkv;
    for (u32 i = 0; i < ng; i++) qa[qn++] = gargs[i];
    if (op_add(d, "gemv_qkv", p, qa, qn)) return -1;

    snprintf(p, sizeof p, "thvm-builtin:mla_prep b=%u h=%u dn=%u dr=%u kv=%u dv=%u maxseq=%u wt=%u eps=%a",
             B, H, dn, dr, kv, dv, c->max_seq, wdt, c->eps);
    u32 pa[12], pnn = 0;
    pa[pnn++] = qkv; pa[pnn++] = wuk;
    if (f8) pa[pnn++] = suk;
    pa[pnn++] = wkvn; pa[pnn++] = cosb; pa[pnn++] = sinb; pa[pnn++] = L;
    pa[pnn++] = ckv; pa[pnn++] = kpe; pa[pnn++] = qlat; pa[pnn++] = qpe;
    if (op_add(d, "mla_prep", p, pa, pnn)) return -1;

    /* attn_cpb > 0 also sets the MFMA latent split's chunks per block */
    const u32 o4 = oqm ? tens_find(d, "o4") : 0;
    snprintf(p, sizeof p,
             "thvm-builtin:mla_attn b=%u h=%u dn=%u dr=%u kv=%u dv=%u maxseq=%u nsplit=%u wt=%u scale=%a cpb=%u oq=%u",
             B, H, dn, dr, kv, dv, c->max_seq, d->n_split, wdt, scale, c->attn_cpb, oqm ? 1u : 0u);
    u32 aa[10], an = 0;
    aa[an++] = oqm ? o4 : o; aa[an++] = qlat; aa[an++] = qpe; aa[an++] = ckv; aa[an++] = kpe; aa[an++] = L;
    aa[an++] = tens_find(d, "mla.part"); aa[an++] = wuv;
    if (f8) aa[an++] = suv;
    if (op_add(d, "mla_attn", p, aa, an)) return -1;

    if (oqm)
      snprintf(p, sizeof p, "thvm-builtin:gemv m=%u n=%u k=%u wt=%u xt=%u yt=%u epi=%u norm=3 xqs=%u ngain=%u",
               B, D, H * dv, wdt, THVM_DT_BF16, THVM_DT_BF16, THVM_EPI_RESID, B * H * dv, f8 ? 1u : 0u);
    else
      snprintf(p, sizeof p, "thvm-builtin:gemv m=%u n=%u k=%u wt=%u xt=%u yt=%u epi=%u", B, D, H * dv,
               wdt, THVM_DT_BF16, THVM_DT_BF16, THVM_EPI_RESID);
    u32 oa[7], on = 0;
    oa[on++] = x; oa[on++] = oqm ? o4 : o; oa[on++] = wo;
    if (f8) oa[on++] = so;
    if (oqm && f8) oa[on++] = suv;                 /* the W_uv row scales as the gain */
    oa[on++] = x;
    if (op_add(d, "gemv_o", p, oa, on)) return -1;

    d->cur_tag = (int32_t)(2 * l + 1);
    if (l < c->first_dense) {   /* dense SwiGLU FFN with the post-attention norm fused */
      u32 wgu, sgu, wd, sd;
      WM("l%u.wgu", 2 * F, D, &wgu, &sgu);
      WM("l%u.wd", D, F, &wd, &sd);
      NormSpec n2 = {1, wpost, 0};
      if (emit_norm(d, &n2, &gin, nsp, sizeof nsp, gargs, &ng)) return -1;
      snprintf(p, sizeof p, "thvm-builtin:gemv m=%u n=%u k=%u wt=%u xt=%u yt=%u epi=%u%s", B, 2 * F,
               D, wdt, THVM_DT_BF16, THVM_DT_BF16, THVM_EPI_SWIGLU, nsp);
      u32 ga[7], gn = 0;
      ga[gn++] = hd; ga[gn++] = gin; ga[gn++] = wgu;
      if (f8) ga[gn++] = sgu;
      for (u32 i = 0; i < ng; i++) ga[gn++] = gargs[i];
      if (op_add(d, "gemv_gateup", p, ga, gn)) return -1;
      snprintf(p, sizeof p, "thvm-builtin:gemv m=%u n=%u k=%u wt=%u xt=%u yt=%u epi=%u", B, D, F, wdt,
               THVM_DT_BF16, THVM_DT_BF16, THVM_EPI_RESID);
      u32 da[6], dnn = 0;
      da[dnn++] = x; da[dnn++] = hd; da[dnn++] = wd;
      if (f8) da[dnn++] = sd;
      da[dnn++] = x;
      if (op_add(d, "gemv_down", p, da, dnn)) return -1;
      continue;
    }
    /* MoE: post-attention norm in f32 (router input), router GEMV, top-K */
    snprintf(nm, sizeof nm, "l%u.gate", l);
    const u32 gate = weight_normal(d, nm, THVM_DT_FP32, (u64)E * D, 0.0f, c->init_std);
    if (!gate) return -1;
    d->weight_bytes += (u64)E * D * 4;
    /* each MoE layer keeps its router logits, selected experts and their
     * probabilities (readable after a step: l<i>.gate_logits/.sel/.probs) */
    snprintf(nm, sizeof nm, "l%u.gate_logits", l);
    const u32 gl = tens_new(d, nm, THVM_DT_FP32, (u64)B * E * 4);
    snprintf(nm, sizeof nm, "l%u.sel", l);
    const u32 sel = tens_new(d, nm, THVM_DT_INT32, (u64)B * K * 4);
    snprintf(nm, sizeof nm, "l%u.probs", l);
    const u32 probs = tens_new(d, nm, THVM_DT_FP32, (u64)B * K * 4);
    if (!gl || !sel || !probs) return -1;
    u32 wgue, sgue, wde, sde, wgus = 0, sgus = 0, wds = 0, sds = 0;
    const u64 wb0 = d->weight_bytes;
    WM("l%u.wgu_e", E * 2 * I, D, &wgue, &sgue);
    WM("l%u.wd_e", E * D, I, &wde, &sde);
    /* only the selected experts stream per step: count K (of E) per row */
    {
      const u64 all = d->weight_bytes - wb0;
      const u32 used = K * B < E ? K * B : E;
      d->weight_bytes = wb0 + all / E * used;
    }
    if (S) {
      WM("l%u.wgu_s", 2 * S, D, &wgus, &sgus);
      WM("l%u.wd_s", D, S, &wds, &sds);
    }
#undef WM
    /* the norm (f32 out) and the f32 router GEMV in one launch, and the top-K
     * inside the per-row gate/up: bit for bit the norm -> GEMV -> route
     * kernels (THVM_HIP_SPLIT_ROUTER=1 runs those three for A/B) */
    const char *sr = getenv("THVM_HIP_SPLIT_ROUTER");
    const int fuse_rt = D <= 4096 && D % 4 == 0 && E <= 64 && !(sr && sr[0] == '1');
    const int route_in_gu = fuse_rt && !grp;
    if (fuse_rt) {
      snprintf(p, sizeof p, "thvm-builtin:moe_gate b=%u d=%u e=%u eps=%a", B, D, E, c->eps);
      u32 ra[5] = {xnf, gl, x, wpost, gate};
      if (op_add(d, "gate", p, ra, 5)) return -1;
    } else {
      snprintf(p, sizeof p, "thvm-builtin:norm m=%u k=%u xt=%u yt=%u eps=%a", B, D, THVM_DT_BF16,
               THVM_DT_FP32, c->eps);
      u32 na[3] = {xnf, x, wpost};
      if (op_add(d, "norm_post", p, na, 3)) return -1;
      snprintf(p, sizeof p, "thvm-builtin:gemv m=%u n=%u k=%u wt=%u xt=%u yt=%u epi=0", B, E, D,
               THVM_DT_FP32, THVM_DT_FP32, THVM_DT_FP32);
      u32 ra[3] = {gl, xnf, gate};
      if (op_add(d, "gemv_gate", p, ra, 3)) return -1;
    }
    if (!route_in_gu) {
      snprintf(p, sizeof p, "thvm-builtin:route b=%u e=%u k=%u", B, E, K);
      u32 rb[3] = {sel, probs, gl};
      if (op_add(d, "route", p, rb, 3)) return -1;
    }
    /* the MFMA grouped form reads tiled copies of the expert weights (see
     * tiled_copy; gate/up 32 bytes per lane, down 16) */
    const int mtile = grp == 2 && wtile_on() && (2 * I) % 16 == 0 && D % 16 == 0 && (2 * S) % 16 == 0 &&
                      ((u64)D * hb_dt_size(wdt)) % 128 == 0 && ((u64)I * hb_dt_size(wdt)) % 64 == 0 &&
                      ((u64)S * hb_dt_size(wdt)) % 64 == 0;
    if (mtile) {
      if (!(wgue = tiled_copy(d, wgue, E * 2 * I, D, wdt, 32))) return -1;
      if (!(wde = tiled_copy(d, wde, E * D, I, wdt, 16))) return -1;
      if (S && (!(wgus = tiled_copy(d, wgus, 2 * S, D, wdt, 32)) || !(wds = tiled_copy(d, wds, D, S, wdt, 16))))
        return -1;
    }
    snprintf(p, sizeof p, "thvm-builtin:moe_gateup b=%u d=%u e=%u k=%u i=%u s=%u wt=%u grouped=%d route=%d%s",
             B, D, E, K, I, S, wdt, grp, route_in_gu, mtile ? " tiled=1" : "");
    u32 ma[12], mn = 0;
    ma[mn++] = hmoe; ma[mn++] = xnf; ma[mn++] = sel; ma[mn++] = wgue;
    if (f8) ma[mn++] = sgue;
    if (S) { ma[mn++] = wgus; if (f8) ma[mn++] = sgus; }
    if (grp) { ma[mn++] = tens_find(d, "moe.plan"); ma[mn++] = tens_find(d, "moe.live"); }
    if (route_in_gu) { ma[mn++] = gl; ma[mn++] = probs; }
    if (op_add(d, "moe_gateup", p, ma, mn)) return -1;
    snprintf(p, sizeof p, "thvm-builtin:moe_down b=%u d=%u e=%u k=%u i=%u s=%u wt=%u grouped=%d%s", B, D, E,
             K, I, S, wdt, grp, mtile ? " tiled=1" : "");
    u32 mb[11], mbn = 0;
    mb[mbn++] = x; mb[mbn++] = hmoe; mb[mbn++] = sel; mb[mbn++] = probs; mb[mbn++] = wde;
    if (f8) mb[mbn++] = sde;
    if (S) { mb[mbn++] = wds; if (f8) mb[mbn++] = sds; }
    if (grp) { mb[mbn++] = tens_find(d, "moe.plan"); mb[mbn++] = tens_find(d, "moe.part"); }
    if (op_add(d, "moe_down", p, mb, mbn)) return -1;
  }
  /* final norm in f32 (rms_f) -> LM head; batches above 4 rows feed the
   * MFMA GEMM, which takes 16-bit x: their normed rows are rounded to bf16 */
  d->cur_tag = -2;
  u32 lw, ls;
  if (weight_matrix(d, "lm", V, D, &lw, &ls)) return -1;
  const u32 lmx = grp ? tens_find(d, "xn") : xnf, lmt = grp ? THVM_DT_BF16 : THVM_DT_FP32;
  snprintf(p, sizeof p, "thvm-builtin:norm m=%u k=%u xt=%u yt=%u eps=%a", B, D, THVM_DT_BF16, lmt, c->eps);
  u32 fa[3] = {lmx, x, tens_find(d, "norm_f")};
  if (op_add(d, "norm_f", p, fa, 3)) return -1;
  snprintf(p, sizeof p, "thvm-builtin:gemv m=%u n=%u k=%u wt=%u xt=%u yt=%u epi=0", B, V, D, wdt, lmt,
           THVM_DT_FP32);
  u32 la[4], ln = 0;
  la[ln++] = tens_find(d, "logits"); la[ln++] = lmx; la[ln++] = lw;
  if (f8) la[ln++] = ls;
  if (op_add(d, "lm_head", p, la, ln)) return -1;
  const u32 nb = V >= 256 * 64 ? 256 : (V + 63) / 64;
  char sk[96];
  snprintf(p, sizeof p, "thvm-builtin:argmax b=%u v=%u nb=%u hist=1 hstride=%u%s", B, V, nb,
           c->max_seq + 1, sample_keys(c, sk, sizeof sk));
  u32 am[6] = {tens_find(d, "tok"), tens_find(d, "logits"), tens_find(d, "am.pv"),
               tens_find(d, "am.pi"), tens_find(d, "hist"), L};
  if (op_add(d, "argmax", p, am, 6)) return -1;
  const int rc = op_add(d, "len_bump", "thvm-builtin:len_bump delta=1", &L, 1);
  d->cur_tag = -1;
  return rc;
}

THVM_API int thvm_hip_decoder_sync_weights(uint32_t h, const char *name) {
  Decoder *d = dec_get(h);
  if (!d) return -1;
  const u32 src = name ? tens_find(d, name) : 0;
  if (name && !src) { hb_set_error("decoder_sync_weights: no tensor %s", name); return -1; }
  for (u32 i = 0; i < d->n_tiles; i++)
    if (!name || d->tiles[i].src == src)
      if (tile_run(d, i)) return -1;
  return 0;
}

THVM_API void thvm_hip_decoder_destroy(uint32_t h) {
  Decoder *d = dec_get(h);
  if (d) dec_free(d);
}

void hb_decoder_reset(void) {
  for (u32 i = 0; i < MAX_DEC; i++)
    if (DEC[i].used) dec_free(&DEC[i]);
}

THVM_API int thvm_hip_decoder_set_state(uint32_t h, const int32_t *tokens, uint32_t pos) {
  Decoder *d = dec_get(h);
  if (!d) return -1;
  if (pos >= d->c.max_seq) { hb_set_error("decoder_set_state: pos %u >= max_seq %u", pos, d->c.max_seq); return -1; }
  for (u32 b = 0; b < d->c.batch; b++)
    if (tokens[b] < 0 || (u32)tokens[b] >= d->c.vocab) {
      hb_set_error("decoder_set_state: token %d of row %u outside [0, %u)", tokens[b], b, d->c.vocab);
      return -1;
    }
  int32_t L = (int32_t)pos + 1;
  if (thvm_hip_buf_write(tens_find(d, "tok"), tokens, (u64)d->c.batch * 4)) return -1;
  if (thvm_hip_buf_write(tens_find(d, "len"), &L, 4)) return -1;
  u32 hist = tens_find(d, "hist");
  for (u32 b = 0; b < d->c.batch; b++)
    if (thvm_hip_buf_write_at(hist, ((u64)b * (d->c.max_seq + 1) + pos) * 4, &tokens[b], 4)) return -1;
  return 0;
}

THVM_API int thvm_hip_decoder_prefill_synthetic(uint32_t h, uint32_t ctx, uint64_t seed) {
  Decoder *d = dec_get(h);
  if (!d) return -1;
  const ThvmDecodeConfig *c = &d->c;
  if (ctx >= c->max_seq) { hb_set_error("prefill: ctx %u >= max_seq", ctx); return -1; }
  char err[256];
  const int mla = c->arch == THVM_ARCH_DSV2;
  for (u32 l = 0; l < c->n_layers; l++) {
    char kn[32], vn[32];
    snprintf(kn, sizeof kn, mla ? "l%u.ckv" : "l%u.kcache", l);
    snprintf(vn, sizeof vn, mla ? "l%u.kpe" : "l%u.vcache", l);
    if (mla) {   /* latent rows [B][max_seq][kv] and pe rows [B][max_seq][dr] */
      void *kp = hb_buf_ptr(tens_find(d, kn)), *vp = hb_buf_ptr(tens_find(d, vn));
      if (!kp || !vp) { hb_set_error("prefill: cache missing"); return -1; }
      if (thvm_k_fill_cache(kp, c->adtype, c->batch, 1, c->max_seq, c->kv_lora, ctx, seed,
                            name_tag(kn), HB_STREAM, err, sizeof err) ||
          thvm_k_fill_cache(vp, c->adtype, c->batch, 1, c->max_seq, c->d_rope, ctx, seed,
                            name_tag(vn), HB_STREAM, err, sizeof err)) {
        hb_set_error("prefill: %s", err);
        return -1;
      }
      continue;
    }
    void *kp = hb_buf_ptr(tens_find(d, kn)), *vp = hb_buf_ptr(tens_find(d, vn));
    if (!kp || !vp) { hb_set_error("prefill: cache missing"); return -1; }
    if (thvm_k_fill_cache(kp, c->adtype, c->batch, c->n_kv_heads, c->max_seq, c->head_dim, ctx,
                          seed, name_tag(kn), HB_STREAM, err, sizeof err) ||
        thvm_k_fill_cache(vp, c->adtype, c->batch, c->n_kv_heads, c->max_seq, c->head_dim, ctx,
                          seed, name_tag(vn), HB_STREAM, err, sizeof err)) {
      hb_set_error("prefill: %s", err);
      return -1;
    }
  }
  int32_t L = (int32_t)ctx + 1;
  return thvm_hip_buf_write(tens_find(d, "len"), &L, 4);
}

static int run_list(const DOp *ops, u32 n);
static int dec_run_ops(Decoder *d) { return run_list(d->ops, d->n_ops); }

int hb_decoder_dims(u32 h, u32 *batch, u32 *max_seq, u32 *vocab) {
  Decoder *d = dec_get(h);
  if (!d) return -1;
  *batch = d->c.batch;
  *max_seq = d->c.max_seq;
  *vocab = d->c.vocab;
  return 0;
}
u32 hb_decoder_slot(u32 h) {
  Decoder *d = dec_get(h);
  return d ? d->jit_slot : 0;
}

THVM_API int thvm_hip_decoder_step(uint32_t h) {
  Decoder *d = dec_get(h);
  if (!d) return -1;
  if (thvm_hip_jit_is_capturing()) { hb_set_error("decoder_step: a JIT capture is open"); return -1; }
  return dec_run_ops(d);
}

THVM_API uint32_t thvm_hip_decoder_capture(uint32_t h) {
  Decoder *d = dec_get(h);
  if (!d) return 0;
  if (d->jit_slot) { thvm_hip_jit_capture_drop(d->jit_slot); d->jit_slot = 0; }
  u32 slot = thvm_hip_jit_capture_begin();
  if (!slot) return 0;
  int rc = dec_run_ops(d);
  thvm_hip_jit_capture_end();
  if (rc) { thvm_hip_jit_capture_drop(slot); return 0; }
  d->jit_slot = slot;
  return slot;
}

THVM_API int thvm_hip_decoder_replay(uint32_t h, uint32_t n) {
  Decoder *d = dec_get(h);
  if (!d) return -1;
  if (!d->jit_slot) { hb_set_error("decoder_replay: no captured step"); return -1; }
  for (u32 i = 0; i < n; i++)
    if (thvm_hip_jit_replay(d->jit_slot)) return -1;
  return 0;
}

static int run_list(const DOp *ops, u32 n) {
  for (u32 i = 0; i < n; i++) {
    const DOp *o = &ops[i];
    if (thvm_hip_dispatch_custom(o->name, o->prog, NULL, NULL, 0, o->args, o->n_args, o->outs))
      return -1;
  }
  return 0;
}

static Decoder *spec_get(uint32_t h, const char *who) {
  Decoder *d = dec_get(h);
  if (d && !d->n_sops) {
    hb_set_error("%s: decoder %u has no speculative step (spec_rows 0)", who, h);
    return NULL;
  }
  return d;
}

THVM_API int thvm_hip_decoder_spec_step(uint32_t h) {
  Decoder *d = spec_get(h, "decoder_spec_step");
  if (!d) return -1;
  if (thvm_hip_jit_is_capturing()) { hb_set_error("decoder_spec_step: a JIT capture is open"); return -1; }
  return run_list(d->sops, d->n_sops);
}

THVM_API uint32_t thvm_hip_decoder_spec_capture(uint32_t h) {
  Decoder *d = spec_get(h, "decoder_spec_capture");
  if (!d) return 0;
  if (d->spec_slot) { thvm_hip_jit_capture_drop(d->spec_slot); d->spec_slot = 0; }
  u32 slot = thvm_hip_jit_capture_begin();
  if (!slot) return 0;
  int rc = run_list(d->sops, d->n_sops);
  thvm_hip_jit_capture_end();
  if (rc) { thvm_hip_jit_capture_drop(slot); return 0; }
  d->spec_slot = slot;
  return slot;
}

THVM_API int thvm_hip_decoder_spec_replay(uint32_t h, uint32_t n) {
  Decoder *d = spec_get(h, "decoder_spec_replay");
  if (!d) return -1;
  if (!d->spec_slot) { hb_set_error("decoder_spec_replay: no captured speculative step"); return -1; }
  for (u32 i = 0; i < n; i++)
    if (thvm_hip_jit_replay(d->spec_slot)) return -1;
  return 0;
}

u32 hb_decoder_spec_rows(u32 h) {
  Decoder *d = dec_get(h);
  return d && d->n_sops ? d->c.spec_rows : 0;
}
u32 hb_decoder_spec_slot(u32 h) {
  Decoder *d = dec_get(h);
  return d ? d->spec_slot : 0;
}

THVM_API int thvm_hip_decoder_read_tokens(uint32_t h, int32_t *dst, uint32_t n) {
  Decoder *d = dec_get(h);
  if (!d || step_status(d)) return -1;
  u32 stride = d->c.max_seq + 1;
  if (n > stride) { hb_set_error("read_tokens: n %u > %u", n, stride); return -1; }
  int32_t *tmp = (int32_t *)malloc((u64)d->c.batch * stride * 4);
  if (!tmp) { hb_set_error("read_tokens: out of host memory"); return -1; }
  int rc = thvm_hip_buf_read(tens_find(d, "hist"), tmp, (u64)d->c.batch * stride * 4);
  if (!rc)
    for (u32 b = 0; b < d->c.batch; b++) memcpy(dst + (u64)b * n, tmp + (u64)b * stride, (u64)n * 4);
  free(tmp);
  return rc;
}

THVM_API int thvm_hip_decoder_read_logits(uint32_t h, float *dst, uint64_t nfloats) {
  Decoder *d = dec_get(h);
  if (!d || step_status(d)) return -1;
  u64 have = (u64)d->c.batch * d->c.vocab;
  if (nfloats > have) nfloats = have;
  return thvm_hip_buf_read(tens_find(d, "logits"), dst, nfloats * 4);
}

THVM_API uint32_t thvm_hip_decoder_position(uint32_t h) {
  Decoder *d = dec_get(h);
  if (!d) return 0;
  int32_t L = 0;
  if (thvm_hip_buf_read(tens_find(d, "len"), &L, 4)) return 0;
  return L > 0 ? (u32)(L - 1) : 0;
}

THVM_API uint32_t thvm_hip_decoder_tensor(uint32_t h, const char *name, uint32_t *dtype_out,
                                          uint64_t *nbytes_out) {
  Decoder *d = dec_get(h);
  if (!d || !name) return 0;
  for (u32 i = 0; i < d->nt; i++)
    if (strcmp(d->t[i].name, name) == 0) {
      if (dtype_out) *dtype_out = d->t[i].dt;
      if (nbytes_out) *nbytes_out = d->t[i].nbytes;
      return d->t[i].id;
    }
  hb_set_error("decoder_tensor: no tensor '%s'", name);
  return 0;
}

THVM_API uint64_t thvm_hip_decoder_step_bytes(uint32_t h) {
  Decoder *d = dec_get(h);
  if (!d) return 0;
  const ThvmDecodeConfig *c = &d->c;
  u32 pos = thvm_hip_decoder_position(h);
  u64 L = (u64)pos + 1;
  u64 as = hb_dt_size(c->adtype);
  /* K and V rows [0, L) of every layer and batch row, plus the new row written */
  u64 kv = 2ull * c->n_layers * c->batch * c->n_kv_heads * c->head_dim * as * (L + 1);
  if (c->arch == THVM_ARCH_DSV2)   /* latent + pe rows; experts counted as selected */
    kv = (u64)c->n_layers * c->batch * (c->kv_lora + c->d_rope) * as * (L + 1);
  return d->weight_bytes + kv;
}

THVM_API uint32_t thvm_hip_decoder_step_kernels(uint32_t h) {
  Decoder *d = dec_get(h);
  return d ? d->n_ops : 0;
}

THVM_API int thvm_hip_decoder_op_tags(uint32_t h, int32_t *tags, uint32_t n) {
  Decoder *d = dec_get(h);
  if (!d) return -1;
  if (!tags && n) { hb_set_error("decoder_op_tags: no output"); return -1; }
  const u32 m = n < d->n_ops ? n : d->n_ops;
  for (u32 i = 0; i < m; i++) tags[i] = d->ops[i].tag;
  return (int)d->n_ops;
}

THVM_API int thvm_hip_decoder_op_info(uint32_t h, uint32_t i, char *name, uint32_t name_cap,
                                      char *prog, uint32_t prog_cap, uint32_t *ids, uint32_t ids_cap) {
  Decoder *d = dec_get(h);
  if (!d) return -1;
  if (i >= d->n_ops) { hb_set_error("decoder_op_info: op %u of %u", i, d->n_ops); return -1; }
  const DOp *o = &d->ops[i];
  if (name && name_cap) snprintf(name, name_cap, "%s", o->name);
  if (prog && prog_cap) snprintf(prog, prog_cap, "%s", o->prog);
  for (u32 k = 0; ids && k < o->n_args && k < ids_cap; k++) ids[k] = o->args[k];
  return (int)o->n_args;
}

THVM_API int thvm_hip_decoder_run_ops(uint32_t h, uint32_t first, uint32_t count) {
  Decoder *d = dec_get(h);
  if (!d) return -1;
  if (thvm_hip_jit_is_capturing()) { hb_set_error("decoder_run_ops: a JIT capture is open"); return -1; }
  if (first > d->n_ops || count > d->n_ops - first) {
    hb_set_error("decoder_run_ops: ops [%u, %u + %u) outside the step's %u", first, first, count, d->n_ops);
    return -1;
  }
  return run_list(d->ops + first, count);
}

THVM_API int thvm_hip_decoder_stage_clock(uint32_t h, double *us_out, uint32_t n) {
  Decoder *d = dec_get(h);
  if (!d) return -1;
  const u32 sy = tens_find(d, "step.sync");
  if (!sy) return 0;
  const u64 nbytes = thvm_k_step_sync_bytes();
  uint32_t *w = (uint32_t *)malloc(nbytes);
  if (!w) { hb_set_error("stage_clock: out of host memory"); return -1; }
  if (thvm_hip_buf_read(sy, w, nbytes)) { free(w); return -1; }
  /* barrier openings (5 L + 2 slots), then 4 detail events per stage
   * (5 L + 1 stages): entry, barrier open, work done, stores drained */
  const u32 nb = d->c.n_layers * 5 + 2, ns = d->c.n_layers * 5 + 1;
  const u32 base = thvm_k_step_clock_word(), dbase = thvm_k_step_dclock_word();
  const u32 slots = nb + 4 * ns;
  const uint64_t t0 = (uint64_t)w[base] | ((uint64_t)w[base + 1] << 32);
  for (u32 i = 0; i < slots && i < n; i++) {
    const u32 wi = i < nb ? base + 2 * i : dbase + 2 * (i - nb);
    const uint64_t t = (uint64_t)w[wi] | ((uint64_t)w[wi + 1] << 32);
    us_out[i] = (double)(int64_t)(t - t0) / 100.0;   /* 100 MHz wall clock */
  }
  free(w);
  return (int)slots;
}
