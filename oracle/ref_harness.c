/* ref_harness.c -- TEST INFRASTRUCTURE ONLY.  Compiles the reference thvm
 * translation unit where it lies (/root/reference/src/thvm.c, the single-TU
 * build every reference test uses: tests/test_*.c `#include "../src/thvm.c"`)
 * and exports a few of its CPU-path entry points with C linkage, so the
 * oracle restatement can be checked against the real reference code.  Built
 * by oracle/Makefile into oracle/_ref/libref.so, only where /root/reference
 * exists; nothing in the product loads it.
 *
 * Exposed:
 *   codecs    src/dtype/fp_convert.c, src/dtype/fp8.c
 *   xexp2f    src/codegen/xexp2f.c (the CPU JIT's exp2)
 *   linear / softmax / layernorm / rmsnorm / gelu / causal attention on f32
 *             through the reference's own Tensor graph + rangeify + CPU JIT
 *             (src/nn/dot.c, src/nn/softmax.c, src/nn/layernorm.c,
 *             src/nn/elementwise.c, src/nn/scaled_dot_product_attention.c,
 *             py/thvm/nn.py:211-224)
 *   capture   every kernel those dispatch: its lifted DAG as renderer rows,
 *             its input buffers and the reference CPU output. */
#include THVM_REF_TU

u8  ref_f32_to_fp8e4m3(f32 v)      { return f32_to_fp8e4m3(v); }
u8  ref_f32_to_fp8e4m3_sat(f32 v)  { return f32_to_fp8e4m3_sat(v); }
u8  ref_f32_to_fp8e5m2(f32 v)      { return f32_to_fp8e5m2(v); }
u8  ref_f32_to_fp8e5m2_sat(f32 v)  { return f32_to_fp8e5m2_sat(v); }
f32 ref_fp8e4m3_to_f32(u8 v)       { return fp8e4m3_to_f32(v); }
f32 ref_fp8e5m2_to_f32(u8 v)       { return fp8e5m2_to_f32(v); }
u16 ref_f32_to_bf16(f32 v)         { return f32_to_bf16(v); }
f32 ref_bf16_to_f32(u16 v)         { return bf16_to_f32(v); }
u16 ref_f32_to_fp16(f32 v)         { return f32_to_fp16(v); }
f32 ref_fp16_to_f32(u16 v)         { return fp16_to_f32(v); }
u16 ref_f32_to_fp16_manual(f32 v)  { return f32_to_fp16_manual(v); }
f32 ref_fp16_to_f32_manual(u16 v)  { return fp16_to_f32_manual(v); }
f32 ref_xexp2f(f32 v)              { return thvm_xexp2f(v); }

static int REF_INIT = 0;
static void ref_init(void) {
  if (!REF_INIT) { thvm_init(); REF_INIT = 1; }
}

static Tensor ref_tensor2(u32 d0, u32 d1, const float *data) {
  Shape sh = {0};
  sh.ndim = 2;
  sh.dims[0] = d0;
  sh.dims[1] = d1;
  u32 tid = tensor_alloc(&CPU_BACKEND, sh, DT_FP32);
  CPU_BACKEND.buf_write(TENS[tid].buf_id, (void *)data, (u64)d0 * d1 * 4);
  Tensor t;
  t.t = term_new(0, TAG_TEN, DT_FP32, tid);
  t.dtype = DT_FP32;
  t.shape = sh;
  return t;
}

static int ref_read(Tensor y, float *out, u64 n) {
  if (y.t == 0) return -1;
  Term r = term_resolve(thvm_realize(y.t));
  if (term_tag(r) != TAG_TEN) return -1;
  u32 tid = (u32)term_val(r);
  if (TENS[tid].view.numel != n) return -1;
  return TENS[tid].backend->buf_read(TENS[tid].buf_id, out, n * 4);
}

/* y[M,N] = x[M,K] @ w[N,K]^T  (tinygrad Linear: x.linear(w.T)) */
int ref_linear_f32(const float *x, const float *w, float *y, u32 M, u32 N, u32 K) {
  ref_init();
  Tensor X = ref_tensor2(M, K, x), W = ref_tensor2(N, K, w);
  u32 perm[2] = {1, 0};
  Tensor Y = nn_dot(X, nn_permute(W, 2, perm));
  return ref_read(Y, y, (u64)M * N);
}

int ref_softmax_f32(const float *x, float *y, u32 M, u32 K) {
  ref_init();
  Tensor X = ref_tensor2(M, K, x);
  return ref_read(nn_softmax(X, -1, 0), y, (u64)M * K);
}

int ref_layernorm_f32(const float *x, float *y, u32 M, u32 K, double eps) {
  ref_init();
  Tensor X = ref_tensor2(M, K, x);
  u32 ax[1] = {1};
  return ref_read(nn_layernorm(X, 1, ax, eps), y, (u64)M * K);
}

/* RMSNorm._norm: x * rsqrt(mean(x^2, -1, keepdim) + eps) (py/thvm/nn.py:219) */
int ref_rmsnorm_f32(const float *x, float *y, u32 M, u32 K, double eps) {
  ref_init();
  Tensor X = ref_tensor2(M, K, x);
  u32 ax[1] = {1};
  Tensor ms = nn_mean(nn_binop(UOP_MUL, X, X), 1, ax, 1);
  Tensor r = nn_elementwise(NN_RSQRT, nn_binop_f(UOP_ADD, ms, eps));
  return ref_read(nn_binop(UOP_MUL, X, r), y, (u64)M * K);
}

/* The DeepSeek-V2 dense layer's h = silu(g) * u as the reference decode bench
 * builds it (bench/dsv2_decode_bench.c:2042-2049 silu, :2372 the product,
 * :2373 rz): bf16 uops over two [1, n] bf16 tensors, realized through the
 * reference CPU path; h is written as bf16 bits. */
int ref_dense_silu_mul_bf16(const u16 *g, const u16 *u, u16 *h, u32 n) {
  ref_init();
  Shape s = {0};
  s.ndim = 2;
  s.dims[0] = 1;
  s.dims[1] = n;
  u32 tg = tensor_alloc(&CPU_BACKEND, s, DT_BF16), tu = tensor_alloc(&CPU_BACKEND, s, DT_BF16);
  CPU_BACKEND.buf_write(TENS[tg].buf_id, (void *)g, (u64)n * 2);
  CPU_BACKEND.buf_write(TENS[tu].buf_id, (void *)u, (u64)n * 2);
  u32 d1k[2] = {1, n};
  union { f32 f; u32 b; } c1 = {.f = -1.4426950408889634f}, c2 = {.f = 1.0f};
  Term x = term_new(0, TAG_TEN, DT_BF16, tg);
  Term nlog2e = uop_expand(uop_const(DT_BF16, c1.b), 2, d1k);
  Term one = uop_expand(uop_const(DT_BF16, c2.b), 2, d1k);
  Term sig = uop_unary(UOP_RECIP, uop_binary(UOP_ADD, one, uop_unary(UOP_EXP2, uop_binary(UOP_MUL, x, nlog2e))));
  Term hh = uop_binary(UOP_MUL, uop_binary(UOP_MUL, x, sig), term_new(0, TAG_TEN, DT_BF16, tu));
  Term r = term_resolve(thvm_realize(hh));
  if (term_tag(r) != TAG_TEN) return -1;
  u32 tid = (u32)term_val(r);
  if (TENS[tid].view.numel != n || TENS[tid].dtype != DT_BF16) return -2;
  return TENS[tid].backend->buf_read(TENS[tid].buf_id, h, (u64)n * 2);
}

/* ---- kernel capture ------------------------------------------------------
 * While capture is on, every kernel the reference CPU path dispatches passes
 * through cap_dispatch, installed in the CPU Backend vtable's dispatch_kernel
 * slot (src/thvm.h:818): it flattens the kernel's lifted DAG
 * (KernelEntry.cached_lift.store_root, src/thvm.h:1023) into rows of the
 * renderer's ThvmUop layout (sources before users), copies the kernel's
 * input buffers, runs the reference dispatch, and copies its output.  The
 * rows and buffers are the renderer target's test vectors.
 * Row payloads: CONST arg0 = bits; RANGE arg0..2 = axis id, KAX type,
 * extent; REDUCE src1..3 = the RANGE rows reduced, arg0 = kind; BUFFER
 * arg0 = slot (the DAG's instance: 0 output, i+1 input i), arg1 = element
 * count; CAST / BITCAST dtype = target.  OPT annotations (src/thvm.h:439-451)
 * are recorded per kernel and flattened through to their target. */
typedef struct { uint32_t op, dtype; int32_t src[4]; int64_t arg[4]; } RefUop;
#define CAP_K 96
#define CAP_ROWS 4096
#define CAP_SLOTS 16
#define CAP_VARS 4
typedef struct {
  RefUop rows[CAP_ROWS];
  Term terms[CAP_ROWS];
  u32 n;
  u32 n_slots;                       /* 1 + inputs */
  u32 dt[CAP_SLOTS];
  u64 numel[CAP_SLOTS];
  void *buf[CAP_SLOTS];              /* slot 0: the output after the dispatch */
  u32 n_opt, opt_kind[8], opt_factor[8];
  /* symbolic extents: the kernel's kvars in first-use order (DEFINE_VAR arg0
   * = the index here), their bounds and the values bound at dispatch */
  u32 n_var, var_id[CAP_VARS], var_lo[CAP_VARS], var_hi[CAP_VARS], var_val[CAP_VARS];
  int ok;
  char why[96];
} CapK;
static CapK *CAPS;
static u32 NCAPS;
static int CAP_ON;
static int (*CAP_ORIG)(KernelEntry *, u32 *, u32);

static int cap_find(CapK *c, Term t) {
  for (u32 i = 0; i < c->n; i++)
    if (c->terms[i] == t) return (int)i;
  return -1;
}
static int cap_row(CapK *c, Term t, u32 op, u32 dt) {
  if (c->n >= CAP_ROWS) { c->ok = 0; snprintf(c->why, sizeof c->why, "over %d rows", CAP_ROWS); return -1; }
  RefUop *r = &c->rows[c->n];
  memset(r, 0, sizeof *r);
  r->op = op; r->dtype = dt;
  r->src[0] = r->src[1] = r->src[2] = r->src[3] = -1;
  c->terms[c->n] = t;
  return (int)c->n++;
}
/* the kernel's index of kvar vid (recorded with its bounds and current value) */
static int cap_var(CapK *c, u32 vid) {
  for (u32 i = 0; i < c->n_var; i++)
    if (c->var_id[i] == vid) return (int)i;
  if (c->n_var >= CAP_VARS) { c->ok = 0; snprintf(c->why, sizeof c->why, "over %d kvars", CAP_VARS); return -1; }
  const u32 i = c->n_var++;
  c->var_id[i] = vid;
  c->var_lo[i] = KVARS[vid].lo;
  c->var_hi[i] = kvar_hi(vid);
  c->var_val[i] = kvar_runtime(vid);
  return (int)i;
}
static int cap_flat(CapK *c, Term t) {
  if (!c->ok) return -1;
  if (term_tag(t) != TAG_UOP) { c->ok = 0; snprintf(c->why, sizeof c->why, "a non-UOP term (tag %u)", term_tag(t)); return -1; }
  const int have = cap_find(c, t);
  if (have >= 0) return have;
  const u32 op = term_ext(t);
  const u64 loc = term_val(t);
  u32 dt = DT_FP32;
  (void)term_dtype_in(t, 0, &dt);
  int s[3] = {-1, -1, -1}, r;
  switch (op) {
    case UOP_CONST: {
      r = cap_row(c, t, op, term_ext(heap_read(loc)));
      if (r >= 0) c->rows[r].arg[0] = (i64)(u32)term_val(heap_read(loc));
      return r;
    }
    case UOP_RANGE: {
      const u32 ext = (u32)term_val(heap_read(loc + 2));
      int dv = -1;
      if (kvar_extent_is_var(ext)) {
        /* a symbolic extent (the reference's kvar loop bound, render_uop.c:
         * 5055-5090): a DEFINE_VAR row (arg0 = the kernel's var index, arg1 /
         * arg2 = its bounds) that the RANGE takes as src0 */
        const int vi = cap_var(c, kvar_extent_var_id(ext));
        if (vi < 0) return -1;
        dv = cap_row(c, 0, UOP_DEFINE_VAR, DT_INT32);
        if (dv < 0) return -1;
        c->rows[dv].arg[0] = vi;
        c->rows[dv].arg[1] = c->var_lo[vi];
        c->rows[dv].arg[2] = c->var_hi[vi];
      }
      r = cap_row(c, t, op, DT_INT32);
      if (r >= 0) {
        c->rows[r].src[0] = dv;
        c->rows[r].arg[0] = (i64)term_val(heap_read(loc));
        c->rows[r].arg[1] = (i64)term_val(heap_read(loc + 1));
        c->rows[r].arg[2] = (i64)kvar_extent_static(ext);
      }
      return r;
    }
    case UOP_BUFFER: {
      if (term_val(heap_read(loc)) != UOP_SCOPE_GLOBAL) { c->ok = 0; snprintf(c->why, sizeof c->why, "a non-global buffer"); return -1; }
      const u32 inst = (u32)term_val(heap_read(loc + 3));
      r = cap_row(c, t, op, (u32)term_val(heap_read(loc + 1)));
      if (r >= 0) { c->rows[r].arg[0] = inst; c->rows[r].arg[1] = inst < CAP_SLOTS ? (i64)c->numel[inst] : 0; }
      return r;
    }
    case UOP_OPT: {
      if (c->n_opt < 8) {
        c->opt_kind[c->n_opt] = (u32)term_val(heap_read(loc + 1));
        c->opt_factor[c->n_opt] = (u32)term_val(heap_read(loc + 2));
        c->n_opt++;
      }
      return cap_flat(c, heap_read(loc));
    }
    case UOP_REDUCE: {
      s[0] = cap_flat(c, heap_read(loc));
      const u32 nax = (u32)term_val(heap_read(loc + 2));
      if (s[0] < 0) return -1;
      if (nax == 0 || nax > 3) { c->ok = 0; snprintf(c->why, sizeof c->why, "a reduce over %u axes", nax); return -1; }
      r = cap_row(c, t, op, dt);
      if (r < 0) return -1;
      c->rows[r].src[0] = s[0];
      c->rows[r].arg[0] = (i64)term_val(heap_read(loc + 1));
      for (u32 k = 0; k < nax; k++) {
        const i64 axis = (i64)term_val(heap_read(loc + 3 + k));
        int found = -1;
        for (u32 j = 0; j < c->n; j++)
          if (c->rows[j].op == UOP_RANGE && c->rows[j].arg[0] == axis) { found = (int)j; break; }
        if (found < 0) { c->ok = 0; snprintf(c->why, sizeof c->why, "a reduce axis %lld no RANGE reads", (long long)axis); return -1; }
        c->rows[r].src[1 + k] = found;
      }
      return r;
    }
    case UOP_CAST: case UOP_BITCAST: {
      s[0] = cap_flat(c, heap_read(loc));
      if (s[0] < 0) return -1;
      r = cap_row(c, t, op, (u32)term_val(heap_read(loc + 1)));
      if (r >= 0) c->rows[r].src[0] = s[0];
      return r;
    }
    case UOP_NEG: case UOP_RECIP: case UOP_EXP2: case UOP_LOG2: case UOP_SQRT: case UOP_SIN:
    case UOP_LOAD: {
      s[0] = cap_flat(c, heap_read(loc));
      if (s[0] < 0) return -1;
      r = cap_row(c, t, op, dt);
      if (r >= 0) c->rows[r].src[0] = s[0];
      return r;
    }
    case UOP_IWHERE: case UOP_STORE: {
      for (int k = 0; k < 3; k++) if ((s[k] = cap_flat(c, heap_read(loc + k))) < 0) return -1;
      /* a select between index values is index arithmetic */
      if (op == UOP_IWHERE && c->rows[s[1]].dtype == DT_INT32 && c->rows[s[2]].dtype == DT_INT32) dt = DT_INT32;
      r = cap_row(c, t, op, dt);
      if (r >= 0) for (int k = 0; k < 3; k++) c->rows[r].src[k] = s[k];
      return r;
    }
    case UOP_ADD: case UOP_MUL: case UOP_CMPLT: case UOP_CMPEQ: case UOP_INDEX_E:
    case UOP_IADD: case UOP_ISUB: case UOP_IMUL: case UOP_IDIV: case UOP_IMOD: case UOP_ILT:
    case UOP_IAND: case UOP_IOR: case UOP_IXOR: case UOP_ISHL: case UOP_ISHR: case UOP_POW: {
      for (int k = 0; k < 2; k++) if ((s[k] = cap_flat(c, heap_read(loc + k))) < 0) return -1;
      /* the I* ops are index arithmetic: int32 (term_dtype_in reports the
       * kernel's value type for them) */
      if (op >= UOP_IADD && op != UOP_INDEX_E && op != UOP_POW) dt = DT_INT32;
      r = cap_row(c, t, op, dt);
      if (r >= 0) { c->rows[r].src[0] = s[0]; c->rows[r].src[1] = s[1]; }
      return r;
    }
    default:
      c->ok = 0;
      snprintf(c->why, sizeof c->why, "op %u", op);
      return -1;
  }
}

/* The reference renderer folds the inner half of a split reduce axis -- an
 * UNROLL / UPCAST RANGE that the store address does not read -- into the
 * innermost REDUCE whose source reads it (render_uop.c:3080-3100,
 * 3946-3970, tinygrad's expand_reduce).  The rows make that explicit: such a
 * RANGE is appended to that REDUCE's axes. */
static void cap_fold_split_axes(CapK *c) {
  const u32 n = c->n;
  u64 *dep = (u64 *)calloc(n, sizeof(u64));      /* RANGE rows read, as bits of rng[] */
  int rng[64], nr = 0;
  if (!dep) { c->ok = 0; return; }
  for (u32 i = 0; i < n; i++) {
    const RefUop *u = &c->rows[i];
    if (u->op == UOP_RANGE) {
      if (nr >= 64) { c->ok = 0; snprintf(c->why, sizeof c->why, "over 64 ranges"); free(dep); return; }
      rng[nr] = (int)i;
      dep[i] = 1ull << nr++;
      continue;
    }
    for (int k = 0; k < 4; k++)
      if (u->src[k] >= 0 && !(u->op == UOP_REDUCE && k > 0)) dep[i] |= dep[u->src[k]];
  }
  const RefUop *st = &c->rows[n - 1];
  const u64 addr = st->op == UOP_STORE && st->src[1] >= 0 ? dep[st->src[1]] : 0;
  u64 owned = 0;
  for (u32 i = 0; i < n && c->ok; i++) {
    RefUop *u = &c->rows[i];
    if (u->op != UOP_REDUCE) continue;
    u64 named = 0;
    for (int k = 1; k < 4; k++)
      for (int j = 0; j < nr; j++)
        if (u->src[k] == rng[j]) named |= 1ull << j;
    owned |= named;
    for (int j = 0; j < nr; j++) {
      const RefUop *rg = &c->rows[rng[j]];
      const u64 b = 1ull << j;
      if ((rg->arg[1] != KAX_UNROLL && rg->arg[1] != KAX_UPCAST) || (addr & b) || (owned & b) ||
          !(dep[u->src[0]] & b))
        continue;
      int slot = -1;
      for (int k = 1; k < 4; k++) if (u->src[k] < 0) { slot = k; break; }
      if (slot < 0) { c->ok = 0; snprintf(c->why, sizeof c->why, "a reduce over more than 3 axes"); break; }
      u->src[slot] = rng[j];
      owned |= b;
    }
    /* the reduce's own value no longer depends on its axes */
    for (int k = 1; k < 4; k++)
      for (int j = 0; j < nr; j++)
        if (u->src[k] == rng[j]) dep[i] &= ~(1ull << j);
  }
  free(dep);
}

static void *cap_copy(u32 buf_id, u32 dt, u64 numel) {
  const u64 nb = dtype_storage_bytes(dt, numel);
  void *p = malloc(nb ? nb : 1);
  if (p && nb && CPU_BACKEND.buf_read(buf_id, p, nb) != 0) { free(p); return NULL; }
  return p;
}

static void *cap_gather(u32 buf_id, u32 dt, u64 buf_numel, const View *v) {
  const u64 es = dtype_storage_bytes(dt, 1);
  char *raw = (char *)cap_copy(buf_id, dt, buf_numel), *out = (char *)malloc(v->numel * es + 1);
  if (!raw || !out) { free(raw); free(out); return NULL; }
  for (u64 e = 0; e < v->numel; e++) {
    u64 q = e;
    i64 at = v->offset;
    for (int d = (int)v->shape.ndim - 1; d >= 0; d--) {
      const u32 ext = v->shape.dims[d];
      at += (i64)(q % ext) * v->strides[d];
      q /= ext;
    }
    if (at < 0 || (u64)at >= buf_numel) { free(raw); free(out); return NULL; }
    memcpy(out + e * es, raw + (u64)at * es, es);
  }
  free(raw);
  return out;
}

static int cap_dispatch(KernelEntry *ke, u32 *in_ids, u32 out_id) {
  CapK *c = NULL;
  if (CAP_ON && NCAPS < CAP_K && !kernel_is_custom(ke) && ke->cached_lift.store_root != 0) {
    c = &CAPS[NCAPS++];
    memset(c, 0, sizeof *c);
    c->ok = 1;
    c->n_slots = 1 + ke->n_inputs;
    if (c->n_slots > CAP_SLOTS) { c->ok = 0; snprintf(c->why, sizeof c->why, "%u inputs", ke->n_inputs); }
    /* a slot holds its whole buffer (a composed strided view indexes it) */
    c->dt[0] = ke->output_dtype;
    c->numel[0] = CPU_BUFS[out_id].req_nbytes / dtype_storage_bytes(ke->output_dtype, 1);
    for (u32 i = 0; c->ok && i < ke->n_inputs; i++) {
      c->dt[1 + i] = ke->input_dtypes[i];
      c->numel[1 + i] = CPU_BUFS[in_ids[i]].req_nbytes / dtype_storage_bytes(ke->input_dtypes[i], 1);
      const int composed = ke->input_chain_composed ? ke->input_chain_composed[i] : 0;
      const View *v = &ke->input_views[i];
      const u32 tid = ke->input_tids ? ke->input_tids[i] : 0;
      if (!composed && !v->contiguous) {
        /* a single strided view: the DAG indexes it in its logical
         * row-major order and the reference's renderer maps that index
         * through the view (KernelEntry.input_views, src/thvm.h:958-969);
         * the slot holds the view gathered in that order */
        if (tid == 0 || TENS[tid].nviews != 0) {
          c->ok = 0;
          snprintf(c->why, sizeof c->why, "input %u is a chain of views", i);
          break;
        }
        c->buf[1 + i] = cap_gather(in_ids[i], c->dt[1 + i], c->numel[1 + i], v);
        c->numel[1 + i] = v->numel;
        if (!c->buf[1 + i]) { c->ok = 0; snprintf(c->why, sizeof c->why, "input %u gather failed", i); break; }
        continue;
      }
      c->buf[1 + i] = cap_copy(in_ids[i], c->dt[1 + i], c->numel[1 + i]);
    }
    if (c->ok) cap_flat(c, ke->cached_lift.store_root);
    if (c->ok) cap_fold_split_axes(c);
  }
  const int rc = CAP_ORIG(ke, in_ids, out_id);
  if (c && c->ok) c->buf[0] = cap_copy(out_id, c->dt[0], c->numel[0]);
  return rc;
}

int ref_capture_begin(void) {
  ref_init();
  if (!CAPS) CAPS = (CapK *)calloc(CAP_K, sizeof(CapK));
  if (!CAPS) return -1;
  for (u32 k = 0; k < NCAPS; k++)
    for (u32 s = 0; s < CAP_SLOTS; s++) { free(CAPS[k].buf[s]); CAPS[k].buf[s] = NULL; }
  NCAPS = 0;
  if (!CAP_ORIG) { CAP_ORIG = CPU_BACKEND.dispatch_kernel; CPU_BACKEND.dispatch_kernel = cap_dispatch; }
  CAP_ON = 1;
  return 0;
}
int ref_capture_end(void) { CAP_ON = 0; return (int)NCAPS; }
/* kernel k: rows (n), slot count, opts; status 1 = captured, 0 = not (why) */
int ref_capture_kernel(u32 k, RefUop *rows, u32 cap, u32 *n, u32 *n_slots, u32 *opts, u32 *n_opt,
                       char *why, u32 whylen) {
  if (k >= NCAPS) return -1;
  CapK *c = &CAPS[k];
  *n = c->n; *n_slots = c->n_slots; *n_opt = c->n_opt;
  for (u32 i = 0; i < c->n_opt; i++) { opts[2 * i] = c->opt_kind[i]; opts[2 * i + 1] = c->opt_factor[i]; }
  snprintf(why, whylen, "%s", c->why);
  if (c->ok && c->n <= cap) memcpy(rows, c->rows, c->n * sizeof(RefUop));
  return c->ok;
}
/* kvars of kernel k: up to cap (value bound at dispatch, lo, hi) triples;
 * returns the count */
int ref_capture_vars(u32 k, u32 *vals, u32 cap) {
  if (k >= NCAPS) return -1;
  const CapK *c = &CAPS[k];
  for (u32 i = 0; i < c->n_var && i < cap; i++) {
    vals[3 * i] = c->var_val[i];
    vals[3 * i + 1] = c->var_lo[i];
    vals[3 * i + 2] = c->var_hi[i];
  }
  return (int)c->n_var;
}
/* slot s of kernel k: dtype, element count and (dst != NULL) the bytes */
int ref_capture_slot(u32 k, u32 s, u32 *dt, u64 *numel, void *dst, u64 cap) {
  if (k >= NCAPS || s >= CAPS[k].n_slots || s >= CAP_SLOTS) return -1;
  CapK *c = &CAPS[k];
  *dt = c->dt[s]; *numel = c->numel[s];
  if (!dst) return 0;
  const u64 nb = dtype_storage_bytes(c->dt[s], c->numel[s]);
  if (!c->buf[s] || nb > cap) return -1;
  memcpy(dst, c->buf[s], nb);
  return 0;
}

/* GELU (tanh form) and scaled dot-product attention on f32 through the
 * reference Tensor graph (src/nn/elementwise.c, src/nn/scaled_dot_product_attention.c) */
int ref_gelu_f32(const float *x, float *y, u32 M, u32 K) {
  ref_init();
  return ref_read(nn_elementwise(NN_GELU, ref_tensor2(M, K, x)), y, (u64)M * K);
}
static Tensor ref_tensor3(u32 d0, u32 d1, u32 d2, const float *data) {
  Shape sh = {0};
  sh.ndim = 3; sh.dims[0] = d0; sh.dims[1] = d1; sh.dims[2] = d2;
  u32 tid = tensor_alloc(&CPU_BACKEND, sh, DT_FP32);
  CPU_BACKEND.buf_write(TENS[tid].buf_id, (void *)data, (u64)d0 * d1 * d2 * 4);
  Tensor t;
  t.t = term_new(0, TAG_TEN, DT_FP32, tid);
  t.dtype = DT_FP32;
  t.shape = sh;
  return t;
}
/* q, k, v [H][T][hd] -> out [H][T][hd], causal */
int ref_sdpa_f32(const float *q, const float *k, const float *v, float *out, u32 H, u32 T, u32 hd) {
  ref_init();
  Tensor Q = ref_tensor3(H, T, hd, q), Kt = ref_tensor3(H, T, hd, k), Vt = ref_tensor3(H, T, hd, v);
  Tensor none;
  memset(&none, 0, sizeof none);
  return ref_read(nn_scaled_dot_product_attention(Q, Kt, Vt, none, 1), out, (u64)H * T * hd);
}

/* One GPT-2 transformer block over T tokens (causal prefill), f32, through
 * the reference Tensor graph (tinygrad's GPT-2 block,
 * bench/gpt2/thvm_gpt2.py:25-75, with q, k and v from three [D][D]
 * matrices): h = x + attn(ln1(x)); out = h + mlp(ln2(h)), ln(z) =
 * layernorm(z) * w + b, mlp(z) = gelu(z Wfc + bfc) Wpr + bpr.  Matrices are
 * [in][out].  Realized on the CPU path; every kernel it schedules is what
 * the capture records. */
static Tensor ref_vec(u32 n, const float *data) {
  Shape sh = {0};
  sh.ndim = 1;
  sh.dims[0] = n;
  u32 tid = tensor_alloc(&CPU_BACKEND, sh, DT_FP32);
  CPU_BACKEND.buf_write(TENS[tid].buf_id, (void *)data, (u64)n * 4);
  Tensor t;
  t.t = term_new(0, TAG_TEN, DT_FP32, tid);
  t.dtype = DT_FP32;
  t.shape = sh;
  return t;
}
static Tensor ref_ln(Tensor z, Tensor w, Tensor b) {
  u32 ax[1] = {1};
  return nn_binop(UOP_ADD, nn_binop(UOP_MUL, nn_layernorm(z, 1, ax, 1e-5), w), b);
}
static Tensor ref_heads(Tensor z, u32 T, u32 H, u32 hd) {      /* [T][D] -> [H][T][hd] */
  u32 d3[3] = {T, H, hd}, perm[3] = {1, 0, 2};
  return nn_permute(nn_reshape(z, 3, d3), 3, perm);
}
int ref_gpt2_block_f32(const float *x, const float *const *p, float *out, u32 T, u32 D, u32 H, u32 F) {
  ref_init();
  const u32 hd = D / H;
  Tensor X = ref_tensor2(T, D, x);
  Tensor ln1w = ref_vec(D, p[0]), ln1b = ref_vec(D, p[1]);
  Tensor wq = ref_tensor2(D, D, p[2]), bq = ref_vec(D, p[3]);
  Tensor wk = ref_tensor2(D, D, p[4]), bk = ref_vec(D, p[5]);
  Tensor wv = ref_tensor2(D, D, p[6]), bv = ref_vec(D, p[7]);
  Tensor wo = ref_tensor2(D, D, p[8]), bo = ref_vec(D, p[9]);
  Tensor ln2w = ref_vec(D, p[10]), ln2b = ref_vec(D, p[11]);
  Tensor wfc = ref_tensor2(D, F, p[12]), bfc = ref_vec(F, p[13]);
  Tensor wpr = ref_tensor2(F, D, p[14]), bpr = ref_vec(D, p[15]);
  Tensor z = ref_ln(X, ln1w, ln1b);
  Tensor q = ref_heads(nn_linear(z, wq, bq), T, H, hd), k = ref_heads(nn_linear(z, wk, bk), T, H, hd),
         v = ref_heads(nn_linear(z, wv, bv), T, H, hd);
  Tensor none;
  memset(&none, 0, sizeof none);
  Tensor a = nn_scaled_dot_product_attention(q, k, v, none, 1);          /* [H][T][hd] */
  u32 perm[3] = {1, 0, 2}, d2[2] = {T, D};
  a = nn_reshape(nn_permute(a, 3, perm), 2, d2);
  Tensor h = nn_binop(UOP_ADD, X, nn_linear(a, wo, bo));
  Tensor m = nn_linear(nn_elementwise(NN_GELU, nn_linear(ref_ln(h, ln2w, ln2b), wfc, bfc)), wpr, bpr);
  return ref_read(nn_binop(UOP_ADD, h, m), out, (u64)T * D);
}

/* ---- narrow-float and symbolic-extent workloads ---------------------------
 * The same operations on fp16 / bf16 tensors (the reference CPU path
 * realizes non-f32 kernels through its uop walker, src/backend/cpu/
 * uop_walk.c:141-293: values evaluated in double, narrowed at CAST / STORE),
 * and decode attention over a cache whose length is a bound kvar (the
 * symbolic extent the GPT-2 decode with a bound start_pos schedules,
 * render_uop.c:5055-5090).  Inputs arrive as f32 and are narrowed with the
 * reference's own encoders; outputs are written in the tensor's storage
 * type (2-byte bits for fp16 / bf16). */
static Tensor ref_tensor_dt(u32 ndim, const u32 *dims, u32 dt, const float *data) {
  Shape sh = {0};
  sh.ndim = ndim;
  u64 n = 1;
  for (u32 i = 0; i < ndim; i++) { sh.dims[i] = dims[i]; n *= kvar_extent_static(dims[i]); }
  u32 tid = tensor_alloc(&CPU_BACKEND, sh, dt);
  if (dt == DT_FP32) {
    CPU_BACKEND.buf_write(TENS[tid].buf_id, (void *)data, n * 4);
  } else {
    u16 *b = (u16 *)malloc(n * 2 + 2);
    for (u64 i = 0; i < n; i++) b[i] = dt == DT_FP16 ? f32_to_fp16(data[i]) : f32_to_bf16(data[i]);
    CPU_BACKEND.buf_write(TENS[tid].buf_id, b, n * 2);
    free(b);
  }
  Tensor t;
  t.t = term_new(0, TAG_TEN, dt, tid);
  t.dtype = dt;
  t.shape = sh;
  return t;
}
static int ref_read_dt(Tensor y, void *out, u64 n) {
  if (y.t == 0) return -1;
  Term r = term_resolve(thvm_realize(y.t));
  if (term_tag(r) != TAG_TEN) return -1;
  u32 tid = (u32)term_val(r);
  if (TENS[tid].view.numel != n) return -2;
  return TENS[tid].backend->buf_read(TENS[tid].buf_id, out, dtype_storage_bytes(TENS[tid].dtype, n));
}

int ref_linear_t(u32 dt, const float *x, const float *w, void *y, u32 M, u32 N, u32 K) {
  ref_init();
  u32 dx[2] = {M, K}, dw[2] = {N, K}, perm[2] = {1, 0};
  Tensor X = ref_tensor_dt(2, dx, dt, x), W = ref_tensor_dt(2, dw, dt, w);
  return ref_read_dt(nn_dot(X, nn_permute(W, 2, perm)), y, (u64)M * N);
}
int ref_softmax_t(u32 dt, const float *x, void *y, u32 M, u32 K) {
  ref_init();
  u32 d[2] = {M, K};
  return ref_read_dt(nn_softmax(ref_tensor_dt(2, d, dt, x), -1, 0), y, (u64)M * K);
}
int ref_layernorm_t(u32 dt, const float *x, void *y, u32 M, u32 K, double eps) {
  ref_init();
  u32 d[2] = {M, K}, ax[1] = {1};
  return ref_read_dt(nn_layernorm(ref_tensor_dt(2, d, dt, x), 1, ax, eps), y, (u64)M * K);
}
int ref_gelu_t(u32 dt, const float *x, void *y, u32 M, u32 K) {
  ref_init();
  u32 d[2] = {M, K};
  return ref_read_dt(nn_elementwise(NN_GELU, ref_tensor_dt(2, d, dt, x)), y, (u64)M * K);
}

/* The GPT-2 block of ref_gpt2_block_f32 on dtype dt tensors (inputs and every
 * parameter stored in dt). */
int ref_gpt2_block_t(u32 dt, const float *x, const float *const *p, void *out, u32 T, u32 D, u32 H, u32 F) {
  ref_init();
  const u32 hd = D / H;
  u32 dTD[2] = {T, D}, dDD[2] = {D, D}, dDF[2] = {D, F}, dFD[2] = {F, D}, dD[1] = {D}, dF[1] = {F};
  Tensor X = ref_tensor_dt(2, dTD, dt, x);
  Tensor ln1w = ref_tensor_dt(1, dD, dt, p[0]), ln1b = ref_tensor_dt(1, dD, dt, p[1]);
  Tensor wq = ref_tensor_dt(2, dDD, dt, p[2]), bq = ref_tensor_dt(1, dD, dt, p[3]);
  Tensor wk = ref_tensor_dt(2, dDD, dt, p[4]), bk = ref_tensor_dt(1, dD, dt, p[5]);
  Tensor wv = ref_tensor_dt(2, dDD, dt, p[6]), bv = ref_tensor_dt(1, dD, dt, p[7]);
  Tensor wo = ref_tensor_dt(2, dDD, dt, p[8]), bo = ref_tensor_dt(1, dD, dt, p[9]);
  Tensor ln2w = ref_tensor_dt(1, dD, dt, p[10]), ln2b = ref_tensor_dt(1, dD, dt, p[11]);
  Tensor wfc = ref_tensor_dt(2, dDF, dt, p[12]), bfc = ref_tensor_dt(1, dF, dt, p[13]);
  Tensor wpr = ref_tensor_dt(2, dFD, dt, p[14]), bpr = ref_tensor_dt(1, dD, dt, p[15]);
  Tensor z = ref_ln(X, ln1w, ln1b);
  Tensor q = ref_heads(nn_linear(z, wq, bq), T, H, hd), k = ref_heads(nn_linear(z, wk, bk), T, H, hd),
         v = ref_heads(nn_linear(z, wv, bv), T, H, hd);
  Tensor none;
  memset(&none, 0, sizeof none);
  Tensor a = nn_scaled_dot_product_attention(q, k, v, none, 1);
  u32 perm[3] = {1, 0, 2}, d2[2] = {T, D};
  a = nn_reshape(nn_permute(a, 3, perm), 2, d2);
  Tensor h = nn_binop(UOP_ADD, X, nn_linear(a, wo, bo));
  Tensor m = nn_linear(nn_elementwise(NN_GELU, nn_linear(ref_ln(h, ln2w, ln2b), wfc, bfc)), wpr, bpr);
  return ref_read_dt(nn_binop(UOP_ADD, h, m), out, (u64)T * D);
}

/* One decode query per head over a KV cache of a bound length: q [H][hd],
 * k, v [H][Lmax][hd] of which rows [0, L) are live, L a kvar of bounds
 * [1, Lmax] bound to L; out [H][hd] = softmax(q k^T * scale) v, built from
 * uops as the reference's symbolic decode tests build it
 * (tests/test_sym_decode_step.c, tests/test_sym_attn.c): scores reduce over
 * hd, the softmax runs over the symbolic axis (exp2 of pre-scaled
 * differences), the weighted sum reduces over the symbolic axis. */
int ref_sym_attn_t(u32 dt, const float *q, const float *k, const float *v, void *out, u32 H, u32 Lmax,
                   u32 L, u32 hd, float scale) {
  ref_init();
  const u32 s = kvar_alloc("L", 1, Lmax);
  if (s == 0) return -3;
  kvar_set_runtime(s, L);
  const u32 P = kvar_pack_extent(s);
  u32 dq[3] = {H, 1, hd}, dk[3] = {H, P, hd};
  Tensor Q = ref_tensor_dt(3, dq, dt, q), K = ref_tensor_dt(3, dk, dt, k), V = ref_tensor_dt(3, dk, dt, v);
  u32 hph[3] = {H, P, hd}, hp[2] = {H, P}, h1[2] = {H, 1}, hp1[3] = {H, P, 1};
  union { f32 f; u32 b; } cs = {.f = scale * 1.4426950408889634f};
  Term qe = uop_expand(Q.t, 3, hph);
  Term sc = uop_reduce(REDUCE_SUM, 2, uop_binary(UOP_MUL, qe, K.t));                  /* {H,P} */
  sc = uop_binary(UOP_MUL, sc, uop_expand(uop_const(dt, cs.b), 2, hp));
  Term mx = uop_expand(uop_reshape(uop_reduce(REDUCE_MAX, 1, sc), 2, h1), 2, hp);
  Term e = uop_unary(UOP_EXP2, uop_binary(UOP_ADD, sc, uop_unary(UOP_NEG, mx)));
  Term den = uop_expand(uop_reshape(uop_reduce(REDUCE_SUM, 1, e), 2, h1), 2, hp);
  Term w = uop_binary(UOP_MUL, e, uop_unary(UOP_RECIP, den));
  Term we = uop_expand(uop_reshape(w, 3, hp1), 3, hph);
  Term o = uop_reduce(REDUCE_SUM, 1, uop_binary(UOP_MUL, we, V.t));                   /* {H,hd} */
  Tensor y;
  y.t = o;
  y.dtype = dt;
  return ref_read_dt(y, out, (u64)H * hd);
}
