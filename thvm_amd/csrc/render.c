/* render.c -- renderer target: one kernel's lifted uop DAG -> HIP source for
 * gfx950 plus its launch geometry.
 *
 * Replaces the reference's CUDA target cg_render_uop_kernel_cuda_root
 * (src/codegen/render_uop.c:4964-5113), its term emitter rmu_emit_term
 * (:454-815) and the CUDA dispatch geometry (src/backend/cuda/jit.c:634-787).
 * The DAG arrives flattened (ThvmUop, sources before users) with the
 * reference's UOP_* op numbers (src/thvm.h:302-512), RANGE axis types
 * (KAX_*, :686-692) and reduce kinds (REDUCE_SUM / REDUCE_MAX, :515-516).
 *
 * gfx950 choices:
 *   - values are SSA locals emitted once per scope; a node that does not read
 *     a reduce loop's axes is hoisted out of that loop;
 *   - fp16 / bf16 values compute in f32 and narrow to their storage type only
 *     at a CAST into that type and at the STORE -- the reference CPU path's
 *     semantics for narrow floats (its uop walker rounds each op to f32 and
 *     narrows at CAST / STORE, src/backend/cpu/uop_walk.c:272-293), pinned by
 *     kernels of fp16 and bf16 graphs captured from the compiled reference;
 *   - geometry (ThvmRenderOpts, the reference's LOCAL / GROUP_REDUCE /
 *     UPCAST opts): `group` consecutive threads share one output's
 *     reductions (strided partial terms, a xor-shuffle tree inside a wave, the
 *     group's waves in order through LDS above 64), `block` threads per
 *     block, `upcast` consecutive outputs per thread (one thread per output
 *     otherwise); without opts the hand-coded choice (hand_opts below), and
 *     thvm_hip_render_autotune searches them on the device;
 *   - fp8 e4m3 outputs store with the reference's kernel-store narrowing
 *     (saturating round to nearest even, NaN -> S.1111.111), and a CAST to
 *     fp8 rounds through it;
 *   - a lifted fp16 / bf16 matmul (REDUCE_SUM of a product of two affine
 *     reads, M, N, K multiples of 16) renders as MFMA 16x16 tiles with its
 *     epilogue through the generic emitter (render_mfma below);
 *   - symbolic extents (DEFINE_VAR) are read from an int32 buffer argument,
 *     not passed by value, so a captured graph stays correct when a bound
 *     variable changes; the grid is sized at the variables' upper bounds and
 *     surplus threads exit.
 * Pure host code: no device is touched. */
#include "internal.h"
#include "thvm_hip.h"

#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

/* reference op numbers (src/thvm.h) */
enum {
  U_CONST = 2, U_ADD = 9, U_MUL = 10, U_NEG = 11, U_RECIP = 12, U_EXP2 = 13, U_LOG2 = 14,
  U_SQRT = 15, U_CMPLT = 16, U_REDUCE = 17, U_DEFINE_VAR = 18, U_CMPEQ = 20, U_LOAD = 21,
  U_CAST = 23, U_BITCAST = 24, U_RANGE = 25, U_INDEX_E = 26, U_IADD = 27, U_ISUB = 28,
  U_IMUL = 29, U_IDIV = 30, U_IMOD = 31, U_ILT = 32, U_IAND = 33, U_IWHERE = 34,
  U_BUFFER = 36, U_STORE = 37, U_IOR = 41, U_IXOR = 42, U_ISHL = 44, U_ISHR = 51, U_SIN = 55
};
enum { RED_SUM = 0, RED_MAX = 1 };

#define RENDER_BLOCK 256
#define RENDER_MAX_RANGES 64
#define RENDER_MAX_SLOTS 64

typedef struct {
  char *p;
  size_t n, cap;
  int bad;
} Sb;

static void sb_put(Sb *s, const char *fmt, ...) __attribute__((format(printf, 2, 3)));
static void sb_put(Sb *s, const char *fmt, ...) {
  if (s->bad) return;
  va_list ap;
  va_start(ap, fmt);
  int k = vsnprintf(s->p + s->n, s->cap - s->n, fmt, ap);
  va_end(ap);
  if (k < 0 || (size_t)k >= s->cap - s->n) { s->bad = 1; return; }
  s->n += (size_t)k;
}

typedef struct {
  const ThvmUop *u;
  uint32_t n;
  uint64_t *dep;       /* bit k: reads reduce axis k (index into red_rng) */
  int *level;          /* scope level a node's local lives in, -1 = none */
  int *is_red_axis;    /* RANGE node: its reduce-axis index, or -1 */
  int cur_level;
  int group;           /* threads per output in a reduction (0: one thread per output) */
  int block;           /* threads per block */
  Sb *s;
  char err[160];
  int depth;
} R;

static int is_float(uint32_t dt) {
  return dt == THVM_DT_FP16 || dt == THVM_DT_BF16 || dt == THVM_DT_FP32 || dt == THVM_DT_FP64 ||
         dt == THVM_DT_FP8E4M3;
}

/* storage type of a buffer element */
static const char *store_t(uint32_t dt) {
  switch (dt) {
    case THVM_DT_BOOL: case THVM_DT_UINT8: case THVM_DT_FP8E4M3: return "unsigned char";
    case THVM_DT_INT8: return "signed char";
    case THVM_DT_INT16: return "short";
    case THVM_DT_UINT16: case THVM_DT_BF16: return "unsigned short";
    case THVM_DT_INT32: return "int";
    case THVM_DT_UINT32: return "unsigned";
    case THVM_DT_INT64: return "long long";
    case THVM_DT_UINT64: return "unsigned long long";
    case THVM_DT_FP16: return "_Float16";
    case THVM_DT_FP32: return "float";
    case THVM_DT_FP64: return "double";
    default: return NULL;
  }
}
/* type a value of dtype `dt` computes in */
static const char *alu_t(uint32_t dt) {
  switch (dt) {
    case THVM_DT_FP16: case THVM_DT_BF16: case THVM_DT_FP32: case THVM_DT_FP8E4M3: return "float";
    case THVM_DT_FP64: return "double";
    case THVM_DT_INT64: return "long long";
    case THVM_DT_UINT64: return "unsigned long long";
    case THVM_DT_UINT32: return "unsigned";
    default: return "int";
  }
}
/* rounding of an f32 value to the storage precision of dt */
static const char *round_fn(uint32_t dt) {
  if (dt == THVM_DT_FP16) return "rt_f16";
  if (dt == THVM_DT_BF16) return "rt_bf16";
  if (dt == THVM_DT_FP8E4M3) return "rt_fp8e4m3";
  return "";
}

static const char *PRELUDE =
    "typedef unsigned int uint;\n"
    "#ifndef INFINITY\n#define INFINITY __builtin_inff()\n#endif\n"
    "__device__ __forceinline__ float bf2f(unsigned short h) { return __uint_as_float(((uint)h) << 16); }\n"
    "__device__ __forceinline__ unsigned short f2bf(float f) {\n"
    "  uint u = __float_as_uint(f);\n"
    "  if ((u & 0x7fffffffu) > 0x7f800000u) return (unsigned short)((u >> 16) | 0x40u);\n"
    "  return (unsigned short)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);\n"
    "}\n"
    "__device__ __forceinline__ float rt_bf16(float f) { return bf2f(f2bf(f)); }\n"
    "__device__ __forceinline__ float rt_f16(float f) { return (float)(_Float16)f; }\n"
    /* e4m3 (bias 7, no infinities, S.1111.111 = NaN) decoded from its fields */
    "__device__ __forceinline__ float fp8e4m3_f(unsigned char b) {\n"
    "  uint e = (b >> 3) & 15u, m = b & 7u;\n"
    "  float v = e ? __uint_as_float(((e + 120u) << 23) | (m << 20)) : (float)m * 0.001953125f;\n"
    "  if (e == 15u && m == 7u) v = __uint_as_float(0x7fc00000u);\n"
    "  return (b & 0x80u) ? -v : v;\n"
    "}\n"
    /* f32 -> e4m3 as the reference's kernel store narrows (src/dtype/fp8.c,
     * tests/test_fp8_nonfinite.c): round to nearest even on the f32
     * significand, subnormals kept, a finite overflow and +-inf saturate to
     * +-448 (S.1111.110), a NaN stores S.1111.111 */
    "__device__ __forceinline__ unsigned char f2fp8e4m3(float x) {\n"
    "  const uint u = __float_as_uint(x), s = (u >> 24) & 0x80u, a = u & 0x7fffffffu;\n"
    "  if (a > 0x7f800000u) return (unsigned char)(s | 0x7fu);\n"
    "  if (a == 0x7f800000u) return (unsigned char)(s | 0x7eu);\n"
    "  int ef = (int)(a >> 23); uint sig = a & 0x7fffffu;\n"
    "  if (ef) sig |= 0x800000u; else ef = 1;\n"
    "  int e = ef - 127; if (e < -6) e = -6;\n"
    "  const int sh = (e - 3) - (ef - 150);\n"
    "  uint n = 0u;\n"
    "  if (sh <= 24) {\n"
    "    const uint rem = sig & ((1u << sh) - 1u), half = 1u << (sh - 1);\n"
    "    n = sig >> sh;\n"
    "    if (rem > half || (rem == half && (n & 1u))) n++;\n"
    "  }\n"
    "  uint code = ((uint)(e + 6) << 3) + n;\n"
    "  if (code > 0x7eu) code = 0x7eu;\n"
    "  return (unsigned char)(s | code);\n"
    "}\n"
    "__device__ __forceinline__ float rt_fp8e4m3(float f) { return fp8e4m3_f(f2fp8e4m3(f)); }\n"
    "__device__ __forceinline__ float wsum(float v) {\n"
    "  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);\n"
    "  return v;\n"
    "}\n"
    "__device__ __forceinline__ float wmax(float v) {\n"
    "  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));\n"
    "  return v;\n"
    "}\n"
    "__device__ __forceinline__ int wsumi(int v) {\n"
    "  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);\n"
    "  return v;\n"
    "}\n"
    "__device__ __forceinline__ int wmaxi(int v) {\n"
    "  for (int o = 32; o > 0; o >>= 1) { const int t = __shfl_xor(v, o, 64); v = t > v ? t : v; }\n"
    "  return v;\n"
    "}\n";

static int emit(R *r, int i);

static int src_ok(const R *r, int i, int k) {
  const int s = r->u[i].src[k];
  return s >= 0 && s < i;
}

/* float literal of an f32 bit pattern */
static void emit_const(R *r, int i) {
  const ThvmUop *u = &r->u[i];
  if (is_float(u->dtype)) {
    sb_put(r->s, "  const float v%d = __uint_as_float(0x%08xu);\n", i, (uint32_t)u->arg[0]);
  } else {
    sb_put(r->s, "  const %s v%d = (%s)%lldll;\n", alu_t(u->dtype), i, alu_t(u->dtype),
           (long long)u->arg[0]);
  }
}

static int emit_reduce(R *r, int i) {
  const ThvmUop *u = &r->u[i];
  const int kind = (int)u->arg[0];
  if (kind != RED_SUM && kind != RED_MAX) {
    snprintf(r->err, sizeof r->err, "node %d: reduce kind %d", i, kind);
    return -1;
  }
  int axes[3], na = 0;
  uint64_t mask = 0;
  for (int k = 1; k < 4; k++) {
    if (u->src[k] < 0) continue;
    if (!src_ok(r, i, k) || r->u[u->src[k]].op != U_RANGE) {
      snprintf(r->err, sizeof r->err, "node %d: reduce axis %d is not a RANGE", i, k);
      return -1;
    }
    axes[na++] = u->src[k];
    mask |= 1ull << r->is_red_axis[u->src[k]];
  }
  if (na == 0) { snprintf(r->err, sizeof r->err, "node %d: reduce over no axis", i); return -1; }
  /* hoist what does not read these axes */
  const int v = u->src[0];
  /* extents first (they read only variables and constants) */
  for (int k = 0; k < na; k++) {
    const ThvmUop *rg = &r->u[axes[k]];
    if (rg->src[0] >= 0 && emit(r, rg->src[0]) < 0) return -1;
  }
  /* pre-emit every node of the body that is independent of the loop */
  {
    int *stack = (int *)malloc(sizeof(int) * r->n), sp = 0;
    char *seen = (char *)calloc(r->n, 1);
    if (!stack || !seen) { free(stack); free(seen); snprintf(r->err, sizeof r->err, "out of memory"); return -1; }
    stack[sp++] = v;
    while (sp) {
      const int x = stack[--sp];
      if (seen[x]) continue;
      seen[x] = 1;
      if ((r->dep[x] & mask) == 0) {
        if (emit(r, x) < 0) { free(stack); free(seen); return -1; }
        continue;
      }
      for (int k = 0; k < 4; k++)
        if (r->u[x].src[k] >= 0 && !(r->u[x].op == U_REDUCE && k > 0)) stack[sp++] = r->u[x].src[k];
    }
    free(stack);
    free(seen);
  }
  const char *acc_t = is_float(r->u[v].dtype) ? "float" : alu_t(r->u[v].dtype);
  const char *init = kind == RED_SUM ? "0" : (is_float(r->u[v].dtype) ? "-INFINITY" : "(-2147483647 - 1)");
  sb_put(r->s, "  %s v%d = %s;\n", acc_t, i, init);
  const int group = r->group;
  if (group) {
    sb_put(r->s, "  {\n  const int rn%d = 1", i);
    for (int k = 0; k < na; k++) {
      const ThvmUop *rg = &r->u[axes[k]];
      if (rg->src[0] >= 0) sb_put(r->s, " * (int)v%d", rg->src[0]);
      else sb_put(r->s, " * %lld", (long long)rg->arg[2]);
    }
    sb_put(r->s, ";\n  for (int rr = gl_; rr < rn%d; rr += %d) {\n    int rq = rr;\n", i, group);
    for (int k = na - 1; k >= 0; k--) {
      const ThvmUop *rg = &r->u[axes[k]];
      char ext[48];
      if (rg->src[0] >= 0) snprintf(ext, sizeof ext, "(int)v%d", rg->src[0]);
      else snprintf(ext, sizeof ext, "%lld", (long long)rg->arg[2]);
      sb_put(r->s, "    const int a%lld = rq %% %s; rq /= %s;\n", (long long)rg->arg[0], ext, ext);
    }
  } else {
    for (int k = 0; k < na; k++) {
      const ThvmUop *rg = &r->u[axes[k]];
      if (rg->src[0] >= 0)
        sb_put(r->s, "  for (int a%lld = 0; a%lld < (int)v%d; a%lld++) {\n", (long long)rg->arg[0],
               (long long)rg->arg[0], rg->src[0], (long long)rg->arg[0]);
      else
        sb_put(r->s, "  for (int a%lld = 0; a%lld < %lld; a%lld++) {\n", (long long)rg->arg[0],
               (long long)rg->arg[0], (long long)rg->arg[2], (long long)rg->arg[0]);
    }
  }
  r->cur_level++;
  if (emit(r, v) < 0) return -1;
  if (kind == RED_SUM) sb_put(r->s, "  v%d += (%s)v%d;\n", i, acc_t, v);
  else if (is_float(r->u[v].dtype)) sb_put(r->s, "  v%d = fmaxf(v%d, (float)v%d);\n", i, i, v);
  else sb_put(r->s, "  v%d = v%d > v%d ? v%d : v%d;\n", i, i, v, i, v);
  /* leave the loop scope */
  for (uint32_t x = 0; x < r->n; x++)
    if (r->level[x] >= r->cur_level) r->level[x] = -1;
  r->cur_level--;
  if (group) {
    sb_put(r->s, "  }\n  }\n");
    /* the group's combine, every lane of the group ends with the result */
    const int fl = is_float(r->u[v].dtype);
    if (!fl && strcmp(acc_t, "int") != 0) {
      snprintf(r->err, sizeof r->err, "node %d: group reduce of a %s value", i, acc_t);
      return -1;
    }
    char comb[96];      /* combine t_ into v */
    if (kind == RED_SUM) snprintf(comb, sizeof comb, "v%d = v%d + t_", i, i);
    else if (fl) snprintf(comb, sizeof comb, "v%d = fmaxf(v%d, t_)", i, i);
    else snprintf(comb, sizeof comb, "v%d = t_ > v%d ? t_ : v%d", i, i, i);
    const char *ty = fl ? "float" : "int";
    if (group <= 64) {  /* the group's lanes are one aligned slice of a wave: xor tree */
      sb_put(r->s, "  for (int o = %d; o > 0; o >>= 1) { const %s t_ = __shfl_xor(v%d, o, 64); %s; }\n",
             group / 2, ty, i, comb);
    } else {            /* whole waves: the wave tree, then the group's waves in order through LDS */
      const char *wf = kind == RED_SUM ? (fl ? "wsum" : "wsumi") : (fl ? "wmax" : "wmaxi");
      const char *ra = fl ? "red_" : "redi_";
      sb_put(r->s,
             "  v%d = %s(v%d);\n"
             "  if ((threadIdx.x & 63u) == 0) %s[threadIdx.x >> 6] = v%d;\n"
             "  __syncthreads();\n"
             "  {\n    const int w0_ = (int)(threadIdx.x / %d) * %d;\n"
             "    v%d = %s[w0_];\n"
             "    for (int w = 1; w < %d; w++) { const %s t_ = %s[w0_ + w]; %s; }\n  }\n"
             "  __syncthreads();\n",
             i, wf, i, ra, i, group, group / 64, i, ra, group / 64, ty, ra, comb);
    }
  } else {
    for (int k = 0; k < na; k++) sb_put(r->s, "  }\n");
  }
  r->level[i] = r->cur_level;
  return i;
}

static const char *bin_op(uint32_t op) {
  switch (op) {
    case U_ADD: case U_IADD: return "+";
    case U_MUL: case U_IMUL: return "*";
    case U_ISUB: return "-";
    case U_IDIV: return "/";
    case U_IMOD: return "%";
    case U_IAND: return "&";
    case U_IOR: return "|";
    case U_IXOR: return "^";
    case U_ISHL: return "<<";
    case U_ISHR: return ">>";
    default: return NULL;
  }
}

static int emit(R *r, int i) {
  if (i < 0 || (uint32_t)i >= r->n) { snprintf(r->err, sizeof r->err, "bad node index %d", i); return -1; }
  if (r->level[i] >= 0) return i;
  if (++r->depth > 4000) { snprintf(r->err, sizeof r->err, "DAG too deep"); return -1; }
  const ThvmUop *u = &r->u[i];
  for (int k = 0; k < 4; k++)
    if (u->src[k] >= i) { snprintf(r->err, sizeof r->err, "node %d: source %d is not earlier", i, u->src[k]); return -1; }
  const char *at = alu_t(u->dtype);
  /* fp16 / bf16 values narrow only where the reference's CPU path narrows
   * them (src/backend/cpu/uop_walk.c:272-293, :725-737): at a CAST into the
   * type and at the STORE; every other op keeps its f32 value */
  const char *rf = u->op == U_CAST ? round_fn(u->dtype) : "";
  int rc = 0;
  switch (u->op) {
    case U_CONST: emit_const(r, i); break;
    case U_DEFINE_VAR:
      sb_put(r->s, "  const int v%d = kv_[%lld];\n", i, (long long)u->arg[0]);
      break;
    case U_RANGE:
      if (r->is_red_axis[i] >= 0 && r->cur_level == 0) {
        snprintf(r->err, sizeof r->err, "node %d: reduce axis %lld read outside its reduce", i, (long long)u->arg[0]);
        return -1;
      }
      sb_put(r->s, "  const int v%d = a%lld;\n", i, (long long)u->arg[0]);
      break;
    case U_REDUCE: rc = emit_reduce(r, i); break;
    case U_BUFFER: break;   /* named by its slot */
    case U_INDEX_E: {      /* the element of buffer src0 at index src1 (a load) */
      const ThvmUop *b = u->src[0] >= 0 ? &r->u[u->src[0]] : NULL;
      if (!b || b->op != U_BUFFER) { snprintf(r->err, sizeof r->err, "node %d: INDEX of a non-BUFFER", i); return -1; }
      if (emit(r, u->src[1]) < 0) return -1;
      const char *conv = b->dtype == THVM_DT_BF16 ? "bf2f" : b->dtype == THVM_DT_FP8E4M3 ? "fp8e4m3_f" : "";
      if (b->arg[1] > 0)   /* capacity known: an index outside the buffer reads 0 */
        sb_put(r->s, "  const %s v%d = (unsigned long long)v%d < %lldull ? (%s)%s(s%lld[v%d]) : (%s)0;\n",
               alu_t(b->dtype), i, u->src[1], (long long)b->arg[1], alu_t(b->dtype), conv,
               (long long)b->arg[0], u->src[1], alu_t(b->dtype));
      else
        sb_put(r->s, "  const %s v%d = (%s)%s(s%lld[v%d]);\n", alu_t(b->dtype), i, alu_t(b->dtype), conv,
               (long long)b->arg[0], u->src[1]);
      break;
    }
    case U_LOAD: {         /* an explicit read of an INDEX: its value */
      const int ix = u->src[0];
      if (ix < 0 || r->u[ix].op != U_INDEX_E) { snprintf(r->err, sizeof r->err, "node %d: LOAD of a non-INDEX", i); return -1; }
      if (emit(r, ix) < 0) return -1;
      sb_put(r->s, "  const %s v%d = v%d;\n", alu_t(r->u[r->u[ix].src[0]].dtype), i, ix);
      break;
    }
    case U_NEG: case U_RECIP: case U_EXP2: case U_LOG2: case U_SQRT: case U_SIN: {
      if (emit(r, u->src[0]) < 0) return -1;
      const int a = u->src[0];
      const char *f = u->op == U_NEG ? "-" : u->op == U_RECIP ? "1.0f / " : u->op == U_EXP2 ? "exp2f" :
                      u->op == U_LOG2 ? "log2f" : u->op == U_SQRT ? "sqrtf" : "sinf";
      if (!is_float(u->dtype) && u->op != U_NEG) { snprintf(r->err, sizeof r->err, "node %d: float op on an int", i); return -1; }
      sb_put(r->s, "  const %s v%d = %s(%s(v%d));\n", at, i, rf, f, a);
      break;
    }
    case U_ADD: case U_MUL: case U_IADD: case U_ISUB: case U_IMUL: case U_IDIV: case U_IMOD:
    case U_IAND: case U_IOR: case U_IXOR: case U_ISHL: case U_ISHR: {
      if (emit(r, u->src[0]) < 0 || emit(r, u->src[1]) < 0) return -1;
      sb_put(r->s, "  const %s v%d = %s((%s)v%d %s (%s)v%d);\n", at, i, rf, at, u->src[0], bin_op(u->op), at,
             u->src[1]);
      break;
    }
    case U_CMPLT: case U_CMPEQ: case U_ILT: {
      if (emit(r, u->src[0]) < 0 || emit(r, u->src[1]) < 0) return -1;
      sb_put(r->s, "  const %s v%d = (v%d %s v%d) ? (%s)1 : (%s)0;\n", at, i, u->src[0],
             u->op == U_CMPEQ ? "==" : "<", u->src[1], at, at);
      break;
    }
    case U_IWHERE: {
      if (emit(r, u->src[0]) < 0 || emit(r, u->src[1]) < 0 || emit(r, u->src[2]) < 0) return -1;
      sb_put(r->s, "  const %s v%d = (v%d != 0) ? (%s)v%d : (%s)v%d;\n", at, i, u->src[0], at, u->src[1], at,
             u->src[2]);
      break;
    }
    case U_CAST: {
      if (emit(r, u->src[0]) < 0) return -1;
      const uint32_t sd = r->u[u->src[0]].dtype;
      if (u->dtype == THVM_DT_BOOL)
        sb_put(r->s, "  const int v%d = (v%d != 0) ? 1 : 0;\n", i, u->src[0]);
      else if (is_float(u->dtype))
        sb_put(r->s, "  const %s v%d = %s((%s)v%d);\n", at, i, rf, at, u->src[0]);
      else if (is_float(sd))   /* float -> int truncates toward zero */
        sb_put(r->s, "  const %s v%d = (%s)v%d;\n", at, i, at, u->src[0]);
      else
        sb_put(r->s, "  const %s v%d = (%s)v%d;\n", at, i, at, u->src[0]);
      break;
    }
    case U_BITCAST: {
      if (emit(r, u->src[0]) < 0) return -1;
      const uint32_t sd = r->u[u->src[0]].dtype;
      if (sd == THVM_DT_FP32 && (u->dtype == THVM_DT_INT32 || u->dtype == THVM_DT_UINT32))
        sb_put(r->s, "  const %s v%d = (%s)__float_as_uint(v%d);\n", at, i, at, u->src[0]);
      else if ((sd == THVM_DT_INT32 || sd == THVM_DT_UINT32) && u->dtype == THVM_DT_FP32)
        sb_put(r->s, "  const float v%d = __uint_as_float((uint)v%d);\n", i, u->src[0]);
      else { snprintf(r->err, sizeof r->err, "node %d: bitcast %u -> %u", i, sd, u->dtype); return -1; }
      break;
    }
    default:
      snprintf(r->err, sizeof r->err, "node %d: op %u is not rendered by this target", i, u->op);
      return -1;
  }
  r->depth--;
  if (rc < 0) return -1;
  r->level[i] = r->cur_level;
  return i;
}

/* upper bound of an integer extent expression at the variables' maxima */
static int64_t ubound(const ThvmUop *u, int i, int *ok) {
  const ThvmUop *x = &u[i];
  switch (x->op) {
    case U_CONST: return x->arg[0];
    case U_DEFINE_VAR: return x->arg[2];
    case U_IADD: return ubound(u, x->src[0], ok) + ubound(u, x->src[1], ok);
    case U_IMUL: return ubound(u, x->src[0], ok) * ubound(u, x->src[1], ok);
    default: *ok = 0; return 0;
  }
}

static int is_pow2(uint32_t x) { return x && !(x & (x - 1)); }
static uint32_t pow2_floor(uint64_t x) {
  uint32_t p = 1;
  while ((uint64_t)p * 2 <= x && p < (1u << 30)) p *= 2;
  return p;
}

/* The geometry the target picks without a search (the role of the
 * reference's hand-coded opts, src/codegen/hand_opts.c:337-802, for gfx950):
 * an un-nested reduction of length R >= 64 over O outputs shares each output
 * among G = min(R / 4, 524288 / O, 1024) threads (powers of 2: at least 4
 * terms per thread, at most about 512K threads in all), one thread per output
 * where that leaves G below 16 (enough outputs to fill the machine one
 * thread each); blocks of max(G, 256) threads.  Few outputs get wide groups
 * (a thread's terms are a serial chain of loads); many outputs get one
 * thread each.  Measured on gfx950 with the search (f32 rows,
 * thvm_hip_render_autotune): 50257 x 768 wants one thread per row,
 * 4096 x 4096 a group of 128, 64 x 65536 groups of 1024.  Everything else
 * runs one output per thread in 256-thread blocks. */
static void hand_opts(int has_red, int nested, int64_t red_len, uint64_t outputs, ThvmRenderOpts *o) {
  memset(o, 0, sizeof *o);
  o->block = RENDER_BLOCK;
  o->upcast = 1;
  o->group = 1;
  if (has_red && !nested && red_len >= 64) {
    uint32_t g = pow2_floor((uint64_t)red_len / 4);
    const uint32_t by_out = pow2_floor(outputs ? (524288 + outputs - 1) / outputs : 1);
    if (by_out < g) g = by_out;
    if (g > 1024) g = 1024;
    if (g >= 16) {
      o->group = g;
      if (g > o->block) o->block = g;
    }
  }
}

/* ---- matmuls on MFMA ------------------------------------------------------
 * The reference renders a tensor-core matmul when its scheduler marks one
 * (WMMA 16x16x16 tiles over shared-memory staging, src/codegen/render_uop.c
 * :1690-1986, :2380-2560).  This target recognises the same computation in
 * the lifted DAG itself:
 *   STORE(out, f(m, n), epilogue(REDUCE_SUM over k (MUL(A[addr_a(m, k)],
 *                                                        B[addr_b(k, n)]))))
 * with A and B fp16 or bf16 of one type (read directly or through a widening
 * CAST / LOAD), exactly two parallel axes m and n of static extents that are
 * multiples of 16, one or two reduce axes forming a flat k (extent a
 * multiple of 16; with two, the outer axis steps A and B by the inner one's
 * extent times its step), and both addresses affine in m, n and k.  Each
 * wave computes one 16x16 output tile with v_mfma_f32_16x16x32 (or x16 at a
 * k extent that is not a multiple of 32): lane l reads A at m = l%16 and B at
 * n = l%16 for the 8 (4) k of its lane group, products exact, f32
 * accumulation; the four results of a lane (rows 4 (l/16) + i, column l%16)
 * then run the DAG's own epilogue and store through the generic emitter, so
 * bias, activation and the narrowing at CAST / STORE are the DAG's.  The sum
 * differs from the walker's serial f32 sum only in its order.  Anything
 * else, and every launch with explicit opts, takes the generic path. */
#define MF_AX 64     /* axis ids the affine analysis tracks */

/* x = c + sum_a coef[a] * axis_a, or 0 when the expression is not affine */
static int affine(const ThvmUop *u, int i, int64_t *c, int64_t *coef, int depth) {
  if (i < 0 || depth > 64) return 0;
  const ThvmUop *x = &u[i];
  memset(coef, 0, sizeof(int64_t) * MF_AX);
  *c = 0;
  switch (x->op) {
    case U_CONST: *c = x->arg[0]; return 1;
    case U_RANGE:
      if (x->arg[0] < 0 || x->arg[0] >= MF_AX) return 0;
      coef[x->arg[0]] = 1;
      return 1;
    case U_IADD: case U_ISUB: case U_IMUL: {
      int64_t c0, c1, k0[MF_AX], k1[MF_AX];
      if (!affine(u, x->src[0], &c0, k0, depth + 1) || !affine(u, x->src[1], &c1, k1, depth + 1)) return 0;
      if (x->op == U_IMUL) {
        int lin0 = 0, lin1 = 0;
        for (int a = 0; a < MF_AX; a++) { lin0 |= k0[a] != 0; lin1 |= k1[a] != 0; }
        if (lin0 && lin1) return 0;
        const int64_t m = lin0 ? c1 : c0;
        const int64_t *kk = lin0 ? k0 : k1;
        *c = c0 * c1;
        for (int a = 0; a < MF_AX; a++) coef[a] = kk[a] * m;
        return 1;
      }
      const int64_t sg = x->op == U_ISUB ? -1 : 1;
      *c = c0 + sg * c1;
      for (int a = 0; a < MF_AX; a++) coef[a] = k0[a] + sg * k1[a];
      return 1;
    }
    default: return 0;
  }
}

/* the INDEX an operand of the MUL reads, through a widening CAST / LOAD */
static int mf_operand(const ThvmUop *u, int i) {
  for (int d = 0; d < 4 && i >= 0; d++) {
    const ThvmUop *x = &u[i];
    if (x->op == U_INDEX_E) return i;
    if (x->op == U_LOAD) { i = x->src[0]; continue; }
    if (x->op == U_CAST && (x->dtype == THVM_DT_FP32 || x->dtype == u[x->src[0]].dtype)) { i = x->src[0]; continue; }
    return -1;
  }
  return -1;
}

typedef struct {
  int red, ia, ib, m_ax, n_ax;
  int64_t M, N, K, ca, cam, cak, cb, cbn, cbk, capa, capb;
  int slot_a, slot_b;
  uint32_t dt;
} MfPlan;

/* the MFMA plan of a DAG, or 0 */
static int mf_match(const ThvmUop *u, uint32_t n, const int *par, int npar, const int *is_red_axis, MfPlan *p) {
  memset(p, 0, sizeof *p);
  p->red = -1;
  for (uint32_t i = 0; i < n; i++) {
    if (u[i].op == U_DEFINE_VAR) return 0;
    if (u[i].op == U_REDUCE) { if (p->red >= 0) return 0; p->red = (int)i; }
  }
  if (p->red < 0 || npar != 2) return 0;
  const ThvmUop *rd = &u[p->red];
  if (rd->arg[0] != RED_SUM || rd->src[3] >= 0 || rd->src[1] < 0) return 0;
  const ThvmUop *mul = &u[rd->src[0]];
  if (mul->op != U_MUL) return 0;
  p->ia = mf_operand(u, mul->src[0]);
  p->ib = mf_operand(u, mul->src[1]);
  if (p->ia < 0 || p->ib < 0) return 0;
  const ThvmUop *ba = &u[u[p->ia].src[0]], *bb = &u[u[p->ib].src[0]];
  if (ba->op != U_BUFFER || bb->op != U_BUFFER || ba->dtype != bb->dtype ||
      (ba->dtype != THVM_DT_FP16 && ba->dtype != THVM_DT_BF16))
    return 0;
  p->dt = ba->dtype;
  p->slot_a = (int)ba->arg[0];
  p->slot_b = (int)bb->arg[0];
  p->capa = ba->arg[1];
  p->capb = bb->arg[1];
  int64_t ka[MF_AX], kb[MF_AX];
  if (!affine(u, u[p->ia].src[1], &p->ca, ka, 0) || !affine(u, u[p->ib].src[1], &p->cb, kb, 0)) return 0;
  /* m and n: the parallel axes A and B read, one each */
  for (int t = 0; t < 2; t++) {
    const ThvmUop *rg = &u[par[t]];
    if (rg->src[0] >= 0 || rg->arg[0] < 0 || rg->arg[0] >= MF_AX) return 0;
  }
  const int64_t a0 = u[par[0]].arg[0], a1 = u[par[1]].arg[0];
  if (ka[a0] && !kb[a0] && kb[a1] && !ka[a1]) { p->m_ax = (int)a0; p->n_ax = (int)a1; p->M = u[par[0]].arg[2]; p->N = u[par[1]].arg[2]; }
  else if (ka[a1] && !kb[a1] && kb[a0] && !ka[a0]) { p->m_ax = (int)a1; p->n_ax = (int)a0; p->M = u[par[1]].arg[2]; p->N = u[par[0]].arg[2]; }
  else return 0;
  p->cam = ka[p->m_ax];
  p->cbn = kb[p->n_ax];
  /* k: one axis, or two forming a flat index (outer step = inner extent x inner step) */
  int ax[2] = {rd->src[1], rd->src[2]}, na = rd->src[2] >= 0 ? 2 : 1;
  for (int t = 0; t < na; t++)
    if (u[ax[t]].op != U_RANGE || u[ax[t]].src[0] >= 0 || u[ax[t]].arg[0] < 0 || u[ax[t]].arg[0] >= MF_AX ||
        is_red_axis[ax[t]] < 0)
      return 0;
  if (na == 1) {
    const int64_t k0 = u[ax[0]].arg[0];
    p->K = u[ax[0]].arg[2];
    p->cak = ka[k0];
    p->cbk = kb[k0];
  } else {
    const int64_t k0 = u[ax[0]].arg[0], k1 = u[ax[1]].arg[0];
    const int64_t e0 = u[ax[0]].arg[2], e1 = u[ax[1]].arg[2];
    if (ka[k0] == e1 * ka[k1] && kb[k0] == e1 * kb[k1]) {          /* k = a0 * e1 + a1 */
      p->cak = ka[k1]; p->cbk = kb[k1];
    } else if (ka[k1] == e0 * ka[k0] && kb[k1] == e0 * kb[k0]) {   /* k = a1 * e0 + a0 */
      p->cak = ka[k0]; p->cbk = kb[k0];
    } else {
      return 0;
    }
    p->K = e0 * e1;
  }
  /* no other axis in the operand addresses; a k step of 0 is a broadcast, not a matmul */
  for (int a = 0; a < MF_AX; a++) {
    const int used = a == p->m_ax || a == p->n_ax;
    int isk = 0;
    for (int t = 0; t < na; t++) isk |= u[ax[t]].arg[0] == a;
    if (!used && !isk && (ka[a] || kb[a])) return 0;
  }
  if (p->cak == 0 || p->cbk == 0) return 0;
  if (p->M <= 0 || p->N <= 0 || p->K <= 0 || p->M % 16 || p->N % 16 || p->K % 16) return 0;
  if (p->M * p->N > (1ll << 31)) return 0;
  return 1;
}

/* the STORE of the value node vi at address ai (a guard when the output's
 * capacity is known), into out slot 0 of dtype odt */
static void emit_store_line(Sb *sb, const ThvmUop *st, const ThvmUop *nodes, uint32_t odt, const char *cond0) {
  char val[64];
  const int vi = st->src[2], ai = st->src[1];
  if (odt == THVM_DT_BF16) snprintf(val, sizeof val, "f2bf((float)v%d)", vi);
  else if (odt == THVM_DT_FP16) snprintf(val, sizeof val, "(_Float16)(float)v%d", vi);
  else if (odt == THVM_DT_BOOL) snprintf(val, sizeof val, "(unsigned char)(v%d != 0)", vi);
  else if (odt == THVM_DT_FP8E4M3) snprintf(val, sizeof val, "f2fp8e4m3((float)v%d)", vi);
  else snprintf(val, sizeof val, "(%s)v%d", store_t(odt), vi);
  char guard[96] = "";
  const int64_t cap0 = nodes[st->src[0]].arg[1];
  if (cap0 > 0) snprintf(guard, sizeof guard, "(unsigned long long)v%d < %lldull", ai, (long long)cap0);
  char cond[192];
  snprintf(cond, sizeof cond, "%s%s%s", cond0, (cond0[0] && guard[0]) ? " && " : "", guard);
  if (cond[0]) sb_put(sb, "  if (%s) s0[v%d] = %s;\n", cond, ai, val);
  else sb_put(sb, "  s0[v%d] = %s;\n", ai, val);
}

static int render_mfma(R *r, const MfPlan *p, const char *name, const uint32_t *slot_dt, int nslot,
                       ThvmRenderInfo *info) {
  Sb *sb = r->s;
  const ThvmUop *u = r->u, *st = &u[r->n - 1];
  const int kw = p->K % 32 == 0 ? 32 : 16, per = kw / 4;     /* k per instruction, per lane */
  const int64_t TN = p->N / 16, tiles = (p->M / 16) * TN;
  const int bf = p->dt == THVM_DT_BF16;
  sb_put(sb, "%s\n", PRELUDE);
  sb_put(sb, "typedef float mf_f4 __attribute__((ext_vector_type(4)));\n");
  if (kw == 32)
    sb_put(sb, "typedef %s mf_op __attribute__((ext_vector_type(8)));\n", bf ? "__bf16" : "_Float16");
  else
    sb_put(sb, "typedef %s mf_op __attribute__((ext_vector_type(4)));\n", bf ? "short" : "_Float16");
  sb_put(sb, "extern \"C\" __global__ void __launch_bounds__(256) %s(\n", name);
  for (int k = 0; k < nslot; k++)
    sb_put(sb, "    %s%s *__restrict__ s%d%s\n", k ? "const " : "", store_t(slot_dt[k]), k, k + 1 < nslot ? "," : "");
  sb_put(sb, ") {\n");
  sb_put(sb, "  /* MFMA matmul: %lldx%lldx%lld, one 16x16 tile per wave, k %d per instruction */\n",
         (long long)p->M, (long long)p->N, (long long)p->K, kw);
  sb_put(sb,
         "  const long long tw_ = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);\n"
         "  if (tw_ >= %lldll) return;\n"
         "  const int ln_ = (int)(threadIdx.x & 63u);\n"
         "  const long long tm_ = tw_ / %lldll, tn_ = tw_ %% %lldll;\n"
         "  const unsigned short *ra_ = (const unsigned short *)s%d, *rb_ = (const unsigned short *)s%d;\n"
         "  const long long ab_ = %lldll + %lldll * (tm_ * 16 + (ln_ & 15));\n"
         "  const long long bb_ = %lldll + %lldll * (tn_ * 16 + (ln_ & 15));\n"
         "  mf_f4 acc_ = {0.f, 0.f, 0.f, 0.f};\n"
         "  for (long long k0_ = 0; k0_ < %lldll; k0_ += %d) {\n"
         "    unsigned short av_[%d], bv_[%d];\n"
         "    for (int j = 0; j < %d; j++) {\n"
         "      const long long k_ = k0_ + %d * (ln_ >> 4) + j;\n"
         "      const long long ia_ = ab_ + %lldll * k_, ib_ = bb_ + %lldll * k_;\n",
         (long long)tiles, (long long)TN, (long long)TN, p->slot_a, p->slot_b, (long long)p->ca, (long long)p->cam,
         (long long)p->cb, (long long)p->cbn, (long long)p->K, kw, per, per, per, per, (long long)p->cak,
         (long long)p->cbk);
  if (p->capa > 0) sb_put(sb, "      av_[j] = (unsigned long long)ia_ < %lldull ? ra_[ia_] : (unsigned short)0;\n", (long long)p->capa);
  else sb_put(sb, "      av_[j] = ra_[ia_];\n");
  if (p->capb > 0) sb_put(sb, "      bv_[j] = (unsigned long long)ib_ < %lldull ? rb_[ib_] : (unsigned short)0;\n", (long long)p->capb);
  else sb_put(sb, "      bv_[j] = rb_[ib_];\n");
  sb_put(sb, "    }\n");
  if (kw == 32)
    sb_put(sb, "    acc_ = __builtin_amdgcn_mfma_f32_16x16x32_%s(__builtin_bit_cast(mf_op, av_), "
           "__builtin_bit_cast(mf_op, bv_), acc_, 0, 0, 0);\n", bf ? "bf16" : "f16");
  else
    sb_put(sb, "    acc_ = __builtin_amdgcn_mfma_f32_16x16x16%s(__builtin_bit_cast(mf_op, av_), "
           "__builtin_bit_cast(mf_op, bv_), acc_, 0, 0, 0);\n", bf ? "bf16_1k" : "f16");
  sb_put(sb, "  }\n");
  /* each lane's 4 results through the DAG's epilogue and store */
  sb_put(sb, "  for (int i_ = 0; i_ < 4; i_++) {\n"
         "  const int a%d = (int)(tm_ * 16 + 4 * (ln_ >> 4) + i_);\n"
         "  const int a%d = (int)(tn_ * 16 + (ln_ & 15));\n"
         "  const float v%d = acc_[i_];\n", p->m_ax, p->n_ax, p->red);
  r->level[p->red] = 0;
  if (emit(r, st->src[1]) < 0 || emit(r, st->src[2]) < 0) return -1;
  emit_store_line(sb, st, u, slot_dt[0], "");
  sb_put(sb, "  }\n}\n");
  info->n_slots = (uint32_t)nslot;
  info->kvar_slot = 0;
  info->group = 1;
  info->block = 256;
  info->upcast = 1;
  info->grid_max = (uint64_t)(tiles + 3) / 4;
  return 0;
}

static int render_impl(const ThvmUop *nodes, uint32_t n, const char *name, const ThvmRenderOpts *opts,
                       char *out, uint64_t cap, ThvmRenderInfo *info) {
  if (!nodes || n == 0 || !name || !out || cap < 1024 || !info) {
    hb_set_error("render: bad arguments");
    return -1;
  }
  memset(info, 0, sizeof *info);
  const int root = (int)n - 1;
  const ThvmUop *st = &nodes[root];
  if (st->op != U_STORE || st->src[0] < 0 || nodes[st->src[0]].op != U_BUFFER || nodes[st->src[0]].arg[0] != 0) {
    hb_set_error("render: the last node must be a STORE into buffer slot 0");
    return -1;
  }
  R r;
  memset(&r, 0, sizeof r);
  r.u = nodes;
  r.n = n;
  r.dep = (uint64_t *)calloc(n, sizeof(uint64_t));
  r.level = (int *)malloc(n * sizeof(int));
  r.is_red_axis = (int *)malloc(n * sizeof(int));
  Sb sb = {out, 0, cap, 0};
  r.s = &sb;
  int rc = -1;
  if (!r.dep || !r.level || !r.is_red_axis) { hb_set_error("render: out of memory"); goto done; }
  for (uint32_t i = 0; i < n; i++) { r.level[i] = -1; r.is_red_axis[i] = -1; }

  /* slots and variables */
  uint32_t slot_dt[RENDER_MAX_SLOTS];
  int slot_used[RENDER_MAX_SLOTS] = {0};
  int nvar = 0, nslot = 0;
  for (uint32_t i = 0; i < n; i++) {
    const ThvmUop *u = &nodes[i];
    for (int k = 0; k < 4; k++)
      if (u->src[k] >= (int32_t)i) { hb_set_error("render: node %u reads a later node", i); goto done; }
    if (u->op == U_BUFFER) {
      const int64_t sl = u->arg[0];
      if (sl < 0 || sl >= RENDER_MAX_SLOTS || !store_t(u->dtype)) { hb_set_error("render: buffer slot %lld / dtype %u", (long long)sl, u->dtype); goto done; }
      if (slot_used[sl] && slot_dt[sl] != u->dtype) { hb_set_error("render: slot %lld has two dtypes", (long long)sl); goto done; }
      slot_used[sl] = 1;
      slot_dt[sl] = u->dtype;
      if ((int)sl + 1 > nslot) nslot = (int)sl + 1;
    } else if (u->op == U_DEFINE_VAR) {
      if (u->arg[0] < 0 || u->arg[0] >= 64) { hb_set_error("render: variable index %lld", (long long)u->arg[0]); goto done; }
      if ((int)u->arg[0] + 1 > nvar) nvar = (int)u->arg[0] + 1;
    }
  }
  /* a slot no BUFFER row names is an argument the kernel does not read (the
   * reference schedules such inputs): it is declared as bytes */
  for (int k = 0; k < nslot; k++)
    if (!slot_used[k]) slot_dt[k] = THVM_DT_UINT8;
  if (!slot_used[0]) { hb_set_error("render: the output slot 0 is never declared"); goto done; }

  /* reduce axes, dependence masks, nesting */
  int nred = 0;
  for (uint32_t i = 0; i < n; i++)
    if (nodes[i].op == U_REDUCE)
      for (int k = 1; k < 4; k++) {
        const int a = nodes[i].src[k];
        if (a < 0) continue;
        if (nodes[a].op != U_RANGE) { hb_set_error("render: reduce %u axis is not a RANGE", i); goto done; }
        if (r.is_red_axis[a] < 0) {
          if (nred >= RENDER_MAX_RANGES) { hb_set_error("render: too many reduce axes"); goto done; }
          r.is_red_axis[a] = nred++;
        }
      }
  int nested = 0, has_red = 0;
  int64_t red_len_min = INT64_MAX;
  for (uint32_t i = 0; i < n; i++) {
    const ThvmUop *u = &nodes[i];
    uint64_t d = 0;
    if (u->op == U_RANGE && r.is_red_axis[i] >= 0) d = 1ull << r.is_red_axis[i];
    for (int k = 0; k < 4; k++) {
      if (u->src[k] < 0) continue;
      if (u->op == U_REDUCE && k > 0) continue;
      d |= r.dep[u->src[k]];
    }
    if (u->op == U_REDUCE) {
      for (int k = 1; k < 4; k++)
        if (u->src[k] >= 0) d &= ~(1ull << r.is_red_axis[u->src[k]]);
      if (d) nested = 1;
      has_red = 1;
      int ok = 1;
      int64_t len = 1;
      for (int k = 1; k < 4; k++) {
        const int a = u->src[k];
        if (a < 0) continue;
        len *= nodes[a].src[0] >= 0 ? ubound(nodes, nodes[a].src[0], &ok) : nodes[a].arg[2];
      }
      if (ok && len < red_len_min) red_len_min = len;
    }
    r.dep[i] = d;
  }

  /* parallel axes: every RANGE that no REDUCE binds, in axis-id order */
  int par[RENDER_MAX_RANGES], npar = 0;
  for (uint32_t i = 0; i < n; i++)
    if (nodes[i].op == U_RANGE && r.is_red_axis[i] < 0) {
      if (npar >= RENDER_MAX_RANGES) { hb_set_error("render: too many axes"); goto done; }
      par[npar++] = (int)i;
    }
  for (int a = 1; a < npar; a++)     /* insertion sort by axis id */
    for (int b = a; b > 0 && nodes[par[b]].arg[0] < nodes[par[b - 1]].arg[0]; b--) {
      int t = par[b]; par[b] = par[b - 1]; par[b - 1] = t;
    }
  uint64_t total_max = 1;
  for (int a = 0; a < npar; a++) {
    const ThvmUop *rg = &nodes[par[a]];
    int ok = 1;
    const int64_t e = rg->src[0] >= 0 ? ubound(nodes, rg->src[0], &ok) : rg->arg[2];
    if (!ok || e < 0) { hb_set_error("render: axis %lld has no upper bound", (long long)rg->arg[0]); goto done; }
    total_max *= (uint64_t)e;
  }
  if (total_max > (1ull << 31)) { hb_set_error("render: %llu output elements", (unsigned long long)total_max); goto done; }
  ThvmRenderOpts o;
  if (opts) {
    o = *opts;
    if (o.block == 0) o.block = RENDER_BLOCK;
    if (o.group == 0) o.group = 1;
    if (o.upcast == 0) o.upcast = 1;
    if (!is_pow2(o.block) || o.block < 64 || o.block > 1024 || !is_pow2(o.group) || o.group > o.block ||
        o.upcast > 8) {
      hb_set_error("render: opts block %u (64..1024, a power of 2), group %u (a power of 2 <= block), "
                   "upcast %u (1..8)", o.block, o.group, o.upcast);
      goto done;
    }
    if (o.group > 1 && (!has_red || nested)) {
      hb_set_error("render: a group applies to un-nested reductions");
      goto done;
    }
    if (o.group > 1 && o.upcast > 1) { hb_set_error("render: upcast applies to one thread per output"); goto done; }
  } else {
    hand_opts(has_red, nested, red_len_min == INT64_MAX ? 0 : red_len_min, total_max, &o);
  }
  r.group = o.group > 1 ? (int)o.group : 0;
  r.block = (int)o.block;
  if (!opts && nvar == 0) {      /* a matmul runs on MFMA (hand-coded path only) */
    MfPlan mp;
    if (mf_match(nodes, n, par, npar, r.is_red_axis, &mp)) {
      if (render_mfma(&r, &mp, name, slot_dt, nslot, info) < 0) goto bad;
      if (sb.bad) { hb_set_error("render: source exceeds %llu bytes", (unsigned long long)cap); goto done; }
      rc = 0;
      goto done;
    }
  }

  /* source */
  sb_put(&sb, "%s\n", PRELUDE);
  sb_put(&sb, "extern \"C\" __global__ void __launch_bounds__(%d) %s(\n", r.block, name);
  for (int k = 0; k < nslot; k++)
    sb_put(&sb, "    %s%s *__restrict__ s%d%s\n", k ? "const " : "", store_t(slot_dt[k]), k,
           (k + 1 < nslot || nvar) ? "," : "");
  if (nvar) sb_put(&sb, "    const int *__restrict__ kv_\n");
  sb_put(&sb, ") {\n");
  /* group mode: G consecutive threads per output, block/G outputs per block
   * (gl_ = the thread's place in its group); thread mode: upcast outputs per
   * thread, consecutive */
  const int G = r.group, U = (int)o.upcast;
  if (G)
    sb_put(&sb, "  __shared__ float red_[%d];\n  __shared__ int redi_[%d];\n  (void)red_; (void)redi_;\n"
           "  const int gl_ = (int)(threadIdx.x %% %d);\n"
           "  const long long gid = (long long)blockIdx.x * %d + threadIdx.x / %d;\n",
           r.block / 64, r.block / 64, G, r.block / G, G);
  else if (U > 1)
    sb_put(&sb, "  for (int uj_ = 0; uj_ < %d; uj_++) {\n"
           "  const long long gid = ((long long)blockIdx.x * %d + threadIdx.x) * %d + uj_;\n", U, r.block, U);
  else sb_put(&sb, "  const long long gid = (long long)blockIdx.x * %d + threadIdx.x;\n", r.block);
  /* extents of the parallel axes, then the element decomposition */
  for (int a = 0; a < npar; a++) {
    const ThvmUop *rg = &nodes[par[a]];
    if (rg->src[0] >= 0) {
      if (emit(&r, rg->src[0]) < 0) goto bad;
      sb_put(&sb, "  const long long e%d = (long long)v%d;\n", a, rg->src[0]);
    } else {
      sb_put(&sb, "  const long long e%d = %lldll;\n", a, (long long)rg->arg[2]);
    }
  }
  /* past the last output: a thread returns (one output per thread, or a
   * group within one wave: no block barrier follows); a group spanning waves
   * stays for the barriers of its reduction and skips the store */
  sb_put(&sb, "  const bool act_ = gid < 1ll");
  for (int a = 0; a < npar; a++) sb_put(&sb, " * e%d", a);
  sb_put(&sb, ";\n");
  if (G > 64) sb_put(&sb, "  long long q_ = act_ ? gid : 0;\n");
  else sb_put(&sb, "  if (!act_) %s;\n  long long q_ = gid;\n", U > 1 ? "break" : "return");
  for (int a = npar - 1; a >= 0; a--)
    sb_put(&sb, "  const int a%lld = (int)(q_ %% e%d); q_ /= e%d;\n", (long long)nodes[par[a]].arg[0], a, a);
  sb_put(&sb, "  (void)q_;\n");
  if (emit(&r, st->src[1]) < 0 || emit(&r, st->src[2]) < 0) goto bad;
  {
    char c0[32];
    snprintf(c0, sizeof c0, "%s%s", G ? "gl_ == 0" : "", G > 64 ? " && act_" : "");
    emit_store_line(&sb, st, nodes, slot_dt[0], c0);
    sb_put(&sb, "%s}\n", U > 1 && !G ? "  }\n" : "");
  }
  if (sb.bad) { hb_set_error("render: source exceeds %llu bytes", (unsigned long long)cap); goto done; }
  info->n_slots = (uint32_t)nslot + (nvar ? 1u : 0u);
  info->kvar_slot = nvar ? (uint32_t)nslot : 0u;
  info->group = (uint32_t)(G ? G : 1);
  info->block = (uint32_t)r.block;
  info->upcast = (uint32_t)U;
  {
    const uint64_t per_block = G ? (uint64_t)(r.block / G) : (uint64_t)r.block * (uint64_t)U;
    info->grid_max = (total_max + per_block - 1) / per_block;
  }
  if (info->grid_max == 0) info->grid_max = 1;
  rc = 0;
  goto done;
bad:
  hb_set_error("render: %s", r.err[0] ? r.err : "emit failed");
done:
  free(r.dep);
  free(r.level);
  free(r.is_red_axis);
  return rc;
}

THVM_API int thvm_hip_render_kernel(const ThvmUop *nodes, uint32_t n, const char *name, char *out,
                                    uint64_t cap, ThvmRenderInfo *info) {
  return render_impl(nodes, n, name, NULL, out, cap, info);
}

THVM_API int thvm_hip_render_kernel_opts(const ThvmUop *nodes, uint32_t n, const char *name,
                                         const ThvmRenderOpts *opts, char *out, uint64_t cap,
                                         ThvmRenderInfo *info) {
  return render_impl(nodes, n, name, opts, out, cap, info);
}
