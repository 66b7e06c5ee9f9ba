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
 *   linear / softmax / layernorm / rmsnorm on f32 through the reference's
 *             own Tensor graph + rangeify + CPU JIT (src/nn/dot.c,
 *             src/nn/softmax.c, src/nn/layernorm.c, py/thvm/nn.py:211-224). */
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
