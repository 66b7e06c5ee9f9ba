/* oracle.h -- TEST INFRASTRUCTURE ONLY.  CPU restatement of the reference
 * (sw1sh/thvm) CPU path for the decode hot path, used as the checker for the
 * HIP kernels.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it; the product library never links it.
 *
 * Every function states the reference file:line it restates.  Floating
 * point follows the reference CPU JIT: f32 arithmetic, serial loops in index
 * order, no contraction (built with -ffp-contract=off, reference
 * src/backend/cpu/jit.c:318-345), narrow floats rounded through storage at
 * the cast/store points (src/backend/cpu/uop_walk.c:272-293). */
#ifndef THVM_ORACLE_H
#define THVM_ORACLE_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- codecs (reference src/dtype/fp_convert.c, src/dtype/fp8.c) ---- */
float    or_bf16_to_f32(uint16_t b);
uint16_t or_f32_to_bf16(float v);
float    or_fp16_to_f32(uint16_t h);
uint16_t or_f32_to_fp16(float v);
float    or_fp8e4m3_to_f32(uint8_t x);
float    or_fp8e5m2_to_f32(uint8_t x);
uint8_t  or_f32_to_fp8e4m3(float v);       /* host encode (CONST payloads)   */
uint8_t  or_f32_to_fp8e4m3_sat(float v);   /* kernel-store encode            */
uint8_t  or_f32_to_fp8e5m2(float v);
uint8_t  or_f32_to_fp8e5m2_sat(float v);
/* bulk: dt is a THVM_DT_* id (FP32, FP16, BF16, FP8E4M3, FP8E5M2) */
void     or_decode(const void *src, uint32_t dt, float *dst, uint64_t n);
void     or_encode(const float *src, uint32_t dt, void *dst, uint64_t n); /* store form (fp8 sat) */

/* ---- ops ---- */
/* y[m*N+n] = sum_k x[m,k] * w~[n,k] (f32, k ascending), w~ = dequantised
 * weight (fp8: q*scale[n]).  Reference: the M=1 matvec of the CPU JIT loop
 * (src/backend/cpu/jit.c:667-743 rendering src/codegen/render_uop.c:4824-4932)
 * and the plain-C GEMV twin (bench/dsv2_decode_bench.c:1054-1085, sk=1). */
void or_gemv(float *y, const void *x, uint32_t xdt, uint32_t ldx,
             const void *w, uint32_t wdt, const float *scale,
             uint32_t M, uint32_t N, uint32_t K);
/* RMSNorm: ss serial, inv = 1/sqrtf(ss*(1/K) + eps), y = rnd((x*inv)*w)
 * (bench/dsv2_decode_bench.c:419-431 C twin; py/thvm/nn.py:211-224). */
void or_rmsnorm(void *y, uint32_t ydt, const void *x, uint32_t xdt, const float *w,
                uint32_t M, uint32_t K, float eps);
/* LayerNorm (src/nn/layernorm.c:1-7): (x-mean)*rsqrt(var+eps)*w + b. */
void or_layernorm(void *y, uint32_t ydt, const void *x, uint32_t xdt, const float *w,
                  const float *b, uint32_t M, uint32_t K, float eps);
/* softmax (src/nn/softmax.c:1-16): e = exp(x - max); y = e * (1/sum e). */
void or_softmax(void *y, uint32_t ydt, const void *x, uint32_t xdt, uint32_t M, uint32_t K);
/* RoPE, interleaved pairs at position pos, in place (dsv2 gred_q :474-483). */
void or_rope(void *x, uint32_t dt, const float *cos_t, const float *sin_t,
             uint32_t B, uint32_t nh, uint32_t hd, uint32_t pos);
/* single-query attention over cache rows [0, L): per head h (kv head h/G),
 * s_j = (q.k_j)*scale; p = exp(s - max); out = (sum p v) / sum p, rnd to odt
 * (src/nn/scaled_dot_product_attention.c:4-30; dsv2 mla_score C twin
 * :700-723 for the serial softmax). */
void or_attn_decode(void *out, uint32_t odt, const void *q, uint32_t qdt,
                    const void *kcache, const void *vcache, uint32_t cdt,
                    uint32_t B, uint32_t H, uint32_t Hkv, uint32_t hd,
                    uint32_t max_seq, uint32_t L, float scale);
/* argmax, lowest index on ties (dsv2 argmax_part/fin C twins :989-1020). */
void or_argmax(int32_t *tok, const float *logits, uint32_t B, uint32_t V);

/* ---- whole decode step ---- */
typedef struct OrLayer {
  const void *wqkv; const float *sqkv;   /* [(H+2Hkv)hd, D] (GPT2: c_attn [3D, D]) */
  const void *wo;   const float *so;     /* [D, H hd]                              */
  const void *wgu;  const float *sgu;    /* LLAMA [2F, D] rows (g0,u0,g1,u1..); GPT2 c_fc [F, D] */
  const void *wd;   const float *sd;     /* [D, F]                                 */
  const float *g1, *b1, *g2, *b2;        /* norm gains / LayerNorm biases          */
  const void *bqkv, *bo, *bfc, *bpr;     /* GPT2 biases (act dtype)                */
  void *kcache, *vcache;                 /* [B][Hkv][max_seq][hd] (act dtype)      */
} OrLayer;

typedef struct OrModel {
  uint32_t arch;                         /* 1 LLAMA, 2 GPT2                        */
  uint32_t n_layers, dim, n_heads, n_kv_heads, head_dim, ffn, vocab, max_seq, batch;
  uint32_t wdt, adt;
  float eps;
  const void *emb;                       /* [V, D] act dtype (GPT2 wte)            */
  const void *pos_emb;                   /* GPT2 wpe [max_seq, D]                  */
  const float *gf, *bf;                  /* final norm                             */
  const void *lm; const float *lm_s;     /* LLAMA LM head [V, D]; GPT2 uses emb    */
  const float *rope_cos, *rope_sin;      /* [max_seq, hd/2]                        */
  OrLayer *layers;
} OrModel;

/* One decode step for every batch row: token tok[b] at position pos (the
 * cache rows [0,pos) already hold the prefix).  Writes the k/v rows at pos,
 * logits [B][V] f32 and next[b] (greedy).  Returns 0, or -1 on bad config. */
int or_decode_step(const OrModel *m, const int32_t *tok, uint32_t pos,
                   float *logits, int32_t *next);

#ifdef __cplusplus
}
#endif
#endif
