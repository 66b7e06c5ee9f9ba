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
/* Temperature sampling as the device's argmax builtin runs it with temp > 0
 * (rowops.hip k_sample_part / k_sample_fin): the same exp (or_sexpf), block
 * partition into nb chunks, fold orders and two-level choice, and the draw
 * u = or_sample_u01(seed, row, L).  Rows whose logits are all -inf keep tok. */
float or_sexpf(float x);
float or_sample_u01(uint64_t seed, uint32_t row, int32_t L);
void  or_sample(int32_t *tok, const float *logits, uint32_t B, uint32_t V, uint32_t nb,
                float inv_temp, uint64_t seed, int32_t L);

/* Blind speculative draft and commit over one sequence's token history
 * hist[0..cap) with the pending id at P = L-1 (reference draft_prep and
 * accept_commit, bench/dsv2_decode_bench.c:1116-1170; ids outside [0, V)
 * become holes).  or_spec_accept writes the committed ids and returns the
 * new length (L unchanged when P+S >= cap). */
void    or_spec_draft(int32_t *ca, int32_t *ce, const int32_t *hist, int32_t L, uint32_t S,
                      uint32_t V, uint32_t cap, int forced);
int32_t or_spec_accept(int32_t *hist, int32_t L, const int32_t *ca, const int32_t *am, uint32_t S,
                       uint32_t cap);

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
  /* Per-sublayer teacher forcing (all optional, NULL = off).  Sublayer t =
   * 2l is layer l's attention, 2l+1 its FFN.  tf_x [2L+1][B][D]: the residual
   * entering each sublayer (t = 2L: entering the final norm), taken from
   * another implementation; when set, the step restarts every sublayer from
   * it, so each sublayer's outputs depend only on that sublayer's inputs.
   * Taps (written): tp_x [2L][B][D] the residual leaving each sublayer;
   * tp_q [L][B][H hd] q after bias/RoPE and rounding; tp_att [L][B][H hd]
   * the attention output; tp_h [L][B][F] the FFN hidden (activation dtype
   * values as f32). */
  const float *tf_x;
  float *tp_x, *tp_q, *tp_att, *tp_h;
  uint32_t b0, b1;                       /* rows [b0, b1) only; b1 = 0: every row  */
} OrModel;

/* One decode step for every batch row: token tok[b] at position pos (the
 * cache rows [0,pos) already hold the prefix).  Writes the k/v rows at pos,
 * logits [B][V] f32 and next[b] (greedy).  Returns 0, or -1 on bad config. */
int or_decode_step(const OrModel *m, const int32_t *tok, uint32_t pos,
                   float *logits, int32_t *next);

/* ---- DeepSeek-V2 (MLA + MoE) decode: stages and whole step ----
 * Restates the reference's DSV2 decode step, bench/dsv2_decode_bench.c
 * step_build :2328-2411 with the plain-C custom-kernel twins of each stage
 * (PRE_C dialect, :355-364).  Weights are fp8 e4m3 with per-row f32 scales
 * (the C5 configuration) or bf16 (scale NULL); layouts are this build's:
 *   wqkv [H(dn+dr) + kv + dr][D]   q heads (dn nope rows, dr pe rows), then
 *                                  the latent kv rows and the k pe rows
 *   wuk  [H][kv][dn]  suk [H*kv]   absorbed k up-projection, row (h, k)
 *   wuv  [H][dv][kv]  suv [H*dv]   absorbed v up-projection, row (h, m)
 *   wo   [D][H dv]
 *   dense: wgu [2F][D] rows (gate_i, up_i) interleaved, wd [D][F]
 *   MoE: gate [E][D] f32; wgu_e [E][2I][D] interleaved, sgu_e [E][2I];
 *        wd_e [E][D][I], sd_e [E][D]; shared wgu_s [2S][D], wd_s [D][S]
 *        (S = n_shared * I)
 *   caches: ckv [B][max_seq][kv], kpe [B][max_seq][dr] bf16
 *   rope tables [max_seq][dr/2] f32 (YaRN, :312-343). */

/* q/kv fold for one batch row (gred_q :435-485 + kv_prep :487-556 + mla_qlat
 * :638-667 C twins).  qkv_raw holds the q|kv GEMV output rounded to bf16.
 * q pe pairs (2j, 2j+1) rotate into halves j and dr/2+j; the latent row is
 * RMS-normed (serial sum of squares) with gain wkvn; qlat[h][k] =
 * sum_d qn[h][d] * wuk~[h][k][d] (f32).  Writes qpe [H][dr] bf16, qlat
 * [H][kv] f32, and the cache rows ckv_row [kv], kpe_row [dr] bf16. */
void or_mla_prep(uint16_t *qpe, float *qlat, uint16_t *ckv_row, uint16_t *kpe_row,
                 const uint16_t *qkv_raw, const void *wuk, uint32_t wdt, const float *suk,
                 const float *wkvn, const float *cos_row, const float *sin_row,
                 uint32_t H, uint32_t dn, uint32_t dr, uint32_t kv, float eps);
/* absorbed MLA attention for one batch row over cache rows [0, L) (mla_score
 * :669-723, mla_mix :725-750, mla_o :752-785 C twins): s_j = (qlat.ckv_j +
 * qpe.kpe_j) * scale, p = softmax(s), olat = sum_j p_j ckv_j (f32),
 * o[h][m] = bf16(sum_k olat[h][k] * wuv~[h][m][k]). */
void or_mla_attn(uint16_t *o, const float *qlat, const uint16_t *qpe, const uint16_t *ckv,
                 const uint16_t *kpe, uint32_t L, const void *wuv, uint32_t wdt,
                 const float *suv, uint32_t H, uint32_t kv, uint32_t dr, uint32_t dv,
                 float scale);
/* router (route C twin :836-862): greedy top-K over E logits, ties to the
 * lowest expert id; probs over the softmax of all E logits, no renorm. */
void or_route(int32_t *sel, float *probs, const float *logits, uint32_t E, uint32_t K);
/* routed + shared experts for one batch row (moe_full_h :865-910,
 * moe_full_out :912-965 C twins): h = silu(g)*u in f32 with g, u the
 * unrounded f32 dots; out[d] = sum_e probs[e] (h_e . wd_e~[d]) + h_s .
 * wd_s~[d] (f32, before the residual add). */
void or_moe(float *out, const uint16_t *xb, const int32_t *sel, const float *probs,
            const void *wgu_e, const float *sgu_e, const void *wd_e, const float *sd_e,
            const void *wgu_s, const float *sgu_s, const void *wd_s, const float *sd_s,
            uint32_t wdt, uint32_t D, uint32_t I, uint32_t S, uint32_t K);

typedef struct OrDsv2Layer {
  const float *win, *wkvn, *wpost;       /* norm gains [D], [kv], [D]             */
  const void *wqkv; const float *sqkv;
  const void *wuk;  const float *suk;
  const void *wuv;  const float *suv;
  const void *wo;   const float *so;
  const void *wgu;  const float *sgu;    /* dense layers                          */
  const void *wd;   const float *sd;
  const float *gate;                     /* MoE layers                            */
  const void *wgu_e; const float *sgu_e;
  const void *wd_e;  const float *sd_e;
  const void *wgu_s; const float *sgu_s;
  const void *wd_s;  const float *sd_s;
  uint16_t *ckv, *kpe;
} OrDsv2Layer;

typedef struct OrDsv2 {
  uint32_t n_layers, dim, n_heads, kv_lora, d_nope, d_rope, d_v;
  uint32_t n_experts, n_shared, top_k, moe_inter, dense_inter, first_dense;
  uint32_t vocab, max_seq, batch, wdt;
  float eps, scale;
  const uint16_t *emb;                   /* [V][D] bf16                           */
  const float *gf;                       /* final norm gain                       */
  const void *lm; const float *lm_s;     /* [V][D]                                */
  const float *rope_cos, *rope_sin;      /* [max_seq][dr/2]                       */
  OrDsv2Layer *layers;
  int32_t *sel_out; float *probs_out;    /* optional [n_layers][B][K]: each MoE layer's routing */
  float *gate_out;                       /* optional [n_layers][B][E]: its router logits         */
  /* Per-sublayer teacher forcing and taps, as in OrModel: tf_x [2L+1][B][D]
   * (bf16 values as f32), tp_x [2L][B][D], tp_o [L][B][H dv] the attention
   * output entering the o projection.  tf_sel / tf_probs [L][B][K]: when
   * set, each MoE layer combines these experts with these weights (another
   * implementation's routing) instead of its own top-K; sel_out, probs_out
   * and gate_out still record the oracle's own routing. */
  const float *tf_x;
  float *tp_x, *tp_o;
  const int32_t *tf_sel; const float *tf_probs;
  uint32_t b0, b1;                       /* rows [b0, b1) only; b1 = 0: every row */
} OrDsv2;

/* One DSV2 decode step for every batch row (step_build :2328-2411): writes
 * the cache rows at pos, logits [B][V] f32 and next[b].  The residual stream
 * and the rms1 / dense-FFN / attention outputs are bf16; the post-attention
 * norm feeds the router in f32 and the experts in bf16; the final norm feeds
 * the LM head in f32 (:2394-2397, rms_f out f32). */
int or_dsv2_step(const OrDsv2 *m, const int32_t *tok, uint32_t pos, float *logits, int32_t *next);
/* the dense first layer's activation: h = bf16(silu(g) * u) over bf16 g, u
 * as the reference's bf16 uop chain evaluates it */
void or_dsv2_dense_act(const uint16_t *g, const uint16_t *u, uint16_t *h, uint64_t n);

#ifdef __cplusplus
}
#endif
#endif
