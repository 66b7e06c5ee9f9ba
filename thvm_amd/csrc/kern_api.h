/* kern_api.h -- internal launch interface between the C host layer and the
 * hand-written gfx950 kernels under thvm_amd/csrc/kernels.  C-compatible.
 * Every launcher validates shapes against the buffers' byte sizes it is
 * given, returns 0 on success and -1 (with a message in *err) otherwise, and
 * enqueues on `stream` without synchronising. */
#ifndef THVM_KERN_API_H
#define THVM_KERN_API_H

#include <stdint.h>
#include <hip/hip_runtime_api.h>
#include "thvm_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Kernel-only timing of the next launcher call: `start` is bound to the
 * start of its first kernel and `stop` to the end of its last kernel
 * (hipExtLaunchKernel), so hipEventElapsedTime over the pair covers the
 * kernels alone, without the dispatch latency that event records placed
 * around the launch would add.  The pair is consumed by that call; passing
 * NULLs clears it.  Not for stream capture. */
void thvm_k_time_next(hipEvent_t start, hipEvent_t stop);
hipEvent_t thvm_k_take_start(void);
hipEvent_t thvm_k_take_stop(void);

/* GEMV / small-M GEMM epilogues */
enum {
  THVM_EPI_STORE    = 0,  /* y = rnd(acc*s + b)                                 */
  THVM_EPI_RESID    = 1,  /* y = rnd(res + rnd(acc*s + b))  (y may alias res)   */
  THVM_EPI_SWIGLU   = 2,  /* rows (2i,2i+1)=(gate_i,up_i): y[i]=rnd(silu(g)*u)  */
  THVM_EPI_GELU     = 3,  /* y = rnd(gelu(rnd(acc*s + b)))                       */
  THVM_EPI_QKV_ROPE = 4,  /* q -> y (roped), k (roped) / v -> caches at pos      */
  THVM_EPI_QKV      = 5   /* as QKV_ROPE without the rotation (GPT-2)          */
};

typedef struct ThvmGemvArgs {
  void        *y;
  const void  *x;
  const void  *w;          /* [N, K] row-major, K contiguous                   */
  const float *scale;      /* [N] per-row scale (fp8) or NULL                  */
  const void  *bias;       /* [N] (ydt) or NULL                                */
  const void  *res;        /* residual [M, ldy] (ydt) or NULL                  */
  const float *rope_cos;   /* [max_seq, head_dim/2]                            */
  const float *rope_sin;
  const int32_t *len;      /* device length L; the write position is L-1     */
  void        *kcache;     /* [M][n_kv][max_seq][head_dim] (ydt)               */
  void        *vcache;
  uint32_t M, N, K;
  uint32_t ldx, ldy;       /* row strides in elements                          */
  uint32_t wdt, xdt, ydt;  /* THVM_DT_*                                        */
  uint32_t epi;
  uint32_t n_heads, n_kv_heads, head_dim, max_seq;
  /* fused norm on x: 0 none, 1 RMSNorm, 2 LayerNorm.  The GEMV rounds the
   * normalised row to xdt, as the standalone norm kernel would store it; the
   * MFMA GEMM (RMSNorm over bf16 x only) rounds x*gain and scales the row
   * sums by 1/rms */
  uint32_t norm;
  float    norm_eps;
  const float *norm_w;     /* [K] gain or NULL                                */
  /* norm = 3 (GEMV, one x row, xdt bf16): x is f32 [4][xqs], and the staged
   * row is bf16(norm_w * ((x0 + x1) + (x2 + x3))) -- the four quarter sums of
   * the MLA merge in latent quarters, with the W_uv row scales as the gain */
  uint32_t xqs;
  const float *norm_b;     /* [K] LayerNorm bias or NULL                      */
  /* launch tuning (0 = heuristic): waves per block, rows per wave (MFMA path:
   * 16-row weight tiles per block), chunks per lane in flight, grid blocks,
   * path (1 GEMV, 2 MFMA GEMM; 0 picks the MFMA GEMM for M > 4) */
  uint32_t tune_waves, tune_r, tune_u, tune_blocks, tune_path;
  /* speculative verify (the QKV epilogues): the M rows are consecutive
   * positions of ONE sequence -- row m rotates at and appends to position
   * L-1+m of cache row 0 -- instead of M independent sequences */
  uint32_t spec;
  /* MFMA path only: W is in the MFMA tile layout of thvm_k_tile_w (rows
   * padded to a multiple of 16 with zeros) instead of row-major */
  uint32_t wtiled;
  /* phase clock (measurement only; NULL = off): per block 10 u64 slots (8
   * marks of the 100 MHz wall clock, the XCD, the hardware id), for the
   * first clk_cap blocks */
  uint64_t *clk;
  uint32_t clk_cap;
} ThvmGemvArgs;
/* W [N, K] (row-major, element size es 1 or 2) -> the MFMA tile layout for
 * lanes reading lb bytes of a row per k step (lb 16 or 32, 0 = 16 es; a step
 * is 4 lb bytes of each of 16 rows, and 4 lb must divide a row): for 16-row
 * group g and step s a block of 64 lb bytes at byte (g * S + s) * 64 lb
 * (S = steps per row), holding lb / 16 pieces jj of 64 lanes x 16 bytes:
 * lane l's bytes are row 16 g + l % 16, bytes s*4lb + (l/16)*lb + jj*16 of
 * the row -- what a kernel's lane l loads for that step, so each load
 * instruction of a wave reads 1 KB contiguous.  Rows N..Npad-1 (Npad = N
 * rounded up to 16) are zero; y holds Npad*K*es bytes.  lb = 16 es is the
 * MFMA GEMM's layout (64 k per step), lb 32 / 16 the grouped MoE's gate/up
 * and down. */
int thvm_k_tile_w(void *y, const void *w, uint32_t N, uint32_t K, uint32_t es, uint32_t lb, hipStream_t s,
                  char *err, int errlen);
/* y = epi(x . W^T): the GEMV for M <= 4, the MFMA GEMM for M <= 64 (fp16 W
 * with fp16 x, bf16 W with bf16 x, fp8 W with bf16/fp16 x; K % 64 == 0; no
 * fused norm). */
int thvm_k_gemv(const ThvmGemvArgs *a, hipStream_t s, char *err, int errlen);
int thvm_k_gemm_mfma(const ThvmGemvArgs *a, hipStream_t s, char *err, int errlen);

/* Row norms over [M, K]: RMSNorm (y = rnd((x*inv)*w), inv=1/sqrt(ss/K+eps))
 * or LayerNorm (y = rnd((x-mu)*rsqrt(var+eps)*w + b)).  x may be f32/bf16/f16,
 * y f32/bf16/f16.  `ldx`/`ldy` are row strides.  For RMSNorm `w` may be NULL
 * (gain 1). */
typedef struct ThvmNormArgs {
  void *y; const void *x; const float *w; const float *b;
  uint32_t M, K, ldx, ldy, xdt, ydt;
  float eps;
  int layernorm;
} ThvmNormArgs;
int thvm_k_norm(const ThvmNormArgs *a, hipStream_t s, char *err, int errlen);

/* Row softmax over [M, K] (x f32/bf16/f16 -> y same family). */
typedef struct ThvmSoftmaxArgs {
  void *y; const void *x; uint32_t M, K, xdt, ydt;
} ThvmSoftmaxArgs;
int thvm_k_softmax(const ThvmSoftmaxArgs *a, hipStream_t s, char *err, int errlen);

/* Split-sequence flash-decode attention over a KV cache.
 * q [B][H][hd] (qdt), caches [B][Hkv][max_seq][hd] (cdt), live length L (device
 * scalar, same for all rows).  Phase 1 writes per-split (m, l, acc[hd]); phase
 * 2 combines into out [B][H*hd] (odt). */
typedef struct ThvmAttnArgs {
  void *out; const void *q; const void *kcache; const void *vcache;
  const int32_t *len;
  float *part;             /* scratch: [B][H][n_split][hd + 2] f32, then B*Hkv
                            * merge counters that must be zero before the first
                            * launch (a zero-filled buffer); every launch leaves
                            * them zero                                       */
  uint32_t B, H, Hkv, hd, max_seq, chunk, n_split;
  uint32_t qdt, cdt, odt;
  float scale;             /* 1/sqrt(hd)                                     */
  uint32_t fused;          /* 1: split and merge in one launch (the last
                            * split block of a (row, kv head) merges); 0: two
                            * launches; 2: picked from the shape            */
  uint32_t cpb;            /* chunks per split block: 0 picks from the unit
                            * count, 1 one chunk per block, above 1 a block
                            * runs that many consecutive chunks (G <= 4);
                            * the partials are per block                    */
  uint32_t spec;           /* speculative verify: the B query rows are
                            * consecutive positions of one sequence; row b
                            * reads cache row 0 over L+b rows (causal)     */
  uint64_t *clk;           /* phase clock (measurement only; NULL = off)   */
  uint32_t clk_cap;        /* blocks recorded per launch (split, then merge) */
  uint32_t mf;             /* the split on MFMA (16-bit caches, hd 64 / 128,
                            * G <= 8, two launches): 0 picked from the shape
                            * (batched decode), 1 on, 2 off                 */
} ThvmAttnArgs;
int thvm_k_attn_decode(const ThvmAttnArgs *a, hipStream_t s, char *err, int errlen);
/* the chunks per split block thvm_k_attn_decode picks for cpb = 0 */
uint32_t thvm_k_attn_auto_cpb(uint32_t B, uint32_t H, uint32_t Hkv, uint32_t n_split, uint32_t fused);
/* the split thvm_k_attn_decode runs for these arguments: *mf 1 the MFMA
 * split, 0 the VALU forms; *cpb its chunks per split block */
void thvm_k_attn_plan(const ThvmAttnArgs *a, uint32_t *mf, uint32_t *cpb);
uint64_t thvm_k_attn_part_bytes(uint32_t B, uint32_t H, uint32_t Hkv, uint32_t hd, uint32_t n_split);
/* The same attention with a->part ignored: partials and merge counters in a
 * static device array of THVM_ATTN_SCRATCH_BYTES per GPU (no allocation).
 * thvm_k_attn_scratch_setup takes the array's address on the current device
 * (once per device, at init); a call needing more partials than the array
 * holds fails with an error.  Calls that overlap on one GPU race. */
#define THVM_ATTN_SCRATCH_BYTES (16u << 20)
int thvm_k_attn_scratch_setup(char *err, int errlen);
int thvm_k_attn_decode_scratch(const ThvmAttnArgs *a, hipStream_t s, char *err, int errlen);

/* DeepSeek-V2 multi-head latent attention (absorbed form) for decode.
 * qkv [B][ldq] bf16 is the q|kv projection output: per head dn nope + dr pe
 * values, then kv latent values and dr k-pe values.  Caches ckv
 * [B][max_seq][kv], kpe [B][max_seq][dr] bf16; rope tables [max_seq][dr/2].
 * mla_prep: qpe [B][H][dr] bf16 (pairs (2j,2j+1) rotated into halves j and
 * dr/2+j), the latent row RMS-normed with gain wkvn and the rotated k pe row
 * appended at L-1, and qlat [B][H][kv] f32 = q_nope . W_uk (W_uk [H][kv][dn]).
 * mla_attn: split-sequence scores over rows [0, L) (s = (qlat.ckv + qpe.kpe)
 * * scale), partials part [B][n_split][H][kv+4] (m, l at kv, kv+1), then the merge and the V
 * up-projection o [B][H*dv] bf16 = olat . W_uv (W_uv [H][dv][kv]).  W_uk /
 * W_uv are fp8 e4m3 with per-row scales (suk [H*kv], suv [H*dv]) or bf16. */
typedef struct ThvmMlaArgs {
  const void *qkv;
  const void *wuk; const float *suk;
  const void *wuv; const float *suv;
  const float *wkvn;
  const float *rope_cos, *rope_sin;
  const int32_t *len;
  void *ckv, *kpe;
  float *qlat;
  void *qpe;
  float *part;
  void *o;
  uint32_t B, H, dn, dr, kv, dv, max_seq, ldq, n_split, wdt;
  float eps, scale;
  /* mla_attn: split kernel (0 auto: the MFMA split for 16 heads x kv 512 x
   * rope 64, the VALU split otherwise; 1 VALU; 2 MFMA) and 64-row chunks per
   * split block (0 auto; the MFMA split takes 1, 2 or 4) */
  uint32_t mode, cpb;
  /* mla_attn: 1 = the merge in latent quarters (k_mla_out_q): o is then f32
   * [4][B][H*dv], the four unscaled quarter sums that a GEMV with norm = 3
   * adds, scales and rounds while staging x; 0 = o is bf16 [B][H*dv] */
  uint32_t oq;
  /* phase clock (measurement build only; NULL = off): mla_attn records the
   * split's blocks, then the merge's, clk_cap blocks each */
  uint64_t *clk;
  uint32_t clk_cap;
} ThvmMlaArgs;
int thvm_k_mla_prep(const ThvmMlaArgs *a, hipStream_t s, char *err, int errlen);
int thvm_k_mla_attn(const ThvmMlaArgs *a, hipStream_t s, char *err, int errlen);
uint64_t thvm_k_mla_part_bytes(uint32_t B, uint32_t H, uint32_t kv, uint32_t n_split);

/* MoE routing (reference bench/dsv2_decode_bench.c route :787-863): per
 * batch row, greedy top-K of E gate logits (ties to the lowest expert id),
 * probs = softmax over all E logits at the chosen ids, no renormalisation.
 * logits [B][E] f32 -> sel [B][K] int32, probs [B][K] f32.  E <= 64. */
typedef struct ThvmRouteArgs {
  int32_t *sel; float *probs; const float *logits;
  uint32_t B, E, K;
} ThvmRouteArgs;
int thvm_k_route(const ThvmRouteArgs *a, hipStream_t s, char *err, int errlen);
/* The post-attention RMSNorm and the router GEMV of a MoE layer in one
 * launch, bit for bit the norm (f32 out) and f32 GEMV kernels in sequence:
 * x [B][D] bf16, w [D] f32 gain, gate [E][D] f32 (16-byte aligned) -> xn
 * [B][D] f32 (the experts' input), logits [B][E] f32.  D <= 4096, a
 * multiple of 4; E <= 64.  Blocks of 8 experts each renormalise the row. */
typedef struct ThvmGateArgs {
  const void *x; const float *w; const float *gate;
  float *xn; float *logits;
  uint32_t B, D, E;
  float eps;
  uint64_t *clk;           /* phase clock (measurement only; NULL = off) */
  uint32_t clk_cap;
} ThvmGateArgs;
int thvm_k_moe_gate(const ThvmGateArgs *a, hipStream_t s, char *err, int errlen);

/* Routed + shared expert FFN (reference moe_full_h / moe_full_out
 * :865-965).  x [B][D] f32 (rounded to bf16 as the experts' input); h
 * [B][K*I + S] f32 scratch; gate/up rows interleaved (gate_i, up_i):
 * wgu_e [E][2I][D] (+ sgu_e [E][2I]), wgu_s [2S][D] (+ sgu_s [2S]); down
 * rows wd_e [E][D][I] (+ sd_e [E][D]), wd_s [D][S] (+ sd_s [D]); weights
 * fp8 e4m3 (scales required) or bf16 (scales NULL).
 * gateup: h[b][e*I+i] = silu(g)*u (f32) for slot e < K and h[b][K*I+i] for
 * the shared rows.  down: res[b][d] = bf16(res + bf16(sum_e probs[b][e] *
 * (h_e . wd_e[sel][d]) + h_s . wd_s[d])). */
typedef struct ThvmMoeArgs {
  const float *x; float *h; void *res;
  const int32_t *sel; const float *probs;
  const void *wgu_e; const float *sgu_e;
  const void *wd_e;  const float *sd_e;
  const void *wgu_s; const float *sgu_s;
  const void *wd_s;  const float *sd_s;
  uint32_t B, D, E, K, I, S, wdt;
  /* expert-grouped form (grouped = 1; any B, meant for B > 4): every live
   * expert's weights are streamed once for all the rows routed to it.
   * plan [E + E*B*K] int32 scratch: rows per expert, then each expert's
   * (b*K + slot) list in ascending order; part [B*K*D + B*D] f32 scratch: the
   * per-slot down outputs, then the shared ones, summed by a combine kernel
   * in the per-row kernels' order (outputs are identical to theirs). */
  uint32_t grouped;
  int32_t *plan;
  float *part;
  int32_t *live;           /* grouped gate/up: += experts with rows (optional) */
  /* per-row gate/up with logits set: every block picks the row's top-K from
   * logits [B][E] itself (the route kernel's arithmetic, so the same ids and
   * probabilities) instead of reading sel; blocks x = 0 write them to
   * sel_out / probs_out for the down kernel */
  const float *logits;
  int32_t *sel_out; float *probs_out;
  /* grouped = 2 only: the expert weights (routed and shared) are in the
   * tile layout of thvm_k_tile_w, 32 bytes per lane for gate/up and 16 for
   * down (each expert's rows a whole number of 16-row groups) */
  uint32_t wtiled;
  uint64_t *clk;           /* phase clock (measurement only; NULL = off) */
  uint32_t clk_cap;
} ThvmMoeArgs;
/* plan / part scratch sizes in bytes for the grouped form */
uint64_t thvm_k_moe_plan_bytes(uint32_t B, uint32_t E, uint32_t K);
uint64_t thvm_k_moe_part_bytes(uint32_t B, uint32_t K, uint32_t D);
int thvm_k_moe_gateup(const ThvmMoeArgs *a, hipStream_t s, char *err, int errlen);
int thvm_k_moe_down(const ThvmMoeArgs *a, hipStream_t s, char *err, int errlen);

/* Embedding gather: x[b][i] = emb[tok[b]][i] (+ pos[L-1][i] when pos != NULL),
 * tok int32 [B]; out of range ids read a zero row. */
typedef struct ThvmEmbedArgs {
  void *x; const void *emb; const void *pos_emb; const int32_t *tok;
  const int32_t *len;
  uint32_t B, D, V, max_seq, edt, xdt;
} ThvmEmbedArgs;
int thvm_k_embed(const ThvmEmbedArgs *a, hipStream_t s, char *err, int errlen);

/* Greedy argmax over logits [B][V] f32, lowest index on ties (reference
 * bench/dsv2_decode_bench.c:967-1022).  Writes tok[b]; when `hist` is set
 * also hist[b*hist_stride + L-1]. */
typedef struct ThvmArgmaxArgs {
  int32_t *tok; const float *logits; float *pv; int32_t *pi;
  int32_t *hist; const int32_t *len;
  uint32_t B, V, nb, hist_stride;
  float inv_temp;          /* > 0: sample from softmax(logits * inv_temp)
                            * instead of the argmax (pi then holds f32 block
                            * sums); the draw is keyed on (seed, row, len[0]) */
  uint64_t seed;
} ThvmArgmaxArgs;
int thvm_k_argmax(const ThvmArgmaxArgs *a, hipStream_t s, char *err, int errlen);

/* One wave sleeping n fixed periods (~3.4 us each): lets a host enqueue work
 * behind it so back-to-back kernels can be timed without host gaps. */
int thvm_k_delay(uint32_t n, hipStream_t s, char *err, int errlen);

/* Blind speculative decode (reference draft_prep / accept_commit,
 * bench/dsv2_decode_bench.c:1110-1170).  The token history hist[0..hist_cap)
 * of one sequence holds the committed ids and, at P = L-1, the pending one.
 * draft: cand_acc[0] = cand_emb[0] = hist[P]; with j the largest index with
 * j+1 < P where (hist[j], hist[j+1]) == (hist[P-1], hist[P]), cand_acc[1+t] =
 * hist[j+2+t] while j+2+t <= P, else -1 (a hole); forced = 1 takes
 * cand_acc[1+t] = hist[P+1+t] (ids seeded there by the host) instead.  Ids
 * outside [0, V) are holes; cand_emb = cand_acc with holes replaced by hist[P].
 * accept: k = the longest prefix with cand_acc[i+1] == am[i] (i < S-1);
 * hist[P+1..P+k] = cand_acc[1..k], hist[P+1+k] = am[k], tok[0] = am[k] (when
 * tok is given), L = P+k+2.  A state with P+S >= hist_cap is left unchanged. */
int thvm_k_spec_draft(int32_t *cand_acc, int32_t *cand_emb, const int32_t *hist, const int32_t *len,
                      uint32_t S, uint32_t V, uint32_t hist_cap, uint32_t forced, hipStream_t s,
                      char *err, int errlen);
int thvm_k_spec_accept(int32_t *hist, int32_t *len, int32_t *tok, const int32_t *cand_acc,
                       const int32_t *am, uint32_t S, uint32_t hist_cap, hipStream_t s, char *err,
                       int errlen);

/* L[0] += delta (reference len_bump, bench/dsv2_decode_bench.c:1024-1041). */
int thvm_k_len_bump(int32_t *len, int32_t delta, hipStream_t s, char *err, int errlen);

/* Synthetic data: counter-based N(mean, std) fill of n elements of dtype dt,
 * stream id `tag` under `seed`; and per-row fp8 e4m3 quantisation of a
 * rows x cols N(0,std) matrix: scale[r] = absmax/448, q = sat_e4m3(w/scale). */
int thvm_k_fill_normal(void *dst, uint32_t dt, uint64_t n, uint64_t seed,
                       uint64_t tag, float mean, float std, hipStream_t s,
                       char *err, int errlen);
int thvm_k_fill_fp8_rows(uint8_t *q, float *scale, uint32_t rows, uint32_t cols,
                         uint64_t seed, uint64_t tag, float std, hipStream_t s,
                         char *err, int errlen);
/* Fill rows [0, ctx) of a [B][Hkv][max_seq][hd] cache with N(0,1). */
int thvm_k_fill_cache(void *cache, uint32_t dt, uint32_t B, uint32_t Hkv,
                      uint32_t max_seq, uint32_t hd, uint32_t ctx,
                      uint64_t seed, uint64_t tag, hipStream_t s,
                      char *err, int errlen);

/* Per-row fp8 e4m3 quantisation of a loaded matrix x [rows][cols] (f32 /
 * bf16 / fp16): scale[r] = absmax/448 (1 for a zero row), q = e4m3_sat(x/scale). */
int thvm_k_quant_fp8_rows(uint8_t *q, float *scale, const void *x, uint32_t xdt, uint32_t rows,
                          uint32_t cols, hipStream_t s, char *err, int errlen);

/* Plain device copy of nbytes (16-byte aligned pointers and size), each
 * byte read once and written once: the calibration of HBM traffic counters. */
int thvm_k_copy(void *y, const void *x, uint64_t nbytes, hipStream_t s, char *err, int errlen);

/* Read nbytes at x (16-byte aligned and sized) with streaming loads, one
 * word per block into sink[nsink] (grid at most nsink blocks): evicts the
 * caches with clean lines, for timing a kernel on cold caches. */
int thvm_k_touch(const void *x, uint64_t nbytes, uint32_t *sink, uint32_t nsink, hipStream_t s,
                 char *err, int errlen);
/* Zero nbytes at y (any alignment) with a kernel, so the fill can sit in a
 * captured graph as a kernel node. */
int thvm_k_zero(void *y, uint64_t nbytes, hipStream_t s, char *err, int errlen);
/* Copy n bytes from x to y + off, off = base + stride * idx[0] with idx[0]
 * read on the device (idx NULL: off = base); an off whose n bytes do not fit
 * in cap bytes writes nothing.  Any alignment; a kernel node when captured. */
int thvm_k_copy_at(void *y, uint64_t cap, uint64_t base, uint64_t stride, const int32_t *idx,
                   const void *x, uint64_t n, hipStream_t s, char *err, int errlen);

/* Element-wise casts / copies (codec probes and glue): y[i] = cvt(x[i]). */
int thvm_k_cast(void *y, uint32_t ydt, const void *x, uint32_t xdt, uint64_t n,
                hipStream_t s, char *err, int errlen);

/* RoPE in place on [B][nh][hd] (interleaved pairs) at position L-1. */
typedef struct ThvmRopeArgs {
  void *x; const float *cos_t; const float *sin_t; const int32_t *len;
  uint32_t B, nh, hd, dt, max_seq;   /* tables hold max_seq positions */
} ThvmRopeArgs;
int thvm_k_rope(const ThvmRopeArgs *a, hipStream_t s, char *err, int errlen);

/* Persistent decode step of the LLAMA architecture: the whole step (embed,
 * per layer RMSNorm + q|k|v + RoPE + KV append, attention, o + residual,
 * RMSNorm + gate/up + SwiGLU, down + residual; final RMSNorm, LM head,
 * argmax, history, L += 1) in one launch of one block per CU, the stages
 * separated by grid barriers.  Every output equals the multi-kernel step's
 * bit for bit (same device functions, same orders).  Per-layer weights come
 * from a device-resident table. */
typedef struct ThvmStepLayer {
  const void *wqkv; const float *sqkv;   /* [(H+2Hkv)hd, D] (+ row scales)  */
  const void *wo;   const float *so;     /* [D, H hd]                       */
  const void *wgu;  const float *sgu;    /* [2F, D], gate/up rows interleaved */
  const void *wd;   const float *sd;     /* [D, F]                          */
  const float *g_attn, *g_ffn;           /* [D] RMSNorm gains               */
  void *kcache, *vcache;                 /* [M][Hkv][max_seq][hd]           */
} ThvmStepLayer;

typedef struct ThvmStepArgs {
  const ThvmStepLayer *layers;           /* device array [n_layers]        */
  const void *emb;                       /* [V, D] (adt)                   */
  const float *norm_f;                   /* [D]                            */
  const void *lm; const float *slm;      /* [V, D] (+ row scales)          */
  const float *rope_cos, *rope_sin;      /* [max_seq][hd/2]                */
  int32_t *tok, *len, *hist;             /* [M], [1], [M][hist_stride]     */
  float *logits;                         /* [M][V]                         */
  void *x, *q, *att, *h;                 /* [M][D], [M][H hd] x2, [M][F]   */
  float *part;                           /* attention partials             */
  float *am_pv; int32_t *am_pi;          /* [M][thvm_k_step_blocks()]      */
  uint32_t *sync;                        /* thvm_k_step_sync_bytes(), zeroed once */
  uint32_t n_layers, M, D, H, Hkv, hd, F, V, max_seq, n_split, hist_stride;
  uint32_t wdt, adt;
  float eps, attn_scale;
} ThvmStepArgs;
int thvm_k_llama_step(const ThvmStepArgs *a, hipStream_t s, char *err, int errlen);
/* grid of the persistent step (one block per CU) and its sync area bytes */
uint32_t thvm_k_step_blocks(void);
uint32_t thvm_k_step_sync_bytes(void);
/* index of the sync area's error word (nonzero: a grid barrier expired) */
uint32_t thvm_k_step_err_word(void);
/* index of the stage clock: 64-bit wall-clock ticks (100 MHz) that block 0
 * of the last launch recorded at its start (slot 0), at the opening of each
 * grid barrier k (slot k + 1) and at the end of the tail (slot barriers + 1) */
uint32_t thvm_k_step_clock_word(void);
/* index of the detail clock: 4 events per stage (entry, barrier open, work
 * done, stores drained) of block 0, stage id l*5 + {0 QKV, 1 ATTN, 2 O, 3 GU,
 * 4 DOWN}, then the LM stage */
uint32_t thvm_k_step_dclock_word(void);
/* check a step configuration without launching (0 / -1 with *err) */
int thvm_k_llama_step_check(const ThvmStepArgs *a, char *err, int errlen);

#ifdef __cplusplus
}
#endif
#endif
