// step.hip -- launcher of the persistent LLAMA decode step (step_core.h):
// configuration checks, instance choice, LDS size and the one-block-per-CU
// grid.  The kernel instances live in step_m{1,2,4}.hip.
#include "step_core.h"
#include "launch.h"
#include <stdio.h>

extern "C" void *thvm_step_pick_m1(uint32_t wdt, uint32_t adt, uint32_t hd, uint32_t G);
extern "C" void *thvm_step_pick_m2(uint32_t wdt, uint32_t adt, uint32_t hd, uint32_t G);
extern "C" void *thvm_step_pick_m4(uint32_t wdt, uint32_t adt, uint32_t hd, uint32_t G);

static step_fn pick(const ThvmStepArgs *a) {
  const uint32_t G = a->Hkv ? a->H / a->Hkv : 0;
  switch (a->M) {
    case 1: return (step_fn)thvm_step_pick_m1(a->wdt, a->adt, a->hd, G);
    case 2: return (step_fn)thvm_step_pick_m2(a->wdt, a->adt, a->hd, G);
    case 4: return (step_fn)thvm_step_pick_m4(a->wdt, a->adt, a->hd, G);
    default: return nullptr;
  }
}

static uint64_t step_lds(const ThvmStepArgs *a) {
  const uint64_t kmax = a->F > a->D ? (a->F > a->H * a->hd ? a->F : a->H * a->hd)
                                    : (a->D > a->H * a->hd ? a->D : a->H * a->hd);
  const uint64_t gemv = (uint64_t)a->M * kmax * 2;
  const uint32_t G = a->Hkv ? a->H / a->Hkv : 1;
  const uint64_t attn = 2 * ((uint64_t)3 * ATT_WAVES * G * 4 + (uint64_t)ATT_WAVES * G * a->hd * 4 + 16) +
                        2 * (uint64_t)MERGE_LDS_BYTES + 64;
  return gemv > attn ? gemv : attn;
}

static uint32_t n_cus(void) {
  static uint32_t n = 0;
  if (!n) {
    int dev = 0, c = 0;
    if (hipGetDevice(&dev) == hipSuccess &&
        hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && c > 0)
      n = (uint32_t)c;
  }
  return n;
}

extern "C" uint32_t thvm_k_step_blocks(void) { return n_cus(); }
extern "C" uint32_t thvm_k_step_sync_bytes(void) { return SYNC_BYTES; }
extern "C" uint32_t thvm_k_step_err_word(void) { return SYNC_W_ERR; }
extern "C" uint32_t thvm_k_step_clock_word(void) { return SYNC_W_CLOCK; }
extern "C" uint32_t thvm_k_step_dclock_word(void) { return SYNC_W_DCLOCK; }

extern "C" int thvm_k_llama_step_check(const ThvmStepArgs *a, char *err, int errlen) {
  if (a->M < 1 || a->M > STEP_MAX_M || a->M == 3) {
    snprintf(err, errlen, "step: batch %u (the persistent step takes 1, 2 or 4 rows)", a->M);
    return -1;
  }
  if (a->n_layers == 0 || a->D == 0 || a->H == 0 || a->Hkv == 0 || a->H % a->Hkv || a->F == 0 ||
      a->V == 0 || a->max_seq == 0) {
    snprintf(err, errlen, "step: zero or inconsistent dimension");
    return -1;
  }
  if (a->hd != 64 && a->hd != 128) { snprintf(err, errlen, "step: head_dim must be 64 or 128"); return -1; }
  const uint32_t G = a->H / a->Hkv;
  if (G != 1 && G != 2 && G != 4) { snprintf(err, errlen, "step: %u query heads per kv head (1, 2 or 4)", G); return -1; }
  if (!pick(a)) {
    snprintf(err, errlen, "step: weight/activation dtypes %u/%u (fp8/bf16 or bf16/bf16)", a->wdt, a->adt);
    return -1;
  }
  if (a->D % 512 || a->F % 512 || (a->H * a->hd) % 512) {
    snprintf(err, errlen, "step: dim, ffn and heads*head_dim must be multiples of 512");
    return -1;
  }
  // fused-norm staging of an 8-wave block holds <= 16 x elements per thread
  if (a->D > 16u * STAGE_THREADS) { snprintf(err, errlen, "step: dim > %u", 16u * STAGE_THREADS); return -1; }
  if (a->n_split * ATT_CHUNK < a->max_seq || a->n_split > ATT_MAX_SPLITS) {
    snprintf(err, errlen, "step: n_split*64 >= max_seq and n_split <= %d", ATT_MAX_SPLITS);
    return -1;
  }
  if (a->M * a->Hkv > SYNC_MAX_MERGE) { snprintf(err, errlen, "step: batch*kv_heads > %d", SYNC_MAX_MERGE); return -1; }
  // system-scope accesses take 32-bit byte offsets
  const uint64_t es = 2;
  const uint64_t cache = (uint64_t)a->M * a->Hkv * a->max_seq * a->hd * es;
  const uint64_t logits = (uint64_t)a->M * a->V * 4;
  const uint64_t part = (uint64_t)a->M * a->H * a->n_split * (a->hd + 2) * 4;
  if (cache >= (1ull << 31) || logits >= (1ull << 31) || part >= (1ull << 31)) {
    snprintf(err, errlen, "step: a cache, logits or partial buffer of 2 GiB or more");
    return -1;
  }
  if (step_lds(a) > 160 * 1024) { snprintf(err, errlen, "step: LDS need above 160 KiB"); return -1; }
  if (!a->layers || !a->emb || !a->norm_f || !a->lm || !a->rope_cos || !a->rope_sin || !a->tok ||
      !a->len || !a->logits || !a->x || !a->q || !a->att || !a->h || !a->part || !a->am_pv ||
      !a->am_pi || !a->sync || (a->wdt == THVM_DT_FP8E4M3 && !a->slm)) {
    snprintf(err, errlen, "step: missing buffer");
    return -1;
  }
  if (n_cus() == 0) { snprintf(err, errlen, "step: no device"); return -1; }
  return 0;
}

extern "C" int thvm_k_llama_step(const ThvmStepArgs *a, hipStream_t s, char *err, int errlen) {
  if (thvm_k_llama_step_check(a, err, errlen)) return -1;
  step_fn f = pick(a);
  const uint32_t lds = (uint32_t)step_lds(a);
  // dynamic LDS above 64 KiB needs the attribute (static LDS counts against
  // the same 160 KiB); checked once per (instance, size)
  static struct { step_fn f; uint32_t lds; } done[64];
  static int n_done = 0;
  bool have = false;
  for (int i = 0; i < n_done; i++) have |= done[i].f == f && done[i].lds == lds;
  if (!have) {
    hipError_t e = hipSuccess;
    if (lds > 64 * 1024) e = hipFuncSetAttribute((const void *)f, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) { snprintf(err, errlen, "step: hipFuncSetAttribute(%u): %s", lds, hipGetErrorString(e)); return -1; }
    int nb = 0;
    e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, (const void *)f, STEP_THREADS, lds);
    if (e != hipSuccess || nb < 1) {
      snprintf(err, errlen, "step: one %d-thread block per CU does not fit (occupancy %d)", STEP_THREADS, nb);
      return -1;
    }
    if (n_done < 64) { done[n_done].f = f; done[n_done].lds = lds; n_done++; }
  }
  thvm_launch(true, true, f, dim3(n_cus()), dim3(STEP_THREADS), lds, s, *a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) { snprintf(err, errlen, "step launch: %s", hipGetErrorString(e)); return -1; }
  return 0;
}
