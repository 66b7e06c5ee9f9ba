/* oracle.c -- TEST INFRASTRUCTURE ONLY (see oracle.h).  A CPU restatement of
 * the reference thvm CPU path for the decode hot path.  Nothing in the
 * product library links or loads this file; it is the checker.
 *
 * Build: oracle/Makefile (gcc -O3 -fno-math-errno -ffp-contract=off, the
 * reference CPU JIT flags of src/backend/cpu/jit.c:318-345 minus -march). */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

enum { DT_FP8E4M3 = 9, DT_FP8E5M2 = 10, DT_FP16 = 11, DT_BF16 = 12, DT_FP32 = 13 };

static uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* ==== bf16: reference src/dtype/fp_convert.c:113-136 ==================== */
float or_bf16_to_f32(uint16_t b) { return u2f((uint32_t)b << 16); }

uint16_t or_f32_to_bf16(float v) {
  uint32_t bits = f2u(v);
  if (((bits >> 23) & 0xFFu) == 0xFFu && (bits & 0x7FFFFFu) != 0u)
    return (uint16_t)(((bits & 0x80000000u) | 0x7F800000u | 0x400000u) >> 16);
  return (uint16_t)(((bits + 0x7FFFu + ((bits >> 16) & 1u)) & 0xFFFF0000u) >> 16);
}

/* ==== fp16: reference src/dtype/fp_convert.c:26-110 (manual forms) ====== */
float or_fp16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h >> 15) & 1u, exp = (uint32_t)(h >> 10) & 0x1Fu, mant = h & 0x3FFu;
  uint32_t out;
  if (exp == 0) {
    if (mant == 0) {
      out = sign << 31;
    } else {
      uint32_t sh = 0;
      while ((mant & 0x400u) == 0) { mant <<= 1; sh++; }
      mant &= 0x3FFu;
      out = (sign << 31) | ((127u - 14u - sh) << 23) | (mant << 13);
    }
  } else if (exp == 0x1F) {
    out = (sign << 31) | (0xFFu << 23) | (mant ? 0x400000u : 0u) | (mant << 13);
  } else {
    out = (sign << 31) | ((exp - 15u + 127u) << 23) | (mant << 13);
  }
  return u2f(out);
}

uint16_t or_f32_to_fp16(float v) {
  uint32_t b = f2u(v);
  uint32_t sign = (b >> 16) & 0x8000u, exp = (b >> 23) & 0xFFu, mant = b & 0x7FFFFFu;
  if (exp == 0xFF) return (uint16_t)(sign | 0x7C00u | (mant ? (0x200u | (mant >> 13)) : 0u));
  if (exp >= 127 + 16) return (uint16_t)(sign | 0x7C00u);
  if (exp >= 127 - 14) {
    uint32_t h = ((exp - 127 + 15) << 10) | (mant >> 13), r = mant & 0x1FFFu;
    if (r > 0x1000u || (r == 0x1000u && (h & 1u))) h++;
    return (uint16_t)(sign | h);
  }
  if (exp < 127 - 25) return (uint16_t)sign;
  uint32_t m = mant | 0x800000u, sh = 126 - exp;
  uint32_t h = m >> sh, rem = m & ((1u << sh) - 1u), half = 1u << (sh - 1u);
  if (rem > half || (rem == half && (h & 1u))) h++;
  return (uint16_t)(sign | h);
}

/* ==== fp8 e4m3 / e5m2 ======================================================
 * Written from the OCP 8-bit floating point specification (OFP8, v1.0):
 *   e4m3: bias 7, 3 mantissa bits, no infinities, S.1111.111 is NaN,
 *         largest finite 0x7E = 448;
 *   e5m2: bias 15, 2 mantissa bits, IEEE-style inf (S.11111.00) and NaN,
 *         largest finite 0x7B = 57344.
 * A finite value rounds to nearest, ties to even, on the f32 significand;
 * subnormals are kept; a finite value whose rounded magnitude exceeds the
 * largest finite one stores the largest finite one (both forms).  The
 * non-finite conventions are the reference's (src/dtype/fp8.c, its store
 * path and tests/test_fp8_nonfinite.c:110-192): the plain form stores
 * +-inf and NaN as S.1111.111 (e4m3) and +-inf as S.11111.00, NaN as
 * S.11111.11 (e5m2); the _sat form stores +-inf as +-max finite and a NaN
 * as the format's all-ones exponent over the top mantissa bits of the f32
 * NaN (e4m3: always S.1111.111). */
typedef struct {
  int mbits, bias;
  uint32_t max_code, inf_code, nan_code;
} Ofp8;
static const Ofp8 OFP8_E4M3 = {3, 7, 0x7E, 0x7F, 0x7F};
static const Ofp8 OFP8_E5M2 = {2, 15, 0x7B, 0x7C, 0x7F};

static uint8_t ofp8_encode(float x, const Ofp8 *f, int sat) {
  const uint32_t u = f2u(x), sign = (u >> 24) & 0x80u, a = u & 0x7FFFFFFFu;
  if (a > 0x7F800000u) { /* NaN */
    if (!sat || f->mbits == 3) return (uint8_t)(sign | f->nan_code);
    return (uint8_t)(sign | f->inf_code | ((a >> (23 - f->mbits)) & ((1u << f->mbits) - 1u)));
  }
  if (a == 0x7F800000u) return (uint8_t)(sign | (sat ? f->max_code : f->inf_code));
  /* |x| = sig * 2^(ef - 150) with sig < 2^24 */
  int ef = (int)(a >> 23);
  uint32_t sig = a & 0x7FFFFFu;
  if (ef) sig |= 0x800000u; else ef = 1;
  const int emin = 1 - f->bias;              /* exponent of the smallest normal */
  int e = ef - 127;                          /* exponent of the leading bit (normal f32) */
  if (e < emin) e = emin;                    /* below emin the quantum stays 2^(emin-mbits) */
  const int sh = (e - f->mbits) - (ef - 150); /* sig / 2^sh = |x| / quantum, sh >= 20 */
  uint32_t n = 0;
  if (sh <= 24) {
    const uint32_t rem = sig & ((1u << sh) - 1u), half = 1u << (sh - 1);
    n = sig >> sh;
    if (rem > half || (rem == half && (n & 1u))) n++;
  } /* sh > 24: |x| is below half a quantum, rounds to zero */
  /* n counts quanta 2^(e - mbits); the code is ((e + bias - 1) << mbits) + n,
   * which also covers the subnormals (e = emin) and a carry into the next
   * binade (n = 2^(mbits+1)). */
  uint32_t code = ((uint32_t)(e + f->bias - 1) << f->mbits) + n;
  if (code > f->max_code) code = f->max_code;
  return (uint8_t)(sign | code);
}

uint8_t or_f32_to_fp8e4m3(float v) { return ofp8_encode(v, &OFP8_E4M3, 0); }
uint8_t or_f32_to_fp8e4m3_sat(float v) { return ofp8_encode(v, &OFP8_E4M3, 1); }
uint8_t or_f32_to_fp8e5m2(float v) { return ofp8_encode(v, &OFP8_E5M2, 0); }
uint8_t or_f32_to_fp8e5m2_sat(float v) { return ofp8_encode(v, &OFP8_E5M2, 1); }

/* (-1)^s * 2^(E - bias) * (1 + M / 2^mbits), or 2^(1 - bias) * M / 2^mbits
 * for E = 0 (OFP8 v1.0 value formulas). */
static float ofp8_decode(uint8_t b, const Ofp8 *f) {
  const int ebits = 7 - f->mbits;
  const uint32_t mag = b & 0x7Fu, E = mag >> f->mbits, M = mag & ((1u << f->mbits) - 1u);
  float v;
  if (f->mbits == 3 && mag == 0x7Fu) return u2f(0x7FC00000u);
  if (f->mbits == 2 && E == (1u << ebits) - 1u) {
    if (M) return u2f(0x7FC00000u);
    v = INFINITY;
  } else if (E == 0) {
    v = ldexpf((float)M, 1 - f->bias - f->mbits);
  } else {
    v = ldexpf((float)((1u << f->mbits) + M), (int)E - f->bias - f->mbits);
  }
  return (b & 0x80u) ? -v : v;
}

float or_fp8e4m3_to_f32(uint8_t x) { return ofp8_decode(x, &OFP8_E4M3); }
float or_fp8e5m2_to_f32(uint8_t x) { return ofp8_decode(x, &OFP8_E5M2); }

static float ld(const void *p, uint64_t i, uint32_t dt) {
  switch (dt) {
    case DT_FP32: return ((const float *)p)[i];
    case DT_BF16: return or_bf16_to_f32(((const uint16_t *)p)[i]);
    case DT_FP16: return or_fp16_to_f32(((const uint16_t *)p)[i]);
    case DT_FP8E4M3: return or_fp8e4m3_to_f32(((const uint8_t *)p)[i]);
    case DT_FP8E5M2: return or_fp8e5m2_to_f32(((const uint8_t *)p)[i]);
    default: return 0.0f;
  }
}
/* store with the kernel-store narrowing (uop_walk.c:189-205) */
static void st(void *p, uint64_t i, uint32_t dt, float v) {
  switch (dt) {
    case DT_FP32: ((float *)p)[i] = v; break;
    case DT_BF16: ((uint16_t *)p)[i] = or_f32_to_bf16(v); break;
    case DT_FP16: ((uint16_t *)p)[i] = or_f32_to_fp16(v); break;
    case DT_FP8E4M3: ((uint8_t *)p)[i] = or_f32_to_fp8e4m3_sat(v); break;
    case DT_FP8E5M2: ((uint8_t *)p)[i] = or_f32_to_fp8e5m2_sat(v); break;
    default: break;
  }
}
/* a value rounded through dtype storage (uop_walk.c:272-284) */
static float rnd(float v, uint32_t dt) {
  if (v != v) return v;
  switch (dt) {
    case DT_BF16: return or_bf16_to_f32(or_f32_to_bf16(v));
    case DT_FP16: return or_fp16_to_f32(or_f32_to_fp16(v));
    case DT_FP8E4M3: return or_fp8e4m3_to_f32(or_f32_to_fp8e4m3_sat(v));
    default: return v;
  }
}

void or_decode(const void *src, uint32_t dt, float *dst, uint64_t n) {
  for (uint64_t i = 0; i < n; i++) dst[i] = ld(src, i, dt);
}
void or_encode(const float *src, uint32_t dt, void *dst, uint64_t n) {
  for (uint64_t i = 0; i < n; i++) st(dst, i, dt, src[i]);
}

/* ==== ops ================================================================ */

void or_gemv(float *y, const void *x, uint32_t xdt, uint32_t ldx, const void *w, uint32_t wdt,
             const float *scale, uint32_t M, uint32_t N, uint32_t K) {
  float lut[256];
  if (wdt == DT_FP8E4M3)
    for (int i = 0; i < 256; i++) lut[i] = or_fp8e4m3_to_f32((uint8_t)i);
  float *xf = (float *)malloc((size_t)K * sizeof(float));
  for (uint32_t m = 0; m < M; m++) {
    for (uint32_t k = 0; k < K; k++) xf[k] = ld(x, (uint64_t)m * ldx + k, xdt);
    for (uint32_t n = 0; n < N; n++) {
      float acc = 0.0f;
      const uint64_t r = (uint64_t)n * K;
      if (wdt == DT_FP8E4M3) {
        const uint8_t *q = (const uint8_t *)w + r;
        const float s = scale[n];
        for (uint32_t k = 0; k < K; k++) {
          float wv = lut[q[k]] * s;
          acc += xf[k] * wv;
        }
      } else if (wdt == DT_FP32) {
        const float *wf = (const float *)w + r;
        for (uint32_t k = 0; k < K; k++) acc += xf[k] * wf[k];
      } else {
        for (uint32_t k = 0; k < K; k++) acc += xf[k] * ld(w, r + k, wdt);
      }
      y[(uint64_t)m * N + n] = acc;
    }
  }
  free(xf);
}

void or_rmsnorm(void *y, uint32_t ydt, const void *x, uint32_t xdt, const float *w, uint32_t M,
                uint32_t K, float eps) {
  const float invK = 1.0f / (float)K;
  for (uint32_t m = 0; m < M; m++) {
    const uint64_t o = (uint64_t)m * K;
    float ss = 0.0f;
    for (uint32_t i = 0; i < K; i++) { float v = ld(x, o + i, xdt); ss += v * v; }
    float inv = 1.0f / sqrtf(ss * invK + eps);
    for (uint32_t i = 0; i < K; i++) {
      float v = ld(x, o + i, xdt) * inv;
      if (w) v = v * w[i];
      st(y, o + i, ydt, v);
    }
  }
}

void or_layernorm(void *y, uint32_t ydt, const void *x, uint32_t xdt, const float *w,
                  const float *b, uint32_t M, uint32_t K, float eps) {
  const float invK = 1.0f / (float)K;
  for (uint32_t m = 0; m < M; m++) {
    const uint64_t o = (uint64_t)m * K;
    float s = 0.0f;
    for (uint32_t i = 0; i < K; i++) s += ld(x, o + i, xdt);
    float mean = s * invK, vs = 0.0f;
    for (uint32_t i = 0; i < K; i++) { float d = ld(x, o + i, xdt) - mean; vs += d * d; }
    float r = 1.0f / sqrtf(vs * invK + eps);
    for (uint32_t i = 0; i < K; i++) {
      float v = (ld(x, o + i, xdt) - mean) * r;
      if (w) v = v * w[i];
      if (b) v = v + b[i];
      st(y, o + i, ydt, v);
    }
  }
}

void or_softmax(void *y, uint32_t ydt, const void *x, uint32_t xdt, uint32_t M, uint32_t K) {
  for (uint32_t m = 0; m < M; m++) {
    const uint64_t o = (uint64_t)m * K;
    float mx = -INFINITY;
    for (uint32_t i = 0; i < K; i++) { float v = ld(x, o + i, xdt); if (v > mx) mx = v; }
    float s = 0.0f;
    for (uint32_t i = 0; i < K; i++) s += expf(ld(x, o + i, xdt) - mx);
    float r = 1.0f / s;
    for (uint32_t i = 0; i < K; i++) st(y, o + i, ydt, expf(ld(x, o + i, xdt) - mx) * r);
  }
}

void or_rope(void *x, uint32_t dt, const float *cos_t, const float *sin_t, uint32_t B, uint32_t nh,
             uint32_t hd, uint32_t pos) {
  const uint32_t half = hd / 2;
  for (uint64_t r = 0; r < (uint64_t)B * nh; r++)
    for (uint32_t j = 0; j < half; j++) {
      float c = cos_t[(uint64_t)pos * half + j], s = sin_t[(uint64_t)pos * half + j];
      uint64_t i = r * hd + 2 * j;
      float xe = ld(x, i, dt), xo = ld(x, i + 1, dt);
      st(x, i, dt, xe * c - xo * s);
      st(x, i + 1, dt, xo * c + xe * s);
    }
}

void or_attn_decode(void *out, uint32_t odt, const void *q, uint32_t qdt, const void *kcache,
                    const void *vcache, uint32_t cdt, uint32_t B, uint32_t H, uint32_t Hkv,
                    uint32_t hd, uint32_t max_seq, uint32_t L, float scale) {
  const uint32_t G = H / Hkv;
  float *sc = (float *)malloc((size_t)(L ? L : 1) * sizeof(float));
  for (uint32_t b = 0; b < B; b++)
    for (uint32_t h = 0; h < H; h++) {
      const uint32_t kh = h / G;
      const uint64_t qo = ((uint64_t)b * H + h) * hd;
      const uint64_t cb = ((uint64_t)b * Hkv + kh) * max_seq;
      float mx = -INFINITY;
      for (uint32_t j = 0; j < L; j++) {
        float s = 0.0f;
        for (uint32_t d = 0; d < hd; d++) s += ld(q, qo + d, qdt) * ld(kcache, (cb + j) * hd + d, cdt);
        sc[j] = s * scale;
        if (sc[j] > mx) mx = sc[j];
      }
      float l = 0.0f;
      for (uint32_t j = 0; j < L; j++) { sc[j] = expf(sc[j] - mx); l += sc[j]; }
      for (uint32_t d = 0; d < hd; d++) {
        float a = 0.0f;
        for (uint32_t j = 0; j < L; j++) a += sc[j] * ld(vcache, (cb + j) * hd + d, cdt);
        st(out, qo + d, odt, a / l);
      }
    }
  free(sc);
}

void or_argmax(int32_t *tok, const float *logits, uint32_t B, uint32_t V) {
  for (uint32_t b = 0; b < B; b++) {
    const float *lg = logits + (uint64_t)b * V;
    float bv = lg[0];
    int32_t bi = 0;
    for (uint32_t i = 1; i < V; i++)
      if (lg[i] > bv) { bv = lg[i]; bi = (int32_t)i; }
    tok[b] = bi;
  }
}

/* ==== temperature sampling (the device's rule, restated) ================== */
/* exp by Cody-Waite reduction and a degree-8 Taylor polynomial (Horner, fused
 * multiply-adds), scaled by ldexpf: only correctly rounded IEEE operations,
 * so this and the device's sexpf agree bit for bit. */
float or_sexpf(float x) {
  if (!(x >= -80.0f)) return 0.0f;
  const float k = rintf(x * 0x1.715476p+0f);
  float r = fmaf(-k, 0x1.62e000p-1f, x);
  r = fmaf(-k, 0x1.0bfbe8p-15f, r);
  float p = 0x1.a01a02p-16f;
  p = fmaf(p, r, 0x1.a01a02p-13f);
  p = fmaf(p, r, 0x1.6c16c2p-10f);
  p = fmaf(p, r, 0x1.111112p-7f);
  p = fmaf(p, r, 0x1.555556p-5f);
  p = fmaf(p, r, 0x1.555556p-3f);
  p = fmaf(p, r, 0x1.0p-1f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  return ldexpf(p, (int)k);
}

static uint64_t mix64(uint64_t z) {           /* splitmix64 finaliser */
  z += 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

float or_sample_u01(uint64_t seed, uint32_t row, int32_t L) {
  const uint64_t h = mix64(mix64(seed ^ mix64((uint64_t)row + 1)) + (uint64_t)(uint32_t)L);
  return (float)(uint32_t)(h >> 40) * (1.0f / 16777216.0f);
}

/* the two-level choice over n weights w(k), lane j of 64 owning [jP, (j+1)P) */
typedef float (*WFn)(const void *ctx, uint32_t k);
static int64_t pick2(WFn w, const void *ctx, uint32_t n, uint32_t P, float t, float *base) {
  float q[64];
  for (uint32_t j = 0; j < 64; j++) {
    q[j] = 0.0f;
    for (uint32_t k = j * P; k < (j + 1) * P && k < n; k++) q[j] += w(ctx, k);
  }
  float A = 0.0f, Astar = 0.0f, Al = 0.0f;
  int js = -1, jl = -1;
  for (int j = 0; j < 64; j++) {
    if (q[j] > 0.0f) {
      if (js < 0 && A + q[j] > t) { js = j; Astar = A; }
      jl = j; Al = A;
    }
    A += q[j];
  }
  if (js < 0) { js = jl; Astar = Al; }
  if (js < 0) { *base = 0.0f; return -1; }
  float c = Astar, cs = 0.0f, cl = 0.0f;
  int64_t ks = -1, kl = -1;
  const uint32_t k0 = (uint32_t)js * P, k1 = k0 + P < n ? k0 + P : n;
  for (uint32_t k = k0; k < k1; k++) {
    const float x = w(ctx, k);
    if (x > 0.0f) {
      if (ks < 0 && c + x > t) { ks = k; cs = c; }
      kl = k; cl = c;
    }
    c += x;
  }
  if (ks < 0) { ks = kl; cs = cl; }
  *base = cs;
  return ks;
}

typedef struct { const float *m, *s; float M; } BlkW;
static float blk_w(const void *ctx, uint32_t k) {
  const BlkW *b = (const BlkW *)ctx;
  return b->m[k] == -INFINITY ? 0.0f : b->s[k] * or_sexpf(b->m[k] - b->M);
}
typedef struct { const float *lg; float inv, m; } ElW;
static float el_w(const void *ctx, uint32_t i) {
  const ElW *e = (const ElW *)ctx;
  return or_sexpf(e->lg[i] * e->inv - e->m);
}

void or_sample(int32_t *tok, const float *logits, uint32_t B, uint32_t V, uint32_t nb,
               float inv_temp, uint64_t seed, int32_t L) {
  const uint32_t C = (V + nb - 1) / nb;
  float *m = (float *)malloc((size_t)nb * 4), *sk = (float *)malloc((size_t)nb * 4);
  for (uint32_t b = 0; b < B; b++) {
    const float *lg = logits + (uint64_t)b * V;
    for (uint32_t k = 0; k < nb; k++) {           /* k_sample_part: one block per chunk */
      const uint64_t lo = (uint64_t)k * C, hi = lo + C < V ? lo + C : V;
      float mx = -INFINITY, sv[256];
      for (uint64_t i = lo; i < hi; i++) mx = fmaxf(mx, lg[i] * inv_temp);
      for (uint32_t t = 0; t < 256; t++) {
        sv[t] = 0.0f;
        if (mx != -INFINITY)
          for (uint64_t i = lo + t; i < hi; i += 256) sv[t] += or_sexpf(lg[i] * inv_temp - mx);
      }
      for (uint32_t st = 128; st > 0; st >>= 1)
        for (uint32_t t = 0; t < st; t++) sv[t] += sv[t + st];
      m[k] = mx;
      sk[k] = sv[0];
    }
    float M = -INFINITY;
    for (uint32_t k = 0; k < nb; k++) M = fmaxf(M, m[k]);
    BlkW bw = {m, sk, M};
    float S = 0.0f;
    const uint32_t P = (nb + 63) / 64;
    for (uint32_t j = 0; j < 64; j++) {               /* lane sums, then lanes in order */
      float q = 0.0f;
      for (uint32_t k = j * P; k < (j + 1) * P && k < nb; k++) q += blk_w(&bw, k);
      S += q;
    }
    const float t = or_sample_u01(seed, b, L) * S;
    float base;
    const int64_t ks = pick2(blk_w, &bw, nb, P, t, &base);
    if (ks < 0) continue;
    const float r = (t - base) / or_sexpf(m[ks] - M);
    const uint64_t lo = (uint64_t)ks * C;
    const uint32_t n = (uint32_t)((lo + C <= V ? lo + C : V) - lo);
    ElW ew = {lg + lo, inv_temp, m[ks]};
    float base2;
    const int64_t is = pick2(el_w, &ew, n, (C + 63) / 64, r, &base2);
    if (is >= 0) tok[b] = (int32_t)(lo + is);
  }
  free(m);
  free(sk);
}

/* ==== blind speculative draft / commit =================================== */

/* draft_prep (bench/dsv2_decode_bench.c:1116-1150): candidate 0 is the
 * pending id; candidates 1.. continue the most recent earlier occurrence of
 * the bigram (hist[P-1], hist[P]) -- the largest j with j+1 < P -- while the
 * continuation stays at or before P; forced takes hist[P+1..] instead. */
void or_spec_draft(int32_t *ca, int32_t *ce, const int32_t *hist, int32_t L, uint32_t S,
                   uint32_t V, uint32_t cap, int forced) {
  const int32_t P = L - 1;
  if (P < 0 || P >= (int32_t)cap) {
    for (uint32_t t = 0; t < S; t++) { ca[t] = -1; ce[t] = 0; }
    return;
  }
  const int32_t pend = hist[P];
  const int32_t pend_ok = pend >= 0 && (uint32_t)pend < V ? pend : 0;
  int32_t best = -1;
  if (!forced && P >= 1)
    for (int32_t j = 0; j + 1 < P; j++)
      if (hist[j] == hist[P - 1] && hist[j + 1] == pend) best = j;
  ca[0] = pend;
  ce[0] = pend_ok;
  for (uint32_t t = 1; t < S; t++) {
    int32_t v;
    if (forced) v = P + (int32_t)t < (int32_t)cap ? hist[P + t] : -1;
    else v = (best >= 0 && best + 1 + (int32_t)t <= P) ? hist[best + 1 + t] : -1;
    if (v < 0 || (uint32_t)v >= V) v = -1;
    ca[t] = v;
    ce[t] = v >= 0 ? v : pend_ok;
  }
}

/* accept_commit (:1152-1170): k = the longest run of drafts equal to the
 * verify argmax of the row before them; commit them and the bonus am[k]. */
int32_t or_spec_accept(int32_t *hist, int32_t L, const int32_t *ca, const int32_t *am, uint32_t S,
                       uint32_t cap) {
  const int32_t P = L - 1;
  if (P < 0 || P + (int32_t)S >= (int32_t)cap) return L;
  uint32_t k = 0;
  while (k + 1 < S && ca[k + 1] >= 0 && ca[k + 1] == am[k]) k++;
  for (uint32_t i = 0; i < k; i++) hist[P + 1 + i] = ca[1 + i];
  hist[P + 1 + k] = am[k];
  return P + (int32_t)k + 2;
}

/* ==== whole decode step ================================================== */

static float silu(float g) { return g / (1.0f + expf(-g)); }
static float gelu(float x) {
  float u = 0.7978845608f * (x + 0.044715f * x * x * x);
  return 0.5f * x * (1.0f + tanhf(u));
}

int or_decode_step(const OrModel *m, const int32_t *tok, uint32_t pos, float *logits, int32_t *next) {
  if (!m || (m->arch != 1 && m->arch != 2) || pos >= m->max_seq) return -1;
  const uint32_t D = m->dim, H = m->n_heads, Hkv = m->n_kv_heads ? m->n_kv_heads : m->n_heads;
  const uint32_t hd = m->head_dim, F = m->ffn, V = m->vocab, adt = m->adt, wdt = m->wdt;
  const uint32_t nqkv = m->arch == 1 ? (H + 2 * Hkv) * hd : 3 * D;
  const int gpt2 = m->arch == 2;
  float *x = (float *)malloc((size_t)D * 4), *xn = (float *)malloc((size_t)D * 4);
  float *qkv = (float *)malloc((size_t)nqkv * 4), *q = (float *)malloc((size_t)H * hd * 4);
  float *att = (float *)malloc((size_t)H * hd * 4), *o = (float *)malloc((size_t)D * 4);
  float *gu = (float *)malloc((size_t)2 * F * 4), *hh = (float *)malloc((size_t)F * 4);
  const float scale = (float)(1.0 / sqrt((double)hd));
  const uint32_t B = m->batch, bend = m->b1 ? m->b1 : B;
  /* teacher input / tap row of sublayer t, batch row b */
#define TROW(a, t, b, w) ((a) + ((uint64_t)(t) * B + (b)) * (w))
  for (uint32_t b = m->b0; b < bend; b++) {
    /* embedding (+ learned position) */
    int32_t t = tok[b];
    for (uint32_t i = 0; i < D; i++) {
      float v = (t >= 0 && (uint32_t)t < V) ? ld(m->emb, (uint64_t)t * D + i, adt) : 0.0f;
      if (gpt2) v = v + ld(m->pos_emb, (uint64_t)pos * D + i, adt);
      x[i] = rnd(v, adt);
    }
    for (uint32_t l = 0; l < m->n_layers; l++) {
      const OrLayer *L = &m->layers[l];
      if (m->tf_x) memcpy(x, TROW(m->tf_x, 2 * l, b, D), (size_t)D * 4);
      if (gpt2) or_layernorm(xn, DT_FP32, x, DT_FP32, L->g1, L->b1, 1, D, m->eps);
      else or_rmsnorm(xn, DT_FP32, x, DT_FP32, L->g1, 1, D, m->eps);
      for (uint32_t i = 0; i < D; i++) xn[i] = rnd(xn[i], adt);
      or_gemv(qkv, xn, DT_FP32, D, L->wqkv, wdt, L->sqkv, 1, nqkv, D);
      for (uint32_t n = 0; n < nqkv; n++) {
        float v = qkv[n] + (gpt2 ? ld(L->bqkv, n, adt) : 0.0f);
        qkv[n] = rnd(v, adt);
      }
      const uint32_t Hq = H * hd, Hk = Hkv * hd;
      if (!gpt2) {
        for (uint32_t n = 0; n < Hq + Hk; n += 2) {
          uint32_t j = (n % hd) / 2;
          float c = m->rope_cos[(uint64_t)pos * (hd / 2) + j], s = m->rope_sin[(uint64_t)pos * (hd / 2) + j];
          float xe = qkv[n], xo = qkv[n + 1];
          qkv[n] = rnd(xe * c - xo * s, adt);
          qkv[n + 1] = rnd(xo * c + xe * s, adt);
        }
      }
      memcpy(q, qkv, (size_t)Hq * 4);
      if (m->tp_q) memcpy(TROW(m->tp_q, l, b, Hq), q, (size_t)Hq * 4);
      for (uint32_t kh = 0; kh < Hkv; kh++)
        for (uint32_t d = 0; d < hd; d++) {
          uint64_t ci = (((uint64_t)b * Hkv + kh) * m->max_seq + pos) * hd + d;
          st(L->kcache, ci, adt, qkv[Hq + kh * hd + d]);
          st(L->vcache, ci, adt, qkv[Hq + Hk + kh * hd + d]);
        }
      /* attention for this row: caches hold row b's history */
      {
        const uint32_t G = H / Hkv;
        const uint32_t Lc = pos + 1;
        float *sc = (float *)malloc((size_t)Lc * 4);
        for (uint32_t h = 0; h < H; h++) {
          const uint64_t cb = ((uint64_t)b * Hkv + h / G) * m->max_seq;
          float mx = -INFINITY;
          for (uint32_t j = 0; j < Lc; j++) {
            float s = 0.0f;
            for (uint32_t d = 0; d < hd; d++) s += q[h * hd + d] * ld(L->kcache, (cb + j) * hd + d, adt);
            sc[j] = s * scale;
            if (sc[j] > mx) mx = sc[j];
          }
          float den = 0.0f;
          for (uint32_t j = 0; j < Lc; j++) { sc[j] = expf(sc[j] - mx); den += sc[j]; }
          for (uint32_t d = 0; d < hd; d++) {
            float a = 0.0f;
            for (uint32_t j = 0; j < Lc; j++) a += sc[j] * ld(L->vcache, (cb + j) * hd + d, adt);
            att[h * hd + d] = rnd(a / den, adt);
          }
        }
        free(sc);
      }
      if (m->tp_att) memcpy(TROW(m->tp_att, l, b, Hq), att, (size_t)Hq * 4);
      or_gemv(o, att, DT_FP32, Hq, L->wo, wdt, L->so, 1, D, Hq);
      for (uint32_t i = 0; i < D; i++) {
        float v = o[i] + (gpt2 ? ld(L->bo, i, adt) : 0.0f);
        x[i] = rnd(x[i] + rnd(v, adt), adt);
      }
      if (m->tp_x) memcpy(TROW(m->tp_x, 2 * l, b, D), x, (size_t)D * 4);
      if (m->tf_x) memcpy(x, TROW(m->tf_x, 2 * l + 1, b, D), (size_t)D * 4);
      if (gpt2) or_layernorm(xn, DT_FP32, x, DT_FP32, L->g2, L->b2, 1, D, m->eps);
      else or_rmsnorm(xn, DT_FP32, x, DT_FP32, L->g2, 1, D, m->eps);
      for (uint32_t i = 0; i < D; i++) xn[i] = rnd(xn[i], adt);
      if (gpt2) {
        or_gemv(gu, xn, DT_FP32, D, L->wgu, wdt, L->sgu, 1, F, D);
        for (uint32_t i = 0; i < F; i++) hh[i] = rnd(gelu(rnd(gu[i] + ld(L->bfc, i, adt), adt)), adt);
      } else {
        or_gemv(gu, xn, DT_FP32, D, L->wgu, wdt, L->sgu, 1, 2 * F, D);
        for (uint32_t i = 0; i < F; i++) {
          float g = rnd(gu[2 * i], adt), u = rnd(gu[2 * i + 1], adt);
          hh[i] = rnd(silu(g) * u, adt);
        }
      }
      if (m->tp_h) memcpy(TROW(m->tp_h, l, b, F), hh, (size_t)F * 4);
      or_gemv(o, hh, DT_FP32, F, L->wd, wdt, L->sd, 1, D, F);
      for (uint32_t i = 0; i < D; i++) {
        float v = o[i] + (gpt2 ? ld(L->bpr, i, adt) : 0.0f);
        x[i] = rnd(x[i] + rnd(v, adt), adt);
      }
      if (m->tp_x) memcpy(TROW(m->tp_x, 2 * l + 1, b, D), x, (size_t)D * 4);
    }
    if (m->tf_x) memcpy(x, TROW(m->tf_x, 2 * m->n_layers, b, D), (size_t)D * 4);
    if (gpt2) or_layernorm(xn, DT_FP32, x, DT_FP32, m->gf, m->bf, 1, D, m->eps);
    else or_rmsnorm(xn, DT_FP32, x, DT_FP32, m->gf, 1, D, m->eps);
    for (uint32_t i = 0; i < D; i++) xn[i] = rnd(xn[i], adt);
    float *lg = logits + (uint64_t)b * V;
    if (gpt2) or_gemv(lg, xn, DT_FP32, D, m->emb, adt, NULL, 1, V, D);
    else or_gemv(lg, xn, DT_FP32, D, m->lm, wdt, m->lm_s, 1, V, D);
    or_argmax(&next[b], lg, 1, V);
  }
  free(x); free(xn); free(qkv); free(q); free(att); free(o); free(gu); free(hh);
  return 0;
}
#undef TROW

/* ==== DeepSeek-V2 decode (bench/dsv2_decode_bench.c) ====================== */

/* The dense layer's h = silu(g) * u as the reference builds it, from bf16
 * uops (bench/dsv2_decode_bench.c:2042-2049, :2372): x * recip(1 + exp2(x *
 * c)) * u with c the bf16 CONST -log2(e).  On the reference CPU path the
 * constant holds its bf16 value (-1.4453125) and, being a non-f32 float
 * constant, is a double literal, so every op of the chain promotes to double
 * and exp2 is libm's double one (src/backend/cpu/uop_walk.c:357-409,
 * :685-730); the bf16 store narrows double -> f32 -> bf16 (:216-229).  Pinned
 * bit for bit against the reference realizing this DAG
 * (oracle/ref_harness.c ref_dense_silu_mul_bf16), including exp2 past the
 * f32 range, and by the dense-layer trajectory fixture. */
static float silu_bf16_uops(float g, float u) {
  const double c = (double)or_bf16_to_f32(or_f32_to_bf16(-1.4426950408889634f));
  const double sig = 1.0 / (1.0 + exp2((double)g * c));
  return (float)(((double)g * sig) * (double)u);
}

void or_dsv2_dense_act(const uint16_t *g, const uint16_t *u, uint16_t *h, uint64_t n) {
  for (uint64_t i = 0; i < n; i++)
    h[i] = or_f32_to_bf16(silu_bf16_uops(or_bf16_to_f32(g[i]), or_bf16_to_f32(u[i])));
}

/* sum_k x[k] * w~[row][k], w~ = decode(w) * scale[row] (scale NULL: 1), serial */
static float wdot(const float *x, const void *w, uint32_t wdt, const float *scale, uint64_t row,
                  uint32_t K) {
  const float s = scale ? scale[row] : 1.0f;
  float acc = 0.0f;
  for (uint32_t k = 0; k < K; k++) {
    float wv = ld(w, row * K + k, wdt);
    if (scale) wv = wv * s;
    acc += x[k] * wv;
  }
  return acc;
}

void or_mla_prep(uint16_t *qpe, float *qlat, uint16_t *ckv_row, uint16_t *kpe_row,
                 const uint16_t *qkv_raw, const void *wuk, uint32_t wdt, const float *suk,
                 const float *wkvn, const float *cos_row, const float *sin_row,
                 uint32_t H, uint32_t dn, uint32_t dr, uint32_t kv, float eps) {
  const uint32_t half = dr / 2, qs = dn + dr, qoff = H * qs;
  float *qn = (float *)malloc((size_t)dn * sizeof(float));
  float *v = (float *)malloc((size_t)kv * sizeof(float));
  for (uint32_t h = 0; h < H; h++) {
    const uint32_t base = h * qs;
    for (uint32_t j = 0; j < half; j++) {           /* gred_q pe pairs :474-483 */
      float xe = or_bf16_to_f32(qkv_raw[base + dn + 2 * j]);
      float xo = or_bf16_to_f32(qkv_raw[base + dn + 2 * j + 1]);
      float c = cos_row[j], sv = sin_row[j];
      qpe[h * dr + j] = or_f32_to_bf16(xe * c - xo * sv);
      qpe[h * dr + half + j] = or_f32_to_bf16(xo * c + xe * sv);
    }
    for (uint32_t d = 0; d < dn; d++) qn[d] = or_bf16_to_f32(qkv_raw[base + d]);
    for (uint32_t k = 0; k < kv; k++)                /* mla_qlat :658-666 */
      qlat[h * kv + k] = wdot(qn, wuk, wdt, suk, (uint64_t)h * kv + k, dn);
  }
  float ss = 0.0f;                                   /* kv_prep :531-540 */
  for (uint32_t t = 0; t < kv; t++) {
    v[t] = or_bf16_to_f32(qkv_raw[qoff + t]);
    ss += v[t] * v[t];
  }
  const float inv = 1.0f / sqrtf(ss * (1.0f / (float)kv) + eps);
  for (uint32_t t = 0; t < kv; t++) ckv_row[t] = or_f32_to_bf16((v[t] * inv) * wkvn[t]);
  for (uint32_t j = 0; j < half; j++) {
    float xe = or_bf16_to_f32(qkv_raw[qoff + kv + 2 * j]);
    float xo = or_bf16_to_f32(qkv_raw[qoff + kv + 2 * j + 1]);
    float c = cos_row[j], sv = sin_row[j];
    kpe_row[j] = or_f32_to_bf16(xe * c - xo * sv);
    kpe_row[half + j] = or_f32_to_bf16(xo * c + xe * sv);
  }
  free(qn);
  free(v);
}

void or_mla_attn(uint16_t *o, const float *qlat, const uint16_t *qpe, const uint16_t *ckv,
                 const uint16_t *kpe, uint32_t L, const void *wuv, uint32_t wdt,
                 const float *suv, uint32_t H, uint32_t kv, uint32_t dr, uint32_t dv,
                 float scale) {
  float *sc = (float *)malloc((size_t)(L ? L : 1) * sizeof(float));
  float *olat = (float *)malloc((size_t)kv * sizeof(float));
  for (uint32_t h = 0; h < H; h++) {
    float gmax = -1e30f;                             /* mla_score C twin :707-719 */
    for (uint32_t j = 0; j < L; j++) {
      float s = 0.0f;
      for (uint32_t k = 0; k < kv; k++) s += qlat[h * kv + k] * or_bf16_to_f32(ckv[(uint64_t)j * kv + k]);
      for (uint32_t r = 0; r < dr; r++) s += or_bf16_to_f32(qpe[h * dr + r]) * or_bf16_to_f32(kpe[(uint64_t)j * dr + r]);
      sc[j] = s * scale;
      if (sc[j] > gmax) gmax = sc[j];
    }
    float gsum = 0.0f;
    for (uint32_t j = 0; j < L; j++) { sc[j] = expf(sc[j] - gmax); gsum += sc[j]; }
    for (uint32_t j = 0; j < L; j++) sc[j] = sc[j] / gsum;
    for (uint32_t k = 0; k < kv; k++) {              /* mla_mix :741-748 */
      float a = 0.0f;
      for (uint32_t j = 0; j < L; j++) a += sc[j] * or_bf16_to_f32(ckv[(uint64_t)j * kv + k]);
      olat[k] = a;
    }
    for (uint32_t mm = 0; mm < dv; mm++)             /* mla_o :775-783 */
      o[h * dv + mm] = or_f32_to_bf16(wdot(olat, wuv, wdt, suv, (uint64_t)h * dv + mm, kv));
  }
  free(sc);
  free(olat);
}

void or_route(int32_t *sel, float *probs, const float *g, uint32_t E, uint32_t K) {
  float mx = g[0];                                   /* route C twin :845-860 */
  for (uint32_t e = 1; e < E; e++) if (g[e] > mx) mx = g[e];
  float sum = 0.0f;
  for (uint32_t e = 0; e < E; e++) sum += expf(g[e] - mx);
  for (uint32_t kk = 0; kk < K; kk++) {
    int32_t best = -1;
    float bv = -3.4e38f;
    for (uint32_t e = 0; e < E; e++) {
      int used = 0;
      for (uint32_t j = 0; j < kk; j++) if (sel[j] == (int32_t)e) used = 1;
      if (!used && g[e] > bv) { bv = g[e]; best = (int32_t)e; }
    }
    sel[kk] = best;
    probs[kk] = expf(g[best] - mx) / sum;
  }
}

void or_moe(float *out, const uint16_t *xb, const int32_t *sel, const float *probs,
            const void *wgu_e, const float *sgu_e, const void *wd_e, const float *sd_e,
            const void *wgu_s, const float *sgu_s, const void *wd_s, const float *sd_s,
            uint32_t wdt, uint32_t D, uint32_t I, uint32_t S, uint32_t K) {
  float *x = (float *)malloc((size_t)D * sizeof(float));
  float *h = (float *)malloc(((size_t)K * I + S) * sizeof(float));
  for (uint32_t k = 0; k < D; k++) x[k] = or_bf16_to_f32(xb[k]);
  for (uint32_t e = 0; e < K; e++)                   /* moe_full_h C twin :895-908 */
    for (uint32_t i = 0; i < I; i++) {
      const uint64_t r = (uint64_t)sel[e] * 2 * I + 2 * i;
      float g = wdot(x, wgu_e, wdt, sgu_e, r, D), u = wdot(x, wgu_e, wdt, sgu_e, r + 1, D);
      h[e * I + i] = silu(g) * u;
    }
  for (uint32_t i = 0; i < S; i++) {
    float g = wdot(x, wgu_s, wdt, sgu_s, 2 * i, D), u = wdot(x, wgu_s, wdt, sgu_s, 2 * i + 1, D);
    h[K * I + i] = silu(g) * u;
  }
  for (uint32_t d = 0; d < D; d++) {                 /* moe_full_out C twin :947-963 */
    float acc = 0.0f;
    for (uint32_t e = 0; e < K; e++)
      acc += probs[e] * wdot(h + e * I, wd_e, wdt, sd_e, (uint64_t)sel[e] * D + d, I);
    acc += wdot(h + K * I, wd_s, wdt, sd_s, d, S);
    out[d] = acc;
  }
  free(x);
  free(h);
}

/* The reference's M=1 projection is a two-phase split-K GEMV: phase 1 sums
 * each of sk contiguous K-chunks into a partial, phase 2 folds the partials in
 * chunk order (gemv_pick_sk :1043-1048, src_gemv C twin :1073-1084, the folds
 * of src_gred :1100-1107 / gred_q / kv_prep / gred_o_rms / route).  sk
 * doubles while ceil(N/256)*sk < 232 and sk*64 < K. */
static uint32_t gemv_pick_sk(uint32_t K, uint32_t N) {
  const uint32_t gx = (N + 255) / 256;
  uint32_t sk = 1;
  while (gx * sk < 232u && sk * 64u < K) sk *= 2;
  return sk;
}
static void gemv_sk(float *y, const float *x, const void *w, uint32_t wdt, const float *scale,
                    uint32_t N, uint32_t K, uint32_t sk) {
  const uint32_t chunk = (K + sk - 1) / sk;
  for (uint32_t n = 0; n < N; n++) {
    float s = 0.0f;
    for (uint32_t i = 0; i < sk; i++) {
      const uint32_t k0 = i * chunk, k1 = k0 + chunk > K ? K : k0 + chunk;
      float acc = 0.0f;
      for (uint32_t k = k0; k < k1; k++) {
        float wv = ld(w, (uint64_t)n * K + k, wdt);
        if (scale) wv = wv * scale[n];
        acc += x[k] * wv;
      }
      s += acc;
    }
    y[n] = s;
  }
}

int or_dsv2_step(const OrDsv2 *m, const int32_t *tok, uint32_t pos, float *logits, int32_t *next) {
  if (!m || pos >= m->max_seq || m->top_k > m->n_experts || m->top_k > 64 || m->d_rope % 2)
    return -1;
  const uint32_t D = m->dim, H = m->n_heads, kv = m->kv_lora, dn = m->d_nope, dr = m->d_rope;
  const uint32_t dv = m->d_v, I = m->moe_inter, S = m->n_shared * m->moe_inter, K = m->top_k;
  const uint32_t F = m->dense_inter, V = m->vocab, E = m->n_experts, wdt = m->wdt;
  const uint32_t nqkv = H * (dn + dr) + kv + dr;
  float *x = (float *)malloc((size_t)D * 4), *xn = (float *)malloc((size_t)D * 4);
  float *qkv = (float *)malloc((size_t)nqkv * 4), *qlat = (float *)malloc((size_t)H * kv * 4);
  uint16_t *qraw = (uint16_t *)malloc((size_t)nqkv * 2), *qpe = (uint16_t *)malloc((size_t)H * dr * 2);
  uint16_t *o = (uint16_t *)malloc((size_t)H * dv * 2), *xb = (uint16_t *)malloc((size_t)D * 2);
  float *of = (float *)malloc((size_t)(H * dv > D ? H * dv : D) * 4), *tmp = (float *)malloc((size_t)D * 4);
  float *gu = (float *)malloc((size_t)2 * F * 4), *hh = (float *)malloc((size_t)F * 4);
  float *lg = (float *)malloc((size_t)E * 4);
  int32_t sel[64];
  float probs[64];
  const uint32_t B = m->batch, bend = m->b1 ? m->b1 : B;
#define TROW(a, t, b, w) ((a) + ((uint64_t)(t) * B + (b)) * (w))
  for (uint32_t b = m->b0; b < bend; b++) {
    int32_t t = tok[b];                              /* embed_row :377-395 */
    for (uint32_t i = 0; i < D; i++)
      x[i] = (t >= 0 && (uint32_t)t < V) ? or_bf16_to_f32(m->emb[(uint64_t)t * D + i]) : 0.0f;
    for (uint32_t l = 0; l < m->n_layers; l++) {
      const OrDsv2Layer *Ly = &m->layers[l];
      uint16_t *ckv = Ly->ckv + (uint64_t)b * m->max_seq * kv;
      uint16_t *kpe = Ly->kpe + (uint64_t)b * m->max_seq * dr;
      if (m->tf_x) memcpy(x, TROW(m->tf_x, 2 * l, b, D), (size_t)D * 4);
      or_rmsnorm(xn, DT_FP32, x, DT_FP32, Ly->win, 1, D, m->eps);
      for (uint32_t i = 0; i < D; i++) xn[i] = rnd(xn[i], DT_BF16);   /* rms1 out bf16 */
      gemv_sk(qkv, xn, Ly->wqkv, wdt, Ly->sqkv, nqkv, D, gemv_pick_sk(D, H * (dn + dr)));
      for (uint32_t n = 0; n < nqkv; n++) qraw[n] = or_f32_to_bf16(qkv[n]);
      or_mla_prep(qpe, qlat, ckv + (uint64_t)pos * kv, kpe + (uint64_t)pos * dr, qraw, Ly->wuk, wdt,
                  Ly->suk, Ly->wkvn, m->rope_cos + (uint64_t)pos * (dr / 2),
                  m->rope_sin + (uint64_t)pos * (dr / 2), H, dn, dr, kv, m->eps);
      or_mla_attn(o, qlat, qpe, ckv, kpe, pos + 1, Ly->wuv, wdt, Ly->suv, H, kv, dr, dv, m->scale);
      for (uint32_t i = 0; i < H * dv; i++) of[i] = or_bf16_to_f32(o[i]);
      if (m->tp_o) memcpy(TROW(m->tp_o, l, b, H * dv), of, (size_t)H * dv * 4);
      gemv_sk(tmp, of, Ly->wo, wdt, Ly->so, D, H * dv, gemv_pick_sk(H * dv, D));
      for (uint32_t i = 0; i < D; i++) x[i] = rnd(x[i] + rnd(tmp[i], DT_BF16), DT_BF16);  /* x1 */
      if (m->tp_x) memcpy(TROW(m->tp_x, 2 * l, b, D), x, (size_t)D * 4);
      if (m->tf_x) memcpy(x, TROW(m->tf_x, 2 * l + 1, b, D), (size_t)D * 4);
      or_rmsnorm(xn, DT_FP32, x, DT_FP32, Ly->wpost, 1, D, m->eps);                       /* xn2f */
      for (uint32_t i = 0; i < D; i++) xb[i] = or_f32_to_bf16(xn[i]);                     /* xn2b */
      if (l < m->first_dense) {
        for (uint32_t i = 0; i < D; i++) tmp[i] = or_bf16_to_f32(xb[i]);
        gemv_sk(gu, tmp, Ly->wgu, wdt, Ly->sgu, 2 * F, D, gemv_pick_sk(D, F));
        for (uint32_t i = 0; i < F; i++) {
          float g = rnd(gu[2 * i], DT_BF16), u = rnd(gu[2 * i + 1], DT_BF16);
          hh[i] = rnd(silu_bf16_uops(g, u), DT_BF16);
        }
        gemv_sk(tmp, hh, Ly->wd, wdt, Ly->sd, D, F, gemv_pick_sk(F, D));
      } else {
        gemv_sk(lg, xn, Ly->gate, DT_FP32, NULL, E, D, gemv_pick_sk(D, E));
        or_route(sel, probs, lg, E, K);
        const uint64_t lb = (uint64_t)l * m->batch + b;     /* [layer][row] records */
        if (m->gate_out) memcpy(m->gate_out + lb * E, lg, E * sizeof(float));
        if (m->sel_out) {
          memcpy(m->sel_out + lb * K, sel, K * sizeof(int32_t));
          memcpy(m->probs_out + lb * K, probs, K * sizeof(float));
        }
        const int32_t *use_sel = m->tf_sel ? m->tf_sel + lb * K : sel;
        const float *use_probs = m->tf_probs ? m->tf_probs + lb * K : probs;
        or_moe(tmp, xb, use_sel, use_probs, Ly->wgu_e, Ly->sgu_e, Ly->wd_e, Ly->sd_e, Ly->wgu_s,
               Ly->sgu_s, Ly->wd_s, Ly->sd_s, wdt, D, I, S, K);
      }
      for (uint32_t i = 0; i < D; i++) x[i] = rnd(x[i] + rnd(tmp[i], DT_BF16), DT_BF16);
      if (m->tp_x) memcpy(TROW(m->tp_x, 2 * l + 1, b, D), x, (size_t)D * 4);
    }
    if (m->tf_x) memcpy(x, TROW(m->tf_x, 2 * m->n_layers, b, D), (size_t)D * 4);
    or_rmsnorm(xn, DT_FP32, x, DT_FP32, m->gf, 1, D, m->eps);                             /* rms_f f32 */
    float *lgb = logits + (uint64_t)b * V;
    gemv_sk(lgb, xn, m->lm, wdt, m->lm_s, V, D, gemv_pick_sk(D, V));
    or_argmax(&next[b], lgb, 1, V);
  }
  free(x); free(xn); free(qkv); free(qlat); free(qraw); free(qpe); free(o); free(xb);
  free(of); free(tmp); free(gu); free(hh); free(lg);
  return 0;
}
#undef TROW
