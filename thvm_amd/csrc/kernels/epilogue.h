// epilogue.h -- output stage shared by the GEMV and the MFMA GEMM: per-row
// fp8 scale and bias, then store / residual add / GELU / SwiGLU over row
// pairs / q,k RoPE with KV-cache append at position L-1.  Rounding points
// follow the reference decode chain (bench/dsv2_decode_bench.c:20-34): a
// projection output is rounded to the activation dtype before it feeds a
// residual add, an activation or the rotation.
#pragma once
#include "dev_common.h"
#include "coh.h"
#include "../kern_api.h"

__device__ __forceinline__ float ld_any(const void *p, uint64_t i, uint32_t dt) {
  switch (dt) {
    case THVM_DT_FP32: return ((const float *)p)[i];
    case THVM_DT_BF16: return bf2f(((const bf16_t *)p)[i]);
    case THVM_DT_FP16: return h2f(((const f16_t *)p)[i]);
    default: return 0.0f;
  }
}
__device__ __forceinline__ void st_any(void *p, uint64_t i, uint32_t dt, float v) {
  switch (dt) {
    case THVM_DT_FP32: ((float *)p)[i] = v; break;
    case THVM_DT_BF16: ((bf16_t *)p)[i] = f2bf(v); break;
    case THVM_DT_FP16: ((f16_t *)p)[i] = f2h(v); break;
    default: break;
  }
}
// COH: system-scope accesses (buffers shared between the blocks of one
// launch); byte offsets stay below 2 GiB
template <bool COH>
__device__ __forceinline__ float ld_anyc(const void *p, uint64_t i, uint32_t dt) {
  if (!COH) return ld_any(p, i, dt);
  switch (dt) {
    case THVM_DT_FP32: return coh_ldf(p, (uint32_t)(i * 4));
    case THVM_DT_BF16: return bf2f(coh_ld2(p, (uint32_t)(i * 2)));
    case THVM_DT_FP16: return h2f(coh_ld2(p, (uint32_t)(i * 2)));
    default: return 0.0f;
  }
}
template <bool COH>
__device__ __forceinline__ void st_anyc(void *p, uint64_t i, uint32_t dt, float v) {
  if (!COH) { st_any(p, i, dt, v); return; }
  switch (dt) {
    case THVM_DT_FP32: coh_stf(p, (uint32_t)(i * 4), v); break;
    case THVM_DT_BF16: coh_st2(p, (uint32_t)(i * 2), f2bf(v)); break;
    case THVM_DT_FP16: coh_st2(p, (uint32_t)(i * 2), f2h(v)); break;
    default: break;
  }
}
__device__ __forceinline__ float rnd_any(float v, uint32_t dt) {
  return dt == THVM_DT_BF16 ? rbf(v) : dt == THVM_DT_FP16 ? rh(v) : v;
}

// The epilogue operands of one row group, loaded ahead of the epilogue (the
// GEMV issues them before its x and weight loads, so the epilogue waits for
// no memory round trip of its own): row scales, the residual values (RESID),
// the position and the RoPE pair of the group's one row pair (QKV*).
template <int R, int M>
struct EpiPre {
  uint32_t sc[R];        // f32 bits of the row scales (read only with a.scale)
  uint32_t rv[R][M];     // the residual values in their storage bits
  float cs[M], sn[M];
  int32_t pos;
};

// Rows n0..n0+R-1 of batch rows mb..mb+M-1; tot[r][m] is the raw f32 sum.
// COH: y, res and the caches are read/written with system-scope accesses.
// pre: the group's operands already loaded (else read here).
template <int R, int M, bool COH = false>
__device__ __forceinline__ void gemv_epilogue(const ThvmGemvArgs &a, const uint32_t n0,
                                              const float (&tot)[R][M],
                                              const uint32_t mb = 0,
                                              const EpiPre<R, M> *pre = nullptr) {
  const uint32_t N = a.N;
  float v[R][M];
#pragma unroll
  for (int r = 0; r < R; r++) {
    uint32_t n = n0 + r;
    float s = (a.scale != nullptr && n < N) ? (pre ? __uint_as_float(pre->sc[r]) : a.scale[n]) : 1.0f;
    float bv = (a.bias != nullptr && n < N) ? ld_any(a.bias, n, a.ydt) : 0.0f;
#pragma unroll
    for (int m = 0; m < M; m++) v[r][m] = tot[r][m] * s + bv;
  }
  const uint32_t ydt = a.ydt;
  switch (a.epi) {
    case THVM_EPI_STORE:
#pragma unroll
      for (int r = 0; r < R; r++)
        if (n0 + r < N)
#pragma unroll
          for (int m = 0; m < M; m++)
            st_anyc<COH>(a.y, (uint64_t)(mb + m) * a.ldy + n0 + r, ydt, v[r][m]);
      break;
    case THVM_EPI_RESID:
#pragma unroll
      for (int r = 0; r < R; r++)
        if (n0 + r < N)
#pragma unroll
          for (int m = 0; m < M; m++) {
            uint64_t i = (uint64_t)(mb + m) * a.ldy + n0 + r;
            const uint32_t rb = pre ? pre->rv[r][m] : 0u;
            float rv = !pre ? ld_anyc<COH>(a.res, i, ydt)
                     : ydt == THVM_DT_FP32 ? __uint_as_float(rb)
                     : ydt == THVM_DT_BF16 ? bf2f((bf16_t)rb) : h2f((f16_t)rb);
            st_anyc<COH>(a.y, i, ydt, rv + rnd_any(v[r][m], ydt));
          }
      break;
    case THVM_EPI_GELU:
#pragma unroll
      for (int r = 0; r < R; r++)
        if (n0 + r < N)
#pragma unroll
          for (int m = 0; m < M; m++)
            st_anyc<COH>(a.y, (uint64_t)(mb + m) * a.ldy + n0 + r, ydt,
                   gelu_tanh_f(rnd_any(v[r][m], ydt)));
      break;
    case THVM_EPI_SWIGLU:
      if (R % 2 == 0) {
#pragma unroll
        for (int r = 0; r + 1 < R; r += 2) {
          if (n0 + r + 1 >= N) break;
#pragma unroll
          for (int m = 0; m < M; m++) {
            float gg = rnd_any(v[r][m], ydt), uu = rnd_any(v[r + 1][m], ydt);
            st_anyc<COH>(a.y, (uint64_t)(mb + m) * a.ldy + (n0 + r) / 2, ydt, silu_f(gg) * uu);
          }
        }
      }
      break;
    case THVM_EPI_QKV_ROPE:
    case THVM_EPI_QKV: {
      if (R % 2) break;
      const uint32_t hd = a.head_dim;
      const uint32_t Hq = a.n_heads * hd, Hk = a.n_kv_heads * hd;
      const int32_t pos = pre ? pre->pos : a.len[0] - 1;
      if (pos < 0 || (uint32_t)pos >= a.max_seq) break;   // no live row to write
      const bool rope = a.epi == THVM_EPI_QKV_ROPE;
#pragma unroll
      for (int r = 0; r + 1 < R; r += 2) {
        const uint32_t nn = n0 + r;
        if (nn + 1 >= N) break;
        const uint32_t d = nn % hd;
#pragma unroll
        for (int m = 0; m < M; m++) {
          // speculative verify: row m is position pos + m of sequence 0
          const uint32_t pm = (uint32_t)pos + (a.spec ? mb + m : 0u);
          if (pm >= a.max_seq) continue;
          float c = 1.0f, sn = 0.0f;
          if (rope && nn < Hq + Hk) {
            if (pre && R == 2) {
              c = pre->cs[m];
              sn = pre->sn[m];
            } else {
              c = a.rope_cos[(uint64_t)pm * (hd / 2) + d / 2];
              sn = a.rope_sin[(uint64_t)pm * (hd / 2) + d / 2];
            }
          }
          float xe = rnd_any(v[r][m], ydt), xo = rnd_any(v[r + 1][m], ydt);
          float oe = xe, oo = xo;
          if (rope && nn < Hq + Hk) { oe = xe * c - xo * sn; oo = xo * c + xe * sn; }
          if (nn < Hq) {
            st_anyc<COH>(a.y, (uint64_t)(mb + m) * a.ldy + nn, ydt, oe);
            st_anyc<COH>(a.y, (uint64_t)(mb + m) * a.ldy + nn + 1, ydt, oo);
          } else {
            const bool isk = nn < Hq + Hk;
            const uint32_t off = isk ? nn - Hq : nn - Hq - Hk;
            const uint32_t h = off / hd;
            const uint64_t cb = a.spec ? 0u : (uint64_t)(mb + m);
            uint64_t ci = ((cb * a.n_kv_heads + h) * a.max_seq + pm) * hd + d;
            void *cache = isk ? a.kcache : a.vcache;
            st_anyc<COH>(cache, ci, ydt, oe);
            st_anyc<COH>(cache, ci + 1, ydt, oo);
          }
        }
      }
    } break;
    default: break;
  }
}
