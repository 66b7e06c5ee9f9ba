// gemv_core.h -- the decode projection y[m,n] = sum_k x[m,k] W[n,k] as a
// block-level device function, shared by the standalone GEMV kernel
// (gemv.hip) and the persistent decode step (step.hip), so both compute every
// output row with the same instructions in the same order.
//
// W is [N, K] with K contiguous, in f32 / fp16 / bf16 / fp8-e4m3 (+ per-row
// f32 scale), M in 1..4 rows of x, fp32 accumulation:
//   * one wave64 owns R consecutive rows and streams them with 128-bit loads
//     (lane l takes 16-byte chunks l, l+64, ..), U chunks per row in flight
//     per lane before any arithmetic;
//   * the first batch of weight loads is issued BEFORE x is staged -- and, in
//     the persistent kernel, before the grid barrier that makes x valid -- so
//     the staging (and a fused norm's block reduction) hides under HBM
//     latency; the next batch is prefetched while the current one is consumed;
//   * x (M rows) is staged once per block into LDS in its storage type, chunk-
//     swizzled so the 64 lanes' 16-byte LDS reads hit distinct banks; a fused
//     RMSNorm / LayerNorm writes the normalised row there already rounded to
//     the activation dtype, exactly as the separate norm kernel would store it;
//     a summed x (XD_SUM4, one row) is staged as bf16(g ((x0 + x1) + (x2 + x3)))
//     from four f32 vectors -- the MLA merge's quarter sums;
//   * 16-bit x against fp8 or same-type 16-bit weights runs on packed dot
//     products (v_dot2c_f32_bf16 / _f16; fp8 pairs converted exactly with
//     v_cvt_scalef32_pk_*_fp8); other pairings decode both operands to f32
//     for FMAs (fp8 with v_cvt_pk_f32_fp8, OCP e4m3, exact); the per-row
//     scale is applied once after the reduction;
//   * each row's K reduction ends in a DPP wave reduction (fixed order,
//     deterministic): no partial buffer and no second fold kernel.
// A row's sum depends only on the chunk order of its lanes, not on which wave,
// block or launch computes it.
#pragma once
#include "dev_common.h"
#include "coh.h"
#include "../kern_api.h"
#include "epilogue.h"

enum { WT_F32 = 0, WT_F16 = 1, WT_BF16 = 2, WT_FP8 = 3 };
enum { XT_BF16 = 0, XT_F16 = 1, XT_F32 = 2 };

template <int WT> struct WTr;
template <> struct WTr<WT_F32>  { static constexpr int E = 4;  };
template <> struct WTr<WT_F16>  { static constexpr int E = 8;  };
template <> struct WTr<WT_BF16> { static constexpr int E = 8;  };
template <> struct WTr<WT_FP8>  { static constexpr int E = 16; };

// decode the 4 elements of quad j of a 16-byte weight chunk
template <int WT>
__device__ __forceinline__ void quad_decode(const uint4 &q, int j, float o[4]);

template <>
__device__ __forceinline__ void quad_decode<WT_FP8>(const uint4 &q, int j, float o[4]) {
  uint32_t w = j == 0 ? q.x : j == 1 ? q.y : j == 2 ? q.z : q.w;
  fp8x4_to_f32(w, o);
}
template <>
__device__ __forceinline__ void quad_decode<WT_F16>(const uint4 &q, int j, float o[4]) {
  uint32_t a = j == 0 ? q.x : q.z, b = j == 0 ? q.y : q.w;
  o[0] = h2f((f16_t)(a & 0xffffu)); o[1] = h2f((f16_t)(a >> 16));
  o[2] = h2f((f16_t)(b & 0xffffu)); o[3] = h2f((f16_t)(b >> 16));
}
template <>
__device__ __forceinline__ void quad_decode<WT_BF16>(const uint4 &q, int j, float o[4]) {
  uint32_t a = j == 0 ? q.x : q.z, b = j == 0 ? q.y : q.w;
  o[0] = __uint_as_float(a << 16); o[1] = __uint_as_float(a & 0xffff0000u);
  o[2] = __uint_as_float(b << 16); o[3] = __uint_as_float(b & 0xffff0000u);
}
template <>
__device__ __forceinline__ void quad_decode<WT_F32>(const uint4 &q, int j, float o[4]) {
  (void)j;
  o[0] = __uint_as_float(q.x); o[1] = __uint_as_float(q.y);
  o[2] = __uint_as_float(q.z); o[3] = __uint_as_float(q.w);
}

// ---- LDS x layout -----------------------------------------------------------
// 16-bit x: element e of row m lives at halfword  m*K + ((e%E)/8 * C + e/E)*8 + e%8
// f32 x:    element e of row m lives at float     m*K + ((e%E)/4 * C + e/E)*4 + e%4
// (C = K/E chunks per row): the 8 (or 4) elements a lane needs for one quad
// pair are one aligned 16-byte LDS word, and lanes c, c+1 read adjacent words.
template <int XT> struct XTr;
template <> struct XTr<XT_BF16> { static constexpr int B = 2, G = 8; };
template <> struct XTr<XT_F16>  { static constexpr int B = 2, G = 8; };
template <> struct XTr<XT_F32>  { static constexpr int B = 4, G = 4; };

template <int XT, int E>
__device__ __forceinline__ uint32_t xs_index(uint32_t K, uint32_t C, uint32_t m, uint32_t e) {
  constexpr int G = XTr<XT>::G;
  const uint32_t c = e / E, r = e - c * E;
  return m * K + ((r / G) * C + c) * G + (r % G);
}

// 8 x elements of a 16-bit group -> floats
template <int XT>
__device__ __forceinline__ void x8_decode(const uint4 &q, float o[8]) {
  uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
  for (int i = 0; i < 4; i++) {
    if (XT == XT_BF16) {
      o[2 * i] = __uint_as_float(w[i] << 16);
      o[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    } else {
      o[2 * i] = h2f((f16_t)(w[i] & 0xffffu));
      o[2 * i + 1] = h2f((f16_t)(w[i] >> 16));
    }
  }
}

// ---- packed dot products: 16-bit x against fp8 / same-type 16-bit weights --
// v_dot2c_f32_{bf16,f16} takes an x pair and a weight pair as they sit in
// registers (two MACs, f32 accumulate, one instruction); fp8 weight pairs go
// to the x type with one v_cvt_scalef32_pk_{bf16,f16}_fp8 (scale 1: exact, an
// e4m3 value has <= 4 significant bits and its exponent range fits both).
// Two to three times fewer VALU instructions per weight byte than decoding
// both operands to f32 for FMAs: the arithmetic a one-round GEMV does after
// its weights land, on the critical path at batch 1.
template <int WT, int XT>
struct Dot2 {
  static constexpr bool ok = (XT == XT_BF16 && (WT == WT_FP8 || WT == WT_BF16)) ||
                             (XT == XT_F16 && (WT == WT_FP8 || WT == WT_F16));
};
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
// the two element pairs of weight quad j of a 16-byte chunk, in the x type
template <int WT, int XT>
__device__ __forceinline__ void quad_pairs(const uint4 &q, int j, uint32_t &p0, uint32_t &p1) {
  if (WT == WT_FP8) {
    const uint32_t w = j == 0 ? q.x : j == 1 ? q.y : j == 2 ? q.z : q.w;
    if (XT == XT_BF16) {
      p0 = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, false));
      p1 = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.0f, true));
    } else {
      p0 = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.0f, false));
      p1 = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.0f, true));
    }
  } else {
    p0 = j == 0 ? q.x : q.z;
    p1 = j == 0 ? q.y : q.w;
  }
}
template <int XT>
__device__ __forceinline__ float dot2acc(uint32_t x, uint32_t w, float acc) {
  if (XT == XT_BF16)
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, x), __builtin_bit_cast(bf16x2_t, w), acc, false);
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, x), __builtin_bit_cast(f16x2_t, w), acc, false);
}

#define GEMV_MAX_WAVES 16
__device__ __forceinline__ float block_sum_g(float v, float *red, int nwaves) {
  float w = wave_sum(v);
  __syncthreads();
  if (lane_id() == 0) red[threadIdx.x >> 6] = w;
  __syncthreads();
  // (every slot read at once, in wave order; slots at or past nwaves add
  // +0, which leaves the sum's bits as they are: it starts at +0 and so is
  // never -0)
  float t = 0.0f;
#pragma unroll
  for (int i = 0; i < GEMV_MAX_WAVES; i++) {
    const float r = red[i];
    t += i < nwaves ? r : 0.0f;
  }
  return t;
}

#define XREG 16   /* x elements per thread kept in registers by the staging */

// the output stage of one row group (one lane, wave-uniform values)
// input x dtype (compile time): vector loads of 16 bytes
// XD_SUM4: x is the sum of four f32 vectors (stride a.xqs elements), each
// element scaled by norm_w (when given) and rounded to bf16 as it is staged
// -- the MLA merge in latent quarters (k_mla_out_q) hands the o projection
// its four quarter sums this way (M = 1, a.norm = 3)
enum { XD_BF16 = 0, XD_F16 = 1, XD_F32 = 2, XD_SUM4 = 3 };
template <int XD> struct XDr { static constexpr int VE = XD == XD_F32 ? 4 : 8, B = XD == XD_BF16 || XD == XD_F16 ? 2 : 4; };
#define GEMV_SQ 2   /* XD_SUM4: element pairs per thread (K <= 4 x block size) */

// 16 bytes of x (its storage type) -> VE floats
template <int XD>
__device__ __forceinline__ void xdec(const uint4 &q, float *o) {
  const uint32_t w[4] = {q.x, q.y, q.z, q.w};
  if (XD == XD_F32) {
#pragma unroll
    for (int i = 0; i < 4; i++) o[i] = __uint_as_float(w[i]);
  } else {
#pragma unroll
    for (int i = 0; i < 4; i++) {
      if (XD == XD_BF16) {
        o[2 * i] = __uint_as_float(w[i] << 16);
        o[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
      } else {
        o[2 * i] = h2f((f16_t)(w[i] & 0xffffu));
        o[2 * i + 1] = h2f((f16_t)(w[i] >> 16));
      }
    }
  }
}
// 16 bytes of x at element e of the row at x (COH: a system-scope load, for
// rows written by other blocks of the same launch)
template <int XD, bool COH = false>
__device__ __forceinline__ void xvec(const void *x, uint64_t e, float *o) {
  const uint4 q = COH ? coh_ld16(x, (uint32_t)(e * XDr<XD>::B)) : ld16((const char *)x + e * XDr<XD>::B);
  xdec<XD>(q, o);
}
template <int XD>
__device__ __forceinline__ float rnd_x(float v) {
  return XD == XD_BF16 ? rbf(v) : XD == XD_F16 ? rh(v) : v;
}
// 16 raw bytes of x at element e (COH as in xvec)
template <int XD, bool COH = false>
__device__ __forceinline__ uint4 xraw(const void *x, uint64_t e) {
  return COH ? coh_ld16(x, (uint32_t)(e * XDr<XD>::B)) : ld16((const char *)x + e * XDr<XD>::B);
}
// Staging stores.  In the LDS layout the G elements from a multiple of G
// are one aligned 16-byte word, so x vector v (VE elements) lands with one
// 16-byte store per G elements, not one store per element.
// xs_put_raw: vector v of row m as loaded (its storage bits are the LDS type
// unless the weights are f32, where 16-bit x is widened exactly);
// xs_put_f: VE values rounded to the x dtype, as a norm kernel would store
// them.
template <int XD, int XT, int E>
__device__ __forceinline__ void xs_put_raw(unsigned char *xs, uint32_t K, uint32_t C, uint32_t m,
                                           uint32_t v, const uint4 &q) {
  constexpr int VE = XDr<XD>::VE;
  if (XT != XT_F32 || XD == XD_F32) {
    *(uint4 *)(xs + (size_t)xs_index<XT, E>(K, C, m, v * VE) * XTr<XT>::B) = q;
  } else {
    float f[VE];
    xdec<XD>(q, f);
#pragma unroll
    for (int h = 0; h < VE; h += 4)
      *(uint4 *)(xs + (size_t)xs_index<XT, E>(K, C, m, v * VE + h) * 4u) =
          make_uint4(__float_as_uint(f[h]), __float_as_uint(f[h + 1]),
                     __float_as_uint(f[h + 2]), __float_as_uint(f[h + 3]));
  }
}
template <int XD, int XT, int E>
__device__ __forceinline__ void xs_put_f(unsigned char *xs, uint32_t K, uint32_t C, uint32_t m,
                                         uint32_t v, const float *f) {
  constexpr int VE = XDr<XD>::VE;
  if (XT != XT_F32) {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; i++)
      w[i] = XT == XT_BF16 ? (uint32_t)f2bf(f[2 * i]) | ((uint32_t)f2bf(f[2 * i + 1]) << 16)
                           : (uint32_t)f2h(f[2 * i]) | ((uint32_t)f2h(f[2 * i + 1]) << 16);
    *(uint4 *)(xs + (size_t)xs_index<XT, E>(K, C, m, v * VE) * 2u) = make_uint4(w[0], w[1], w[2], w[3]);
  } else {
#pragma unroll
    for (int h = 0; h < VE; h += 4)
      *(uint4 *)(xs + (size_t)xs_index<XT, E>(K, C, m, v * VE + h) * 4u) =
          make_uint4(__float_as_uint(rnd_x<XD>(f[h])), __float_as_uint(rnd_x<XD>(f[h + 1])),
                     __float_as_uint(rnd_x<XD>(f[h + 2])), __float_as_uint(rnd_x<XD>(f[h + 3])));
  }
}

// One block's share of a GEMV.  The calling wave owns row groups g, g +
// gstride, ...; `wait()` runs after the first weight batch is in flight and
// before x is read (return false to abandon the call); `xrow(m)` gives the
// start of x row m; `hook(n0, tot)` runs on lane 0 after each row group's
// epilogue with the raw sums.  COH selects system-scope x loads and epilogue
// accesses (data shared between the blocks of one launch).  x staging uses
// the first nthr threads (nw = nthr / 64 waves reduce a fused norm); the rest
// of the block only joins its barriers.  bdim is the block size, read once by
// the caller (bdim inside a loop was re-read from the implicit kernel
// arguments with a vector load and a full wait, between the early x loads).
// Returns false when wait() did.
template <int WT, int XD, int M, int R, int U, bool COH, class WaitF, class XRowF, class HookF>
__device__ __forceinline__ bool gemv_core(const ThvmGemvArgs &a, unsigned char *xs_raw, float *red,
                                          const uint32_t g, const uint32_t gstride,
                                          const uint32_t nthr, const int nw, WaitF &&wait,
                                          XRowF &&xrow, HookF &&hook, const uint32_t bdim) {
  constexpr int E = WTr<WT>::E;
  // LDS keeps x in its 16-bit storage type unless weights or x are f32
  constexpr int XT = (WT == WT_F32 || XD == XD_F32) ? XT_F32 : (XD == XD_BF16 || XD == XD_SUM4 ? XT_BF16 : XT_F16);
  static_assert(XD != XD_SUM4 || (M == 1 && !COH && WT != WT_F32), "summed x: one row, standalone");
  constexpr int VE = XDr<XD>::VE;
  const uint32_t K = a.K, N = a.N;
  const uint32_t C = K / E;              // 16-byte weight chunks per row
  const int lane = lane_id();
  const uint32_t G = (N + R - 1) / R;
  const uint64_t rowbytes = (uint64_t)K * (16 / E);
  const char *wb = (const char *)a.w;

  // ---- 1. loads in flight before any arithmetic ----
  // Each wave's loads return in issue order.  Standalone at M = 1 with 16-bit
  // x: x and a fused norm's gain / bias vectors are issued first, then the
  // first weight batch, so the staging and the norm's block reductions run
  // while the weights are in flight (measured on gfx950: 1.2-1.3 us less per
  // fused-norm launch at the C4 shapes; no change without a norm; f32 x
  // measured slower).  With more rows (x would hold too many registers across
  // the weight loads) and in the persistent kernel (COH: x is written by other
  // blocks of the launch and is read only after wait()), the weights go first.
  // The weight loads of row group gg, chunk batch c0: raw buffer loads
  // through a resource over the group's rows, so a row past N or a chunk past
  // C reads zero by the hardware range check with no memory access and every
  // wave issues the same load instructions whatever the bounds.  (A guarded
  // load is branched around; the compiler then cannot count the loads issued
  // after any earlier one and makes every wait drain all of them, vmcnt(0):
  // x staging waited for the whole first weight batch and each row group's
  // epilogue for the next batch.)  The resource base is wave-uniform.
  auto wload = [&](uint4 (&X)[R][U], uint32_t gg, uint32_t c0) {
    const bool gok = gg < G;
    const uint32_t n0 = gok ? gg * R : 0u;
    const uint32_t nr = gok ? (N - n0 < (uint32_t)R ? N - n0 : (uint32_t)R) : 0u;
    const uint64_t base = (uint64_t)(uintptr_t)wb + (uint64_t)n0 * rowbytes;
    const uint32_t blo = __builtin_amdgcn_readfirstlane((uint32_t)base);
    const uint32_t bhi = __builtin_amdgcn_readfirstlane((uint32_t)(base >> 32));
    const buf_t rs = buf_rsrc((const void *)(uintptr_t)(((uint64_t)bhi << 32) | blo),
                              __builtin_amdgcn_readfirstlane(nr * (uint32_t)rowbytes));
#pragma unroll
    for (int r = 0; r < R; r++) {
#pragma unroll
      for (int u = 0; u < U; u++) {
        const uint32_t c = c0 + u * 64 + lane;
        X[r][u] = buf_ld_stream16(rs, c < C ? (uint32_t)(r * rowbytes) + c * 16u : BUF_OOB);
      }
    }
  };
  uint4 wq[R][U];
  auto load_batch = [&](uint32_t gg, uint32_t c0) { wload(wq, gg, c0); };
  // The first row group's epilogue operands (standalone kernel), issued
  // before x and the weights so the epilogue waits for no round trip of its
  // own (the qkv epilogue's len -> cos/sin chain was two): unconditional
  // buffer loads, an operand the epilogue does not use reads zero through an
  // empty range; the RoPE pair follows once the position is back (after x
  // staging).  Values only: the epilogue's arithmetic is unchanged.
  constexpr bool PRE = !COH;
  EpiPre<R, M> pre;
  uint32_t pre_len = 0;
  const bool pre_qkv = a.epi == THVM_EPI_QKV || a.epi == THVM_EPI_QKV_ROPE;
  const uint32_t pre_n0 = (g < G ? g : 0u) * R;
  if (PRE) {
    const buf_t rsc = buf_rsrc(a.scale, a.scale ? N * 4u : 0u);
#pragma unroll
    for (int r = 0; r < R; r++) pre.sc[r] = buf_ld4(rsc, (pre_n0 + r) * 4u);
    const bool resid = a.epi == THVM_EPI_RESID && a.res != nullptr;
    const uint32_t ys = a.ydt == THVM_DT_FP32 ? 4u : 2u;
    const buf_t rrs = buf_rsrc(a.res, resid ? (uint32_t)M * a.ldy * ys : 0u);
    // (two 16-bit halves per value whatever the type -- one load kind, so
    // the instruction stream does not branch on the type)
#pragma unroll
    for (int r = 0; r < R; r++)
#pragma unroll
      for (int m = 0; m < M; m++) {
        const uint32_t off = ((uint32_t)m * a.ldy + pre_n0 + r) * ys;
        const uint32_t lo = buf_ld2(rrs, off), hi = buf_ld2(rrs, ys == 4u ? off + 2u : BUF_OOB);
        pre.rv[r][m] = lo | (hi << 16);
      }
    const buf_t rls = buf_rsrc(a.len, pre_qkv ? 4u : 0u);
    pre_len = buf_ld4(rls, 0);
  }
  const uint32_t NVt = K / VE;           // x vectors per row
  // (with a fused norm, threads at or beyond nthr take no part in the staging
  // but join its block barriers: the norm's reduction order is that of an
  // nthr-thread block)
  const uint32_t tid = threadIdx.x < nthr ? threadIdx.x : NVt;
  constexpr int XN = 4;                  // no norm: x vectors per thread per staging pass
  constexpr int NVN = XREG / VE;         // fused norm: x vectors per thread
  constexpr int NPRE = XN > NVN ? XN : NVN;
  // x row 0 as raw 16-byte vectors (!COH): the norm path's vectors tid + j*nthr,
  // or the no-norm path's first pass threadIdx.x + j*bdim (clamped
  // indices; out-of-row vectors are never stored)
  constexpr bool XPRE = !COH && M == 1 && XD != XD_F32 && XD != XD_SUM4;
  // summed x: thread t's element pairs 2 (t + j bdim) of the four quarters
  // and their gains, requested before the weights (8-byte unguarded loads)
  constexpr bool XSUM = XD == XD_SUM4;
  uint2 sqv[XSUM ? GEMV_SQ : 1][4], sgv[XSUM ? GEMV_SQ : 1];
  if constexpr (XSUM) {
    const buf_t xr = buf_rsrc_u(a.x, (3u * a.xqs + K) * 4u);
    const buf_t gr = buf_rsrc_u(a.norm_w, a.norm_w ? K * 4u : 0u);
#pragma unroll
    for (int j = 0; j < GEMV_SQ; j++) {
      const uint32_t e = 2u * (threadIdx.x + j * bdim);
      const bool ok = e < K;
#pragma unroll
      for (int q = 0; q < 4; q++) sqv[j][q] = buf_ld8(xr, ok ? (q * a.xqs + e) * 4u : BUF_OOB);
      sgv[j] = buf_ld8(gr, ok ? e * 4u : BUF_OOB);
    }
  }
  uint4 xpre[NPRE];
  if (XPRE) {
    const char *x0 = (const char *)xrow(0);
#pragma unroll
    for (int j = 0; j < NPRE; j++) {
      // (a uniform skip of vectors past the row for every thread: K below
      // the staging's reach needs fewer loads)
      const uint32_t stride = a.norm == 0 ? bdim : nthr;
      if ((a.norm == 0 ? j >= XN : j >= NVN) || j * stride >= NVt) break;
      const uint32_t v = (a.norm == 0 ? threadIdx.x : tid) + j * stride;
      const uint32_t vc = v < NVt ? v : 0;
      xpre[j] = ld16(x0 + (uint64_t)vc * VE * XDr<XD>::B);
    }
  }
  // a fused norm's gain (and LayerNorm bias) vectors: loaded with the first
  // x loads, not after the reduction, so they cost no round trip of their
  // own (clamped indices; lanes past the row never use them)
  float gw[NVN][VE], gb[NVN][VE];
  auto load_gains = [&] {
    if (XSUM || a.norm == 0) return;
    const bool hw = a.norm_w != nullptr, hb = a.norm == 2 && a.norm_b != nullptr;
#pragma unroll
    for (int j = 0; j < NVN; j++) {
      const uint32_t v = tid + j * nthr, vc = v < NVt ? v : 0;
#pragma unroll
      for (int i = 0; i < VE; i += 4) {
        const float4 t = hw ? *(const float4 *)(a.norm_w + vc * VE + i) : make_float4(1.f, 1.f, 1.f, 1.f);
        gw[j][i] = t.x; gw[j][i + 1] = t.y; gw[j][i + 2] = t.z; gw[j][i + 3] = t.w;
        const float4 u = hb ? *(const float4 *)(a.norm_b + vc * VE + i) : make_float4(0.f, 0.f, 0.f, 0.f);
        gb[j][i] = u.x; gb[j][i + 1] = u.y; gb[j][i + 2] = u.z; gb[j][i + 3] = u.w;
      }
    }
  };
  if (XPRE) load_gains();
  // (in a persistent kernel, wave 0 polls the grid barrier inside wait():
  // its own loads are issued after the wait, so the poll does not queue
  // behind them)
  // phase clock (standalone kernel only): 0 entry, 1 first loads issued,
  // 2 x staged, 3 first weight batch consumed, 4 wave 0's rows done
  uint64_t *const clk = COH ? nullptr : a.clk;
  pclk(clk, a.clk_cap, 0);
  const bool early = !COH || (threadIdx.x >> 6) != 0;
  if (early) load_batch(g, 0);
  if (!wait()) return false;
  if (!early) load_batch(g, 0);
  if (!XPRE) load_gains();
  pclk(clk, a.clk_cap, 1);
  if (XPRE) pclk_after(clk, a.clk_cap, 6, xpre[0].x);

  // ---- 2. stage x into LDS (16-byte loads), with the fused norm if asked ----
  if constexpr (XSUM) {
    // x = bf16(g * ((q0 + q1) + (q2 + q3))) per element, two per 4-byte
    // store; pairs past K store into the spare word after the row (the host
    // sizes LDS for it), so no store -- and no load -- sits in a branch
#pragma unroll
    for (int j = 0; j < GEMV_SQ; j++) {
      const uint32_t e = 2u * (threadIdx.x + j * bdim);
      float v[2];
#pragma unroll
      for (int h = 0; h < 2; h++) {
        const float q0 = __uint_as_float(h ? sqv[j][0].y : sqv[j][0].x);
        const float q1 = __uint_as_float(h ? sqv[j][1].y : sqv[j][1].x);
        const float q2 = __uint_as_float(h ? sqv[j][2].y : sqv[j][2].x);
        const float q3 = __uint_as_float(h ? sqv[j][3].y : sqv[j][3].x);
        const float gn = a.norm_w ? __uint_as_float(h ? sgv[j].y : sgv[j].x) : 1.0f;
        v[h] = ((q0 + q1) + (q2 + q3)) * gn;
      }
      const uint32_t hi = e < K ? xs_index<XT, E>(K, C, 0, e) : K;
      *(uint32_t *)(xs_raw + (size_t)hi * 2u) = (uint32_t)f2bf(v[0]) | ((uint32_t)f2bf(v[1]) << 16);
    }
  } else
  for (int m = 0; m < M; m++) {
    const void *xr = xrow(m);
    const bool pre = XPRE && m == 0;     // row 0 already in xpre
    if (a.norm == 0) {
      // no reduction: every thread of the block stages, XN vectors of x in
      // flight per thread before the first LDS store
      for (uint32_t v0 = threadIdx.x; v0 < NVt; v0 += XN * bdim) {
        uint4 q[XN];
        const bool first = v0 == threadIdx.x;
#pragma unroll
        for (int j = 0; j < XN; j++) {
          const uint32_t v = v0 + j * bdim;
          if (v < NVt) q[j] = (pre && first) ? xpre[j] : xraw<XD, COH>(xr, (uint64_t)v * VE);
        }
#pragma unroll
        for (int j = 0; j < XN; j++) {
          const uint32_t v = v0 + j * bdim;
          if (v < NVt) xs_put_raw<XD, XT, E>(xs_raw, K, C, m, v, q[j]);
        }
      }
    } else {
      constexpr int NV = NVN;
      float xv[NV][VE];
#pragma unroll
      for (int j = 0; j < NV; j++) {
        const uint32_t v = tid + j * nthr;
        if (v < NVt) {
          if (pre) xdec<XD>(xpre[j], xv[j]);
          else xvec<XD, COH>(xr, (uint64_t)v * VE, xv[j]);
        } else {
#pragma unroll
          for (int i = 0; i < VE; i++) xv[j][i] = 0.0f;
        }
      }
      const float invK = 1.0f / (float)K;
      float mean = 0.0f, s1 = 0.0f, s2 = 0.0f;
      if (a.norm == 2) {
#pragma unroll
        for (int j = 0; j < NV; j++)
#pragma unroll
          for (int i = 0; i < VE; i++) s1 += xv[j][i];
        mean = block_sum_g(s1, red, nw) * invK;
      }
#pragma unroll
      for (int j = 0; j < NV; j++) {
        const bool vok = tid + j * nthr < NVt;
#pragma unroll
        for (int i = 0; i < VE; i++) {
          const float d = xv[j][i] - mean;
          s2 += vok ? d * d : 0.0f;
        }
      }
      const float inv = 1.0f / sqrtf(block_sum_g(s2, red, nw) * invK + a.norm_eps);
#pragma unroll
      for (int j = 0; j < NV; j++) {
        const uint32_t v = tid + j * nthr;
        if (v < NVt) {
          float val[VE];
#pragma unroll
          for (int i = 0; i < VE; i++) {
            // (x - mean) * inv * w (+ b), the norm kernel's own formula
            val[i] = (xv[j][i] - mean) * inv;
            if (a.norm_w) val[i] = val[i] * gw[j][i];
            if (a.norm == 2 && a.norm_b) val[i] = val[i] + gb[j][i];
          }
          xs_put_f<XD, XT, E>(xs_raw, K, C, m, v, val);
        }
      }
    }
  }
  __syncthreads();
  pclk(clk, a.clk_cap, 2);
  if (PRE) {   // the position is back (loaded first): the RoPE pair's loads
    // (the empty asm keeps the loaded length in a vector register and its
    // first use here: read as a uniform value, the compiler moved it to a
    // scalar register right after the load and waited for it before x)
    asm volatile("" : "+v"(pre_len));
    pre.pos = (int32_t)pre_len - 1;
    const uint32_t hd = a.head_dim ? a.head_dim : 2u, half = hd / 2;
    const bool rope = a.epi == THVM_EPI_QKV_ROPE && R == 2 && a.rope_cos && a.rope_sin;
    const uint32_t tab = rope ? a.max_seq * half * 4u : 0u;
    const buf_t rcs = buf_rsrc(a.rope_cos, tab), rsn = buf_rsrc(a.rope_sin, tab);
    const uint32_t d = pre_n0 % hd;
#pragma unroll
    for (int m = 0; m < M; m++) {
      const int32_t pm = pre.pos + (a.spec ? m : 0);
      const uint32_t pmc = pm >= 0 && (uint32_t)pm < a.max_seq ? (uint32_t)pm : 0u;
      const uint32_t off = (pmc * half + d / 2) * 4u;
      pre.cs[m] = __uint_as_float(buf_ld4(rcs, off));
      pre.sn[m] = __uint_as_float(buf_ld4(rsn, off));
    }
  }

  // ---- 3. stream the weight rows ----
  // A flat sequence of (row group, chunk batch) steps per wave; two register
  // sets ping-pong so the next batch is in flight while one is consumed (the
  // wait before a consume covers only the older batch's loads).
  const uint32_t NB = (C + 64 * U - 1) / (64 * U);      // batches per row group
  const uint32_t g0 = g;
  const uint32_t ngw = g0 < G ? (G - 1 - g0) / gstride + 1 : 0;
  const uint32_t T = ngw * NB;
  float acc[R][M];
#pragma unroll
  for (int r = 0; r < R; r++)
#pragma unroll
    for (int m = 0; m < M; m++) acc[r][m] = 0.0f;

  auto consume = [&](const uint4 (&X)[R][U], uint32_t t) {
    const uint32_t gi = t / NB, bi = t - gi * NB;
    const uint32_t c0 = bi * 64 * U;
#pragma unroll
    for (int u = 0; u < U; u++) {
      const uint32_t c = c0 + u * 64 + lane;
      if (c < C) {
        if (XT == XT_F32) {
#pragma unroll
          for (int j = 0; j < E / 4; j++) {
            float4 xv[M];
#pragma unroll
            for (int m = 0; m < M; m++)
              xv[m] = *(const float4 *)((const float *)xs_raw + m * K + (j * C + c) * 4);
#pragma unroll
            for (int r = 0; r < R; r++) {
              float wf[4];
              quad_decode<WT>(X[r][u], j, wf);
#pragma unroll
              for (int m = 0; m < M; m++) {
                acc[r][m] += xv[m].x * wf[0];
                acc[r][m] += xv[m].y * wf[1];
                acc[r][m] += xv[m].z * wf[2];
                acc[r][m] += xv[m].w * wf[3];
              }
            }
          }
        } else if (Dot2<WT, XT>::ok) {
#pragma unroll
          for (int h = 0; h < (E + 7) / 8; h++) {     // 8-element x groups: 4 pairs
            uint4 xq[M];
#pragma unroll
            for (int m = 0; m < M; m++)
              xq[m] = *(const uint4 *)((const uint16_t *)xs_raw + m * K + (h * C + c) * 8);
#pragma unroll
            for (int jj = 0; jj < 2 && (h * 2 + jj) < E / 4; jj++) {
              const int j = h * 2 + jj;
#pragma unroll
              for (int r = 0; r < R; r++) {
                uint32_t w0, w1;
                quad_pairs<WT, XT>(X[r][u], j, w0, w1);
#pragma unroll
                for (int m = 0; m < M; m++) {
                  acc[r][m] = dot2acc<XT>(jj ? xq[m].z : xq[m].x, w0, acc[r][m]);
                  acc[r][m] = dot2acc<XT>(jj ? xq[m].w : xq[m].y, w1, acc[r][m]);
                }
              }
            }
          }
        } else {
#pragma unroll
          for (int h = 0; h < (E + 7) / 8; h++) {     // 8-element x groups
            float xf[M][8];
#pragma unroll
            for (int m = 0; m < M; m++) {
              uint4 q = *(const uint4 *)((const uint16_t *)xs_raw + m * K + (h * C + c) * 8);
              x8_decode<XT>(q, xf[m]);
            }
#pragma unroll
            for (int jj = 0; jj < 2 && (h * 2 + jj) < E / 4; jj++) {
              const int j = h * 2 + jj;
#pragma unroll
              for (int r = 0; r < R; r++) {
                float wf[4];
                quad_decode<WT>(X[r][u], j, wf);
#pragma unroll
                for (int m = 0; m < M; m++) {
                  acc[r][m] += xf[m][jj * 4 + 0] * wf[0];
                  acc[r][m] += xf[m][jj * 4 + 1] * wf[1];
                  acc[r][m] += xf[m][jj * 4 + 2] * wf[2];
                  acc[r][m] += xf[m][jj * 4 + 3] * wf[3];
                }
              }
            }
          }
        }
      }
    }
    if (bi == NB - 1) {
      float tot[R][M];
#pragma unroll
      for (int r = 0; r < R; r++)
#pragma unroll
        for (int m = 0; m < M; m++) {
          tot[r][m] = wave_sum(acc[r][m]);
          acc[r][m] = 0.0f;
        }
      if (lane == 0) {
        const uint32_t n0 = (g0 + gi * gstride) * R;
        gemv_epilogue<R, M, COH>(a, n0, tot, 0, PRE && gi == 0 ? &pre : nullptr);
        hook(n0, tot);
      }
    }
  };
  auto load_step = [&](uint4 (&X)[R][U], uint32_t t) {
    const uint32_t gi = t / NB, bi = t - gi * NB;
    wload(X, g0 + gi * gstride, bi * 64 * U);
  };
  uint4 wq2[R][U];
  for (uint32_t t = 0; t < T; t += 2) {          // step 0 is already in wq
    if (t + 1 < T) load_step(wq2, t + 1);
    consume(wq, t);
    if (t == 0) pclk(clk, a.clk_cap, 3);
    if (t + 1 >= T) break;
    if (t + 2 < T) load_step(wq, t + 2);
    consume(wq2, t + 1);
  }
  pclk(clk, a.clk_cap, 4);
  return true;
}
