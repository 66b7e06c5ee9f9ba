// dev_common.h -- gfx950 device helpers shared by the hand-written decode
// kernels: narrow-float codecs, wave64 DPP reductions, 128-bit loads.
//
// Numerics follow the reference codecs bit for bit:
//   bf16 <-> f32  reference src/dtype/fp_convert.c:113-136 (RNE, NaN -> quiet
//                 NaN keeping the sign);
//   fp16 <-> f32  IEEE RNE (reference src/dtype/fp_convert.c:26-110; the
//                 gfx950 v_cvt_f16_f32 / v_cvt_f32_f16 pair is IEEE RNE);
//   e4m3  -> f32  exact decode (reference src/dtype/fp8.c:149-175), done by the
//                 gfx950 OCP-fp8 converter v_cvt_pk_f32_fp8;
//   f32 -> e4m3   saturating RNE encode with subnormals (reference
//                 src/dtype/fp8.c:60-133, the _sat kernel-store form).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef uint16_t bf16_t;
typedef uint16_t f16_t;

#define THVM_WAVE 64

// ---- bf16 ------------------------------------------------------------------
__device__ __forceinline__ float bf2f(bf16_t h) {
  return __uint_as_float(((uint32_t)h) << 16);
}
// f32 -> bf16, round to nearest even; a NaN becomes the quiet NaN of its
// sign.  Written as a select: the early-return form compiled to two exec-mask
// branches per conversion.
__device__ __forceinline__ bf16_t f2bf(float f) {
  const uint32_t b = __float_as_uint(f);
  const uint32_t r = (b + 0x7fffu + ((b >> 16) & 1u)) >> 16;
  const uint32_t q = ((b >> 16) & 0x8000u) | 0x7fc0u;
  return (bf16_t)((b & 0x7fffffffu) > 0x7f800000u ? q : r);
}
// round a float through bf16 storage
__device__ __forceinline__ float rbf(float f) { return bf2f(f2bf(f)); }
// two f32 -> a packed bf16 pair, round to nearest even (f2bf's rounding for
// every non-NaN input), in one v_cvt_pk_bf16_f32; element 0 in the low half
typedef float f32x2_cvt_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_cvt_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pk_bf16(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_cvt_t){a, b}, bf16x2_cvt_t));
}

// ---- fp16 ------------------------------------------------------------------
__device__ __forceinline__ float h2f(f16_t h) {
  _Float16 v = __builtin_bit_cast(_Float16, h);
  return (float)v;
}
__device__ __forceinline__ f16_t f2h(float f) {
  _Float16 v = (_Float16)f;
  return __builtin_bit_cast(f16_t, v);
}
__device__ __forceinline__ float rh(float f) { return h2f(f2h(f)); }

// ---- fp8 e4m3 (OCP e4m3fn, the gfx950 fp8 format) --------------------------
// Four packed bytes -> four floats.  Exact for every finite pattern; 0x7F /
// 0xFF decode to NaN, as the reference does (fp8.c:156-158).
__device__ __forceinline__ void fp8x4_to_f32(uint32_t w, float o[4]) {
  auto lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, false);
  auto hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, true);
  o[0] = lo[0]; o[1] = lo[1]; o[2] = hi[0]; o[3] = hi[1];
}
__device__ __forceinline__ float fp82f(uint8_t b) {
  auto lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)b, false);
  return lo[0];
}

// Saturating e4m3 encode, written from the OCP definition: round to nearest
// even on the f32 significand, finite overflow and +-inf to +-448 (0x7E/0xFE),
// NaN to sign|0x7F, subnormals kept (min subnormal 2^-9).
__device__ __forceinline__ uint8_t f2fp8_sat(float x) {
  uint32_t u = __float_as_uint(x);
  uint32_t sign = (u >> 24) & 0x80u;
  uint32_t a = u & 0x7fffffffu;
  if (a > 0x7f800000u) return (uint8_t)(sign | 0x7Fu);     // NaN
  if (a >= 0x43E00000u) {                                   // >= 448 (incl inf)
    // values in [448, 464) round to 448, >= 464 overflow: both saturate
    return (uint8_t)(sign | 0x7Eu);
  }
  int e = (int)(a >> 23) - 127;                             // unbiased exp
  if (e < -6) {
    // subnormal range: value = m * 2^-9, m in [0, 8]
    // q = round_even(|x| * 2^9)
    float s = __uint_as_float(a) * 512.0f;                  // exact (power of 2)
    // round half to even on a float known < 8
    float r = __builtin_rintf(s);                           // RNE (default mode)
    uint32_t m = (uint32_t)r;                               // 0..8
    // m == 8 is the smallest normal 2^-6 = exp field 1, mantissa 0
    return (uint8_t)(sign | m);
  }
  // normal: keep 3 mantissa bits, RNE on the dropped 20 bits
  uint32_t mant = a & 0x7fffffu;
  uint32_t q = ((uint32_t)(e + 7) << 3) | (mant >> 20);
  uint32_t rem = mant & 0xfffffu;
  if (rem > 0x80000u || (rem == 0x80000u && (q & 1u))) q += 1;
  if (q > 0x7Eu) q = 0x7Eu;                                 // 464 boundary
  return (uint8_t)(sign | q);
}

// ---- wave64 DPP reductions --------------------------------------------------
// Sum / max over all 64 lanes.  The DPP sequence fixes the association order,
// so the result is deterministic run to run: quad pairs, quads, half-row
// mirror, row mirror, then row_bcast:15 and row_bcast:31 carry the partial
// row sums up to lane 63, whose value is broadcast.
template <int CTRL, int ROWMASK = 0xf>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL,
                                                    ROWMASK, 0xf, true));
}
template <int CTRL, int ROWMASK = 0xf>
__device__ __forceinline__ float dpp_f_old(float old, float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(old),
                                                    __float_as_int(v), CTRL,
                                                    ROWMASK, 0xf, false));
}

// sum within each row of 16 lanes; every lane of the row holds the row sum
__device__ __forceinline__ float row16_sum(float v) {
  v += dpp_f<0xB1>(v);    // quad_perm [1,0,3,2]
  v += dpp_f<0x4E>(v);    // quad_perm [2,3,0,1]
  v += dpp_f<0x141>(v);   // row_half_mirror
  v += dpp_f<0x140>(v);   // row_mirror
  return v;
}
__device__ __forceinline__ float row16_max(float v) {
  v = fmaxf(v, dpp_f<0xB1>(v));
  v = fmaxf(v, dpp_f<0x4E>(v));
  v = fmaxf(v, dpp_f<0x141>(v));
  v = fmaxf(v, dpp_f<0x140>(v));
  return v;
}

__device__ __forceinline__ float wave_sum(float v) {
  v = row16_sum(v);
  v += dpp_f<0x142, 0xa>(v);   // row_bcast:15 into rows 1 and 3
  v += dpp_f<0x143, 0xc>(v);   // row_bcast:31 into rows 2 and 3
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}
__device__ __forceinline__ float wave_max(float v) {
  v = row16_max(v);
  // rows 0/2 keep their own value (old = v) so the max stays correct
  v = fmaxf(v, dpp_f_old<0x142, 0xa>(v, v));
  v = fmaxf(v, dpp_f_old<0x143, 0xc>(v, v));
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// lanes l, l^16, l^32, l^48 combined (the 4 rows of a wave), all lanes
__device__ __forceinline__ float xrow_sum(float v) {
  v += __shfl_xor(v, 16);
  v += __shfl_xor(v, 32);
  return v;
}
__device__ __forceinline__ float xrow_max(float v) {
  v = fmaxf(v, __shfl_xor(v, 16));
  v = fmaxf(v, __shfl_xor(v, 32));
  return v;
}

__device__ __forceinline__ int lane_id() { return (int)(threadIdx.x & 63u); }

// 128-bit global load of streamed (read-once) data
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 ld_stream16(const void *p) {
  u32x4_t v = __builtin_nontemporal_load((const u32x4_t *)p);
  return make_uint4(v[0], v[1], v[2], v[3]);
}
__device__ __forceinline__ uint4 ld16(const void *p) {
  return *(const uint4 *)p;
}

// Raw buffer loads through a buffer resource over [p, p + bytes) (stride 0,
// the gfx9 untyped-access word): an offset at or beyond `bytes` reads zero by
// the hardware range check, so masked loads need neither branches nor selects
// (a guarded load lets the compiler sink it into a branch and wait for it
// there).  BUF_OOB is an offset that is always out of range.
#define BUF_OOB 0x80000000u
typedef __amdgpu_buffer_rsrc_t buf_t;
__device__ __forceinline__ buf_t buf_rsrc(const void *p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc((void *)p, 0, (int)bytes, 0x00020000);
}
// the same over a base and range that are wave-uniform but held in VGPRs:
// their first lane's values (readfirstlane keeps the resource in SGPRs, where
// a per-lane resource compiles to a waterfall loop around every load)
__device__ __forceinline__ buf_t buf_rsrc_u(const void *p, uint32_t bytes) {
  const uint64_t v = (uint64_t)(uintptr_t)p;
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return buf_rsrc((const void *)(uintptr_t)(((uint64_t)hi << 32) | lo), __builtin_amdgcn_readfirstlane(bytes));
}
__device__ __forceinline__ uint4 buf_ld16(buf_t r, uint32_t off) {
  u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
  return make_uint4(v[0], v[1], v[2], v[3]);
}
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint2 buf_ld8(buf_t r, uint32_t off) {
  u32x2_t v = __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0);
  return make_uint2(v[0], v[1]);
}
__device__ __forceinline__ uint32_t buf_ld4(buf_t r, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0);
}
__device__ __forceinline__ uint32_t buf_ld2(buf_t r, uint32_t off) {
  return (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0);
}
__device__ __forceinline__ uint4 buf_ld_stream16(buf_t r, uint32_t off) {   // nontemporal
  u32x4_t v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 2);
  return make_uint4(v[0], v[1], v[2], v[3]);
}

// LDS slot of element k of a vector that lanes read in 16-byte weight chunks
// of EPC elements (chunk ch = k / EPC belongs to one lane, consecutive chunks
// to consecutive lanes): quad q of every chunk is stored contiguously across
// chunks, so one lane's float4 read of quad q and its neighbours' reads fall on
// consecutive 16-byte LDS words (no bank conflicts).  nch = chunks in the vector.
template <int EPC>
__device__ __forceinline__ uint32_t chunk_swz(uint32_t k, uint32_t nch) {
  return (((k % EPC) >> 2) * nch + k / EPC) * 4 + (k & 3);
}

__device__ __forceinline__ float silu_f(float g) { return g / (1.0f + expf(-g)); }
__device__ __forceinline__ float gelu_tanh_f(float x) {
  // tinygrad Tensor.gelu: 0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3)))
  float u = 0.7978845608f * (x + 0.044715f * x * x * x);
  return 0.5f * x * (1.0f + tanhf(u));
}

// v of lane (lane ^ 16) / (lane ^ 32) with gfx950's v_permlane16_swap /
// v_permlane32_swap (VALU: no LDS round trip as a ds_bpermute shuffle takes).
// permlane32_swap(a, b) swaps lanes 32..63 of a with lanes 0..31 of b, so with
// a = b = v the new a holds v[lane - 32] in its upper half and the new b
// v[lane + 32] in its lower half; permlane16_swap does the same between the
// odd 16-lane rows of a and the even rows of b.
__device__ __forceinline__ float xor32_f(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float((threadIdx.x & 32u) ? r[0] : r[1]);
}
__device__ __forceinline__ float xor16_f(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float((threadIdx.x & 16u) ? r[0] : r[1]);
}

// ---- phase clock (measurement build only) -----------------------------------
// Compiled in only with -DTHVM_PCLK (the library variant libthvm_hip_pclk.so,
// `python -m thvm_amd.build --variant pclk`): the marks constrain the
// compiler's scheduling and cost ~2% of a decode step even when off, so the
// product library has none.  There, with clk set (a kernel argument, so the
// test is uniform), thread 0 of each of the first cap blocks stores the 100
// MHz wall clock (s_memrealtime) at mark i (0..7) of its PCLK_MARKS slots;
// mark 0 also records the block's XCD (slot 8, HW_REG_XCC_ID) and hardware
// id word (slot 9, HW_REG_HW_ID: SE, CU, SIMD), so launch order across the
// XCDs shows.  pclk_end first drains the block's memory operations and waits
// for every wave.
#define PCLK_MARKS 10
__device__ __forceinline__ void pclk(uint64_t *clk, uint32_t cap, int i) {
#ifndef THVM_PCLK
  (void)clk; (void)cap; (void)i;
  return;
#endif
  if (clk == nullptr || threadIdx.x != 0) return;
  const uint32_t blk = blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z);
  if (blk >= cap) return;
  uint64_t *p = clk + (uint64_t)blk * PCLK_MARKS;
  p[i] = __builtin_amdgcn_s_memrealtime();
  if (i == 0) {
    uint32_t xcc, hw;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_HW_ID)" : "=s"(hw));
    p[8] = xcc;
    p[9] = hw;
  }
}
// mark i once thread 0 holds v (the empty asm needs v in a register, so the
// wait for its load comes first)
__device__ __forceinline__ void pclk_after(uint64_t *clk, uint32_t cap, int i, uint32_t v) {
#ifndef THVM_PCLK
  (void)clk; (void)cap; (void)i; (void)v;
  return;
#endif
  if (clk == nullptr || threadIdx.x != 0) return;
  asm volatile("" ::"v"(v));
  pclk(clk, cap, i);
}
__device__ __forceinline__ void pclk_end(uint64_t *clk, uint32_t cap) {
#ifndef THVM_PCLK
  (void)clk; (void)cap;
  return;
#endif
  if (clk == nullptr) return;
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  pclk(clk, cap, 7);
}
