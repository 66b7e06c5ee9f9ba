// mla.hip -- DeepSeek-V2 multi-head latent attention for decode on gfx950:
// the absorbed form over a shared latent cache (one ckv row of kv_lora
// values and one roped k-pe row per position, read by every query head).
//
// Replaces the reference's MLA kernels (bench/dsv2_decode_bench.c gred_q
// :435-485, kv_prep :487-556, mla_qlat :638-667, mla_score :669-723, mla_mix
// :725-750, mla_o :752-785): five single-purpose launches and a materialised
// [H, max_seq] score matrix become three kernels:
//   k_mla_prep   q pe rotation, latent-row RMSNorm + k pe rotation + cache
//                append at L-1, and qlat = q_nope . W_uk (fp8/bf16 rows, per
//                row scale) -- one launch, blocks split between the jobs;
//   k_mla_split  split-sequence flash decode: a block owns 64 cache rows of
//                one batch row and a group of 4 heads, stages the rows in LDS
//                once, scores the group against them (lanes split the latent
//                dimension, DPP wave sums), and writes per-split (olat
//                partial, max, sum); the head groups of a split re-read its
//                rows from L2, so HBM sees each latent row once per step;
//   k_mla_out    merges the live splits per (row, head) in fixed order and
//                applies the absorbed V up-projection W_uv, rounding o to
//                bf16.
// The live length L is read from device memory, so one captured graph
// serves every position.
#include "dev_common.h"
#include "../kern_api.h"
#include "launch.h"
#include "mfma_ops.h"
#include <stdio.h>

#define MLA_CHUNK 64
#define MLA_THREADS 512

__device__ __forceinline__ float bfv(const void *p, uint64_t i) {
  return bf2f(((const bf16_t *)p)[i]);
}

// 16 weights of one row chunk (fp8 or bf16 storage) as f32
template <bool FP8>
__device__ __forceinline__ void w16(const uint4 &q0, const uint4 &q1, float o[16]) {
  if (FP8) {
    const uint32_t w[4] = {q0.x, q0.y, q0.z, q0.w};
#pragma unroll
    for (int i = 0; i < 4; i++) fp8x4_to_f32(w[i], o + 4 * i);
  } else {
    const uint32_t w[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
#pragma unroll
    for (int i = 0; i < 8; i++) {
      o[2 * i] = __uint_as_float(w[i] << 16);
      o[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
  }
}

// sum over aligned groups of G lanes (G a power of two <= 64); every lane of
// a group gets the sum.  DPP within a row of 16 lanes (quad pairs, quads,
// half-row mirror, row mirror), then the permlane swaps across rows: VALU
// operations with no LDS round trip, where a __shfl_xor butterfly compiles to
// dependent ds_bpermute waits.
__device__ __forceinline__ float group_sum(float v, int G) {
  if (G >= 2) v += dpp_f<0xB1>(v);     // quad_perm [1,0,3,2]
  if (G >= 4) v += dpp_f<0x4E>(v);     // quad_perm [2,3,0,1]
  if (G >= 8) v += dpp_f<0x141>(v);    // row_half_mirror
  if (G >= 16) v += dpp_f<0x140>(v);   // row_mirror
  if (G >= 32) v += xor16_f(v);
  if (G >= 64) v += xor32_f(v);
  return v;
}

// ---- k_mla_prep ---------------------------------------------------------
// blocks [0, H*QB*BG): qlat rows (h, 64 latent rows each) for a group of
// MLA_PREP_ROWS batch rows (BG groups); blocks [H*QB*BG, H*QB*BG + B): batch
// row b's q pe rotation, latent norm and cache append.  256 threads.  (One
// block per (h, 64 rows) over all 32 rows of C5 batch 32 left 160 blocks,
// each a 32-step serial loop: 33.7 us; groups of 8 rows give 512 blocks.)
#define MLA_PREP_ROWS 8
#define MLA_PREP_PASS 4    /* W_uk row passes requested at once */
template <bool FP8>
__global__ __launch_bounds__(256) void k_mla_prep(ThvmMlaArgs a) {
  extern __shared__ float sm[];
  const uint32_t H = a.H, dn = a.dn, dr = a.dr, kv = a.kv, half = dr / 2, qs = dn + dr;
  const uint32_t qoff = H * qs, QB = kv / 64, BG = (a.B + MLA_PREP_ROWS - 1) / MLA_PREP_ROWS;
  const int32_t pos = a.len[0] - 1;
  // phase clock: 0 entry, 1 q nope staged (absorption blocks) or latent row
  // read (the append block), 7 drained
  pclk(a.clk, a.clk_cap, 0);
  if (blockIdx.x < H * QB * BG) {
    const uint32_t h = blockIdx.x / (QB * BG), rem = blockIdx.x % (QB * BG);
    const uint32_t k0 = (rem / BG) * 64, b0 = (rem % BG) * MLA_PREP_ROWS;
    const uint32_t nb = min(a.B - b0, (uint32_t)MLA_PREP_ROWS);
    const uint32_t rowb = dn * (FP8 ? 1 : 2), LPR = rowb / 16;     // lanes per row
    const uint32_t lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const uint32_t rpp = 64 / LPR;                                 // rows per wave pass
    const uint32_t sub = lane / LPR, c = lane % LPR;
    const uint32_t npass = (64 + 4 * rpp - 1) / (4 * rpp);
    // head h's W_uk rows and scales through buffer resources (rows past kv
    // read zero): MLA_PREP_PASS passes' rows are requested before q nope is
    // staged, so the block waits one round trip for both instead of one per
    // pass
    const buf_t wr = buf_rsrc((const char *)a.wuk + (uint64_t)h * kv * rowb, kv * rowb);
    const buf_t sr = buf_rsrc(a.suk ? a.suk + (uint64_t)h * kv : nullptr, a.suk ? kv * 4u : 0u);
    for (uint32_t pg = 0; pg < npass; pg += MLA_PREP_PASS) {
      uint4 wq[MLA_PREP_PASS];
      uint32_t sq[MLA_PREP_PASS];
#pragma unroll
      for (int p = 0; p < MLA_PREP_PASS; p++) {
        const uint32_t r = wv * rpp + (pg + p) * 4 * rpp + sub, k = k0 + r;
        const bool ok = pg + p < npass && r < 64 && k < kv;
        wq[p] = buf_ld_stream16(wr, ok ? k * rowb + c * 16u : BUF_OOB);
        sq[p] = buf_ld4(sr, ok ? k * 4u : BUF_OOB);
      }
      if (pg == 0) {
        // q nope of the group's batch rows into LDS (f32)
        for (uint32_t i = threadIdx.x; i < nb * dn; i += blockDim.x) {
          const uint32_t b = i / dn, d = i % dn;
          sm[i] = bfv(a.qkv, (uint64_t)(b0 + b) * a.ldq + h * qs + d);
        }
        __syncthreads();
        pclk(a.clk, a.clk_cap, 1);
      }
#pragma unroll
      for (int p = 0; p < MLA_PREP_PASS; p++) {
        const uint32_t r = wv * rpp + (pg + p) * 4 * rpp + sub, k = k0 + r;
        if (pg + p >= npass) break;                              // block-uniform
        const bool ok = r < 64 && k < kv;
        float w[16];
        w16<FP8>(wq[p], make_uint4(0, 0, 0, 0), w);
        const uint32_t e0 = c * (FP8 ? 16 : 8), ne = FP8 ? 16 : 8;
        const float s = a.suk ? __uint_as_float(sq[p]) : 1.0f;
        for (uint32_t b = 0; b < nb; b++) {
          float acc = 0.0f;
          for (uint32_t i = 0; i < ne; i++) acc += sm[b * dn + e0 + i] * w[i];
          acc = group_sum(acc, (int)LPR);
          if (ok && c == 0) a.qlat[((uint64_t)(b0 + b) * H + h) * kv + k] = acc * s;
        }
      }
    }
    pclk_end(a.clk, a.clk_cap);
    return;
  }
  const uint32_t b = blockIdx.x - H * QB * BG;
  if (b >= a.B || pos < 0 || (uint32_t)pos >= a.max_seq) return;
  const uint64_t qb = (uint64_t)b * a.ldq;
  // q pe pairs (2j, 2j+1) -> halves j and half+j, after rounding through bf16
  for (uint32_t i = threadIdx.x; i < H * half; i += blockDim.x) {
    const uint32_t h = i / half, j = i % half, base = h * qs + dn;
    const float xe = bfv(a.qkv, qb + base + 2 * j), xo = bfv(a.qkv, qb + base + 2 * j + 1);
    const float c = a.rope_cos[(uint64_t)pos * half + j], sn = a.rope_sin[(uint64_t)pos * half + j];
    bf16_t *q = (bf16_t *)a.qpe + ((uint64_t)b * H + h) * dr;
    q[j] = f2bf(xe * c - xo * sn);
    q[half + j] = f2bf(xo * c + xe * sn);
  }
  // latent row: RMSNorm over kv values, gain wkvn, append at pos
  float ss = 0.0f;
  for (uint32_t t = threadIdx.x; t < kv; t += blockDim.x) {
    const float v = bfv(a.qkv, qb + qoff + t);
    sm[t] = v;
    ss += v * v;
  }
  ss = wave_sum(ss);
  float *red = sm + kv;
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
  __syncthreads();
  pclk(a.clk, a.clk_cap, 1);
  float tot = 0.0f;
  for (uint32_t w = 0; w < blockDim.x / 64; w++) tot += red[w];
  const float inv = 1.0f / sqrtf(tot * (1.0f / (float)kv) + a.eps);
  bf16_t *crow = (bf16_t *)a.ckv + ((uint64_t)b * a.max_seq + (uint32_t)pos) * kv;
  for (uint32_t t = threadIdx.x; t < kv; t += blockDim.x) crow[t] = f2bf((sm[t] * inv) * a.wkvn[t]);
  bf16_t *prow = (bf16_t *)a.kpe + ((uint64_t)b * a.max_seq + (uint32_t)pos) * dr;
  for (uint32_t j = threadIdx.x; j < half; j += blockDim.x) {
    const float xe = bfv(a.qkv, qb + qoff + kv + 2 * j), xo = bfv(a.qkv, qb + qoff + kv + 2 * j + 1);
    const float c = a.rope_cos[(uint64_t)pos * half + j], sn = a.rope_sin[(uint64_t)pos * half + j];
    prow[j] = f2bf(xe * c - xo * sn);
    prow[half + j] = f2bf(xo * c + xe * sn);
  }
  pclk_end(a.clk, a.clk_cap);
}

// ---- k_mla_split --------------------------------------------------------
// grid (n_split, H / MLA_HG, B), 512 threads: 64 cache rows of batch row b
// against a group of MLA_HG heads (the latent rows of a split are re-read by
// the H / MLA_HG head groups from L2, which buys 4x the blocks).  KPL latent
// values per lane (kv = 64 * KPL).
#define MLA_HG 4
template <int KPL>
__global__ __launch_bounds__(MLA_THREADS) void k_mla_split(ThvmMlaArgs a) {
  extern __shared__ float smem[];
  constexpr uint32_t KV = 64 * KPL;
  constexpr int HG = MLA_HG;
  bf16_t *cs = (bf16_t *)smem;                          // [64][KV]
  float *sp = smem + (MLA_CHUNK * KV) / 2;              // [64][HG]: scores, then weights
  const uint32_t split = blockIdx.x, h0 = blockIdx.y * HG, b = blockIdx.z, dr = a.dr, H = a.H;
  const int32_t L = min(a.len[0], (int32_t)a.max_seq);   // rows [0, L) are live
  const uint32_t j0 = split * MLA_CHUNK;
  if (L <= 0 || j0 >= (uint32_t)L) return;
  const uint32_t nj = min((uint32_t)L - j0, (uint32_t)MLA_CHUNK);
  const uint32_t lane = threadIdx.x & 63, wv = threadIdx.x >> 6;

  // issue the cache-row loads first: wave wv takes rows wv, wv+8, ...  The
  // loads are unconditional from clamped, always-live addresses (row j0 and
  // lane 0 exist) and masked afterwards: a guarded load whose value is used
  // inside its branch makes the compiler drain every outstanding load there.
  constexpr int RPW = MLA_CHUNK / 8;
  uint32_t cw[RPW][(KPL + 1) / 2];
  bf16_t pr[RPW];
  const bf16_t *cb = (const bf16_t *)a.ckv + ((uint64_t)b * a.max_seq + j0) * KV;
  const bf16_t *pb = (const bf16_t *)a.kpe + ((uint64_t)b * a.max_seq + j0) * dr;
  const uint32_t pl_lane = lane < dr ? lane : 0;
#pragma unroll
  for (int r = 0; r < RPW; r++) {
    const uint32_t j = wv + 8 * r;
    const uint32_t jc = j < nj ? j : 0;
    const bf16_t *row = cb + (uint64_t)jc * KV + lane * KPL;
    if (KPL == 8) {
      uint4 v = ld_stream16(row);
      cw[r][0] = v.x; cw[r][1] = v.y; cw[r][2] = v.z; cw[r][3] = v.w;
    } else if (KPL == 4) {
      uint2 v = *(const uint2 *)row;
      cw[r][0] = v.x; cw[r][1] = v.y;
    } else if (KPL == 2) {
      cw[r][0] = *(const uint32_t *)row;
    } else {
      cw[r][0] = (uint32_t)row[0];
    }
    pr[r] = pb[(uint64_t)jc * dr + pl_lane];
  }
  float pv[RPW];
#pragma unroll
  for (int r = 0; r < RPW; r++) pv[r] = (wv + 8 * r < nj && lane < dr) ? bf2f(pr[r]) : 0.0f;
  // this lane's slice of the group's qlat and q pe
  float ql[HG][KPL], qp[HG];
  bf16_t qr[HG];
#pragma unroll
  for (int h = 0; h < HG; h++) {
    const float *src = a.qlat + ((uint64_t)b * H + h0 + h) * KV + lane * KPL;
#pragma unroll
    for (int i = 0; i < KPL; i++) ql[h][i] = src[i];
    qr[h] = ((const bf16_t *)a.qpe)[((uint64_t)b * H + h0 + h) * dr + pl_lane];
  }
#pragma unroll
  for (int h = 0; h < HG; h++) qp[h] = lane < dr ? bf2f(qr[h]) : 0.0f;
#pragma unroll
  for (int r = 0; r < RPW; r++) {
    const uint32_t j = wv + 8 * r;
    if (j >= nj) break;                                  // wave-uniform
    float c[KPL];
    if (KPL == 1) {
      c[0] = __uint_as_float(cw[r][0] << 16);
      cs[j * KV + lane] = (bf16_t)cw[r][0];
    } else {
#pragma unroll
      for (int i = 0; i < KPL / 2; i++) {
        c[2 * i] = __uint_as_float(cw[r][i] << 16);
        c[2 * i + 1] = __uint_as_float(cw[r][i] & 0xffff0000u);
      }
      uint32_t *dst = (uint32_t *)(cs + j * KV + lane * KPL);
#pragma unroll
      for (int i = 0; i < KPL / 2; i++) dst[i] = cw[r][i];
    }
#pragma unroll
    for (int h = 0; h < HG; h++) {
      float s = qp[h] * pv[r];
#pragma unroll
      for (int i = 0; i < KPL; i++) s += ql[h][i] * c[i];
      s = wave_sum(s);
      if (lane == 0) sp[j * HG + h] = s * a.scale;
    }
  }
  __syncthreads();
  // per-head softmax partial over this block's rows (wave h, lane = row)
  float *part = a.part + ((uint64_t)b * a.n_split + split) * H * (KV + 4);
  if (wv < HG) {
    const uint32_t h = wv;
    const float s = lane < nj ? sp[lane * HG + h] : -INFINITY;
    const float m = wave_max(s);
    const float e = lane < nj ? expf(s - m) : 0.0f;
    const float l = wave_sum(e);
    sp[lane * HG + h] = e;
    if (lane == 0) {
      part[(h0 + h) * (KV + 4) + KV] = m;
      part[(h0 + h) * (KV + 4) + KV + 1] = l;
    }
  }
  __syncthreads();
  // olat partial: thread t owns latent column t for the group's heads; lane j
  // holds row j's HG softmax weights and v_readlane broadcasts them (a
  // wave-wide LDS read of one address would serialise on its banks)
  const uint32_t t = threadIdx.x;
  if (t < KV) {                                        // whole waves: KV is a multiple of 64
    float acc[HG];
#pragma unroll
    for (int h = 0; h < HG; h++) acc[h] = 0.0f;
    const float4 pl = ((const float4 *)sp)[lane];      // HG == 4 weights of row `lane`
    for (uint32_t j0r = 0; j0r < nj; j0r += 8) {     // eight rows of LDS reads in flight
      float c[8];
#pragma unroll
      for (int u = 0; u < 8; u++) {
        const uint32_t j = j0r + u;
        c[u] = j < nj ? bf2f(cs[j * KV + t]) : 0.0f;
      }
#pragma unroll
      for (int u = 0; u < 8; u++) {
        const int j = (int)(j0r + u);                  // rows past nj carry weight 0
        acc[0] += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(pl.x), j)) * c[u];
        acc[1] += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(pl.y), j)) * c[u];
        acc[2] += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(pl.z), j)) * c[u];
        acc[3] += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(pl.w), j)) * c[u];
      }
    }
#pragma unroll
    for (int h = 0; h < HG; h++) part[(h0 + h) * (KV + 4) + t] = acc[h];
  }
}

// ---- k_mla_split_mf -----------------------------------------------------
// The split on MFMA for the DeepSeek-V2 attention shape (16 heads, kv_lora
// 512, rope 64): the 16 heads are the M side of v_mfma_f32_16x16x32_bf16.
// A chunk's 64 cache rows (1152 bytes each: the latent row, then the pe row)
// are loaded as contiguous 16-byte pieces -- thread t takes pieces t, t +
// 512, ... of the chunk's 64 x 72 -- and staged row-major in LDS (pitch
// MF_RP).  (Loading each lane's MFMA operand straight from HBM touched 16
// rows per load instruction: a block's rows landed after ~2.9 us, against
// ~1.5 us for contiguous pieces, measured on gfx950.)
//   scores  S[h][row] = qlat[h] . c_row + qpe[h] . pe_row over k = 576 (18
//           steps of 32): A = q (16 heads x 32 k), B = the staged rows (32 k
//           x 16 rows: a lane's 8 consecutive values of one row, one 16-byte
//           LDS read), two waves per 16-row tile (k-steps 0..8 and 9..17,
//           summed through LDS);
//   mix     olat[h][:] += p[h][row] c_row: A = p (16 heads x 32 rows), B =
//           the staged rows (32 rows x 16 columns), 4 column tiles per wave.
//           A lane's B operand is one column of 8 consecutive rows (lane
//           group g: rows 8 g .. 8 g + 7 of the 32), read with two LDS
//           transpose reads (ds_read_b64_tr_b16: each 16-lane group reads a
//           4-row x 16-column tile, lane s of the group the 4 columns
//           4 (s % 4) .. of row s / 4, and lane i receives column i's 4
//           rows) -- four 2-byte reads per lane before; p is stored in row
//           order, so A is one 8-float read.
// q and p (f32) enter as bf16 hi + lo pairs (two MFMAs each), so a product
// keeps ~16 significant bits of the f32 operand against the exact bf16 cache
// value: f32-level agreement with the VALU split.  A block runs cpb
// consecutive 64-row chunks of one batch row with an online softmax (olat and
// the running sum rescaled by exp(m_old - m_new)), the next chunk's rows in
// flight during the current chunk, and writes one partial (olat, m, l) at
// slot blockIdx.x; k_mla_out merges ceil(L / (64 cpb)) of them.  MFMA operand
// k order: A and B give lane group g the same 8 k values (scores: k = 32
// step + 8 g + j; mix: row 32 step + 8 g + j), so each instruction adds a
// full partial dot product.
#define MF_H 16
#define MF_KV 512
#define MF_DR 64
#define MF_KS ((MF_KV + MF_DR) / 32)       /* 18 k-steps */
#define MF_ROWB ((MF_KV + MF_DR) * 2)      /* bytes of a staged row: latent, then pe */
#define MF_RP (MF_ROWB + 16)               /* LDS pitch of a staged row (bytes) */
#define MF_PC (MF_ROWB / 16)               /* 16-byte pieces per row (72) */
#define MF_PT (64 * MF_PC / 512)           /* pieces per thread per chunk (9) */
#define MF_PWP 68                          /* LDS pitch of a head's softmax weights (floats) */
#define MF_QLP (MF_KV + 4)                 /* LDS pitch of a staged qlat row (floats) */
static_assert(64 * MF_PC == MF_PT * 512 && MF_KV / 8 * 64 == (MF_PT - 1) * 512 && MF_DR / 8 * 64 == 512,
              "a chunk's pieces: 8 latent loads and 1 pe load per thread");
static_assert(MF_H * MF_QLP * 4 <= 64 * MF_RP, "qlat staging fits the row staging area");
#define MF_THREADS 512                     /* 8 waves: two per 16-row tile */
#define MF_KH (MF_KS / 2)                  /* k-steps per wave */
#define MF_LDS (64 * MF_RP + MF_KS * 2 * 64 * 16 + MF_H * MF_PWP * 4 + 2 * 4 * MF_H * 4 + 4 * 64 * 16)

// four 16-bit values of LDS by the gfx950 transpose read (the lane layout
// above), as two packed dwords
typedef short mf_v4s __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint2 lds_tr16(const unsigned char *p) {
  const mf_v4s r = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) mf_v4s *)(__attribute__((address_space(3))) unsigned char *)p);
  return __builtin_bit_cast(uint2, r);
}

// eight f32 -> bf16 hi (RNE) and lo = bf16(v - hi), packed in operand order
// (v - hi is exact in f32)
__device__ __forceinline__ void split8(const float4 &a, const float4 &b, uint4 &hi, uint4 &lo) {
  const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
  uint32_t h[4], l[4];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    h[i] = pk_bf16(v[2 * i], v[2 * i + 1]);
    l[i] = pk_bf16(v[2 * i] - __uint_as_float(h[i] << 16), v[2 * i + 1] - __uint_as_float(h[i] & 0xffff0000u));
  }
  hi = make_uint4(h[0], h[1], h[2], h[3]);
  lo = make_uint4(l[0], l[1], l[2], l[3]);
}

// grid (ceil(n_split / cpb), B), 512 threads: wave w computes row tile
// w % 4 over k-steps [9 (w / 4), 9 (w / 4) + 9) -- the two halves of a tile's
// 576 k meet through LDS -- and column tiles 4w..4w+3 of the mix; cpb =
// a.cpb chunks per block, two chunks' rows in flight.  (With one wave per
// tile, each chunk's phases ran at one wave per SIMD: ~5.5 us per chunk.)
__global__ __launch_bounds__(MF_THREADS) void k_mla_split_mf(ThvmMlaArgs a) {
  extern __shared__ __align__(16) unsigned char lds_mf[];
  unsigned char *cl = lds_mf;                                        // [64 rows][MF_RP]
  uint4 *qa = (uint4 *)(lds_mf + 64 * MF_RP);                        // [MF_KS][hi, lo][64 lanes]
  float *pw = (float *)(lds_mf + 64 * MF_RP + MF_KS * 2 * 64 * 16);  // [16 heads][MF_PWP]
  float *rmax = pw + MF_H * MF_PWP, *rsum = rmax + 4 * MF_H;         // [4 tiles][16 heads]
  float4 *spart = (float4 *)(rsum + 4 * MF_H);                       // [4 tiles][64 lanes]
  const uint32_t cpb = a.cpb, grp = blockIdx.x, b = blockIdx.y;
  const int32_t L = min(a.len[0], (int32_t)a.max_seq);               // rows [0, L) are live
  const uint32_t cbeg = grp * cpb;
  if (L <= 0 || cbeg * 64 >= (uint32_t)L) return;                    // block-uniform
  const uint32_t cend = min(cbeg + cpb, ((uint32_t)L + 63) / 64);
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6, li = lane & 15, lg = lane >> 4;
  const int rt = wv & 3, kh = wv >> 2;                               // row tile, k half
  // phase clock: 0 entry, 1 q staged, 2 first chunk's scores, 3 first
  // chunk's softmax, 4 chunks done, 5 rows issued, 6 first rows arrived, 7
  // drained
  pclk(a.clk, a.clk_cap, 0);
  // the batch row's caches through buffer resources (rows past max_seq read
  // zero; they are never live)
  const buf_t crs = buf_rsrc((const char *)a.ckv + (uint64_t)b * a.max_seq * (MF_KV * 2), a.max_seq * (MF_KV * 2));
  const buf_t prs = buf_rsrc((const char *)a.kpe + (uint64_t)b * a.max_seq * (MF_DR * 2), a.max_seq * (MF_DR * 2));

  // q first (its staging waits for these loads only), then the first two
  // chunks' rows.  q as A operands (hi, lo) in LDS: fragment f = 64 ks +
  // lane holds head lane % 16, k = 32 ks + 8 (lane / 16) + j; k-steps 0..15
  // from qlat (f32), 16..17 from qpe (bf16: exact, lo = 0).  qlat [16][512]
  // is read coalesced (thread t: float4s t, t + 512, ...) and regrouped
  // through LDS -- a fragment's 16 heads lie 2 KB apart, so loading the
  // fragments directly touched 64 cache lines per load instruction
  const float *ql = a.qlat + (uint64_t)b * MF_H * MF_KV;
  const bf16_t *qp = (const bf16_t *)a.qpe + (uint64_t)b * MF_H * MF_DR;
  static_assert(MF_H * MF_KV / 4 == 4 * MF_THREADS, "four qlat float4s per thread");
  const float4 q0 = ((const float4 *)ql)[tid], q1 = ((const float4 *)ql)[tid + MF_THREADS];
  const float4 q2 = ((const float4 *)ql)[tid + 2 * MF_THREADS], q3 = ((const float4 *)ql)[tid + 3 * MF_THREADS];
  const uint32_t fp = 16 * 64 + (tid & 127), lp = fp & 63;
  const uint4 qpv = *(const uint4 *)(qp + (lp & 15) * MF_DR + ((fp >> 6) - 16) * 32 + (lp >> 4) * 8);

  // chunk c's rows as this thread's MF_PT pieces: loads i < 8 the latent
  // rows' pieces tid + 512 i (row f / 64, piece f % 64), load 8 the pe rows'
  // (row tid / 8, piece 64 + tid % 8), so each load instruction reads one
  // cache; rows past L load a live row of the chunk and are masked out of
  // the softmax
  uint4 cfa[MF_PT], cfb[MF_PT];
  auto issue = [&](uint4 (&cf)[MF_PT], uint32_t c) {
#pragma unroll
    for (int i = 0; i < MF_PT; i++) {
      const uint32_t r = i < MF_PT - 1 ? (tid + 512 * i) / 64 : tid / 8;
      const uint32_t pc = i < MF_PT - 1 ? (tid + 512 * i) % 64 : tid % 8;
      const uint32_t j = c * 64 + r, jc = j < (uint32_t)L ? j : c * 64;
      cf[i] = i < MF_PT - 1 ? buf_ld_stream16(crs, jc * (MF_KV * 2) + pc * 16)
                            : buf_ld_stream16(prs, jc * (MF_DR * 2) + pc * 16);
    }
  };
  issue(cfa, cbeg);
  pclk(a.clk, a.clk_cap, 5);

  // qlat rows into the row staging area (free until the first chunk is
  // staged), a head's 512 values at a pitch of MF_QLP floats; the second
  // chunk's rows go out after these stores (q live across that branch
  // spilled to scratch)
  float *qs = (float *)cl;
  {
    const uint32_t e = 4 * tid, r = e / MF_KV, k = e % MF_KV;   // element e + 2048 i: row r + 4 i
    *(float4 *)(qs + r * MF_QLP + k) = q0;
    *(float4 *)(qs + (r + 4) * MF_QLP + k) = q1;
    *(float4 *)(qs + (r + 8) * MF_QLP + k) = q2;
    *(float4 *)(qs + (r + 12) * MF_QLP + k) = q3;
  }
  if (cbeg + 1 < cend) issue(cfb, cbeg + 1);
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 2; i++) {
    const uint32_t f = tid + MF_THREADS * i, l = f & 63;
    const float *src = qs + (l & 15) * MF_QLP + (f >> 6) * 32 + (l >> 4) * 8;
    uint4 hi, lo;
    split8(*(const float4 *)src, *(const float4 *)(src + 4), hi, lo);
    qa[(f >> 6) * 128 + (f & 63)] = hi;
    qa[(f >> 6) * 128 + 64 + (f & 63)] = lo;
  }
  if (tid < 128) {
    qa[(fp >> 6) * 128 + lp] = qpv;
    qa[(fp >> 6) * 128 + 64 + lp] = make_uint4(0, 0, 0, 0);
  }
  __syncthreads();
  pclk(a.clk, a.clk_cap, 1);

  float m_run[4], l_run[4];
  f32x4_t oacc[4];
#pragma unroll
  for (int i = 0; i < 4; i++) { m_run[i] = -INFINITY; l_run[i] = 0.0f; }
#pragma unroll
  for (int t = 0; t < 4; t++) oacc[t] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};

  // one chunk: its rows are in cf; chunk c + 2 goes into cf once they are
  // staged
  auto chunk = [&](uint4 (&cf)[MF_PT], uint32_t c) {
    const uint32_t nj = min((uint32_t)L - c * 64, 64u);
    if (c == cbeg) pclk_after(a.clk, a.clk_cap, 6, cf[MF_PT - 1].x);
#pragma unroll
    for (int i = 0; i < MF_PT; i++) {
      const uint32_t r = i < MF_PT - 1 ? (tid + 512 * i) / 64 : tid / 8;
      const uint32_t pc = i < MF_PT - 1 ? (tid + 512 * i) % 64 : MF_KV / 8 + tid % 8;
      *(uint4 *)(cl + r * MF_RP + pc * 16) = cf[i];
    }
    __syncthreads();
    if (c + 2 < cend) issue(cf, c + 2);   // in flight during this chunk and the next
    // 1. this wave's half of its tile's scores: lane holds S[head 4 lg + i]
    //    [row 16 rt + li] over its 9 k-steps (four independent chains)
    f32x4_t sc[4];
#pragma unroll
    for (int u = 0; u < 4; u++) sc[u] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    const unsigned char *rowp = cl + (rt * 16 + li) * MF_RP + lg * 16;
#pragma unroll
    for (int st = 0; st < MF_KH; st++) {
      const int ks = kh * MF_KH + st;
      const uint4 bv = *(const uint4 *)(rowp + ks * 64);
      sc[(st & 1) * 2] = mfma16<GX_BF16>(qa[ks * 128 + lane], bv, sc[(st & 1) * 2]);
      sc[(st & 1) * 2 + 1] = mfma16<GX_BF16>(qa[ks * 128 + 64 + lane], bv, sc[(st & 1) * 2 + 1]);
    }
    float4 part_s;
    part_s.x = (sc[0][0] + sc[1][0]) + (sc[2][0] + sc[3][0]);
    part_s.y = (sc[0][1] + sc[1][1]) + (sc[2][1] + sc[3][1]);
    part_s.z = (sc[0][2] + sc[1][2]) + (sc[2][2] + sc[3][2]);
    part_s.w = (sc[0][3] + sc[1][3]) + (sc[2][3] + sc[3][3]);
    if (kh == 1) spart[rt * 64 + lane] = part_s;
    __syncthreads();
    if (c == cbeg) pclk(a.clk, a.clk_cap, 2);

    // 2. softmax over the chunk's rows (the first-half waves hold the full
    //    scores), online across the block's chunks; p is stored in row order
    const uint32_t row = rt * 16 + li;
    const bool rok = row < nj;
    const uint32_t ppos = row;
    float sv[4];
    if (kh == 0) {
      const float4 o = spart[rt * 64 + lane];
      const float full[4] = {part_s.x + o.x, part_s.y + o.y, part_s.z + o.z, part_s.w + o.w};
#pragma unroll
      for (int i = 0; i < 4; i++) {
        sv[i] = rok ? full[i] * a.scale : -INFINITY;
        const float m = row16_max(sv[i]);
        if (li == 0) rmax[rt * MF_H + 4 * lg + i] = m;
      }
    }
    __syncthreads();
    float mn[4], al[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int h = 4 * lg + i;
      const float m = fmaxf(fmaxf(rmax[h], rmax[MF_H + h]), fmaxf(rmax[2 * MF_H + h], rmax[3 * MF_H + h]));
      mn[i] = fmaxf(m_run[i], m);
      al[i] = m_run[i] == -INFINITY ? 0.0f : expf(m_run[i] - mn[i]);
      if (kh == 0) {
        const float p = rok ? expf(sv[i] - mn[i]) : 0.0f;
        const float ps = row16_sum(p);
        if (li == 0) rsum[rt * MF_H + h] = ps;
        pw[h * MF_PWP + ppos] = p;
      }
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int h = 4 * lg + i;
      const float l = rsum[h] + rsum[MF_H + h] + rsum[2 * MF_H + h] + rsum[3 * MF_H + h];
      l_run[i] = l_run[i] * al[i] + l;
      m_run[i] = mn[i];
    }
    if (c == cbeg) pclk(a.clk, a.clk_cap, 3);
    // 3. mix: olat tiles kt = 4 wv + t, lane holds O[head 4 lg + i][16 kt + li]
#pragma unroll
    for (int t = 0; t < 4; t++)
#pragma unroll
      for (int i = 0; i < 4; i++) oacc[t][i] *= al[i];
#pragma unroll
    for (int q = 0; q < 2; q++) {                  // 32-row k-steps
      const float *pr = pw + li * MF_PWP + q * 32 + lg * 8;
      uint4 ah, alo;
      split8(*(const float4 *)pr, *(const float4 *)(pr + 4), ah, alo);
      // rows 32 q + 8 lg + j, j = 0..7, of column (wv * 4 + t) * 16 + li:
      // lane li of the group reads row 32 q + 8 lg + li / 4 (+ 4), columns
      // (wv * 4 + t) * 16 + 4 (li % 4) ..
      const unsigned char *cb = cl + (q * 32 + lg * 8 + (li >> 2)) * MF_RP + (li & 3) * 8;
#pragma unroll
      for (int t = 0; t < 4; t++) {
        const unsigned char *cp = cb + (wv * 4 + t) * 32;
        const uint2 r0 = lds_tr16(cp), r1 = lds_tr16(cp + 4 * MF_RP);
        const uint4 bv = make_uint4(r0.x, r0.y, r1.x, r1.y);
        oacc[t] = mfma16<GX_BF16>(ah, bv, oacc[t]);
        oacc[t] = mfma16<GX_BF16>(alo, bv, oacc[t]);
      }
    }
    __syncthreads();                               // cl, pw, spart and the reductions are reused
  };
  for (uint32_t c = cbeg; c < cend; c += 2) {
    chunk(cfa, c);
    if (c + 1 < cend) chunk(cfb, c + 1);
  }
  pclk(a.clk, a.clk_cap, 4);

  // the partial goes out as streaming stores: the merge kernel reads it
  // from memory, and lines left dirty in L2 would be written back at the
  // kernel boundary, ahead of the merge
  float *part = a.part + ((uint64_t)b * a.n_split + grp) * MF_H * (MF_KV + 4);
#pragma unroll
  for (int t = 0; t < 4; t++)
#pragma unroll
    for (int i = 0; i < 4; i++)
      __builtin_nontemporal_store(oacc[t][i], part + (4 * lg + i) * (MF_KV + 4) + (wv * 4 + t) * 16 + li);
  if (wv == 0 && li == 0) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
      __builtin_nontemporal_store(m_run[i], part + (4 * lg + i) * (MF_KV + 4) + MF_KV);
      __builtin_nontemporal_store(l_run[i], part + (4 * lg + i) * (MF_KV + 4) + MF_KV + 1);
    }
  }
  pclk_end(a.clk, a.clk_cap);
}

// ---- k_mla_out ----------------------------------------------------------
// grid (B*H, MLA_OUT_SPLIT), 512 threads: merge the live splits of (b, h)
// into olat -- split weights computed once, threads split into (float4
// column, split group) so each issues a few 16-byte loads, groups summed in
// order in LDS -- then o[b][h][m] = bf16(scale_m * sum_k olat[k] W_uv[h][m][k])
// for this block's share of the dv rows, whose weight loads are issued before
// the merge (they do not depend on it).
#define MLA_MAX_SPLITS 512
#define MLA_OUT_THREADS 512
#define MLA_OUT_SPLIT 2
#define MLA_WPASS 8
#define MLA_OPRE_MAX 20   /* partial vectors per thread loaded up front, long caches */
template <bool FP8, int OPRE, int WP>
__global__ __launch_bounds__(MLA_OUT_THREADS) void k_mla_out(ThvmMlaArgs a) {
  extern __shared__ float ol[];                       // [kv] olat | [ns] weights | [nsg][kv]
  constexpr uint32_t EPC = FP8 ? 16 : 8;
  const uint32_t bh = blockIdx.x, b = bh / a.H, h = bh % a.H, kv = a.kv, dv = a.dv;
  const uint32_t tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  constexpr uint32_t nw = MLA_OUT_THREADS / 64;
  // phase clock: the merge's blocks follow the split's in the clock buffer;
  // 0 entry, 1 split weights, 2 partials summed per group, 3 olat in LDS,
  // 7 drained
  uint64_t *const clk = a.clk ? a.clk + (uint64_t)a.clk_cap * PCLK_MARKS : nullptr;
  pclk(clk, a.clk_cap, 0);
  const uint32_t rowb = kv * (FP8 ? 1 : 2), LPR = rowb / 16;     // kv <= 512: LPR <= 64
  const uint32_t rpp = 64 / LPR, sub = lane / LPR, c = lane % LPR;
  const uint32_t rows_pb = (dv + gridDim.y - 1) / gridDim.y;
  const uint32_t m0 = blockIdx.y * rows_pb, m1 = min(m0 + rows_pb, dv);
  const int32_t L = min(a.len[0], (int32_t)a.max_seq);
  const uint32_t span = MLA_CHUNK * (a.cpb > 1 ? a.cpb : 1);   // cache rows per partial
  const uint32_t ns = L > 0 ? ((uint32_t)L + span - 1) / span : 0;
  const uint64_t pst = (uint64_t)a.H * (kv + 4);
  const float *p0 = a.part + (uint64_t)b * a.n_split * pst + (uint64_t)h * (kv + 4);
  float *wsp = ol + kv, *grp = wsp + MLA_MAX_SPLITS;
  __shared__ float red[16];
  // Every load is an unguarded buffer load (offsets past a range read zero
  // with no access), issued in the order the merge consumes them: m and l,
  // the partial vectors, then the W_uv rows and their scales.  Loads complete
  // in issue order, so each wait covers only what its step needs (a guarded
  // load made every wait drain all of them, W_uv included).
  const buf_t prs = buf_rsrc_u(p0, (uint32_t)((uint64_t)ns * pst * 4u));
  // split weights w_s = exp(m_s - M) / sum_s exp(m_s - M) l_s (one split per thread)
  const uint32_t mlo = tid < ns ? (uint32_t)(((uint64_t)tid * pst + kv) * 4u) : BUF_OOB;
  const uint32_t mb = buf_ld4(prs, mlo), lb = buf_ld4(prs, mlo == BUF_OOB ? BUF_OOB : mlo + 4u);
  // the thread's first OPRE partial vectors go out with m and l (they do not
  // depend on the weights): thread -> (float4 column c4, split group g),
  // splits g, g + nsg, ...; the weights' reductions then run while they are
  // in flight, and the merge waits for one round trip instead of one per
  // four splits (same splits in the same order: the same sums).  OPRE = 20
  // (160 VGPRs, one block per CU) where a row has more than 4 nsg partials
  // (C5 batch 1: 65), else 4 (80 VGPRs; at C5 batch 32, 8 partials per row
  // and 1024 blocks, 20 measured 66 -> 77 us per layer)
  const uint32_t nc4 = kv / 4, nsg = MLA_OUT_THREADS / nc4;
  const uint32_t c4 = tid % nc4, g = tid / nc4;
  float4 vp[OPRE];
#pragma unroll
  for (int u = 0; u < OPRE; u++) {
    const uint32_t sp = g + u * nsg;
    const uint4 v = buf_ld16(prs, sp < ns ? (uint32_t)(((uint64_t)sp * pst + 4 * c4) * 4u) : BUF_OOB);
    vp[u] = make_float4(__uint_as_float(v.x), __uint_as_float(v.y), __uint_as_float(v.z), __uint_as_float(v.w));
  }
  // this block's W_uv rows and their scales (independent of the merge)
  const buf_t wrs = buf_rsrc(a.wuv, a.H * dv * rowb);
  const buf_t srs = buf_rsrc(a.suv, a.suv ? a.H * dv * 4u : 0u);
  // (WP passes of 8 waves x rpp rows cover the block's rows: no pass of
  // load instructions that would all read past them)
  uint4 wq[WP];
  uint32_t scw[WP];
#pragma unroll
  for (int q = 0; q < WP; q++) {
    const uint32_t mm = m0 + (wv + q * nw) * rpp + sub;
    wq[q] = buf_ld_stream16(wrs, mm < m1 ? (h * dv + mm) * rowb + c * 16u : BUF_OOB);
    scw[q] = buf_ld4(srs, mm < m1 ? (h * dv + mm) * 4u : BUF_OOB);
  }
  pclk(clk, a.clk_cap, 4);
  pclk_after(clk, a.clk_cap, 5, mb);
  pclk_after(clk, a.clk_cap, 6, wq[0].x);
  const float ms = tid < ns ? __uint_as_float(mb) : -INFINITY, ls = __uint_as_float(lb);
  float M = wave_max(ms);
  if (lane == 0) red[wv] = M;
  __syncthreads();
  M = red[0];
  for (uint32_t w = 1; w < MLA_OUT_THREADS / 64; w++) M = fmaxf(M, red[w]);
  const float ws = tid < ns ? expf(ms - M) : 0.0f;
  const float dsum = wave_sum(ws * ls);
  if (lane == 0) red[8 + wv] = dsum;
  __syncthreads();
  float den = 0.0f;
  for (uint32_t w = 0; w < MLA_OUT_THREADS / 64; w++) den += red[8 + w];
  if (tid < ns) wsp[tid] = ws / den;
  __syncthreads();
  pclk(clk, a.clk_cap, 1);
  // partial merge: groups stride the splits
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
  for (int u = 0; u < OPRE; u++) {
    const uint32_t sp = g + u * nsg;
    const float w = sp < ns ? wsp[sp] : 0.0f;
    acc.x += w * vp[u].x; acc.y += w * vp[u].y; acc.z += w * vp[u].z; acc.w += w * vp[u].w;
  }
  for (uint32_t s0 = g + OPRE * nsg; s0 < ns; s0 += 4 * nsg) {     // four 16-byte loads in flight
    float4 v[4];
#pragma unroll
    for (int u = 0; u < 4; u++) {
      const uint32_t s = s0 + u * nsg;
      const uint4 r = buf_ld16(prs, s < ns ? (uint32_t)(((uint64_t)s * pst + 4 * c4) * 4u) : BUF_OOB);
      v[u] = make_float4(__uint_as_float(r.x), __uint_as_float(r.y), __uint_as_float(r.z), __uint_as_float(r.w));
    }
#pragma unroll
    for (int u = 0; u < 4; u++) {
      const uint32_t s = s0 + u * nsg;
      const float w = s < ns ? wsp[s] : 0.0f;
      acc.x += w * v[u].x; acc.y += w * v[u].y; acc.z += w * v[u].z; acc.w += w * v[u].w;
    }
  }
  ((float4 *)grp)[g * nc4 + c4] = acc;
  __syncthreads();
  pclk(clk, a.clk_cap, 2);
  const uint32_t nchk = kv / EPC;
  if (tid < nc4) {
    float4 s = ((const float4 *)grp)[tid];
    for (uint32_t q = 1; q < nsg; q++) {
      const float4 v = ((const float4 *)grp)[q * nc4 + tid];
      s.x += v.x; s.y += v.y; s.z += v.z; s.w += v.w;
    }
    ((float4 *)ol)[chunk_swz<EPC>(4 * tid, nchk) / 4] = s;   // W_uv chunk order
  }
  __syncthreads();
  pclk(clk, a.clk_cap, 3);
#pragma unroll
  for (int q = 0; q < WP; q++) {
    const uint32_t r0 = m0 + (wv + q * nw) * rpp;
    if (r0 >= m1) break;                               // wave-uniform
    const uint32_t mm = r0 + sub;
    float w[16];
    w16<FP8>(wq[q], make_uint4(0, 0, 0, 0), w);
    const float4 *o4 = (const float4 *)ol;
    float accw = 0.0f;
#pragma unroll
    for (uint32_t qd = 0; qd < EPC / 4; qd++) {
      const float4 x = o4[qd * nchk + c];
      accw += x.x * w[4 * qd] + x.y * w[4 * qd + 1] + x.z * w[4 * qd + 2] + x.w * w[4 * qd + 3];
    }
    accw = group_sum(accw, (int)LPR);
    if (mm < m1 && c == 0) {
      const uint64_t row = (uint64_t)h * dv + mm;
      const float s = a.suv ? __uint_as_float(scw[q]) : 1.0f;
      ((bf16_t *)a.o)[(uint64_t)b * a.H * dv + row] = f2bf(accw * s);
    }
  }
  pclk_end(clk, a.clk_cap);
}

// ---- k_mla_out_q --------------------------------------------------------
// The merge in latent quarters, for decodes whose o projection runs on the
// GEMV (at most 4 rows): k_mla_out's 2 blocks per head each read all of the
// head's partials (65 x 2 KB at C5 batch 1), and 32 blocks are bound by what
// one CU can load.  Grid (B*H, MLA_OQ): block (b h, q) merges the live splits
// over latent columns [q kv/4, (q+1) kv/4) -- the same split weights, each
// column's partials summed in split-group order -- and applies that quarter
// of W_uv, writing the unscaled quarter sum oq[q][b][h dv + m] (f32).  The o
// projection's GEMV adds the four quarters, applies the W_uv row scale and
// rounds to bf16 as it stages x (norm = 3), where k_mla_out rounds one sum
// over all kv columns: another summation order, so not the same bits.
#define MLA_OQ 4
#define MLA_OQ_WP 4      /* W_uv load passes at most */
// PRE partial vectors per thread loaded up front (a longer cache's rest in a
// loop), WP W_uv load passes: both chosen at launch to what the rows need --
// load instructions that only read past the data still cost a CU's issue
template <bool FP8, int PRE, int WP>
__global__ __launch_bounds__(MLA_OUT_THREADS) void k_mla_out_q(ThvmMlaArgs a) {
  constexpr uint32_t EPC = FP8 ? 16 : 8;
  __shared__ float red[16];
  __shared__ float wsp[MLA_MAX_SPLITS];
  __shared__ __align__(16) float4 grp[MLA_OUT_THREADS];
  __shared__ __align__(16) float olq[MF_KV / MLA_OQ];
  const uint32_t bh = blockIdx.x, b = bh / a.H, h = bh % a.H, kv = a.kv, dv = a.dv, qd = blockIdx.y;
  const uint32_t kq = kv / MLA_OQ;                                  // this quarter's columns
  const uint32_t tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  constexpr uint32_t nw = MLA_OUT_THREADS / 64;
  uint64_t *const clk = a.clk ? a.clk + (uint64_t)a.clk_cap * PCLK_MARKS : nullptr;
  pclk(clk, a.clk_cap, 0);
  const uint32_t rowq = kq * (FP8 ? 1 : 2), LPR = rowq / 16;          // lanes per W_uv row quarter
  const uint32_t rpp = 64 / LPR, sub = lane / LPR, c = lane % LPR;
  const int32_t L = min(a.len[0], (int32_t)a.max_seq);
  const uint32_t span = MLA_CHUNK * (a.cpb > 1 ? a.cpb : 1);
  const uint32_t ns = L > 0 ? ((uint32_t)L + span - 1) / span : 0;
  const uint64_t pst = (uint64_t)a.H * (kv + 4);
  const float *p0 = a.part + (uint64_t)b * a.n_split * pst + (uint64_t)h * (kv + 4);
  // loads in consumption order: m and l, this quarter's partial vectors, the
  // W_uv row quarters (unguarded buffer loads)
  const buf_t prs = buf_rsrc_u(p0, (uint32_t)((uint64_t)ns * pst * 4u));
  const uint32_t mlo = tid < ns ? (uint32_t)(((uint64_t)tid * pst + kv) * 4u) : BUF_OOB;
  const uint32_t mb = buf_ld4(prs, mlo), lb = buf_ld4(prs, mlo == BUF_OOB ? BUF_OOB : mlo + 4u);
  const uint32_t nc4 = kq / 4, nsg = MLA_OUT_THREADS / nc4;
  const uint32_t c4 = tid % nc4, g = tid / nc4;
  float4 vp[PRE];
#pragma unroll
  for (int u = 0; u < PRE; u++) {
    const uint32_t sp = g + u * nsg;
    const uint4 v = buf_ld16(prs, sp < ns ? (uint32_t)(((uint64_t)sp * pst + qd * kq + 4 * c4) * 4u) : BUF_OOB);
    vp[u] = make_float4(__uint_as_float(v.x), __uint_as_float(v.y), __uint_as_float(v.z), __uint_as_float(v.w));
  }
  const buf_t wrs = buf_rsrc(a.wuv, a.H * dv * kv * (FP8 ? 1u : 2u));
  uint4 wq[WP], wq2[WP];
#pragma unroll
  for (int q = 0; q < WP; q++) {
    const uint32_t mm = (wv + q * nw) * rpp + sub;
    const uint32_t off = (h * dv + mm) * (kv * (FP8 ? 1u : 2u)) + qd * rowq + c * 16u;
    wq[q] = buf_ld_stream16(wrs, mm < dv ? off : BUF_OOB);
    wq2[q] = make_uint4(0, 0, 0, 0);
  }
  pclk(clk, a.clk_cap, 4);
  // split weights w_s = exp(m_s - M) / sum_s exp(m_s - M) l_s, as k_mla_out
  const float ms = tid < ns ? __uint_as_float(mb) : -INFINITY, ls = __uint_as_float(lb);
  float M = wave_max(ms);
  if (lane == 0) red[wv] = M;
  __syncthreads();
  M = red[0];
  for (uint32_t w = 1; w < nw; w++) M = fmaxf(M, red[w]);
  const float ws = tid < ns ? expf(ms - M) : 0.0f;
  const float dsum = wave_sum(ws * ls);
  if (lane == 0) red[8 + wv] = dsum;
  __syncthreads();
  float den = 0.0f;
  for (uint32_t w = 0; w < nw; w++) den += red[8 + w];
  if (tid < ns) wsp[tid] = ws / den;
  __syncthreads();
  pclk(clk, a.clk_cap, 1);
  float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
  for (int u = 0; u < PRE; u++) {
    const uint32_t sp = g + u * nsg;
    const float w = sp < ns ? wsp[sp] : 0.0f;
    acc.x += w * vp[u].x; acc.y += w * vp[u].y; acc.z += w * vp[u].z; acc.w += w * vp[u].w;
  }
  for (uint32_t s0 = g + PRE * nsg; s0 < ns; s0 += 4 * nsg) {     // longer caches
    float4 v[4];
#pragma unroll
    for (int u = 0; u < 4; u++) {
      const uint32_t sp = s0 + u * nsg;
      const uint4 r = buf_ld16(prs, sp < ns ? (uint32_t)(((uint64_t)sp * pst + qd * kq + 4 * c4) * 4u) : BUF_OOB);
      v[u] = make_float4(__uint_as_float(r.x), __uint_as_float(r.y), __uint_as_float(r.z), __uint_as_float(r.w));
    }
#pragma unroll
    for (int u = 0; u < 4; u++) {
      const uint32_t sp = s0 + u * nsg;
      const float w = sp < ns ? wsp[sp] : 0.0f;
      acc.x += w * v[u].x; acc.y += w * v[u].y; acc.z += w * v[u].z; acc.w += w * v[u].w;
    }
  }
  grp[g * nc4 + c4] = acc;
  __syncthreads();
  pclk(clk, a.clk_cap, 2);
  // the nsg group sums of each column in two rounds (groups of 4, then the
  // nsg / 4 of those, each in group order): a serial pass over nsg = 16
  // groups by one thread per column had been 16 dependent LDS reads
  const uint32_t nchk = kq / EPC, nsg4 = nsg / 4;
  float4 r1 = make_float4(0.f, 0.f, 0.f, 0.f);
  if (tid < nc4 * nsg4) {
    const uint32_t cc = tid % nc4, gg = tid / nc4;
    float4 t = grp[(4 * gg) * nc4 + cc];
#pragma unroll
    for (uint32_t q = 1; q < 4; q++) {
      const float4 v = grp[(4 * gg + q) * nc4 + cc];
      t.x += v.x; t.y += v.y; t.z += v.z; t.w += v.w;
    }
    r1 = t;
  }
  __syncthreads();
  if (tid < nc4 * nsg4) grp[tid] = r1;                             // (gg, cc) at gg nc4 + cc
  __syncthreads();
  if (tid < nc4) {
    float4 t = grp[tid];
    for (uint32_t q = 1; q < nsg4; q++) {
      const float4 v = grp[q * nc4 + tid];
      t.x += v.x; t.y += v.y; t.z += v.z; t.w += v.w;
    }
    ((float4 *)olq)[chunk_swz<EPC>(4 * tid, nchk) / 4] = t;      // W_uv chunk order
  }
  __syncthreads();
  pclk(clk, a.clk_cap, 3);
  float *oq = (float *)a.o + (uint64_t)qd * a.B * a.H * dv + (uint64_t)b * a.H * dv;
#pragma unroll
  for (int q = 0; q < WP; q++) {
    const uint32_t r0 = (wv + q * nw) * rpp;
    if (r0 >= dv) break;                                           // wave-uniform
    const uint32_t mm = r0 + sub;
    float w[16];
    w16<FP8>(wq[q], wq2[q], w);
    const float4 *o4 = (const float4 *)olq;
    float accw = 0.0f;
#pragma unroll
    for (uint32_t qd4 = 0; qd4 < EPC / 4; qd4++) {
      const float4 x = o4[qd4 * nchk + c];
      accw += x.x * w[4 * qd4] + x.y * w[4 * qd4 + 1] + x.z * w[4 * qd4 + 2] + x.w * w[4 * qd4 + 3];
    }
    accw = group_sum(accw, (int)LPR);
    if (mm < dv && c == 0) oq[(uint64_t)h * dv + mm] = accw;
  }
  pclk_end(clk, a.clk_cap);
}

// -------------------------------------------------------------------------
static int mla_common(const ThvmMlaArgs *a, char *err, int errlen) {
  if (a->B == 0 || a->H == 0 || a->dn == 0 || a->dr == 0 || a->dr % 2 || a->dr > 64 ||
      (a->kv != 64 && a->kv != 128 && a->kv != 256 && a->kv != 512) || a->dv == 0 ||
      a->max_seq == 0) {
    snprintf(err, errlen, "mla: bad geometry B=%u H=%u dn=%u dr=%u kv=%u dv=%u", a->B, a->H,
             a->dn, a->dr, a->kv, a->dv);
    return -1;
  }
  if (a->wdt != THVM_DT_FP8E4M3 && a->wdt != THVM_DT_BF16) {
    snprintf(err, errlen, "mla: absorbed weights must be fp8 e4m3 or bf16");
    return -1;
  }
  return 0;
}

extern "C" int thvm_k_mla_prep(const ThvmMlaArgs *a, hipStream_t s, char *err, int errlen) {
  if (mla_common(a, err, errlen)) return -1;
  const uint32_t wsz = a->wdt == THVM_DT_FP8E4M3 ? 1 : 2;
  const uint32_t lpr = a->dn * wsz / 16;
  if ((a->dn * wsz) % 16 || lpr > 64 || (lpr & (lpr - 1)) ||
      a->ldq < a->H * (a->dn + a->dr) + a->kv + a->dr || ((uintptr_t)a->wuk & 15)) {
    snprintf(err, errlen, "mla_prep: d_nope rows must be a power-of-two number of 16-byte chunks "
             "(<= 64) and ldq hold the q|kv row");
    return -1;
  }
  const uint32_t QB = a->kv / 64, BG = (a->B + MLA_PREP_ROWS - 1) / MLA_PREP_ROWS;
  uint64_t lds = (uint64_t)(a->B < MLA_PREP_ROWS ? a->B : MLA_PREP_ROWS) * a->dn * 4;
  if ((uint64_t)a->kv * 4 + 64 > lds) lds = (uint64_t)a->kv * 4 + 64;
  if (lds > 64 * 1024) { snprintf(err, errlen, "mla_prep: d_nope too large for LDS staging"); return -1; }
  const dim3 grid(a->H * QB * BG + a->B);
  if (a->wdt == THVM_DT_FP8E4M3) thvm_launch(true, true, k_mla_prep<true>, grid, dim3(256), (uint32_t)lds, s, *a);
  else thvm_launch(true, true, k_mla_prep<false>, grid, dim3(256), (uint32_t)lds, s, *a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) { snprintf(err, errlen, "mla_prep launch: %s", hipGetErrorString(e)); return -1; }
  return 0;
}

typedef void (*mla_split_fn)(ThvmMlaArgs);
static mla_split_fn pick_kpl(uint32_t kv) {
  switch (kv / 64) {
    case 1: return k_mla_split<1>;
    case 2: return k_mla_split<2>;
    case 4: return k_mla_split<4>;
    case 8: return k_mla_split<8>;
    default: return nullptr;
  }
}

extern "C" uint64_t thvm_k_mla_part_bytes(uint32_t B, uint32_t H, uint32_t kv, uint32_t n_split) {
  return (uint64_t)B * n_split * H * (kv + 4) * 4;
}

extern "C" int thvm_k_mla_attn(const ThvmMlaArgs *a, hipStream_t s, char *err, int errlen) {
  if (mla_common(a, err, errlen)) return -1;
  const uint32_t wsz = a->wdt == THVM_DT_FP8E4M3 ? 1 : 2;
  if (a->n_split * MLA_CHUNK < a->max_seq) {
    snprintf(err, errlen, "mla_attn: n_split %u * %u < max_seq %u", a->n_split, MLA_CHUNK, a->max_seq);
    return -1;
  }
  if ((a->kv * wsz) % 16 || (a->kv * wsz / 16 > 64 && (a->kv * wsz / 16) % 64) || ((uintptr_t)a->wuv & 15)) {
    snprintf(err, errlen, "mla_attn: W_uv rows must be 16-byte multiples");
    return -1;
  }
  {
    const uint32_t lpr = a->kv * wsz / 16, rpp = 64 / lpr;
    const uint32_t rows_pb = (a->dv + MLA_OUT_SPLIT - 1) / MLA_OUT_SPLIT;
    if ((rows_pb + 8 * rpp - 1) / (8 * rpp) > MLA_WPASS) {
      snprintf(err, errlen, "mla_attn: d_v %u too large for the V projection tiling", a->dv);
      return -1;
    }
  }
  if (a->n_split > MLA_MAX_SPLITS) { snprintf(err, errlen, "mla_attn: more than %d splits", MLA_MAX_SPLITS); return -1; }
  const bool mf_shape = a->H == MF_H && a->kv == MF_KV && a->dr == MF_DR;
  if (a->mode > 2 || (a->mode == 2 && !mf_shape)) {
    snprintf(err, errlen, "mla_attn: mode %u (0 auto, 1 VALU, 2 MFMA for H=%d kv=%d dr=%d)", a->mode, MF_H, MF_KV, MF_DR);
    return -1;
  }
  ThvmMlaArgs ak = *a;
  if (a->mode == 2 || (a->mode == 0 && mf_shape)) {
    // MFMA split: cpb 64-row chunks per block (fewer partials to write and
    // merge with more rows per block)
    // (a block holds ~109 KB of LDS, so one block per CU: the smallest chunk
    // count that keeps the grid within one block per CU of the 256, so the
    // split runs in a single round)
    uint32_t cpb = a->cpb;
    if (cpb == 0) cpb = (uint32_t)(((uint64_t)a->B * a->n_split + 255) / 256);
    if (cpb > a->n_split) cpb = a->n_split;       // one block takes every chunk
    ak.cpb = cpb;
    mla_split_fn f = k_mla_split_mf;
    hipError_t e = hipFuncSetAttribute((const void *)f, hipFuncAttributeMaxDynamicSharedMemorySize, MF_LDS);
    if (e != hipSuccess) { snprintf(err, errlen, "mla_attn: hipFuncSetAttribute: %s", hipGetErrorString(e)); return -1; }
    thvm_launch(true, false, f, dim3((a->n_split + cpb - 1) / cpb, a->B), dim3(MF_THREADS), MF_LDS, s, ak);
  } else {
    if (a->cpb > 1) { snprintf(err, errlen, "mla_attn: the VALU split runs one chunk per block"); return -1; }
    ak.cpb = 1;
    mla_split_fn f = a->H % MLA_HG == 0 ? pick_kpl(a->kv) : nullptr;
    if (!f) { snprintf(err, errlen, "mla_attn: no kernel for H=%u kv=%u (H a multiple of %d)", a->H, a->kv, MLA_HG); return -1; }
    const uint32_t lds = (uint32_t)(MLA_CHUNK * a->kv * 2 + MLA_HG * MLA_CHUNK * 4);
    if (lds > 64 * 1024) {
      hipError_t e = hipFuncSetAttribute((const void *)f, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
      if (e != hipSuccess) { snprintf(err, errlen, "mla_attn: hipFuncSetAttribute: %s", hipGetErrorString(e)); return -1; }
    }
    thvm_launch(true, false, f, dim3(a->n_split, a->H / MLA_HG, a->B), dim3(MLA_THREADS), lds, s, ak);
  }
  if (a->oq) {                                    // the merge in latent quarters
    const uint32_t kq = a->kv / MLA_OQ, lpr = kq * wsz / 16, rpp = lpr ? 64 / lpr : 0;
    if (kq * wsz % 16 || lpr == 0 || lpr > 64 || kq % (wsz == 1 ? 16 : 8) ||
        a->dv > MLA_OQ_WP * 8 * rpp) {
      snprintf(err, errlen, "mla_attn: oq=1 needs kv/4 a multiple of the 16-byte chunk and d_v <= %u",
               MLA_OQ_WP * 8 * rpp);
      return -1;
    }
    // up front: the partials a split group folds (65 at C5 batch 1, 16 groups:
    // 5), else 8 and a loop; W_uv passes: 8 waves x rpp rows each over d_v
    const uint32_t nsg = MLA_OUT_THREADS / (kq / 4), nsp = (a->n_split + ak.cpb - 1) / ak.cpb;
    const bool pre5 = nsp <= 5 * nsg, wp2 = a->dv <= 2 * 8 * rpp;
    const bool f8 = a->wdt == THVM_DT_FP8E4M3;
    void (*fq)(ThvmMlaArgs) =
        f8 ? (pre5 ? (wp2 ? k_mla_out_q<true, 5, 2> : k_mla_out_q<true, 5, 4>)
                   : (wp2 ? k_mla_out_q<true, 8, 2> : k_mla_out_q<true, 8, 4>))
           : (pre5 ? (wp2 ? k_mla_out_q<false, 5, 2> : k_mla_out_q<false, 5, 4>)
                   : (wp2 ? k_mla_out_q<false, 8, 2> : k_mla_out_q<false, 8, 4>));
    thvm_launch(false, true, fq, dim3(a->B * a->H, MLA_OQ), dim3(MLA_OUT_THREADS), 0, s, ak);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) { snprintf(err, errlen, "mla_attn launch: %s", hipGetErrorString(e)); return -1; }
    return 0;
  }
  const dim3 g2(a->B * a->H, MLA_OUT_SPLIT);
  const uint32_t lds2 = (a->kv + MLA_MAX_SPLITS + MLA_OUT_THREADS * 4) * 4;
  // partials per row at most: n_split / cpb; over 4 per split group -> 20 up front
  const uint32_t nsg = MLA_OUT_THREADS / (a->kv / 4);
  const bool longp = (a->n_split + ak.cpb - 1) / ak.cpb > 4 * nsg;
  // W_uv passes: 8 waves x rpp rows each cover the block's share of d_v
  const uint32_t rpp = 64 / (a->kv * wsz / 16), rows_pb = (a->dv + MLA_OUT_SPLIT - 1) / MLA_OUT_SPLIT;
  const bool wp4 = (rows_pb + 8 * rpp - 1) / (8 * rpp) <= 4;
  void (*fo)(ThvmMlaArgs);
  if (a->wdt == THVM_DT_FP8E4M3)
    fo = longp ? (wp4 ? k_mla_out<true, MLA_OPRE_MAX, 4> : k_mla_out<true, MLA_OPRE_MAX, MLA_WPASS>)
               : (wp4 ? k_mla_out<true, 4, 4> : k_mla_out<true, 4, MLA_WPASS>);
  else
    fo = longp ? (wp4 ? k_mla_out<false, MLA_OPRE_MAX, 4> : k_mla_out<false, MLA_OPRE_MAX, MLA_WPASS>)
               : (wp4 ? k_mla_out<false, 4, 4> : k_mla_out<false, 4, MLA_WPASS>);
  thvm_launch(false, true, fo, g2, dim3(MLA_OUT_THREADS), lds2, s, ak);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) { snprintf(err, errlen, "mla_attn launch: %s", hipGetErrorString(e)); return -1; }
  return 0;
}
