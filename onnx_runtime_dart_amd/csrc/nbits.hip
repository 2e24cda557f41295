// MatMulNBits (int4, block-quantized) on gfx950.
//
// Reference semantics: opMatMulNBits, lib/src/onnx_qlinear_ops.dart:115-228:
//   y[m, n] = sum_k a[m, k] * fl32((q[n, k] - zp[n, blk]) * s[n, blk]) (+ bias[n])
// with q the 4-bit code (low nibble = even k), blk = k / block_size and the
// zero point 8 by default, packed uint4, or float.
//
// Device weight layout (built once on upload by the repack kernels of
// mg_nbits_upload):
//   columns are grouped by 64 ("column group"), k by 128 ("k group").
//   wq[cg][kg][g][col][j] is one dword holding the 8 nibbles of column
//   (cg*64 + col) at k = kg*128 + 32*j + 8*g + t, t = 0..7, with even t in the
//   low half-word and odd t in the high half-word (nibble position
//   t/2 resp. 4 + t/2).  A lane reading 16 bytes at (g, col) gets j = 0..3.
//   scales[cg][blk][col], zero points zp4[cg][blk/2][col] (original packed
//   byte) or zpf[cg][blk][col].
//
// Compute paths (plan_nbits picks one per call):
//   * M <= 2, and M <= 4 with float zero points ("decode"): activations are
//     quantised per (row, 128-or-block k slice) to 15-bit fixed point split
//     into four signed int4 digits; each lane owns one column and streams
//     16-byte weight loads, multiplying with v_dot8_i32_i4 against the digit
//     planes.  Zero point and scale are applied once per block in fp32.  At
//     one row: column-slice, split-K and persistent forms of the same sums.
//   * 3 <= M <= 16 with integer zero points: the 16-row MFMA GEMV
//     (k_gemv_mfma: fp16 hi/lo activations, weights dequantised per lane).
//   * Prefill, block >= 128 (nbits_f8.hip): on weights with prefill images
//     the fp6 GEMM (three e2m3 activation digits; float zero points taken
//     out as row sums), otherwise the fp8 GEMM that dequantises each tile.
//   * Prefill, blocks of 32 or 64 with integer zero points: activations as an
//     fp16 pair hi + lo (scaled by a power of two per row, ~22 bits); each
//     workgroup unpacks its weight tile once into LDS as exact fp16 (q - zp)
//     (times 16 for half of the k, matched by a 2^-4 on those activations);
//     v_mfma_f32_32x32x16_f16 accumulates hi*W and lo*W in fp32 and the block
//     scale is applied on the fp32 accumulator.
//   * The rest with M > 4 (float zero points without images or below block
//     128, 16-k blocks): columns dequantised to fp32 as the reference does,
//     in chunks, each chunk on the fp32 MFMA GEMM.
#include <hip/hip_runtime.h>

#include <errno.h>
#include <fcntl.h>
#include <unistd.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <string>
#include <thread>
#include <vector>

#include "mg_internal.h"
#include "nbits_common.h"

namespace {

// ------------------------------------------------------------- prepasses

// Activation prepass of the MFMA path.  Per row: an exponent e that puts the
// row's largest finite |a| in [2^13, 2^14), and the fp16 hi/lo split of
// a * 2^e (hi = fp16(x), lo = fp16(x - hi)); k offsets 2, 3, 6, 7 of every 8
// take a further 2^-4 to meet weights carried as 16 (q - zp).  Output order is
// the GEMM's fragment order: for 32-row tile m32, k group kg, 16-k step st,
// ahl[((m32 * c4n + kg) * 8 + st) * 128 + 32 h + r] holds the hi fp16 x 8 of
// row r, k = 128 kg + 16 st + 8 h .. +7, and +64 the lo part; texp[row] = e.
// Rows past M and k past K are zeros.  Non-finite values pass through in hi.
// Workgroup: 4 rows, each row on one wave.  UL > 0: the row's 16-k pieces are
// at most 64 UL, and each lane reads its UL pieces once, with all loads in
// flight together, and keeps them in registers for the split; UL = 0 (longer
// rows) reads the row twice.
template <int UL>
__global__ __launch_bounds__(256) void k_af16split(
    const float *__restrict__ a, int64_t M, int64_t K, int c4n, int vec,
    uint4 *__restrict__ ahl, int *__restrict__ texp) {
  const int t = threadIdx.x;
  const int u0 = t & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (t >> 6);
  const int64_t m32 = row >> 5;
  const int r = (int)(row & 31);
  const int units = c4n * 8;  // 16-k pieces of the row
  const float *arow = a + row * K;
  auto load16 = [&](int u, float v[16]) {
    const int64_t k0 = (int64_t)u * 16;
    if (row < M && vec && k0 + 16 <= K) {
      const float4 *src = reinterpret_cast<const float4 *>(arow + k0);
#pragma unroll
      for (int q4 = 0; q4 < 4; q4++) {
        const float4 x = src[q4];
        v[4 * q4] = x.x; v[4 * q4 + 1] = x.y; v[4 * q4 + 2] = x.z; v[4 * q4 + 3] = x.w;
      }
    } else {
#pragma unroll
      for (int i = 0; i < 16; i++) v[i] = (row < M && k0 + i < K) ? arow[k0 + i] : 0.f;
    }
  };
  auto row_exponent = [&](float mx) {
    for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
    int e = 0;
    if (mx > 0.f) {
      int ex;
      frexpf(mx, &ex);
      e = 14 - ex;
    }
    if (u0 == 0) texp[row] = e;
    return e;
  };
  auto split = [&](int u, const float v[16], int e) {
    uint4 *o = ahl + ((m32 * c4n + (u >> 3)) * 8 + (u & 7)) * 128;
#pragma unroll
    for (int h = 0; h < 2; h++) {
      half8 hi, lo;
#pragma unroll
      for (int i = 0; i < 8; i++) {
        const float x = ldexpf(v[8 * h + i], (i & 2) ? e - 4 : e);
        const _Float16 hh = (_Float16)x;
        float res = x - (float)hh;
        if (!isfinite(res)) res = 0.f;
        hi[i] = hh;
        lo[i] = (_Float16)res;
      }
      o[r + 32 * h] = __builtin_bit_cast(uint4, hi);
      o[64 + r + 32 * h] = __builtin_bit_cast(uint4, lo);
    }
  };
  float mx = 0.f;
  if constexpr (UL > 0) {
    float v[UL][16];
#pragma unroll
    for (int j = 0; j < UL; j++) {
      if (u0 + 64 * j < units) {
        load16(u0 + 64 * j, v[j]);
      } else {
#pragma unroll
        for (int i = 0; i < 16; i++) v[j][i] = 0.f;
      }
    }
#pragma unroll
    for (int j = 0; j < UL; j++)
#pragma unroll
      for (int i = 0; i < 16; i++) {
        const float x = fabsf(v[j][i]);
        mx = x < INFINITY ? fmaxf(mx, x) : mx;  // finite values only
      }
    const int e = row_exponent(mx);
#pragma unroll
    for (int j = 0; j < UL; j++)
      if (u0 + 64 * j < units) split(u0 + 64 * j, v[j], e);
  } else {
    for (int u = u0; u < units; u += 64) {
      float v[16];
      load16(u, v);
#pragma unroll
      for (int i = 0; i < 16; i++) {
        const float x = fabsf(v[i]);
        mx = x < INFINITY ? fmaxf(mx, x) : mx;
      }
    }
    const int e = row_exponent(mx);
    for (int u = u0; u < units; u += 64) {
      float v[16];
      load16(u, v);
      split(u, v, e);
    }
  }
}

// ---------------------------------------------------------- decode GEMV

// Up to GMAX weights that share K, block size, zero-point kind and the input
// activations, launched together (q/k/v or gate/up of a decoder layer): the
// grid's column groups are the concatenation of the members' column groups,
// and each workgroup picks its member from the running totals cg_end.
struct GemvSet {
  const uint4 *wq[GMAX];
  const float *scales[GMAX];
  const uint8_t *zp4[GMAX];
  const float *zpf[GMAX];
  const float *bias[GMAX];
  float *y[GMAX];
  int64_t part_off[GMAX];  // split-K partials of member m: part + part_off[m] + split * M * N
  int N[GMAX];
  int cg_end[GMAX];
  int n;
};

// Member of workgroup x and its local column group (workgroup-uniform).
__device__ inline int gemv_member(const GemvSet &gs, int x, int *cg) {
  int m = 0;
  while (m + 1 < gs.n && x >= gs.cg_end[m]) m++;
  *cg = x - (m ? gs.cg_end[m - 1] : 0);
  return m;
}


// MR activation rows (M <= 4); QPG = quantisation blocks per k group
// (128 / min(bs, 128)); ZPK = zero-point kind; PF = k groups of loads each
// wave keeps in flight (4 with 4 waves per workgroup, 2 with up to 16).  One
// workgroup per column group (64 columns, one per lane); its NW = blockDim /
// 64 waves split K, wave w taking k groups w, w + NW, ...  Packed codes are
// read once, with non-temporal loads (they stream past the caches).  The
// activations are handled in chunks of kc k groups (one chunk unless M * K is
// large):
//
// Phase 0: each wave issues the loads of its first PF k groups of packed
// codes, scales and zero points, so HBM is busy while phase 1 runs.
// Phase 1: the workgroup quantises the chunk of the activations into LDS:
// per (row, qblock of qb = min(bs, 128) k) the step alpha = max|a| / FIX_MAX
// (NaN when the block holds a non-finite value), fix = rint(a / alpha)
// clamped to +-FIX_MAX and split into four balanced signed int4 digits
// (fix = sum_d 16^d dig_d, dig_d in [-8, 7]) packed 8 per dword in the nibble
// order of wq: sdig[r][l][g][j][d]; srsum = sum of fix over the qblock.
// Thread per (row, k group, 8-k octet o = 4j + g); a qblock is 16 / QPG
// consecutive lanes.
// Phase 2: v_dot8_i32_i4 multiplies (q - 8) with each digit plane (digits are
// wave-uniform LDS broadcasts) and per block
//   y += alpha * s * (sum_d 16^d D_d + (8 - zp) * rsum),
// keeping PF k groups of loads in flight ahead of the arithmetic.
// Phase 3: the NW per-wave sums are added in wave order through LDS
// (deterministic), plus the bias, and written to y.

// Packed codes, scales and zero points of one k group of one column group.
template <int QPG, int ZPK>
struct GemvSlot {
  uint4 w[4];
  float s[QPG];
  uint32_t z[(QPG + 1) / 2];
  float zf[QPG];
};

// Loads of k group kg of the column group whose packed codes start at wp and
// whose scale / zero-point columns start at sp / zq / zfp (lane's column).
template <int QPG, int ZPK>
__device__ inline void gemv_issue(GemvSlot<QPG, ZPK> &sl, const uint4 *wp, const float *sp,
                                  const uint8_t *zq, const float *zfp, int kg, int nb,
                                  int lbs) {
#pragma unroll
  for (int g = 0; g < 4; g++)
    sl.w[g] = __builtin_bit_cast(
        uint4, __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(wp + kg * 256 + g * 64)));
#pragma unroll
  for (int s = 0; s < QPG; s++) {
    const int b = min((kg * KGRP + s * (KGRP / QPG)) >> lbs, nb - 1);
    sl.s[s] = sp[(int64_t)b * 64];
    if (ZPK == 2) sl.zf[s] = zfp[(int64_t)b * 64];
  }
  if (ZPK == 1) {
#pragma unroll
    for (int h = 0; h < (QPG + 1) / 2; h++) {
      const int b = min((kg * KGRP + 2 * h * (KGRP / QPG)) >> lbs, nb - 1);
      sl.z[h] = zq[(int64_t)(b >> 1) * 64];
    }
  }
}

// Phase 1, one task (row r, k group slot l, 8-k octet o): the activation
// loads, then the digits into LDS.  The loads are branch-free (addresses
// clamped into the row, values outside it replaced by 0 afterwards), so a
// caller can keep several tasks' loads in flight.  VEC: K % 4 == 0 and
// 16-byte rows (two float4 loads).
template <bool VEC>
__device__ inline void gemv_digits_load(const float *__restrict__ a, int64_t K, int c0, int nk,
                                        int task, float (&v)[8]) {
  const int o = task & 15, rl = task >> 4;
  const int l = rl % nk, r = rl / nk;
  const int64_t k0 = (int64_t)(c0 + l) * KGRP + 8 * o;
  const float *ar = a + (int64_t)r * K;
  if constexpr (VEC) {
    const bool ok0 = k0 + 4 <= K, ok1 = k0 + 8 <= K;
    const float4 x0 = *reinterpret_cast<const float4 *>(ar + (ok0 ? k0 : 0));
    const float4 x1 = *reinterpret_cast<const float4 *>(ar + (ok1 ? k0 + 4 : 0));
    v[0] = x0.x; v[1] = x0.y; v[2] = x0.z; v[3] = x0.w;
    v[4] = x1.x; v[5] = x1.y; v[6] = x1.z; v[7] = x1.w;
  } else {
#pragma unroll
    for (int i = 0; i < 8; i++) v[i] = ar[min(k0 + i, K - 1)];
  }
}

// Zeroes the values of a task's loads that lie past the end of the row
// (VEC: by float4; K % 4 == 0 there).
__device__ inline void gemv_digits_mask(int64_t K, int c0, int nk, int task, float (&v)[8]) {
  const int o = task & 15, l = (task >> 4) % nk;
  const int64_t k0 = (int64_t)(c0 + l) * KGRP + 8 * o;
#pragma unroll
  for (int i = 0; i < 8; i++)
    if (k0 + i >= K) v[i] = 0.f;
}

template <int QPG>
__device__ inline void gemv_digits_put(const float (&v)[8], int nk, int kc, int task,
                                       uint32_t *sdig, float *salpha, int *srsum) {
  constexpr int G = 16 / QPG;  // octets per qblock
  const int o = task & 15, rl = task >> 4;
  const int l = rl % nk, r = rl / nk;
  float mx = 0.f;
  int bad = 0;
#pragma unroll
  for (int i = 0; i < 8; i++) {
    if (!isfinite(v[i])) bad = 1;
    mx = fmaxf(mx, fabsf(v[i]));
  }
#pragma unroll
  for (int off = 1; off < G; off <<= 1) {
    mx = fmaxf(mx, __shfl_xor(mx, off));
    bad |= __shfl_xor(bad, off);
  }
  const float inv = (mx > 0.f && !bad) ? (float)FIX_MAX / mx : 0.f;
  int rs = 0;
  uint32_t dg[4] = {0u, 0u, 0u, 0u};
#pragma unroll
  for (int i = 0; i < 8; i++) {
    int fix = (int)rintf(v[i] * inv);
    fix = min(max(fix, -FIX_MAX), FIX_MAX);
    rs += fix;
    const int pos = nib_pos(i);
    int x = fix;
#pragma unroll
    for (int d = 0; d < 4; d++) {
      const int di = ((x + 8) & 15) - 8;
      x = (x - di) >> 4;
      dg[d] |= (uint32_t)(di & 15) << (4 * pos);
    }
  }
#pragma unroll
  for (int off = 1; off < G; off <<= 1) rs += __shfl_xor(rs, off);
  const int j = o >> 2, g = o & 3;
  *reinterpret_cast<uint4 *>(&sdig[((r * kc + l) * 4 + g) * 16 + j * 4]) =
      make_uint4(dg[0], dg[1], dg[2], dg[3]);
  if (o % G == 0) {
    const int q = (r * kc + l) * QPG + o / G;
    salpha[q] = bad ? __builtin_nanf("") : (mx > 0.f ? mx / (float)FIX_MAX : 0.f);
    srsum[q] = rs;
  }
}

// Phase 1 for k groups [c0, c0 + nk) into LDS slots l = 0 .. nk - 1 (kc slots
// per row), by nthr threads.  Tasks are 16 consecutive lanes per (row, k
// group), so the shuffles inside a qblock see only active lanes.
template <int MR, int QPG>
__device__ inline void gemv_digits(const float *__restrict__ a, int64_t K, int vec, int c0,
                                   int nk, int kc, uint32_t *sdig, float *salpha, int *srsum,
                                   int t, int nthr) {
  const int ntask = MR * nk * 16;
  for (int task = t; task < ntask; task += nthr) {
    float v[8];
    if (vec) gemv_digits_load<true>(a, K, c0, nk, task, v);
    else gemv_digits_load<false>(a, K, c0, nk, task, v);
    gemv_digits_mask(K, c0, nk, task, v);
    gemv_digits_put<QPG>(v, nk, kc, task, sdig, salpha, srsum);
  }
}

// The float arithmetic of one (row, block) term, shared by every M <= 4
// GEMV kernel so that all of them round alike: the block's integer sum comb
// (sum over its k of activation fixed point times q - 8) plus the zero-point
// correction, then y = fma(alpha * scale, v, y) in k order.
template <int ZPK>
__device__ inline float gemv_block_value(int comb, int zc, int R, float zf) {
  if (ZPK == 2) return __builtin_fmaf(8.f - zf, (float)R, (float)comb);
  return (float)(comb + zc * R);
}
__device__ inline float gemv_term(float y, float p, float v) { return __builtin_fmaf(p, v, y); }

// Phase 2 for one k group kg (LDS slot l) held in sl: yacc[r] += its share.
template <int MR, int QPG, int ZPK>
__device__ inline void gemv_kgroup(const GemvSlot<QPG, ZPK> &sl, int kg, int l, int kc, int nb,
                                   int lbs, const uint32_t *sdig, const float *salpha,
                                   const int *srsum, float (&yacc)[MR]) {
  uint32_t wv[4][4];
#pragma unroll
  for (int g = 0; g < 4; g++) {
    wv[g][0] = sl.w[g].x ^ 0x88888888u; wv[g][1] = sl.w[g].y ^ 0x88888888u;
    wv[g][2] = sl.w[g].z ^ 0x88888888u; wv[g][3] = sl.w[g].w ^ 0x88888888u;
  }
  // One quantisation block at a time: dword (g, j) holds k = 32j + 8g + t,
  // so block s covers j in [4s/QPG, 4(s+1)/QPG) for QPG <= 4 and, for
  // QPG = 8, j = s/2 with g in {2(s%2), 2(s%2) + 1}.
#pragma unroll
  for (int s = 0; s < QPG; s++) {
    int acc[MR][4];
#pragma unroll
    for (int r = 0; r < MR; r++)
#pragma unroll
      for (int d = 0; d < 4; d++) acc[r][d] = 0;
#pragma unroll
    for (int g = 0; g < 4; g++)
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const bool mine = QPG == 8 ? (j == s / 2 && g / 2 == s % 2) : (j * QPG / 4 == s);
        if (!mine) continue;
        const int x = (int)wv[g][j];
#pragma unroll
        for (int r = 0; r < MR; r++) {
          const uint4 dd =
              *reinterpret_cast<const uint4 *>(&sdig[((r * kc + l) * 4 + g) * 16 + j * 4]);
          acc[r][0] = __builtin_amdgcn_sdot8((int)dd.x, x, acc[r][0], false);
          acc[r][1] = __builtin_amdgcn_sdot8((int)dd.y, x, acc[r][1], false);
          acc[r][2] = __builtin_amdgcn_sdot8((int)dd.z, x, acc[r][2], false);
          acc[r][3] = __builtin_amdgcn_sdot8((int)dd.w, x, acc[r][3], false);
        }
      }
    const int b = (kg * KGRP + s * (KGRP / QPG)) >> lbs;
    if (b >= nb) continue;  // k padding beyond the last block
    int zc = 0;
    if (ZPK == 1) {
      // Zero-point byte h of this k group holds blocks 2h (low) and 2h+1.
      const uint32_t zb = sl.z[QPG == 1 ? 0 : s / 2];
      zc = 8 - (int)((b & 1) ? (zb >> 4) : (zb & 15));
    }
#pragma unroll
    for (int r = 0; r < MR; r++) {
      const int comb = ((acc[r][3] * 16 + acc[r][2]) * 16 + acc[r][1]) * 16 + acc[r][0];
      const int q = (r * kc + l) * QPG + s;
      const float al = salpha[q];
      const int R = srsum[q];
      yacc[r] = gemv_term(yacc[r], al * sl.s[s], gemv_block_value<ZPK>(comb, zc, R, sl.zf[s]));
    }
  }
}

template <int MR, int QPG, int ZPK, int PF>
__global__ __launch_bounds__(PF == 4 ? 256 : 1024) void k_gemv_dot8(
    const float *__restrict__ a, int64_t K, int vec, const GemvSet gs, int c4, int nb,
    int nbh, int lbs, int kc, int kps, float *__restrict__ part) {
  extern __shared__ uint32_t smem[];
  uint32_t *sdig = smem;                                            // [MR][kc][64]
  float *salpha = reinterpret_cast<float *>(smem + MR * kc * 64);   // [MR][kc][QPG]
  int *srsum = reinterpret_cast<int *>(salpha + MR * kc * QPG);     // [MR][kc][QPG]
  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int NW = blockDim.x >> 6;
  const int nthr = blockDim.x;
  int cg;
  const int gm = gemv_member(gs, blockIdx.x, &cg);
  float *__restrict__ y = gs.y[gm];
  const float *__restrict__ bias = gs.bias[gm];
  const int N = gs.N[gm];

  const uint4 *wp = gs.wq[gm] + (int64_t)cg * c4 * 256 + lane;
  const float *sp = gs.scales[gm] + (int64_t)cg * nb * 64 + sz_pos(lane);
  const uint8_t *zq = gs.zp4[gm] + (int64_t)cg * nbh * 64 + sz_pos(lane);
  const float *zfp = gs.zpf[gm] + (int64_t)cg * nb * 64 + sz_pos(lane);
  GemvSlot<QPG, ZPK> ring[PF];
  // Split-K (gridDim.y > 1): this workgroup takes k groups [kb, kb + cs)
  // and writes its sum, without the bias, to the split's partials.
  const int kb = (int)blockIdx.y * kps;
  const int cs = min(kps, c4 - kb);
  // This wave's k groups: kb + wave, kb + wave + NW, ...; the n-th is
  // kb + wave + n * NW.
  const int nmine = wave < cs ? (cs - wave + NW - 1) / NW : 0;

  // Phase 0.  (Issuing the activation loads ahead of these, so that the
  // digits wait for them alone, measured slower here: 5.2 -> 6.1 us on a
  // 2048 x 512 weight, 31 -> 38 us on the 2048 x 128256 lm_head.)
#pragma unroll
  for (int i = 0; i < PF; i++)
    if (i < nmine) gemv_issue(ring[i], wp, sp, zq, zfp, kb + wave + i * NW, nb, lbs);

  float yacc[MR];
#pragma unroll
  for (int r = 0; r < MR; r++) yacc[r] = 0.f;
  // kc is c4 (one chunk) or a multiple of PF * NW, so every chunk starts at a
  // multiple of PF of this wave's k groups and ring slots stay static.
  for (int c0 = 0; c0 < cs; c0 += kc) {
    const int nk = min(cs, c0 + kc) - c0;
    if (c0 > 0) __syncthreads();  // previous chunk's digits fully consumed
    // Phase 1.
    gemv_digits<MR, QPG>(a, K, vec, kb + c0, nk, kc, sdig, salpha, srsum, t, nthr);
    __syncthreads();

    // Phase 2: this wave's k groups inside the chunk.  The ring slot of the
    // n-th k group is n % PF; the loop is unrolled by PF so slots are static.
    const int nend = min(nmine, (c0 + nk - wave + NW - 1) / NW);
    for (int n = c0 / NW; n < nend; n += PF) {
#pragma unroll
      for (int i = 0; i < PF; i++) {
        const int nn = n + i;
        if (nn >= nend) break;
        const int kl = wave + nn * NW;  // within the split
        const GemvSlot<QPG, ZPK> cur = ring[i];
        if (nn + PF < nmine)
          gemv_issue(ring[i], wp, sp, zq, zfp, kb + wave + (nn + PF) * NW, nb, lbs);
        gemv_kgroup<MR, QPG, ZPK>(cur, kb + kl, kl - c0, kc, nb, lbs, sdig, salpha, srsum, yacc);
      }
    }
  }

  // Phase 3.
  __syncthreads();  // all waves are done with the digits; reuse LDS
  float *red = reinterpret_cast<float *>(smem);  // [NW][MR][64]
#pragma unroll
  for (int r = 0; r < MR; r++) red[(wave * MR + r) * 64 + lane] = yacc[r];
  __syncthreads();
  if (wave == 0) {
    const int col = cg * 64 + lane;
#pragma unroll
    for (int r = 0; r < MR; r++) {
      // All NW wave sums are read before the ordered adds, so the LDS reads
      // overlap (NW <= 16; the launch bounds allow no more).
      float wsum[16];
#pragma unroll
      for (int w = 0; w < 16; w++) wsum[w] = w < NW ? red[(w * MR + r) * 64 + lane] : 0.f;
      float s = wsum[0];
#pragma unroll
      for (int w = 1; w < 16; w++)
        if (w < NW) s += wsum[w];
      if (col >= N) continue;
      if (part)
        part[gs.part_off[gm] + ((int64_t)blockIdx.y * MR + r) * N + col] = s;
      else
        y[(int64_t)r * N + col] = s + (bias ? bias[col] : 0.f);
    }
  }
}

// Persistent form for wide weights whose k groups split evenly over 4 waves
// (c4 = 4 * PF, PF = 1 or 2): the activation digits of all k groups are made once per
// workgroup, which then takes column groups blockIdx.x, + gridDim.x, ...;
// wave w owns k groups w + 4i, i < PF, of each, and refills ring slot i with
// the next column group's k group as soon as it has copied the current one,
// so the stream of packed codes continues across column groups.  Per column
// group the four wave sums meet in LDS (double-buffered, one barrier) and
// wave 0 adds them in wave order and stores: results are bitwise those of
// k_gemv_dot8.
template <int MR, int QPG, int ZPK, int PF>
__global__ __launch_bounds__(256) void k_gemv_dot8p(
    const float *__restrict__ a, int64_t K, int vec, const GemvSet gs, int c4, int nb,
    int nbh, int lbs) {
  extern __shared__ uint32_t smem[];
  uint32_t *sdig = smem;                                            // [MR][c4][64]
  float *salpha = reinterpret_cast<float *>(smem + MR * c4 * 64);   // [MR][c4][QPG]
  int *srsum = reinterpret_cast<int *>(salpha + MR * c4 * QPG);     // [MR][c4][QPG]
  float *red = reinterpret_cast<float *>(srsum + MR * c4 * QPG);    // [2][4][MR][64]
  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int ncg = gs.cg_end[gs.n - 1];
  GemvSlot<QPG, ZPK> ring[PF];
  auto issue_cg = [&](int x) {
    int cg;
    const int gm = gemv_member(gs, x, &cg);
    const uint4 *wp = gs.wq[gm] + (int64_t)cg * c4 * 256 + lane;
    const float *sp = gs.scales[gm] + (int64_t)cg * nb * 64 + sz_pos(lane);
    const uint8_t *zq = gs.zp4[gm] + (int64_t)cg * nbh * 64 + sz_pos(lane);
    const float *zfp = gs.zpf[gm] + (int64_t)cg * nb * 64 + sz_pos(lane);
#pragma unroll
    for (int i = 0; i < PF; i++) gemv_issue(ring[i], wp, sp, zq, zfp, wave + 4 * i, nb, lbs);
  };
  if ((int)blockIdx.x < ncg) issue_cg(blockIdx.x);
  gemv_digits<MR, QPG>(a, K, vec, 0, c4, c4, sdig, salpha, srsum, t, 256);
  __syncthreads();
  int it = 0;
  for (int x = blockIdx.x; x < ncg; x += gridDim.x, it++) {
    float yacc[MR];
#pragma unroll
    for (int r = 0; r < MR; r++) yacc[r] = 0.f;
    const int nx = x + gridDim.x;
    GemvSlot<QPG, ZPK> cur[PF];
#pragma unroll
    for (int i = 0; i < PF; i++) cur[i] = ring[i];
    if (nx < ncg) issue_cg(nx);
#pragma unroll
    for (int i = 0; i < PF; i++) {
      const int kg = wave + 4 * i;
      gemv_kgroup<MR, QPG, ZPK>(cur[i], kg, kg, c4, nb, lbs, sdig, salpha, srsum, yacc);
    }
    float *rb = red + (it & 1) * (4 * MR * 64);
#pragma unroll
    for (int r = 0; r < MR; r++) rb[(wave * MR + r) * 64 + lane] = yacc[r];
    __syncthreads();
    if (wave == 0) {
      int cg;
      const int gm = gemv_member(gs, x, &cg);
      const int col = cg * 64 + lane;
      const float *bias = gs.bias[gm];
#pragma unroll
      for (int r = 0; r < MR; r++) {
        float s = rb[r * 64 + lane];
        for (int w = 1; w < 4; w++) s += rb[(w * MR + r) * 64 + lane];
        if (col < gs.N[gm]) gs.y[gm][(int64_t)r * gs.N[gm] + col] = s + (bias ? bias[col] : 0.f);
      }
    }
  }
}

// Column-slice form for one row, narrow weights and block_size >= 128 (one
// quantisation block per k group): a workgroup takes 16 columns (a quarter
// of a column group) over all of K, so a weight spreads over four times the
// workgroups of k_gemv_dot8 and each CU streams a quarter of the bytes.
// Lane l works on column cl = 16 (x % 4) + l % 16 and octet g = l / 16 of
// every k group: its packed uint4 is 16 bytes of a 256-byte run (16 columns
// of one octet), so each wave reads whole lines.  Wave w takes k groups w,
// w + 4, ... (those of wave w in k_gemv_dot8 with four waves), PF of them in
// flight.  Per k group the lanes' integer sums over their octet are added
// over the four octets with shuffles (exact), so every lane holds the
// block's integer sum for its column and runs the same float chain over k
// groups as k_gemv_dot8's lane for that column; the four wave sums are added
// in wave order.  Results are bitwise those of k_gemv_dot8 (four waves) and
// k_gemv_dot8p.  (With smaller blocks the per-block scale and zero-point
// loads of 16 columns cost more than the wider spread gains.)
constexpr int CS_TASKS = 4;  // digits tasks per thread: K <= 64 k groups

template <int ZPK>
struct CsSlot {
  uint4 w;
  float s;
  uint32_t z;
  float zf;
};

template <int ZPK, int PF, bool VEC>
__global__ __launch_bounds__(256) void k_gemv_cs(const float *__restrict__ a, int64_t K,
                                                 const GemvSet gs, int c4, int nb, int nbh,
                                                 int lbs) {
  extern __shared__ uint32_t smem[];
  uint32_t *sdig = smem;                                       // [c4][64]
  float *salpha = reinterpret_cast<float *>(smem + c4 * 64);   // [c4]
  int *srsum = reinterpret_cast<int *>(salpha + c4);           // [c4]
  const int t = threadIdx.x;
  const int lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int g = lane >> 4, c = lane & 15;
  int cg;
  const int gm = gemv_member(gs, (int)(blockIdx.x >> 2), &cg);
  const int cl = (int)(blockIdx.x & 3) * 16 + c;
  const uint4 *wp = gs.wq[gm] + (int64_t)cg * c4 * 256 + g * 64 + cl;
  const float *sp = gs.scales[gm] + (int64_t)cg * nb * 64 + sz_pos(cl);
  const uint8_t *zq = gs.zp4[gm] + (int64_t)cg * nbh * 64 + sz_pos(cl);
  const float *zfp = gs.zpf[gm] + (int64_t)cg * nb * 64 + sz_pos(cl);

  auto issue = [&](CsSlot<ZPK> &sl, int kg) {
    sl.w = __builtin_bit_cast(
        uint4, __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(wp + kg * 256)));
    const int b = min((kg * KGRP) >> lbs, nb - 1);
    sl.s = sp[(int64_t)b * 64];
    if (ZPK == 1) sl.z = zq[(int64_t)(b >> 1) * 64];
    if (ZPK == 2) sl.zf = zfp[(int64_t)b * 64];
  };

  // The activation loads go first: the vector memory counter retires loads
  // in issue order, so the digits then wait for them alone.  Tasks: k group
  // slot l, octet o (at most CS_TASKS per thread: c4 <= 16 * CS_TASKS).
  const int ntask = c4 * 16;
  float av[CS_TASKS][8];
#pragma unroll
  for (int i = 0; i < CS_TASKS; i++)
    gemv_digits_load<VEC>(a, K, 0, c4, min(t + 256 * i, ntask - 1), av[i]);
  __builtin_amdgcn_sched_barrier(0);  // keep the issue order: activations, weights
  // This wave's k groups are wave + 4 n, n < nk; the loads of the n-th sit
  // in ring slot n % PF.  Loads are issued in straight-line code (addresses
  // clamped to the last k group where a slot has nothing left to take), so
  // the wait before each slot's use counts exactly the loads issued after it.
  const int nk = (c4 - wave + 3) / 4;  // 0 for waves past c4 < 4
  const int niter = (c4 + 3) / 4;      // nk of wave 0, the largest
  auto kg_at = [&](int n) { return min(wave + 4 * n, c4 - 1); };
  CsSlot<ZPK> ring[PF];
#pragma unroll
  for (int i = 0; i < PF; i++) issue(ring[i], kg_at(i));
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int i = 0; i < CS_TASKS; i++)
    if (t + 256 * i < ntask) {
      gemv_digits_mask(K, 0, c4, t + 256 * i, av[i]);
      gemv_digits_put<1>(av[i], c4, c4, t + 256 * i, sdig, salpha, srsum);
    }
  __syncthreads();

  float y = 0.f;
  auto kgroup = [&](const CsSlot<ZPK> &cur, int kg) {
    // Integer sum over dword j (k = 32 j + 8 g + 0..7) and the four digit
    // planes, then over the four octets (lanes c, c + 16, c + 32, c + 48).
    const uint32_t wv[4] = {cur.w.x ^ 0x88888888u, cur.w.y ^ 0x88888888u,
                            cur.w.z ^ 0x88888888u, cur.w.w ^ 0x88888888u};
    int v = 0;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const uint4 dd = *reinterpret_cast<const uint4 *>(&sdig[(kg * 4 + g) * 16 + j * 4]);
      const int a0 = __builtin_amdgcn_sdot8((int)dd.x, (int)wv[j], 0, false);
      const int a1 = __builtin_amdgcn_sdot8((int)dd.y, (int)wv[j], 0, false);
      const int a2 = __builtin_amdgcn_sdot8((int)dd.z, (int)wv[j], 0, false);
      const int a3 = __builtin_amdgcn_sdot8((int)dd.w, (int)wv[j], 0, false);
      v += ((a3 * 16 + a2) * 16 + a1) * 16 + a0;
    }
    v += __shfl_xor(v, 16);
    v += __shfl_xor(v, 32);
    const int b = (kg * KGRP) >> lbs;
    if (b >= nb) return;  // k padding beyond the last block
    int zc = 0;
    if (ZPK == 1) zc = 8 - (int)((b & 1) ? (cur.z >> 4) : (cur.z & 15));
    y = gemv_term(y, salpha[kg] * cur.s, gemv_block_value<ZPK>(v, zc, srsum[kg], cur.zf));
  };
  for (int n = 0; n < niter; n += PF) {
    if (n + PF < niter) {
#pragma unroll
      for (int i = 0; i < PF; i++) {
        const CsSlot<ZPK> cur = ring[i];
        issue(ring[i], kg_at(n + i + PF));
        if (n + i < nk) kgroup(cur, wave + 4 * (n + i));
      }
    } else {
#pragma unroll
      for (int i = 0; i < PF; i++)
        if (n + i < nk) kgroup(ring[i], wave + 4 * (n + i));
    }
  }
  __syncthreads();  // every wave is done with the digits; reuse LDS
  float *red = reinterpret_cast<float *>(smem);  // [4][16]
  if (g == 0) red[wave * 16 + c] = y;
  __syncthreads();
  if (wave == 0 && g == 0) {
    float s = red[c];
    s += red[16 + c];
    s += red[32 + c];
    s += red[48 + c];
    const int col = cg * 64 + cl;
    const float *bias = gs.bias[gm];
    if (col < gs.N[gm]) gs.y[gm][col] = s + (bias ? bias[col] : 0.f);
  }
}

// --------------------------------------------------------- prefill GEMM

// Workgroup tile: 128 rows x 32*NT columns (NT/2 column groups), 4 waves;
// wave w owns rows [32*w, +32) of the tile and all its columns (NT MFMA tiles
// of 32x32, v_mfma_f32_32x32x16_f16).  NT = 4 for wide weights; NT = 2 halves
// the tile so that narrow weights still give enough workgroups without
// splitting K.  Per k group (128 k = 8 steps of 16 k):
//   * the workgroup dequantises the 128 x 32*NT weight tile once into LDS, in
//     MFMA B-fragment order (double-buffered; the next k group's packed codes
//     are loaded at the start of the current one and unpacked step by step
//     between its MFMAs);
//   * each wave streams its activation fragments (hi and lo) from global, PD
//     steps ahead of use, into a per-segment fp32 accumulator D;
//   * at the end of each scale segment (SEGJ 32-k quarters = min(block_size,
//     128) k) the block scale is applied: acc += s * D.
// The epilogue applies the row factor 2^-e, restages each wave's 32-row tile
// through LDS and writes Y (or the split-K partials) as 16-byte,
// row-contiguous, non-temporal stores.
// Grid: x = tiles in XCD-aware order (workgroup L runs on XCD L % 8; all row
// tiles of one column tile get the same L % 8, so its weights are read from
// HBM once into that XCD's L2); y = k splits, each over kps k groups, whose
// partial sums go to the partials and are added by k_gemm_reduce (ksplit > 1).
template <int SEGJ, int NT>
__global__ __launch_bounds__(256, NT == 4 ? 2 : 3) void k_gemm_f16split(
    const uint4 *__restrict__ ahl, const int *__restrict__ texp, const PrefillSet ps,
    float *__restrict__ part, int M, int c4n, int nb, int nbh, int lbs, int has_zp,
    int mtiles, int ntiles, int kps) {
  constexpr int PH = NT / 2;                 // column groups per tile
  constexpr int TC = 32 * NT;                // tile columns
  __shared__ uint4 bl[2][NT * 8 * 64];       // [buf][n32][step][lane] fp16 x 8
  __shared__ float scl[2][4][32][4];         // [buf][segment][col % 32][n32]
  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int L = blockIdx.x;
  const int xcd = L & 7, q = L >> 3;
  const int mt = q % mtiles;
  const int ntg = (q / mtiles) * 8 + xcd;
  if (ntg >= ntiles) return;
  int nt;
  const int mem = prefill_member(ps, ntg, &nt);
  const uint4 *__restrict__ wq = ps.wq[mem];
  const float *__restrict__ scales = ps.scales[mem];
  const uint8_t *__restrict__ zp4 = ps.zp4[mem];
  const float *__restrict__ bias = ps.bias[mem];
  const int N = ps.N[mem];
  const int ks = blockIdx.y;
  const int kg0 = ks * kps;
  const int kg1 = min(c4n, kg0 + kps);
  const int m32 = mt * 4 + wave;  // this wave's 32-row subtile
  const int lc = lane & 31, lh = lane >> 5;

  // Cooperative dequantisation of the 256*PH packed uint4 of a k group:
  // thread t handles u = t + 256 h, h < PH -> (column group PH*nt + h,
  // g = wave, col = lane); its dword j (k = 32j + 8g .. +7) is MFMA step
  // 2j + g/2, half g%2.  The thread with g = s also stages the column's scale
  // of segment s (threads with g >= segments per k group write an unused
  // slot).
  const int dq_g = wave;
  int dq_cgi[PH], dq_col[PH], dq_dst[PH], dq_c[PH];
#pragma unroll
  for (int h = 0; h < PH; h++) {
    const int u = t + 256 * h;
    dq_cgi[h] = PH * nt + h;  // u >> 8 == h (t < 256), written so it is seen as uniform
    dq_col[h] = u & 63;
    dq_c[h] = (u >> 8) * 64 + dq_col[h];  // column within the tile
    const int n32 = dq_c[h] >> 5;
    dq_dst[h] = (n32 * 8 + (dq_g >> 1)) * 64 + (dq_c[h] & 31) + 32 * (dq_g & 1);
  }
  const int nbm1 = nb - 1, nbhm1 = nbh - 1;
  // Weight tables and activations are read with raw buffer loads: a
  // wave-uniform resource (the column group's, or the wave's 32-row tile's,
  // base), a fixed per-lane byte offset and a uniform offset, so no per-lane
  // 64-bit address arithmetic is needed.  All offsets stay inside the tensors.
  auto rsrc = [](const void *base) __attribute__((always_inline)) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, 0x7ffffff0,
                                             0x00020000);
  };
  __amdgpu_buffer_rsrc_t r_wq[PH], r_zp[PH], r_sc[PH];
#pragma unroll
  for (int h = 0; h < PH; h++) {
    const int64_t cgi = dq_cgi[h];
    r_wq[h] = rsrc(wq + cgi * c4n * 256);
    r_zp[h] = rsrc(zp4 + cgi * nbh * 64);
    r_sc[h] = rsrc(scales + cgi * nb * 64);
  }
  const unsigned vo16 = 16u * lane;                   // this lane's uint4
  const unsigned vo_zp = (unsigned)sz_pos(lane);      // dq_col[h] == lane for every h
  const unsigned vo_sc = 4u * vo_zp;
  // Dequantisation masks held in VGPRs so that each pair is one v_and_or_b32
  // (VOP3 takes no literal operands here).
  uint32_t v_mlo, v_mhi, v_magic;
  asm volatile("v_mov_b32 %0, %1" : "=v"(v_mlo) : "s"(0x000F000Fu));
  asm volatile("v_mov_b32 %0, %1" : "=v"(v_mhi) : "s"(0x00F000F0u));
  asm volatile("v_mov_b32 %0, %1" : "=v"(v_magic) : "s"(0x64006400u));
  struct Meta {
    uint4 pk[PH];
    uint32_t zb[PH], zb2[PH];  // zero-point bytes of the k group's first two byte slots
    float sc[PH];
    uint32_t z1[PH], z16[PH];  // dequantisation constants (SEGJ == 4: one block per k group)
  };
  // Branch-free: indices are clamped; blocks past the last (k padding) get a
  // zero scale when the scale is staged.
  auto load_meta = [&](int kg, Meta &m) {
    const int blk0 = (kg * KGRP) >> lbs;
    const int blks = (kg * KGRP + 32 * SEGJ * dq_g) >> lbs;
    const int zbyte0 = min(blk0 / 2, nbhm1), zbyte1 = min(blk0 / 2 + 1, nbhm1);
#pragma unroll
    for (int h = 0; h < PH; h++) {
      m.pk[h] = __builtin_bit_cast(
          uint4, __builtin_amdgcn_raw_buffer_load_b128(r_wq[h], vo16, (kg * 4 + dq_g) * 1024, 0));
      m.zb[h] = __builtin_amdgcn_raw_buffer_load_b8(r_zp[h], vo_zp, zbyte0 * 64, 0);
      m.zb2[h] = SEGJ == 1 ? __builtin_amdgcn_raw_buffer_load_b8(r_zp[h], vo_zp, zbyte1 * 64, 0)
                           : 0u;
      m.sc[h] = __builtin_bit_cast(
          float, __builtin_amdgcn_raw_buffer_load_b32(r_sc[h], vo_sc, min(blks, nbm1) * 256, 0));
    }
  };
  // Dequantises dword j (32-k quarter j) of the packed uint4 into buffer buf.
  auto dequant_quarter = [&](int kg, Meta &m, int buf, int j) {
    const int blk0 = (kg * KGRP) >> lbs;
    const int blk = (kg * KGRP + 32 * j) >> lbs;
    const int sh = ((blk & 1) + 2 * (blk / 2 - blk0 / 2)) * 4;
#pragma unroll
    for (int h = 0; h < PH; h++) {
      // Loaded values are first touched here (empty asm): arithmetic on them
      // would otherwise be hoisted next to the loads and wait on them there.
      uint32_t w = j == 0 ? m.pk[h].x : j == 1 ? m.pk[h].y : j == 2 ? m.pk[h].z : m.pk[h].w;
      asm volatile("" : "+v"(w));
      uint32_t z1, z16;
      if (SEGJ < 4 || j == 0) {  // with SEGJ == 4 the block (and z) spans the k group
        uint32_t zb = m.zb[h], zb2 = m.zb2[h];
        asm volatile("" : "+v"(zb), "+v"(zb2));
        zb |= zb2 << 8;
        const uint32_t z = has_zp ? (zb >> sh) & 15u : 8u;
        // -(1024 + z) and -(1024 + 16 z) in fp16 are 0xE400 + z and + 16 z.
        z1 = 0xE400E400u + z * 0x00010001u;
        z16 = 0xE400E400u + z * 0x00100010u;
        m.z1[h] = z1, m.z16[h] = z16;
      } else {
        z1 = m.z1[h], z16 = m.z16[h];
      }
      bl[buf][dq_dst[h] + 2 * j * 64] = deq8(w, v_mlo, v_mhi, v_magic,
                                             __builtin_bit_cast(half2v, z1),
                                             __builtin_bit_cast(half2v, z16));
    }
    if (j == 0) {
      const bool in_range = ((kg * KGRP + 32 * SEGJ * dq_g) >> lbs) < nb;
#pragma unroll
      for (int h = 0; h < PH; h++) {
        float sc = m.sc[h];
        asm volatile("" : "+v"(sc));
        scl[buf][dq_g][dq_c[h] & 31][dq_c[h] >> 5] = in_range ? sc : 0.f;
      }
    }
  };
  // Activation fragment of step s of k group kg: hi at +0, lo at +64 uint4.
  const __amdgpu_buffer_rsrc_t r_a = rsrc(ahl + (int64_t)m32 * c4n * 1024);
  auto a_load = [&](int kg, int st, int part) __attribute__((always_inline)) {
    return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(
                                         r_a, vo16, ((kg * 8 + st) * 128 + 64 * part) * 16, 0));
  };

  // D holds the running scale segment.  With one segment per k group
  // (DEFER), acc += s * D of a finished segment is deferred to the first step
  // of the next one, tile by tile just before the MFMA that restarts D[n], so
  // those FMAs overlap the other tiles' MFMAs instead of stalling on the last
  // ones before the barrier (s_pend: the finished segment's scales; zero
  // before the first segment).  Shorter segments apply it at once (deferring
  // there costs more registers than the tile has).
  constexpr bool DEFER = SEGJ == 4;
  float16v acc[NT], D[NT];
#pragma unroll
  for (int n = 0; n < NT; n++) acc[n] = (float16v){}, D[n] = (float16v){};
  float s_pend[4] = {0.f, 0.f, 0.f, 0.f};
  const float16v zero16 = (float16v){};

  // Ring of activation fragments (slot = step), loaded PD steps ahead.  Loads
  // past the last k group re-read it (results unused).  The next k group's
  // weights, loaded at step 0, are dequantised in steps PD..7.
  constexpr int PD = 4;
  uint4 ah[8], al[8];
#pragma unroll
  for (int ss = 0; ss < PD; ss++) {
    ah[ss] = a_load(kg0, ss, 0);
    al[ss] = a_load(kg0, ss, 1);
  }
  {
    Meta m0;
    load_meta(kg0, m0);
#pragma unroll
    for (int j = 0; j < 4; j++) dequant_quarter(kg0, m0, 0, j);
  }
  __syncthreads();

  for (int kg = kg0; kg < kg1; kg++) {
    const int buf = (kg - kg0) & 1;
    const int kgn = min(kg + 1, kg1 - 1);  // next k group (clamped)
    Meta mnext;
    load_meta(kgn, mnext);
    // Keep the scheduler from sinking these loads towards their use.
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int st = 0; st < 8; st++) {
      {
        const int sn = (st + PD) & 7;
        const int kn = min(kg + ((st + PD) >> 3), kg1 - 1);
        ah[sn] = a_load(kn, sn, 0);
        al[sn] = a_load(kn, sn, 1);
      }
      __builtin_amdgcn_sched_barrier(0);
      const bool seg_start = (st % (2 * SEGJ)) == 0;
      const half8 a_h = __builtin_bit_cast(half8, ah[st]);
      const half8 a_l = __builtin_bit_cast(half8, al[st]);
#pragma unroll
      for (int n = 0; n < NT; n++) {
        const half8 b = __builtin_bit_cast(half8, bl[buf][(n * 8 + st) * 64 + lane]);
        if (DEFER && seg_start) {
#pragma unroll
          for (int v = 0; v < 16; v++) acc[n][v] = fmaf(s_pend[n], D[n][v], acc[n][v]);
        }
        D[n] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a_h, b, seg_start ? zero16 : D[n], 0, 0, 0);
        D[n] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a_l, b, D[n], 0, 0, 0);
      }
      // The next k group's weights, a quarter per step in steps PD..7 (VALU
      // work the scheduler interleaves with these MFMAs).
      if (st >= PD) dequant_quarter(kgn, mnext, buf ^ 1, st - PD);
      if ((st + 1) % (2 * SEGJ) == 0) {
        const float4 s4 = *reinterpret_cast<const float4 *>(&scl[buf][st / (2 * SEGJ)][lc][0]);
        s_pend[0] = s4.x, s_pend[1] = s4.y, s_pend[2] = s4.z, s_pend[3] = s4.w;
        if constexpr (!DEFER) {
#pragma unroll
          for (int n = 0; n < NT; n++)
#pragma unroll
            for (int v = 0; v < 16; v++) acc[n][v] = fmaf(s_pend[n], D[n][v], acc[n][v]);
        }
      }
    }
    __syncthreads();
  }
  if constexpr (DEFER) {
#pragma unroll
    for (int n = 0; n < NT; n++)
#pragma unroll
      for (int v = 0; v < 16; v++) acc[n][v] = fmaf(s_pend[n], D[n][v], acc[n][v]);
  }

  // Epilogue: stage the wave's 32 x TC tile row-major in LDS (the weight
  // buffers are free now; every wave passed the last barrier), then write
  // 16-byte row pieces.
  float *stage = reinterpret_cast<float *>(&bl[0][0]) + wave * (32 * TC);
  // Row exponents of the lane's 16 output rows 8*(v/4) + 4*lh + v%4; the row
  // factor 2^-e is applied with ldexp (exact, and graded into subnormals).
  int4 ex[4];
#pragma unroll
  for (int i = 0; i < 4; i++)
    ex[i] = reinterpret_cast<const int4 *>(texp)[(int64_t)m32 * 8 + 2 * i + lh];
#pragma unroll
  for (int n = 0; n < NT; n++)
#pragma unroll
    for (int v = 0; v < 16; v++) {
      const int r = 8 * (v >> 2) + 4 * lh + (v & 3);
      const int4 e4 = ex[v >> 2];
      const int e = (v & 3) == 0 ? e4.x : (v & 3) == 1 ? e4.y : (v & 3) == 2 ? e4.z : e4.w;
      stage[r * TC + n * 32 + lc] = ldexpf(acc[n][v], -e);
    }
  __syncthreads();
  const bool split = gridDim.y > 1;
  float *dst = split ? part + ps.part_off[mem] + (int64_t)ks * M * N : ps.y[mem];
  // Lane -> (row offset, 4-column piece): a row is 8*NT pieces.
  constexpr int PPR = 8 * NT, RPI = 64 / PPR;  // pieces per row, rows per iteration
  const int c4 = lane % PPR, ro = lane / PPR;
  const int col = nt * TC + 4 * c4;
  float4 bv = make_float4(0.f, 0.f, 0.f, 0.f);
  if (!split && bias) {
    if (col + 3 < N) {
      bv = make_float4(bias[col], bias[col + 1], bias[col + 2], bias[col + 3]);
    } else {
      if (col < N) bv.x = bias[col];
      if (col + 1 < N) bv.y = bias[col + 1];
      if (col + 2 < N) bv.z = bias[col + 2];
    }
  }
  // 16-byte stores need N % 4 == 0 and a 16-byte aligned destination (the
  // partials buffer always is; y is checked by the host).
  const bool vec_ok = (N % 4) == 0 && (split || ps.y_vec[mem]);
#pragma unroll 4
  for (int it = 0; it < 32 / RPI; it++) {
    const int r = RPI * it + ro;
    const int row = m32 * 32 + r;
    float4v v = *reinterpret_cast<const float4v *>(&stage[r * TC + 4 * c4]);
    v[0] += bv.x; v[1] += bv.y; v[2] += bv.z; v[3] += bv.w;
    if (row < M) {
      float *p = dst + (int64_t)row * N + col;
      if (vec_ok && col + 3 < N) {
        __builtin_nontemporal_store(v, reinterpret_cast<float4v *>(p));
      } else {
        if (col < N) p[0] = v[0];
        if (col + 1 < N) p[1] = v[1];
        if (col + 2 < N) p[2] = v[2];
        if (col + 3 < N) p[3] = v[3];
      }
    }
  }
}

// ------------------------------------------------------ decode MFMA GEMV

// Activation prepass of the 16-row MFMA path (3 <= M <= 16): as k_af16split
// (per-row power-of-two exponent e, hi = fp16(x), lo = fp16(x - hi), k offsets
// 2, 3, 6, 7 of every 8 scaled by a further 2^-4) but in the operand order of
// v_mfma_f32_16x16x32_f16: for k group kg and 32-k step j,
// ahl16[((kg * 4 + j) * 2 + h) * 64 + 16 g + r] holds the 8 fp16 (hi for
// h = 0, lo for h = 1) of row r at k = 128 kg + 32 j + 8 g .. +7.  Rows >= M
// and k >= K are zeros.  One workgroup per row (16 rows).  P > 0: the row has
// at most 256 P octets (8 k each, padding included) and thread t reads octets
// t + 256 i (i < P) once, all loads in flight, converting them from registers;
// P = 0 (longer rows) reads the row twice.
template <int P>
__global__ __launch_bounds__(256) void k_af16split16(const float *__restrict__ a, int64_t M,
                                                     int64_t K, int c4n, int vec,
                                                     uint4 *__restrict__ ahl,
                                                     int *__restrict__ texp) {
  __shared__ float red[4];
  const int t = threadIdx.x, r = blockIdx.x;
  const bool live = r < M;
  const float *ar = a + (int64_t)r * K;
  const int octets = c4n * 16;
  auto load8 = [&](int o, float v[8]) __attribute__((always_inline)) {
    const int64_t k0 = (int64_t)o * 8;
    if (live && vec && k0 + 8 <= K) {
      const float4 x0 = *reinterpret_cast<const float4 *>(ar + k0);
      const float4 x1 = *reinterpret_cast<const float4 *>(ar + k0 + 4);
      v[0] = x0.x; v[1] = x0.y; v[2] = x0.z; v[3] = x0.w;
      v[4] = x1.x; v[5] = x1.y; v[6] = x1.z; v[7] = x1.w;
    } else {
#pragma unroll
      for (int i = 0; i < 8; i++) v[i] = (live && k0 + i < K) ? ar[k0 + i] : 0.f;
    }
  };
  auto row_exponent = [&](float mx) __attribute__((always_inline)) {
    for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
    if ((t & 63) == 0) red[t >> 6] = mx;
    __syncthreads();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    int e = 0;
    if (mx > 0.f) {
      int ex;
      frexpf(mx, &ex);
      e = 14 - ex;
    }
    if (t == 0) texp[r] = e;
    return e;
  };
  auto split = [&](int o, const float v[8], int e) __attribute__((always_inline)) {
    half8 hi, lo;
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const float x = ldexpf(v[i], (i & 2) ? e - 4 : e);
      const _Float16 hh = (_Float16)x;
      float res = x - (float)hh;
      if (!isfinite(res)) res = 0.f;
      hi[i] = hh;
      lo[i] = (_Float16)res;
    }
    const int kg = o >> 4, j = (o >> 2) & 3, g = o & 3;
    uint4 *dst = ahl + ((int64_t)(kg * 4 + j) * 2) * 64 + 16 * g + r;
    dst[0] = __builtin_bit_cast(uint4, hi);
    dst[64] = __builtin_bit_cast(uint4, lo);
  };
  if constexpr (P > 0) {
    float v[P][8];
#pragma unroll
    for (int i = 0; i < P; i++) {
      if (t + 256 * i < octets) {
        load8(t + 256 * i, v[i]);
      } else {
#pragma unroll
        for (int q = 0; q < 8; q++) v[i][q] = 0.f;
      }
    }
    float mx = 0.f;
#pragma unroll
    for (int i = 0; i < P; i++)
#pragma unroll
      for (int q = 0; q < 8; q++) {
        const float f = fabsf(v[i][q]);
        mx = f < INFINITY ? fmaxf(mx, f) : mx;  // finite values only
      }
    const int e = row_exponent(mx);
#pragma unroll
    for (int i = 0; i < P; i++)
      if (t + 256 * i < octets) split(t + 256 * i, v[i], e);
    return;
  }
  float mx = 0.f;
  if (live) {
    if (vec) {
      for (int64_t k = 4 * (int64_t)t; k + 3 < K; k += 1024) {
        const float4 x = *reinterpret_cast<const float4 *>(ar + k);
        const float v[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const float f = fabsf(v[i]);
          mx = f < INFINITY ? fmaxf(mx, f) : mx;  // finite values only
        }
      }
      for (int64_t k = (K & ~(int64_t)3) + t; k < K; k += 256) {
        const float f = fabsf(ar[k]);
        mx = f < INFINITY ? fmaxf(mx, f) : mx;
      }
    } else {
      for (int64_t k = t; k < K; k += 256) {
        const float f = fabsf(ar[k]);
        mx = f < INFINITY ? fmaxf(mx, f) : mx;
      }
    }
  }
  const int e = row_exponent(mx);
  for (int o = t; o < octets; o += 256) {
    float v[8];
    load8(o, v);
    split(o, v, e);
  }
}

// 16-row MFMA GEMV for 3 <= M <= 16 rows (decode with a few tokens).  One
// workgroup per column group (64 columns = four 16-column tiles); its 4 waves
// split K, wave w taking k groups w, w + 4, ...  Lane l works on column
// 16 tile + l % 16 and k octet g = l / 16 of every 32-k step j: the 16 bytes
// of packed codes at (g, column) hold exactly that lane's B operand for
// steps j = 0..3 (wq's nibble order), so each lane dequantises only its own
// operands (deq8, exact fp16 (q - zp) and 16 (q - zp)) and no LDS is needed
// for B.  The activations come from k_af16split16 (hi and lo fp16, two
// v_mfma_f32_16x16x32_f16 per step and tile); block scales are applied to the
// fp32 per-segment sum D once per block: acc += s * D.  The four waves' sums
// are added in wave order through LDS; the row exponents come off at the end.
// Packed codes, scales, zero points and activation fragments of the next k
// group are loaded while the current one is computed.
// TPW = 16-column tiles per workgroup (4: the whole column group; 2 or 1
// give narrow weights 2 or 4 workgroups per column group, tiles t0 ..).
#ifndef MG_DEC_PD
#define MG_DEC_PD 2
#endif
// Split K (gridDim.y > 1, part not null): the workgroup takes k groups
// [kps * y, + kps) and writes its sum, the row exponent taken off, to the
// partials; k_gemm_reduce adds the splits in order with the bias.
template <int SEGJ, int NW, int TPW, int PD = MG_DEC_PD>
__global__ __launch_bounds__(NW * 64) void k_gemv_mfma(
    const uint4 *__restrict__ ahl, const int *__restrict__ texp, const GemvSet gs, int M,
    int c4n, int nb, int nbh, int lbs, int has_zp, int kps, float *__restrict__ part) {
  __shared__ float4 red[NW][TPW][64];  // [wave][tile][lane]
  constexpr int NBK = 4 / SEGJ;       // blocks (scale segments) per k group
  constexpr int WPG = 4 / TPW;        // workgroups per column group
  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  int cg;
  const int gm = gemv_member(gs, (int)blockIdx.x / WPG, &cg);
  const int t0 = ((int)blockIdx.x % WPG) * TPW;  // first tile of this workgroup
  const uint4 *__restrict__ wq = gs.wq[gm];
  const float *__restrict__ scales = gs.scales[gm];
  const uint8_t *__restrict__ zp4 = gs.zp4[gm];
  const float *__restrict__ bias = gs.bias[gm];
  float *__restrict__ y = gs.y[gm];
  const int N = gs.N[gm];
  const int c16 = lane & 15, g = lane >> 4;
  // Raw buffer loads: wave-uniform resources (the column group's tables, the
  // activation fragments), a fixed lane byte offset and a uniform offset.  The
  // scale resource spans exactly the column group's nb blocks and the block
  // offset goes in the vector offset (the range check ignores the scalar
  // one), so blocks past the last (k padding) read as zero scales.
  auto rsrc = [](const void *base, int bytes) __attribute__((always_inline)) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, bytes,
                                             0x00020000);
  };
  const __amdgpu_buffer_rsrc_t r_w = rsrc(wq + (int64_t)cg * c4n * 256, 0x7ffffff0);
  const __amdgpu_buffer_rsrc_t r_a = rsrc(ahl, 0x7ffffff0);
  // Scales and zero-point bytes of the lane's four columns are adjacent
  // (sz_pos): one 16-byte and one 4-byte load per block.
  const __amdgpu_buffer_rsrc_t r_s = rsrc(scales + (int64_t)cg * nb * 64, nb * 256);
  const __amdgpu_buffer_rsrc_t r_z = rsrc(zp4 + (int64_t)cg * nbh * 64, 0x7ffffff0);
  // Lanes of activation rows >= M load nothing (an offset past the
  // resource reads as zero without a memory access): at M = 4 that is three
  // quarters of the activation traffic.
  const unsigned vo_w = 16u * (unsigned)(g * 64 + c16);
  const unsigned vo_a = c16 < M ? 16u * (unsigned)lane : 0x7ffffff0u;
  const unsigned vo_s = 16u * (unsigned)c16, vo_z = 4u * (unsigned)c16;

  // Raw loads of one k group; they are first touched in compute(), so the
  // wait for them does not also wait for the next k group's loads.
  struct Ring {
    uint4 ah[4], al[4];  // activation fragments (hi, lo) per 32-k step
    uint4 w[TPW];        // packed codes per tile
    float s[NBK][TPW];   // scales of the workgroup's tiles per block
    uint32_t zw[NBK];    // zero-point bytes of the four tiles per block
  };
  auto ld16 = [](__amdgpu_buffer_rsrc_t r, unsigned vo, int so) __attribute__((always_inline)) {
    return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, vo, so, 0));
  };
  // live == false: a slot that is never read (past the wave's last k
  // group): every offset past its resource, so the loads touch no memory.
  auto fetch = [&](int kg, Ring &R, bool live) {
    const unsigned ob = live ? 0u : 0x80000000u;
#pragma unroll
    for (int tl = 0; tl < TPW; tl++)
      R.w[tl] = ld16(r_w, vo_w + ob, (kg * 256 + (t0 + tl) * 16) * 16);
#pragma unroll
    for (int j = 0; j < 4; j++) {
      R.ah[j] = ld16(r_a, vo_a + ob, (kg * 4 + j) * 2048);
      R.al[j] = ld16(r_a, vo_a + ob, (kg * 4 + j) * 2048 + 1024);
    }
#pragma unroll
    for (int q = 0; q < NBK; q++) {
      const int b = (kg * KGRP + q * 32 * SEGJ) >> lbs;  // past nb: k padding, zero scale
      const unsigned so = vo_s + 4u * (unsigned)t0 + 256u * (unsigned)b + ob;
      if constexpr (TPW == 4) {
        const float4 x = __builtin_bit_cast(float4, ld16(r_s, so, 0));
        R.s[q][0] = x.x, R.s[q][1] = x.y, R.s[q][2] = x.z, R.s[q][3] = x.w;
      } else if constexpr (TPW == 2) {
        const float2 x = __builtin_bit_cast(float2, __builtin_amdgcn_raw_buffer_load_b64(r_s, so, 0, 0));
        R.s[q][0] = x.x, R.s[q][1] = x.y;
      } else {
        R.s[q][0] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r_s, so, 0, 0));
      }
      // Loaded whether or not the weight has zero points (the table then
      // points at the scales): a load under a branch would leave the wait
      // counts uncertain, and the compiler would then wait for every load
      // in flight, the next k group's included.  compute() picks the value.
      const int bc = min(b, nb - 1);
      R.zw[q] = __builtin_amdgcn_raw_buffer_load_b32(r_z, vo_z + ob, (bc >> 1) * 64, 0);
    }
  };
  uint32_t v_mlo, v_mhi, v_magic;
  asm volatile("v_mov_b32 %0, %1" : "=v"(v_mlo) : "s"(0x000F000Fu));
  asm volatile("v_mov_b32 %0, %1" : "=v"(v_mhi) : "s"(0x00F000F0u));
  asm volatile("v_mov_b32 %0, %1" : "=v"(v_magic) : "s"(0x64006400u));

  float4v acc[TPW], D[TPW];
#pragma unroll
  for (int tl = 0; tl < TPW; tl++) acc[tl] = (float4v){0.f, 0.f, 0.f, 0.f};
  const float4v zero4 = (float4v){0.f, 0.f, 0.f, 0.f};

  // At the start of each block: its scales (zero past the last block, i.e.
  // k padding) and the dequantisation constants -(1024 + z), -(1024 + 16 z)
  // as fp16 pairs; -(1024 + z) in fp16 is 0xE400 + z (exact), so they are
  // built with integer arithmetic.
  auto compute = [&](int kg, const Ring &R) {
    float sq[TPW];
    uint32_t z1[TPW], z16[TPW];
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int q = j / SEGJ;
      const bool seg_start = (j % SEGJ) == 0;
      if (seg_start) {
        const int b = (kg * KGRP + q * 32 * SEGJ) >> lbs;
        const uint32_t sh = (min(b, nb - 1) & 1) * 4;
#pragma unroll
        for (int tl = 0; tl < TPW; tl++) sq[tl] = R.s[q][tl];
        const uint32_t zwq = has_zp ? R.zw[q] : 0x88888888u;
#pragma unroll
        for (int tl = 0; tl < TPW; tl++) {
          const uint32_t zv = (zwq >> (8 * (t0 + tl) + sh)) & 15u;
          z1[tl] = 0xE400E400u + zv * 0x00010001u;
          z16[tl] = 0xE400E400u + zv * 0x00100010u;
        }
      }
      const half8 a_h = __builtin_bit_cast(half8, R.ah[j]);
      const half8 a_l = __builtin_bit_cast(half8, R.al[j]);
      half8 bt[TPW];
#pragma unroll
      for (int tl = 0; tl < TPW; tl++) {
        const uint32_t x = j == 0 ? R.w[tl].x : j == 1 ? R.w[tl].y : j == 2 ? R.w[tl].z : R.w[tl].w;
        bt[tl] = __builtin_bit_cast(
            half8, deq8(x, v_mlo, v_mhi, v_magic, __builtin_bit_cast(half2v, z1[tl]),
                        __builtin_bit_cast(half2v, z16[tl])));
      }
      // All hi products first, then all lo: each lo MFMA then follows its
      // tile's hi MFMA by three others instead of waiting on it.
#pragma unroll
      for (int tl = 0; tl < TPW; tl++)
        D[tl] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a_h, bt[tl], seg_start ? zero4 : D[tl], 0,
                                                       0, 0);
#pragma unroll
      for (int tl = 0; tl < TPW; tl++)
        D[tl] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a_l, bt[tl], D[tl], 0, 0, 0);
      if ((j + 1) % SEGJ == 0) {
#pragma unroll
        for (int tl = 0; tl < TPW; tl++)
#pragma unroll
          for (int i = 0; i < 4; i++) acc[tl][i] = fmaf(sq[tl], D[tl][i], acc[tl][i]);
      }
    }
  };

  // PD-slot ring over this wave's k groups (unrolled by PD so slots are
  // static registers).  Wave w takes k groups w, w + NW, ... with the loads
  // of the next PD - 1 in flight: one k group of work is far shorter than
  // a load's latency, so a wave with several k groups needs them in flight.
  const int kbeg = part ? (int)blockIdx.y * kps : 0;
  const int kend = part ? min(c4n, kbeg + kps) : c4n;
  // The blocks of PD k groups whose every prefetch is in range run first,
  // with no branch around a fetch: under such a branch the compiler cannot
  // count the loads issued after a slot's and waits for all of them before
  // each compute, the prefetch included.  The last block or two (bounded
  // fetches) follow.
  Ring R[PD];
#pragma unroll
  for (int j = 0; j < PD - 1; j++)
    if (kbeg + wave + j * NW < kend) fetch(kbeg + wave + j * NW, R[j], true);
  int kb = kbeg + wave;
  for (; kb + (2 * PD - 2) * NW < kend; kb += PD * NW) {
#pragma unroll
    for (int j = 0; j < PD; j++) {
      const int kg = kb + j * NW;
      fetch(kg + (PD - 1) * NW, R[(j + PD - 1) % PD], true);
      __builtin_amdgcn_sched_barrier(0);
      compute(kg, R[j]);
    }
  }
  for (; kb < kend; kb += PD * NW) {
#pragma unroll
    for (int j = 0; j < PD; j++) {
      const int kg = kb + j * NW;
      if (kg >= kend) break;
      if (kg + (PD - 1) * NW < kend) fetch(kg + (PD - 1) * NW, R[(j + PD - 1) % PD], true);
      __builtin_amdgcn_sched_barrier(0);
      compute(kg, R[j]);
    }
  }

#pragma unroll
  for (int tl = 0; tl < TPW; tl++)
    red[wave][tl][lane] = make_float4(acc[tl][0], acc[tl][1], acc[tl][2], acc[tl][3]);
  __syncthreads();
  if (wave == 0) {
#pragma unroll
    for (int tl = 0; tl < TPW; tl++) {
      float4 s = red[0][tl][lane];
#pragma unroll
      for (int w = 1; w < NW; w++) {
        const float4 o = red[w][tl][lane];
        s.x += o.x; s.y += o.y; s.z += o.z; s.w += o.w;
      }
      const int col = cg * 64 + (t0 + tl) * 16 + c16;
      const float bv = (bias && col < N && !part) ? bias[col] : 0.f;
      const float sv[4] = {s.x, s.y, s.z, s.w};
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int row = 4 * g + i;
        if (row >= M || col >= N) continue;
        if (part)
          part[gs.part_off[gm] + ((int64_t)blockIdx.y * M + row) * N + col] =
              ldexpf(sv[i], -texp[row]);
        else
          y[(int64_t)row * N + col] = ldexpf(sv[i], -texp[row]) + bv;
      }
    }
  }
}

// ------------------------------------- float zero points, 16-k blocks

// Columns [n0, n0 + nc) of a packed weight dequantised to fp32 as the
// reference does before its GEMM (onnx_qlinear_ops.dart:208-226): w = (q -
// zp) * scale in double, one rounding to fp32.  Output row cl holds column
// n0 + cl over all K (the [N][K] operand of the fp32 GEMM).  Thread = the 8
// consecutive k of one packed dword: k = 128 kg + 8 o, o = 4 j + g.
__global__ __launch_bounds__(256) void k_nbits_dequant_f32(
    const uint32_t *__restrict__ wq, const float *__restrict__ scales,
    const uint8_t *__restrict__ zp4, const float *__restrict__ zpf, int zpk, int64_t n0,
    int64_t nc, int64_t K, int c4, int nb, int nbh, int bs, float *__restrict__ out) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= nc * c4 * 16) return;
  const int o = (int)(idx & 15);
  const int64_t rest = idx >> 4;
  const int kg = (int)(rest % c4);
  const int64_t cl = rest / c4;
  const int64_t col = n0 + cl;
  const int64_t cgi = col >> 6;
  const int cg = (int)(col & 63);
  const int j = o >> 2, g = o & 3;
  const int64_t k0 = (int64_t)kg * KGRP + 8 * o;
  if (k0 >= K) return;
  const uint32_t dw = wq[((((int64_t)cgi * c4 + kg) * 4 + g) * 64 + cg) * 4 + j];
  float v[8];
#pragma unroll
  for (int t = 0; t < 8; t++) {
    const int64_t k = k0 + t;
    const int q = (int)((dw >> (4 * nib_pos(t))) & 15);
    const int64_t blk = min(k, K - 1) / bs;
    double z = 8.0;
    if (zpk == 1) {
      const uint8_t zb = zp4[(cgi * nbh + blk / 2) * 64 + sz_pos(cg)];
      z = (double)((blk & 1) ? (zb >> 4) : (zb & 15));
    } else if (zpk == 2) {
      z = (double)zpf[(cgi * nb + blk) * 64 + sz_pos(cg)];
    }
    v[t] = (float)(((double)q - z) * (double)scales[(cgi * nb + blk) * 64 + sz_pos(cg)]);
  }
  float *dst = out + cl * K + k0;
  if (K % 4 == 0 && k0 + 8 <= K) {
    *reinterpret_cast<float4 *>(dst) = make_float4(v[0], v[1], v[2], v[3]);
    *reinterpret_cast<float4 *>(dst + 4) = make_float4(v[4], v[5], v[6], v[7]);
  } else {
#pragma unroll
    for (int t = 0; t < 8; t++)
      if (k0 + t < K) dst[t] = v[t];
  }
}

// ------------------------------------------------------------ host side

}  // namespace

// The fp8 prefill GEMM (nbits_f8.hip): workspace layout for mpad rows and c4
// k groups (returns the bytes before the split-K partials), and the launch.
size_t mg_nbits_f8_ws(int64_t mpad, int64_t c4, size_t *off_asc, size_t *off_nf,
                      size_t *off_rs);
mg_status mg_nbits_prefill_f8(mg_ctx *ctx, int n, const mg_weight *const *w, const float *a_dev,
                              int64_t M, float *const *y_dev, void *ws, int64_t mpad, int nt,
                              int ksplit, int kps, size_t off_part, int kwave);

namespace {

struct NbitsPlan {
  int path;  // 0 gemv (dot8), 1 prefill mfma (fp16), 2 generic, 3 decode mfma, 4 prefill fp8
  int64_t M;
  // gemv
  int qpg = 1, qb = 128, ksplit = 1, kps = 0, nw = 4, kc = 0;
  size_t lds = 0;
  // mfma
  int64_t mpad = 0;
  int nt = 4;  // prefill tile width in 32-column MFMA tiles (4 or 2)
  int64_t chunk = 0;  // fp32 path: columns dequantised per chunk
  int pers = 0;       // GEMV on the persistent kernel (k_gemv_dot8p)
  int pers_grid = 0;  // its workgroups
  int cs = 0;         // GEMV on the column-slice kernel (k_gemv_cs)
  int cs_pf = 4;      // its k groups in flight per wave
  int kwave = 0;      // fp6 prefill on k_gemm_f6kw (32 x 64 tiles, waves split K)
  size_t off_a = 0, off_b = 0, off_c = 0, off_d = 0, total = 0;
};

// ng_total / n_total: column groups / columns of all weights launched together
// (sibling weights sharing one input).
NbitsPlan plan_nbits(const mg_ctx *ctx, const mg_weight *w, int64_t M, int64_t ng_total,
                     int64_t n_total, bool imgs) {
  const mg_nbits_dev &d = w->nbits;
  NbitsPlan p;
  p.M = M;
  const bool int_zp = d.zp_kind != MG_ZP_FLOAT;
#ifndef MG_DECODE_MFMA_MIN_M
#define MG_DECODE_MFMA_MIN_M 3
#endif
  if (M >= MG_DECODE_MFMA_MIN_M && M <= 16 && d.bs >= 32 && int_zp) {
    p.path = 3;
    p.off_a = 0;  // ahl16: 16 rows x kpad x (hi, lo) fp16
    p.off_b = mg_align((size_t)16 * d.kpad * 4);  // texp[16]
    p.off_c = mg_align(p.off_b + 16 * 4);          // split-K partials
#ifndef MG_DEC_SPLIT
#define MG_DEC_SPLIT 1
#endif
    // Narrow weights (fewer column groups than CUs) with long rows: whole
    // column groups per workgroup with K split over workgroups (at least 8
    // k groups each), summed by k_gemm_reduce.  Each workgroup reads the
    // 16-row activation block of its k range only, where 16-column slices
    // over all of K read it whole per slice (Llama down 8192 x 2048: 64 MB
    // of activation reads for 8.4 MB of weights).
    const int64_t cus = std::max(ctx->num_cus, 1);
    if (MG_DEC_SPLIT && ng_total < cus && d.c4 >= 32) {
      int64_t ks = 1;
      while (ng_total * ks * 2 <= 2 * cus && d.c4 / (ks * 2) >= 8) ks *= 2;
      if (ks > 1) {
        p.kps = (int)((d.c4 + ks - 1) / ks);
        p.ksplit = (int)((d.c4 + p.kps - 1) / p.kps);
      }
    }
    p.total = mg_align(p.off_c + (p.ksplit > 1 ? (size_t)p.ksplit * M * n_total * 4 : 0));
  } else if (M <= 4 && d.bs <= 4096) {
    p.path = 0;
    p.qb = (int)std::min<int64_t>(d.bs, KGRP);
    p.qpg = KGRP / p.qb;
    // One workgroup per column group; its waves split K.  Wide weights use
    // 4 waves (4 k groups of loads in flight each); narrow ones use up to 16
    // (2 in flight each) so that their few workgroups still keep enough bytes
    // in flight per CU.
    // (The 16-wave form is register-limited to one row and blocks <= 64.)
#ifndef MG_GEMV_MAX_NW
#define MG_GEMV_MAX_NW 16
#endif
    // One row, blocks <= 64, K >= 4096 and fewer than half a column group
    // per CU: K is also split over workgroups (kps k groups each, at least
    // 4) until the grid covers the CUs, and an ordered sum of the splits'
    // partials adds the bias (k_gemm_reduce): a CU streams at most ~100
    // GB/s, so a long narrow weight must spread over many CUs.  (Llama down
    // 8192 x 2048: 14.2 -> 8.1 us with the sum; at K = 2048 the extra launch
    // costs more than the spread gains.)
#ifndef MG_GEMV_SPLIT
#define MG_GEMV_SPLIT 1
#endif
    const int64_t cus = std::max(ctx->num_cus, 1);
    int64_t kspan = d.c4;
    if (MG_GEMV_SPLIT && M == 1 && p.qpg >= 2 && ng_total * 2 < cus && d.c4 >= 32) {
      int64_t ks = 1;
      while (ng_total * ks * 2 <= cus && d.c4 / (ks * 2) >= 4) ks *= 2;
      if (ks > 1) {
        p.kps = (int)((d.c4 + ks - 1) / ks);
        p.ksplit = (int)((d.c4 + p.kps - 1) / p.kps);
        kspan = p.kps;
      }
    }
    int64_t nw = 4;
    if (M == 1 && p.qpg >= 2 && ng_total * p.ksplit * 4 < 8 * cus) nw = MG_GEMV_MAX_NW;
    nw = std::min<int64_t>(nw, std::max<int64_t>(kspan, 4));
    if (nw > 4) nw = nw > 8 ? 16 : 8;
    const int pf = nw == 4 ? 4 : 2;
    // Activation digits of a chunk of kc k groups live in LDS (<= 64 KiB); a
    // partial chunk size is a multiple of pf * nw.
    const int64_t per_kg = M * (64 + 2 * p.qpg) * 4;
    const int64_t kc_max = 65536 / per_kg;
    int64_t kc = kspan;
    if (kc > kc_max) kc = kc_max / (pf * nw) * (pf * nw);
    p.nw = (int)nw;
    p.kc = (int)kc;
    p.lds = (size_t)std::max<int64_t>(kc * per_kg, nw * M * 64 * 4);
    p.total = p.ksplit > 1 ? mg_align((size_t)p.ksplit * M * n_total * 4) : 0;
    // One row, k groups that split evenly over 4 waves (1 or 2 each) and
    // enough column groups for several per workgroup: the persistent kernel,
    // with the column groups dealt evenly over about MG_GEMV_WG_PER_CU
    // workgroups per CU.  (With 4 k groups per wave its per-column-group work
    // is long enough that the one-workgroup-per-column-group form, with more
    // waves resident per SIMD, streams as fast.)
#ifndef MG_GEMV_WG_PER_CU
#define MG_GEMV_WG_PER_CU 2
#endif
    const int64_t slots = MG_GEMV_WG_PER_CU * (int64_t)std::max(ctx->num_cus, 1);
    const int64_t per_wave = d.c4 / 4;
    if (M == 1 && p.ksplit == 1 && nw == 4 && kc == d.c4 && d.c4 % 4 == 0 &&
        (per_wave == 1 || per_wave == 2) &&
        ng_total >= 2 * slots) {
      const int64_t per = (ng_total + slots - 1) / slots;
      p.pers = 1;
      p.pers_grid = (int)((ng_total + per - 1) / per);
      p.lds = (size_t)(d.c4 * per_kg + 2 * 4 * M * 64 * 4);
    }
    // One row, one quantisation block per k group and fewer column groups
    // than MG_GEMV_CS_MAX_CG: 16-column slices (four workgroups per column
    // group), for K up to 64 k groups (the digits of all of K in LDS).
    // Measured on the Qwen3 shapes (graph replay, rotated weights): 16-64
    // column groups 4.1-6.5 us against 4.5-8.0 us on k_gemv_dot8; at 96
    // (gate/up grouped) 5.3 against 5.0 us.
#ifndef MG_GEMV_CS_MAX_CG
#define MG_GEMV_CS_MAX_CG 96
#endif
    if (M == 1 && p.qpg == 1 && p.ksplit == 1 && !p.pers && ng_total < MG_GEMV_CS_MAX_CG &&
        kc == d.c4 &&
        d.c4 <= 16 * CS_TASKS) {
      p.cs = 1;
      p.cs_pf = d.c4 > 16 ? 8 : 4;
      p.lds = (size_t)std::max<int64_t>(d.c4 * per_kg, 4 * 16 * 4);
    }
  } else if ((d.bs >= 32 && int_zp) || (d.bs >= KGRP && imgs)) {
    // (Float zero points at blocks >= 128 on weights with prefill images:
    // the fp6 GEMM with the zero point taken out as a row sum.)
#ifndef MG_PREFILL_F8
#define MG_PREFILL_F8 1
#endif
    p.path = (MG_PREFILL_F8 && d.bs >= KGRP) ? 4 : 1;
    // Workgroups per CU to aim for, and k groups per split to keep.
#ifndef MG_PREFILL_WG_PER_CU
#define MG_PREFILL_WG_PER_CU 1
#endif
#ifndef MG_PREFILL_MIN_KG
#define MG_PREFILL_MIN_KG 2
#endif
    const int64_t target = MG_PREFILL_WG_PER_CU * (int64_t)std::max(ctx->num_cus, 1);
    const int64_t rows = 128;  // workgroup tile rows
    p.mpad = (M + rows - 1) / rows * rows;
    const int64_t mt = p.mpad / rows;
    // 128-column tiles when they alone cover the chip, else 64-column tiles;
    // then split K until the grid covers it.
    p.nt = mt * (ng_total / 2) >= target ? 4 : 2;
    const int64_t tiles = mt * (p.nt == 4 ? ng_total / 2 : ng_total);
    int64_t ks = 1;
    while (tiles * ks * 2 <= target && d.c4 / (ks * 2) >= MG_PREFILL_MIN_KG) ks *= 2;
#ifndef MG_PREFILL_KWAVE
#define MG_PREFILL_KWAVE 1
#endif
    // Where even 128 x 64 tiles leave the chip short and K would be split
    // over workgroups (fp6 images, integer zero points): 32 x 64 tiles whose
    // four waves split K instead (k_gemm_f6kw), with the partial sums added
    // in the same launch.  Qwen3 o / down at M = 512: 10.0 + 5.2 -> 11.4 us
    // and 12.2 + 5.1 -> 14.9 us.  Where the grid is already full without a
    // split it is slower (three rounds of small workgroups, each paying the
    // load latency: q/k/v 13.8 -> 17.4 us), so it is not used there.
    if (MG_PREFILL_KWAVE && p.path == 4 && p.nt == 2 && ks > 1 && imgs && int_zp) {
      p.kwave = 1;
      ks = 1;
    }
    p.kps = (int)((d.c4 + ks - 1) / ks);
    p.ksplit = (int)((d.c4 + p.kps - 1) / p.kps);
    if (p.path == 4) {
      size_t o_asc = 0, o_nf = 0, o_rs = 0;  // digits, scale words, flags, row sums
      p.off_c = mg_nbits_f8_ws(p.mpad, d.c4, &o_asc, &o_nf, &o_rs);  // split-K partials after
    } else {
      p.off_a = 0;  // ahl: mpad * kpad * 2 fp16
      p.off_b = mg_align(p.off_a + (size_t)p.mpad * d.kpad * 4);  // texp [row]
      p.off_c = mg_align(p.off_b + (size_t)p.mpad * 4);           // split-K partials
    }
    p.total = mg_align(p.off_c + (p.ksplit > 1 ? (size_t)p.ksplit * M * n_total * 4 : 0));
  } else {
    // Float zero points or 16-k blocks with more rows: the columns are
    // dequantised to fp32 in chunks of about 64 MiB and each chunk runs
    // through the fp32 MFMA GEMM.
    p.path = 2;
    const int64_t per_col = d.c4 * KGRP;  // floats a column takes (K rounded up)
    p.chunk = std::max<int64_t>(64, ((int64_t)(16 << 20) / per_col) / 64 * 64);
    p.chunk = std::min<int64_t>(p.chunk, (n_total + 63) / 64 * 64);
    p.total = mg_align((size_t)p.chunk * per_col * 4);
  }
  return p;
}

GemvSet make_set(int n, const mg_weight *const *w, float *const *y) {
  GemvSet gs{};
  gs.n = n;
  int acc = 0;
  for (int i = 0; i < n; i++) {
    const mg_nbits_dev &d = w[i]->nbits;
    gs.wq[i] = reinterpret_cast<const uint4 *>(d.wq);
    gs.scales[i] = d.scales;
    // Unused zero-point arrays point at the scales (never dereferenced).
    gs.zp4[i] = d.zp4 ? d.zp4 : reinterpret_cast<const uint8_t *>(d.scales);
    gs.zpf[i] = d.zpf ? d.zpf : d.scales;
    gs.bias[i] = d.bias;
    gs.y[i] = y[i];
    gs.N[i] = (int)w[i]->N;
    acc += (int)d.ng;
    gs.cg_end[i] = acc;
  }
  return gs;
}

template <int MR, int QPG>
void launch_gemv_zp(const mg_weight *w, const GemvSet &gs, const NbitsPlan &p,
                    hipStream_t st, const float *a, int vec, float *part) {
  const mg_nbits_dev &d = w->nbits;
  const dim3 grid((unsigned)gs.cg_end[gs.n - 1], (unsigned)p.ksplit),
      block((unsigned)(64 * p.nw));
#define MG_GEMV_ARGS                                                                        \
  a, w->K, vec, gs, (int)d.c4, (int)d.nb, (int)d.nbh, __builtin_ctzll(d.bs), p.kc,       \
      p.ksplit > 1 ? p.kps : (int)d.c4, p.ksplit > 1 ? part : nullptr
  // The 8/16-wave form (PF 2) is planned only for one row and QPG >= 2.
#define MG_GEMV_LAUNCH(Z_)                                                                   \
  do {                                                                                       \
    if constexpr (MR == 1 && QPG >= 2) {                                                     \
      if (p.nw != 4) {                                                                       \
        hipLaunchKernelGGL((k_gemv_dot8<MR, QPG, Z_, 2>), grid, block, p.lds, st,            \
                           MG_GEMV_ARGS);                                                    \
        break;                                                                               \
      }                                                                                      \
    }                                                                                        \
    hipLaunchKernelGGL((k_gemv_dot8<MR, QPG, Z_, 4>), grid, block, p.lds, st, MG_GEMV_ARGS); \
  } while (0)
  if (d.zp_kind == 0) MG_GEMV_LAUNCH(0);
  else if (d.zp_kind == 1) MG_GEMV_LAUNCH(1);
  else MG_GEMV_LAUNCH(2);
#undef MG_GEMV_LAUNCH
#undef MG_GEMV_ARGS
}

template <int QPG, int ZPK>
void launch_gemv_pers_pf(const mg_weight *w, const GemvSet &gs, const NbitsPlan &p,
                         hipStream_t st, const float *a, int vec) {
  const mg_nbits_dev &d = w->nbits;
  const dim3 grid((unsigned)p.pers_grid), block(256);
#define MG_PERS_LAUNCH(PF_)                                                                  \
  hipLaunchKernelGGL((k_gemv_dot8p<1, QPG, ZPK, PF_>), grid, block, p.lds, st, a, w->K, vec, gs, \
                     (int)d.c4, (int)d.nb, (int)d.nbh, __builtin_ctzll(d.bs))
  if (d.c4 == 4) MG_PERS_LAUNCH(1);
  else MG_PERS_LAUNCH(2);
#undef MG_PERS_LAUNCH
}

template <int QPG>
void launch_gemv_pers(const mg_weight *w, const GemvSet &gs, const NbitsPlan &p, hipStream_t st,
                      const float *a, int vec) {
  if (w->nbits.zp_kind == 0) launch_gemv_pers_pf<QPG, 0>(w, gs, p, st, a, vec);
  else if (w->nbits.zp_kind == 1) launch_gemv_pers_pf<QPG, 1>(w, gs, p, st, a, vec);
  else launch_gemv_pers_pf<QPG, 2>(w, gs, p, st, a, vec);
}

template <int ZPK>
void launch_gemv_cs_z(const mg_weight *w, const GemvSet &gs, const NbitsPlan &p, hipStream_t st,
                      const float *a, int vec) {
  const mg_nbits_dev &d = w->nbits;
  const dim3 grid((unsigned)gs.cg_end[gs.n - 1] * 4), block(256);
#define MG_CS_LAUNCH(PF_, V_)                                                            \
  hipLaunchKernelGGL((k_gemv_cs<ZPK, PF_, V_>), grid, block, p.lds, st, a, w->K, gs,      \
                     (int)d.c4, (int)d.nb, (int)d.nbh, __builtin_ctzll(d.bs))
  if (p.cs_pf == 8) {
    if (vec) MG_CS_LAUNCH(8, true);
    else MG_CS_LAUNCH(8, false);
  } else {
    if (vec) MG_CS_LAUNCH(4, true);
    else MG_CS_LAUNCH(4, false);
  }
#undef MG_CS_LAUNCH
}

void launch_gemv_cs(const mg_weight *w, const GemvSet &gs, const NbitsPlan &p, hipStream_t st,
                    const float *a, int vec) {
  if (w->nbits.zp_kind == 0) launch_gemv_cs_z<0>(w, gs, p, st, a, vec);
  else if (w->nbits.zp_kind == 1) launch_gemv_cs_z<1>(w, gs, p, st, a, vec);
  else launch_gemv_cs_z<2>(w, gs, p, st, a, vec);
}

template <int MR>
void launch_gemv_q(const mg_weight *w, const GemvSet &gs, const NbitsPlan &p, hipStream_t st,
                   const float *a, int vec, float *part) {
  if (MR == 1 && p.cs) {
    launch_gemv_cs(w, gs, p, st, a, vec);
    return;
  }
  if (MR == 1 && p.pers) {
    switch (p.qpg) {
      case 1: launch_gemv_pers<1>(w, gs, p, st, a, vec); break;
      case 2: launch_gemv_pers<2>(w, gs, p, st, a, vec); break;
      case 4: launch_gemv_pers<4>(w, gs, p, st, a, vec); break;
      default: launch_gemv_pers<8>(w, gs, p, st, a, vec); break;
    }
    return;
  }
  switch (p.qpg) {
    case 1: launch_gemv_zp<MR, 1>(w, gs, p, st, a, vec, part); break;
    case 2: launch_gemv_zp<MR, 2>(w, gs, p, st, a, vec, part); break;
    case 4: launch_gemv_zp<MR, 4>(w, gs, p, st, a, vec, part); break;
    default: launch_gemv_zp<MR, 8>(w, gs, p, st, a, vec, part); break;
  }
}

}  // namespace

// ------------------------------------------------------------- uploading

namespace {

// Device repack of one chunk of columns [n0, n0 + rows) (column groups
// [cg0, cg0 + cgs)) from the raw ONNX tensors in `raw` (B [rows][nb][bs/2],
// low nibble = even k) into the layout above.  Columns past N and k past
// nb * bs get code 8; all eight codes of a dword share one block
// (block_size >= 16 is a power of two and a dword spans 8 aligned k).
__global__ __launch_bounds__(256) void k_nbits_repack_codes(
    const uint32_t *__restrict__ raw, int64_t n0, int64_t N, int64_t nb, int64_t bs,
    int64_t c4, int64_t cg0, int64_t cgs, uint32_t *__restrict__ wq) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= cgs * c4 * 1024) return;
  const int j = (int)(idx & 3), col = (int)((idx >> 2) & 63), g = (int)((idx >> 8) & 3);
  const int64_t t2 = idx >> 10;
  const int64_t kg = t2 % c4, cg = cg0 + t2 / c4;
  const int64_t n = cg * 64 + col;
  const int64_t k0 = kg * KGRP + 32 * j + 8 * g;
  uint32_t dw = 0x88888888u;
  if (n < N && k0 < nb * bs) {
    // 4 bytes = k0 .. k0 + 7; byte i holds k0 + 2i (low) and k0 + 2i + 1 (high)
    const uint32_t v = raw[(((n - n0) * nb + k0 / bs) * (bs / 2) + (k0 % bs) / 2) / 4];
    // even k -> nibbles 0..3, odd k -> nibbles 4..7 (nib_pos)
    dw = 0;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const uint32_t by = (v >> (8 * i)) & 0xFFu;
      dw |= (by & 15u) << (4 * i);
      dw |= (by >> 4) << (16 + 4 * i);
    }
  }
  wq[(((cg * c4 + kg) * 4 + g) * 64 + col) * 4 + j] = dw;
}

// Per-block tables of the chunk: scales [cg][blk][sz_pos(col)] (0 past N),
// zero points as packed bytes [cg][blk/2][sz_pos(col)] (0x88 past N) or
// floats [cg][blk][sz_pos(col)] (8 past N).
__global__ __launch_bounds__(256) void k_nbits_repack_tables(
    const float *__restrict__ sc_raw, const uint8_t *__restrict__ zp_raw, int zp_kind,
    int64_t n0, int64_t N, int64_t nb, int64_t nbh, int64_t cg0, int64_t cgs,
    float *__restrict__ sp, uint8_t *__restrict__ zp4, float *__restrict__ zpf) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= cgs * nb * 64) return;
  const int col = (int)(idx & 63);
  const int64_t blk = (idx >> 6) % nb, cg = cg0 + (idx >> 6) / nb;
  const int64_t n = cg * 64 + col;
  const bool in = n < N;
  const int64_t o = (cg * nb + blk) * 64 + sz_pos(col);
  sp[o] = in ? sc_raw[(n - n0) * nb + blk] : 0.f;
  if (zp_kind == MG_ZP_FLOAT)
    zpf[o] = in ? reinterpret_cast<const float *>(zp_raw)[(n - n0) * nb + blk] : 8.f;
  if (zp_kind == MG_ZP_UINT4 && blk < nbh)
    zp4[(cg * nbh + blk) * 64 + sz_pos(col)] = in ? zp_raw[(n - n0) * nbh + blk] : 0x88;
}

// Reads bytes [off, off + len) of a source into dst.
// Bytes [off, off + len) of one source into dst; returns false on a failed
// read (the caller reports it).
bool read_part(const mg_byte_source &s, int fd, int64_t off, int64_t len, uint8_t *dst) {
  if (s.host) {
    std::memcpy(dst, s.host + off, (size_t)len);
    return true;
  }
  int64_t done = 0;
  while (done < len) {
    const ssize_t r = pread(fd, dst + done, (size_t)(len - done), (off_t)(s.offset + off + done));
    if (r < 0 && errno == EINTR) continue;
    if (r <= 0) return false;
    done += r;
  }
  return true;
}

// A large read is split over up to 4 threads in pieces of at least 8 MiB:
// one thread's memcpy (or page-cache read) into pinned memory ran at about
// the rate of the whole upload, below what the host-to-device copy takes.
mg_status read_source(const mg_byte_source &s, int fd, int64_t off, int64_t len, uint8_t *dst) {
  if (len == 0) return MG_OK;
  constexpr int64_t kPiece = 8ll << 20;
  const int parts = (int)std::min<int64_t>(4, std::max<int64_t>(1, len / kPiece));
  bool ok = true;
  if (parts == 1) {
    ok = read_part(s, fd, off, len, dst);
  } else {
    const int64_t step = (len + parts - 1) / parts;
    bool part_ok[4] = {true, true, true, true};
    std::thread th[3];
    int started = 0;
    for (int i = 1; i < parts; i++) {
      const int64_t o = i * step, l = std::min(len, o + step) - o;
      try {
        th[i - 1] = std::thread([&, i, o, l] { part_ok[i] = read_part(s, fd, off + o, l, dst + o); });
        started = i;
      } catch (...) {  // no thread: read the piece here
        part_ok[i] = read_part(s, fd, off + o, l, dst + o);
      }
    }
    part_ok[0] = read_part(s, fd, off, std::min(len, step), dst);
    for (int i = 0; i < started; i++)
      if (th[i].joinable()) th[i].join();
    for (int i = 0; i < parts; i++) ok = ok && part_ok[i];
  }
  if (!ok)
    return mg_fail(MG_INVALID_ARGUMENT, std::string("MatMulNBits: cannot read ") +
                                            std::to_string(len) + " bytes of " +
                                            (s.path ? s.path : "host data") + " at offset " +
                                            std::to_string(s.offset + off));
  return MG_OK;
}

struct OpenFiles {
  int fd[3] = {-1, -1, -1};
  ~OpenFiles() {
    for (int f : fd)
      if (f >= 0) close(f);
  }
};

}  // namespace

namespace {
// Grows the context's upload slots to two of at least `slot` bytes (pinned
// host and device, 8 MiB at least, so that the smaller weights of a model
// share the first allocation); every later upload of the context reuses them.
mg_status upload_slots(mg_ctx *ctx, size_t slot) {
  for (hipEvent_t &e : ctx->up_done)
    if (!e) MG_HIP(hipEventCreateWithFlags(&e, hipEventDisableTiming));
  if (ctx->up_slot >= slot) return MG_OK;
  slot = std::max(slot, (size_t)8 << 20);
  MG_HIP(hipStreamSynchronize(ctx->stream));
  if (ctx->up_pin) MG_HIP(hipHostFree(ctx->up_pin));
  if (ctx->up_dev) MG_HIP(hipFree(ctx->up_dev));
  ctx->up_pin = ctx->up_dev = nullptr;
  ctx->up_slot = 0;
  MG_HIP(hipHostMalloc(&ctx->up_pin, 2 * slot, hipHostMallocDefault));
  MG_HIP(hipMalloc(&ctx->up_dev, 2 * slot));
  ctx->up_slot = slot;
  return MG_OK;
}
}  // namespace

mg_status mg_nbits_upload(mg_ctx *ctx, mg_weight *w, const mg_byte_source &b,
                          const mg_byte_source &scales, int32_t zp_kind,
                          const mg_byte_source &zp, const float *bias, int64_t chunk_bytes) {
  mg_nbits_dev &d = w->nbits;
  const int64_t N = w->N, K = w->K, bs = d.bs;
  d.nb = (K + bs - 1) / bs;
  d.nbh = (d.nb + 1) / 2;
  d.kpad = std::max<int64_t>((d.nb * bs + KGRP - 1) / KGRP * KGRP, KGRP);
  d.c4 = d.kpad / KGRP;
  d.ng = ((N + CGRP - 1) / CGRP + 1) / 2 * 2;  // even: the GEMM pairs groups
  d.zp_kind = zp_kind;
  const int64_t ng = d.ng, nb = d.nb, nbh = d.nbh, c4 = d.c4;
  const int64_t blob = bs / 2;
  // Raw bytes per column of each tensor.
  const int64_t col_b = nb * blob, col_s = nb * 4;
  const int64_t col_z = zp_kind == MG_ZP_UINT4 ? nbh : zp_kind == MG_ZP_FLOAT ? nb * 4 : 0;
  const int64_t col_all = mg_align(col_b) + col_s + col_z;  // rough per-column footprint

  OpenFiles files;
  const mg_byte_source *srcs[3] = {&b, &scales, &zp};
  for (int i = 0; i < 3; i++) {
    if (i == 2 && zp_kind == MG_ZP_NONE) break;
    if (!srcs[i]->host) {
      if (!srcs[i]->path) return mg_fail(MG_INVALID_ARGUMENT, "MatMulNBits: missing tensor data");
      files.fd[i] = open(srcs[i]->path, O_RDONLY | O_CLOEXEC);
      if (files.fd[i] < 0)
        return mg_fail(MG_INVALID_ARGUMENT,
                       std::string("MatMulNBits: cannot open ") + srcs[i]->path);
    }
  }

  auto alloc = [&](void **dst, size_t bytes) -> mg_status {
    MG_HIP(hipMalloc(dst, bytes));
    w->device_bytes += (int64_t)bytes;
    return MG_OK;
  };
  MG_TRY(alloc((void **)&d.wq, (size_t)(ng * c4 * 1024) * 4));
  MG_TRY(alloc((void **)&d.scales, (size_t)(ng * nb * 64) * 4));
  if (zp_kind == MG_ZP_UINT4) MG_TRY(alloc((void **)&d.zp4, (size_t)(ng * nbh * 64)));
  if (zp_kind == MG_ZP_FLOAT) MG_TRY(alloc((void **)&d.zpf, (size_t)(ng * nb * 64) * 4));
  if (bias) {
    MG_TRY(alloc((void **)&d.bias, (size_t)N * 4));
    MG_HIP(hipMemcpy(d.bias, bias, (size_t)N * 4, hipMemcpyHostToDevice));
  }

  // Chunks of whole column groups; two staging slots (pinned host + device,
  // the context's) so that reading chunk i + 1 overlaps the copy and repack
  // of chunk i.
  if (chunk_bytes <= 0) chunk_bytes = 32ll << 20;
  const int64_t cgs_per = std::min<int64_t>(ng, std::max<int64_t>(1, chunk_bytes / (64 * col_all)));
  const int64_t rows_per = cgs_per * 64;
  const size_t off_s = mg_align((size_t)(rows_per * col_b));
  const size_t off_z = off_s + mg_align((size_t)(rows_per * col_s));
  const size_t slot = off_z + mg_align((size_t)(rows_per * col_z));
  hipStream_t st = ctx->stream;
  uint8_t *pinned[2], *stage[2];
  auto run = [&]() -> mg_status {
    MG_TRY(upload_slots(ctx, slot));
    for (int i = 0; i < 2; i++) {
      pinned[i] = static_cast<uint8_t *>(ctx->up_pin) + i * slot;
      stage[i] = static_cast<uint8_t *>(ctx->up_dev) + i * slot;
    }
    hipEvent_t *done = ctx->up_done;
    for (int64_t ci = 0, cg0 = 0; cg0 < ng; ci++, cg0 += cgs_per) {
      const int sl = (int)(ci & 1);
      const int64_t cgs = std::min(cgs_per, ng - cg0);
      const int64_t n0 = cg0 * 64, n1 = std::min(N, (cg0 + cgs) * 64);
      const int64_t rows = std::max<int64_t>(0, n1 - n0);
      if (ci >= 2) MG_HIP(hipEventSynchronize(done[sl]));  // the slot's last copy and kernels
      MG_TRY(read_source(b, files.fd[0], n0 * col_b, rows * col_b, pinned[sl]));
      MG_TRY(read_source(scales, files.fd[1], n0 * col_s, rows * col_s, pinned[sl] + off_s));
      if (col_z) MG_TRY(read_source(zp, files.fd[2], n0 * col_z, rows * col_z, pinned[sl] + off_z));
      if (rows > 0) MG_HIP(hipMemcpyAsync(stage[sl], pinned[sl], slot, hipMemcpyHostToDevice, st));
      const int64_t ncodes = cgs * c4 * 1024, ntab = cgs * nb * 64;
      hipLaunchKernelGGL(k_nbits_repack_codes, dim3((unsigned)((ncodes + 255) / 256)), dim3(256),
                         0, st, reinterpret_cast<const uint32_t *>(stage[sl]), n0, N, nb, bs, c4,
                         cg0, cgs, d.wq);
      hipLaunchKernelGGL(k_nbits_repack_tables, dim3((unsigned)((ntab + 255) / 256)), dim3(256),
                         0, st, reinterpret_cast<const float *>(stage[sl] + off_s),
                         stage[sl] + off_z, zp_kind, n0, N, nb, nbh, cg0, cgs, d.scales, d.zp4,
                         d.zpf);
      MG_TRY(mg_launch_check("k_nbits_repack"));
      MG_HIP(hipEventRecord(done[sl], st));
    }
    MG_HIP(hipStreamSynchronize(st));
    return MG_OK;
  };
  mg_status status = run();
  (void)hipStreamSynchronize(st);  // the slots are free for the next upload
  if (status == MG_OK && ctx->prefill_images && mg_nbits_f8_eligible(d))
    status = mg_nbits_f8_images(ctx, w);
  return status;
}

void mg_nbits_free(mg_weight *w) {
  mg_nbits_dev &d = w->nbits;
  if (d.wq) (void)hipFree(d.wq);
  if (d.img) (void)hipFree(d.img);
  if (d.scales) (void)hipFree(d.scales);
  if (d.zp4) (void)hipFree(d.zp4);
  if (d.zpf) (void)hipFree(d.zpf);
  if (d.bias) (void)hipFree(d.bias);
  d = mg_nbits_dev{};
}

size_t mg_nbits_ws_bytes(const mg_ctx *ctx, const mg_weight *w, int64_t M) {
  return plan_nbits(ctx, w, M, w->nbits.ng, w->N, w->nbits.img != nullptr).total;
}

namespace {
// The plan of a group of weights launched together: member 0's kind of path,
// sized for all members.
NbitsPlan plan_group(const mg_ctx *ctx, int n, const mg_weight *const *w, int64_t M) {
  int64_t ng = 0, nn = 0;
  bool imgs = true;  // every member has prefill images
  for (int i = 0; i < n; i++) {
    ng += w[i]->nbits.ng;
    nn += w[i]->N;
    imgs = imgs && w[i]->nbits.img != nullptr;
  }
  return plan_nbits(ctx, w[0], M, ng, nn, imgs);
}
}  // namespace

size_t mg_nbits_group_ws_bytes(const mg_ctx *ctx, int n, const mg_weight *const *w,
                               int64_t M) {
  return plan_group(ctx, n, w, M).total;
}

namespace {
mg_status nbits_run_f32(mg_ctx *ctx, const mg_weight *w, const float *a_dev, int64_t M,
                        float *y_dev, float *wd, int64_t chunk);
mg_status prefill_run(mg_ctx *ctx, int n, const mg_weight *const *w, const float *a_dev,
                      int64_t M, float *const *y_dev, void *ws, const NbitsPlan &p);
}  // namespace

mg_status mg_nbits_run_group(mg_ctx *ctx, int n, const mg_weight *const *w,
                             const float *a_dev, int64_t M, float *const *y_dev, void *ws,
                             const void *split) {
  if (M == 0 || n == 0) return MG_OK;
  int64_t ng = 0;
  for (int i = 0; i < n; i++) ng += w[i]->nbits.ng;
  const mg_weight *w0 = w[0];
  const mg_nbits_dev &d = w0->nbits;
  const NbitsPlan p = plan_group(ctx, n, w, M);
  hipStream_t st = ctx->stream;
  char *base = static_cast<char *>(ws);
  if (p.path == 0) {
    GemvSet gs = make_set(n, w, y_dev);
    const int vec = (reinterpret_cast<uintptr_t>(a_dev) % 16 == 0 && w0->K % 4 == 0) ? 1 : 0;
    float *part = reinterpret_cast<float *>(base);
    ReduceSet rs{};
    int64_t eend = 0;
    if (p.ksplit > 1) {
      rs.n = n;
      int64_t poff = 0;
      for (int i = 0; i < n; i++) {
        gs.part_off[i] = rs.part_off[i] = poff;
        poff += (int64_t)p.ksplit * M * w[i]->N;
        eend += M * w[i]->N;
        rs.e_end[i] = eend;
        rs.bias[i] = w[i]->nbits.bias;
        rs.y[i] = y_dev[i];
        rs.N[i] = (int)w[i]->N;
      }
    }
    switch (M) {
      case 1: launch_gemv_q<1>(w0, gs, p, st, a_dev, vec, part); break;
      case 2: launch_gemv_q<2>(w0, gs, p, st, a_dev, vec, part); break;
      case 3: launch_gemv_q<3>(w0, gs, p, st, a_dev, vec, part); break;
      default: launch_gemv_q<4>(w0, gs, p, st, a_dev, vec, part); break;
    }
    MG_TRY(mg_launch_check("k_gemv_dot8"));
    if (p.ksplit > 1) return launch_gemm_reduce(st, part, rs, eend, p.ksplit);
    return MG_OK;
  }
  if (p.path == 3) {
    GemvSet gs = make_set(n, w, y_dev);
    float *part = p.ksplit > 1 ? reinterpret_cast<float *>(base + p.off_c) : nullptr;
    ReduceSet rs{};
    int64_t eend = 0;
    if (p.ksplit > 1) {
      rs.n = n;
      int64_t poff = 0;
      for (int i = 0; i < n; i++) {
        gs.part_off[i] = rs.part_off[i] = poff;
        poff += (int64_t)p.ksplit * M * w[i]->N;
        eend += M * w[i]->N;
        rs.e_end[i] = eend;
        rs.bias[i] = w[i]->nbits.bias;
        rs.y[i] = y_dev[i];
        rs.N[i] = (int)w[i]->N;
      }
    }
    uint4 *ahl = reinterpret_cast<uint4 *>(base + p.off_a);
    int *texp = reinterpret_cast<int *>(base + p.off_b);
    const int vec = (w0->K % 4 == 0) && (reinterpret_cast<uintptr_t>(a_dev) % 16 == 0);
    if (split) {  // written by the producer of a (same layout as the prepass's)
      ahl = static_cast<uint4 *>(const_cast<void *>(split));
      texp = reinterpret_cast<int *>(static_cast<char *>(const_cast<void *>(split)) +
                                     mg_align((size_t)16 * d.kpad * 4));
    } else {
      const int per = (int)((d.c4 * 16 + 255) / 256);  // octets per thread
#define MG_SPLIT16(P_)                                                                          \
  hipLaunchKernelGGL((k_af16split16<P_>), dim3(16), dim3(256), 0, st, a_dev, M, w0->K,        \
                     (int)d.c4, vec, ahl, texp)
      if (per == 1) MG_SPLIT16(1);
      else if (per == 2) MG_SPLIT16(2);
      else if (per <= 4) MG_SPLIT16(4);
      else MG_SPLIT16(0);
#undef MG_SPLIT16
      MG_TRY(mg_launch_check("k_af16split16"));
    }
    const int has_zp = d.zp_kind == MG_ZP_UINT4;
    const int segj = (int)(std::min<int64_t>(d.bs, KGRP) / 32);
    // Waves per workgroup: 4 for wide weights; narrow ones (fewer than two
    // workgroups per CU) split K over 8 waves, so that their few workgroups
    // keep more k groups' loads in flight.  (16 waves would cap the kernel
    // at 128 registers and spill.)  The widest (at least four workgroups of
    // whole column groups per CU) take one wave: all k groups in one wave
    // behind one prologue, no cross-wave sum, four times the workgroups
    // resident per CU (Llama lm_head 2048 x 128256 at M = 4 / 16: 50.5 /
    // 51.1 us with 4 waves, 47.2 / 47.9 with 2, 44.0 / 44.7 with 1).
    // Tiles per workgroup: narrow weights (fewer column groups than CUs)
    // take 2 or 1 of a column group's four 16-column tiles per workgroup.
#ifndef MG_GEMV16_WG_PER_CU
#define MG_GEMV16_WG_PER_CU 1
#endif
    const int64_t cus = std::max(ctx->num_cus, 1) * (int64_t)MG_GEMV16_WG_PER_CU;
    const bool ksplit = p.ksplit > 1;
    const int tpw = ksplit || ng >= cus ? 4 : (2 * ng >= cus ? 2 : 1);
    const int64_t wgs = ng * (4 / tpw);
    int nw = 4;
    if (ksplit ? p.kps >= 8 : (wgs < 2 * cus && d.c4 >= 8)) nw = 8;
    if (!ksplit && wgs >= 4 * cus && tpw == 4) nw = 1;
#define MG_DEC_LAUNCH(SJ_, NW_, TPW_)                                                      \
  hipLaunchKernelGGL((k_gemv_mfma<SJ_, NW_, TPW_>), dim3((unsigned)wgs, (unsigned)p.ksplit), \
                     dim3(NW_ * 64), 0, st, ahl, texp, gs, (int)M, (int)d.c4, (int)d.nb,    \
                     (int)d.nbh, __builtin_ctzll(d.bs), has_zp, p.kps, part)
#define MG_DEC_TPW(SJ_, NW_)                  \
  if (tpw == 4) MG_DEC_LAUNCH(SJ_, NW_, 4);  \
  else if (tpw == 2) MG_DEC_LAUNCH(SJ_, NW_, 2); \
  else MG_DEC_LAUNCH(SJ_, NW_, 1)
#define MG_DEC_NW(SJ_)               \
  if (nw == 8) { MG_DEC_TPW(SJ_, 8); } \
  else if (nw == 1) { MG_DEC_LAUNCH(SJ_, 1, 4); } \
  else { MG_DEC_TPW(SJ_, 4); }
    if (segj == 1) { MG_DEC_NW(1); }
    else if (segj == 2) { MG_DEC_NW(2); }
    else { MG_DEC_NW(4); }
#undef MG_DEC_NW
#undef MG_DEC_TPW
#undef MG_DEC_LAUNCH
    MG_TRY(mg_launch_check("k_gemv_mfma"));
    if (ksplit) return launch_gemm_reduce(st, part, rs, eend, p.ksplit);
    return MG_OK;
  }
  if (p.path == 1) return prefill_run(ctx, n, w, a_dev, M, y_dev, ws, p);
  if (p.path == 4)
    return mg_nbits_prefill_f8(ctx, n, w, a_dev, M, y_dev, ws, p.mpad, p.nt, p.ksplit, p.kps,
                               p.off_c, p.kwave);
  // Float zero points / 16-k blocks: one weight at a time.
  for (int i = 0; i < n; i++)
    MG_TRY(nbits_run_f32(ctx, w[i], a_dev, M, y_dev[i], static_cast<float *>(ws), p.chunk));
  return MG_OK;
}

mg_status mg_nbits_run(mg_ctx *ctx, const mg_weight *w, const float *a_dev,
                       int64_t M, float *y_dev, void *ws) {
  return mg_nbits_run_group(ctx, 1, &w, a_dev, M, &y_dev, ws);
}

namespace {
// Prefill: one activation prepass shared by the n weights, one GEMM launch
// over their concatenated column tiles, and (split K) one reduction launch.
mg_status prefill_run(mg_ctx *ctx, int n, const mg_weight *const *w, const float *a_dev,
                      int64_t M, float *const *y_dev, void *ws, const NbitsPlan &p) {
  const mg_weight *w0 = w[0];
  const mg_nbits_dev &d = w0->nbits;
  hipStream_t st = ctx->stream;
  char *base = static_cast<char *>(ws);
  uint4 *ahl = reinterpret_cast<uint4 *>(base + p.off_a);
  int *texp = reinterpret_cast<int *>(base + p.off_b);
  float *part = p.ksplit > 1 ? reinterpret_cast<float *>(base + p.off_c) : nullptr;
  const int vec = (w0->K % 4 == 0) && (reinterpret_cast<uintptr_t>(a_dev) % 16 == 0);
  {
    const int ul = (int)((d.c4 * 8 + 63) / 64);  // 16-k pieces per lane
#define MG_SPLIT_LAUNCH(UL_)                                                                   \
  hipLaunchKernelGGL((k_af16split<UL_>), dim3((unsigned)(p.mpad / 4)), dim3(256), 0, st, a_dev, \
                     M, w0->K, (int)d.c4, vec, ahl, texp)
    if (ul == 1) MG_SPLIT_LAUNCH(1);
    else if (ul == 2) MG_SPLIT_LAUNCH(2);
    else if (ul == 3) MG_SPLIT_LAUNCH(3);
    else if (ul == 4) MG_SPLIT_LAUNCH(4);
    else MG_SPLIT_LAUNCH(0);
#undef MG_SPLIT_LAUNCH
  }
  MG_TRY(mg_launch_check("k_af16split"));
  const int has_zp = d.zp_kind == MG_ZP_UINT4;
  PrefillSet ps{};
  ReduceSet rs{};
  int ct = 0;
  int64_t eend = 0;
  make_prefill_sets(n, w, y_dev, M, p.ksplit, p.nt, &ps, &rs, &ct, &eend);
  const int mtiles = (int)(p.mpad / 128);
  const dim3 grid((unsigned)(8 * mtiles * ((ct + 7) / 8)), (unsigned)p.ksplit);
  const int segj = (int)(std::min<int64_t>(d.bs, KGRP) / 32);
#define MG_GEMM_LAUNCH(SJ_, NT_)                                                           \
  hipLaunchKernelGGL((k_gemm_f16split<SJ_, NT_>), grid, dim3(256), 0, st, ahl, texp, ps, part, \
                     (int)M, (int)d.c4, (int)d.nb, (int)d.nbh, __builtin_ctzll(d.bs), has_zp, \
                     mtiles, ct, p.kps)
  if (p.nt == 4) {
    if (segj == 1) MG_GEMM_LAUNCH(1, 4);
    else if (segj == 2) MG_GEMM_LAUNCH(2, 4);
    else MG_GEMM_LAUNCH(4, 4);
  } else {
    if (segj == 1) MG_GEMM_LAUNCH(1, 2);
    else if (segj == 2) MG_GEMM_LAUNCH(2, 2);
    else MG_GEMM_LAUNCH(4, 2);
  }
#undef MG_GEMM_LAUNCH
  MG_TRY(mg_launch_check("k_gemm_f16split"));
  if (p.ksplit > 1) MG_TRY(launch_gemm_reduce(st, part, rs, eend, p.ksplit));
  return MG_OK;
}

mg_status nbits_run_f32(mg_ctx *ctx, const mg_weight *w, const float *a_dev, int64_t M,
                        float *y_dev, float *wd, int64_t chunk) {
  const mg_nbits_dev &d = w->nbits;
  const int64_t N = w->N, K = w->K;
  for (int64_t n0 = 0; n0 < N; n0 += chunk) {
    const int64_t nc = std::min(chunk, N - n0);
    const int64_t threads = nc * d.c4 * 16;
    hipLaunchKernelGGL(k_nbits_dequant_f32, dim3((unsigned)((threads + 255) / 256)), dim3(256),
                       0, ctx->stream, reinterpret_cast<const uint32_t *>(d.wq), d.scales,
                       d.zp4, d.zpf, (int)d.zp_kind, n0, nc, K, (int)d.c4, (int)d.nb,
                       (int)d.nbh, (int)d.bs, wd);
    MG_TRY(mg_launch_check("k_nbits_dequant_f32"));
    // Y[:, n0 : n0 + nc] = A * Wd^T (+ bias): Wd is [nc][K], row stride of Y is N.
    mg_f32_problem q{};
    q.M = M;
    q.N = nc;
    q.K = K;
    q.batch = 1;
    q.lda = K;
    q.ldb = K;
    q.trans_b = 1;
    q.alpha = 1.f;
    q.beta = 1.f;
    q.c = d.bias ? d.bias + n0 : nullptr;
    q.c_rs = 0;
    q.c_cs = 1;
    q.ldy = N;
    MG_TRY(mg_f32_run(ctx, q, a_dev, wd, y_dev + n0));
  }
  return MG_OK;
}
}  // namespace
