// MatMulNBits (int4, block-quantized) on gfx950.
//
// Reference semantics: opMatMulNBits, lib/src/onnx_qlinear_ops.dart:115-228:
//   y[m, n] = sum_k a[m, k] * fl32((q[n, k] - zp[n, blk]) * s[n, blk]) (+ bias[n])
// with q the 4-bit code (low nibble = even k), blk = k / block_size and the
// zero point 8 by default, packed uint4, or float.
//
// Device weight layout (built once on upload, mg_nbits_upload):
//   columns are grouped by 64 ("column group"), k by 128 ("k group").
//   wq[cg][kg][g][col][j] is one dword holding the 8 nibbles of column
//   (cg*64 + col) at k = kg*128 + 32*j + 8*g + t, t = 0..7, with even t in the
//   low half-word and odd t in the high half-word (nibble position
//   t/2 resp. 4 + t/2).  A lane reading 16 bytes at (g, col) gets j = 0..3.
//   scales[cg][blk][col], zero points zp4[cg][blk/2][col] (original packed
//   byte) or zpf[cg][blk][col].
//
// Two compute paths:
//   * M <= 4 ("decode"): activations are quantised per (row, 128-or-block k
//     slice) to 15-bit fixed point split into four signed int4 digits; each
//     lane owns one column and streams 16-byte weight loads, multiplying with
//     v_dot8_i32_i4 against the digit planes (wave-uniform, scalar-loaded).
//     Zero point and scale are applied once per block in fp32.
//   * M > 4 ("prefill"): activations become an fp16 pair hi + lo (scaled by a
//     power of two per row and 128-k slice, so hi + lo carries ~22 bits of each
//     element); each workgroup unpacks its weight tile once into LDS as exact
//     fp16 (q - zp); v_mfma_f32_16x16x32_f16 accumulates hi*W and lo*W in fp32
//     and the block scale is applied on the fp32 accumulator.
// Rare forms (float zero points or block_size 16 with M > 4) take a simple
// per-output kernel.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <thread>
#include <vector>

#include "mg_internal.h"

namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float float4v __attribute__((ext_vector_type(4)));

constexpr int KGRP = 128;  // k per k group
constexpr int CGRP = 64;   // columns per column group
constexpr int FIX_MAX = 30583;  // 7 * (1 + 16 + 256 + 4096): 4 balanced int4 digits

__host__ __device__ inline int nib_pos(int t) {
  return (t & 1) ? 4 + (t >> 1) : (t >> 1);
}

// ------------------------------------------------------------- prepasses

// Activations -> int4 digit planes for the decode path.  One wave per
// (row, qblock); qblock = min(block_size, 128) consecutive k.
//   dig[row][kg][g][j][d]: digit plane d of the 8 k of dword (g, j), nibble
//   order as in wq; alpha[row][qb] = dequant step; rsum[row][qb] = sum of the
//   fixed-point values (for the zero-point term).
__global__ __launch_bounds__(256) void k_adigits(
    const float *__restrict__ a, int64_t M, int64_t K, int qb, int nqb,
    int c4n, uint32_t *__restrict__ dig, float *__restrict__ alpha,
    int *__restrict__ rsum) {
  const int64_t widx = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (widx >= M * nqb) return;
  const int64_t row = widx / nqb;
  const int qbi = (int)(widx % nqb);
  const int64_t k0 = (int64_t)qbi * qb;
  const float *ar = a + row * K;
  float mx = 0.f;
  int bad = 0;
  for (int i = lane; i < qb; i += 64) {
    const int64_t k = k0 + i;
    const float v = k < K ? ar[k] : 0.f;
    if (!isfinite(v)) bad = 1;
    mx = fmaxf(mx, fabsf(v));
  }
  for (int o = 32; o > 0; o >>= 1) {
    mx = fmaxf(mx, __shfl_xor(mx, o));
    bad |= __shfl_xor(bad, o);
  }
  const float inv = (mx > 0.f && !bad) ? (float)FIX_MAX / mx : 0.f;
  int rs = 0;
  for (int d = lane; d < qb / 8; d += 64) {
    const int64_t kb = k0 + 8 * d;
    uint32_t dg[4] = {0u, 0u, 0u, 0u};
    for (int t = 0; t < 8; t++) {
      const int64_t k = kb + t;
      const float v = k < K ? ar[k] : 0.f;
      int fix = (int)rintf(v * inv);
      fix = min(max(fix, -FIX_MAX), FIX_MAX);
      rs += fix;
      const int p = nib_pos(t);
      int x = fix;
      for (int dd = 0; dd < 4; dd++) {
        const int di = ((x + 8) & 15) - 8;
        x = (x - di) >> 4;
        dg[dd] |= (uint32_t)(di & 15) << (4 * p);
      }
    }
    const int kg = (int)(kb / KGRP);
    const int rem = (int)(kb % KGRP);
    const int j = rem / 32, g = (rem % 32) / 8;
    uint32_t *o = dig + (((row * c4n + kg) * 4 + g) * 16 + j * 4);
    o[0] = dg[0];
    o[1] = dg[1];
    o[2] = dg[2];
    o[3] = dg[3];
  }
  for (int o = 32; o > 0; o >>= 1) rs += __shfl_xor(rs, o);
  if (lane == 0) {
    alpha[row * nqb + qbi] =
        bad ? __builtin_nanf("") : (mx > 0.f ? mx / (float)FIX_MAX : 0.f);
    rsum[row * nqb + qbi] = rs;
  }
}

// Activations -> fp16 hi/lo fragments for the MFMA path.  One workgroup per
// (16-row subtile, k group): 256 threads, thread t owns row t/16 and the 8
// consecutive k at 8*(t%16) of the group.  Output ahl[m16][kg][j][hl][lane]
// (uint4 = 8 fp16): MFMA lane (r = lane%16, g = lane/16) holds row r,
// k = kg*128 + 32*j + 8*g + 0..7.  Each row's 128-k slice is scaled by 2^e so
// that its max magnitude lies in [2^13, 2^14): far from fp16 overflow, and
// hi = fp16(x), lo = fp16(x - hi) keeps ~22 bits of every element.
// texp[m16][kg][row] = e is undone with the block scale on the fp32
// accumulator.
__global__ __launch_bounds__(256) void k_af16split(
    const float *__restrict__ a, int64_t M, int64_t K, int c4n, int vec,
    uint4 *__restrict__ ahl, int *__restrict__ texp) {
  const int t = threadIdx.x;
  const int kg = blockIdx.x;
  const int64_t m16 = blockIdx.y;
  const int r = t >> 4, c8 = t & 15;
  const int64_t row = m16 * 16 + r;
  const int64_t k0 = (int64_t)kg * KGRP + 8 * c8;
  float v[8];
  if (row < M && vec && k0 + 8 <= K) {
    const float4 *src = reinterpret_cast<const float4 *>(a + row * K + k0);
    const float4 x0 = src[0], x1 = src[1];
    v[0] = x0.x; v[1] = x0.y; v[2] = x0.z; v[3] = x0.w;
    v[4] = x1.x; v[5] = x1.y; v[6] = x1.z; v[7] = x1.w;
  } else {
#pragma unroll
    for (int i = 0; i < 8; i++) v[i] = (row < M && k0 + i < K) ? a[row * K + k0 + i] : 0.f;
  }
  float mx = 0.f;
#pragma unroll
  for (int i = 0; i < 8; i++) mx = fmaxf(mx, fabsf(v[i]));
  // The 16 threads of a row are 16 consecutive lanes of one wave.
  for (int o = 8; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
  int e = 0;
  if (mx > 0.f && isfinite(mx)) {
    int ex;
    frexpf(mx, &ex);
    e = 14 - ex;
  }
  half8 hi, lo;
#pragma unroll
  for (int i = 0; i < 8; i++) {
    const float x = ldexpf(v[i], e);
    const _Float16 h = (_Float16)x;
    float res = x - (float)h;
    if (!isfinite(res)) res = 0.f;
    hi[i] = h;
    lo[i] = (_Float16)res;
  }
  const int j = c8 >> 2, g = c8 & 3, lane = g * 16 + r;
  uint4 *o = ahl + (((m16 * c4n + kg) * 4 + j) * 2) * 64 + lane;
  o[0] = __builtin_bit_cast(uint4, hi);
  o[64] = __builtin_bit_cast(uint4, lo);
  if (c8 == 0) texp[(m16 * c4n + kg) * 16 + r] = e;
}

// ---------------------------------------------------------- decode GEMV

// MR activation rows; QPG = qblocks per k group (128 / min(bs, 128));
// ZPK = zero-point kind.  Grid (column groups, k slices); 4 waves per
// workgroup, each wave a different k slice of the same 64 columns.
template <int MR, int QPG, int ZPK>
__global__ __launch_bounds__(256) void k_gemv_dot8(
    const uint4 *__restrict__ wq, const float *__restrict__ scales,
    const uint8_t *__restrict__ zp4, const float *__restrict__ zpf,
    const uint32_t *__restrict__ dig, const float *__restrict__ alpha,
    const int *__restrict__ rsum, const float *__restrict__ bias,
    float *__restrict__ y, float *__restrict__ part, int N, int c4n, int nb,
    int nbh, int bs, int nqb, int ncolp) {
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int cgi = blockIdx.x;
  const int nslices = gridDim.y * 4;
  const int slice = blockIdx.y * 4 + wave;
  const int qb = KGRP / QPG;
  float yacc[MR];
#pragma unroll
  for (int r = 0; r < MR; r++) yacc[r] = 0.f;

  for (int kg = slice; kg < c4n; kg += nslices) {
    int acc[MR][QPG][4];
#pragma unroll
    for (int r = 0; r < MR; r++)
#pragma unroll
      for (int s = 0; s < QPG; s++)
#pragma unroll
        for (int d = 0; d < 4; d++) acc[r][s][d] = 0;
    const uint4 *wp = wq + (((int64_t)cgi * c4n + kg) * 4) * 64 + lane;
#pragma unroll
    for (int g = 0; g < 4; g++) {
      const uint4 w = wp[g * 64];
      const uint32_t wv[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const int x = (int)(wv[j] ^ 0x88888888u);
        const int slot = QPG == 1 ? 0 : (QPG == 2 ? j / 2 : (QPG == 4 ? j : 2 * j + g / 2));
#pragma unroll
        for (int r = 0; r < MR; r++) {
          const uint32_t *dr =
              dig + ((((int64_t)r * c4n + kg) * 4 + g) * 16 + j * 4);
#pragma unroll
          for (int d = 0; d < 4; d++)
            acc[r][slot][d] =
                __builtin_amdgcn_sdot8((int)dr[d], x, acc[r][slot][d], false);
        }
      }
    }
#pragma unroll
    for (int s = 0; s < QPG; s++) {
      const int qbi = kg * QPG + s;
      const int b = (int)(((int64_t)qbi * qb) / bs);
      if (b >= nb) continue;  // k padding beyond the last block
      const float sc = scales[((int64_t)cgi * nb + b) * 64 + lane];
      int zc = 0;
      float zf = 8.f;
      if (ZPK == 1) {
        const uint8_t zb = zp4[((int64_t)cgi * nbh + b / 2) * 64 + lane];
        zc = 8 - ((b & 1) ? (zb >> 4) : (zb & 15));
      } else if (ZPK == 2) {
        zf = zpf[((int64_t)cgi * nb + b) * 64 + lane];
      }
#pragma unroll
      for (int r = 0; r < MR; r++) {
        const int comb =
            ((acc[r][s][3] * 16 + acc[r][s][2]) * 16 + acc[r][s][1]) * 16 +
            acc[r][s][0];
        const float al = alpha[(int64_t)r * nqb + qbi];
        const int R = rsum[(int64_t)r * nqb + qbi];
        float v;
        if (ZPK == 2)
          v = (float)comb + (8.f - zf) * (float)R;
        else
          v = (float)(comb + zc * R);
        yacc[r] += (al * sc) * v;
      }
    }
  }
  __shared__ float red[4][MR][64];
#pragma unroll
  for (int r = 0; r < MR; r++) red[wave][r][lane] = yacc[r];
  __syncthreads();
  if (wave == 0) {
    const int col = cgi * 64 + lane;
#pragma unroll
    for (int r = 0; r < MR; r++) {
      const float s = red[0][r][lane] + red[1][r][lane] + red[2][r][lane] +
                      red[3][r][lane];
      if (gridDim.y == 1) {
        if (col < N) y[(int64_t)r * N + col] = s + (bias ? bias[col] : 0.f);
      } else {
        part[((int64_t)blockIdx.y * MR + r) * ncolp + col] = s;
      }
    }
  }
}

__global__ void k_gemv_reduce(const float *__restrict__ part,
                              const float *__restrict__ bias,
                              float *__restrict__ y, int M, int N, int ncolp,
                              int ksplit) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (int64_t)M * N) return;
  const int r = (int)(idx / N), c = (int)(idx % N);
  float s = 0.f;
  for (int ks = 0; ks < ksplit; ks++) s += part[((int64_t)ks * M + r) * ncolp + c];
  y[idx] = s + (bias ? bias[c] : 0.f);
}

// --------------------------------------------------------- prefill GEMM

// Dequantises one weight dword (8 codes, nibble order of wq) to 8 exact fp16
// values q - zp: the half-word (1024 + q) is built by masking into the fp16
// pattern 0x6400 and zz = -(1024 + zp) is added in packed fp16.
__device__ inline uint4 deq8(uint32_t x, half2v zz) {
  uint32_t r[4];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const uint32_t h = ((x >> (4 * i)) & 0x000F000Fu) | 0x64006400u;
    r[i] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2v, h) + zz);
  }
  return make_uint4(r[0], r[1], r[2], r[3]);
}

// Workgroup tile: (64*WM) rows x 128 columns (two column groups), 4 waves;
// wave w owns rows [16*WM*w, +16*WM) of the tile and all 128 columns
// (WM x 8 MFMA subtiles of 16x16).  Per k group (128 k):
//   * the workgroup dequantises the 128x128 weight tile once into LDS, in
//     MFMA B-fragment order (double-buffered; the packed codes of the next k
//     group are loaded while the current one computes);
//   * each wave streams its activation fragments (hi and lo) from global,
//     two 32-k steps ahead of use, and issues the hi MFMAs of a step for all
//     subtiles before the lo MFMAs, into a per-segment fp32 accumulator D;
//   * at the end of each scale segment (SEGJ steps = min(block_size, 128) k)
//     the block scale times the row's 2^-e is applied: acc += s * 2^-e * D.
// Grid: x = tiles in XCD-aware order (workgroup L runs on XCD L % 8; all row
// tiles of one column tile get the same L % 8, so its weights are read from
// HBM once into that XCD's L2); y = k splits, each over kps k groups, whose
// partial sums go to `part` and are added by k_gemm_reduce (ksplit > 1).
template <int WM, int SEGJ>
__global__ __launch_bounds__(256, 2) void k_gemm_f16split(
    const uint4 *__restrict__ ahl, const int *__restrict__ texp,
    const uint4 *__restrict__ wq, const float *__restrict__ scales,
    const uint8_t *__restrict__ zp4, const float *__restrict__ bias,
    float *__restrict__ y, float *__restrict__ part, int M, int N, int c4n,
    int nb, int nbh, int bs, int has_zp, int mtiles, int ntiles, int kps) {
  __shared__ uint4 bl[2][8 * 4 * 64];
  __shared__ float scl[2][4][16][8];  // [buf][segment][col % 16][subtile]
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int L = blockIdx.x;
  const int xcd = L & 7, q = L >> 3;
  const int mt = q % mtiles;
  const int nt = (q / mtiles) * 8 + xcd;
  if (nt >= ntiles) return;
  const int ks = blockIdx.y;
  const int kg0 = ks * kps;
  const int kg1 = min(c4n, kg0 + kps);
  const int m16w = (mt * 4 + wave) * WM;
  const int cl = lane & 15, lg = lane >> 4;

  // Cooperative dequantisation: thread t handles packed uint4 u = t, t + 256
  // -> (column group 2*nt + (u >> 8), g = (u >> 6) & 3, col = u & 63).  The
  // thread with g = s also stages the column's scale of segment s (threads
  // with g >= segments per k group write an unused slot).
  const int dq_g = wave;  // (t >> 6) & 3
  int dq_cgi[2], dq_col[2], dq_dst[2], dq_ns[2];
#pragma unroll
  for (int h = 0; h < 2; h++) {
    const int u = t + 256 * h;
    dq_cgi[h] = 2 * nt + (u >> 8);
    dq_col[h] = u & 63;
    dq_ns[h] = (u >> 8) * 4 + (dq_col[h] >> 4);
    dq_dst[h] = dq_ns[h] * 4 * 64 + dq_g * 16 + (dq_col[h] & 15);
  }
  const int nbm1 = nb - 1, nbhm1 = nbh - 1;
  struct Meta {
    uint4 pk[2];
    uint32_t zb[2];  // zero-point byte(s) of the k group, first block's byte low
    float sc[2];
  };
  // Branch-free: indices are clamped, out-of-range blocks (k padding) give a
  // zero scale.
  auto load_meta = [&](int kg, Meta &m) {
    const int blk0 = (kg * KGRP) / bs;
    const int blks = (kg * KGRP + 32 * SEGJ * dq_g) / bs;
    const int zbyte0 = min(blk0 / 2, nbhm1), zbyte1 = min(blk0 / 2 + 1, nbhm1);
#pragma unroll
    for (int h = 0; h < 2; h++) {
      const int64_t cgi = dq_cgi[h];
      m.pk[h] = wq[((cgi * c4n + kg) * 4 + dq_g) * 64 + dq_col[h]];
      uint32_t zb = zp4[(cgi * nbh + zbyte0) * 64 + dq_col[h]];
      if (SEGJ == 1) zb |= (uint32_t)zp4[(cgi * nbh + zbyte1) * 64 + dq_col[h]] << 8;
      m.zb[h] = zb;
      const float sv = scales[(cgi * nb + min(blks, nbm1)) * 64 + dq_col[h]];
      m.sc[h] = blks < nb ? sv : 0.f;
    }
  };
  // Dequantises step j of both packed uint4 into LDS buffer `buf`.
  auto dequant_step = [&](int kg, const Meta &m, int buf, int j) {
    const int blk0 = (kg * KGRP) / bs;
    const int blk = (kg * KGRP + 32 * j) / bs;
    const int sh = ((blk & 1) + 2 * (blk / 2 - blk0 / 2)) * 4;
#pragma unroll
    for (int h = 0; h < 2; h++) {
      const uint32_t w = j == 0 ? m.pk[h].x : j == 1 ? m.pk[h].y : j == 2 ? m.pk[h].z : m.pk[h].w;
      const int z = has_zp ? (int)((m.zb[h] >> sh) & 15u) : 8;
      const _Float16 zh = (_Float16)(-(1024.f + (float)z));
      bl[buf][dq_dst[h] + j * 64] = deq8(w, (half2v){zh, zh});
    }
    if (j == 0) {
#pragma unroll
      for (int h = 0; h < 2; h++) scl[buf][dq_g][dq_col[h] & 15][dq_ns[h]] = m.sc[h];
    }
  };
  // Activation fragment of step (kg, j) for row subtile i: hi at +0, lo at +64.
  const uint4 *abase = ahl + (int64_t)m16w * c4n * 512 + lane;
  auto a_ptr = [&](int kg, int j, int i) { return abase + ((int64_t)i * c4n + kg) * 512 + j * 128; };

  float4v acc[WM][8], D[WM][8];
#pragma unroll
  for (int i = 0; i < WM; i++)
#pragma unroll
    for (int n = 0; n < 8; n++) acc[i][n] = (float4v){0.f, 0.f, 0.f, 0.f};
  const float4v zero4 = (float4v){0.f, 0.f, 0.f, 0.f};

  // Ring of activation fragments (slot = j), loaded PD steps ahead of use:
  // two steps for one row subtile per wave, one step for two (registers).
  // Loads past the last k group re-read it (results unused).
  constexpr int PD = WM == 1 ? 2 : 1;
  uint4 ah[4][WM], al[4][WM];
#pragma unroll
  for (int jj = 0; jj < PD; jj++)
#pragma unroll
    for (int i = 0; i < WM; i++) {
      ah[jj][i] = a_ptr(kg0, jj, i)[0];
      al[jj][i] = a_ptr(kg0, jj, i)[64];
    }
  {
    Meta m0;
    load_meta(kg0, m0);
#pragma unroll
    for (int j = 0; j < 4; j++) dequant_step(kg0, m0, 0, j);
  }
  __syncthreads();

  for (int kg = kg0; kg < kg1; kg++) {
    const int buf = (kg - kg0) & 1;
    const int kgn = min(kg + 1, kg1 - 1);  // next k group (clamped)
    Meta mnext;
    load_meta(kgn, mnext);
    int4 ex[WM];  // row exponents of the lane's four output rows
#pragma unroll
    for (int i = 0; i < WM; i++)
      ex[i] = reinterpret_cast<const int4 *>(texp)[((int64_t)(m16w + i) * c4n + kg) * 4 + lg];
#pragma unroll
    for (int j = 0; j < 4; j++) {
      {
        const int jn = (j + PD) & 3;
        const int kn = min(kg + ((j + PD) >> 2), kg1 - 1);
#pragma unroll
        for (int i = 0; i < WM; i++) {
          ah[jn][i] = a_ptr(kn, jn, i)[0];
          al[jn][i] = a_ptr(kn, jn, i)[64];
        }
      }
      // Column subtiles in pairs: the hi MFMAs of a pair, then its lo MFMAs
      // (each lo depends on the hi issued 2*WM MFMAs earlier).
#pragma unroll
      for (int p2 = 0; p2 < 4; p2++) {
        const half8 b0 = __builtin_bit_cast(half8, bl[buf][((2 * p2) * 4 + j) * 64 + lane]);
        const half8 b1 = __builtin_bit_cast(half8, bl[buf][((2 * p2 + 1) * 4 + j) * 64 + lane]);
#pragma unroll
        for (int i = 0; i < WM; i++) {
          const half8 a_h = __builtin_bit_cast(half8, ah[j][i]);
          D[i][2 * p2] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
              a_h, b0, (j % SEGJ == 0) ? zero4 : D[i][2 * p2], 0, 0, 0);
          D[i][2 * p2 + 1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
              a_h, b1, (j % SEGJ == 0) ? zero4 : D[i][2 * p2 + 1], 0, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < WM; i++) {
          const half8 a_l = __builtin_bit_cast(half8, al[j][i]);
          D[i][2 * p2] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a_l, b0, D[i][2 * p2], 0, 0, 0);
          D[i][2 * p2 + 1] =
              __builtin_amdgcn_mfma_f32_16x16x32_f16(a_l, b1, D[i][2 * p2 + 1], 0, 0, 0);
        }
      }
      // The next k group's weights, one step's worth per step (VALU work the
      // scheduler interleaves with this step's MFMAs).
      dequant_step(kgn, mnext, buf ^ 1, j);
      if ((j + 1) % SEGJ == 0) {
        const float4 s0 = *reinterpret_cast<const float4 *>(&scl[buf][j / SEGJ][cl][0]);
        const float4 s1 = *reinterpret_cast<const float4 *>(&scl[buf][j / SEGJ][cl][4]);
        const float sc[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
#pragma unroll
        for (int i = 0; i < WM; i++) {
          const float rf[4] = {ldexpf(1.f, -ex[i].x), ldexpf(1.f, -ex[i].y),
                               ldexpf(1.f, -ex[i].z), ldexpf(1.f, -ex[i].w)};
#pragma unroll
          for (int r = 0; r < 4; r++)
#pragma unroll
            for (int n = 0; n < 8; n++) acc[i][n][r] += (sc[n] * rf[r]) * D[i][n][r];
        }
      }
    }
    __syncthreads();
  }

  const bool split = gridDim.y > 1;
#pragma unroll
  for (int i = 0; i < WM; i++) {
    const int rbase = (m16w + i) * 16 + 4 * lg;
#pragma unroll
    for (int n = 0; n < 8; n++) {
      const int col = nt * 128 + n * 16 + cl;
      if (col >= N) continue;
      const float bv = (!split && bias) ? bias[col] : 0.f;
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const int row = rbase + r;
        if (row >= M) continue;
        if (split)
          part[((int64_t)ks * M + row) * N + col] = acc[i][n][r];
        else
          y[(int64_t)row * N + col] = acc[i][n][r] + bv;
      }
    }
  }
}

// y = sum over k splits of part + bias (deterministic split-K reduction).
__global__ __launch_bounds__(256) void k_gemm_reduce(const float *__restrict__ part,
                                                     const float *__restrict__ bias,
                                                     float *__restrict__ y, int64_t MN, int N,
                                                     int ksplit) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= MN) return;
  float s = 0.f;
  for (int k = 0; k < ksplit; k++) s += part[(int64_t)k * MN + i];
  y[i] = s + (bias ? bias[i % N] : 0.f);
}

// ---------------------------------------------------------- generic path

// One thread per output; dequantises exactly as the reference (q - zp in
// double times the f32 scale, one rounding) and accumulates in double.
__global__ __launch_bounds__(256) void k_nbits_generic(
    const float *__restrict__ a, const uint32_t *__restrict__ wq,
    const float *__restrict__ scales, const uint8_t *__restrict__ zp4,
    const float *__restrict__ zpf, int zpk, const float *__restrict__ bias,
    float *__restrict__ y, int M, int N, int K, int c4n, int nb, int nbh,
    int bs) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (int64_t)M * N) return;
  const int row = (int)(idx / N), col = (int)(idx % N);
  const int cgi = col / 64, cg = col % 64;
  double acc = 0.0;
  for (int k = 0; k < K; k++) {
    const int kg = k / KGRP, rem = k % KGRP;
    const int j = rem / 32, g = (rem % 32) / 8, t = k % 8;
    const uint32_t dw = wq[((((int64_t)cgi * c4n + kg) * 4 + g) * 64 + cg) * 4 + j];
    const int q = (dw >> (4 * nib_pos(t))) & 15;
    const int blk = k / bs;
    double z = 8.0;
    if (zpk == 1) {
      const uint8_t zb = zp4[((int64_t)cgi * nbh + blk / 2) * 64 + cg];
      z = (double)((blk & 1) ? (zb >> 4) : (zb & 15));
    } else if (zpk == 2) {
      z = (double)zpf[((int64_t)cgi * nb + blk) * 64 + cg];
    }
    const float w = (float)(((double)q - z) * (double)scales[((int64_t)cgi * nb + blk) * 64 + cg]);
    acc += (double)a[(int64_t)row * K + k] * (double)w;
  }
  y[idx] = (float)(acc + (bias ? (double)bias[col] : 0.0));
}

// ------------------------------------------------------------ host side

struct NbitsPlan {
  int path;  // 0 gemv, 1 mfma, 2 generic
  int64_t M;
  // gemv
  int qpg = 1, qb = 128, nqb = 0, ksplit = 1, kps = 0;
  // mfma
  int wms = 2;
  int64_t mpad = 0;
  size_t off_a = 0, off_b = 0, off_c = 0, off_d = 0, total = 0;
};

NbitsPlan plan_nbits(const mg_weight *w, int64_t M) {
  const mg_nbits_dev &d = w->nbits;
  NbitsPlan p;
  p.M = M;
  if (M <= 4 && d.bs <= 4096) {
    p.path = 0;
    p.qb = (int)std::min<int64_t>(d.bs, KGRP);
    p.qpg = KGRP / p.qb;
    p.nqb = (int)(d.kpad / p.qb);
    const int64_t waves_per_slice = d.ng * 4;
    int64_t ks = (2048 + waves_per_slice - 1) / waves_per_slice;
    ks = std::min<int64_t>(ks, std::max<int64_t>(1, d.c4 / 4));
    ks = std::max<int64_t>(ks, 1);
    p.ksplit = (int)ks;
    p.off_a = 0;  // digits: M * c4 * 64 dwords
    p.off_b = mg_align(p.off_a + (size_t)M * d.c4 * 64 * 4);  // alpha
    p.off_c = mg_align(p.off_b + (size_t)M * p.nqb * 4);      // rsum
    p.off_d = mg_align(p.off_c + (size_t)M * p.nqb * 4);      // partials
    p.total = mg_align(p.off_d + (p.ksplit > 1 ? (size_t)p.ksplit * M * d.ng * 64 * 4 : 0));
  } else if (d.bs >= 32 && d.zp_kind != MG_ZP_FLOAT) {
    p.path = 1;
    p.wms = (M <= 64 || d.bs < KGRP) ? 1 : 2;
    const int64_t rows = 64 * p.wms;
    p.mpad = (M + rows - 1) / rows * rows;
    // Split K until the grid covers the chip (~2 workgroups per CU), keeping
    // at least 2 k groups per split.
    const int64_t tiles = (p.mpad / rows) * (d.ng / 2);
    int64_t ks = 1;
    while (tiles * ks * 2 <= 512 && d.c4 / (ks * 2) >= 2) ks *= 2;
    p.kps = (int)((d.c4 + ks - 1) / ks);
    p.ksplit = (int)((d.c4 + p.kps - 1) / p.kps);
    p.off_a = 0;  // ahl: mpad * kpad * 2 fp16
    p.off_b = mg_align(p.off_a + (size_t)p.mpad * d.kpad * 4);  // texp
    p.off_c = mg_align(p.off_b + (size_t)p.mpad * d.c4 * 4);    // split-K partials
    p.total = mg_align(p.off_c + (p.ksplit > 1 ? (size_t)p.ksplit * M * w->N * 4 : 0));
  } else {
    p.path = 2;
    p.total = 0;
  }
  return p;
}

template <int MR, int QPG>
void launch_gemv_zp(const mg_weight *w, int zpk, dim3 grid, hipStream_t st,
                    const uint32_t *dig, const float *alpha, const int *rsum,
                    float *y, float *part, int nqb) {
  const mg_nbits_dev &d = w->nbits;
  const int ncolp = (int)(d.ng * 64);
#define MG_GEMV_ARGS                                                           \
  reinterpret_cast<const uint4 *>(d.wq), d.scales, d.zp4, d.zpf, dig, alpha,   \
      rsum, d.bias, y, part, (int)w->N, (int)d.c4, (int)d.nb, (int)d.nbh,      \
      (int)d.bs, nqb, ncolp
  if (zpk == 0)
    hipLaunchKernelGGL((k_gemv_dot8<MR, QPG, 0>), grid, dim3(256), 0, st, MG_GEMV_ARGS);
  else if (zpk == 1)
    hipLaunchKernelGGL((k_gemv_dot8<MR, QPG, 1>), grid, dim3(256), 0, st, MG_GEMV_ARGS);
  else
    hipLaunchKernelGGL((k_gemv_dot8<MR, QPG, 2>), grid, dim3(256), 0, st, MG_GEMV_ARGS);
#undef MG_GEMV_ARGS
}

template <int MR>
void launch_gemv_q(const mg_weight *w, int qpg, int zpk, dim3 grid,
                   hipStream_t st, const uint32_t *dig, const float *alpha,
                   const int *rsum, float *y, float *part, int nqb) {
  switch (qpg) {
    case 1: launch_gemv_zp<MR, 1>(w, zpk, grid, st, dig, alpha, rsum, y, part, nqb); break;
    case 2: launch_gemv_zp<MR, 2>(w, zpk, grid, st, dig, alpha, rsum, y, part, nqb); break;
    case 4: launch_gemv_zp<MR, 4>(w, zpk, grid, st, dig, alpha, rsum, y, part, nqb); break;
    default: launch_gemv_zp<MR, 8>(w, zpk, grid, st, dig, alpha, rsum, y, part, nqb); break;
  }
}

}  // namespace

// ------------------------------------------------------------- uploading

mg_status mg_nbits_upload(mg_ctx *ctx, mg_weight *w, const uint8_t *b,
                          const float *scales, int32_t zp_kind, const void *zp,
                          const float *bias) {
  mg_nbits_dev &d = w->nbits;
  const int64_t N = w->N, K = w->K, bs = d.bs;
  d.nb = (K + bs - 1) / bs;
  d.nbh = (d.nb + 1) / 2;
  d.kpad = std::max<int64_t>((d.nb * bs + KGRP - 1) / KGRP * KGRP, KGRP);
  d.c4 = d.kpad / KGRP;
  d.ng = ((N + CGRP - 1) / CGRP + 1) / 2 * 2;  // even: the GEMM pairs groups
  d.zp_kind = zp_kind;
  const int64_t ng = d.ng, nb = d.nb, nbh = d.nbh, c4 = d.c4;
  const int64_t blob = bs / 2, kstored = nb * bs;

  std::vector<uint32_t> wq((size_t)(ng * c4 * 4 * 64 * 4));
  std::vector<float> sp((size_t)(ng * nb * 64), 0.f);
  std::vector<uint8_t> zp4;
  std::vector<float> zpf;
  auto work = [&](int64_t g0, int64_t g1) {
    for (int64_t cg = g0; cg < g1; cg++) {
      for (int64_t kg = 0; kg < c4; kg++)
        for (int g = 0; g < 4; g++)
          for (int col = 0; col < 64; col++) {
            const int64_t n = cg * 64 + col;
            for (int j = 0; j < 4; j++) {
              uint32_t dw = 0;
              for (int t = 0; t < 8; t++) {
                const int64_t k = kg * KGRP + 32 * j + 8 * g + t;
                uint32_t q = 8;
                if (n < N && k < kstored) {
                  const uint8_t by = b[(n * nb + k / bs) * blob + (k % bs) / 2];
                  q = (k & 1) ? (by >> 4) : (by & 15);
                }
                dw |= q << (4 * nib_pos(t));
              }
              wq[(size_t)((((cg * c4 + kg) * 4 + g) * 64 + col) * 4 + j)] = dw;
            }
          }
      for (int64_t blk = 0; blk < nb; blk++)
        for (int col = 0; col < 64; col++) {
          const int64_t n = cg * 64 + col;
          if (n < N) sp[(size_t)((cg * nb + blk) * 64 + col)] = scales[n * nb + blk];
        }
    }
  };
  {
    const int64_t nthreads = std::max<int64_t>(
        1, std::min<int64_t>(ng, std::thread::hardware_concurrency()));
    std::vector<std::thread> th;
    const int64_t per = (ng + nthreads - 1) / nthreads;
    for (int64_t t = 0; t < nthreads; t++) {
      const int64_t g0 = t * per, g1 = std::min(ng, g0 + per);
      if (g0 < g1) th.emplace_back(work, g0, g1);
    }
    for (auto &t : th) t.join();
  }
  if (zp_kind == MG_ZP_UINT4) {
    zp4.assign((size_t)(ng * nbh * 64), 0x88);
    const uint8_t *z = static_cast<const uint8_t *>(zp);
    for (int64_t cg = 0; cg < ng; cg++)
      for (int64_t h = 0; h < nbh; h++)
        for (int col = 0; col < 64; col++) {
          const int64_t n = cg * 64 + col;
          if (n < N) zp4[(size_t)((cg * nbh + h) * 64 + col)] = z[n * nbh + h];
        }
  } else if (zp_kind == MG_ZP_FLOAT) {
    zpf.assign((size_t)(ng * nb * 64), 8.f);
    const float *z = static_cast<const float *>(zp);
    for (int64_t cg = 0; cg < ng; cg++)
      for (int64_t blk = 0; blk < nb; blk++)
        for (int col = 0; col < 64; col++) {
          const int64_t n = cg * 64 + col;
          if (n < N) zpf[(size_t)((cg * nb + blk) * 64 + col)] = z[n * nb + blk];
        }
  }

  auto up = [&](void **dst, const void *src, size_t bytes) -> mg_status {
    if (bytes == 0) return MG_OK;
    MG_HIP(hipMalloc(dst, bytes));
    w->device_bytes += (int64_t)bytes;
    MG_HIP(hipMemcpy(*dst, src, bytes, hipMemcpyHostToDevice));
    return MG_OK;
  };
  MG_TRY(up((void **)&d.wq, wq.data(), wq.size() * 4));
  MG_TRY(up((void **)&d.scales, sp.data(), sp.size() * 4));
  if (!zp4.empty()) MG_TRY(up((void **)&d.zp4, zp4.data(), zp4.size()));
  if (!zpf.empty()) MG_TRY(up((void **)&d.zpf, zpf.data(), zpf.size() * 4));
  if (bias) MG_TRY(up((void **)&d.bias, bias, (size_t)N * 4));
  (void)ctx;
  return MG_OK;
}

void mg_nbits_free(mg_weight *w) {
  mg_nbits_dev &d = w->nbits;
  if (d.wq) (void)hipFree(d.wq);
  if (d.scales) (void)hipFree(d.scales);
  if (d.zp4) (void)hipFree(d.zp4);
  if (d.zpf) (void)hipFree(d.zpf);
  if (d.bias) (void)hipFree(d.bias);
  d = mg_nbits_dev{};
}

size_t mg_nbits_ws_bytes(const mg_weight *w, int64_t M) {
  return plan_nbits(w, M).total;
}

mg_status mg_nbits_run(mg_ctx *ctx, const mg_weight *w, const float *a_dev,
                       int64_t M, float *y_dev, void *ws) {
  const mg_nbits_dev &d = w->nbits;
  if (M == 0) return MG_OK;
  const NbitsPlan p = plan_nbits(w, M);
  hipStream_t st = ctx->stream;
  char *base = static_cast<char *>(ws);
  const int zpk = d.zp_kind;
  if (p.path == 0) {
    uint32_t *dig = reinterpret_cast<uint32_t *>(base + p.off_a);
    float *alpha = reinterpret_cast<float *>(base + p.off_b);
    int *rsum = reinterpret_cast<int *>(base + p.off_c);
    float *part = p.ksplit > 1 ? reinterpret_cast<float *>(base + p.off_d) : nullptr;
    const int64_t pairs = M * p.nqb;
    hipLaunchKernelGGL(k_adigits, dim3((unsigned)((pairs + 3) / 4)), dim3(256), 0, st,
                       a_dev, M, w->K, p.qb, p.nqb, (int)d.c4, dig, alpha, rsum);
    MG_TRY(mg_launch_check("k_adigits"));
    const dim3 grid((unsigned)d.ng, (unsigned)p.ksplit);
    switch (M) {
      case 1: launch_gemv_q<1>(w, p.qpg, zpk, grid, st, dig, alpha, rsum, y_dev, part, p.nqb); break;
      case 2: launch_gemv_q<2>(w, p.qpg, zpk, grid, st, dig, alpha, rsum, y_dev, part, p.nqb); break;
      case 3: launch_gemv_q<3>(w, p.qpg, zpk, grid, st, dig, alpha, rsum, y_dev, part, p.nqb); break;
      default: launch_gemv_q<4>(w, p.qpg, zpk, grid, st, dig, alpha, rsum, y_dev, part, p.nqb); break;
    }
    MG_TRY(mg_launch_check("k_gemv_dot8"));
    if (p.ksplit > 1) {
      const int64_t tot = M * w->N;
      hipLaunchKernelGGL(k_gemv_reduce, dim3((unsigned)((tot + 255) / 256)), dim3(256), 0, st,
                         part, d.bias, y_dev, (int)M, (int)w->N, (int)(d.ng * 64), p.ksplit);
      MG_TRY(mg_launch_check("k_gemv_reduce"));
    }
    return MG_OK;
  }
  if (p.path == 1) {
    uint4 *ahl = reinterpret_cast<uint4 *>(base + p.off_a);
    int *texp = reinterpret_cast<int *>(base + p.off_b);
    float *part = p.ksplit > 1 ? reinterpret_cast<float *>(base + p.off_c) : nullptr;
    const int vec = (w->K % 4 == 0) && (reinterpret_cast<uintptr_t>(a_dev) % 16 == 0);
    hipLaunchKernelGGL(k_af16split, dim3((unsigned)d.c4, (unsigned)(p.mpad / 16)), dim3(256), 0,
                       st, a_dev, M, w->K, (int)d.c4, vec, ahl, texp);
    MG_TRY(mg_launch_check("k_af16split"));
    const int rows = 64 * p.wms;
    const int mtiles = (int)(p.mpad / rows), ntiles = (int)(d.ng / 2);
    const dim3 grid((unsigned)(8 * mtiles * ((ntiles + 7) / 8)), (unsigned)p.ksplit);
    const int has_zp = zpk == MG_ZP_UINT4;
    // The kernel reads zero-point bytes unconditionally (branch-free); without
    // zero points it is pointed at the scales, which are at least as large.
    const uint8_t *zp_arg = has_zp ? d.zp4 : reinterpret_cast<const uint8_t *>(d.scales);
    const int segj = (int)(std::min<int64_t>(d.bs, KGRP) / 32);
#define MG_GEMM_ARGS                                                                   \
  ahl, texp, reinterpret_cast<const uint4 *>(d.wq), d.scales, zp_arg, d.bias, y_dev, part,   \
      (int)M, (int)w->N, (int)d.c4, (int)d.nb, (int)d.nbh, (int)d.bs, has_zp, mtiles, ntiles, \
      p.kps
#define MG_GEMM_LAUNCH(WM_, SJ_) \
  hipLaunchKernelGGL((k_gemm_f16split<WM_, SJ_>), grid, dim3(256), 0, st, MG_GEMM_ARGS)
    if (p.wms == 1) {
      if (segj == 1) MG_GEMM_LAUNCH(1, 1);
      else if (segj == 2) MG_GEMM_LAUNCH(1, 2);
      else MG_GEMM_LAUNCH(1, 4);
    } else {
      MG_GEMM_LAUNCH(2, 4);
    }
#undef MG_GEMM_LAUNCH
#undef MG_GEMM_ARGS
    MG_TRY(mg_launch_check("k_gemm_f16split"));
    if (p.ksplit > 1) {
      const int64_t mn = M * w->N;
      hipLaunchKernelGGL(k_gemm_reduce, dim3((unsigned)((mn + 255) / 256)), dim3(256), 0, st,
                         part, d.bias, y_dev, mn, (int)w->N, p.ksplit);
      MG_TRY(mg_launch_check("k_gemm_reduce"));
    }
    return MG_OK;
  }
  const int64_t tot = M * w->N;
  hipLaunchKernelGGL(k_nbits_generic, dim3((unsigned)((tot + 255) / 256)), dim3(256), 0, st,
                     a_dev, d.wq, d.scales, d.zp4, d.zpf, zpk, d.bias, y_dev, (int)M,
                     (int)w->N, (int)w->K, (int)d.c4, (int)d.nb, (int)d.nbh, (int)d.bs);
  return mg_launch_check("k_nbits_generic");
}
