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
//   * M > 4 ("prefill"): activations become an fp16 pair hi + lo (per-row
//     power-of-two scaled, so hi + lo carries ~22 bits); weights are unpacked
//     in registers to exact fp16 (q - zp); v_mfma_f32_16x16x32_f16 accumulates
//     hi*W and lo*W per block in fp32, then the block scale is applied on the
//     fp32 accumulator.
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
// 16-row subtile.  ahl[m16][kg][j][hl][lane] (uint4 = 8 fp16): lane
// (r = lane%16, g = lane/16) holds rows r, k = kg*128 + 32*j + 8*g + 0..7.
// Each row is scaled by 2^e so that its max magnitude lies in [2^13, 2^14);
// rowexp[row] = e is undone on the fp32 result.
__global__ __launch_bounds__(256) void k_af16split(
    const float *__restrict__ a, int64_t M, int64_t K, int c4n,
    uint4 *__restrict__ ahl, int *__restrict__ rowexp) {
  __shared__ int sexp[16];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t row0 = (int64_t)blockIdx.x * 16;
  for (int rr = 0; rr < 4; rr++) {
    const int r = wave * 4 + rr;
    const int64_t row = row0 + r;
    float mx = 0.f;
    if (row < M)
      for (int64_t k = lane; k < K; k += 64) mx = fmaxf(mx, fabsf(a[row * K + k]));
    for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
    if (lane == 0) {
      int e = 0;
      if (mx > 0.f && isfinite(mx)) {
        int ex;
        frexpf(mx, &ex);
        e = 14 - ex;
      }
      sexp[r] = e;
      if (row < M) rowexp[row] = e;
    }
  }
  __syncthreads();
  const int total = c4n * 4 * 64;
  for (int idx = threadIdx.x; idx < total; idx += 256) {
    const int ln = idx & 63, j = (idx >> 6) & 3, kg = idx >> 8;
    const int r = ln & 15, g = ln >> 4;
    const int64_t row = row0 + r;
    const int64_t kb = (int64_t)kg * KGRP + 32 * j + 8 * g;
    const int e = sexp[r];
    half8 hi, lo;
    for (int t = 0; t < 8; t++) {
      const int64_t k = kb + t;
      const float v = (row < M && k < K) ? ldexpf(a[row * K + k], e) : 0.f;
      const _Float16 h = (_Float16)v;
      float res = v - (float)h;
      if (!isfinite(res)) res = 0.f;
      hi[t] = h;
      lo[t] = (_Float16)res;
    }
    uint4 *o = ahl + ((((int64_t)blockIdx.x * c4n + kg) * 4 + j) * 2) * 64 + ln;
    o[0] = *reinterpret_cast<uint4 *>(&hi);
    o[64] = *reinterpret_cast<uint4 *>(&lo);
  }
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

// Workgroup tile: (32*WMS) rows x 128 columns; 4 waves as 2 (rows) x 2
// (column groups); each wave WMS x 4 subtiles of 16x16.  The activation
// fragments of one k group are staged in LDS; weights go global -> VGPR and
// are unpacked there.
template <int WMS>
__global__ __launch_bounds__(256, 2) void k_gemm_f16split(
    const uint4 *__restrict__ ahl, const int *__restrict__ rowexp,
    const uint4 *__restrict__ wq, const float *__restrict__ scales,
    const uint8_t *__restrict__ zp4, const float *__restrict__ bias,
    float *__restrict__ y, int M, int N, int c4n, int nb, int nbh, int bs,
    int has_zp) {
  constexpr int SUB = 2 * WMS;
  __shared__ uint4 lds[SUB * 512];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int wm = wave & 1, wn = wave >> 1;
  const int cgi = blockIdx.x * 2 + wn;
  const int m16_0 = blockIdx.y * SUB;
  const int cl = lane & 15, lg = lane >> 4;

  float4v acc[WMS][4], D[WMS][4];
#pragma unroll
  for (int i = 0; i < WMS; i++)
#pragma unroll
    for (int n = 0; n < 4; n++) {
      acc[i][n] = (float4v){0.f, 0.f, 0.f, 0.f};
      D[i][n] = (float4v){0.f, 0.f, 0.f, 0.f};
    }
  float sc[4] = {0.f, 0.f, 0.f, 0.f};
  half2v zz[4];
#pragma unroll
  for (int n = 0; n < 4; n++) zz[n] = (half2v){(_Float16)-1032.f, (_Float16)-1032.f};

  for (int kg = 0; kg < c4n; kg++) {
    __syncthreads();
    for (int i = threadIdx.x; i < SUB * 512; i += 256) {
      const int s = i >> 9, off = i & 511;
      lds[i] = ahl[((int64_t)(m16_0 + s) * c4n + kg) * 512 + off];
    }
    uint4 braw[4];
    const uint4 *wp = wq + (((int64_t)cgi * c4n + kg) * 4 + lg) * 64 + cl;
#pragma unroll
    for (int n = 0; n < 4; n++) braw[n] = wp[n * 16];
    __syncthreads();
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int kk = kg * KGRP + 32 * j;
      if (kk % bs == 0) {
        const int blk = kk / bs;
#pragma unroll
        for (int n = 0; n < 4; n++) {
          const int cg = n * 16 + cl;
          if (blk < nb) {
            sc[n] = scales[((int64_t)cgi * nb + blk) * 64 + cg];
            int z = 8;
            if (has_zp) {
              const uint8_t zb = zp4[((int64_t)cgi * nbh + blk / 2) * 64 + cg];
              z = (blk & 1) ? (zb >> 4) : (zb & 15);
            }
            const _Float16 zh = (_Float16)(-(1024.f + (float)z));
            zz[n] = (half2v){zh, zh};
          } else {
            sc[n] = 0.f;
          }
        }
      }
      half8 bf[4];
#pragma unroll
      for (int n = 0; n < 4; n++) {
        const uint32_t x = j == 0 ? braw[n].x : j == 1 ? braw[n].y : j == 2 ? braw[n].z : braw[n].w;
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const uint32_t h = ((x >> (4 * i)) & 0x000F000Fu) | 0x64006400u;
          half2v hv = __builtin_bit_cast(half2v, h) + zz[n];
          bf[n][2 * i] = hv[0];
          bf[n][2 * i + 1] = hv[1];
        }
      }
#pragma unroll
      for (int i = 0; i < WMS; i++) {
        const int s = wm * WMS + i;
        const uint4 hu = lds[((s * 4 + j) * 2 + 0) * 64 + lane];
        const uint4 lu = lds[((s * 4 + j) * 2 + 1) * 64 + lane];
        const half8 ah = __builtin_bit_cast(half8, hu);
        const half8 al = __builtin_bit_cast(half8, lu);
#pragma unroll
        for (int n = 0; n < 4; n++) {
          D[i][n] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ah, bf[n], D[i][n], 0, 0, 0);
          D[i][n] = __builtin_amdgcn_mfma_f32_16x16x32_f16(al, bf[n], D[i][n], 0, 0, 0);
        }
      }
      if ((kk + 32) % bs == 0) {
#pragma unroll
        for (int i = 0; i < WMS; i++)
#pragma unroll
          for (int n = 0; n < 4; n++) {
            acc[i][n] += sc[n] * D[i][n];
            D[i][n] = (float4v){0.f, 0.f, 0.f, 0.f};
          }
      }
    }
  }
#pragma unroll
  for (int i = 0; i < WMS; i++) {
    const int rbase = (m16_0 + wm * WMS + i) * 16 + 4 * lg;
#pragma unroll
    for (int n = 0; n < 4; n++) {
      const int col = cgi * 64 + n * 16 + cl;
      if (col >= N) continue;
      const float bv = bias ? bias[col] : 0.f;
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const int row = rbase + r;
        if (row < M) y[(int64_t)row * N + col] = ldexpf(acc[i][n][r], -rowexp[row]) + bv;
      }
    }
  }
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
  int qpg = 1, qb = 128, nqb = 0, ksplit = 1;
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
    p.wms = M <= 64 ? 1 : 2;
    const int64_t rows = 32 * p.wms;
    p.mpad = (M + rows - 1) / rows * rows;
    p.off_a = 0;  // ahl: mpad * kpad * 2 fp16
    p.off_b = mg_align(p.off_a + (size_t)p.mpad * d.kpad * 4);  // rowexp
    p.total = mg_align(p.off_b + (size_t)p.mpad * 4);
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
    int *rowexp = reinterpret_cast<int *>(base + p.off_b);
    hipLaunchKernelGGL(k_af16split, dim3((unsigned)(p.mpad / 16)), dim3(256), 0, st,
                       a_dev, M, w->K, (int)d.c4, ahl, rowexp);
    MG_TRY(mg_launch_check("k_af16split"));
    const int rows = 32 * p.wms;
    const dim3 grid((unsigned)(d.ng / 2), (unsigned)(p.mpad / rows));
    const int has_zp = zpk == MG_ZP_UINT4;
    if (p.wms == 1)
      hipLaunchKernelGGL((k_gemm_f16split<1>), grid, dim3(256), 0, st, ahl, rowexp,
                         reinterpret_cast<const uint4 *>(d.wq), d.scales, d.zp4, d.bias,
                         y_dev, (int)M, (int)w->N, (int)d.c4, (int)d.nb, (int)d.nbh,
                         (int)d.bs, has_zp);
    else
      hipLaunchKernelGGL((k_gemm_f16split<2>), grid, dim3(256), 0, st, ahl, rowexp,
                         reinterpret_cast<const uint4 *>(d.wq), d.scales, d.zp4, d.bias,
                         y_dev, (int)M, (int)w->N, (int)d.c4, (int)d.nb, (int)d.nbh,
                         (int)d.bs, has_zp);
    return mg_launch_check("k_gemm_f16split");
  }
  const int64_t tot = M * w->N;
  hipLaunchKernelGGL(k_nbits_generic, dim3((unsigned)((tot + 255) / 256)), dim3(256), 0, st,
                     a_dev, d.wq, d.scales, d.zp4, d.zpf, zpk, d.bias, y_dev, (int)M,
                     (int)w->N, (int)w->K, (int)d.c4, (int)d.nb, (int)d.nbh, (int)d.bs);
  return mg_launch_check("k_nbits_generic");
}
