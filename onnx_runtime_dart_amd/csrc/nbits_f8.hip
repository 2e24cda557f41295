// MatMulNBits prefill GEMM on gfx950 block-scaled fp8 MFMA
// (v_mfma_scale_f32_32x32x64_f8f6f4), for block_size >= 128 with integer
// zero points.
//
// Reference semantics: opMatMulNBits, lib/src/onnx_qlinear_ops.dart:115-228
// (M > 1: dequantised fp32 weights times fp32 activations, :208-226).
//
// Numbers.  Each weight (q - zp) is an integer in [-15, 15] and each
// 16 (q - zp) one in [-240, 240]: both are exact in fp8 e4m3.  Each fp32
// activation is carried as the sum of three e4m3 digits, each digit of a
// 32-element block with its own power-of-two (E8M0) scale that the MFMA
// applies in hardware: r0 = a, d_i = e4m3(r_i / 2^E_i) rounded to nearest
// even, r_{i+1} = r_i - d_i 2^E_i, with 2^E_i putting the block's largest
// |r_i| in [128, 256).  Every digit keeps 4 significant bits of what is left,
// so the residual after three digits is below 2^-12 of each element; products
// and sums are fp32 in the MFMA.  Measured against fp64 on 512 x 1024 x 8192
// Gaussian activations this is ~1e-4 of the output rms at the largest
// element, against ~1.3e-3 for fp16 activations.  Three fp8 MFMAs cost 1.5
// fp16 ones (the fp16 hi/lo split of the other prefill path costs 2), and the
// weight tile in LDS is 1 byte per weight instead of 2.
//
// Non-finite activations: the digits carry the finite values only and the
// prepass flags the 32-element blocks that held Inf or NaN; for a flagged row
// the epilogue rebuilds the reference's Inf / NaN pattern of each output
// column from the non-finite activations of the launch's k range and the
// dequantised weights there (inf * w = +-inf by sign, inf * 0 and NaN give
// NaN, opposite infinities give NaN).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <type_traits>

#include "mg_internal.h"
#include "nbits_common.h"

namespace {

typedef int int8v __attribute__((ext_vector_type(8)));
typedef short short2v __attribute__((ext_vector_type(2)));
typedef unsigned uint6v __attribute__((ext_vector_type(6)));
typedef float float32v __attribute__((ext_vector_type(32)));

// --------------------------------------------------------------- prepass

// Activations -> three e4m3 digits per element in the A-operand order of
// v_mfma_scale_f32_32x32x64_f8f6f4.  Lane l of the operand holds row l % 32
// of 32-row tile m32; in 64-k step st of k group kg, byte i of lane half
// h = l / 32 holds k = 128 kg + 32 j + 8 g + t with g = 2 h + i / 16,
// j = 2 st + (i / 8) % 2, t = i % 8 (the weight fragments in LDS use the
// same order).  The MFMA's scale blocks are bytes 0-15 of both lane halves
// (block 0, scale from lane r) and bytes 16-31 of both (block 1, scale from
// lane r + 32): block b holds the octets g = b and g = b + 2.  Bytes at t in
// {2, 3, 6, 7} carry a * 2^-4: the weights there are 16 (q - zp), as deq8
// makes them.
// Output per (m32, kg): aq[((m32 * c4n + kg) * 2 + st) * 3 + d][lane][2]
// (uint4: bytes 0-15, 16-31), asc[(m32 * c4n + kg) * 2 + st][r + 32 b] = the
// three E8M0 scale bytes of block b (digit d in byte d), nf[(row * c4n + kg)
// * 4 + 2 st + b] = 1 when the block held a non-finite value.  Rows >= M and
// k >= K are zeros.  Four threads per scale block (r, b), eight elements each
// (octet o of the block's four); the block maxima meet by shuffles over the
// four lanes.  Workgroup = one (m32, kg, st): its 64 blocks are blk = t / 4,
// r = blk % 32, b = blk / 32.
__global__ __launch_bounds__(256) void k_af8x3(const float *__restrict__ a, int64_t M,
                                               int64_t K, int c4n, int vec,
                                               uint4 *__restrict__ aq,
                                               uint32_t *__restrict__ asc,
                                               uint8_t *__restrict__ nf) {
  const int t = threadIdx.x;
  const int64_t wv = blockIdx.x;  // (m32 * c4n + kg) * 2 + st
  const int st = (int)(wv & 1);
  const int64_t mk = wv >> 1;  // m32 * c4n + kg
  const int kg = (int)(mk % c4n);
  const int64_t m32 = mk / c4n;
  const int o = t & 3, blk = t >> 2;
  const int r = blk & 31, b = blk >> 5;
  const int64_t row = m32 * 32 + r;
  const bool live = row < M;
  const float *arow = a + (live ? row : 0) * K;
  // Octet o = 2 hh + jj of the block: lane half hh, g = 2 hh + b, j = 2 st + jj.
  const int hh = o >> 1, jj = o & 1;
  const int g = 2 * hh + b, j = 2 * st + jj;
  const int64_t k0 = (int64_t)kg * KGRP + 32 * j + 8 * g;
  float v[8];
  if (live && vec && k0 + 8 <= K) {
    const float4 x0 = *reinterpret_cast<const float4 *>(arow + k0);
    const float4 x1 = *reinterpret_cast<const float4 *>(arow + k0 + 4);
    v[0] = x0.x; v[1] = x0.y; v[2] = x0.z; v[3] = x0.w;
    v[4] = x1.x; v[5] = x1.y; v[6] = x1.z; v[7] = x1.w;
  } else {
#pragma unroll
    for (int i = 0; i < 8; i++) v[i] = (live && k0 + i < K) ? arow[k0 + i] : 0.f;
  }
  int bad = 0;
#pragma unroll
  for (int i = 0; i < 8; i++) {
    float x = v[i];
    if (!isfinite(x)) {
      bad = 1;
      x = 0.f;
    }
    v[i] = (i & 2) ? x * 0.0625f : x;  // exact
  }
  bad |= __shfl_xor(bad, 1);
  bad |= __shfl_xor(bad, 2);
  uint32_t scales = 0;
  uint2 *out = reinterpret_cast<uint2 *>(aq + (wv * 3) * 128 + hh * 64 + 2 * r + b) + jj;
#pragma unroll
  for (int d = 0; d < 3; d++) {
    float mx = 0.f;
#pragma unroll
    for (int i = 0; i < 8; i++) mx = fmaxf(mx, fabsf(v[i]));
    mx = fmaxf(mx, __shfl_xor(mx, 1));
    mx = fmaxf(mx, __shfl_xor(mx, 2));
    int E = 0;
    if (mx > 0.f) {
      int ex;
      frexpf(mx, &ex);  // mx in [2^(ex-1), 2^ex)
      E = min(max(ex - 8, -127), 127);
    }
    uint32_t wd[2];
#pragma unroll
    for (int q = 0; q < 2; q++) {
      int w = 0;
      w = __builtin_amdgcn_cvt_pk_fp8_f32(ldexpf(v[4 * q], -E), ldexpf(v[4 * q + 1], -E), w,
                                          false);
      w = __builtin_amdgcn_cvt_pk_fp8_f32(ldexpf(v[4 * q + 2], -E), ldexpf(v[4 * q + 3], -E),
                                          w, true);
      wd[q] = (uint32_t)w;
      v[4 * q] -= ldexpf(__builtin_amdgcn_cvt_f32_fp8(w, 0), E);
      v[4 * q + 1] -= ldexpf(__builtin_amdgcn_cvt_f32_fp8(w, 1), E);
      v[4 * q + 2] -= ldexpf(__builtin_amdgcn_cvt_f32_fp8(w, 2), E);
      v[4 * q + 3] -= ldexpf(__builtin_amdgcn_cvt_f32_fp8(w, 3), E);
    }
    // Octet o's 8 bytes of plane b: lane r (half 0, o < 2) or lane r + 32.
    out[d * 256] = make_uint2(wd[0], wd[1]);
    scales |= (uint32_t)(E + 127) << (8 * d);
  }
  if (o == 0) {
    asc[wv * 64 + r + 32 * b] = scales;
    nf[(row * c4n + kg) * 4 + 2 * st + b] = (uint8_t)bad;
  }
}

// ------------------------------------------------- fp6 prefill (images)

// Sixteen 6-bit fields, field i at bits 6 i of three dwords.
__device__ inline void pack6x16(const uint32_t (&c)[16], uint32_t (&w)[3]) {
  w[0] = w[1] = w[2] = 0u;
#pragma unroll
  for (int i = 0; i < 16; i++) {
    const int bit = 6 * i, wd = bit >> 5, sh = bit & 31;
    w[wd] |= c[i] << sh;
    if (sh > 26) w[wd + 1] |= c[i] >> (32 - sh);
  }
}

// Activations -> three e2m3 digits per element in the A-operand order of the
// fp6 MFMA (v_mfma_scale_f32_32x32x64_f8f6f4, both operands e2m3): lane l
// holds row l % 32 of 32-row tile m32; in 64-k step st of k group kg, field i
// (bits 6 i of the lane's six dwords) holds k = 128 kg + 64 st + 32 (l / 32)
// + i.  With fp6 operands the MFMA's scale block h is the 32 fields of lane
// half h (unlike fp8, whose blocks take 16 bytes from each half), its scale
// from the lane itself.
// Digit d of a block: e_d = e2m3(r_d / 2^E_d) rounded to nearest even,
// r_{d+1} = r_d - e_d 2^E_d (exact: Sterbenz), where 2^E_d puts the block's
// largest |r_d| in [2, 4) (E_d >= -126, so 2^E_d is a normal float and the
// block still fits below 4), so every digit leaves at most 2^-4 of the
// block's largest residual.
// One thread per 32-k scale block, i.e. per (row, lane half): it converts
// its 32 values with gfx950's fp6 conversions.  v_cvt_scalef32_2xpk16_fp6_f32
// (x, y, s) writes field 2 j = e2m3(x_j / s) and field 2 j + 1 = e2m3(y_j /
// s), rounded to nearest even, and v_cvt_scalef32_pk32_f32_fp6 (w, s) gives
// field j's value times s (a probe on the GPU matched these to a software
// rounding bit for bit, ties and the subnormal e2m3 values included); so the
// even k go to x, the odd k to y, and the decoded digit is subtracted
// exactly.
// Output per (m32, kg, st, d), at aq + (((m32 * c4n + kg) * 2 + st) * 3 + d)
// * 1536: dwords 0-3 of lane l at byte 16 l, dwords 4-5 at 1024 + 8 l;
// asc[(m32 * c4n + kg) * 2 + st][l] = the three E8M0 scale bytes of lane l's
// block (digit d in byte d), nf[(row * c4n + kg) * 4 + 2 st + h] = 1 when
// the block held a non-finite value.  Rows >= M and k >= K are zeros.
// Workgroup = one wave for one (m32, kg, st); lane = the MFMA lane.
// With rsum (float zero points), also the sum over the step's 64 k of the
// values the three digits represent (input minus final residual), added in a
// fixed order, rsum[(row * c4n + kg) * 2 + st]: the GEMM subtracts z times
// it, so the zero point meets the same activations as the weights do.
__global__ __launch_bounds__(64) void k_af6x3(const float *__restrict__ a, int64_t M, int64_t K,
                                              int c4n, int vec, uint8_t *__restrict__ aq,
                                              uint32_t *__restrict__ asc,
                                              uint8_t *__restrict__ nf,
                                              float *__restrict__ rsum) {
  const int lane = threadIdx.x;
  const int r = lane & 31, h = lane >> 5;
  const int64_t bid = blockIdx.x;  // (m32 * c4n + kg) * 2 + st
  const int st = (int)(bid & 1);
  const int64_t mk = bid >> 1;     // m32 * c4n + kg
  const int kg = (int)(mk % c4n);
  const int64_t m32 = mk / c4n;
  const int64_t row = m32 * 32 + r;
  const bool live = row < M;
  const float *arow = a + (live ? row : 0) * K;
  const int64_t k0 = (int64_t)kg * KGRP + 64 * st + 32 * h;
  float v[32];
  if (live && vec && k0 + 32 <= K) {
#pragma unroll
    for (int q = 0; q < 8; q++) {
      const float4 x = *reinterpret_cast<const float4 *>(arow + k0 + 4 * q);
      v[4 * q] = x.x, v[4 * q + 1] = x.y, v[4 * q + 2] = x.z, v[4 * q + 3] = x.w;
    }
  } else {
#pragma unroll
    for (int i = 0; i < 32; i++) v[i] = (live && k0 + i < K) ? arow[k0 + i] : 0.f;
  }
  int bad = 0;
#pragma unroll
  for (int i = 0; i < 32; i++) {
    if (!isfinite(v[i])) {
      bad = 1;
      v[i] = 0.f;
    }
  }
  float v0[32];
  if (rsum) {
#pragma unroll
    for (int i = 0; i < 32; i++) v0[i] = v[i];
  }
  uint8_t *base = aq + bid * 3 * 1536;
  uint32_t scales = 0;
#pragma unroll
  for (int d = 0; d < 3; d++) {
    float mx = 0.f;
#pragma unroll
    for (int i = 0; i < 32; i++) mx = fmaxf(mx, fabsf(v[i]));
    int E = 0;
    if (mx > 0.f) {
      int ex;
      frexpf(mx, &ex);  // mx in [2^(ex-1), 2^ex)
      E = max(ex - 2, -126);
    }
    const float sc = __uint_as_float((uint32_t)(E + 127) << 23);  // 2^E
    float16v xe, xo;
#pragma unroll
    for (int j = 0; j < 16; j++) xe[j] = v[2 * j], xo[j] = v[2 * j + 1];
    const uint6v w = __builtin_amdgcn_cvt_scalef32_2xpk16_fp6_f32(xe, xo, sc);
    const float32v dv = __builtin_amdgcn_cvt_scalef32_pk32_f32_fp6(w, sc);
#pragma unroll
    for (int i = 0; i < 32; i++) v[i] -= dv[i];  // exact
    *reinterpret_cast<uint4 *>(base + d * 1536 + 16 * lane) = make_uint4(w[0], w[1], w[2], w[3]);
    *reinterpret_cast<uint2 *>(base + d * 1536 + 1024 + 8 * lane) = make_uint2(w[4], w[5]);
    scales |= (uint32_t)(E + 127) << (8 * d);
  }
  asc[bid * 64 + lane] = scales;
  nf[(row * c4n + kg) * 4 + 2 * st + h] = (uint8_t)bad;
  if (rsum) {
    float p[8];
#pragma unroll
    for (int q = 0; q < 8; q++)
      p[q] = ((v0[4 * q] - v[4 * q]) + (v0[4 * q + 1] - v[4 * q + 1])) +
             ((v0[4 * q + 2] - v[4 * q + 2]) + (v0[4 * q + 3] - v[4 * q + 3]));
    float sum = ((p[0] + p[1]) + (p[2] + p[3])) + ((p[4] + p[5]) + (p[6] + p[7]));
    sum += __shfl_xor(sum, 32);
    if (h == 0) rsum[(row * c4n + kg) * 2 + st] = sum;
  }
}

// e2m3 code of the weight integer v / 2, v = q - zp in [-15, 15] (all exact:
// magnitudes m / 2 below 2 are codes 4 m, in [2, 4) codes 8 + 2 m, in [4, 7.5]
// codes 16 + m); the GEMM scales the weight operand by 2.
__device__ inline uint32_t e2m3_half_int(int v) {
  const int m = v < 0 ? -v : v;
  const uint32_t c = (uint32_t)(m < 4 ? 4 * m : m < 8 ? 8 + 2 * m : 16 + m);
  return v < 0 ? (c | 32u) : c;
}

// Prefill images, built once per weight at upload: for 32-column slab u
// (columns 32 u .. + 31) and k group kg, the 3072 bytes of B operands of the
// fp6 GEMM: per step st, lane l = column (l % 32) and fields as the A operand
// (k = 64 st + 32 (l / 32) + i), dwords 0-3 of lane l at st * 1536 + 16 l
// and dwords 4-5 at st * 1536 + 1024 + 8 l.  Thread = the four packed uint4
// of wq (g = 0..3) of column group cg, k group kg, column col, i = (cg * c4n
// + kg) * 64 + col: dword j of octet row g holds k = 32 j + 8 g + t, so dword
// j of all four gives the 32 fields (i = 8 g + t) of step j / 2, lane half
// j % 2.
// Without packed zero points the codes are of (q - zdef) / 2: zdef = 8 (the
// default zero point), or 0 for float zero points, which the GEMM then takes
// out as z * (sum of the activations).
__global__ __launch_bounds__(256) void k_f6_images(const uint4 *__restrict__ wq,
                                                   const uint8_t *__restrict__ zp4, int has_zp,
                                                   int zdef, int64_t n, int c4n, int nbh,
                                                   int lbs, uint8_t *__restrict__ img) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const int col = (int)(i & 63);
  const int64_t cgk = i >> 6;  // cg * c4n + kg
  const int kg = (int)(cgk % c4n);
  const int64_t cg = cgk / c4n;
  uint4 p[4];
#pragma unroll
  for (int g = 0; g < 4; g++) p[g] = wq[(cgk * 4 + g) * 64 + col];
  const int blk = (kg * KGRP) >> lbs;
  int z = zdef;
  if (has_zp)
    z = (int)((zp4[(cg * nbh + min(blk / 2, nbh - 1)) * 64 + sz_pos(col)] >> ((blk & 1) * 4)) &
              15u);
  uint8_t *dst = img + ((2 * cg + (col >> 5)) * c4n + kg) * 3072;
#pragma unroll
  for (int j = 0; j < 4; j++) {
    uint32_t c[2][16];
#pragma unroll
    for (int g = 0; g < 4; g++) {
      const uint32_t dw = j == 0 ? p[g].x : j == 1 ? p[g].y : j == 2 ? p[g].z : p[g].w;
#pragma unroll
      for (int tt = 0; tt < 8; tt++)
        c[g >> 1][8 * (g & 1) + tt] = e2m3_half_int((int)((dw >> (4 * nib_pos(tt))) & 15u) - z);
    }
    uint32_t w0[3], w1[3];
    pack6x16(c[0], w0);
    pack6x16(c[1], w1);
    const int lane = (col & 31) + 32 * (j & 1), st = j >> 1;
    *reinterpret_cast<uint4 *>(dst + st * 1536 + 16 * lane) = make_uint4(w0[0], w0[1], w0[2], w1[0]);
    *reinterpret_cast<uint2 *>(dst + st * 1536 + 1024 + 8 * lane) = make_uint2(w1[1], w1[2]);
  }
}

// ------------------------------------------------------------------ GEMM

// One digit's MFMA: the op_sel byte of the A scale word is the digit.
template <int DG>
__device__ inline float16v mfma_digit(const int8v &a, const int8v &b, const float16v &c, int sa,
                                      int sb) {
  return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, DG, sa, 0, sb);
}

// Dequantised weight (q - zp) * s of column col at k, in fp32 (the
// non-finite pattern only needs its sign and whether it is zero); zpk is the
// zero-point kind (MG_ZP_NONE: 8, MG_ZP_UINT4: packed zp4, MG_ZP_FLOAT: zpf).
__device__ inline float nbits_weight(const uint4 *__restrict__ wq, const float *__restrict__ sc,
                                     const uint8_t *__restrict__ zp4,
                                     const float *__restrict__ zpf, int c4n, int nb, int nbh,
                                     int lbs, int zpk, int col, int k) {
  const int cg = col >> 6, cl = col & 63;
  const int kg = k >> 7, kk = k & 127;
  const int j = kk >> 5, g = (kk >> 3) & 3, tt = kk & 7;
  const uint32_t *wd = reinterpret_cast<const uint32_t *>(wq) +
                       (((int64_t)cg * c4n + kg) * 256 + g * 64 + cl) * 4 + j;
  const int q = (int)((*wd >> (4 * nib_pos(tt))) & 15u);
  const int blk = min(k >> lbs, nb - 1);
  const float s = sc[((int64_t)cg * nb + blk) * 64 + sz_pos(cl)];
  if (zpk == MG_ZP_FLOAT) return ((float)q - zpf[((int64_t)cg * nb + blk) * 64 + sz_pos(cl)]) * s;
  const int z = zpk == MG_ZP_UINT4 ? (int)((zp4[((int64_t)cg * nbh + blk / 2) * 64 + sz_pos(cl)] >>
                                            (4 * (blk & 1))) & 15u)
                                   : 8;
  return (float)(q - z) * s;
}

// What the epilogue reads that nothing in the k loop produces, loaded when
// the workgroup starts so that the latency hides under the loop (read at the
// end, the bias and the flags were two dependent round trips after the last
// k group): the bias quad of this lane's output columns (zeros past N,
// without a bias and for k-split partials) and, for lanes < 32, the
// non-finite flag words of the wave's row lane for the first 8 k groups of
// the launch's range (clamped to the last; rows past M read zeros).
// Buffer loads with out-of-range offsets read zeros and touch no memory,
// so no load sits under a branch.
struct EpiPre {
  float4 bv;
  uint32_t w[8];
  int flag;
};
template <int NT>
__device__ inline void epi_prefetch(EpiPre &e, int nt, int m32, int M, int c4n, int kg0,
                                    int kg1, const uint8_t *__restrict__ nf,
                                    const float *__restrict__ bias, int N) {
  constexpr int TC = 32 * NT, PPR = 8 * NT;
  const int lane = threadIdx.x & 63;
  const unsigned col = (unsigned)(nt * TC + 4 * (lane % PPR));
  const bool use_bias = gridDim.y == 1 && bias != nullptr;
  const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<float *>(bias), (short)0, use_bias ? N * 4 : 0, 0x00020000);
  e.bv.x = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rb, 4 * col, 0, 0));
  e.bv.y = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rb, 4 * col + 4, 0, 0));
  e.bv.z = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rb, 4 * col + 8, 0, 0));
  e.bv.w = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rb, 4 * col + 12, 0, 0));
  const __amdgpu_buffer_rsrc_t rf = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint8_t *>(nf), (short)0, 0x7ffffff0, 0x00020000);
  const int row = m32 * 32 + lane;
  const unsigned ob = (lane < 32 && row < M) ? 0u : 0x80000000u;
  const unsigned vo = 4u * (unsigned)((int64_t)(lane < 32 && row < M ? row : 0) * c4n) + ob;
#pragma unroll
  for (int j = 0; j < 8; j++)
    e.w[j] = __builtin_amdgcn_raw_buffer_load_b32(rf, vo, 4 * min(kg0 + j, kg1 - 1), 0);
}
// The flag of the prefetched words (after they have landed).
__device__ inline void epi_flags(EpiPre &e) {
  int f = 0;
#pragma unroll
  for (int j = 0; j < 8; j++) f |= e.w[j] != 0u;
  e.flag = f;
}

// Epilogue of the prefill GEMMs: stages each wave's 32 x 32 NT tile of
// fp32 sums row-major in LDS (free then: every wave has passed the main
// loop's last barrier), rebuilds the reference's Inf / NaN pattern on rows
// with a non-finite activation, and writes 16-byte row pieces of y (with the
// bias) or of this k split's partials.  pre holds the bias quad and the
// flags of the first 8 k groups (epi_prefetch).
template <int NT>
__device__ inline void prefill_epilogue(
    const float16v (&acc)[NT], uint4 *lds, const PrefillSet &ps, int mem, int nt, int m32, int M,
    int c4n, int kg0, int kg1, int64_t K, const float *__restrict__ a,
    const uint8_t *__restrict__ nf, const uint4 *__restrict__ wq,
    const float *__restrict__ scales, const uint8_t *__restrict__ zp4,
    const float *__restrict__ zpf, int nb, int nbh, int lbs, int zpk, int N,
    const EpiPre &pre, float *__restrict__ part, int ks) {
  constexpr int TC = 32 * NT;
  const int t = threadIdx.x, lane = t & 63, lc = lane & 31;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  float *stage = reinterpret_cast<float *>(lds) + wave * (32 * TC);
  const int lh = lane >> 5;
#pragma unroll
  for (int n = 0; n < NT; n++)
#pragma unroll
    for (int v = 0; v < 16; v++) {
      const int r = 8 * (v >> 2) + 4 * lh + (v & 3);
      stage[r * TC + n * 32 + lc] = acc[n][v];
    }
  __syncthreads();
  // Rows of this wave's tile with a non-finite activation in this launch's
  // k range get the reference's Inf / NaN pattern (rare: a uniform branch).
  {
    int flag = pre.flag;
    if (lane < 32 && m32 * 32 + lane < M) {
      const uint32_t *nfw = reinterpret_cast<const uint32_t *>(nf) + (int64_t)(m32 * 32 + lane) * c4n;
      // The rest of the range, eight flag words in flight at a time (one at
      // a time, each load's latency would add up over the k groups).
      for (int kb = kg0 + 8; kb < kg1; kb += 8) {
        uint32_t w[8];
#pragma unroll
        for (int j = 0; j < 8; j++) w[j] = nfw[min(kb + j, kg1 - 1)];  // branch-free
#pragma unroll
        for (int j = 0; j < 8; j++) flag |= w[j] != 0u;
      }
    }
    uint64_t rows = __ballot(flag);
    const int klo = kg0 * KGRP;
    const int64_t khi = min((int64_t)kg1 * KGRP, K);
    while (rows) {
      const int r = __builtin_ctzll(rows);
      rows &= rows - 1;
      const float *arow = a + (int64_t)(m32 * 32 + r) * K;
      bool fnan[2] = {false, false}, fpos[2] = {false, false}, fneg[2] = {false, false};
      for (int64_t k0 = klo; k0 < khi; k0 += 64) {
        const float x = k0 + lane < khi ? arow[k0 + lane] : 0.f;
        uint64_t m = __ballot(!isfinite(x));
        while (m) {
          const int b = __builtin_ctzll(m);
          m &= m - 1;
          const float xv = __shfl(x, b);
#pragma unroll
          for (int u = 0; u < 2; u++) {
            const int c = lane + 64 * u;
            const int col = nt * TC + c;
            if (c >= TC || col >= N) continue;
            const float wv = nbits_weight(wq, scales, zp4, zpf, c4n, nb, nbh, lbs, zpk, col,
                                          (int)(k0 + b));
            if (isnan(xv) || !(wv != 0.f)) fnan[u] = true;
            else if ((xv > 0.f) == (wv > 0.f)) fpos[u] = true;
            else fneg[u] = true;
          }
        }
      }
#pragma unroll
      for (int u = 0; u < 2; u++) {
        const int c = lane + 64 * u;
        if (c >= TC || !(fnan[u] || fpos[u] || fneg[u])) continue;
        stage[r * TC + c] = (fnan[u] || (fpos[u] && fneg[u])) ? __builtin_nanf("")
                            : fpos[u] ? INFINITY : -INFINITY;
      }
    }
  }
  __syncthreads();
  const bool split = gridDim.y > 1;
  float *dst = split ? part + ps.part_off[mem] + (int64_t)ks * M * N : ps.y[mem];
  constexpr int PPR = 8 * NT, RPI = 64 / PPR;  // pieces per row, rows per iteration
  const int c4 = lane % PPR, ro = lane / PPR;
  const int col = nt * TC + 4 * c4;
  const float4 bv = pre.bv;
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

// Workgroup tile: 128 rows x 32*NT columns (NT/2 column groups), 4 waves;
// wave w owns rows [32 w, +32) of the tile and all its columns (NT MFMA
// tiles of 32 x 32).  Per k group (128 k = 2 steps of 64 k):
//   * the workgroup dequantises the 128 x 32*NT weight tile once into LDS as
//     e4m3 fragments (double-buffered: the next k group's packed codes are
//     loaded at the start of the current one and converted a quarter at a
//     time between its MFMAs);
//   * per step each wave runs three MFMA rounds (digits d = 0, 1, 2) over its
//     NT tiles into the k group's fp32 accumulator D, the digit's scales
//     selected with op_sel; after round d the digit-d fragment of the next
//     step is loaded into the same registers (three rounds ahead of use);
//   * the block scale (one per k group: block_size >= 128) is applied on the
//     fp32 accumulator, acc += s * D, deferred to the next k group's first
//     round so those FMAs overlap MFMAs.
// Grid, member choice, split-K partials and the epilogue's row-contiguous
// 16-byte stores are those of the fp16 prefill kernel.
template <int NT, int MW>
__global__ __launch_bounds__(64 * MW, MW == 8 ? 1 : (NT == 4 ? 2 : 3)) void k_gemm_f8x3(
    const uint4 *__restrict__ aq, const uint32_t *__restrict__ asc,
    const uint8_t *__restrict__ nf, const float *__restrict__ a, int64_t K,
    const PrefillSet ps, float *__restrict__ part, int M, int c4n, int nb, int nbh, int lbs,
    int has_zp, int mtiles, int ntiles, int kps) {
  constexpr int PH = NT / 2;          // column groups per tile
  constexpr int HPW = PH * 4 / MW;    // column groups each thread dequantises
  static_assert(HPW >= 1, "tile too narrow for the waves");
  constexpr int TC = 32 * NT;         // tile columns
  constexpr int BU4 = NT * 2 * 2 * 64;  // uint4 per weight buffer: [n32][st][plane][lane]
  constexpr int STAGE_U4 = 8 * MW * TC;  // MW waves x 32 rows x TC floats, in uint4
  constexpr int LDS_U4 = 2 * BU4 > STAGE_U4 ? 2 * BU4 : STAGE_U4;
  __shared__ uint4 lds[LDS_U4];
  __shared__ float scl[2][32][NT];  // [buf][col % 32][n32]
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
  const int m32 = mt * MW + wave;  // this wave's 32-row subtile
  const int lc = lane & 31;

  // Cooperative dequantisation: thread t handles the packed uint4 (column
  // group PH*nt + hb + h, g = wave % 4, col = lane) for h < HPW, hb = HPW *
  // (wave / 4); its dword j (k = 32 j + 8 g .. +7) becomes 8 e4m3 bytes of
  // lane (c % 32) + 32 (g / 2), step j / 2, plane g % 2, 8-byte slot j % 2,
  // where c = 64 (hb + h) + lane is the tile column.
  const int dq_g = wave & 3;
  const int hb = HPW * (wave >> 2);
  int dq_dst[HPW];
#pragma unroll
  for (int h = 0; h < HPW; h++) {
    const int c = 64 * (hb + h) + lane;
    dq_dst[h] = ((c >> 5) * 4 + (dq_g & 1)) * 64 + (c & 31) + 32 * (dq_g >> 1);
  }
  const int nbm1 = nb - 1, nbhm1 = nbh - 1;
  auto rsrc = [](const void *base) __attribute__((always_inline)) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, 0x7ffffff0,
                                             0x00020000);
  };
  __amdgpu_buffer_rsrc_t r_wq[HPW], r_zp[HPW], r_sc[HPW];
#pragma unroll
  for (int h = 0; h < HPW; h++) {
    const int64_t cgi = PH * nt + hb + h;
    r_wq[h] = rsrc(wq + cgi * c4n * 256);
    r_zp[h] = rsrc(zp4 + cgi * nbh * 64);
    r_sc[h] = rsrc(scales + cgi * nb * 64);
  }
  const unsigned vo16 = 16u * lane;
  const unsigned vo_zp = (unsigned)sz_pos(lane);
  const unsigned vo_sc = 4u * vo_zp;
  uint32_t v_mlo, v_mhi, v_magic;
  asm volatile("v_mov_b32 %0, %1" : "=v"(v_mlo) : "s"(0x000F000Fu));
  asm volatile("v_mov_b32 %0, %1" : "=v"(v_mhi) : "s"(0x00F000F0u));
  asm volatile("v_mov_b32 %0, %1" : "=v"(v_magic) : "s"(0x64006400u));
  struct Meta {
    uint4 pk[HPW];
    uint32_t zb[HPW];
    float sc[HPW];
    uint32_t z1[HPW], z16[HPW];
  };
  auto load_meta = [&](int kg, Meta &m) {
    const int blk = (kg * KGRP) >> lbs;
    const int zbyte = min(blk / 2, nbhm1);
#pragma unroll
    for (int h = 0; h < HPW; h++) {
      m.pk[h] = __builtin_bit_cast(
          uint4, __builtin_amdgcn_raw_buffer_load_b128(r_wq[h], vo16, (kg * 4 + dq_g) * 1024, 0));
      m.zb[h] = __builtin_amdgcn_raw_buffer_load_b8(r_zp[h], vo_zp, zbyte * 64, 0);
      m.sc[h] = __builtin_bit_cast(
          float, __builtin_amdgcn_raw_buffer_load_b32(r_sc[h], vo_sc, min(blk, nbm1) * 256, 0));
    }
  };
  // Converts dword j of the packed uint4 into buffer buf (and, with j == 0,
  // stages the k group's block scale).
  auto dequant_quarter = [&](int kg, Meta &m, int buf, int j) {
    const int blk = (kg * KGRP) >> lbs;
#pragma unroll
    for (int h = 0; h < HPW; h++) {
      uint32_t w = j == 0 ? m.pk[h].x : j == 1 ? m.pk[h].y : j == 2 ? m.pk[h].z : m.pk[h].w;
      asm volatile("" : "+v"(w));
      if (j == 0) {
        uint32_t zb = m.zb[h];
        asm volatile("" : "+v"(zb));
        const uint32_t z = has_zp ? (zb >> ((blk & 1) * 4)) & 15u : 8u;
        m.z1[h] = 0xE400E400u + z * 0x00010001u;
        m.z16[h] = 0xE400E400u + z * 0x00100010u;
      }
      const uint4 f = deq8(w, v_mlo, v_mhi, v_magic, __builtin_bit_cast(half2v, m.z1[h]),
                           __builtin_bit_cast(half2v, m.z16[h]));
      short2v b0 = (short2v){0, 0}, b1 = (short2v){0, 0};
      b0 = __builtin_amdgcn_cvt_scalef32_pk_fp8_f16(b0, __builtin_bit_cast(half2v, f.x), 1.0f,
                                                    false);
      b0 = __builtin_amdgcn_cvt_scalef32_pk_fp8_f16(b0, __builtin_bit_cast(half2v, f.y), 1.0f,
                                                    true);
      b1 = __builtin_amdgcn_cvt_scalef32_pk_fp8_f16(b1, __builtin_bit_cast(half2v, f.z), 1.0f,
                                                    false);
      b1 = __builtin_amdgcn_cvt_scalef32_pk_fp8_f16(b1, __builtin_bit_cast(half2v, f.w), 1.0f,
                                                    true);
      uint2 *dst = reinterpret_cast<uint2 *>(&lds[buf * BU4 + dq_dst[h] + (j >> 1) * 128]);
      dst[j & 1] = make_uint2(__builtin_bit_cast(uint32_t, b0), __builtin_bit_cast(uint32_t, b1));
    }
    if (j == 0 && dq_g == 0) {
      const bool in_range = blk < nb;
#pragma unroll
      for (int h = 0; h < HPW; h++) {
        float sc = m.sc[h];
        asm volatile("" : "+v"(sc));
        const int c = 64 * (hb + h) + lane;
        scl[buf][c & 31][c >> 5] = in_range ? sc : 0.f;
      }
    }
  };
  // Digit d of step st of k group kg: 32 bytes (two uint4) of this lane.
  const __amdgpu_buffer_rsrc_t r_a = rsrc(aq + (int64_t)m32 * c4n * 768);
  const __amdgpu_buffer_rsrc_t r_s = rsrc(asc + (int64_t)m32 * c4n * 128);
  const unsigned vo32 = 32u * lane, vo4 = 4u * lane;
  auto a_load = [&](int kg, int st, int d) __attribute__((always_inline)) {
    const int off = ((kg * 2 + st) * 3 + d) * 2048;
    const uint4 x0 = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r_a, vo32, off, 0));
    const uint4 x1 =
        __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r_a, vo32, off + 16, 0));
    return (int8v){(int)x0.x, (int)x0.y, (int)x0.z, (int)x0.w,
                   (int)x1.x, (int)x1.y, (int)x1.z, (int)x1.w};
  };
  auto s_load = [&](int kg, int st) __attribute__((always_inline)) {
    return __builtin_amdgcn_raw_buffer_load_b32(r_s, vo4, (kg * 2 + st) * 256, 0);
  };
  auto b_load = [&](int buf, int n, int st) __attribute__((always_inline)) {
    const uint4 x0 = lds[buf * BU4 + ((n * 2 + st) * 2) * 64 + lane];
    const uint4 x1 = lds[buf * BU4 + ((n * 2 + st) * 2 + 1) * 64 + lane];
    return (int8v){(int)x0.x, (int)x0.y, (int)x0.z, (int)x0.w,
                   (int)x1.x, (int)x1.y, (int)x1.z, (int)x1.w};
  };

  float16v acc[NT], D[NT];
#pragma unroll
  for (int n = 0; n < NT; n++) acc[n] = (float16v){}, D[n] = (float16v){};
  float s_pend[NT];
#pragma unroll
  for (int n = 0; n < NT; n++) s_pend[n] = 0.f;
  const float16v zero16 = (float16v){};
  const int sb = 127;  // weight scale 2^0

  int8v A[3];
  uint32_t sa;
#pragma unroll
  for (int d = 0; d < 3; d++) A[d] = a_load(kg0, 0, d);
  sa = s_load(kg0, 0);
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
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int st = 0; st < 2; st++) {
      int8v B[NT];
#pragma unroll
      for (int n = 0; n < NT; n++) B[n] = b_load(buf, n, st);
      // The fragments of the step after this one: this k group's step 1, or
      // the next k group's step 0 (re-read on the last k group, unused).
      const int nkg = st == 0 ? kg : kgn, nst = st ^ 1;
#pragma unroll
      for (int d = 0; d < 3; d++) {
#pragma unroll
        for (int n = 0; n < NT; n++) {
          if (st == 0 && d == 0) {
#pragma unroll
            for (int v = 0; v < 16; v++) acc[n][v] = fmaf(s_pend[n], D[n][v], acc[n][v]);
          }
          const float16v cin = (st == 0 && d == 0) ? zero16 : D[n];
          D[n] = d == 0   ? mfma_digit<0>(A[0], B[n], cin, (int)sa, sb)
                 : d == 1 ? mfma_digit<1>(A[1], B[n], cin, (int)sa, sb)
                          : mfma_digit<2>(A[2], B[n], cin, (int)sa, sb);
        }
        A[d] = a_load(nkg, nst, d);
        if (d == 2) sa = s_load(nkg, nst);
        __builtin_amdgcn_sched_barrier(0);
      }
      // The next k group's weights, two quarters per step.
      dequant_quarter(kgn, mnext, buf ^ 1, 2 * st);
      dequant_quarter(kgn, mnext, buf ^ 1, 2 * st + 1);
    }
#pragma unroll
    for (int n = 0; n < NT; n++) s_pend[n] = scl[buf][lc][n];
    __syncthreads();
  }
#pragma unroll
  for (int n = 0; n < NT; n++)
#pragma unroll
    for (int v = 0; v < 16; v++) acc[n][v] = fmaf(s_pend[n], D[n][v], acc[n][v]);

  // (Here the loads are issued after the loop: held across it they made
  // this kernel spill.)
  EpiPre pre;
  epi_prefetch<NT>(pre, nt, m32, M, c4n, kg0, kg1, nf, bias, N);
  epi_flags(pre);
  prefill_epilogue<NT>(acc, lds, ps, mem, nt, m32, M, c4n, kg0, kg1, K, a, nf, wq, scales, zp4,
                       nullptr, nb, nbh, lbs, has_zp ? MG_ZP_UINT4 : MG_ZP_NONE, N, pre, part,
                       ks);
}


// Global -> LDS copies (gfx950 global_load_lds_dwordx4 / _dword): lane i's
// 16 (4) bytes land at LDS byte address lds + 16 i (4 i), lds wave-uniform.
// Issued as asm so that the compiler's waits do not treat them as writes to
// every LDS location; the caller waits for them (vmcnt, which returns in
// issue order) before the barrier that publishes the data.
__device__ inline void lds_load16(const void *g, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off"
               :
               : "s"(lds), "v"(g)
               : "memory", "m0");
}
__device__ inline void lds_load4(const void *g, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dword %1, off"
               :
               : "s"(lds), "v"(g)
               : "memory", "m0");
}

// One digit's fp6 MFMA: A and B e2m3 (format 2), the B scale 2 (E8M0 128)
// turning the stored (q - zp) / 2 back into q - zp.
template <int DG>
__device__ inline float16v mfma6_digit(const int8v &a, const int8v &b, const float16v &c,
                                       int sa) {
  return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 2, 2, DG, sa, 0, 128);
}

// The prefill GEMM on weights with prefill images (k_f6_images), with the
// activations as three e2m3 digits (k_af6x3): both MFMA operands fp6, which
// gfx950 runs at twice the fp8 rate.  Tiles, grid, member choice, split-K
// partials, the deferred block scale and the epilogue are those of
// k_gemm_f8x3; per k group the workgroup copies its NT slab images (NT x 3
// KiB: three pieces of NT x 4 bytes per thread, loaded at the start of the
// previous k group) into LDS instead of dequantising, and stages the
// columns' block scales.
// FZP (float zero points, block_size >= 128): the images hold q / 2 and the
// k group adds s (sum a q - z R) with R = sum a over its 128 k (the
// prepass's row sums): its accumulator D starts at -z R instead of zero,
// with z per column and R per row staged in LDS.
template <int NT, bool FZP>
__global__ __launch_bounds__(256, NT == 4 || FZP ? 2 : 3) void k_gemm_f6x3(
    const uint8_t *__restrict__ aq, const uint32_t *__restrict__ asc,
    const uint8_t *__restrict__ nf, const float *__restrict__ rsum,
    const float *__restrict__ a, int64_t K, const PrefillSet ps, float *__restrict__ part,
    int M, int c4n, int nb, int nbh, int lbs, int zpk, int mtiles, int ntiles, int kps) {
  constexpr int PH = NT / 2;           // column groups per tile
  constexpr int TC = 32 * NT;          // tile columns
  constexpr int SLAB = 192;            // uint4 per slab image of a k group
  constexpr int BU4 = NT * SLAB;       // uint4 per weight buffer
  constexpr int STAGE_U4 = 8 * 4 * TC; // 4 waves x 32 rows x TC floats, in uint4
  constexpr int LDS_U4 = 2 * BU4 > STAGE_U4 ? 2 * BU4 : STAGE_U4;
  constexpr int PB = NT * 4;           // bytes per image piece (3 per thread)
  typedef typename std::conditional<NT == 4, uint4, uint2>::type piece_t;
  // LD (integer zero points, both tile widths): the images and block scales
  // go global -> LDS directly (no registers, no LDS stores to schedule), and
  // the activations run in a two-step ring: every load issued in k group kg
  // is for kg + 1, so the in-order return of vector loads never makes a step
  // wait for the images behind its own A, and a step's activations have a
  // whole k group to arrive (with one step of lead, as in the register-staged
  // form, 64-column launches that fill the chip once waited ~0.6 us a step).
  constexpr bool LD = !FZP;
  constexpr int AR = LD ? 2 : 1;
  __shared__ uint4 lds[LDS_U4];
  __shared__ float scl[2][32 * NT];  // [buf][n32][col % 32] (LD), else [buf][col % 32][n32]
  auto si = [](int n, int c) { return LD ? n * 32 + c : c * NT + n; };
  __shared__ float czl[FZP ? 2 : 1][32][NT];  // s * z per column (FZP)
  __shared__ __align__(16) float rl[FZP ? 2 : 1][128];  // row sums of the tile's rows (FZP)
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
  const float *__restrict__ zpf = ps.zpf[mem];
  const float *__restrict__ bias = ps.bias[mem];
  const int N = ps.N[mem];
  const int ks = blockIdx.y;
  const int kg0 = ks * kps;
  const int kg1 = min(c4n, kg0 + kps);
  const int m32 = mt * 4 + wave;  // this wave's 32-row subtile
  const int lc = lane & 31;

  auto rsrc = [](const void *base) __attribute__((always_inline)) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, 0x7ffffff0,
                                             0x00020000);
  };
  // Image pieces p = t + 256 j of the tile's k group (NT slabs x 3072 bytes).
  const uint8_t *__restrict__ img = reinterpret_cast<const uint8_t *>(ps.img[mem]);
  const __amdgpu_buffer_rsrc_t r_im = rsrc(img + (int64_t)NT * nt * c4n * 3072);
  unsigned vo_im[3];
#pragma unroll
  for (int j = 0; j < 3; j++) {
    const int pb = (t + 256 * j) * (LD ? 16 : PB);
    vo_im[j] = (unsigned)((pb / 3072) * c4n * 3072 + pb % 3072);
  }
  // Block scale of tile column tc = t % TC (threads t < TC stage it).
  const int tc = t % TC;
  // (tc / 64 is wave-uniform: one column group per wave.)
  const int tcg = __builtin_amdgcn_readfirstlane(tc / 64);
  const __amdgpu_buffer_rsrc_t r_sc = rsrc(scales + (int64_t)(PH * nt + tcg) * nb * 64);
  const unsigned vo_sc = 4u * (unsigned)sz_pos(tc & 63);
  const int nbm1 = nb - 1;
  // FZP: float zero points like the scales; row sums of row mt * 128 + t % 128
  // (a uniform resource for the tile's rows, the row in the lane offset).
  __amdgpu_buffer_rsrc_t r_zf = r_sc, r_rs = r_sc;
  const unsigned vo_rs = (unsigned)(t & 127) * (unsigned)c4n * 8u;
  if constexpr (FZP) {
    r_zf = rsrc(zpf + (int64_t)(PH * nt + tcg) * nb * 64);
    r_rs = rsrc(rsum + (int64_t)mt * 128 * c4n * 2);
  }
  struct Meta {
    piece_t im[3];
    float sc, zf;
    float2 rs;
  };
  auto load_meta = [&](int kg, Meta &m) {
#pragma unroll
    for (int j = 0; j < 3; j++) {
      if constexpr (NT == 4)
        m.im[j] = __builtin_bit_cast(
            uint4, __builtin_amdgcn_raw_buffer_load_b128(r_im, vo_im[j], kg * 3072, 0));
      else
        m.im[j] = __builtin_bit_cast(
            uint2, __builtin_amdgcn_raw_buffer_load_b64(r_im, vo_im[j], kg * 3072, 0));
    }
    // Blocks past the last (k padding) read as zero scales: the offset goes
    // past the resource (a select on the loaded value would make the
    // compiler wait for it where it computes the select).
    const int blk = (kg * KGRP) >> lbs;
    const unsigned vo_b = vo_sc + (blk < nb ? 0u : 0x80000000u);
    m.sc = __builtin_bit_cast(
        float, __builtin_amdgcn_raw_buffer_load_b32(r_sc, vo_b, min(blk, nbm1) * 256, 0));
    if constexpr (FZP) {
      m.zf = __builtin_bit_cast(
          float, __builtin_amdgcn_raw_buffer_load_b32(r_zf, vo_b, min(blk, nbm1) * 256, 0));
      m.rs = __builtin_bit_cast(float2,
                                __builtin_amdgcn_raw_buffer_load_b64(r_rs, vo_rs, kg * 8, 0));
    }
  };
  // Piece j of the images into buffer buf (j < 3); with j == 0 also the
  // block scales.
  // Every thread stores the block scale (and zero point, row sum) of tile
  // column tc = t % TC (row t % 128): threads t and t + TC loaded the same
  // value, so the duplicate stores write what the first writes.  A store
  // under a branch here let the compiler hoist the piece stores above the
  // k group's products, waiting there for the loads just issued.
  auto store_piece = [&](int kg, Meta &m, int buf, int j) {
    if (j < 3) reinterpret_cast<piece_t *>(&lds[buf * BU4])[t + 256 * j] = m.im[j];
    if (j == 0) {
      scl[buf][si(tc >> 5, tc & 31)] = m.sc;
      if constexpr (FZP) czl[buf][tc & 31][tc >> 5] = m.zf;
      if constexpr (FZP) rl[buf][t & 127] = m.rs.x + m.rs.y;
    }
  };
  // Digit d of step st of k group kg: this lane's six dwords.
  const __amdgpu_buffer_rsrc_t r_a = rsrc(aq + (int64_t)m32 * c4n * 9216);
  const __amdgpu_buffer_rsrc_t r_s = rsrc(asc + (int64_t)m32 * c4n * 128);
  const unsigned vo16 = 16u * lane, vo8 = 1024u + 8u * lane, vo4 = 4u * lane;
  auto a_load = [&](int kg, int st, int d) __attribute__((always_inline)) {
    const int off = ((kg * 2 + st) * 3 + d) * 1536;
    const uint4 x0 = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r_a, vo16, off, 0));
    const uint2 x1 = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(r_a, vo8, off, 0));
    return (int8v){(int)x0.x, (int)x0.y, (int)x0.z, (int)x0.w, (int)x1.x, (int)x1.y, 0, 0};
  };
  auto s_load = [&](int kg, int st) __attribute__((always_inline)) {
    return __builtin_amdgcn_raw_buffer_load_b32(r_s, vo4, (kg * 2 + st) * 256, 0);
  };
  auto b_load = [&](int buf, int n, int st) __attribute__((always_inline)) {
    const int base = buf * BU4 + n * SLAB + st * 96;
    const uint4 x0 = lds[base + lane];
    const uint2 x1 = reinterpret_cast<const uint2 *>(&lds[base + 64])[lane];
    return (int8v){(int)x0.x, (int)x0.y, (int)x0.z, (int)x0.w, (int)x1.x, (int)x1.y, 0, 0};
  };

  float16v acc[NT], D[NT];
#pragma unroll
  for (int n = 0; n < NT; n++) acc[n] = (float16v){}, D[n] = (float16v){};
  float s_pend[NT];
#pragma unroll
  for (int n = 0; n < NT; n++) s_pend[n] = 0.f;
  const float16v zero16 = (float16v){};

  // LD: the image pieces p = t + 256 j of k group kg (16 bytes each: three
  // per thread at NT = 4, one and a half at NT = 2, where waves 2 and 3 skip
  // the second) and the block scales of tile column tc = t (threads t < TC,
  // whole waves) straight into buffer buf.
  auto issue_lds = [&](int kg, int buf) {
    const uint8_t *ib = img + ((int64_t)NT * nt * c4n + kg) * 3072;
    const uint32_t lb = (uint32_t)reinterpret_cast<uintptr_t>(&lds[buf * BU4]);
#pragma unroll
    for (int j = 0; j < 3; j++)
      if ((64 * wave + 256 * j) * 16 < NT * 3072)
        lds_load16(ib + vo_im[j], lb + (64 * wave + 256 * j) * 16);
    if (t < TC) {
      const int blk = min((kg * KGRP) >> lbs, nbm1);  // < nb here: bs >= 128 and kpad = nb bs
      lds_load4(scales + ((int64_t)(PH * nt + tcg) * nb + blk) * 64 + sz_pos(tc & 63),
                (uint32_t)reinterpret_cast<uintptr_t>(&scl[buf][0]) + 256 * wave);
    }
  };

  EpiPre pre;
  epi_prefetch<NT>(pre, nt, m32, M, c4n, kg0, kg1, nf, bias, N);
  // Activation ring: AR steps of the three digits and their scale word.
  int8v A[AR][3];
  uint32_t sa[AR];
  if constexpr (LD) issue_lds(kg0, 0);
#pragma unroll
  for (int j = 0; j < AR; j++) {
#pragma unroll
    for (int d = 0; d < 3; d++) A[j][d] = a_load(kg0, j, d);
    sa[j] = s_load(kg0, j);
  }
  if constexpr (LD) {
    // All of it landed (the compiler also sees the ring consumed here, so
    // its own wait counts in the loop start from an empty queue).
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#pragma unroll
    for (int j = 0; j < AR; j++)
      asm volatile("" ::"v"(A[j][0][0]), "v"(A[j][0][4]), "v"(A[j][1][0]), "v"(A[j][1][4]),
                   "v"(A[j][2][0]), "v"(A[j][2][4]), "v"(sa[j]));
  } else {
    Meta m0;
    load_meta(kg0, m0);
#pragma unroll
    for (int j = 0; j < 4; j++) store_piece(kg0, m0, 0, j);
  }
  __syncthreads();
  epi_flags(pre);

  for (int kg = kg0; kg < kg1; kg++) {
    const int buf = (kg - kg0) & 1;
    const int kgn = min(kg + 1, kg1 - 1);  // next k group (clamped)
    Meta mnext;
    // LD: four small loads of this k group's activation slices (in L2),
    // then the copies for the next one.  The compiler counts only its own
    // loads in its waits, so a wait for a load older than the copies
    // would also wait for up to four copies behind it; with these four
    // between, such waits end before the copies.  Consuming the last of
    // them at the end of the k group waits for the copies themselves.
    uint32_t pad[4];
    if constexpr (LD) {
#pragma unroll
      for (int j = 0; j < 4; j++)
        pad[j] = __builtin_amdgcn_raw_buffer_load_b32(r_a, vo4, (kg * 6 + j) * 1536, 0);
      if (kg + 1 < kg1) issue_lds(kg + 1, buf ^ 1);
    } else {
      load_meta(kgn, mnext);
    }
    // FZP: this k group's -z R (the lane's 16 rows are 8 i + 4 (lane / 32) +
    // 0..3 of the wave's 32, i = v / 4).
    float rr[FZP ? 16 : 1];
    if constexpr (FZP) {
      const int lh = lane >> 5;
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const float4 x = *reinterpret_cast<const float4 *>(&rl[buf][wave * 32 + 8 * i + 4 * lh]);
        rr[4 * i] = x.x, rr[4 * i + 1] = x.y, rr[4 * i + 2] = x.z, rr[4 * i + 3] = x.w;
      }
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int st = 0; st < 2; st++) {
      int8v B[NT];
#pragma unroll
      for (int n = 0; n < NT; n++) B[n] = b_load(buf, n, st);
      // Ring slot of this step and the step its registers are reloaded with
      // (AR = 2: the same step of the next k group).
      const int sl = AR == 2 ? st : 0;
      const int nkg = AR == 2 || st == 1 ? kgn : kg, nst = AR == 2 ? st : st ^ 1;
#pragma unroll
      for (int d = 0; d < 3; d++) {
#pragma unroll
        for (int n = 0; n < NT; n++) {
          if (st == 0 && d == 0) {
#pragma unroll
            for (int v = 0; v < 16; v++) acc[n][v] = fmaf(s_pend[n], D[n][v], acc[n][v]);
          }
          float16v cin = (st == 0 && d == 0) ? zero16 : D[n];
          if constexpr (FZP) {
            if (st == 0 && d == 0) {
              const float z = czl[buf][lc][n];
#pragma unroll
              for (int v = 0; v < 16; v++) cin[v] = -z * rr[v];
            }
          }
          D[n] = d == 0   ? mfma6_digit<0>(A[sl][0], B[n], cin, (int)sa[sl])
                 : d == 1 ? mfma6_digit<1>(A[sl][1], B[n], cin, (int)sa[sl])
                          : mfma6_digit<2>(A[sl][2], B[n], cin, (int)sa[sl]);
        }
        A[sl][d] = a_load(nkg, nst, d);
        if (d == 2) sa[sl] = s_load(nkg, nst);
        __builtin_amdgcn_sched_barrier(0);
      }
      if constexpr (!LD) {
        store_piece(kgn, mnext, buf ^ 1, 2 * st);
        store_piece(kgn, mnext, buf ^ 1, 2 * st + 1);
      }
    }
    if constexpr (LD) asm volatile("" ::"v"(pad[0]), "v"(pad[1]), "v"(pad[2]), "v"(pad[3]));
#pragma unroll
    for (int n = 0; n < NT; n++) s_pend[n] = scl[buf][si(n, lc)];
    __syncthreads();
  }
#pragma unroll
  for (int n = 0; n < NT; n++)
#pragma unroll
    for (int v = 0; v < 16; v++) acc[n][v] = fmaf(s_pend[n], D[n][v], acc[n][v]);
  prefill_epilogue<NT>(acc, lds, ps, mem, nt, m32, M, c4n, kg0, kg1, K, a, nf, wq, scales, zp4,
                       zpf, nb, nbh, lbs, zpk, N, pre, part, ks);
}

// The fp6 prefill GEMM for small launches (weights with prefill images,
// integer zero points, too few 128 x 128 tiles to fill the chip): a
// workgroup takes 32 rows x 64 columns (one column group), and its four
// waves take a quarter of the k groups each.  A wave streams its activation
// digits and image fragments straight into registers, reloading each slot
// for the next k group right after its last use (the vector-memory queue
// then always holds one k group ahead), and applies the block scale per k
// group (acc += s D).  No LDS holds operands and no barrier separates the
// k groups, so the serial chain of a workgroup is a quarter of K; the four
// partial tiles meet in LDS and are added in wave order (deterministic),
// with no split-K launch.  Rows with a non-finite activation get the
// reference's Inf / NaN pattern as in prefill_epilogue.
__global__ __launch_bounds__(256, 2) void k_gemm_f6kw(
    const uint8_t *__restrict__ aq, const uint32_t *__restrict__ asc,
    const uint8_t *__restrict__ nf, const float *__restrict__ a, int64_t K,
    const PrefillSet ps, int M, int c4n, int nb, int nbh, int lbs, int zpk, int mt32,
    int ntiles) {
  __shared__ __align__(16) float part[4][32 * 64];
  __shared__ int sflag[4][32];
  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int L = blockIdx.x;
  const int xcd = L & 7, q = L >> 3;
  const int mt = q % mt32;  // 32-row tile
  const int ntg = (q / mt32) * 8 + xcd;
  if (ntg >= ntiles) return;
  int cg;
  const int mem = prefill_member(ps, ntg, &cg);  // column group of the member
  const int N = ps.N[mem];
  const int lc = lane & 31;
  auto rsrc = [](const void *base) __attribute__((always_inline)) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, 0x7ffffff0,
                                             0x00020000);
  };
  const __amdgpu_buffer_rsrc_t r_a = rsrc(aq + (int64_t)mt * c4n * 9216);
  const __amdgpu_buffer_rsrc_t r_s = rsrc(asc + (int64_t)mt * c4n * 128);
  const __amdgpu_buffer_rsrc_t r_b =
      rsrc(reinterpret_cast<const uint8_t *>(ps.img[mem]) + (int64_t)2 * cg * c4n * 3072);
  const __amdgpu_buffer_rsrc_t r_c = rsrc(ps.scales[mem] + (int64_t)cg * nb * 64);
  const unsigned vo16 = 16u * lane, vo8 = 1024u + 8u * lane, vo4 = 4u * lane;
  const unsigned vo_c0 = 4u * (unsigned)sz_pos(lc), vo_c1 = 4u * (unsigned)sz_pos(32 + lc);
  // ob: added to every lane offset; 0x80000000 puts a load past its
  // resource, so it touches no memory (the loads after a wave's last k
  // group are issued that way rather than under a branch: behind one the
  // compiler waits for every load in flight before the products).
  auto frag = [&](const __amdgpu_buffer_rsrc_t &r, int off, unsigned ob)
                  __attribute__((always_inline)) {
    const uint4 x0 =
        __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, vo16 + ob, off, 0));
    const uint2 x1 =
        __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(r, vo8 + ob, off, 0));
    return (int8v){(int)x0.x, (int)x0.y, (int)x0.z, (int)x0.w, (int)x1.x, (int)x1.y, 0, 0};
  };
  auto a_load = [&](int kg, int st, int d, unsigned ob = 0u) __attribute__((always_inline)) {
    return frag(r_a, ((kg * 2 + st) * 3 + d) * 1536, ob);
  };
  auto b_load = [&](int kg, int st, int n, unsigned ob = 0u) __attribute__((always_inline)) {
    return frag(r_b, (n * c4n + kg) * 3072 + st * 1536, ob);
  };
  auto s_load = [&](int kg, int st, unsigned ob = 0u) __attribute__((always_inline)) {
    return __builtin_amdgcn_raw_buffer_load_b32(r_s, vo4 + ob, (kg * 2 + st) * 256, 0);
  };
  auto c_load = [&](int kg, unsigned vo, unsigned ob = 0u) __attribute__((always_inline)) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                         r_c, vo + ob, ((kg * KGRP) >> lbs) * 256, 0));
  };

  // What the epilogue reads that the k loop does not produce, loaded now so
  // that its latency hides under the loop (read at the end, the flag words
  // and the bias were up to four dependent round trips): the non-finite flag
  // words of row lane (lanes < 32) for k groups 8 w .. 8 w + 7 of wave w, and
  // the bias of this thread's eight output columns.  Offsets past the
  // resources (words past c4n, rows past M, columns past N, no bias) read
  // zeros and touch no memory.
  uint32_t fw[8];
  {
    const __amdgpu_buffer_rsrc_t r_f = rsrc(nf);
    const int frow = mt * 32 + lane;
    const bool frow_ok = lane < 32 && frow < M;
    const unsigned vo_f = 4u * (unsigned)((int64_t)(frow_ok ? frow : 0) * c4n);
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const int wd = 8 * wave + i;
      fw[i] = __builtin_amdgcn_raw_buffer_load_b32(
          r_f, vo_f + 4u * (unsigned)wd + (frow_ok && wd < c4n ? 0u : 0x80000000u), 0, 0);
    }
  }
  float bv[8];
  {
    const float *bias = ps.bias[mem];
    const __amdgpu_buffer_rsrc_t r_bias = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float *>(bias), (short)0, bias ? N * 4 : 0, 0x00020000);
    const unsigned vo_bias = 4u * (unsigned)(cg * 64 + 8 * (t & 7));
#pragma unroll
    for (int i = 0; i < 8; i++)
      bv[i] = __builtin_bit_cast(float,
                                 __builtin_amdgcn_raw_buffer_load_b32(r_bias, vo_bias + 4u * i, 0, 0));
  }

  float16v acc[2], D[2];
#pragma unroll
  for (int n = 0; n < 2; n++) acc[n] = (float16v){}, D[n] = (float16v){};
  const int kpw = (c4n + 3) >> 2;
  const int kb = min(c4n, wave * kpw), ke = min(c4n, kb + kpw);
  if (kb < ke) {
    int8v A[2][3], B[2][2];
    uint32_t sa[2];
    float sc[2];
#pragma unroll
    for (int st = 0; st < 2; st++) {
#pragma unroll
      for (int d = 0; d < 3; d++) A[st][d] = a_load(kb, st, d);
      B[st][0] = b_load(kb, st, 0);
      B[st][1] = b_load(kb, st, 1);
      sa[st] = s_load(kb, st);
    }
    sc[0] = c_load(kb, vo_c0);
    sc[1] = c_load(kb, vo_c1);
    const float16v zero16 = (float16v){};
    for (int kg = kb; kg < ke; kg++) {
      const bool more = kg + 1 < ke;  // wave-uniform
      const int kn = min(kg + 1, ke - 1);
      const unsigned ob = more ? 0u : 0x80000000u;
#pragma unroll
      for (int st = 0; st < 2; st++) {
#pragma unroll
        for (int d = 0; d < 3; d++) {
#pragma unroll
          for (int n = 0; n < 2; n++) {
            const float16v cin = (st == 0 && d == 0) ? zero16 : D[n];
            D[n] = d == 0   ? mfma6_digit<0>(A[st][0], B[st][n], cin, (int)sa[st])
                   : d == 1 ? mfma6_digit<1>(A[st][1], B[st][n], cin, (int)sa[st])
                            : mfma6_digit<2>(A[st][2], B[st][n], cin, (int)sa[st]);
          }
          A[st][d] = a_load(kn, st, d, ob);
        }
        B[st][0] = b_load(kn, st, 0, ob);
        B[st][1] = b_load(kn, st, 1, ob);
        sa[st] = s_load(kn, st, ob);
      }
      const float s0 = sc[0], s1 = sc[1];
      sc[0] = c_load(kn, vo_c0, ob);
      sc[1] = c_load(kn, vo_c1, ob);
#pragma unroll
      for (int v = 0; v < 16; v++) {
        acc[0][v] = fmaf(s0, D[0][v], acc[0][v]);
        acc[1][v] = fmaf(s1, D[1][v], acc[1][v]);
      }
    }
  }
  // The four partial tiles, row-major, then their sum in wave order.
  {
    float *pw = part[wave];
    const int lh = lane >> 5;
#pragma unroll
    for (int n = 0; n < 2; n++)
#pragma unroll
      for (int v = 0; v < 16; v++)
        pw[(8 * (v >> 2) + 4 * lh + (v & 3)) * 64 + n * 32 + lc] = acc[n][v];
    int f = 0;
#pragma unroll
    for (int i = 0; i < 8; i++) f |= fw[i] != 0u;
    if (lane < 32) sflag[wave][lane] = f;
  }
  __syncthreads();
  const int r = t >> 3, c0 = 8 * (t & 7);
  float4v y0 = *reinterpret_cast<const float4v *>(&part[0][r * 64 + c0]);
  float4v y1 = *reinterpret_cast<const float4v *>(&part[0][r * 64 + c0 + 4]);
#pragma unroll
  for (int w = 1; w < 4; w++) {
    y0 += *reinterpret_cast<const float4v *>(&part[w][r * 64 + c0]);
    y1 += *reinterpret_cast<const float4v *>(&part[w][r * 64 + c0 + 4]);
  }
  // Rows of the tile with a non-finite activation (rare; every wave computes
  // the same mask, so the branch is uniform over the workgroup).
  int flag = lane < 32 ? (sflag[0][lane] | sflag[1][lane] | sflag[2][lane] | sflag[3][lane]) : 0;
  if (lane < 32 && mt * 32 + lane < M) {
    const uint32_t *nfw = reinterpret_cast<const uint32_t *>(nf) + (int64_t)(mt * 32 + lane) * c4n;
    // Words past the 32 prefetched (K > 4096).
    for (int kq = 32; kq < c4n; kq += 8) {
      uint32_t fr[8];
#pragma unroll
      for (int j = 0; j < 8; j++) fr[j] = nfw[min(kq + j, c4n - 1)];
#pragma unroll
      for (int j = 0; j < 8; j++) flag |= fr[j] != 0u;
    }
  }
  uint64_t rows = __ballot(flag);
  if (rows) {
    *reinterpret_cast<float4v *>(&part[0][r * 64 + c0]) = y0;
    *reinterpret_cast<float4v *>(&part[0][r * 64 + c0 + 4]) = y1;
    __syncthreads();
    if (wave == 0) {
      const int col = cg * 64 + lane;
      while (rows) {
        const int rr = __builtin_ctzll(rows);
        rows &= rows - 1;
        const float *arow = a + (int64_t)(mt * 32 + rr) * K;
        bool fnan = false, fpos = false, fneg = false;
        for (int64_t k0 = 0; k0 < K; k0 += 64) {
          const float x = k0 + lane < K ? arow[k0 + lane] : 0.f;
          uint64_t m = __ballot(!isfinite(x));
          while (m) {
            const int bi = __builtin_ctzll(m);
            m &= m - 1;
            const float xv = __shfl(x, bi);
            if (col >= N) continue;
            const float wv = nbits_weight(ps.wq[mem], ps.scales[mem], ps.zp4[mem], ps.zpf[mem],
                                          c4n, nb, nbh, lbs, zpk, col, (int)(k0 + bi));
            if (isnan(xv) || !(wv != 0.f)) fnan = true;
            else if ((xv > 0.f) == (wv > 0.f)) fpos = true;
            else fneg = true;
          }
        }
        if (fnan || fpos || fneg)
          part[0][rr * 64 + lane] = (fnan || (fpos && fneg)) ? __builtin_nanf("")
                                    : fpos ? INFINITY : -INFINITY;
      }
    }
    __syncthreads();
    y0 = *reinterpret_cast<const float4v *>(&part[0][r * 64 + c0]);
    y1 = *reinterpret_cast<const float4v *>(&part[0][r * 64 + c0 + 4]);
  }
  const int row = mt * 32 + r;
  if (row >= M) return;
  const int col = cg * 64 + c0;
  float yv[8] = {y0[0], y0[1], y0[2], y0[3], y1[0], y1[1], y1[2], y1[3]};
#pragma unroll
  for (int j = 0; j < 8; j++) yv[j] += bv[j];
  float *p = ps.y[mem] + (int64_t)row * N + col;
  if (ps.y_vec[mem] && (N % 4) == 0 && col + 7 < N) {
    __builtin_nontemporal_store((float4v){yv[0], yv[1], yv[2], yv[3]},
                                reinterpret_cast<float4v *>(p));
    __builtin_nontemporal_store((float4v){yv[4], yv[5], yv[6], yv[7]},
                                reinterpret_cast<float4v *>(p + 4));
  } else {
#pragma unroll
    for (int j = 0; j < 8; j++)
      if (col + j < N) p[j] = yv[j];
  }
}

}  // namespace

size_t mg_nbits_f8_ws(int64_t mpad, int64_t c4, size_t *off_asc, size_t *off_nf,
                      size_t *off_rs) {
  const size_t aq = (size_t)mpad * c4 * 128 * 3;  // 3 bytes per element
  *off_asc = mg_align(aq);
  *off_nf = mg_align(*off_asc + (size_t)mpad * c4 * 16);  // 4 scale words per 128 k per row
  *off_rs = mg_align(*off_nf + (size_t)mpad * c4 * 4);     // row sums per 64 k
  return mg_align(*off_rs + (size_t)mpad * c4 * 8);
}

mg_status mg_nbits_prefill_f8(mg_ctx *ctx, int n, const mg_weight *const *w, const float *a_dev,
                              int64_t M, float *const *y_dev, void *ws, int64_t mpad, int nt,
                              int ksplit, int kps, size_t off_part, int kwave) {
  const mg_weight *w0 = w[0];
  const mg_nbits_dev &d = w0->nbits;
  hipStream_t st = ctx->stream;
  char *base = static_cast<char *>(ws);
  size_t off_asc = 0, off_nf = 0, off_rs = 0;
  (void)mg_nbits_f8_ws(mpad, d.c4, &off_asc, &off_nf, &off_rs);
  uint4 *aq = reinterpret_cast<uint4 *>(base);
  uint32_t *asc = reinterpret_cast<uint32_t *>(base + off_asc);
  uint8_t *nf = reinterpret_cast<uint8_t *>(base + off_nf);
  float *rsum = reinterpret_cast<float *>(base + off_rs);
  float *part = ksplit > 1 ? reinterpret_cast<float *>(base + off_part) : nullptr;
  const int vec = (w0->K % 4 == 0) && (reinterpret_cast<uintptr_t>(a_dev) % 16 == 0);
  const int has_zp = d.zp_kind == MG_ZP_UINT4;
  const bool fzp = d.zp_kind == MG_ZP_FLOAT;
  PrefillSet ps{};
  ReduceSet rs{};
  int ct = 0;
  int64_t eend = 0;
  make_prefill_sets(n, w, y_dev, M, ksplit, nt, &ps, &rs, &ct, &eend);
  bool f6 = true;  // every member has its prefill images
  for (int i = 0; i < n; i++) f6 = f6 && ps.img[i] != nullptr;
  if (fzp && !f6)  // the planner sends float zero points here only with images
    return mg_fail(MG_INVALID_ARGUMENT, "MatMulNBits: float zero points without prefill images");
  if (f6)
    hipLaunchKernelGGL(k_af6x3, dim3((unsigned)((mpad / 32) * d.c4 * 2)), dim3(64), 0, st, a_dev, M,
                       w0->K, (int)d.c4, vec, reinterpret_cast<uint8_t *>(aq), asc, nf,
                       fzp ? rsum : nullptr);
  else
    hipLaunchKernelGGL(k_af8x3, dim3((unsigned)((mpad / 32) * d.c4 * 2)), dim3(256), 0, st, a_dev,
                       M, w0->K, (int)d.c4, vec, aq, asc, nf);
  MG_TRY(mg_launch_check(f6 ? "k_af6x3" : "k_af8x3"));
  if (kwave) {  // the planner sends only fp6, integer-zero-point, 64-column plans here
    if (!f6 || fzp || nt != 2 || ksplit != 1)
      return mg_fail(MG_DEVICE_ERROR, "MatMulNBits: invalid wave-split prefill plan");
    const int mt32 = (int)((M + 31) / 32);
    hipLaunchKernelGGL(k_gemm_f6kw, dim3((unsigned)(8 * mt32 * ((ct + 7) / 8))), dim3(256), 0,
                       st, reinterpret_cast<const uint8_t *>(aq), asc, nf, a_dev, w0->K, ps,
                       (int)M, (int)d.c4, (int)d.nb, (int)d.nbh, __builtin_ctzll(d.bs),
                       (int)d.zp_kind, mt32, ct);
    return mg_launch_check("k_gemm_f6kw");
  }
  // (256-row workgroups of 8 waves, k_gemm_f8x3<4, 8>, dequantise each
  // weight tile once for twice the rows; measured 2-4% slower on the lm_head
  // at M = 512, so 128-row tiles are used.)
  const int mtiles = (int)(mpad / 128);
  const dim3 grid((unsigned)(8 * mtiles * ((ct + 7) / 8)), (unsigned)ksplit);
#define MG_F8_ARGS                                                                         \
  aq, asc, nf, a_dev, w0->K, ps, part, (int)M, (int)d.c4, (int)d.nb, (int)d.nbh,          \
      __builtin_ctzll(d.bs), has_zp, mtiles, ct, kps
  const uint8_t *aq6 = reinterpret_cast<const uint8_t *>(aq);
  const int zpk = d.zp_kind;
#define MG_F6_ARGS                                                                         \
  aq6, asc, nf, rsum, a_dev, w0->K, ps, part, (int)M, (int)d.c4, (int)d.nb, (int)d.nbh,   \
      __builtin_ctzll(d.bs), zpk, mtiles, ct, kps
  if (f6 && fzp && nt == 4)
    hipLaunchKernelGGL((k_gemm_f6x3<4, true>), grid, dim3(256), 0, st, MG_F6_ARGS);
  else if (f6 && fzp)
    hipLaunchKernelGGL((k_gemm_f6x3<2, true>), grid, dim3(256), 0, st, MG_F6_ARGS);
  else if (f6 && nt == 4)
    hipLaunchKernelGGL((k_gemm_f6x3<4, false>), grid, dim3(256), 0, st, MG_F6_ARGS);
  else if (f6)
    hipLaunchKernelGGL((k_gemm_f6x3<2, false>), grid, dim3(256), 0, st, MG_F6_ARGS);
  else if (nt == 4)
    hipLaunchKernelGGL((k_gemm_f8x3<4, 4>), grid, dim3(256), 0, st, MG_F8_ARGS);
  else
    hipLaunchKernelGGL((k_gemm_f8x3<2, 4>), grid, dim3(256), 0, st, MG_F8_ARGS);
#undef MG_F8_ARGS
#undef MG_F6_ARGS
  MG_TRY(mg_launch_check(f6 ? "k_gemm_f6x3" : "k_gemm_f8x3"));
  if (ksplit > 1) MG_TRY(launch_gemm_reduce(st, part, rs, eend, ksplit));
  return MG_OK;
}

bool mg_nbits_f8_eligible(const mg_nbits_dev &d) { return d.bs >= KGRP; }

mg_status mg_nbits_f8_images(mg_ctx *ctx, mg_weight *w) {
  mg_nbits_dev &d = w->nbits;
  const size_t bytes = (size_t)d.ng * 2 * d.c4 * 3072;  // 3/4 byte per (padded) weight
  MG_HIP(hipMalloc(&d.img, bytes));
  w->device_bytes += (int64_t)bytes;
  const int64_t n = d.ng * d.c4 * 64;  // (cg, kg, col)
  const int has_zp = d.zp_kind == MG_ZP_UINT4;
  hipLaunchKernelGGL(k_f6_images, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, ctx->stream,
                     reinterpret_cast<const uint4 *>(d.wq), d.zp4, has_zp,
                     d.zp_kind == MG_ZP_FLOAT ? 0 : 8, n, (int)d.c4, (int)d.nbh,
                     __builtin_ctzll(d.bs), static_cast<uint8_t *>(d.img));
  MG_TRY(mg_launch_check("k_f6_images"));
  MG_HIP(hipStreamSynchronize(ctx->stream));
  return MG_OK;
}
