// Shared by the MatMulNBits kernels (nbits.hip, nbits_f8.hip): the device
// weight layout helpers, the dequantiser of packed codes, and the structures
// and reduction of the prefill GEMMs.  Everything here is internal to the
// library (anonymous namespace: each translation unit has its own copy).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "mg_internal.h"

namespace {

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float float4v __attribute__((ext_vector_type(4)));
typedef float float16v __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int KGRP = 128;  // k per k group
constexpr int CGRP = 64;   // columns per column group
constexpr int FIX_MAX = 30583;  // 7 * (1 + 16 + 256 + 4096): 4 balanced int4 digits

__host__ __device__ inline int nib_pos(int t) {
  return (t & 1) ? 4 + (t >> 1) : (t >> 1);
}

// Position of column c (0..63) of a column group in the per-block scale and
// zero-point rows: the four 16-column tiles of one column residue are
// adjacent, so a lane that owns columns c, c + 16, c + 32, c + 48 (the
// 16-row MFMA GEMV) reads their four values with one load.
__host__ __device__ inline int sz_pos(int c) { return (c & 15) * 4 + (c >> 4); }

constexpr int GMAX = 4;  // weights launched together at most

// Dequantises one weight dword (8 codes, nibble order of wq) to 8 exact fp16
// values for the MFMA path.  Masking a nibble into the fp16 pattern 0x6400
// (1024.0) gives 1024 + q for a nibble at bits 0-3 of a half-word and
// 1024 + 16q for one at bits 4-7, so the pairs (t0,t1), (t4,t5) come out as
// q - zp and (t2,t3), (t6,t7) as 16(q - zp) with a single shift for all
// eight; the activation prepass scales k offsets 2,3,6,7 of every 8 by 1/16
// to match.  `mask`/`magic` are register operands (one v_and_or_b32 each).
__device__ inline uint4 deq8(uint32_t x, uint32_t mlo, uint32_t mhi, uint32_t magic,
                             half2v zz1, half2v zz16) {
  const uint32_t y = x >> 8;
  const uint32_t d0 = (x & mlo) | magic, d1 = (x & mhi) | magic;
  const uint32_t d2 = (y & mlo) | magic, d3 = (y & mhi) | magic;
  return make_uint4(__builtin_bit_cast(uint32_t, __builtin_bit_cast(half2v, d0) + zz1),
                    __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2v, d1) + zz16),
                    __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2v, d2) + zz1),
                    __builtin_bit_cast(uint32_t, __builtin_bit_cast(half2v, d3) + zz16));
}

// Up to GMAX weights that share K, block size, zero-point kind and the input
// activations, run as one prefill launch: the grid's column tiles are the
// concatenation of the members' column tiles (ct_end holds the running
// totals), and each workgroup picks its member from them.  Split-K partials of
// member i start at part + part_off[i] ([ksplit][M][N_i]).
struct PrefillSet {
  const uint4 *wq[GMAX];
  const uint4 *img[GMAX];  // prefill images (mg_nbits_dev::img) or null
  const float *scales[GMAX];
  const uint8_t *zp4[GMAX];
  const float *zpf[GMAX];  // float zero points (MG_ZP_FLOAT) or null
  const float *bias[GMAX];
  float *y[GMAX];
  int64_t part_off[GMAX];
  int N[GMAX];
  int ct_end[GMAX];
  int y_vec[GMAX];  // y base 16-byte aligned
  int n;
};

// Member of global column tile x and its local tile index (workgroup-uniform).
__device__ inline int prefill_member(const PrefillSet &ps, int x, int *nt) {
  int m = 0;
#pragma unroll
  for (int i = 0; i < GMAX - 1; i++)
    if (i + 1 < ps.n && x >= ps.ct_end[i]) m = i + 1;
  *nt = x - (m ? ps.ct_end[m - 1] : 0);
  return m;
}

// y_i = sum over k splits of the partials of member i + bias_i
// (deterministic split-K reduction); elements of the members concatenated,
// member i starting at element e_end[i - 1] (M * N_i elements each).
struct ReduceSet {
  const float *bias[GMAX];
  float *y[GMAX];
  int64_t part_off[GMAX];
  int64_t e_end[GMAX];
  int N[GMAX];
  int n;
};
// Thread = VW consecutive elements of one member (VW = 4: every N % 4 == 0
// and y 16-byte aligned, so a piece never straddles rows or members).  The
// splits are added in split order, four loads in flight at a time.
template <int VW>
__global__ __launch_bounds__(256) void k_gemm_reduce(const float *__restrict__ part,
                                                     const ReduceSet rs, int ksplit) {
  typedef float fv __attribute__((ext_vector_type(VW)));
  const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * VW;
  if (i >= rs.e_end[rs.n - 1]) return;
  int m = 0;
#pragma unroll
  for (int j = 0; j < GMAX - 1; j++)
    if (j + 1 < rs.n && i >= rs.e_end[j]) m = j + 1;
  const int64_t li = i - (m ? rs.e_end[m - 1] : 0);
  const int64_t mn = rs.e_end[m] - (m ? rs.e_end[m - 1] : 0);
  const fv *p = reinterpret_cast<const fv *>(part + rs.part_off[m] + li);
  const int64_t step = mn / VW;
  fv s = (fv)(0.f);
  int k = 0;
  for (; k + 4 <= ksplit; k += 4) {
    const fv x0 = p[k * step], x1 = p[(k + 1) * step];
    const fv x2 = p[(k + 2) * step], x3 = p[(k + 3) * step];
    s += x0;
    s += x1;
    s += x2;
    s += x3;
  }
  for (; k < ksplit; k++) s += p[k * step];
  const float *b = rs.bias[m];
  float *y = rs.y[m] + li;
  if constexpr (VW == 1) {
    *y = s[0] + (b ? b[li % rs.N[m]] : 0.f);
  } else {
    const int64_t c = li % rs.N[m];
    if (b) s += *reinterpret_cast<const fv *>(b + c);
    *reinterpret_cast<fv *>(y) = s;
  }
}

// The member tables of n sibling weights launched as one prefill GEMM
// (column tiles of 32 * nt columns), and of its split-K reduction; ct and
// eend receive the total column tiles and output elements.
inline void make_prefill_sets(int n, const mg_weight *const *w, float *const *y_dev, int64_t M,
                              int ksplit, int nt, PrefillSet *ps, ReduceSet *rs, int *ct,
                              int64_t *eend) {
  const bool has_zp = w[0]->nbits.zp_kind == MG_ZP_UINT4;
  ps->n = rs->n = n;
  int c = 0;
  int64_t poff = 0, e = 0;
  for (int i = 0; i < n; i++) {
    const mg_nbits_dev &di = w[i]->nbits;
    ps->wq[i] = reinterpret_cast<const uint4 *>(di.wq);
    ps->img[i] = static_cast<const uint4 *>(di.img);
    ps->scales[i] = di.scales;
    // The kernels read zero-point bytes unconditionally (branch-free); without
    // zero points they are pointed at the scales, which are at least as large.
    ps->zp4[i] = has_zp ? di.zp4 : reinterpret_cast<const uint8_t *>(di.scales);
    ps->zpf[i] = di.zpf;
    ps->bias[i] = rs->bias[i] = di.bias;
    ps->y[i] = rs->y[i] = y_dev[i];
    ps->N[i] = rs->N[i] = (int)w[i]->N;
    ps->y_vec[i] = (reinterpret_cast<uintptr_t>(y_dev[i]) % 16) == 0;
    ps->part_off[i] = rs->part_off[i] = poff;
    poff += (int64_t)ksplit * M * w[i]->N;
    e += M * w[i]->N;
    rs->e_end[i] = e;
    c += (int)(nt == 4 ? di.ng / 2 : di.ng);
    ps->ct_end[i] = c;
  }
  *ct = c;
  *eend = e;
}

// Launches the split-K sum: four elements per thread when no piece can
// straddle a row (every N % 4 == 0, y and the bias 16-byte aligned: partial
// offsets are then multiples of 4 elements and the buffer is aligned).
inline mg_status launch_gemm_reduce(hipStream_t st, const float *part, const ReduceSet &rs,
                                    int64_t eend, int ksplit) {
  bool v4 = true;
  for (int i = 0; i < rs.n; i++)
    v4 = v4 && rs.N[i] % 4 == 0 && reinterpret_cast<uintptr_t>(rs.y[i]) % 16 == 0 &&
         reinterpret_cast<uintptr_t>(rs.bias[i]) % 16 == 0;
  if (v4)
    hipLaunchKernelGGL(k_gemm_reduce<4>, dim3((unsigned)((eend / 4 + 255) / 256)), dim3(256), 0,
                       st, part, rs, ksplit);
  else
    hipLaunchKernelGGL(k_gemm_reduce<1>, dim3((unsigned)((eend + 255) / 256)), dim3(256), 0, st,
                       part, rs, ksplit);
  return mg_launch_check("k_gemm_reduce");
}

}  // namespace
