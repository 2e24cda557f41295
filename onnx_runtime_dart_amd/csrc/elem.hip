// Elementwise device ops between the matrix products of a decoder layer, so
// that its activations stay in HBM from one product to the next:
//   * Add / Sub / Mul / Div of float tensors with broadcasting
//     (lib/src/onnx_ops.dart:26-44, :103-330, :402, :444-448, :476);
//   * Sigmoid (lib/src/onnx_ops.dart:2349-2350);
//   * RMSNorm (opRMSNorm, lib/src/onnx_ops.dart:1771-1815) and the residual
//     add + RMSNorm of SkipSimplifiedLayerNormalization
//     (lib/src/onnx_graph.dart:1793-1813).
//
// Numbers.  The reference computes each op in double and stores f32; for
// + - * / of two f32 values that equals the correctly rounded f32 op (53 >=
// 2 * 24 + 2 bits), which is what these kernels compute.  Sigmoid and the
// RMSNorm scale are computed in double as the reference does; the RMSNorm
// sum of squares is a fixed-order parallel double sum (the reference adds in
// k order: the two differ only by double rounding, far below an f32 ulp).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>

#include "mg_internal.h"

namespace {

template <int OP>
__device__ inline float bin_op(float x, float y) {
  if (OP == MG_BIN_ADD) return x + y;
  if (OP == MG_BIN_SUB) return x - y;
  if (OP == MG_BIN_MUL) return x * y;
  return x / y;
}

// Equal shapes: four elements per thread (VEC: 16-byte aligned operands).
// y may be a or b (each element is read before it is written).
template <int OP, bool VEC>
__global__ __launch_bounds__(256) void k_bin_same(const float *a, const float *b, float *y,
                                                  int64_t n) {
  const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
  if (i >= n) return;
  if (VEC && i + 4 <= n) {
    const float4 x = *reinterpret_cast<const float4 *>(a + i);
    const float4 v = *reinterpret_cast<const float4 *>(b + i);
    *reinterpret_cast<float4 *>(y + i) = make_float4(bin_op<OP>(x.x, v.x), bin_op<OP>(x.y, v.y),
                                                     bin_op<OP>(x.z, v.z), bin_op<OP>(x.w, v.w));
  } else {
    for (int64_t k = i; k < std::min<int64_t>(i + 4, n); k++) y[k] = bin_op<OP>(a[k], b[k]);
  }
}

// Broadcast: output element -> coordinates over the merged output dims ->
// operand offsets (stride 0 along broadcast dims).
template <int OP>
__global__ __launch_bounds__(256) void k_bin_bcast(const float *a, const float *b, float *y,
                                                   int64_t n, const mg_elem_bcast s) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  int64_t rem = i, ia = 0, ib = 0;
#pragma unroll
  for (int k = MG_ELEM_MAXRANK - 1; k >= 0; k--) {
    if (k >= s.rank) continue;
    const int64_t c = rem % s.dim[k];
    rem /= s.dim[k];
    ia += c * s.sa[k];
    ib += c * s.sb[k];
  }
  y[i] = bin_op<OP>(a[ia], b[ib]);
}

__global__ __launch_bounds__(256) void k_sigmoid(const float *x, float *y, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  y[i] = (float)(1.0 / (1.0 + exp(-(double)x[i])));
}

// Fixed-order double sum over the 256 threads of a workgroup (shuffles within
// each wave, then the four wave sums in wave order).  Every thread gets it.
__device__ inline double block_sum(double v, double *red) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off);
  const int t = threadIdx.x;
  __syncthreads();  // red may still be read from a previous call
  if ((t & 63) == 0) red[t >> 6] = v;
  __syncthreads();
  return ((red[0] + red[1]) + red[2]) + red[3];
}

// RMSNorm over the last axis: one workgroup per row of d elements.  With a
// skip input the row is s = x + skip (f32), written to sum when asked; with
// a bias, out = normed + bias (f32), as the reference's Add after the norm.
// Thread t owns elements t, t + 256, ...: with P > 0 (d <= 256 P) it keeps
// them in registers between the sum of squares and the output, so the row
// is read once; P = 0 walks the row twice.  Any of x, skip, sum and y may be
// the same buffer (an in-place residual): each element is read and written
// by one thread only, and with P = 0, once sum holds s the second pass reads
// s back from it instead of re-adding x and skip.  With ybuf, y is also
// staged there (the split producer) and *mx receives the largest finite |y|
// of the thread's elements.
template <int P>
__device__ inline void rms_row(const float *x, const float *skip,
                               const float *__restrict__ gamma, const float *__restrict__ bias,
                               double eps, int64_t d, float *y, float *sum, double *red,
                               float *ybuf, float *mx) {
  const int64_t base = (int64_t)blockIdx.x * d;
  const int t = threadIdx.x;
  double ss = 0;
  float v[P > 0 ? P : 1];
  if constexpr (P > 0) {
#pragma unroll
    for (int i = 0; i < P; i++) {
      const int64_t j = t + 256 * i;
      v[i] = 0.f;
      if (j < d) {
        v[i] = x[base + j];
        if (skip) v[i] = v[i] + skip[base + j];
      }
    }
#pragma unroll
    for (int i = 0; i < P; i++) {
      const int64_t j = t + 256 * i;
      if (j < d) {
        if (skip && sum) sum[base + j] = v[i];
        ss += (double)v[i] * (double)v[i];
      }
    }
  } else {
    for (int64_t j = t; j < d; j += 256) {
      float w = x[base + j];
      if (skip) {
        w = w + skip[base + j];
        if (sum) sum[base + j] = w;
      }
      ss += (double)w * (double)w;
    }
  }
  ss = block_sum(ss, red);
  const double inv = 1.0 / sqrt(ss / (double)d + eps);
  float m = 0.f;
  auto out = [&](int64_t j, float w) __attribute__((always_inline)) {
    float o = (float)((double)w * inv * (double)gamma[j]);
    if (bias) o = o + bias[j];
    y[base + j] = o;
    if (ybuf) {
      ybuf[j] = o;
      const float f = fabsf(o);
      m = f < INFINITY ? fmaxf(m, f) : m;  // finite values only
    }
  };
  if constexpr (P > 0) {
#pragma unroll
    for (int i = 0; i < P; i++)
      if (t + 256 * i < d) out(t + 256 * i, v[i]);
  } else {
    for (int64_t j = t; j < d; j += 256) {
      float w;
      if (skip && sum) w = sum[base + j];
      else if (skip) w = x[base + j] + skip[base + j];
      else w = x[base + j];
      out(j, w);
    }
  }
  if (mx) *mx = m;
}

template <int P>
__global__ __launch_bounds__(256) void k_rms_last(const float *x, const float *skip,
                                                  const float *__restrict__ gamma,
                                                  const float *__restrict__ bias, double eps,
                                                  int64_t d, float *y, float *sum) {
  __shared__ double red[4];
  rms_row<P>(x, skip, gamma, bias, eps, d, y, sum, red, nullptr, nullptr);
}

// RMSNorm over another axis: one thread per (outer, inner) slice, walking the
// reduce axis in order as the reference does; gamma follows the last axis.
__global__ __launch_bounds__(256) void k_rms_axis(const float *x,
                                                  const float *__restrict__ gamma, double eps,
                                                  int64_t outer, int64_t dim, int64_t inner,
                                                  int64_t last, float *y) {
  const int64_t s = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (s >= outer * inner) return;
  const int64_t o = s / inner, i = s % inner;
  const int64_t base = o * dim * inner + i;
  double ss = 0;
  for (int64_t j = 0; j < dim; j++) {
    const double v = x[base + j * inner];
    ss += v * v;
  }
  const double inv = 1.0 / sqrt(ss / (double)dim + eps);
  for (int64_t j = 0; j < dim; j++) {
    const int64_t idx = base + j * inner;
    y[idx] = (float)((double)x[idx] * inv * (double)gamma[idx % last]);
  }
}

// ---------------------------------------------- split activations for the GEMV
//
// The MatMulNBits decode GEMV (3 to 16 rows) takes its activations as an
// fp16 hi/lo pair per element with a power-of-two row exponent, in its MFMA
// A-operand order; its own prepass builds them from the fp32 rows.  The
// RMSNorm / SkipSimplifiedLayerNormalization kernel over the last axis can
// also write that split of the row it produces (a norm owns whole rows, so
// the row maximum costs it one more reduction), and the GEMV that consumes
// it then needs no prepass launch.  It computes y exactly as without the
// split, stages the row in LDS, and converts
// it exactly as the prepass would convert the stored y (same row maximum,
// exponent and rounding): the GEMV's results are bitwise those of the
// prepass path.
//
// Layout (mg_nbits_split_bytes): uint4 at ((kg * 4 + j) * 2 + part) * 64 +
// 16 g + row holds the 8 halves of k = 128 kg + 32 j + 8 g + 0..7 (part 0
// hi, 1 lo), for rows 0..15 and k up to kpad (zeros past the row); the int32
// row exponents follow at byte mg_align(16 * kpad * 4).

typedef _Float16 half8e __attribute__((ext_vector_type(8)));
constexpr int SPLIT_MAXD = 8192;  // longest row the producers stage in LDS

// Block-wide maximum (every thread gets it); red holds 4 floats.
__device__ inline float block_max(float v, float *red) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
  const int t = threadIdx.x;
  __syncthreads();
  if ((t & 63) == 0) red[t >> 6] = v;
  __syncthreads();
  return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

// Row `row` of the split from the d values staged in ybuf (mx: the largest
// finite |y| of this thread's elements).  256 threads; octets up to kpad / 8.
__device__ inline void write_split_row(const float *ybuf, int64_t d, int64_t kpad, float mx,
                                       int row, uint4 *__restrict__ ahl, int *__restrict__ texp,
                                       float *red) {
  mx = block_max(mx, red);
  int e = 0;
  if (mx > 0.f) {
    int ex;
    frexpf(mx, &ex);
    e = 14 - ex;
  }
  const int t = threadIdx.x;
  if (t == 0) texp[row] = e;
  for (int64_t o = t; o < kpad / 8; o += 256) {
    half8e hi, lo;
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const int64_t k = o * 8 + i;
      const float x = ldexpf(k < d ? ybuf[k] : 0.f, (i & 2) ? e - 4 : e);
      const _Float16 hh = (_Float16)x;
      float res = x - (float)hh;
      if (!isfinite(res)) res = 0.f;
      hi[i] = hh;
      lo[i] = (_Float16)res;
    }
    const int64_t kg = o >> 4, j = (o >> 2) & 3, g = o & 3;
    uint4 *dst = ahl + ((kg * 4 + j) * 2) * 64 + 16 * g + row;
    dst[0] = __builtin_bit_cast(uint4, hi);
    dst[64] = __builtin_bit_cast(uint4, lo);
  }
}

// RMSNorm over the last axis (k_rms_last's arithmetic, element for element)
// writing y, the optional sum, and the split of y.  One workgroup per row,
// rows < 16, d <= SPLIT_MAXD.
template <int P>
__global__ __launch_bounds__(256) void k_rms_last_split(
    const float *x, const float *skip, const float *__restrict__ gamma,
    const float *__restrict__ bias, double eps, int64_t d, float *y, float *sum, int64_t kpad,
    uint4 *__restrict__ ahl, int *__restrict__ texp) {
  __shared__ double red[4];
  __shared__ float redf[4];
  __shared__ float ybuf[SPLIT_MAXD];
  float mx;
  rms_row<P>(x, skip, gamma, bias, eps, d, y, sum, red, ybuf, &mx);
  write_split_row(ybuf, d, kpad, mx, (int)blockIdx.x, ahl, texp, redf);
}

inline unsigned blocks(int64_t n, int64_t per) { return (unsigned)((n + per - 1) / per); }

// Elements per thread kept in registers for a row of d (0: two passes).
inline int rms_regs(int64_t d) {
  return d <= 256 ? 1 : d <= 1024 ? 4 : d <= 2048 ? 8 : d <= 4096 ? 16 : 0;
}

}  // namespace

mg_status mg_elem_binary(mg_ctx *ctx, int op, const float *a, const float *b, float *y,
                         int64_t n, bool same, const mg_elem_bcast &s) {
  if (n == 0) return MG_OK;
  hipStream_t st = ctx->stream;
  if (same) {
    const bool vec = (reinterpret_cast<uintptr_t>(a) | reinterpret_cast<uintptr_t>(b) |
                      reinterpret_cast<uintptr_t>(y)) % 16 == 0;
#define MG_SAME(OP_)                                                                        \
  if (vec) hipLaunchKernelGGL((k_bin_same<OP_, true>), dim3(blocks(n, 1024)), dim3(256), 0, st, \
                              a, b, y, n);                                                  \
  else hipLaunchKernelGGL((k_bin_same<OP_, false>), dim3(blocks(n, 1024)), dim3(256), 0, st, a, \
                          b, y, n)
    switch (op) {
      case MG_BIN_ADD: MG_SAME(MG_BIN_ADD); break;
      case MG_BIN_SUB: MG_SAME(MG_BIN_SUB); break;
      case MG_BIN_MUL: MG_SAME(MG_BIN_MUL); break;
      default: MG_SAME(MG_BIN_DIV); break;
    }
#undef MG_SAME
    return mg_launch_check("k_bin_same");
  }
#define MG_BC(OP_) \
  hipLaunchKernelGGL((k_bin_bcast<OP_>), dim3(blocks(n, 256)), dim3(256), 0, st, a, b, y, n, s)
  switch (op) {
    case MG_BIN_ADD: MG_BC(MG_BIN_ADD); break;
    case MG_BIN_SUB: MG_BC(MG_BIN_SUB); break;
    case MG_BIN_MUL: MG_BC(MG_BIN_MUL); break;
    default: MG_BC(MG_BIN_DIV); break;
  }
#undef MG_BC
  return mg_launch_check("k_bin_bcast");
}

mg_status mg_elem_sigmoid(mg_ctx *ctx, const float *x, float *y, int64_t n) {
  if (n == 0) return MG_OK;
  hipLaunchKernelGGL(k_sigmoid, dim3(blocks(n, 256)), dim3(256), 0, ctx->stream, x, y, n);
  return mg_launch_check("k_sigmoid");
}

mg_status mg_elem_rms_norm(mg_ctx *ctx, const float *x, const float *skip, const float *gamma,
                           const float *bias, double eps, int64_t outer, int64_t dim,
                           int64_t inner, int64_t last, float *y, float *sum) {
  if (outer * dim * inner == 0) return MG_OK;
  if (inner == 1) {  // the caller keeps rows (outer) below 2^31
#define MG_RMS(P_)                                                                           \
  hipLaunchKernelGGL((k_rms_last<P_>), dim3((unsigned)outer), dim3(256), 0, ctx->stream, x, \
                     skip, gamma, bias, eps, dim, y, sum)
    switch (rms_regs(dim)) {
      case 1: MG_RMS(1); break;
      case 4: MG_RMS(4); break;
      case 8: MG_RMS(8); break;
      case 16: MG_RMS(16); break;
      default: MG_RMS(0); break;
    }
#undef MG_RMS
    return mg_launch_check("k_rms_last");
  }
  hipLaunchKernelGGL(k_rms_axis, dim3(blocks(outer * inner, 256)), dim3(256), 0, ctx->stream, x,
                     gamma, eps, outer, dim, inner, last, y);
  return mg_launch_check("k_rms_axis");
}

mg_status mg_elem_rms_norm_split(mg_ctx *ctx, const float *x, const float *skip,
                                 const float *gamma, const float *bias, double eps, int64_t rows,
                                 int64_t d, float *y, float *sum, int64_t kpad, void *split) {
  if (rows == 0 || d == 0) return MG_OK;
  uint4 *ahl = static_cast<uint4 *>(split);
  int *texp = reinterpret_cast<int *>(static_cast<char *>(split) + mg_align((size_t)16 * kpad * 4));
#define MG_RMS(P_)                                                                        \
  hipLaunchKernelGGL((k_rms_last_split<P_>), dim3((unsigned)rows), dim3(256), 0, ctx->stream, \
                     x, skip, gamma, bias, eps, d, y, sum, kpad, ahl, texp)
  switch (rms_regs(d)) {
    case 1: MG_RMS(1); break;
    case 4: MG_RMS(4); break;
    case 8: MG_RMS(8); break;
    case 16: MG_RMS(16); break;
    default: MG_RMS(0); break;
  }
#undef MG_RMS
  return mg_launch_check("k_rms_last_split");
}
