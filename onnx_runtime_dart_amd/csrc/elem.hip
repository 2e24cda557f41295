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
#include <initializer_list>

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

// Fixed-order double sum over the NT threads of a workgroup (shuffles within
// each wave, then the wave sums in wave order).  Every thread gets it.
template <int NT>
__device__ inline double block_sum(double v, double *red) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off);
  const int t = threadIdx.x;
  __syncthreads();  // red may still be read from a previous call
  if ((t & 63) == 0) red[t >> 6] = v;
  __syncthreads();
  double r = red[0];
#pragma unroll
  for (int w = 1; w < NT / 64; w++) r += red[w];
  return r;
}

// W consecutive floats (W = 4: one 16-byte access).
template <int W>
__device__ inline void ld_w(const float *p, float (&v)[W]) {
  if constexpr (W == 4) {
    const float4 q = *reinterpret_cast<const float4 *>(p);
    v[0] = q.x, v[1] = q.y, v[2] = q.z, v[3] = q.w;
  } else {
    v[0] = p[0];
  }
}
template <int W>
__device__ inline void st_w(float *p, const float (&v)[W]) {
  if constexpr (W == 4) *reinterpret_cast<float4 *>(p) = make_float4(v[0], v[1], v[2], v[3]);
  else p[0] = v[0];
}

// RMSNorm over the last axis: one workgroup of NT threads per row of d
// elements.  With a skip input the row is s = x + skip (f32), written to sum
// when asked; with a bias, out = normed + bias (f32), as the reference's Add
// after the norm.  With P > 0 thread t owns P slots of W elements, slot i at
// W (t + NT i) (W = 4: float4 accesses; the host takes it when d % 4 == 0
// and every buffer is 16-byte aligned), and keeps them, with their gamma and
// bias, in registers between the sum of squares and the output: the row is
// read once.  P = 0 walks the row twice, one element per thread per step.
// Any of x, skip, sum and y may be the same buffer (an in-place residual):
// each element is read and written by one thread only, and with P = 0, once
// sum holds s the second pass reads s back from it instead of re-adding x
// and skip.  With ybuf, y is also staged there (the split producer) and *mx
// receives the largest finite |y| of the thread's elements.
template <int NT, int P, int W>
__device__ inline void rms_row(const float *x, const float *skip,
                               const float *__restrict__ gamma, const float *__restrict__ bias,
                               double eps, int64_t d, float *y, float *sum, double *red,
                               float *ybuf, float *mx) {
  const int64_t base = (int64_t)blockIdx.x * d;
  const int t = threadIdx.x;
  double ss = 0;
  float m = 0.f;
  auto keep = [&](int64_t j, const auto &o) __attribute__((always_inline)) {
    if (ybuf) {
      st_w(ybuf + j, o);
      for (float f : o) m = fabsf(f) < INFINITY ? fmaxf(m, fabsf(f)) : m;  // finite values only
    }
  };
  if constexpr (P > 0) {
    float v[P][W], g[P][W], b[P][W];
#pragma unroll
    for (int i = 0; i < P; i++) {
      const int64_t j = (int64_t)W * (t + NT * i);
#pragma unroll
      for (int c = 0; c < W; c++) v[i][c] = g[i][c] = b[i][c] = 0.f;
      if (j < d) {  // d % W == 0: the whole slot is in the row
        ld_w<W>(x + base + j, v[i]);
        ld_w<W>(gamma + j, g[i]);
        if (bias) ld_w<W>(bias + j, b[i]);
        if (skip) {
          float k[W];
          ld_w<W>(skip + base + j, k);
#pragma unroll
          for (int c = 0; c < W; c++) v[i][c] = v[i][c] + k[c];
        }
      }
    }
#pragma unroll
    for (int i = 0; i < P; i++) {
      const int64_t j = (int64_t)W * (t + NT * i);
      if (j < d) {
        if (skip && sum) st_w<W>(sum + base + j, v[i]);
#pragma unroll
        for (int c = 0; c < W; c++) ss += (double)v[i][c] * (double)v[i][c];
      }
    }
    ss = block_sum<NT>(ss, red);
    const double inv = 1.0 / sqrt(ss / (double)d + eps);
#pragma unroll
    for (int i = 0; i < P; i++) {
      const int64_t j = (int64_t)W * (t + NT * i);
      if (j < d) {
        float o[W];
#pragma unroll
        for (int c = 0; c < W; c++) {
          o[c] = (float)((double)v[i][c] * inv * (double)g[i][c]);
          if (bias) o[c] = o[c] + b[i][c];
        }
        st_w<W>(y + base + j, o);
        keep(j, o);
      }
    }
  } else {
    for (int64_t j = t; j < d; j += NT) {
      float w = x[base + j];
      if (skip) {
        w = w + skip[base + j];
        if (sum) sum[base + j] = w;
      }
      ss += (double)w * (double)w;
    }
    ss = block_sum<NT>(ss, red);
    const double inv = 1.0 / sqrt(ss / (double)d + eps);
    for (int64_t j = t; j < d; j += NT) {
      float w;
      if (skip && sum) w = sum[base + j];
      else if (skip) w = x[base + j] + skip[base + j];
      else w = x[base + j];
      float o[1] = {(float)((double)w * inv * (double)gamma[j])};
      if (bias) o[0] = o[0] + bias[j];
      y[base + j] = o[0];
      keep(j, o);
    }
  }
  if (mx) *mx = m;
}

template <int NT, int P, int W>
__global__ __launch_bounds__(NT) void k_rms_last(const float *x, const float *skip,
                                                 const float *__restrict__ gamma,
                                                 const float *__restrict__ bias, double eps,
                                                 int64_t d, float *y, float *sum) {
  __shared__ double red[NT / 64];
  rms_row<NT, P, W>(x, skip, gamma, bias, eps, d, y, sum, red, nullptr, nullptr);
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

// Block-wide maximum over NT threads (every thread gets it); red holds NT / 64.
template <int NT>
__device__ inline float block_max(float v, float *red) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
  const int t = threadIdx.x;
  __syncthreads();
  if ((t & 63) == 0) red[t >> 6] = v;
  __syncthreads();
  float r = red[0];
#pragma unroll
  for (int w = 1; w < NT / 64; w++) r = fmaxf(r, red[w]);
  return r;
}

// Row `row` of the split from the d values staged in ybuf (mx: the largest
// finite |y| of this thread's elements; the barrier in block_max makes every
// thread's ybuf stores visible).  NT threads; octets up to kpad / 8.
template <int NT>
__device__ inline void write_split_row(const float *ybuf, int64_t d, int64_t kpad, float mx,
                                       int row, uint4 *__restrict__ ahl, int *__restrict__ texp,
                                       float *red) {
  mx = block_max<NT>(mx, red);
  int e = 0;
  if (mx > 0.f) {
    int ex;
    frexpf(mx, &ex);
    e = 14 - ex;
  }
  const int t = threadIdx.x;
  if (t == 0) texp[row] = e;
  for (int64_t o = t; o < kpad / 8; o += NT) {
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

// RMSNorm over the last axis (k_rms_last's arithmetic and plan, element for
// element) writing y, the optional sum, and the split of y.  One workgroup
// per row, at most 16 rows, d <= SPLIT_MAXD.
template <int NT, int P, int W>
__global__ __launch_bounds__(NT) void k_rms_last_split(
    const float *x, const float *skip, const float *__restrict__ gamma,
    const float *__restrict__ bias, double eps, int64_t d, float *y, float *sum, int64_t kpad,
    uint4 *__restrict__ ahl, int *__restrict__ texp) {
  __shared__ double red[NT / 64];
  __shared__ float redf[NT / 64];
  __shared__ float ybuf[SPLIT_MAXD];
  float mx;
  rms_row<NT, P, W>(x, skip, gamma, bias, eps, d, y, sum, red, ybuf, &mx);
  write_split_row<NT>(ybuf, d, kpad, mx, (int)blockIdx.x, ahl, texp, redf);
}

inline unsigned blocks(int64_t n, int64_t per) { return (unsigned)((n + per - 1) / per); }

template <int NT_, int P_, int W_>
struct RmsPlan {
  static constexpr int NT = NT_, P = P_, W = W_;
};

// The row norm's plan for rows of d: float4 slots when d % 4 == 0 and every
// buffer is 16-byte aligned (vec), with enough threads for one or a few
// slots each; else one element per slot; rows too long for registers walk
// twice.  The plain and the split kernel take the same plan, so their y
// are bitwise equal.
template <class F>
void rms_dispatch(int64_t d, bool vec, F &&f) {
  if (vec && d % 4 == 0) {
    const int64_t q = d / 4;
    if (q <= 256) return f(RmsPlan<256, 1, 4>{});
    if (q <= 512) return f(RmsPlan<512, 1, 4>{});
    if (q <= 1024) return f(RmsPlan<1024, 1, 4>{});
    if (q <= 2048) return f(RmsPlan<1024, 2, 4>{});
    if (q <= 4096) return f(RmsPlan<1024, 4, 4>{});
  }
  if (d <= 256) return f(RmsPlan<256, 1, 1>{});
  if (d <= 1024) return f(RmsPlan<256, 4, 1>{});
  if (d <= 2048) return f(RmsPlan<256, 8, 1>{});
  if (d <= 4096) return f(RmsPlan<256, 16, 1>{});
  f(RmsPlan<256, 0, 1>{});
}

bool aligned16(std::initializer_list<const void *> ps) {
  for (const void *p : ps)
    if (reinterpret_cast<uintptr_t>(p) % 16) return false;  // null passes
  return true;
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
    rms_dispatch(dim, aligned16({x, skip, gamma, bias, y, sum}), [&](auto plan) {
      using C = decltype(plan);
      hipLaunchKernelGGL((k_rms_last<C::NT, C::P, C::W>), dim3((unsigned)outer), dim3(C::NT), 0,
                         ctx->stream, x, skip, gamma, bias, eps, dim, y, sum);
    });
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
  rms_dispatch(d, aligned16({x, skip, gamma, bias, y, sum}), [&](auto plan) {
    using C = decltype(plan);
    hipLaunchKernelGGL((k_rms_last_split<C::NT, C::P, C::W>), dim3((unsigned)rows), dim3(C::NT),
                       0, ctx->stream, x, skip, gamma, bias, eps, d, y, sum, kpad, ahl, texp);
  });
  return mg_launch_check("k_rms_last_split");
}
