/* CPU oracle for the matrix-multiply operator family of onnx_runtime_dart.
 *
 * TEST INFRASTRUCTURE ONLY.  This is the checker the parity tests compare the
 * HIP kernels against, and the CPU baseline bench.py times beside them.  It is
 * never linked into, loaded by, or called from the product library
 * (onnx_runtime_dart_amd/), which fails loudly when its HIP build is missing.
 *
 * Each function restates one reference routine; the citation on each names
 * the file:line it follows (paths relative to the reference checkout).
 * Status codes mirror the product ABI: 0 ok, 1 invalid argument (Dart
 * ArgumentError), 2 unsupported (Dart UnsupportedError).
 */
#ifndef MIGEMM_ORACLE_H
#define MIGEMM_ORACLE_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { ORC_OK = 0, ORC_INVALID_ARGUMENT = 1, ORC_UNSUPPORTED = 2 };

/* matmulKernel: out[m x n] = a[m x k] . b[k x n], row-major, out overwritten.
 * lib/src/gemm_kernel_simd.dart:32-239 (routing), :244-389 (4x16 direct),
 * :480-538 / :543-610 (GEMV), :616-675 (small M).  f32 lanes multiply then add
 * with one rounding each, in k order; the scalar column tails of the m<4
 * paths accumulate in double (:601-609, :665-673). */
void orc_matmul_kernel(const float *a, const float *b, float *out, int64_t m,
                       int64_t k, int64_t n);

/* GemmPool (lib/src/parallel_pool.dart:217-261, :299-329): b [k x n] split
 * by columns over `workers` threads (n / W each, the first n % W one more),
 * each running matmulKernel on its slice with its own copy of a; the result
 * is bitwise orc_matmul_kernel's.  create returns NULL on bad arguments. */
void *orc_pool_create(const float *b, int64_t k, int64_t n, int workers);
int orc_pool_matmul(void *pool, const float *a, int64_t m, float *y);
void orc_pool_destroy(void *pool);

/* opMatMul: numpy-broadcast batched matmul, lib/src/onnx_ops.dart:1710-1766.
 * Shapes have rank >= 2.  y is sized by the broadcast output shape. */
int orc_matmul_f32(const float *a, const int64_t *a_shape, int a_rank,
                   const float *b, const int64_t *b_shape, int b_rank,
                   float *y);
/* MatMul on non-float operands given as doubles (double sum over k in
 * order, one rounding to f32). */
int orc_matmul_f64acc(const double *a, const int64_t *a_shape, int a_rank,
                      const double *b, const int64_t *b_shape, int b_rank,
                      float *y);

/* opGemm (+ the graph's transB prepack): lib/src/onnx_ops.dart:2152-2172,
 * lib/src/onnx_graph.dart:2156-2173.  a, b rank 2; c may be NULL or any shape
 * that broadcasts to [M, N]. */
int orc_gemm_f32(const float *a, const int64_t *a_shape, const float *b,
                 const int64_t *b_shape, const float *c, const int64_t *c_shape,
                 int c_rank, double alpha, double beta, int trans_a,
                 int trans_b, float *y);

/* opMatMulNBits, lib/src/onnx_qlinear_ops.dart:115-228.
 * zp_kind: 0 none (default 8), 1 packed uint4 [N * ceil(nb/2)], 2 float
 * [N * nb].  bias may be NULL.  Shapes are assumed validated by the caller
 * except for the checks on k, n, bits and block_size. */
int orc_matmul_nbits(const float *a, int64_t m, int64_t k, int64_t n,
                     int64_t bits, int64_t block_size, const uint8_t *b,
                     const float *scales, int zp_kind, const void *zp,
                     const float *bias, float *y);

/* Dequantized weight element w(col, kk) of opMatMulNBits (the `weight`
 * closure at lib/src/onnx_qlinear_ops.dart:177-191). */
float orc_nbits_weight(int64_t col, int64_t kk, int64_t k, int64_t block_size,
                       const uint8_t *b, const float *scales, int zp_kind,
                       const void *zp);

/* opMatMulInteger, lib/src/onnx_qlinear_ops.dart:32-81.  a/b are uint8 or
 * int8 (per *_signed) with a_batch*m*k and b_batch*k*n elements; zero-point
 * arrays are already widened to int32 (NULL = absent).  y: int64, batch*m*n
 * elements with batch = max(a_batch, b_batch). */
int orc_matmul_integer(const void *a, int a_signed, int64_t a_batch,
                       const void *b, int b_signed, int64_t b_batch, int64_t m,
                       int64_t k, int64_t n, const int32_t *a_zp,
                       int64_t a_zp_len, const int32_t *b_zp, int64_t b_zp_len,
                       int64_t *y);

/* opQLinearMatMul, lib/src/onnx_qlinear_ops.dart:85-108 (lo/hi from the
 * output zero point's dtype, lib/src/onnx_graph.dart:2902-2917). */
int orc_qlinear_matmul(const void *a, int a_signed, int64_t a_batch,
                       const void *b, int b_signed, int64_t b_batch, int64_t m,
                       int64_t k, int64_t n, float a_scale,
                       const int32_t *a_zp, int64_t a_zp_len, float b_scale,
                       const int32_t *b_zp, int64_t b_zp_len, float y_scale,
                       int32_t y_zp, int32_t lo, int32_t hi, int64_t *y);

/* opDynamicQuantizeLinear, lib/src/onnx_ops.dart:3556-3583. */
int orc_dynamic_quantize_linear(const float *x, int64_t n, uint8_t *y,
                                float *scale, int32_t *zp);

/* opFusedSDPA, lib/src/onnx_ops.dart:2106-2149: s = opMatMul(a, b); per score
 * row val = s * scale + mask (double, stored as f32; mask broadcast
 * right-aligned, a last dim != T read with stride 0), e = exp(val - max),
 * val = e / sum; y = opMatMul(s, v).  y sized by the broadcast output shape. */
int orc_fused_sdpa(const float *a, const int64_t *a_shape, int a_rank,
                   const float *b, const int64_t *b_shape, int b_rank,
                   const float *v, const int64_t *v_shape, int v_rank,
                   const float *mask, const int64_t *mask_shape, int mask_rank,
                   double scale, float *y);

/* opMultiHeadAttention, lib/src/onnx_ops.dart:2019-2098: per (batch, head)
 * the gathered Q.K^T (matmulKernel), scale + bias [batch, bias_heads, seq,
 * kv_seq] (head h reads bias head h % bias_heads), row softmax multiplied by
 * the inverse sum, then . V; out [batch, seq, hidden]. */
int orc_multi_head_attention(const float *q, const float *k, const float *v,
                             int64_t batch, int64_t seq, int64_t kv_seq,
                             int64_t hidden, int64_t num_heads, const float *bias,
                             int64_t bias_heads, int has_scale, double scale,
                             float *out);

/* opRotaryEmbedding, lib/src/onnx_ops.dart:2659-2722, for a [batch, seq,
 * heads * hs] input at positions pos[seq] (one row shared by the batch):
 * the first 2 half_rot dims of every head rotated (GPT-J pairs when
 * interleaved, else rotate-half) in double, stored as f32; the tail copied. */
void orc_rotary_embedding(const float *x, int64_t batch, int64_t seq, int64_t heads,
                          int64_t hs, const int64_t *pos, const float *cos_cache,
                          const float *sin_cache, int64_t half_rot, int interleaved,
                          float *out);

/* opGroupQueryAttention, lib/src/onnx_ops.dart:1844-2012: optional RoPE of
 * q and k at positions past_len + s; present K/V = past followed by the
 * current (rotated) K / raw V; per query head h (KV head h / group) the
 * gathered Q.K^T (matmulKernel), scale + bias (head h % bias_heads), a
 * softmax over keys 0 .. past_len + i only (the rest 0), then . V. */
int orc_group_query_attention(const float *q, const float *k, const float *v, int64_t batch,
                              int64_t seq, int64_t hidden, int64_t heads, int64_t kv_heads,
                              const float *past_k, const float *past_v, int64_t past_len,
                              const float *cos_cache, const float *sin_cache, int64_t half_rot,
                              int do_rotary, int interleaved, const float *bias,
                              int64_t bias_heads, int has_scale, double scale, float *out,
                              float *present_k, float *present_v);

/* Convolution sums, direct loops over (channel, tap) per output element,
 * spatial dims right-aligned in 3 slots.  kind 0 = f32, 1 = u8, 2 = i8.
 *   trans = 0 (opConv, lib/src/onnx_nn_ops.dart:179-817, and _convIntAcc,
 *     lib/src/onnx_qlinear_ops.dart:232-283): w [M][C/group][taps], input
 *     position i = o * str - pad + k * dil, out-of-range taps skipped.
 *   trans = 1 (opConvTranspose, lib/src/onnx_nn_ops.dart:1009-1047): w
 *     [C][M/group][taps]; input i contributes to o = i * str + k * dil - pad.
 * Integer kinds subtract x_zp and w_zp[m] (w_zp NULL = 0).  acc receives the
 * exact products summed in double [N][M][out]. */
int orc_conv(const void *x, int x_kind, const void *w, int w_kind, int64_t n, int64_t c,
             int64_t m, int64_t group, const int64_t *in, const int64_t *ker,
             const int64_t *out, const int64_t *str, const int64_t *dil,
             const int64_t *pad, int trans, int32_t x_zp, const int32_t *w_zp,
             double *acc);

/* Float binary ops with broadcasting: _broadcastShape (lib/src/onnx_ops.dart:
 * 26-44) and _elementwiseBinary / _arithFloatFast (:103-330): each output
 * element is op(a, b) of the broadcast operands computed in double and
 * stored to f32.  op: 0 add, 1 sub, 2 mul, 3 div.  Shapes are right-aligned;
 * y holds the broadcast shape (out_shape receives it, rank max(ra, rb)). */
int orc_binary_f32(int op, const float *a, const int64_t *a_shape, int a_rank, const float *b,
                   const int64_t *b_shape, int b_rank, float *y, int64_t *out_shape);

/* opSigmoid, lib/src/onnx_ops.dart:2349-2350: 1 / (1 + exp(-x)) in double. */
void orc_sigmoid_f32(const float *x, int64_t n, float *y);

/* opRMSNorm, lib/src/onnx_ops.dart:1771-1815: per slice along axis, ss =
 * sum of v*v in double (in order), inv = 1 / sqrt(ss / dim + eps), out =
 * x * inv * gamma[i % last_dim] (double, one rounding to f32).  gamma has
 * the last dim's length. */
int orc_rms_norm_f32(const float *x, const int64_t *shape, int rank, const float *gamma,
                     int64_t gamma_len, int64_t axis, double eps, float *y);

/* _roundEven, lib/src/onnx_qlinear_ops.dart:19-26 / onnx_ops.dart:3480-3487.
 * Returns ORC_UNSUPPORTED through *err for non-finite input (Dart's toInt
 * throws UnsupportedError there). */
int64_t orc_round_even(double v, int *err);

#ifdef __cplusplus
}
#endif
#endif
