/* migemm — MI355X (gfx950) matrix-multiply operators for onnx_runtime_dart.
 *
 * C ABI of libmigemm.so.  Every entry point takes plain pointers and sizes,
 * returns an mg_status, and leaves a human-readable message for the calling
 * thread in mg_last_error() when it fails.  The Dart graph interpreter binds
 * these through dart:ffi and keeps its own op functions' signatures; the
 * citation on each declaration names the reference routine it replaces
 * (paths are relative to the onnx_runtime_dart checkout).
 *
 * Conventions
 *   - Host-pointer ops (no _dev suffix) are synchronous: inputs are borrowed
 *     for the call, outputs are written into caller-allocated host memory
 *     before the call returns (the reference's ops return fresh tensors
 *     synchronously, lib/src/onnx_qlinear_ops.dart:174).
 *   - _dev ops take device pointers (from mg_buffer_alloc or any HIP
 *     allocation on the context's device) and are asynchronous on the
 *     context's stream; mg_ctx_synchronize waits for them.
 *   - Weights are uploaded once into an mg_weight handle (repacked for the
 *     kernels on upload, resident in HBM until mg_weight_release); the caller
 *     may drop its host copy after create returns.  This is the device form of
 *     the graph's lazily built prepacked Gemm weight
 *     (lib/src/onnx_graph.dart:102-105, :2159-2161).
 *   - One mg_ctx per isolate / thread.  Calls on one context are serialised
 *     by the caller; contexts share nothing but the device.
 *   - Integer outputs are int32 (ONNX's MatMulInteger type); the Dart shim
 *     widens them to Tensor.int64 (lib/src/onnx_qlinear_ops.dart:77-80).
 */
#ifndef MIGEMM_H
#define MIGEMM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes; the Dart shim maps them to the exceptions the reference
 * throws (lib/src/onnx_qlinear_ops.dart:39-40,127,135,152,162,165;
 * lib/src/execution_control.dart:43-57; lib/src/onnx_graph.dart:1274-1281). */
typedef enum mg_status {
  MG_OK = 0,
  MG_INVALID_ARGUMENT = 1, /* ArgumentError */
  MG_UNSUPPORTED = 2,      /* UnsupportedError */
  MG_OUT_OF_MEMORY = 3,    /* OnnxMemoryLimitException (budget) or HBM OOM */
  MG_CANCELLED = 4,        /* OnnxCancelledException */
  MG_DEVICE_ERROR = 5      /* StateError: HIP runtime failure */
} mg_status;

typedef struct mg_ctx mg_ctx;
typedef struct mg_weight mg_weight;

/* Message of the last failing call on this thread ("" if none).  The pointer
 * stays valid until the next migemm call on the same thread.  Plays the role
 * of the ORT status message (lib/src/ort/ort_backend.dart:774-782). */
const char *mg_last_error(void);

/* When the last failing call on this thread failed on the byte budget of
 * mg_ctx_set_control, returns 1 and stores the bytes the op needed and the
 * limit: the fields of OnnxMemoryLimitException
 * (lib/src/execution_control.dart:12-19).  Returns 0 otherwise (an
 * MG_OUT_OF_MEMORY from the device allocator maps to StateError).  Either
 * pointer may be NULL. */
int32_t mg_last_error_budget(int64_t *required_bytes, int64_t *limit_bytes);

/* Library version as "major.minor.patch". */
const char *mg_version(void);

/* ----------------------------------------------------------------- context */

/* Creates a context on HIP device `device` with its own stream.
 * Replaces the process-wide kernel state of lib/src/gemm_kernel_simd.dart:26-28
 * (isolate-local scratch) with a per-caller device context. */
mg_status mg_ctx_create(int32_t device, mg_ctx **out);
mg_status mg_ctx_destroy(mg_ctx *ctx);

/* Uses `hip_stream` (a hipStream_t, may be NULL for the null stream) for all
 * later work of the context instead of its own stream.  The caller keeps
 * ownership of the stream. */
mg_status mg_ctx_set_stream(mg_ctx *ctx, void *hip_stream);
/* The hipStream_t the context launches on. */
mg_status mg_ctx_get_stream(mg_ctx *ctx, void **hip_stream);
mg_status mg_ctx_synchronize(mg_ctx *ctx);

/* Per-op device timing, the ABI's part of ExecutionProfile
 * (lib/src/onnx_graph.dart:27-86: per-node times by op type).  While enabled,
 * every op entry point records HIP events on the context's stream around its
 * work, in issue order; mg_ctx_profile_get waits for record i and returns its
 * op type ("MatMulNBits", "Gemm", ..., "<op>.upload" for weight creation) and
 * device milliseconds (host-pointer ops include their transfers).  Enabling or
 * clearing discards the records (after waiting for the stream). */
mg_status mg_ctx_set_profiling(mg_ctx *ctx, int32_t enable);
mg_status mg_ctx_profile_count(mg_ctx *ctx, int64_t *n);
mg_status mg_ctx_profile_get(mg_ctx *ctx, int64_t i, const char **op, float *ms);
mg_status mg_ctx_profile_clear(mg_ctx *ctx);

/* Whether MatMulNBits weights created on this context from now on also keep
 * prefill images (default: enabled).  An image holds the weight's integers
 * (q - zp) / 2 (q / 2 with float zero points) as fp6 e2m3 MFMA operands, 3/4
 * byte per weight on top of the packed half byte, built on the device at
 * upload; prefill calls (M > 16, or M > 4 with float zero points) on weights
 * with images run the fp6 GEMM, those without run the fp8 GEMM that
 * dequantises each tile (or, for float zero points, the fp32 path).  Both
 * meet the MatMulNBits tolerance; their results differ in rounding.  Only
 * block sizes >= 128 have images.  No counterpart in the reference, which
 * dequantises the weight to fp32 on every call
 * (lib/src/onnx_qlinear_ops.dart:208-226); for callers that run only decode
 * rows and want the smaller footprint. */
mg_status mg_ctx_set_prefill_images(mg_ctx *ctx, int32_t enable);

/* Cooperative cancellation and byte budget, checked before every launch
 * (lib/src/execution_control.dart:43-57: checkpoint / checkAdditionalBytes).
 * `cancel_flag` (may be NULL) is polled: non-zero => MG_CANCELLED.
 * `max_bytes` < 0 disables the budget; otherwise an op whose device
 * workspace plus staging would exceed it fails with MG_OUT_OF_MEMORY. */
mg_status mg_ctx_set_control(mg_ctx *ctx, const volatile int32_t *cancel_flag,
                             int64_t max_bytes);

/* ----------------------------------------------------------- device memory */

mg_status mg_buffer_alloc(mg_ctx *ctx, size_t bytes, void **dev_ptr);
mg_status mg_buffer_free(mg_ctx *ctx, void *dev_ptr);
mg_status mg_buffer_upload(mg_ctx *ctx, void *dev_dst, const void *host_src,
                           size_t bytes);
mg_status mg_buffer_download(mg_ctx *ctx, void *host_dst, const void *dev_src,
                             size_t bytes);

/* ------------------------------------------------------------- MatMulNBits */

/* Zero-point forms of MatMulNBits (lib/src/onnx_qlinear_ops.dart:178-188). */
typedef enum mg_zp_kind {
  MG_ZP_NONE = 0,   /* default zero point 8 */
  MG_ZP_UINT4 = 1,  /* packed uint8, [N * ceil(nb/2)] or [N, ceil(nb/2)] */
  MG_ZP_FLOAT = 2   /* float32, [N * nb] or [N, nb] */
} mg_zp_kind;

/* Uploads an int4 block-quantized weight: validation of
 * opMatMulNBits (lib/src/onnx_qlinear_ops.dart:126-166) plus the dispatch's
 * g_idx rejection (lib/src/onnx_graph.dart:2919-2921, pass has_g_idx).
 *   b      uint8 [N, nb, block_size/2], low nibble = even k  (b_shape, rank 3)
 *   scales float32 [N*nb] or [N, nb]                          (scales_shape)
 *   zp     per zp_kind, NULL for MG_ZP_NONE                   (zp_shape)
 *   bias   float32 [N] or NULL                                (bias_shape)
 * nb = ceil(K / block_size). */
mg_status mg_weight_nbits_create(
    mg_ctx *ctx, int64_t K, int64_t N, int64_t bits, int64_t block_size,
    const uint8_t *b, const int64_t *b_shape, int32_t b_rank,
    const float *scales, const int64_t *scales_shape, int32_t scales_rank,
    int32_t zp_kind, const void *zp, const int64_t *zp_shape, int32_t zp_rank,
    const float *bias, const int64_t *bias_shape, int32_t bias_rank,
    int32_t has_g_idx, mg_weight **out);

/* Where one weight tensor's bytes are: host memory (host != NULL), or the
 * byte range [offset, offset + length) of the file at path, which is how an
 * ONNX initializer with external data is stored (location / offset / length
 * entries, lib/src/onnx_proto_loader.dart:96-125).  length 0 means "implied
 * by the shape", as the reference's resolver falls back to. */
typedef struct mg_tensor_source {
  const void *host;
  const char *path;
  int64_t offset;
  int64_t length;
} mg_tensor_source;

/* The load path for big int4 models (lib/src/onnx_proto_loader.dart:96-125,
 * :252-266; lib/src/model_source.dart:58): uploads a MatMulNBits weight with
 * b / scales / zp taken from their sources in the raw ONNX layouts of
 * mg_weight_nbits_create (B [N, nb, bs/2] bytes, scales f32 [N * nb], zero
 * points packed [N * ceil(nb/2)] or f32 [N * nb]).  The bytes stream through
 * pinned staging in column-group chunks of about chunk_bytes (0 = 32 MiB)
 * and are repacked on the GPU, so no host copy of the whole tensor is made.
 * bias: host float [N] or NULL.  Same validation and results as
 * mg_weight_nbits_create. */
mg_status mg_weight_nbits_create_streamed(
    mg_ctx *ctx, int64_t K, int64_t N, int64_t bits, int64_t block_size,
    const mg_tensor_source *b, const mg_tensor_source *scales, int32_t zp_kind,
    const mg_tensor_source *zp, const float *bias, int32_t has_g_idx,
    int64_t chunk_bytes, mg_weight **out);

/* y[M, N] = a[M, K] . dequant(B)^T (+ bias): opMatMulNBits
 * (lib/src/onnx_qlinear_ops.dart:115-228).  `a` holds M rows of K floats
 * (the caller flattens leading dims, a.shape.last == K); y holds M*N floats.
 * M == 0 is a no-op, as in the reference (:169-171). */
mg_status mg_matmul_nbits(mg_ctx *ctx, const mg_weight *w, const float *a,
                          int64_t M, float *y);
mg_status mg_matmul_nbits_dev(mg_ctx *ctx, const mg_weight *w,
                              const float *a_dev, int64_t M, float *y_dev);

/* mg_matmul_nbits_dev without any allocation.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * Results are those of mg_matmul_nbits_dev.  The kernels' workspace
 * (activation prepasses, split-K partial sums) is a static per-device scratch
 * array of MG_NOALLOC_SCRATCH_BYTES bytes, held by each GPU the library runs
 * on until the process ends; a call that would need more fails with
 * MG_INVALID_ARGUMENT before launching anything.  Every call on one GPU uses
 * that GPU's array: calls that overlap on one GPU (several contexts or
 * streams in flight at once) race. */
#define MG_NOALLOC_SCRATCH_BYTES (32u << 20)
mg_status mg_matmul_nbits_dev_noalloc(mg_ctx *ctx, const mg_weight *w,
                                      const float *a_dev, int64_t M,
                                      float *y_dev);

/* Several MatMulNBits nodes that read the same activations (a decoder layer's
 * q/k/v or gate/up projections): y_dev[i] = opMatMulNBits(a, W_i) for
 * 1 <= n <= 4 weights sharing K, block_size, zero-point form and device, each
 * result identical to a separate mg_matmul_nbits_dev call
 * (lib/src/onnx_qlinear_ops.dart:115-228).  Decode shapes (M <= 16) run as
 * one launch over all the weights' columns, which halves or thirds the
 * per-token launch count of a layer. */
mg_status mg_matmul_nbits_group_dev(mg_ctx *ctx, int32_t n,
                                    const mg_weight *const *w,
                                    const float *a_dev, int64_t M,
                                    float *const *y_dev);
/* Split activations for the decode GEMV (3 to 16 rows, integer zero
 * points, block_size >= 32).  That GEMV takes each activation as an fp16
 * hi/lo pair with a power-of-two row exponent; without help it converts its
 * fp32 input in a prepass launch of its own.  The norm producer
 * (mg_skip_rms_norm_f32_split_dev) also writes that split of the rows it
 * computes into a device buffer of
 * mg_nbits_split_bytes bytes, and this entry reads it instead of running the
 * prepass: the results are bitwise those of mg_matmul_nbits_group_dev on
 * a_dev.  a_dev is still required (plans other than the 3..16-row GEMV read
 * it); split_dev may be NULL.  The split must come from a_dev's producer for
 * the weights' K and block size.  No counterpart in the reference, whose ops
 * exchange fp32 tensors only (lib/src/onnx_graph.dart:1227-1309); it saves
 * one launch per decode GEMV whose input comes from a norm (q/k/v and
 * gate/up of a decoder layer). */
mg_status mg_matmul_nbits_group_split_dev(mg_ctx *ctx, int32_t n,
                                          const mg_weight *const *w,
                                          const float *a_dev,
                                          const void *split_dev, int64_t M,
                                          float *const *y_dev);
/* Bytes of a split activation buffer for rows of K elements read by
 * MatMulNBits weights of this block_size. */
mg_status mg_nbits_split_bytes(int64_t K, int64_t block_size, size_t *bytes);

/* ------------------------------------------- MatMulInteger / QLinearMatMul */

/* Uploads an 8-bit B [K, N] (`b_signed`: int8 else uint8) with its zero
 * point (scalar when b_zp_len == 1, per-column [N], or none when NULL);
 * column sums are computed once here.  Mirrors the operand checks of
 * opMatMulInteger (lib/src/onnx_qlinear_ops.dart:36-45). */
mg_status mg_weight_int8_create(mg_ctx *ctx, const void *b, int32_t b_signed,
                                int64_t K, int64_t N, const int32_t *b_zp,
                                int64_t b_zp_len, mg_weight **out);

/* y_int32[batch, M, N] = (A - aZp) . (B - bZp): opMatMulInteger
 * (lib/src/onnx_qlinear_ops.dart:32-81).  A and B are given with their full
 * shapes (rank >= 2); batches must be equal or 1 (:46-54).  Zero points are
 * int32 arrays: scalar (len 1), per-row A [M], per-column B [N], or NULL. */
mg_status mg_matmul_integer(mg_ctx *ctx, const void *a, int32_t a_signed,
                            const int64_t *a_shape, int32_t a_rank,
                            const void *b, int32_t b_signed,
                            const int64_t *b_shape, int32_t b_rank,
                            const int32_t *a_zp, int64_t a_zp_len,
                            const int32_t *b_zp, int64_t b_zp_len, int32_t *y);
/* opMatMulInteger with the reference's own output type: y_int64[batch, M,
 * N], Tensor.int64 accumulated in 64-bit ints (lib/src/onnx_qlinear_ops.dart:
 * 55-80), for any K.  mg_matmul_integer's int32 output is exact only for
 * K <= 33025 (a k term is at most 255 * 255) and refuses longer rows with
 * MG_UNSUPPORTED; this form cuts K into segments of 32768 whose int32 sums
 * are exact and adds them in int64 on the device. */
mg_status mg_matmul_integer_i64(mg_ctx *ctx, const void *a, int32_t a_signed,
                                const int64_t *a_shape, int32_t a_rank,
                                const void *b, int32_t b_signed,
                                const int64_t *b_shape, int32_t b_rank,
                                const int32_t *a_zp, int64_t a_zp_len,
                                const int32_t *b_zp, int64_t b_zp_len, int64_t *y);
/* Same with an uploaded B; a is [rows = batch*M, K].  The uploaded-weight
 * forms (here and below) need K <= 33025 (MG_UNSUPPORTED otherwise). */
mg_status mg_matmul_integer_w(mg_ctx *ctx, const void *a, int32_t a_signed,
                              int64_t rows, int64_t K, const int32_t *a_zp,
                              int64_t a_zp_len, const mg_weight *w, int32_t *y);
mg_status mg_matmul_integer_w_dev(mg_ctx *ctx, const void *a_dev,
                                  int32_t a_signed, int64_t rows, int64_t K,
                                  const int32_t *a_zp, int64_t a_zp_len,
                                  const mg_weight *w, int32_t *y_dev);

/* QLinearMatMul (lib/src/onnx_qlinear_ops.dart:85-108): MatMulInteger, then
 * q = roundHalfEven(fl32(acc * fl32(fl32(aS*bS)/yS))) + yZp clamped to
 * [lo, hi].  lo/hi are -128/127 when the y zero point is int8, else 0/255
 * (lib/src/onnx_graph.dart:2903,2914-2915); y holds uint8 when lo >= 0 and
 * int8 otherwise.  Scales are per-tensor (:88-90).  Any K: rows longer than
 * 33025 are summed in int64 (as the reference's int accumulator) before the
 * requantisation. */
mg_status mg_qlinear_matmul(mg_ctx *ctx, const void *a, int32_t a_signed,
                            const int64_t *a_shape, int32_t a_rank,
                            float a_scale, const int32_t *a_zp,
                            int64_t a_zp_len, const void *b, int32_t b_signed,
                            const int64_t *b_shape, int32_t b_rank,
                            float b_scale, const int32_t *b_zp,
                            int64_t b_zp_len, float y_scale, int32_t y_zp,
                            int32_t lo, int32_t hi, void *y);
mg_status mg_qlinear_matmul_w(mg_ctx *ctx, const void *a, int32_t a_signed,
                              int64_t rows, int64_t K, float a_scale,
                              const int32_t *a_zp, int64_t a_zp_len,
                              const mg_weight *w, float b_scale, float y_scale,
                              int32_t y_zp, int32_t lo, int32_t hi, void *y);
mg_status mg_qlinear_matmul_w_dev(mg_ctx *ctx, const void *a_dev,
                                  int32_t a_signed, int64_t rows, int64_t K,
                                  float a_scale, const int32_t *a_zp,
                                  int64_t a_zp_len, const mg_weight *w,
                                  float b_scale, float y_scale, int32_t y_zp,
                                  int32_t lo, int32_t hi, void *y_dev);

/* DynamicQuantizeLinear (lib/src/onnx_ops.dart:3556-3583): y uint8[n],
 * scale and zero point as the reference computes them (f64 arithmetic,
 * rounded to f32; round-half-even).  Non-finite input => MG_UNSUPPORTED
 * (the reference's toInt on NaN throws UnsupportedError). */
mg_status mg_dynamic_quantize_linear(mg_ctx *ctx, const float *x, int64_t n,
                                     uint8_t *y, float *scale, int32_t *zp);
/* Device form: scale/zp are written to device memory, so a following integer
 * matmul can stay on device.  scale_zp_dev receives 12 bytes: the float
 * scale, the int32 zero point, then an int32 that is 1 when the input held
 * Infinity or NaN (where the host form fails with MG_UNSUPPORTED; y, scale
 * and zp are then unspecified) and 0 otherwise. */
mg_status mg_dynamic_quantize_linear_dev(mg_ctx *ctx, const float *x_dev,
                                         int64_t n, uint8_t *y_dev,
                                         void *scale_zp_dev);

/* DynamicQuantizeLinear -> MatMulInteger / QLinearMatMul with the quantized
 * activation consumed where DQL left it: a_dev is DQL's uint8 [rows, K] and
 * a_scale_zp_dev its scale/zp words, read on the device, so the chain needs
 * no host synchronisation.  This is the dynamic-quantisation subgraph as the
 * graph runs it (lib/src/onnx_graph.dart:2878-2917: DQL's y_scale and
 * y_zero_point outputs feed QLinearMatMul's a_scale / a_zero_point inputs,
 * or MatMulInteger's a_zero_point); results equal mg_matmul_integer_w_dev /
 * mg_qlinear_matmul_w_dev called with the same scale and zero point. */
mg_status mg_matmul_integer_w_dq_dev(mg_ctx *ctx, const uint8_t *a_dev,
                                     int64_t rows, int64_t K,
                                     const void *a_scale_zp_dev,
                                     const mg_weight *w, int32_t *y_dev);
mg_status mg_qlinear_matmul_w_dq_dev(mg_ctx *ctx, const uint8_t *a_dev,
                                     int64_t rows, int64_t K,
                                     const void *a_scale_zp_dev,
                                     const mg_weight *w, float b_scale,
                                     float y_scale, int32_t y_zp, int32_t lo,
                                     int32_t hi, void *y_dev);

/* ---------------------------------------------------------- fp32 MatMul/Gemm */

/* numpy-broadcast batched MatMul (lib/src/onnx_ops.dart:1710-1766);
 * y has the broadcast shape [..., M, N]. */
mg_status mg_matmul_f32(mg_ctx *ctx, const float *a, const int64_t *a_shape,
                        int32_t a_rank, const float *b, const int64_t *b_shape,
                        int32_t b_rank, float *y);
mg_status mg_matmul_f32_dev(mg_ctx *ctx, const float *a_dev,
                            const int64_t *a_shape, int32_t a_rank,
                            const float *b_dev, const int64_t *b_shape,
                            int32_t b_rank, float *y_dev);
/* opMatMul on operands that are not both float tensors (integer tensors,
 * or one float and one integer): the reference's fallback
 * (lib/src/onnx_ops.dart:1753-1762) sums a.getD * b.getD over k in order
 * in double and stores f32.  The operands are passed as doubles (each
 * element's getD value); products and sums are rounded separately, so y is
 * bitwise the reference's.  Shapes and broadcasting as mg_matmul_f32. */
mg_status mg_matmul_f64acc(mg_ctx *ctx, const double *a, const int64_t *a_shape,
                           int32_t a_rank, const double *b,
                           const int64_t *b_shape, int32_t b_rank, float *y);
/* Output shape of MatMul over these operand shapes (the broadcast of
 * lib/src/onnx_ops.dart:1717-1722 plus [M, N]); y_shape holds up to 16
 * entries.  Lets the caller allocate y before mg_matmul_f32(_dev).  No
 * device is touched. */
mg_status mg_matmul_f32_output_shape(const int64_t *a_shape, int32_t a_rank,
                                     const int64_t *b_shape, int32_t b_rank,
                                     int64_t *y_shape, int32_t *y_rank);
/* Element offsets into A and B of kernel batches [first, first + count) as
 * the kernels compute them (the per-batch broadcast offsets of
 * lib/src/onnx_ops.dart:1742-1764); *batches (if not NULL) receives the
 * number of kernel batches.  Host-only; for checking the batch planner
 * without a device.  With the shared-weight collapse
 * (lib/src/onnx_ops.dart:1728-1735) there is one batch at offsets 0. */
mg_status mg_matmul_f32_batch_offsets(const int64_t *a_shape, int32_t a_rank,
                                      const int64_t *b_shape, int32_t b_rank,
                                      int64_t first, int64_t count,
                                      int64_t *a_off, int64_t *b_off,
                                      int64_t *batches);

/* Gemm: y = alpha * op(A) . op(B) + beta * C (lib/src/onnx_ops.dart:2152-2172).
 * a, b rank 2; c NULL or rank <= 2 broadcasting to [M, N]. */
mg_status mg_gemm_f32(mg_ctx *ctx, const float *a, const int64_t *a_shape,
                      const float *b, const int64_t *b_shape, int32_t trans_a,
                      int32_t trans_b, float alpha, float beta, const float *c,
                      const int64_t *c_shape, int32_t c_rank, float *y);

/* Uploads an fp32 B given as stored ([rows, cols]); with trans_b the operand
 * is B^T, i.e. K = cols, N = rows (the transB prepack of
 * lib/src/onnx_graph.dart:2159-2161 done once on upload). */
mg_status mg_weight_f32_create(mg_ctx *ctx, const float *b, int64_t rows,
                               int64_t cols, int32_t trans_b, mg_weight **out);
/* y[rows, N] = alpha * a[rows, K] . W + beta * C, C as in mg_gemm_f32 (may be
 * NULL).  With alpha = 1, beta = 0, C = NULL this is MatMul against an
 * initializer, including the shared-weight batch collapse
 * (lib/src/onnx_ops.dart:1728-1735).  With K >= 1024 and rows <= 8192 the
 * product is split over K: the call then takes up to 64 MiB of the
 * context's workspace for the partial sums (wider weights run in column
 * chunks; counted against the byte budget), also with device pointers. */
mg_status mg_gemm_f32_w(mg_ctx *ctx, const float *a, int64_t rows, int64_t K,
                        const mg_weight *w, float alpha, float beta,
                        const float *c, const int64_t *c_shape, int32_t c_rank,
                        float *y);
mg_status mg_gemm_f32_w_dev(mg_ctx *ctx, const float *a_dev, int64_t rows,
                            int64_t K, const mg_weight *w, float alpha,
                            float beta, const float *c_dev,
                            const int64_t *c_shape, int32_t c_rank,
                            float *y_dev);

/* --------------------------------------------------------------- attention */

/* _FusedSDPA (lib/src/onnx_ops.dart:2100-2149, the graph fusion of
 * MatMul(Softmax(MatMul(A, B) * scale + mask), V) at
 * lib/src/onnx_graph.dart:560-620, dispatched at :1812-1821):
 * y = MatMul(softmax_row(MatMul(a, b) * scale + mask), v) in fp32.  a is
 * [..., S, D], b [..., D, T] (K^T), v [..., T, DV]; batch dims broadcast as
 * in MatMul (a with b, then the scores with v); the mask (any rank up to the
 * score rank) broadcasts right-aligned into the scores [..., S, T].  y is the
 * broadcast [..., S, DV].  A row whose scores are all -inf is NaN, as in the
 * reference.  D and DV <= 128; at most 4 batch dims (else MG_UNSUPPORTED). */
mg_status mg_fused_sdpa(mg_ctx *ctx, const float *a, const int64_t *a_shape,
                        int32_t a_rank, const float *b, const int64_t *b_shape,
                        int32_t b_rank, const float *v, const int64_t *v_shape,
                        int32_t v_rank, const float *mask,
                        const int64_t *mask_shape, int32_t mask_rank,
                        float scale, float *y);
mg_status mg_fused_sdpa_dev(mg_ctx *ctx, const float *a_dev,
                            const int64_t *a_shape, int32_t a_rank,
                            const float *b_dev, const int64_t *b_shape,
                            int32_t b_rank, const float *v_dev,
                            const int64_t *v_shape, int32_t v_rank,
                            const float *mask_dev, const int64_t *mask_shape,
                            int32_t mask_rank, float scale, float *y_dev);

/* MultiHeadAttention (com.microsoft; lib/src/onnx_ops.dart:2014-2098,
 * dispatched at lib/src/onnx_graph.dart:1670-1680): q [batch, seq, hidden],
 * k and v [batch, kv_seq, hidden], num_heads heads of hidden / num_heads;
 * bias (optional) [batch, bias_heads, seq, kv_seq] with bias_heads 1 or
 * num_heads, added to the scaled scores; scale = 1 / sqrt(head size) unless
 * has_scale.  y [batch, seq, hidden]. */
mg_status mg_multi_head_attention(mg_ctx *ctx, const float *q, const float *k,
                                  const float *v, int64_t batch, int64_t seq,
                                  int64_t kv_seq, int64_t hidden,
                                  int32_t num_heads, const float *bias,
                                  int32_t bias_heads, int32_t has_scale,
                                  float scale, float *y);
mg_status mg_multi_head_attention_dev(mg_ctx *ctx, const float *q_dev,
                                      const float *k_dev, const float *v_dev,
                                      int64_t batch, int64_t seq,
                                      int64_t kv_seq, int64_t hidden,
                                      int32_t num_heads, const float *bias_dev,
                                      int32_t bias_heads, int32_t has_scale,
                                      float scale, float *y_dev);

/* GroupQueryAttention (com.microsoft; lib/src/onnx_ops.dart:1829-2012,
 * dispatched at lib/src/onnx_graph.dart:1649-1668): q [batch, seq, hidden]
 * with num_heads heads of hidden / num_heads; k and v [batch, seq,
 * kv_num_heads * head_size]; query head h uses KV head
 * h / (num_heads / kv_num_heads).  past_key / past_value NULL (past_len 0)
 * or [batch, kv_num_heads, past_len, head_size].  With do_rotary, RoPE at
 * positions past_len + s from cos_cache / sin_cache [max_pos, half_rot]
 * (GPT-J pairs when rotary_interleaved) is applied to q and k.  Query s sees
 * keys 0 .. past_len + s (causal), plus attention_bias [batch, bias_heads,
 * seq, past_len + seq] (bias_heads 1 or num_heads) if given.  scale defaults
 * to 1 / sqrt(head_size).  softcap != 0 or local_window > 0 is
 * MG_UNSUPPORTED, as in the reference.  Outputs: y [batch, seq, hidden] and
 * present_key / present_value [batch, kv_num_heads, past_len + seq,
 * head_size] (the past followed by the rotated K / raw V).  Head size <= 128. */
mg_status mg_group_query_attention(
    mg_ctx *ctx, const float *q, const float *k, const float *v, int64_t batch,
    int64_t seq, int64_t hidden, int32_t num_heads, int32_t kv_num_heads,
    const float *past_key, const float *past_value, int64_t past_len,
    const float *cos_cache, const float *sin_cache, int64_t max_pos,
    int64_t half_rot, int32_t do_rotary, int32_t rotary_interleaved,
    const float *attention_bias, int32_t bias_heads, int32_t has_scale,
    float scale, float softcap, int32_t local_window, float *y,
    float *present_key, float *present_value);
mg_status mg_group_query_attention_dev(
    mg_ctx *ctx, const float *q_dev, const float *k_dev, const float *v_dev,
    int64_t batch, int64_t seq, int64_t hidden, int32_t num_heads,
    int32_t kv_num_heads, const float *past_key_dev,
    const float *past_value_dev, int64_t past_len, const float *cos_cache_dev,
    const float *sin_cache_dev, int64_t max_pos, int64_t half_rot,
    int32_t do_rotary, int32_t rotary_interleaved,
    const float *attention_bias_dev, int32_t bias_heads, int32_t has_scale,
    float scale, float softcap, int32_t local_window, float *y_dev,
    float *present_key_dev, float *present_value_dev);

/* ---------------------------------------------------------- convolution */

/* Conv (lib/src/onnx_nn_ops.dart:179-817, dispatched at
 * lib/src/onnx_graph.dart:2436-2490): x [N, C, spatial...] with 1 to 3
 * spatial dims, w [M, C / group, kernel...], bias NULL or [M].  strides and
 * dilations NULL (all 1) or [nd]; pads NULL (all 0) or [2 nd] (all begins,
 * then all ends); auto_pad 0 NOTSET, 1 SAME_UPPER, 2 SAME_LOWER, 3 VALID,
 * resolved as the reference's _resolvePads (lib/src/onnx_nn_ops.dart:38-87).
 * y [N, M, out...] from mg_conv_output_shape (x_rank values). */
mg_status mg_conv_output_shape(const int64_t *x_shape, int32_t x_rank,
                               const int64_t *w_shape, const int64_t *strides,
                               const int64_t *pads, const int64_t *dilations,
                               int32_t group, int32_t auto_pad,
                               int64_t *y_shape);
mg_status mg_conv_f32(mg_ctx *ctx, const float *x, const int64_t *x_shape,
                      int32_t x_rank, const float *w, const int64_t *w_shape,
                      const float *bias, const int64_t *strides,
                      const int64_t *pads, const int64_t *dilations,
                      int32_t group, int32_t auto_pad, float *y);
mg_status mg_conv_f32_dev(mg_ctx *ctx, const float *x_dev,
                          const int64_t *x_shape, int32_t x_rank,
                          const float *w_dev, const int64_t *w_shape,
                          const float *bias_dev, const int64_t *strides,
                          const int64_t *pads, const int64_t *dilations,
                          int32_t group, int32_t auto_pad, float *y_dev);

/* ConvTranspose (lib/src/onnx_nn_ops.dart:818-1059, dispatched at
 * lib/src/onnx_graph.dart:2491-2513; auto_pad is not read there):
 * w [C, M / group, kernel...]; output_padding NULL or [nd]; output_shape
 * NULL or at least nd entries (its last nd are the spatial dims; the pads are
 * then derived, the larger half at the beginning). */
mg_status mg_conv_transpose_output_shape(
    const int64_t *x_shape, int32_t x_rank, const int64_t *w_shape,
    const int64_t *strides, const int64_t *pads, const int64_t *dilations,
    const int64_t *output_padding, const int64_t *output_shape,
    int32_t output_shape_len, int32_t group, int64_t *y_shape);
mg_status mg_conv_transpose_f32(mg_ctx *ctx, const float *x,
                                const int64_t *x_shape, int32_t x_rank,
                                const float *w, const int64_t *w_shape,
                                const float *bias, const int64_t *strides,
                                const int64_t *pads, const int64_t *dilations,
                                const int64_t *output_padding,
                                const int64_t *output_shape,
                                int32_t output_shape_len, int32_t group,
                                float *y);
mg_status mg_conv_transpose_f32_dev(
    mg_ctx *ctx, const float *x_dev, const int64_t *x_shape, int32_t x_rank,
    const float *w_dev, const int64_t *w_shape, const float *bias_dev,
    const int64_t *strides, const int64_t *pads, const int64_t *dilations,
    const int64_t *output_padding, const int64_t *output_shape,
    int32_t output_shape_len, int32_t group, float *y_dev);

/* ConvInteger (lib/src/onnx_qlinear_ops.dart:232-337, dispatched at
 * lib/src/onnx_graph.dart:2889-2901): y = sum (x - x_zp)(w - w_zp[m]) as
 * exact int32 (the shim widens to Tensor.int64); x and w are bytes, uint8
 * or int8 per *_signed; w_zp NULL, scalar (len 1) or per output channel
 * (len M), else MG_UNSUPPORTED.  Geometry as mg_conv_f32 with auto_pad
 * NOTSET.  The _dev form takes device x / w / y; w_zp stays a host array. */
mg_status mg_conv_integer(mg_ctx *ctx, const void *x, int32_t x_signed,
                          const int64_t *x_shape, int32_t x_rank,
                          const void *w, int32_t w_signed,
                          const int64_t *w_shape, int32_t x_zp,
                          const int32_t *w_zp, int64_t w_zp_len,
                          const int64_t *strides, const int64_t *pads,
                          const int64_t *dilations, int32_t group,
                          int32_t *y);
mg_status mg_conv_integer_dev(mg_ctx *ctx, const void *x_dev,
                              int32_t x_signed, const int64_t *x_shape,
                              int32_t x_rank, const void *w_dev,
                              int32_t w_signed, const int64_t *w_shape,
                              int32_t x_zp, const int32_t *w_zp,
                              int64_t w_zp_len, const int64_t *strides,
                              const int64_t *pads, const int64_t *dilations,
                              int32_t group, int32_t *y_dev);

/* QLinearConv (lib/src/onnx_qlinear_ops.dart:339-382, dispatched at
 * lib/src/onnx_graph.dart:2935-2955): q = roundHalfEven((acc + bias[m]) *
 * x_scale * w_scale[m] / y_scale, in double) + y_zp clamped to [lo, hi]
 * ([-128, 127] when the y_zp initializer is int8, else [0, 255]), stored as
 * bytes.  w_scale scalar or per output channel; bias NULL or int32 [M].  The
 * _dev form takes device x / w / bias / y; w_scale and w_zp stay host arrays. */
mg_status mg_qlinear_conv(mg_ctx *ctx, const void *x, int32_t x_signed,
                          const int64_t *x_shape, int32_t x_rank,
                          float x_scale, int32_t x_zp, const void *w,
                          int32_t w_signed, const int64_t *w_shape,
                          const float *w_scale, int64_t w_scale_len,
                          const int32_t *w_zp, int64_t w_zp_len,
                          float y_scale, int32_t y_zp, const int32_t *bias,
                          const int64_t *strides, const int64_t *pads,
                          const int64_t *dilations, int32_t group,
                          int32_t lo, int32_t hi, uint8_t *y);
mg_status mg_qlinear_conv_dev(
    mg_ctx *ctx, const void *x_dev, int32_t x_signed, const int64_t *x_shape,
    int32_t x_rank, float x_scale, int32_t x_zp, const void *w_dev,
    int32_t w_signed, const int64_t *w_shape, const float *w_scale,
    int64_t w_scale_len, const int32_t *w_zp, int64_t w_zp_len,
    float y_scale, int32_t y_zp, const int32_t *bias_dev,
    const int64_t *strides, const int64_t *pads, const int64_t *dilations,
    int32_t group, int32_t lo, int32_t hi, uint8_t *y_dev);

/* ------------------------------------------------------- elementwise ops */

/* The elementwise ops between the products of a decoder layer, on device
 * buffers (asynchronous on the context's stream), so activations stay in HBM
 * from one product to the next.  f32 in, f32 out. */
typedef enum mg_binary_op {
  MG_BIN_ADD = 0, /* opAdd, lib/src/onnx_ops.dart:402-404 */
  MG_BIN_SUB = 1, /* opSub, :444-446 */
  MG_BIN_MUL = 2, /* opMul, :447-449 */
  MG_BIN_DIV = 3  /* opDiv on floats, :476 */
} mg_binary_op;

/* y = a op b with broadcasting (_broadcastShape, lib/src/onnx_ops.dart:26-44;
 * _arithFloatFast / _elementwiseBinary, :103-330): shapes right-aligned,
 * y holds the broadcast shape (rank max(a_rank, b_rank)).  Incompatible
 * shapes: MG_INVALID_ARGUMENT "Cannot broadcast shapes [..] and [..]"
 * (ArgumentError); ranks up to 16.  y may be a_dev or b_dev when that
 * operand has the output's shape (an in-place residual add). */
mg_status mg_binary_f32_dev(mg_ctx *ctx, int32_t op, const float *a_dev,
                            const int64_t *a_shape, int32_t a_rank, const float *b_dev,
                            const int64_t *b_shape, int32_t b_rank, float *y_dev);
/* opSigmoid (lib/src/onnx_ops.dart:2349-2350): 1 / (1 + exp(-x)) in double.
 * y may be x. */
mg_status mg_sigmoid_f32_dev(mg_ctx *ctx, const float *x_dev, int64_t n, float *y_dev);
/* opRMSNorm (lib/src/onnx_ops.dart:1771-1815), the op behind _FusedRMSNorm and
 * SimplifiedLayerNormalization (lib/src/onnx_graph.dart:1640-1649,
 * :1783-1792): x * rsqrt(mean(x^2, axis) + epsilon) * gamma, gamma along the
 * last axis.  gamma_len != last dim: MG_INVALID_ARGUMENT ("RMSNorm gamma
 * length .. != last dim ..").  y may be x. */
mg_status mg_rms_norm_f32_dev(mg_ctx *ctx, const float *x_dev, const int64_t *shape,
                              int32_t rank, const float *gamma_dev, int64_t gamma_len,
                              int64_t axis, double epsilon, float *y_dev);
/* SkipSimplifiedLayerNormalization (lib/src/onnx_graph.dart:1793-1813):
 * sum = x + skip (equal shapes), y = RMSNorm(sum, gamma, last axis) (+ bias
 * when bias_dev is not null); sum_dev (may be null) receives sum.  Any of
 * x_dev, skip_dev, y_dev and sum_dev may be the same buffer (an in-place
 * residual stream: sum written over x or skip, y over either). */
mg_status mg_skip_rms_norm_f32_dev(mg_ctx *ctx, const float *x_dev, const float *skip_dev,
                                   const int64_t *shape, int32_t rank, const float *gamma_dev,
                                   int64_t gamma_len, const float *bias_dev, double epsilon,
                                   float *y_dev, float *sum_dev);
/* mg_skip_rms_norm_f32_dev (skip_dev not NULL) or mg_rms_norm_f32_dev over
 * the last axis (skip_dev NULL: sum_dev is ignored), with y and the sum
 * bitwise as there, also writing the decode GEMV's split of y into
 * split_dev (mg_nbits_split_bytes(last dim, block_size) bytes), for at most
 * 16 rows of at most 8192 elements (MG_INVALID_ARGUMENT otherwise). */
mg_status mg_skip_rms_norm_f32_split_dev(mg_ctx *ctx, const float *x_dev,
                                         const float *skip_dev, const int64_t *shape,
                                         int32_t rank, const float *gamma_dev,
                                         int64_t gamma_len, const float *bias_dev,
                                         double epsilon, float *y_dev, float *sum_dev,
                                         int64_t block_size, void *split_dev);

/* ----------------------------------------------------------------- weights */

mg_status mg_weight_release(mg_weight *w);
/* K, N of an uploaded weight, and its resident device bytes. */
mg_status mg_weight_info(const mg_weight *w, int64_t *K, int64_t *N,
                         int64_t *device_bytes);

#ifdef __cplusplus
}
#endif
#endif /* MIGEMM_H */
