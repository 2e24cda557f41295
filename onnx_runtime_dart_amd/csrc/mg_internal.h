// Internal declarations shared by the migemm C-ABI and its HIP kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstddef>
#include <cstdint>
#include <string>
#include <vector>

#include "../../include/migemm.h"

// ---------------------------------------------------------------- errors

// Records `msg` as this thread's last error and returns `st`.
mg_status mg_fail(mg_status st, const std::string &msg);

#define MG_HIP(call)                                                         \
  do {                                                                       \
    hipError_t e_ = (call);                                                  \
    if (e_ != hipSuccess)                                                    \
      return mg_fail(e_ == hipErrorOutOfMemory ? MG_OUT_OF_MEMORY            \
                                               : MG_DEVICE_ERROR,            \
                     std::string(#call) + ": " + hipGetErrorString(e_));     \
  } while (0)

#define MG_TRY(expr)                    \
  do {                                  \
    mg_status s_ = (expr);              \
    if (s_ != MG_OK) return s_;         \
  } while (0)

// ------------------------------------------------------------ structures

// Pinned staging of small host tables (zero points, requant multipliers)
// that _dev calls copy on the stream: MG_PIN_SLOTS slots of MG_PIN_SLOT_BYTES
// used round-robin, each reused only after the event recorded behind its
// last copy has completed.
constexpr int MG_PIN_SLOTS = 16;
constexpr size_t MG_PIN_SLOT_BYTES = 256 << 10;

// One profiled op: its name and the events recorded around its work.
struct mg_prof_rec {
  const char *op;
  hipEvent_t e0, e1;
};

struct mg_ctx {
  int device = 0;
  hipStream_t stream = nullptr;
  bool own_stream = false;
  const volatile int32_t *cancel_flag = nullptr;
  int64_t max_bytes = -1;
  // Grow-only device workspace for prepasses, partial sums and staging of
  // host-pointer calls.  Reused across calls of this context only.
  void *ws = nullptr;
  size_t ws_bytes = 0;
  // Compute units of the device (grid sizing).
  int num_cus = 256;
  void *pin = nullptr;  // MG_PIN_SLOTS * MG_PIN_SLOT_BYTES pinned host bytes
  hipEvent_t pin_ev[MG_PIN_SLOTS] = {};
  int pin_next = 0;
  // Per-op device timing (mg_ctx_set_profiling): records in issue order and
  // a pool of spare events.
  bool prof = false;
  std::vector<mg_prof_rec> prof_recs;
  std::vector<hipEvent_t> prof_pool;
  // MatMulNBits weights created afterwards keep their prefill images
  // (mg_ctx_set_prefill_images).
  bool prefill_images = true;
  // The two chunk slots of the MatMulNBits upload (pinned host and device,
  // up_slot bytes each, grow-only), held until the context is destroyed so
  // that the weights of a model pin host memory once.
  void *up_pin = nullptr;
  void *up_dev = nullptr;
  size_t up_slot = 0;
  hipEvent_t up_done[2] = {};
};

// Records events on the context's stream around one op's work when the
// context profiles (constructed at the op's entry, destroyed at its return).
class ProfScope {
 public:
  ProfScope(mg_ctx *ctx, const char *op);
  ~ProfScope();
  ProfScope(const ProfScope &) = delete;
  ProfScope &operator=(const ProfScope &) = delete;

 private:
  mg_ctx *ctx_;
  const char *op_;
  hipEvent_t e0_ = nullptr;
};
// An event from the context's pool (or a new one); null on failure.
hipEvent_t prof_event(mg_ctx *ctx);

enum mg_weight_kind { MG_W_NBITS = 1, MG_W_INT8 = 2, MG_W_F32 = 3 };

// Device form of an int4 MatMulNBits weight.  Column group = 64 columns,
// k group = 128 k.  See nbits.hip for the layouts.
struct mg_nbits_dev {
  int64_t bs = 0;     // block_size
  int64_t nb = 0;     // ceil(K / bs)
  int64_t nbh = 0;    // ceil(nb / 2) (bytes of packed zero points per column)
  int64_t kpad = 0;   // K padded to a multiple of 128 (and >= nb*bs)
  int64_t c4 = 0;     // kpad / 128
  int64_t ng = 0;     // ceil(N / 64)
  int32_t zp_kind = 0;
  uint32_t *wq = nullptr;     // [ng][c4][4 g][64 col][4 j] nibble dwords
  float *scales = nullptr;    // [ng][nb][64]
  uint8_t *zp4 = nullptr;     // [ng][nbh][64]  (MG_ZP_UINT4)
  float *zpf = nullptr;       // [ng][nb][64]   (MG_ZP_FLOAT)
  float *bias = nullptr;      // [N] or null
  // Prefill images ([2 ng][c4][3072] bytes, or null): per 32-column slab and
  // k group, the fp6 e2m3 MFMA B operands of (q - zp) / 2 (q / 2 with float
  // zero points), 3/4 byte per weight, that the fp6 prefill GEMM copies into
  // LDS (mg_nbits_f8_images).
  void *img = nullptr;
};

// Device form of an 8-bit MatMulInteger weight B [K, N].
struct mg_int8_dev {
  int32_t b_signed = 0;
  int64_t kpad = 0;        // K padded to a multiple of 256
  int64_t npad = 0;        // N padded to a multiple of 128
  int8_t *bq = nullptr;    // B - (b_signed ? 0 : 128) as int8, fragment layout
  int32_t *colsum = nullptr;  // [npad] column sums of the stored int8 B'
  int32_t *cb = nullptr;      // [npad] (b_signed ? 0 : 128) - bZp[col]
};

struct mg_f32_dev {
  float *b = nullptr;  // [N][K] row-major (B^T; transposed at upload unless transB)
};

struct mg_weight {
  mg_weight_kind kind;
  int device = 0;
  int64_t K = 0, N = 0;
  int64_t device_bytes = 0;
  mg_nbits_dev nbits;
  mg_int8_dev i8;
  mg_f32_dev f32;
};

// ------------------------------------------------------- context helpers

// Cancellation flag and byte budget check before a launch.
mg_status mg_check_control(mg_ctx *ctx, int64_t additional_bytes);
// Ensures ctx->ws holds at least `bytes` (grow-only).
mg_status mg_ws_reserve(mg_ctx *ctx, size_t bytes);
// Sets the context's device current on this thread.
mg_status mg_use_device(mg_ctx *ctx);
// Copies `bytes` of host memory to device memory on the context's stream.
// The bytes are first copied into the context's pinned staging, so the
// caller's array may go away as soon as this returns; tables larger than a
// staging slot are copied and waited for.
mg_status mg_h2d_table(mg_ctx *ctx, void *dst_dev, const void *src_host, size_t bytes);
mg_status mg_launch_check(const char *what);

static inline size_t mg_align(size_t x, size_t a = 256) {
  return (x + a - 1) / a * a;
}

// ----------------------------------------------------------- NBits entry

// Where the bytes of one weight tensor come from: host memory, or a byte
// range of a file (ONNX external data).
struct mg_byte_source {
  const uint8_t *host = nullptr;
  const char *path = nullptr;
  int64_t offset = 0;
};
// Uploads a MatMulNBits weight: the raw tensors stream through pinned
// staging in column-group chunks of about chunk_bytes (0 = default) and are
// repacked on the device.  zp unused for MG_ZP_NONE; bias host [N] or null.
mg_status mg_nbits_upload(mg_ctx *ctx, mg_weight *w, const mg_byte_source &b,
                          const mg_byte_source &scales, int32_t zp_kind,
                          const mg_byte_source &zp, const float *bias, int64_t chunk_bytes);
void mg_nbits_free(mg_weight *w);
// Whether a weight can have prefill images and run the block-scaled fp6 /
// fp8 prefill GEMMs (block_size >= 128, any zero-point form), and the build
// of its images (allocates w->nbits.img; synchronous).
bool mg_nbits_f8_eligible(const mg_nbits_dev &d);
mg_status mg_nbits_f8_images(mg_ctx *ctx, mg_weight *w);
// Workspace bytes mg_nbits_run needs for M rows.
size_t mg_nbits_ws_bytes(const mg_ctx *ctx, const mg_weight *w, int64_t M);
// a_dev [M, K] f32, y_dev [M, N] f32; ws holds mg_nbits_ws_bytes bytes.
mg_status mg_nbits_run(mg_ctx *ctx, const mg_weight *w, const float *a_dev,
                       int64_t M, float *y_dev, void *ws);
// n <= 4 weights with the same K, block size and zero-point kind applied to
// one activation a_dev: y_dev[i] = a . W_i^T.  Decode shapes run as one
// launch; ws holds mg_nbits_group_ws_bytes bytes.
size_t mg_nbits_group_ws_bytes(const mg_ctx *ctx, int n, const mg_weight *const *w,
                               int64_t M);
// split (may be null): the activations already split for the decode GEMV
// (mg_nbits_split_bytes layout, written by a producer op); when the plan is
// the 3..16-row GEMV it replaces the activation prepass.
mg_status mg_nbits_run_group(mg_ctx *ctx, int n, const mg_weight *const *w,
                             const float *a_dev, int64_t M, float *const *y_dev, void *ws,
                             const void *split = nullptr);
// K padded as a MatMulNBits weight of this block size pads it (the split
// activation buffer covers k < kpad).
inline int64_t mg_nbits_kpad(int64_t K, int64_t bs) {
  const int64_t nb = (K + bs - 1) / bs;
  return std::max<int64_t>((nb * bs + 127) / 128 * 128, 128);
}
// Bytes of a split activation buffer for rows of K (16 rows, fp16 hi and lo
// per element up to kpad, then 16 int32 row exponents).
inline size_t mg_nbits_split_size(int64_t kpad) { return mg_align((size_t)16 * kpad * 4) + 64; }

// ------------------------------------------------------------ int8 entry

mg_status mg_int8_upload(mg_ctx *ctx, mg_weight *w, const void *b,
                         int32_t b_signed, const int32_t *b_zp,
                         int64_t b_zp_len);
void mg_int8_free(mg_weight *w);
// max_ks > 0 caps the GEMM's K split (the workspace then holds fewer partials).
size_t mg_int8_ws_bytes(const mg_weight *w, int64_t rows, int max_ks = 0);
// Requant parameters for QLinearMatMul; null => plain int32 output.
// a_zp_dev, when set, is the A zero point (one int32) in device memory and
// replaces the host one; quantized_out = 0 then keeps the int32 output of
// MatMulInteger.  a_scale_dev, when set, is the A scale (one float) in device
// memory: the multiplier is then formed on the device from it, b_scale and
// y_scale instead of taken from mult.
struct mg_requant {
  float mult = 0.f;
  int32_t y_zp = 0, lo = 0, hi = 255;
  int quantized_out = 1;
  const float *a_scale_dev = nullptr;
  const int32_t *a_zp_dev = nullptr;
  float b_scale = 0.f, y_scale = 1.f;
};
inline bool mg_requant_out(const mg_requant *rq) { return rq && rq->quantized_out; }
// a_dev [rows, K] (u8 or i8), a zero point array on host (len 0, 1 or rows),
// y_dev int32 [rows, N] or (with rq) uint8/int8 [rows, N].
mg_status mg_int8_run(mg_ctx *ctx, const mg_weight *w, const void *a_dev,
                      int32_t a_signed, int64_t rows, const int32_t *a_zp,
                      int64_t a_zp_len, const mg_requant *rq, void *y_dev,
                      void *ws, int max_ks = 0);
// Device-side prepack of a runtime B [K, N] into a temporary weight whose
// arrays live in `ws_weight` (mg_int8_weight_ws_bytes bytes).
size_t mg_int8_weight_ws_bytes(int64_t K, int64_t N);
mg_status mg_int8_prepack_dev(mg_ctx *ctx, mg_weight *w, const void *b_dev,
                              int32_t b_signed, const int32_t *b_zp,
                              int64_t b_zp_len, void *ws_weight);

// Where the GEMM of mg_int8_run keeps its A operand in `ws` for `rows` rows
// (one batch): afrag [m32n][kqp][64] int4 fragments of A' = A - (a_signed ? 0
// : 128), rowsum [m32n * 32] of A' over k < K, ca [m32n * 32] = (a_signed ? 0
// : 128) - aZp, all as k_i8_prep_a writes them; total: the workspace bytes.
// small_tiles: 128-row workgroup tiles even for rows > 128 (more tiles).
struct mg_i8_a_layout {
  size_t off_a = 0, off_rs = 0, off_ca = 0, total = 0;
  int m32n = 0, kqp = 0;
};
mg_i8_a_layout mg_int8_a_layout(int64_t rows, int64_t K, int64_t N, int max_ks = 0,
                                bool small_tiles = false);
// mg_int8_run on an A operand its caller already wrote in that layout.
mg_status mg_int8_run_a_ready(mg_ctx *ctx, const mg_weight *w, int64_t rows,
                              const mg_requant *rq, void *y_dev, void *ws, int max_ks = 0,
                              bool small_tiles = false);
// The same from B given transposed, bt_dev [N, K] row-major (a convolution
// filter), without a transposed copy.
mg_status mg_int8_prepack_t_dev(mg_ctx *ctx, mg_weight *w, const void *bt_dev,
                                int32_t b_signed, const int32_t *b_zp, int64_t b_zp_len,
                                void *ws_weight);

// ------------------------------------------------------------- fp32 entry

// Broadcast batch dims of a batched product, innermost first, after size-1
// dims are dropped and dims that step both operands contiguously are merged.
// Output batch z has coordinates c[0] = z % dim[0], c[1] = (z / dim[0]) %
// dim[1], ...; operand element offsets are sum_d c[d] * a_bs[d] (b_bs[d]), a
// stride of 0 broadcasting that operand over the dim.
constexpr int MG_F32_MAX_BATCH_DIMS = 4;
struct mg_f32_bcast {
  int32_t nbd = 0;
  uint32_t dim[MG_F32_MAX_BATCH_DIMS] = {1, 1, 1, 1};
  int64_t a_bs[MG_F32_MAX_BATCH_DIMS] = {0, 0, 0, 0};
  int64_t b_bs[MG_F32_MAX_BATCH_DIMS] = {0, 0, 0, 0};
};

// Operand offsets of output batch z (host and device; fixed trip count so a
// kernel keeps the descriptor in scalar registers).
__host__ __device__ inline void mg_f32_batch_offsets(const mg_f32_bcast bc, uint32_t z,
                                                     int64_t *ao, int64_t *bo) {
  int64_t a = 0, b = 0;
#pragma unroll
  for (int d = 0; d < MG_F32_MAX_BATCH_DIMS; d++) {
    if (d < bc.nbd) {
      const uint32_t c = z % bc.dim[d];
      z /= bc.dim[d];
      a += (int64_t)c * bc.a_bs[d];
      b += (int64_t)c * bc.b_bs[d];
    }
  }
  *ao = a;
  *bo = b;
}

// y[batch][M][N] = alpha * A . B + beta * C with broadcast batch offsets.
struct mg_f32_problem {
  int64_t M, N, K;
  int64_t batch;
  mg_f32_bcast bc;       // batch dims (nbd = 0: one batch, or batches laid out contiguously)
  int64_t lda, ldb;      // row strides of the (non-transposed views)
  int32_t trans_a, trans_b;
  float alpha, beta;
  const float *c;        // null or device C
  int64_t c_rs, c_cs;    // element strides of C over rows / cols (0 = bcast)
  int64_t ldy = 0;       // row stride of Y (0: N; batches then lie M * ldy apart)
  // K split over workgroups (one batch): kspl partial sums of M x N floats
  // in part, added by a second launch (mg_f32_ksplit picks kspl).
  int kspl = 1;
  float *part = nullptr;
  int64_t part_cols = 0;  // columns part holds (0: N); wider problems run in column chunks
};
mg_status mg_f32_run(mg_ctx *ctx, const mg_f32_problem &p, const float *a_dev,
                     const float *b_dev, float *y_dev);
// The K split for one batch of M x K by K x N: 2 where K >= 1024 and M <= 8192
// (few row tiles, long chains of k stages), else 1.  It depends on M and K
// only, so column slices of a weight take the same split (bitwise equal
// columns).
int mg_f32_ksplit(int64_t M, int64_t K, int64_t batch);
// MatMul on operands given as doubles (the reference's non-float fallback):
// double products summed in k order, one rounding to f32.  Uses p.M, K, N,
// batch and bc (row-major A [M, K] and B [K, N] per batch).
mg_status mg_f64acc_run(mg_ctx *ctx, const mg_f32_problem &p, const double *a_dev,
                        const double *b_dev, float *y_dev);

// ------------------------------------------------------- elementwise ops

// Broadcast operand strides over the merged output dims (stride 0 along a
// broadcast dim), innermost last.
constexpr int MG_ELEM_MAXRANK = 16;  // every rank the API takes
struct mg_elem_bcast {
  int rank;
  int64_t dim[MG_ELEM_MAXRANK];
  int64_t sa[MG_ELEM_MAXRANK], sb[MG_ELEM_MAXRANK];
};
// y = a op b over n output elements; same: equal shapes (s unused).
mg_status mg_elem_binary(mg_ctx *ctx, int op, const float *a, const float *b, float *y,
                         int64_t n, bool same, const mg_elem_bcast &s);
mg_status mg_elem_sigmoid(mg_ctx *ctx, const float *x, float *y, int64_t n);
// RMSNorm over the middle dim of [outer][dim][inner]; skip / bias / sum only
// with inner == 1 (the last axis).
mg_status mg_elem_rms_norm(mg_ctx *ctx, const float *x, const float *skip, const float *gamma,
                           const float *bias, double eps, int64_t outer, int64_t dim,
                           int64_t inner, int64_t last, float *y, float *sum);
// The last-axis RMSNorm over at most 16 rows of d <= 8192, also writing the
// decode GEMV's split of y into split (kpad: its padded K).
mg_status mg_elem_rms_norm_split(mg_ctx *ctx, const float *x, const float *skip,
                                 const float *gamma, const float *bias, double eps, int64_t rows,
                                 int64_t d, float *y, float *sum, int64_t kpad, void *split);

// --------------------------------------------------------------- conv entry

// Convolution as an implicit GEMM per (batch, group): rows = output channels
// of the group, columns = output positions, k = (input channel, kernel tap).
// Spatial dims are padded to 3 (depth, height, width) with size-1 leading
// dims.  Conv reads input position i = o * str - pad + kk * dil; the
// transposed form (ConvTranspose) reads i = (o + pad - kk * dil) / str where
// that division is exact.  Element kinds: MG_CONV_F32, MG_CONV_U8,
// MG_CONV_I8.  Integer kinds use (x - x_zp) and (w - w_zp[channel]); taps in
// the padding contribute 0.
enum { MG_CONV_F32 = 0, MG_CONV_U8 = 1, MG_CONV_I8 = 2 };
// Output modes: fp32 (+ fp32 bias), int32 accumulators, requantised bytes.
enum { MG_CONV_OUT_F32 = 0, MG_CONV_OUT_I32 = 1, MG_CONV_OUT_Q8 = 2 };
struct mg_conv_problem {
  const void *x = nullptr, *w = nullptr;
  const void *bias = nullptr;  // f32 [M] (fp32 mode) or int32 [M] (requant mode), or null
  void *y = nullptr;
  int xk = MG_CONV_F32, wk = MG_CONV_F32, mode = MG_CONV_OUT_F32, trans = 0;
  int64_t n = 0, c = 0, m = 0;  // batch, input channels, output channels
  int64_t group = 1, cg = 0, mg = 0;
  int64_t in[3] = {1, 1, 1}, out[3] = {1, 1, 1}, ker[3] = {1, 1, 1};
  int64_t str[3] = {1, 1, 1}, dil[3] = {1, 1, 1}, pad[3] = {0, 0, 0};  // begin pads
  // Weight element (group g, out channel m of the group, in channel c of the
  // group, tap r) sits at g * w_gs + m * w_ms + c * w_cs + r.
  int64_t w_gs = 0, w_ms = 0, w_cs = 0;
  int32_t x_zp = 0;
  const float *w_zp = nullptr;   // device [M] (integer kinds)
  // The caller's weight zero points (host, len 0, 1 or M; integer kinds): the
  // int8 MFMA route prepacks the weights with them.
  const int32_t *w_zp_host = nullptr;
  int64_t w_zp_len = 0;
  const double *mult = nullptr;  // device [M] requant multipliers
  int32_t y_zp = 0, lo = 0, hi = 255;
  // Output placement of a sub-pixel phase (set by the phase split of a
  // strided ConvTranspose): output position o' of this problem lands at
  // o = o' * ys + yb in an output of dims yo.  phased = 0: o = o'.
  int phased = 0;
  int64_t yo[3] = {1, 1, 1}, ys[3] = {1, 1, 1}, yb[3] = {0, 0, 0};
};
// Workspace a call needs (the sub-pixel phase weights of a strided fp32
// ConvTranspose; 0 otherwise), and the launch.
size_t mg_conv_ws_bytes(const mg_conv_problem &p);
// Whether p runs on the int8 MFMA route (ConvInteger / QLinearConv, one
// group), which takes the weight zero points from w_zp_host, not w_zp.
bool mg_conv_int8_route(const mg_conv_problem &p);
mg_status mg_conv_run(mg_ctx *ctx, const mg_conv_problem &p, void *ws);

// ---------------------------------------------------------- attention entry

// y[b][q][:DV] = softmax_t(scale * sum_d Q[b][q][d] K[b][t][d] + mask[b][q][t])
//                . V[b][t][:DV] over strided views; b runs over up to
// MG_ATTN_MAX_BATCH_DIMS batch dims bdim with per-operand element strides
// (0 = broadcast).  Element (q, d) of Q is at q_rs * q + q_cs * d past the
// batch offset, and likewise (t, d) of K, (t, dv) of V and (q, t) of the
// mask; output rows are contiguous (row stride y_rs).  mask may be null.
constexpr int MG_ATTN_MAX_BATCH_DIMS = 4;
struct mg_attn_problem {
  const float *q, *k, *v, *mask;
  float *y;
  int nbd;
  int64_t bdim[MG_ATTN_MAX_BATCH_DIMS];
  int64_t q_bs[MG_ATTN_MAX_BATCH_DIMS], k_bs[MG_ATTN_MAX_BATCH_DIMS],
      v_bs[MG_ATTN_MAX_BATCH_DIMS], m_bs[MG_ATTN_MAX_BATCH_DIMS],
      y_bs[MG_ATTN_MAX_BATCH_DIMS];
  int64_t q_rs, q_cs, k_ts, k_ds, v_ts, v_ds, m_qs, m_ts, y_rs;
  int S, T, D, DV;
  float scale;
  // Causal masking: key t is excluded for query q when t > q + causal_off.
  int causal = 0;
  int64_t causal_off = 0;
  // Key split (flash-decoding): kc keys per split, partials in part (device,
  // mg_attn_plan_split's bytes), merged by a second kernel.  0 = no split.
  int kc = 0;
  float *part = nullptr;
};
mg_status mg_attn_run(mg_ctx *ctx, const mg_attn_problem &p);
size_t mg_attn_plan_split(const mg_ctx *ctx, mg_attn_problem *p);

// GroupQueryAttention's data movement before the attention products: the
// present K/V caches [batch][kv_heads][past + seq][hs] (past rows copied,
// current rows appended, K rotated when rotary) and, when rotary, the
// rotated Q [batch][seq][heads * hs] into q_rot.  RoPE at positions
// past + s from cos/sin [max_pos][half_rot], GPT-J pairs when interleaved,
// else rotate-half; dims past 2 half_rot pass through.
struct mg_gqa_prep {
  const float *q, *k, *v, *past_k, *past_v, *cos, *sin;
  float *q_rot, *present_k, *present_v;
  int64_t batch, seq, heads, kv_heads, hs, past, half_rot;
  int rotary, interleaved;
};
mg_status mg_gqa_prep_run(mg_ctx *ctx, const mg_gqa_prep &g);

// --------------------------------------------------------------- DQL entry

mg_status mg_dql_run(mg_ctx *ctx, const float *x_dev, int64_t n,
                     uint8_t *y_dev, void *scale_zp_dev, void *ws);
size_t mg_dql_ws_bytes(int64_t n);
