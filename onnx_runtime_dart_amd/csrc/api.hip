// C-ABI of libmigemm.so: contexts, device buffers, weight upload, operator
// validation (mirroring the reference's checks and their error classes) and
// dispatch to the HIP kernels.  Declarations and reference citations are in
// include/migemm.h.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "mg_internal.h"

// Defined in int8.hip.
mg_status mg_int8_run_batched(mg_ctx *ctx, const void *a_dev, int32_t a_signed,
                              int64_t a_batch, const void *b_dev,
                              int32_t b_signed, int64_t b_batch, int64_t M,
                              int64_t K, int64_t N, const int32_t *a_zp,
                              int64_t a_zp_len, const int32_t *b_zp,
                              int64_t b_zp_len, const mg_requant *rq,
                              void *y_dev, void *ws);
size_t mg_int8_long_k_ws_bytes(int64_t a_batch, int64_t b_batch, int64_t M, int64_t K, int64_t N,
                               bool requant);
mg_status mg_int8_run_long_k(mg_ctx *ctx, const void *a_dev, int32_t a_signed, int64_t a_batch,
                             const void *b_dev, int32_t b_signed, int64_t b_batch, int64_t M,
                             int64_t K, int64_t N, const int32_t *a_zp, int64_t a_zp_len,
                             const int32_t *b_zp, int64_t b_zp_len, const mg_requant *rq,
                             void *y_dev, void *ws);
size_t mg_int8_batched_ws_bytes(int64_t a_batch, int64_t b_batch, int64_t M,
                                int64_t K, int64_t N);

// Workspace of mg_matmul_nbits_dev_noalloc: one array per device, held by
// each GPU the library runs on until the process ends.  In host code the name
// `scratch` is a host-side stand-in, not a device address: the device address
// is taken with hipGetSymbolAddress once per device (scratch_init, with that
// device current) and only that address is used.
static __device__ __align__(256) unsigned char scratch[MG_NOALLOC_SCRATCH_BYTES];

namespace {
thread_local std::string g_last_error;
// Set when the last failure was the byte budget (mg_last_error_budget).
thread_local bool g_budget_failed = false;
thread_local int64_t g_budget_required = 0, g_budget_limit = 0;

int64_t prod(const int64_t *s, int32_t from, int32_t to) {
  int64_t p = 1;
  for (int32_t i = from; i < to; i++) p *= s[i];
  return p;
}

bool shape_ok(const int64_t *s, int32_t r) {
  if (r < 0 || r > 16 || (r > 0 && !s)) return false;
  for (int32_t i = 0; i < r; i++)
    if (s[i] < 0) return false;
  return true;
}

// Stages host buffers through the context workspace around a device call.
struct Staging {
  size_t off = 0;
  size_t take(size_t bytes) {
    const size_t o = off;
    off += mg_align(bytes ? bytes : 1);
    return o;
  }
};
}  // namespace

mg_status mg_fail(mg_status st, const std::string &msg) {
  g_last_error = msg;
  g_budget_failed = false;
  return st;
}

mg_status mg_launch_check(const char *what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return mg_fail(MG_DEVICE_ERROR, std::string(what) + " launch: " + hipGetErrorString(e));
  return MG_OK;
}

mg_status mg_use_device(mg_ctx *ctx) {
  MG_HIP(hipSetDevice(ctx->device));
  return MG_OK;
}

mg_status mg_check_control(mg_ctx *ctx, int64_t additional_bytes) {
  if (ctx->cancel_flag && *ctx->cancel_flag)
    return mg_fail(MG_CANCELLED, "operation cancelled");
  if (ctx->max_bytes >= 0 && additional_bytes > ctx->max_bytes) {
    mg_fail(MG_OUT_OF_MEMORY, "device memory limit exceeded: " +
                                  std::to_string(additional_bytes) + " bytes required, limit " +
                                  std::to_string(ctx->max_bytes));
    g_budget_failed = true;
    g_budget_required = additional_bytes;
    g_budget_limit = ctx->max_bytes;
    return MG_OUT_OF_MEMORY;
  }
  return MG_OK;
}

namespace {
constexpr int MG_MAX_DEVICES = 64;
std::mutex g_scratch_mu;
void *g_scratch_dev[MG_MAX_DEVICES] = {};

// With `device` current: records the device address of `scratch` on it.
mg_status scratch_init(int device) {
  if (device < 0 || device >= MG_MAX_DEVICES)
    return mg_fail(MG_UNSUPPORTED, "device index beyond " + std::to_string(MG_MAX_DEVICES));
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (g_scratch_dev[device]) return MG_OK;
  void *p = nullptr;
  const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (e != hipSuccess || !p)
    return mg_fail(MG_DEVICE_ERROR,
                   std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e));
  g_scratch_dev[device] = p;
  return MG_OK;
}

void *scratch_dev(int device) {
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  return device >= 0 && device < MG_MAX_DEVICES ? g_scratch_dev[device] : nullptr;
}
}  // namespace

ProfScope::ProfScope(mg_ctx *ctx, const char *op) : ctx_(ctx), op_(op) {
  if (!ctx_ || !ctx_->prof) {
    ctx_ = nullptr;
    return;
  }
  e0_ = prof_event(ctx_);
  if (!e0_ || hipEventRecord(e0_, ctx_->stream) != hipSuccess) ctx_ = nullptr;
}

ProfScope::~ProfScope() {
  if (!ctx_) return;
  hipEvent_t e1 = prof_event(ctx_);
  if (e1 && hipEventRecord(e1, ctx_->stream) == hipSuccess)
    ctx_->prof_recs.push_back({op_, e0_, e1});
}

hipEvent_t prof_event(mg_ctx *ctx) {
  if (!ctx->prof_pool.empty()) {
    hipEvent_t e = ctx->prof_pool.back();
    ctx->prof_pool.pop_back();
    return e;
  }
  hipEvent_t e = nullptr;
  if (hipEventCreate(&e) != hipSuccess) return nullptr;
  return e;
}

mg_status mg_ws_reserve(mg_ctx *ctx, size_t bytes) {
  if (bytes <= ctx->ws_bytes) return MG_OK;
  if (ctx->ws) {
    MG_HIP(hipStreamSynchronize(ctx->stream));
    MG_HIP(hipFree(ctx->ws));
    ctx->ws = nullptr;
    ctx->ws_bytes = 0;
  }
  const size_t want = mg_align(bytes, 1 << 20);
  MG_HIP(hipMalloc(&ctx->ws, want));
  ctx->ws_bytes = want;
  return MG_OK;
}

mg_status mg_h2d_table(mg_ctx *ctx, void *dst_dev, const void *src_host, size_t bytes) {
  if (bytes == 0) return MG_OK;
  if (bytes > MG_PIN_SLOT_BYTES) {
    MG_HIP(hipMemcpyAsync(dst_dev, src_host, bytes, hipMemcpyHostToDevice, ctx->stream));
    MG_HIP(hipStreamSynchronize(ctx->stream));
    return MG_OK;
  }
  if (!ctx->pin) {
    MG_HIP(hipHostMalloc(&ctx->pin, (size_t)MG_PIN_SLOTS * MG_PIN_SLOT_BYTES,
                         hipHostMallocDefault));
    for (int i = 0; i < MG_PIN_SLOTS; i++)
      MG_HIP(hipEventCreateWithFlags(&ctx->pin_ev[i], hipEventDisableTiming));
  }
  const int slot = ctx->pin_next;
  ctx->pin_next = (slot + 1) % MG_PIN_SLOTS;
  // The slot's previous copy must have run before its bytes are replaced
  // (an event never recorded counts as complete).
  MG_HIP(hipEventSynchronize(ctx->pin_ev[slot]));
  char *stage = static_cast<char *>(ctx->pin) + (size_t)slot * MG_PIN_SLOT_BYTES;
  std::memcpy(stage, src_host, bytes);
  MG_HIP(hipMemcpyAsync(dst_dev, stage, bytes, hipMemcpyHostToDevice, ctx->stream));
  MG_HIP(hipEventRecord(ctx->pin_ev[slot], ctx->stream));
  return MG_OK;
}

extern "C" {

const char *mg_last_error(void) { return g_last_error.c_str(); }

int32_t mg_last_error_budget(int64_t *required_bytes, int64_t *limit_bytes) {
  if (!g_budget_failed || g_last_error.empty()) return 0;
  if (required_bytes) *required_bytes = g_budget_required;
  if (limit_bytes) *limit_bytes = g_budget_limit;
  return 1;
}
const char *mg_version(void) { return "0.1.0"; }

// ------------------------------------------------------------------ context

mg_status mg_ctx_create(int32_t device, mg_ctx **out) {
  g_last_error.clear();
  if (!out) return mg_fail(MG_INVALID_ARGUMENT, "mg_ctx_create: out is null");
  *out = nullptr;
  int n = 0;
  MG_HIP(hipGetDeviceCount(&n));
  if (device < 0 || device >= n)
    return mg_fail(MG_INVALID_ARGUMENT, "mg_ctx_create: no HIP device " + std::to_string(device));
  MG_HIP(hipSetDevice(device));
  mg_ctx *c = new mg_ctx();
  c->device = device;
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) == hipSuccess &&
      cus > 0)
    c->num_cus = cus;
  hipError_t e = hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking);
  if (e != hipSuccess) {
    delete c;
    return mg_fail(MG_DEVICE_ERROR, std::string("hipStreamCreate: ") + hipGetErrorString(e));
  }
  c->own_stream = true;
  const mg_status ss = scratch_init(device);
  if (ss != MG_OK) {
    (void)hipStreamDestroy(c->stream);
    delete c;
    return ss;
  }
  *out = c;
  return MG_OK;
}

mg_status mg_ctx_destroy(mg_ctx *ctx) {
  if (!ctx) return MG_OK;
  (void)hipSetDevice(ctx->device);
  if (ctx->stream) (void)hipStreamSynchronize(ctx->stream);
  if (ctx->ws) (void)hipFree(ctx->ws);
  for (int i = 0; i < MG_PIN_SLOTS; i++)
    if (ctx->pin_ev[i]) (void)hipEventDestroy(ctx->pin_ev[i]);
  for (const mg_prof_rec &r : ctx->prof_recs) {
    (void)hipEventDestroy(r.e0);
    (void)hipEventDestroy(r.e1);
  }
  for (hipEvent_t e : ctx->prof_pool) (void)hipEventDestroy(e);
  if (ctx->pin) (void)hipHostFree(ctx->pin);
  if (ctx->up_pin) (void)hipHostFree(ctx->up_pin);
  if (ctx->up_dev) (void)hipFree(ctx->up_dev);
  for (hipEvent_t e : ctx->up_done)
    if (e) (void)hipEventDestroy(e);
  if (ctx->own_stream && ctx->stream) (void)hipStreamDestroy(ctx->stream);
  delete ctx;
  return MG_OK;
}

mg_status mg_ctx_set_stream(mg_ctx *ctx, void *hip_stream) {
  if (!ctx) return mg_fail(MG_INVALID_ARGUMENT, "mg_ctx_set_stream: null context");
  MG_TRY(mg_use_device(ctx));
  if (ctx->stream) MG_HIP(hipStreamSynchronize(ctx->stream));
  if (ctx->own_stream && ctx->stream) MG_HIP(hipStreamDestroy(ctx->stream));
  ctx->stream = static_cast<hipStream_t>(hip_stream);
  ctx->own_stream = false;
  return MG_OK;
}

mg_status mg_ctx_get_stream(mg_ctx *ctx, void **hip_stream) {
  if (!ctx || !hip_stream) return mg_fail(MG_INVALID_ARGUMENT, "mg_ctx_get_stream: null argument");
  *hip_stream = ctx->stream;
  return MG_OK;
}

mg_status mg_ctx_set_profiling(mg_ctx *ctx, int32_t enable) {
  if (!ctx) return mg_fail(MG_INVALID_ARGUMENT, "mg_ctx_set_profiling: null context");
  MG_TRY(mg_ctx_profile_clear(ctx));
  ctx->prof = enable != 0;
  return MG_OK;
}

mg_status mg_ctx_set_prefill_images(mg_ctx *ctx, int32_t enable) {
  if (!ctx) return mg_fail(MG_INVALID_ARGUMENT, "mg_ctx_set_prefill_images: null context");
  ctx->prefill_images = enable != 0;
  return MG_OK;
}

mg_status mg_ctx_profile_count(mg_ctx *ctx, int64_t *n) {
  if (!ctx || !n) return mg_fail(MG_INVALID_ARGUMENT, "mg_ctx_profile_count: null argument");
  *n = (int64_t)ctx->prof_recs.size();
  return MG_OK;
}

mg_status mg_ctx_profile_get(mg_ctx *ctx, int64_t i, const char **op, float *ms) {
  if (!ctx || !op || !ms) return mg_fail(MG_INVALID_ARGUMENT, "mg_ctx_profile_get: null argument");
  if (i < 0 || i >= (int64_t)ctx->prof_recs.size())
    return mg_fail(MG_INVALID_ARGUMENT, "mg_ctx_profile_get: record index out of range");
  const mg_prof_rec &r = ctx->prof_recs[(size_t)i];
  MG_HIP(hipEventSynchronize(r.e1));
  MG_HIP(hipEventElapsedTime(ms, r.e0, r.e1));
  *op = r.op;
  return MG_OK;
}

mg_status mg_ctx_profile_clear(mg_ctx *ctx) {
  if (!ctx) return mg_fail(MG_INVALID_ARGUMENT, "mg_ctx_profile_clear: null context");
  if (!ctx->prof_recs.empty()) MG_HIP(hipStreamSynchronize(ctx->stream));
  for (const mg_prof_rec &r : ctx->prof_recs) {
    ctx->prof_pool.push_back(r.e0);
    ctx->prof_pool.push_back(r.e1);
  }
  ctx->prof_recs.clear();
  return MG_OK;
}

mg_status mg_ctx_synchronize(mg_ctx *ctx) {
  if (!ctx) return mg_fail(MG_INVALID_ARGUMENT, "mg_ctx_synchronize: null context");
  MG_TRY(mg_use_device(ctx));
  MG_HIP(hipStreamSynchronize(ctx->stream));
  return MG_OK;
}

mg_status mg_ctx_set_control(mg_ctx *ctx, const volatile int32_t *cancel_flag,
                             int64_t max_bytes) {
  if (!ctx) return mg_fail(MG_INVALID_ARGUMENT, "mg_ctx_set_control: null context");
  ctx->cancel_flag = cancel_flag;
  ctx->max_bytes = max_bytes;
  return MG_OK;
}

// ---------------------------------------------------------------- buffers

mg_status mg_buffer_alloc(mg_ctx *ctx, size_t bytes, void **dev_ptr) {
  if (!ctx || !dev_ptr) return mg_fail(MG_INVALID_ARGUMENT, "mg_buffer_alloc: null argument");
  *dev_ptr = nullptr;
  MG_TRY(mg_use_device(ctx));
  MG_TRY(mg_check_control(ctx, (int64_t)bytes));
  MG_HIP(hipMalloc(dev_ptr, bytes ? bytes : 1));
  return MG_OK;
}

mg_status mg_buffer_free(mg_ctx *ctx, void *dev_ptr) {
  if (!ctx) return mg_fail(MG_INVALID_ARGUMENT, "mg_buffer_free: null context");
  if (!dev_ptr) return MG_OK;
  MG_TRY(mg_use_device(ctx));
  MG_HIP(hipStreamSynchronize(ctx->stream));
  MG_HIP(hipFree(dev_ptr));
  return MG_OK;
}

mg_status mg_buffer_upload(mg_ctx *ctx, void *dev_dst, const void *host_src, size_t bytes) {
  if (!ctx || (bytes && (!dev_dst || !host_src)))
    return mg_fail(MG_INVALID_ARGUMENT, "mg_buffer_upload: null argument");
  MG_TRY(mg_use_device(ctx));
  MG_HIP(hipMemcpyAsync(dev_dst, host_src, bytes, hipMemcpyHostToDevice, ctx->stream));
  MG_HIP(hipStreamSynchronize(ctx->stream));
  return MG_OK;
}

mg_status mg_buffer_download(mg_ctx *ctx, void *host_dst, const void *dev_src, size_t bytes) {
  if (!ctx || (bytes && (!host_dst || !dev_src)))
    return mg_fail(MG_INVALID_ARGUMENT, "mg_buffer_download: null argument");
  MG_TRY(mg_use_device(ctx));
  MG_HIP(hipMemcpyAsync(host_dst, dev_src, bytes, hipMemcpyDeviceToHost, ctx->stream));
  MG_HIP(hipStreamSynchronize(ctx->stream));
  return MG_OK;
}

// ---------------------------------------------------------------- weights

mg_status mg_weight_release(mg_weight *w) {
  if (!w) return MG_OK;
  (void)hipSetDevice(w->device);
  (void)hipDeviceSynchronize();
  if (w->kind == MG_W_NBITS) mg_nbits_free(w);
  if (w->kind == MG_W_INT8) mg_int8_free(w);
  if (w->kind == MG_W_F32 && w->f32.b) (void)hipFree(w->f32.b);
  delete w;
  return MG_OK;
}

mg_status mg_weight_info(const mg_weight *w, int64_t *K, int64_t *N, int64_t *device_bytes) {
  if (!w) return mg_fail(MG_INVALID_ARGUMENT, "mg_weight_info: null weight");
  if (K) *K = w->K;
  if (N) *N = w->N;
  if (device_bytes) *device_bytes = w->device_bytes;
  return MG_OK;
}

mg_status mg_weight_nbits_create(
    mg_ctx *ctx, int64_t K, int64_t N, int64_t bits, int64_t block_size,
    const uint8_t *b, const int64_t *b_shape, int32_t b_rank,
    const float *scales, const int64_t *scales_shape, int32_t scales_rank,
    int32_t zp_kind, const void *zp, const int64_t *zp_shape, int32_t zp_rank,
    const float *bias, const int64_t *bias_shape, int32_t bias_rank,
    int32_t has_g_idx, mg_weight **out) {
  ProfScope prof_(ctx, "MatMulNBits.upload");
  g_last_error.clear();
  if (!ctx || !out) return mg_fail(MG_INVALID_ARGUMENT, "mg_weight_nbits_create: null argument");
  *out = nullptr;
  // lib/src/onnx_graph.dart:2919-2921
  if (has_g_idx) return mg_fail(MG_UNSUPPORTED, "MatMulNBits: g_idx input not supported");
  // lib/src/onnx_qlinear_ops.dart:126-128
  if (bits != 4)
    return mg_fail(MG_UNSUPPORTED,
                   "MatMulNBits: only bits=4 supported, got " + std::to_string(bits));
  // :129-136 (the activation-shape half of this check is made per call)
  if (K <= 0 || N <= 0 || block_size < 16 || (block_size & (block_size - 1)) != 0)
    return mg_fail(MG_INVALID_ARGUMENT, "MatMulNBits: invalid K, N, block_size or input shape");
  const int64_t nb = (K + block_size - 1) / block_size;
  const int64_t blob = block_size / 2;
  const int64_t zp_stride = (nb + 1) / 2;
  // :140-152
  if (!b || !scales || !shape_ok(b_shape, b_rank) || !shape_ok(scales_shape, scales_rank) ||
      b_rank != 3 || b_shape[0] != N || b_shape[1] != nb || b_shape[2] != blob ||
      prod(scales_shape, 0, scales_rank) != N * nb || (scales_rank != 1 && scales_rank != 2) ||
      (scales_rank == 2 && (scales_shape[0] != N || scales_shape[1] != nb)))
    return mg_fail(MG_INVALID_ARGUMENT, "MatMulNBits: invalid packed weights or scales");
  // :155-163
  if (zp_kind != MG_ZP_NONE) {
    if (!zp || !shape_ok(zp_shape, zp_rank) || (zp_kind != MG_ZP_UINT4 && zp_kind != MG_ZP_FLOAT) ||
        (zp_rank != 1 && zp_rank != 2) || (zp_rank == 2 && zp_shape[0] != N) ||
        (zp_kind == MG_ZP_UINT4 ? prod(zp_shape, 0, zp_rank) != N * zp_stride
                                : prod(zp_shape, 0, zp_rank) != N * nb))
      return mg_fail(MG_INVALID_ARGUMENT, "MatMulNBits: invalid zero_points");
  }
  // :164-166
  if (bias && (!shape_ok(bias_shape, bias_rank) || bias_rank != 1 || bias_shape[0] != N))
    return mg_fail(MG_INVALID_ARGUMENT, "MatMulNBits: bias must be floating point [N]");
  MG_TRY(mg_use_device(ctx));
  mg_weight *w = new mg_weight();
  w->kind = MG_W_NBITS;
  w->device = ctx->device;
  w->K = K;
  w->N = N;
  w->nbits.bs = block_size;
  mg_byte_source sb, ss, sz;
  sb.host = b;
  ss.host = reinterpret_cast<const uint8_t *>(scales);
  sz.host = static_cast<const uint8_t *>(zp);
  mg_status st = mg_nbits_upload(ctx, w, sb, ss, zp_kind, sz, bias, 0);
  if (st != MG_OK) {
    mg_nbits_free(w);
    delete w;
    return st;
  }
  *out = w;
  return MG_OK;
}

mg_status mg_weight_nbits_create_streamed(mg_ctx *ctx, int64_t K, int64_t N, int64_t bits,
                                          int64_t block_size, const mg_tensor_source *b,
                                          const mg_tensor_source *scales, int32_t zp_kind,
                                          const mg_tensor_source *zp, const float *bias,
                                          int32_t has_g_idx, int64_t chunk_bytes,
                                          mg_weight **out) {
  ProfScope prof_(ctx, "MatMulNBits.upload");
  g_last_error.clear();
  if (!ctx || !out || !b || !scales)
    return mg_fail(MG_INVALID_ARGUMENT, "mg_weight_nbits_create_streamed: null argument");
  *out = nullptr;
  if (has_g_idx) return mg_fail(MG_UNSUPPORTED, "MatMulNBits: g_idx input not supported");
  if (bits != 4)
    return mg_fail(MG_UNSUPPORTED,
                   "MatMulNBits: only bits=4 supported, got " + std::to_string(bits));
  if (K <= 0 || N <= 0 || block_size < 16 || (block_size & (block_size - 1)) != 0)
    return mg_fail(MG_INVALID_ARGUMENT, "MatMulNBits: invalid K, N, block_size or input shape");
  if (zp_kind != MG_ZP_NONE && zp_kind != MG_ZP_UINT4 && zp_kind != MG_ZP_FLOAT)
    return mg_fail(MG_INVALID_ARGUMENT, "MatMulNBits: invalid zero_points");
  if (zp_kind != MG_ZP_NONE && !zp)
    return mg_fail(MG_INVALID_ARGUMENT, "MatMulNBits: invalid zero_points");
  const int64_t nb = (K + block_size - 1) / block_size;
  // Byte counts implied by the shapes; a stated length must cover them (a
  // shorter tensor is malformed, lib/src/onnx_proto_loader.dart:96-125).
  const int64_t need[3] = {N * nb * (block_size / 2), N * nb * 4,
                           zp_kind == MG_ZP_UINT4 ? N * ((nb + 1) / 2)
                                                  : zp_kind == MG_ZP_FLOAT ? N * nb * 4 : 0};
  const mg_tensor_source *src[3] = {b, scales, zp};
  const char *what[3] = {"B", "scales", "zero_points"};
  mg_byte_source bsrc[3];
  for (int i = 0; i < 3; i++) {
    if (i == 2 && zp_kind == MG_ZP_NONE) break;
    const mg_tensor_source &t = *src[i];
    if ((!t.host && !t.path) || t.offset < 0 || t.length < 0 ||
        (t.length > 0 && t.length < need[i]))
      return mg_fail(MG_INVALID_ARGUMENT, std::string("MatMulNBits: ") + what[i] +
                                              " source must hold " + std::to_string(need[i]) +
                                              " bytes");
    bsrc[i].host = static_cast<const uint8_t *>(t.host);
    bsrc[i].path = t.host ? nullptr : t.path;
    bsrc[i].offset = t.offset;
  }
  MG_TRY(mg_use_device(ctx));
  mg_weight *w = new mg_weight();
  w->kind = MG_W_NBITS;
  w->device = ctx->device;
  w->K = K;
  w->N = N;
  w->nbits.bs = block_size;
  mg_status st = mg_nbits_upload(ctx, w, bsrc[0], bsrc[1], zp_kind, bsrc[2], bias, chunk_bytes);
  if (st != MG_OK) {
    mg_nbits_free(w);
    delete w;
    return st;
  }
  *out = w;
  return MG_OK;
}

mg_status mg_weight_int8_create(mg_ctx *ctx, const void *b, int32_t b_signed, int64_t K,
                                int64_t N, const int32_t *b_zp, int64_t b_zp_len,
                                mg_weight **out) {
  ProfScope prof_(ctx, "MatMulInteger.upload");
  g_last_error.clear();
  if (!ctx || !out || (!b && K * N > 0))
    return mg_fail(MG_INVALID_ARGUMENT, "mg_weight_int8_create: null argument");
  *out = nullptr;
  if (K < 0 || N < 0) return mg_fail(MG_INVALID_ARGUMENT, "MatMulInteger: invalid B shape");
  if (b_zp && b_zp_len != 1 && b_zp_len != N)
    return mg_fail(MG_UNSUPPORTED,
                   "MatMulInteger: zero points must be scalar, per-row [M] for A or "
                   "per-column [N] for B");
  MG_TRY(mg_use_device(ctx));
  mg_weight *w = new mg_weight();
  w->kind = MG_W_INT8;
  w->device = ctx->device;
  w->K = K;
  w->N = N;
  mg_status st = mg_int8_upload(ctx, w, b, b_signed, b_zp, b_zp ? b_zp_len : 0);
  if (st != MG_OK) {
    delete w;
    return st;
  }
  *out = w;
  return MG_OK;
}

mg_status mg_weight_f32_create(mg_ctx *ctx, const float *b, int64_t rows, int64_t cols,
                               int32_t trans_b, mg_weight **out) {
  ProfScope prof_(ctx, "Gemm.upload");
  g_last_error.clear();
  if (!ctx || !out || (!b && rows * cols > 0))
    return mg_fail(MG_INVALID_ARGUMENT, "mg_weight_f32_create: null argument");
  *out = nullptr;
  if (rows < 0 || cols < 0) return mg_fail(MG_INVALID_ARGUMENT, "Gemm: invalid B shape");
  MG_TRY(mg_use_device(ctx));
  const int64_t K = trans_b ? cols : rows, N = trans_b ? rows : cols;
  // Device layout [N][K] (k contiguous, the GEMM's operand order): a
  // transB weight is stored as given, a plain [K][N] one is transposed once
  // here (the prepack of lib/src/onnx_graph.dart:2159-2161, reversed).
  std::vector<float> t;
  const float *src = b;
  if (!trans_b) {
    t.resize((size_t)(K * N));
    for (int64_t k = 0; k < K; k++)
      for (int64_t n = 0; n < N; n++) t[(size_t)(n * K + k)] = b[k * N + n];
    src = t.data();
  }
  mg_weight *w = new mg_weight();
  w->kind = MG_W_F32;
  w->device = ctx->device;
  w->K = K;
  w->N = N;
  const size_t bytes = (size_t)(K * N) * 4;
  hipError_t e = hipMalloc((void **)&w->f32.b, bytes ? bytes : 4);
  if (e != hipSuccess) {
    delete w;
    return mg_fail(MG_OUT_OF_MEMORY, "mg_weight_f32_create: allocation failed");
  }
  w->device_bytes = (int64_t)bytes;
  if (bytes && hipMemcpy(w->f32.b, src, bytes, hipMemcpyHostToDevice) != hipSuccess) {
    (void)hipFree(w->f32.b);
    delete w;
    return mg_fail(MG_DEVICE_ERROR, "mg_weight_f32_create: upload failed");
  }
  *out = w;
  return MG_OK;
}

// ------------------------------------------------------------ MatMulNBits

mg_status mg_matmul_nbits_dev(mg_ctx *ctx, const mg_weight *w, const float *a_dev, int64_t M,
                              float *y_dev) {
  ProfScope prof_(ctx, "MatMulNBits");
  g_last_error.clear();
  if (!ctx || !w || w->kind != MG_W_NBITS)
    return mg_fail(MG_INVALID_ARGUMENT, "mg_matmul_nbits: not a MatMulNBits weight");
  if (M < 0) return mg_fail(MG_INVALID_ARGUMENT, "MatMulNBits: invalid K, N, block_size or input shape");
  if (M == 0) return MG_OK;
  if (!a_dev || !y_dev) return mg_fail(MG_INVALID_ARGUMENT, "mg_matmul_nbits: null buffer");
  MG_TRY(mg_use_device(ctx));
  const size_t ws = mg_nbits_ws_bytes(ctx, w, M);
  MG_TRY(mg_check_control(ctx, (int64_t)ws));
  MG_TRY(mg_ws_reserve(ctx, ws));
  return mg_nbits_run(ctx, w, a_dev, M, y_dev, ctx->ws);
}

mg_status mg_matmul_nbits_dev_noalloc(mg_ctx *ctx, const mg_weight *w, const float *a_dev,
                                      int64_t M, float *y_dev) {
  g_last_error.clear();
  if (!ctx || !w || w->kind != MG_W_NBITS)
    return mg_fail(MG_INVALID_ARGUMENT, "mg_matmul_nbits: not a MatMulNBits weight");
  if (M < 0) return mg_fail(MG_INVALID_ARGUMENT, "MatMulNBits: invalid K, N, block_size or input shape");
  if (M == 0) return MG_OK;
  if (!a_dev || !y_dev) return mg_fail(MG_INVALID_ARGUMENT, "mg_matmul_nbits: null buffer");
  const size_t ws = mg_nbits_ws_bytes(ctx, w, M);
  if (ws > (size_t)MG_NOALLOC_SCRATCH_BYTES)
    return mg_fail(MG_INVALID_ARGUMENT,
                   "mg_matmul_nbits_dev_noalloc: " + std::to_string(M) + " rows need " +
                       std::to_string(ws) + " bytes of workspace, the scratch holds " +
                       std::to_string((size_t)MG_NOALLOC_SCRATCH_BYTES));
  MG_TRY(mg_use_device(ctx));
  MG_TRY(mg_check_control(ctx, 0));
  void *s = scratch_dev(ctx->device);
  if (!s) return mg_fail(MG_DEVICE_ERROR, "mg_matmul_nbits_dev_noalloc: no scratch on this device");
  return mg_nbits_run(ctx, w, a_dev, M, y_dev, s);
}

namespace {
mg_status nbits_group(mg_ctx *ctx, const std::string &what, int32_t n, const mg_weight *const *w,
                      const float *a_dev, const void *split_dev, int64_t M,
                      float *const *y_dev) {
  ProfScope prof_(ctx, "MatMulNBits");
  g_last_error.clear();
  if (!ctx || !w || !y_dev || n < 1 || n > 4)
    return mg_fail(MG_INVALID_ARGUMENT, what + ": 1 to 4 weights expected");
  for (int32_t i = 0; i < n; i++) {
    if (!w[i] || w[i]->kind != MG_W_NBITS)
      return mg_fail(MG_INVALID_ARGUMENT, what + ": not a MatMulNBits weight");
    if (w[i]->K != w[0]->K || w[i]->nbits.bs != w[0]->nbits.bs ||
        w[i]->nbits.zp_kind != w[0]->nbits.zp_kind || w[i]->device != w[0]->device)
      return mg_fail(MG_INVALID_ARGUMENT,
                     what + ": weights must share K, block_size, zero-point form and device");
    if (!y_dev[i]) return mg_fail(MG_INVALID_ARGUMENT, what + ": null output");
  }
  if (M < 0) return mg_fail(MG_INVALID_ARGUMENT, "MatMulNBits: invalid K, N, block_size or input shape");
  if (M == 0) return MG_OK;
  if (!a_dev) return mg_fail(MG_INVALID_ARGUMENT, what + ": null input");
  MG_TRY(mg_use_device(ctx));
  const size_t ws = mg_nbits_group_ws_bytes(ctx, n, w, M);
  MG_TRY(mg_check_control(ctx, (int64_t)ws));
  MG_TRY(mg_ws_reserve(ctx, ws));
  return mg_nbits_run_group(ctx, n, w, a_dev, M, y_dev, ctx->ws, split_dev);
}
}  // namespace

mg_status mg_matmul_nbits_group_dev(mg_ctx *ctx, int32_t n, const mg_weight *const *w,
                                    const float *a_dev, int64_t M, float *const *y_dev) {
  return nbits_group(ctx, "mg_matmul_nbits_group_dev", n, w, a_dev, nullptr, M, y_dev);
}

mg_status mg_matmul_nbits_group_split_dev(mg_ctx *ctx, int32_t n, const mg_weight *const *w,
                                          const float *a_dev, const void *split_dev, int64_t M,
                                          float *const *y_dev) {
  return nbits_group(ctx, "mg_matmul_nbits_group_split_dev", n, w, a_dev, split_dev, M, y_dev);
}

mg_status mg_nbits_split_bytes(int64_t K, int64_t block_size, size_t *bytes) {
  g_last_error.clear();
  if (!bytes || K < 1 || block_size < 16 || (block_size & (block_size - 1)))
    return mg_fail(MG_INVALID_ARGUMENT, "mg_nbits_split_bytes: invalid K or block_size");
  *bytes = mg_nbits_split_size(mg_nbits_kpad(K, block_size));
  return MG_OK;
}

mg_status mg_matmul_nbits(mg_ctx *ctx, const mg_weight *w, const float *a, int64_t M, float *y) {
  ProfScope prof_(ctx, "MatMulNBits");
  g_last_error.clear();
  if (!ctx || !w || w->kind != MG_W_NBITS)
    return mg_fail(MG_INVALID_ARGUMENT, "mg_matmul_nbits: not a MatMulNBits weight");
  if (M < 0) return mg_fail(MG_INVALID_ARGUMENT, "MatMulNBits: invalid K, N, block_size or input shape");
  if (M == 0) return MG_OK;
  if (!a || !y) return mg_fail(MG_INVALID_ARGUMENT, "mg_matmul_nbits: null buffer");
  MG_TRY(mg_use_device(ctx));
  Staging s;
  const size_t oa = s.take((size_t)(M * w->K) * 4);
  const size_t oy = s.take((size_t)(M * w->N) * 4);
  const size_t ow = s.take(mg_nbits_ws_bytes(ctx, w, M));
  MG_TRY(mg_check_control(ctx, (int64_t)s.off));
  MG_TRY(mg_ws_reserve(ctx, s.off));
  char *base = static_cast<char *>(ctx->ws);
  MG_HIP(hipMemcpyAsync(base + oa, a, (size_t)(M * w->K) * 4, hipMemcpyHostToDevice, ctx->stream));
  MG_TRY(mg_nbits_run(ctx, w, reinterpret_cast<float *>(base + oa), M,
                      reinterpret_cast<float *>(base + oy), base + ow));
  MG_HIP(hipMemcpyAsync(y, base + oy, (size_t)(M * w->N) * 4, hipMemcpyDeviceToHost, ctx->stream));
  MG_HIP(hipStreamSynchronize(ctx->stream));
  return MG_OK;
}

// ------------------------------------------------ MatMulInteger / QLinear

namespace {

struct IntProblem {
  int64_t M = 0, K = 0, N = 0, a_batch = 1, b_batch = 1, batch = 1;
};

// Longest K whose int32 sum is exact for every operand: 33025 * 255 * 255 <
// 2^31.  Longer rows take the int64 segment path (mg_int8_run_long_k).
constexpr int64_t MG_I8_MAX_K32 = 33025;

mg_status check_integer(const int64_t *a_shape, int32_t a_rank, const int64_t *b_shape,
                        int32_t b_rank, int64_t a_zp_len, bool has_azp, int64_t b_zp_len,
                        bool has_bzp, IntProblem *p) {
  if (!shape_ok(a_shape, a_rank) || !shape_ok(b_shape, b_rank) || a_rank < 2 || b_rank < 2)
    return mg_fail(MG_INVALID_ARGUMENT, "MatMulInteger: operands must have rank >= 2");
  p->M = a_shape[a_rank - 2];
  p->K = a_shape[a_rank - 1];
  p->N = b_shape[b_rank - 1];
  if (b_shape[b_rank - 2] != p->K)
    return mg_fail(MG_INVALID_ARGUMENT, "MatMulInteger inner dim mismatch");
  // lib/src/onnx_qlinear_ops.dart:37-45
  if ((has_azp && a_zp_len != 1 && a_zp_len != p->M) ||
      (has_bzp && b_zp_len != 1 && b_zp_len != p->N))
    return mg_fail(MG_UNSUPPORTED,
                   "MatMulInteger: zero points must be scalar, per-row [M] for A or "
                   "per-column [N] for B");
  p->a_batch = prod(a_shape, 0, a_rank - 2);
  p->b_batch = prod(b_shape, 0, b_rank - 2);
  p->batch = std::max(p->a_batch, p->b_batch);
  // :46-54
  if ((p->a_batch != p->batch && p->a_batch != 1) || (p->b_batch != p->batch && p->b_batch != 1))
    return mg_fail(MG_INVALID_ARGUMENT, "MatMulInteger batch mismatch");
  return MG_OK;
}

// Host-pointer MatMulInteger / QLinearMatMul on a runtime B.  y: int32
// (out_i64 false), int64 (out_i64 true) or requantised bytes (rq).  Rows
// longer than MG_I8_MAX_K32 k, and every int64 call, take the segment path
// with int64 sums; int32 output is refused there (the sums may not fit).
mg_status integer_host(mg_ctx *ctx, const void *a, int32_t a_signed, const int64_t *a_shape,
                       int32_t a_rank, const int32_t *a_zp, int64_t a_zp_len, const void *b,
                       int32_t b_signed, const int64_t *b_shape, int32_t b_rank,
                       const int32_t *b_zp, int64_t b_zp_len, const mg_requant *rq, void *y,
                       bool out_i64 = false) {
  IntProblem p;
  MG_TRY(check_integer(a_shape, a_rank, b_shape, b_rank, a_zp_len, a_zp != nullptr, b_zp_len,
                       b_zp != nullptr, &p));
  const bool long_k = out_i64 || p.K > MG_I8_MAX_K32;
  if (long_k && !out_i64 && !mg_requant_out(rq))
    return mg_fail(MG_UNSUPPORTED,
                   "MatMulInteger: K > 33025 may exceed the int32 output; use the int64 form "
                   "(mg_matmul_integer_i64)");
  const int64_t ysz = p.batch * p.M * p.N * (mg_requant_out(rq) ? 1 : (out_i64 ? 8 : 4));
  if (p.batch * p.M * p.N == 0) return MG_OK;
  if ((!a && p.a_batch * p.M * p.K) || (!b && p.b_batch * p.K * p.N) || !y)
    return mg_fail(MG_INVALID_ARGUMENT, "MatMulInteger: null buffer");
  MG_TRY(mg_use_device(ctx));
  Staging s;
  const size_t abytes = (size_t)(p.a_batch * p.M * p.K), bbytes = (size_t)(p.b_batch * p.K * p.N);
  const size_t oa = s.take(abytes), ob = s.take(bbytes), oy = s.take((size_t)ysz);
  const size_t ow = s.take(
      long_k ? mg_int8_long_k_ws_bytes(p.a_batch, p.b_batch, p.M, p.K, p.N, mg_requant_out(rq))
             : mg_int8_batched_ws_bytes(p.a_batch, p.b_batch, p.M, p.K, p.N));
  MG_TRY(mg_check_control(ctx, (int64_t)s.off));
  MG_TRY(mg_ws_reserve(ctx, s.off));
  char *base = static_cast<char *>(ctx->ws);
  if (abytes) MG_HIP(hipMemcpyAsync(base + oa, a, abytes, hipMemcpyHostToDevice, ctx->stream));
  if (bbytes) MG_HIP(hipMemcpyAsync(base + ob, b, bbytes, hipMemcpyHostToDevice, ctx->stream));
  if (long_k)
    MG_TRY(mg_int8_run_long_k(ctx, base + oa, a_signed, p.a_batch, base + ob, b_signed,
                              p.b_batch, p.M, p.K, p.N, a_zp, a_zp ? a_zp_len : 0, b_zp,
                              b_zp ? b_zp_len : 0, rq, base + oy, base + ow));
  else
    MG_TRY(mg_int8_run_batched(ctx, base + oa, a_signed, p.a_batch, base + ob, b_signed,
                               p.b_batch, p.M, p.K, p.N, a_zp, a_zp ? a_zp_len : 0, b_zp,
                               b_zp ? b_zp_len : 0, rq, base + oy, base + ow));
  MG_HIP(hipMemcpyAsync(y, base + oy, (size_t)ysz, hipMemcpyDeviceToHost, ctx->stream));
  MG_HIP(hipStreamSynchronize(ctx->stream));
  return MG_OK;
}

mg_status requant_params(float a_scale, float b_scale, float y_scale, int32_t y_zp, int32_t lo,
                         int32_t hi, mg_requant *rq) {
  if (!(lo == 0 && hi == 255) && !(lo == -128 && hi == 127))
    return mg_fail(MG_INVALID_ARGUMENT, "QLinearMatMul: [lo, hi] must be [0, 255] or [-128, 127]");
  // lib/src/onnx_qlinear_ops.dart:95-98: each step rounded to f32.
  const float ab = (float)((double)a_scale * (double)b_scale);
  rq->mult = (float)((double)ab / (double)y_scale);
  rq->y_zp = y_zp;
  rq->lo = lo;
  rq->hi = hi;
  return MG_OK;
}

mg_status check_weight_rows(const mg_weight *w, int64_t rows, int64_t K, const int32_t *a_zp,
                            int64_t a_zp_len) {
  if (!w || w->kind != MG_W_INT8)
    return mg_fail(MG_INVALID_ARGUMENT, "MatMulInteger: not an 8-bit weight");
  if (rows < 0 || K != w->K) return mg_fail(MG_INVALID_ARGUMENT, "MatMulInteger inner dim mismatch");
  if (a_zp && (a_zp_len < 1 || (a_zp_len > 1 && rows % a_zp_len != 0)))
    return mg_fail(MG_UNSUPPORTED,
                   "MatMulInteger: zero points must be scalar, per-row [M] for A or "
                   "per-column [N] for B");
  if (K > MG_I8_MAX_K32)
    return mg_fail(MG_UNSUPPORTED,
                   "MatMulInteger: K > 33025 may exceed the int32 accumulator of an uploaded "
                   "weight; use the runtime-B forms (mg_matmul_integer_i64, mg_qlinear_matmul)");
  return MG_OK;
}

mg_status integer_w(mg_ctx *ctx, const void *a, bool a_on_device, int32_t a_signed, int64_t rows,
                    int64_t K, const int32_t *a_zp, int64_t a_zp_len, const mg_weight *w,
                    const mg_requant *rq, void *y, bool y_on_device) {
  MG_TRY(check_weight_rows(w, rows, K, a_zp, a_zp_len));
  if (rows == 0 || w->N == 0) return MG_OK;
  if (!a || !y) return mg_fail(MG_INVALID_ARGUMENT, "MatMulInteger: null buffer");
  MG_TRY(mg_use_device(ctx));
  const size_t ysz = (size_t)(rows * w->N) * (mg_requant_out(rq) ? 1 : 4);
  Staging s;
  const size_t oa = a_on_device ? 0 : s.take((size_t)(rows * K));
  const size_t oy = y_on_device ? 0 : s.take(ysz);
  const size_t ow = s.take(mg_int8_ws_bytes(w, rows) + mg_align((size_t)rows * 4 + 4));
  MG_TRY(mg_check_control(ctx, (int64_t)s.off));
  MG_TRY(mg_ws_reserve(ctx, s.off));
  char *base = static_cast<char *>(ctx->ws);
  const void *ad = a;
  void *yd = y;
  if (!a_on_device) {
    MG_HIP(hipMemcpyAsync(base + oa, a, (size_t)(rows * K), hipMemcpyHostToDevice, ctx->stream));
    ad = base + oa;
  }
  if (!y_on_device) yd = base + oy;
  MG_TRY(mg_int8_run(ctx, w, ad, a_signed, rows, a_zp, a_zp ? a_zp_len : 0, rq, yd, base + ow));
  if (!y_on_device) {
    MG_HIP(hipMemcpyAsync(y, yd, ysz, hipMemcpyDeviceToHost, ctx->stream));
    MG_HIP(hipStreamSynchronize(ctx->stream));
  }
  return MG_OK;
}

}  // namespace

mg_status mg_matmul_integer(mg_ctx *ctx, const void *a, int32_t a_signed, const int64_t *a_shape,
                            int32_t a_rank, const void *b, int32_t b_signed,
                            const int64_t *b_shape, int32_t b_rank, const int32_t *a_zp,
                            int64_t a_zp_len, const int32_t *b_zp, int64_t b_zp_len,
                            int32_t *y) {
  ProfScope prof_(ctx, "MatMulInteger");
  g_last_error.clear();
  if (!ctx) return mg_fail(MG_INVALID_ARGUMENT, "mg_matmul_integer: null context");
  return integer_host(ctx, a, a_signed, a_shape, a_rank, a_zp, a_zp_len, b, b_signed, b_shape,
                      b_rank, b_zp, b_zp_len, nullptr, y);
}

mg_status mg_matmul_integer_i64(mg_ctx *ctx, const void *a, int32_t a_signed,
                                const int64_t *a_shape, int32_t a_rank, const void *b,
                                int32_t b_signed, const int64_t *b_shape, int32_t b_rank,
                                const int32_t *a_zp, int64_t a_zp_len, const int32_t *b_zp,
                                int64_t b_zp_len, int64_t *y) {
  ProfScope prof_(ctx, "MatMulInteger");
  g_last_error.clear();
  if (!ctx) return mg_fail(MG_INVALID_ARGUMENT, "mg_matmul_integer_i64: null context");
  return integer_host(ctx, a, a_signed, a_shape, a_rank, a_zp, a_zp_len, b, b_signed, b_shape,
                      b_rank, b_zp, b_zp_len, nullptr, y, true);
}

mg_status mg_matmul_integer_w(mg_ctx *ctx, const void *a, int32_t a_signed, int64_t rows,
                              int64_t K, const int32_t *a_zp, int64_t a_zp_len,
                              const mg_weight *w, int32_t *y) {
  ProfScope prof_(ctx, "MatMulInteger");
  g_last_error.clear();
  if (!ctx) return mg_fail(MG_INVALID_ARGUMENT, "mg_matmul_integer_w: null context");
  return integer_w(ctx, a, false, a_signed, rows, K, a_zp, a_zp_len, w, nullptr, y, false);
}

mg_status mg_matmul_integer_w_dev(mg_ctx *ctx, const void *a_dev, int32_t a_signed, int64_t rows,
                                  int64_t K, const int32_t *a_zp, int64_t a_zp_len,
                                  const mg_weight *w, int32_t *y_dev) {
  ProfScope prof_(ctx, "MatMulInteger");
  g_last_error.clear();
  if (!ctx) return mg_fail(MG_INVALID_ARGUMENT, "mg_matmul_integer_w_dev: null context");
  return integer_w(ctx, a_dev, true, a_signed, rows, K, a_zp, a_zp_len, w, nullptr, y_dev, true);
}

mg_status mg_qlinear_matmul(mg_ctx *ctx, const void *a, int32_t a_signed, const int64_t *a_shape,
                            int32_t a_rank, float a_scale, const int32_t *a_zp, int64_t a_zp_len,
                            const void *b, int32_t b_signed, const int64_t *b_shape,
                            int32_t b_rank, float b_scale, const int32_t *b_zp,
                            int64_t b_zp_len, float y_scale, int32_t y_zp, int32_t lo,
                            int32_t hi, void *y) {
  ProfScope prof_(ctx, "QLinearMatMul");
  g_last_error.clear();
  if (!ctx) return mg_fail(MG_INVALID_ARGUMENT, "mg_qlinear_matmul: null context");
  mg_requant rq;
  MG_TRY(requant_params(a_scale, b_scale, y_scale, y_zp, lo, hi, &rq));
  return integer_host(ctx, a, a_signed, a_shape, a_rank, a_zp, a_zp_len, b, b_signed, b_shape,
                      b_rank, b_zp, b_zp_len, &rq, y);
}

mg_status mg_qlinear_matmul_w(mg_ctx *ctx, const void *a, int32_t a_signed, int64_t rows,
                              int64_t K, float a_scale, const int32_t *a_zp, int64_t a_zp_len,
                              const mg_weight *w, float b_scale, float y_scale, int32_t y_zp,
                              int32_t lo, int32_t hi, void *y) {
  ProfScope prof_(ctx, "QLinearMatMul");
  g_last_error.clear();
  if (!ctx) return mg_fail(MG_INVALID_ARGUMENT, "mg_qlinear_matmul_w: null context");
  mg_requant rq;
  MG_TRY(requant_params(a_scale, b_scale, y_scale, y_zp, lo, hi, &rq));
  return integer_w(ctx, a, false, a_signed, rows, K, a_zp, a_zp_len, w, &rq, y, false);
}

mg_status mg_qlinear_matmul_w_dev(mg_ctx *ctx, const void *a_dev, int32_t a_signed, int64_t rows,
                                  int64_t K, float a_scale, const int32_t *a_zp,
                                  int64_t a_zp_len, const mg_weight *w, float b_scale,
                                  float y_scale, int32_t y_zp, int32_t lo, int32_t hi,
                                  void *y_dev) {
  ProfScope prof_(ctx, "QLinearMatMul");
  g_last_error.clear();
  if (!ctx) return mg_fail(MG_INVALID_ARGUMENT, "mg_qlinear_matmul_w_dev: null context");
  mg_requant rq;
  MG_TRY(requant_params(a_scale, b_scale, y_scale, y_zp, lo, hi, &rq));
  return integer_w(ctx, a_dev, true, a_signed, rows, K, a_zp, a_zp_len, w, &rq, y_dev, true);
}

// DynamicQuantizeLinear output consumed in place: A is uint8 and its scale
// and zero point are the words at a_scale_zp_dev (float scale, int32 zp), so
// DQL -> MatMulInteger / QLinearMatMul needs no host round trip.
mg_status mg_matmul_integer_w_dq_dev(mg_ctx *ctx, const uint8_t *a_dev, int64_t rows, int64_t K,
                                     const void *a_scale_zp_dev, const mg_weight *w,
                                     int32_t *y_dev) {
  ProfScope prof_(ctx, "MatMulInteger");
  g_last_error.clear();
  if (!ctx || !a_scale_zp_dev)
    return mg_fail(MG_INVALID_ARGUMENT, "mg_matmul_integer_w_dq_dev: null context or scale/zp");
  mg_requant rq;
  rq.quantized_out = 0;
  rq.a_zp_dev = static_cast<const int32_t *>(a_scale_zp_dev) + 1;
  return integer_w(ctx, a_dev, true, 0, rows, K, nullptr, 0, w, &rq, y_dev, true);
}

mg_status mg_qlinear_matmul_w_dq_dev(mg_ctx *ctx, const uint8_t *a_dev, int64_t rows, int64_t K,
                                     const void *a_scale_zp_dev, const mg_weight *w,
                                     float b_scale, float y_scale, int32_t y_zp, int32_t lo,
                                     int32_t hi, void *y_dev) {
  ProfScope prof_(ctx, "QLinearMatMul");
  g_last_error.clear();
  if (!ctx || !a_scale_zp_dev)
    return mg_fail(MG_INVALID_ARGUMENT, "mg_qlinear_matmul_w_dq_dev: null context or scale/zp");
  mg_requant rq;
  MG_TRY(requant_params(1.f, b_scale, y_scale, y_zp, lo, hi, &rq));
  rq.a_scale_dev = static_cast<const float *>(a_scale_zp_dev);
  rq.a_zp_dev = static_cast<const int32_t *>(a_scale_zp_dev) + 1;
  rq.b_scale = b_scale;
  rq.y_scale = y_scale;
  return integer_w(ctx, a_dev, true, 0, rows, K, nullptr, 0, w, &rq, y_dev, true);
}

// ------------------------------------------------------------------ DQL

mg_status mg_dynamic_quantize_linear_dev(mg_ctx *ctx, const float *x_dev, int64_t n,
                                         uint8_t *y_dev, void *scale_zp_dev) {
  ProfScope prof_(ctx, "DynamicQuantizeLinear");
  g_last_error.clear();
  if (!ctx || n < 0 || (n > 0 && (!x_dev || !y_dev)) || !scale_zp_dev)
    return mg_fail(MG_INVALID_ARGUMENT, "mg_dynamic_quantize_linear: invalid argument");
  MG_TRY(mg_use_device(ctx));
  const size_t ws = mg_dql_ws_bytes(n);
  MG_TRY(mg_check_control(ctx, (int64_t)ws));
  MG_TRY(mg_ws_reserve(ctx, ws));
  return mg_dql_run(ctx, x_dev, n, y_dev, scale_zp_dev, ctx->ws);
}

mg_status mg_dynamic_quantize_linear(mg_ctx *ctx, const float *x, int64_t n, uint8_t *y,
                                     float *scale, int32_t *zp) {
  ProfScope prof_(ctx, "DynamicQuantizeLinear");
  g_last_error.clear();
  if (!ctx || n < 0 || (n > 0 && (!x || !y)) || !scale || !zp)
    return mg_fail(MG_INVALID_ARGUMENT, "mg_dynamic_quantize_linear: invalid argument");
  MG_TRY(mg_use_device(ctx));
  Staging s;
  const size_t ox = s.take((size_t)n * 4), oy = s.take((size_t)n), osz = s.take(16);
  const size_t ow = s.take(mg_dql_ws_bytes(n));
  MG_TRY(mg_check_control(ctx, (int64_t)s.off));
  MG_TRY(mg_ws_reserve(ctx, s.off));
  char *base = static_cast<char *>(ctx->ws);
  if (n) MG_HIP(hipMemcpyAsync(base + ox, x, (size_t)n * 4, hipMemcpyHostToDevice, ctx->stream));
  MG_TRY(mg_dql_run(ctx, reinterpret_cast<float *>(base + ox), n,
                    reinterpret_cast<uint8_t *>(base + oy), base + osz, base + ow));
  int32_t szp[3];
  MG_HIP(hipMemcpyAsync(szp, base + osz, 12, hipMemcpyDeviceToHost, ctx->stream));
  if (n) MG_HIP(hipMemcpyAsync(y, base + oy, (size_t)n, hipMemcpyDeviceToHost, ctx->stream));
  MG_HIP(hipStreamSynchronize(ctx->stream));
  if (szp[2])
    return mg_fail(MG_UNSUPPORTED, "DynamicQuantizeLinear: non-finite input (Infinity or NaN toInt)");
  std::memcpy(scale, &szp[0], 4);
  *zp = szp[1];
  return MG_OK;
}

// ------------------------------------------------------------ fp32 ops

namespace {

struct F32Batch {
  int64_t M, K, N, batch;
  std::vector<int64_t> out_shape;
  // Inner merged batch dims run in one launch (bc); merged dims beyond
  // MG_F32_MAX_BATCH_DIMS become host loops over launches (outer_*,
  // innermost first), each launch offsetting A, B and Y by its coordinates.
  mg_f32_bcast bc;
  int64_t inner_batch = 1;
  std::vector<int64_t> outer_dim, outer_a, outer_b;
};

// numpy broadcasting of the batch dims (lib/src/onnx_ops.dart:1717-1722,
// per-batch offsets :1742-1764) as strides: output dim d steps A by
// a_bs[d] elements (0 where A's dim is 1) and B by b_bs[d].
mg_status plan_matmul_f32(const int64_t *a_shape, int32_t a_rank, const int64_t *b_shape,
                          int32_t b_rank, F32Batch *p) {
  if (!shape_ok(a_shape, a_rank) || !shape_ok(b_shape, b_rank) || a_rank < 2 || b_rank < 2)
    return mg_fail(MG_INVALID_ARGUMENT, "MatMul: operands must have rank >= 2");
  p->M = a_shape[a_rank - 2];
  p->K = a_shape[a_rank - 1];
  p->N = b_shape[b_rank - 1];
  if (b_shape[b_rank - 2] != p->K)
    return mg_fail(MG_INVALID_ARGUMENT, "MatMul inner dims mismatch: " + std::to_string(p->K) +
                                            " vs " + std::to_string(b_shape[b_rank - 2]));
  const int32_t ar = a_rank - 2, br = b_rank - 2, r = std::max(ar, br);
  std::vector<int64_t> ob(r);
  for (int32_t d = 0; d < r; d++) {
    const int64_t x = d < r - ar ? 1 : a_shape[d - (r - ar)];
    const int64_t y = d < r - br ? 1 : b_shape[d - (r - br)];
    if (x != y && x != 1 && y != 1)
      return mg_fail(MG_INVALID_ARGUMENT, "MatMul: batch dims do not broadcast");
    ob[d] = x == 1 ? y : x;
  }
  p->batch = 1;
  for (auto v : ob) p->batch *= v;
  p->out_shape = ob;
  p->out_shape.push_back(p->M);
  p->out_shape.push_back(p->N);
  p->bc = mg_f32_bcast{};
  p->inner_batch = p->batch;
  p->outer_dim.clear();
  p->outer_a.clear();
  p->outer_b.clear();
  if (p->batch > 1 && prod(b_shape, 0, br) == 1) {
    // Shared-weight collapse (lib/src/onnx_ops.dart:1728-1735).
    p->M *= p->batch;
    p->batch = p->inner_batch = 1;
    return MG_OK;
  }
  if (p->batch <= 1) return MG_OK;
  // Strides from the innermost batch dim out; size-1 output dims dropped,
  // neighbours that step both operands contiguously merged.
  std::vector<int64_t> dim, as, bs;
  int64_t sa = p->M * p->K, sb = p->K * p->N;
  for (int32_t d = r - 1; d >= 0; d--) {
    const int64_t x = d < r - ar ? 1 : a_shape[d - (r - ar)];
    const int64_t y = d < r - br ? 1 : b_shape[d - (r - br)];
    const int64_t da = x == 1 ? 0 : sa, db = y == 1 ? 0 : sb;
    sa *= x;
    sb *= y;
    if (ob[d] == 1) continue;
    if (!dim.empty() && da == as.back() * dim.back() && db == bs.back() * dim.back()) {
      dim.back() *= ob[d];
      continue;
    }
    dim.push_back(ob[d]);
    as.push_back(da);
    bs.push_back(db);
  }
  const size_t nin = std::min<size_t>(dim.size(), MG_F32_MAX_BATCH_DIMS);
  p->bc.nbd = (int32_t)nin;
  p->inner_batch = 1;
  for (size_t d = 0; d < nin; d++) {
    p->bc.dim[d] = (uint32_t)dim[d];
    p->bc.a_bs[d] = as[d];
    p->bc.b_bs[d] = bs[d];
    p->inner_batch *= dim[d];
  }
  for (size_t d = nin; d < dim.size(); d++) {
    p->outer_dim.push_back(dim[d]);
    p->outer_a.push_back(as[d]);
    p->outer_b.push_back(bs[d]);
  }
  return MG_OK;
}

// Launch-level offsets of outer launch `o` (coordinates over outer_dim,
// innermost first).
void outer_offsets(const F32Batch &p, int64_t o, int64_t *ao, int64_t *bo) {
  int64_t a = 0, b = 0;
  for (size_t d = 0; d < p.outer_dim.size(); d++) {
    const int64_t c = o % p.outer_dim[d];
    o /= p.outer_dim[d];
    a += c * p.outer_a[d];
    b += c * p.outer_b[d];
  }
  *ao = a;
  *bo = b;
}

mg_status c_strides(const int64_t *c_shape, int32_t c_rank, int64_t M, int64_t N, int64_t *rs,
                    int64_t *cs) {
  if (c_rank > 2 || !shape_ok(c_shape, c_rank))
    return mg_fail(MG_INVALID_ARGUMENT, "Gemm: C must broadcast to [M, N]");
  int64_t s0 = 1, s1 = 1;
  if (c_rank == 2) {
    s0 = c_shape[0];
    s1 = c_shape[1];
  } else if (c_rank == 1) {
    s1 = c_shape[0];
  }
  if ((s0 != 1 && s0 != M) || (s1 != 1 && s1 != N))
    return mg_fail(MG_INVALID_ARGUMENT, "Gemm: C must broadcast to [M, N]");
  *cs = s1 == 1 ? 0 : 1;
  *rs = s0 == 1 ? 0 : s1;
  return MG_OK;
}

// Runs p on device buffers: one launch per outer coordinate (a single one
// unless more than MG_F32_MAX_BATCH_DIMS merged batch dims remain); the
// batch offsets are kernel arguments, so nothing is staged.
mg_status run_f32_batched(mg_ctx *ctx, const F32Batch &p, const float *a, const float *b,
                          float *y) {
  mg_f32_problem q{};
  q.M = p.M;
  q.N = p.N;
  q.K = p.K;
  q.batch = p.inner_batch;
  q.bc = p.bc;
  q.lda = p.K;
  q.ldb = p.N;
  q.alpha = 1.f;
  q.beta = 1.f;
  const int64_t outer = p.batch / std::max<int64_t>(p.inner_batch, 1);
  for (int64_t o = 0; o < outer; o++) {
    int64_t ao = 0, bo = 0;
    outer_offsets(p, o, &ao, &bo);
    MG_TRY(mg_f32_run(ctx, q, a + ao, b + bo, y + o * p.inner_batch * p.M * p.N));
  }
  return MG_OK;
}

}  // namespace

mg_status mg_matmul_f32_output_shape(const int64_t *a_shape, int32_t a_rank,
                                     const int64_t *b_shape, int32_t b_rank, int64_t *y_shape,
                                     int32_t *y_rank) {
  g_last_error.clear();
  if (!y_shape || !y_rank)
    return mg_fail(MG_INVALID_ARGUMENT, "mg_matmul_f32_output_shape: null output");
  F32Batch p;
  MG_TRY(plan_matmul_f32(a_shape, a_rank, b_shape, b_rank, &p));
  *y_rank = (int32_t)p.out_shape.size();
  for (size_t i = 0; i < p.out_shape.size(); i++) y_shape[i] = p.out_shape[i];
  return MG_OK;
}

mg_status mg_matmul_f32_batch_offsets(const int64_t *a_shape, int32_t a_rank,
                                      const int64_t *b_shape, int32_t b_rank, int64_t first,
                                      int64_t count, int64_t *a_off, int64_t *b_off,
                                      int64_t *batches) {
  g_last_error.clear();
  F32Batch p;
  MG_TRY(plan_matmul_f32(a_shape, a_rank, b_shape, b_rank, &p));
  if (batches) *batches = p.batch;
  if (first < 0 || count < 0 || first + count > p.batch)
    return mg_fail(MG_INVALID_ARGUMENT, "mg_matmul_f32_batch_offsets: batch range out of bounds");
  if (count && (!a_off || !b_off))
    return mg_fail(MG_INVALID_ARGUMENT, "mg_matmul_f32_batch_offsets: null output");
  const int64_t ib = std::max<int64_t>(p.inner_batch, 1);
  for (int64_t z = first; z < first + count; z++) {
    int64_t ao = 0, bo = 0, ai = 0, bi = 0;
    outer_offsets(p, z / ib, &ao, &bo);
    mg_f32_batch_offsets(p.bc, (uint32_t)(z % ib), &ai, &bi);
    a_off[z - first] = ao + ai;
    b_off[z - first] = bo + bi;
  }
  return MG_OK;
}

mg_status mg_matmul_f32(mg_ctx *ctx, const float *a, const int64_t *a_shape, int32_t a_rank,
                        const float *b, const int64_t *b_shape, int32_t b_rank, float *y) {
  ProfScope prof_(ctx, "MatMul");
  g_last_error.clear();
  if (!ctx) return mg_fail(MG_INVALID_ARGUMENT, "mg_matmul_f32: null context");
  F32Batch p;
  MG_TRY(plan_matmul_f32(a_shape, a_rank, b_shape, b_rank, &p));
  const int64_t ny = p.batch * p.M * p.N;
  if (ny == 0) return MG_OK;
  const int64_t na = prod(a_shape, 0, a_rank), nb = prod(b_shape, 0, b_rank);
  if ((!a && na) || (!b && nb) || !y) return mg_fail(MG_INVALID_ARGUMENT, "MatMul: null buffer");
  MG_TRY(mg_use_device(ctx));
  Staging s;
  const size_t oa = s.take((size_t)na * 4), ob = s.take((size_t)nb * 4), oy = s.take((size_t)ny * 4);
  MG_TRY(mg_check_control(ctx, (int64_t)s.off));
  MG_TRY(mg_ws_reserve(ctx, s.off));
  char *base = static_cast<char *>(ctx->ws);
  if (na) MG_HIP(hipMemcpyAsync(base + oa, a, (size_t)na * 4, hipMemcpyHostToDevice, ctx->stream));
  if (nb) MG_HIP(hipMemcpyAsync(base + ob, b, (size_t)nb * 4, hipMemcpyHostToDevice, ctx->stream));
  MG_TRY(run_f32_batched(ctx, p, reinterpret_cast<float *>(base + oa),
                         reinterpret_cast<float *>(base + ob), reinterpret_cast<float *>(base + oy)));
  MG_HIP(hipMemcpyAsync(y, base + oy, (size_t)ny * 4, hipMemcpyDeviceToHost, ctx->stream));
  MG_HIP(hipStreamSynchronize(ctx->stream));
  return MG_OK;
}

mg_status mg_matmul_f64acc(mg_ctx *ctx, const double *a, const int64_t *a_shape, int32_t a_rank,
                           const double *b, const int64_t *b_shape, int32_t b_rank, float *y) {
  ProfScope prof_(ctx, "MatMul");
  g_last_error.clear();
  if (!ctx) return mg_fail(MG_INVALID_ARGUMENT, "mg_matmul_f64acc: null context");
  F32Batch p;
  MG_TRY(plan_matmul_f32(a_shape, a_rank, b_shape, b_rank, &p));
  const int64_t ny = p.batch * p.M * p.N;
  if (ny == 0) return MG_OK;
  const int64_t na = prod(a_shape, 0, a_rank), nb = prod(b_shape, 0, b_rank);
  if ((!a && na) || (!b && nb) || !y) return mg_fail(MG_INVALID_ARGUMENT, "MatMul: null buffer");
  MG_TRY(mg_use_device(ctx));
  Staging s;
  const size_t oa = s.take((size_t)na * 8), ob = s.take((size_t)nb * 8), oy = s.take((size_t)ny * 4);
  MG_TRY(mg_check_control(ctx, (int64_t)s.off));
  MG_TRY(mg_ws_reserve(ctx, s.off));
  char *base = static_cast<char *>(ctx->ws);
  if (na) MG_HIP(hipMemcpyAsync(base + oa, a, (size_t)na * 8, hipMemcpyHostToDevice, ctx->stream));
  if (nb) MG_HIP(hipMemcpyAsync(base + ob, b, (size_t)nb * 8, hipMemcpyHostToDevice, ctx->stream));
  mg_f32_problem q{};
  q.M = p.M;
  q.N = p.N;
  q.K = p.K;
  q.batch = p.inner_batch;
  q.bc = p.bc;
  const double *ad = reinterpret_cast<const double *>(base + oa);
  const double *bd = reinterpret_cast<const double *>(base + ob);
  float *yd = reinterpret_cast<float *>(base + oy);
  const int64_t outer = p.batch / std::max<int64_t>(p.inner_batch, 1);
  for (int64_t o = 0; o < outer; o++) {
    int64_t ao = 0, bo = 0;
    outer_offsets(p, o, &ao, &bo);
    MG_TRY(mg_f64acc_run(ctx, q, ad + ao, bd + bo, yd + o * p.inner_batch * p.M * p.N));
  }
  MG_HIP(hipMemcpyAsync(y, yd, (size_t)ny * 4, hipMemcpyDeviceToHost, ctx->stream));
  MG_HIP(hipStreamSynchronize(ctx->stream));
  return MG_OK;
}

mg_status mg_matmul_f32_dev(mg_ctx *ctx, const float *a_dev, const int64_t *a_shape,
                            int32_t a_rank, const float *b_dev, const int64_t *b_shape,
                            int32_t b_rank, float *y_dev) {
  ProfScope prof_(ctx, "MatMul");
  g_last_error.clear();
  if (!ctx) return mg_fail(MG_INVALID_ARGUMENT, "mg_matmul_f32_dev: null context");
  F32Batch p;
  MG_TRY(plan_matmul_f32(a_shape, a_rank, b_shape, b_rank, &p));
  if (p.batch * p.M * p.N == 0) return MG_OK;
  const int64_t na = prod(a_shape, 0, a_rank), nb = prod(b_shape, 0, b_rank);
  if ((!a_dev && na) || (!b_dev && nb) || !y_dev)
    return mg_fail(MG_INVALID_ARGUMENT, "MatMul: null buffer");
  MG_TRY(mg_use_device(ctx));
  MG_TRY(mg_check_control(ctx, 0));
  return run_f32_batched(ctx, p, a_dev, b_dev, y_dev);
}

mg_status mg_gemm_f32(mg_ctx *ctx, const float *a, const int64_t *a_shape, const float *b,
                      const int64_t *b_shape, int32_t trans_a, int32_t trans_b, float alpha,
                      float beta, const float *c, const int64_t *c_shape, int32_t c_rank,
                      float *y) {
  ProfScope prof_(ctx, "Gemm");
  g_last_error.clear();
  if (!ctx || !a_shape || !b_shape) return mg_fail(MG_INVALID_ARGUMENT, "mg_gemm_f32: null argument");
  if (!shape_ok(a_shape, 2) || !shape_ok(b_shape, 2))
    return mg_fail(MG_INVALID_ARGUMENT, "Gemm: invalid operand shape");
  const int64_t M = trans_a ? a_shape[1] : a_shape[0], K = trans_a ? a_shape[0] : a_shape[1];
  const int64_t Kb = trans_b ? b_shape[1] : b_shape[0], N = trans_b ? b_shape[0] : b_shape[1];
  if (K != Kb)
    return mg_fail(MG_INVALID_ARGUMENT, "MatMul inner dims mismatch: " + std::to_string(K) +
                                            " vs " + std::to_string(Kb));
  mg_f32_problem q{};
  q.M = M;
  q.N = N;
  q.K = K;
  q.batch = 1;
  q.lda = a_shape[1];
  q.ldb = b_shape[1];
  q.trans_a = trans_a;
  q.trans_b = trans_b;
  q.alpha = alpha;
  q.beta = beta;
  int64_t nc = 0;
  if (c) {
    MG_TRY(c_strides(c_shape, c_rank, M, N, &q.c_rs, &q.c_cs));
    nc = prod(c_shape, 0, c_rank);
  }
  if (M * N == 0) return MG_OK;
  if (!a || !b || !y) return mg_fail(MG_INVALID_ARGUMENT, "Gemm: null buffer");
  MG_TRY(mg_use_device(ctx));
  Staging s;
  const size_t oa = s.take((size_t)(M * K) * 4), ob = s.take((size_t)(K * N) * 4);
  const size_t oc = s.take((size_t)nc * 4), oy = s.take((size_t)(M * N) * 4);
  MG_TRY(mg_check_control(ctx, (int64_t)s.off));
  MG_TRY(mg_ws_reserve(ctx, s.off));
  char *base = static_cast<char *>(ctx->ws);
  MG_HIP(hipMemcpyAsync(base + oa, a, (size_t)(M * K) * 4, hipMemcpyHostToDevice, ctx->stream));
  MG_HIP(hipMemcpyAsync(base + ob, b, (size_t)(K * N) * 4, hipMemcpyHostToDevice, ctx->stream));
  if (c) {
    MG_HIP(hipMemcpyAsync(base + oc, c, (size_t)nc * 4, hipMemcpyHostToDevice, ctx->stream));
    q.c = reinterpret_cast<const float *>(base + oc);
  }
  MG_TRY(mg_f32_run(ctx, q, reinterpret_cast<float *>(base + oa),
                    reinterpret_cast<float *>(base + ob), reinterpret_cast<float *>(base + oy)));
  MG_HIP(hipMemcpyAsync(y, base + oy, (size_t)(M * N) * 4, hipMemcpyDeviceToHost, ctx->stream));
  MG_HIP(hipStreamSynchronize(ctx->stream));
  return MG_OK;
}

namespace {
mg_status gemm_w(mg_ctx *ctx, const float *a, bool a_dev_ptr, int64_t rows, int64_t K,
                 const mg_weight *w, float alpha, float beta, const float *c, bool c_dev_ptr,
                 const int64_t *c_shape, int32_t c_rank, float *y, bool y_dev_ptr) {
  if (!w || w->kind != MG_W_F32) return mg_fail(MG_INVALID_ARGUMENT, "Gemm: not an fp32 weight");
  if (rows < 0 || K != w->K)
    return mg_fail(MG_INVALID_ARGUMENT, "MatMul inner dims mismatch: " + std::to_string(K) +
                                            " vs " + std::to_string(w->K));
  mg_f32_problem q{};
  q.M = rows;
  q.N = w->N;
  q.K = K;
  q.batch = 1;
  q.lda = K;
  q.ldb = K;
  q.trans_b = 1;  // the weight is stored [N][K]
  q.alpha = alpha;
  q.beta = beta;
  int64_t nc = 0;
  if (c) {
    MG_TRY(c_strides(c_shape, c_rank, rows, w->N, &q.c_rs, &q.c_cs));
    nc = prod(c_shape, 0, c_rank);
  }
  if (rows * w->N == 0) return MG_OK;
  if (!a || !y) return mg_fail(MG_INVALID_ARGUMENT, "Gemm: null buffer");
  MG_TRY(mg_use_device(ctx));
  Staging s;
  const size_t oa = a_dev_ptr ? 0 : s.take((size_t)(rows * K) * 4);
  const size_t oc = (c && !c_dev_ptr) ? s.take((size_t)nc * 4) : 0;
  const size_t oy = y_dev_ptr ? 0 : s.take((size_t)(rows * w->N) * 4);
  q.kspl = mg_f32_ksplit(rows, K, 1);
  // Partials of at most 64 MiB: wider weights run in column chunks.
  if (q.kspl > 1)
    q.part_cols = std::min<int64_t>(
        w->N, std::max<int64_t>(64, ((64ll << 20) / ((int64_t)q.kspl * rows * 4)) / 64 * 64));
  const size_t op = q.kspl > 1 ? s.take((size_t)q.kspl * rows * q.part_cols * 4) : 0;
  MG_TRY(mg_check_control(ctx, (int64_t)s.off));
  MG_TRY(mg_ws_reserve(ctx, s.off));
  char *base = static_cast<char *>(ctx->ws);
  if (q.kspl > 1) q.part = reinterpret_cast<float *>(base + op);
  const float *ad = a;
  float *yd = y;
  if (!a_dev_ptr) {
    MG_HIP(hipMemcpyAsync(base + oa, a, (size_t)(rows * K) * 4, hipMemcpyHostToDevice, ctx->stream));
    ad = reinterpret_cast<const float *>(base + oa);
  }
  if (c) {
    if (!c_dev_ptr) {
      MG_HIP(hipMemcpyAsync(base + oc, c, (size_t)nc * 4, hipMemcpyHostToDevice, ctx->stream));
      q.c = reinterpret_cast<const float *>(base + oc);
    } else {
      q.c = c;
    }
  }
  if (!y_dev_ptr) yd = reinterpret_cast<float *>(base + oy);
  MG_TRY(mg_f32_run(ctx, q, ad, w->f32.b, yd));
  if (!y_dev_ptr) {
    MG_HIP(hipMemcpyAsync(y, yd, (size_t)(rows * w->N) * 4, hipMemcpyDeviceToHost, ctx->stream));
    MG_HIP(hipStreamSynchronize(ctx->stream));
  }
  return MG_OK;
}
}  // namespace

mg_status mg_gemm_f32_w(mg_ctx *ctx, const float *a, int64_t rows, int64_t K, const mg_weight *w,
                        float alpha, float beta, const float *c, const int64_t *c_shape,
                        int32_t c_rank, float *y) {
  ProfScope prof_(ctx, "Gemm");
  g_last_error.clear();
  if (!ctx) return mg_fail(MG_INVALID_ARGUMENT, "mg_gemm_f32_w: null context");
  return gemm_w(ctx, a, false, rows, K, w, alpha, beta, c, false, c_shape, c_rank, y, false);
}

mg_status mg_gemm_f32_w_dev(mg_ctx *ctx, const float *a_dev, int64_t rows, int64_t K,
                            const mg_weight *w, float alpha, float beta, const float *c_dev,
                            const int64_t *c_shape, int32_t c_rank, float *y_dev) {
  ProfScope prof_(ctx, "Gemm");
  g_last_error.clear();
  if (!ctx) return mg_fail(MG_INVALID_ARGUMENT, "mg_gemm_f32_w_dev: null context");
  return gemm_w(ctx, a_dev, true, rows, K, w, alpha, beta, c_dev, true, c_shape, c_rank, y_dev,
                true);
}

}  // extern "C"

// ------------------------------------------------------------ attention

namespace {

// Right-aligned broadcast of two shapes; false if they do not broadcast.
bool bcast(const std::vector<int64_t> &x, const std::vector<int64_t> &y,
           std::vector<int64_t> *out) {
  const size_t r = std::max(x.size(), y.size());
  out->assign(r, 1);
  for (size_t d = 0; d < r; d++) {
    const int64_t xd = d < r - x.size() ? 1 : x[d - (r - x.size())];
    const int64_t yd = d < r - y.size() ? 1 : y[d - (r - y.size())];
    if (xd != yd && xd != 1 && yd != 1) return false;
    (*out)[d] = xd == 1 ? yd : xd;
  }
  return true;
}

// Element strides, over the output batch dims `ob`, of an operand whose
// leading dims `xb` (right-aligned to `ab`, itself right-aligned to `ob`)
// are laid out contiguously with `inner` elements per batch entry: 0 where
// either shape has size 1 or the dim is absent.
void batch_strides(const std::vector<int64_t> &ob, const std::vector<int64_t> &ab,
                   const std::vector<int64_t> &xb, int64_t inner, int64_t *out) {
  std::vector<int64_t> xs(xb.size());
  int64_t s = inner;
  for (size_t d = xb.size(); d-- > 0;) {
    xs[d] = xb[d] == 1 ? 0 : s;
    s *= xb[d];
  }
  for (size_t d = 0; d < ob.size(); d++) {
    out[d] = 0;
    const int64_t da = (int64_t)d - (int64_t)(ob.size() - ab.size());
    if (da < 0 || ab[(size_t)da] == 1) continue;
    const int64_t dx = da - (int64_t)(ab.size() - xb.size());
    if (dx >= 0) out[d] = xs[(size_t)dx];
  }
}

bool fits_lane_offsets(const mg_attn_problem &p) {
  // Lane parts of the kernel's byte offsets (32 rows/keys and 128 dims per
  // stride, 4 bytes each) stay below 2^31, the kernel's out-of-range marker.
  const int64_t lim = (int64_t)1 << 28;
  for (int64_t s : {p.k_ts, p.k_ds, p.v_ts, p.v_ds, p.m_ts, p.m_qs, p.q_cs})
    if (s < 0 || s * 160 >= lim) return false;
  return true;
}

// _FusedSDPA shapes -> kernel problem (y contiguous [out batch..., S, DV]).
mg_status plan_sdpa(const int64_t *as, int32_t ar, const int64_t *bs, int32_t br,
                    const int64_t *vs, int32_t vr, const int64_t *ms, int32_t mr, float scale,
                    mg_attn_problem *p, int64_t *ny) {
  if (!shape_ok(as, ar) || !shape_ok(bs, br) || !shape_ok(vs, vr) || !shape_ok(ms, mr) ||
      ar < 2 || br < 2 || vr < 2)
    return mg_fail(MG_INVALID_ARGUMENT, "_FusedSDPA: operands need rank >= 2");
  const int64_t S = as[ar - 2], D = as[ar - 1], D2 = bs[br - 2], T = bs[br - 1];
  const int64_t T2 = vs[vr - 2], DV = vs[vr - 1];
  if (D != D2)
    return mg_fail(MG_INVALID_ARGUMENT, "MatMul inner dims mismatch: " + std::to_string(D) +
                                            " vs " + std::to_string(D2));
  if (T != T2)
    return mg_fail(MG_INVALID_ARGUMENT, "MatMul inner dims mismatch: " + std::to_string(T) +
                                            " vs " + std::to_string(T2));
  std::vector<int64_t> ab(as, as + ar - 2), bb(bs, bs + br - 2), vb(vs, vs + vr - 2), sb, ob;
  if (!bcast(ab, bb, &sb) || !bcast(sb, vb, &ob))
    return mg_fail(MG_INVALID_ARGUMENT, "MatMul: batch dims do not broadcast");
  // The mask broadcasts (right-aligned) into the score shape [sb..., S, T].
  std::vector<int64_t> sc(sb);
  sc.push_back(S);
  sc.push_back(T);
  if ((size_t)mr > sc.size())
    return mg_fail(MG_INVALID_ARGUMENT, "_FusedSDPA: mask rank exceeds the score rank");
  for (int32_t d = 0; d < mr; d++) {
    const int64_t md = ms[d], sd = sc[sc.size() - mr + d];
    if (md != 1 && md != sd)
      return mg_fail(MG_INVALID_ARGUMENT, "_FusedSDPA: mask does not broadcast to the scores");
  }
  if (ob.size() > (size_t)MG_ATTN_MAX_BATCH_DIMS)
    return mg_fail(MG_UNSUPPORTED, "_FusedSDPA: more than 4 batch dimensions");
  *p = mg_attn_problem{};
  p->nbd = (int)ob.size();
  for (size_t d = 0; d < ob.size(); d++) p->bdim[d] = ob[d];
  batch_strides(ob, sb, ab, S * D, p->q_bs);
  batch_strides(ob, sb, bb, D * T, p->k_bs);
  batch_strides(ob, ob, vb, T * DV, p->v_bs);
  std::vector<int64_t> mb(ms, ms + std::max<int32_t>(mr - 2, 0));
  const int64_t m_last = mr >= 1 ? ms[mr - 1] : 1, m_row = mr >= 2 ? ms[mr - 2] : 1;
  batch_strides(ob, sb, mb, m_last * m_row, p->m_bs);
  {
    int64_t s = S * DV;
    for (size_t d = ob.size(); d-- > 0;) {
      p->y_bs[d] = s;
      s *= ob[d];
    }
    *ny = s;
  }
  p->q_rs = D;
  p->q_cs = 1;
  p->k_ts = 1;  // b holds K^T: element (t, d) at d * T + t
  p->k_ds = T;
  p->v_ts = DV;
  p->v_ds = 1;
  p->m_qs = m_row == 1 ? 0 : m_last;
  p->m_ts = m_last == 1 ? 0 : 1;
  p->y_rs = DV;
  p->S = (int)S;
  p->T = (int)T;
  p->D = (int)D;
  p->DV = (int)DV;
  p->scale = scale;
  if (S > 0x7fffffff || T > 0x7fffffff || !fits_lane_offsets(*p))
    return mg_fail(MG_UNSUPPORTED, "_FusedSDPA: dimensions too large");
  return MG_OK;
}

// MultiHeadAttention [batch, seq, hidden] views -> kernel problem.
mg_status plan_mha(int64_t batch, int64_t seq, int64_t kv_seq, int64_t hidden, int32_t heads,
                   int32_t bias_heads, int32_t has_bias, int32_t has_scale, float scale,
                   mg_attn_problem *p) {
  if (batch < 0 || seq < 0 || kv_seq < 0 || hidden < 0 || heads <= 0 || hidden % heads != 0)
    return mg_fail(MG_INVALID_ARGUMENT,
                   "MultiHeadAttention: hidden must be a multiple of num_heads");
  if (has_bias && bias_heads != 1 && bias_heads != heads)
    return mg_fail(MG_UNSUPPORTED, "MultiHeadAttention: bias heads must be 1 or num_heads");
  const int64_t hs = hidden / heads;
  *p = mg_attn_problem{};
  p->nbd = 2;
  p->bdim[0] = batch;
  p->bdim[1] = heads;
  p->q_bs[0] = seq * hidden;
  p->q_bs[1] = hs;
  p->k_bs[0] = p->v_bs[0] = kv_seq * hidden;
  p->k_bs[1] = p->v_bs[1] = hs;
  p->y_bs[0] = seq * hidden;
  p->y_bs[1] = hs;
  if (has_bias) {
    p->m_bs[0] = (int64_t)bias_heads * seq * kv_seq;
    p->m_bs[1] = bias_heads == 1 ? 0 : seq * kv_seq;
    p->m_qs = kv_seq;
    p->m_ts = 1;
  }
  p->q_rs = p->k_ts = p->v_ts = p->y_rs = hidden;
  p->q_cs = p->k_ds = p->v_ds = 1;
  p->S = (int)seq;
  p->T = (int)kv_seq;
  p->D = p->DV = (int)hs;
  // lib/src/onnx_ops.dart:2030: scale ?? 1 / sqrt(headSize).
  p->scale = has_scale ? scale : (float)(1.0 / std::sqrt((double)hs));
  if (seq > 0x7fffffff || kv_seq > 0x7fffffff || !fits_lane_offsets(*p))
    return mg_fail(MG_UNSUPPORTED, "MultiHeadAttention: dimensions too large");
  return MG_OK;
}

mg_status run_attn_host(mg_ctx *ctx, mg_attn_problem p, const float *q, int64_t nq,
                        const float *k, int64_t nk, const float *v, int64_t nv,
                        const float *mask, int64_t nm, float *y, int64_t ny) {
  if (ny == 0) return MG_OK;
  if ((!q && nq) || (!k && nk) || (!v && nv) || !y)
    return mg_fail(MG_INVALID_ARGUMENT, "attention: null buffer");
  MG_TRY(mg_use_device(ctx));
  Staging s;
  const size_t pb = mg_attn_plan_split(ctx, &p);
  const size_t oq = s.take((size_t)nq * 4), ok = s.take((size_t)nk * 4),
               ov = s.take((size_t)nv * 4), om = s.take((size_t)nm * 4),
               oy = s.take((size_t)ny * 4), opart = s.take(pb);
  MG_TRY(mg_check_control(ctx, (int64_t)s.off));
  MG_TRY(mg_ws_reserve(ctx, s.off));
  char *base = static_cast<char *>(ctx->ws);
  if (pb) p.part = reinterpret_cast<float *>(base + opart);
  hipStream_t st = ctx->stream;
  if (nq) MG_HIP(hipMemcpyAsync(base + oq, q, (size_t)nq * 4, hipMemcpyHostToDevice, st));
  if (nk) MG_HIP(hipMemcpyAsync(base + ok, k, (size_t)nk * 4, hipMemcpyHostToDevice, st));
  if (nv) MG_HIP(hipMemcpyAsync(base + ov, v, (size_t)nv * 4, hipMemcpyHostToDevice, st));
  if (mask && nm) MG_HIP(hipMemcpyAsync(base + om, mask, (size_t)nm * 4, hipMemcpyHostToDevice, st));
  p.q = reinterpret_cast<float *>(base + oq);
  p.k = reinterpret_cast<float *>(base + ok);
  p.v = reinterpret_cast<float *>(base + ov);
  p.mask = mask ? reinterpret_cast<float *>(base + om) : nullptr;
  p.y = reinterpret_cast<float *>(base + oy);
  MG_TRY(mg_attn_run(ctx, p));
  MG_HIP(hipMemcpyAsync(y, base + oy, (size_t)ny * 4, hipMemcpyDeviceToHost, st));
  MG_HIP(hipStreamSynchronize(st));
  return MG_OK;
}

}  // namespace

mg_status mg_fused_sdpa(mg_ctx *ctx, const float *a, const int64_t *a_shape, int32_t a_rank,
                        const float *b, const int64_t *b_shape, int32_t b_rank, const float *v,
                        const int64_t *v_shape, int32_t v_rank, const float *mask,
                        const int64_t *mask_shape, int32_t mask_rank, float scale, float *y) {
  ProfScope prof_(ctx, "_FusedSDPA");
  g_last_error.clear();
  if (!ctx || !mask) return mg_fail(MG_INVALID_ARGUMENT, "mg_fused_sdpa: null context or mask");
  mg_attn_problem p;
  int64_t ny = 0;
  MG_TRY(plan_sdpa(a_shape, a_rank, b_shape, b_rank, v_shape, v_rank, mask_shape, mask_rank,
                   scale, &p, &ny));
  return run_attn_host(ctx, p, a, prod(a_shape, 0, a_rank), b, prod(b_shape, 0, b_rank), v,
                       prod(v_shape, 0, v_rank), mask, prod(mask_shape, 0, mask_rank), y, ny);
}

mg_status mg_fused_sdpa_dev(mg_ctx *ctx, const float *a_dev, const int64_t *a_shape,
                            int32_t a_rank, const float *b_dev, const int64_t *b_shape,
                            int32_t b_rank, const float *v_dev, const int64_t *v_shape,
                            int32_t v_rank, const float *mask_dev, const int64_t *mask_shape,
                            int32_t mask_rank, float scale, float *y_dev) {
  ProfScope prof_(ctx, "_FusedSDPA");
  g_last_error.clear();
  if (!ctx || !mask_dev)
    return mg_fail(MG_INVALID_ARGUMENT, "mg_fused_sdpa_dev: null context or mask");
  mg_attn_problem p;
  int64_t ny = 0;
  MG_TRY(plan_sdpa(a_shape, a_rank, b_shape, b_rank, v_shape, v_rank, mask_shape, mask_rank,
                   scale, &p, &ny));
  if (ny == 0) return MG_OK;
  MG_TRY(mg_use_device(ctx));
  const size_t pb = mg_attn_plan_split(ctx, &p);
  MG_TRY(mg_check_control(ctx, (int64_t)pb));
  if (pb) {
    MG_TRY(mg_ws_reserve(ctx, pb));
    p.part = static_cast<float *>(ctx->ws);
  }
  p.q = a_dev;
  p.k = b_dev;
  p.v = v_dev;
  p.mask = mask_dev;
  p.y = y_dev;
  return mg_attn_run(ctx, p);
}

mg_status mg_multi_head_attention(mg_ctx *ctx, const float *q, const float *k, const float *v,
                                  int64_t batch, int64_t seq, int64_t kv_seq, int64_t hidden,
                                  int32_t num_heads, const float *bias, int32_t bias_heads,
                                  int32_t has_scale, float scale, float *y) {
  ProfScope prof_(ctx, "MultiHeadAttention");
  g_last_error.clear();
  if (!ctx) return mg_fail(MG_INVALID_ARGUMENT, "mg_multi_head_attention: null context");
  mg_attn_problem p;
  MG_TRY(plan_mha(batch, seq, kv_seq, hidden, num_heads, bias_heads, bias != nullptr, has_scale,
                  scale, &p));
  return run_attn_host(ctx, p, q, batch * seq * hidden, k, batch * kv_seq * hidden, v,
                       batch * kv_seq * hidden, bias,
                       bias ? batch * (int64_t)bias_heads * seq * kv_seq : 0, y,
                       batch * seq * hidden);
}

mg_status mg_multi_head_attention_dev(mg_ctx *ctx, const float *q_dev, const float *k_dev,
                                      const float *v_dev, int64_t batch, int64_t seq,
                                      int64_t kv_seq, int64_t hidden, int32_t num_heads,
                                      const float *bias_dev, int32_t bias_heads,
                                      int32_t has_scale, float scale, float *y_dev) {
  ProfScope prof_(ctx, "MultiHeadAttention");
  g_last_error.clear();
  if (!ctx) return mg_fail(MG_INVALID_ARGUMENT, "mg_multi_head_attention_dev: null context");
  mg_attn_problem p;
  MG_TRY(plan_mha(batch, seq, kv_seq, hidden, num_heads, bias_heads, bias_dev != nullptr,
                  has_scale, scale, &p));
  if (batch * seq * hidden == 0) return MG_OK;
  MG_TRY(mg_use_device(ctx));
  const size_t pb = mg_attn_plan_split(ctx, &p);
  MG_TRY(mg_check_control(ctx, (int64_t)pb));
  if (pb) {
    MG_TRY(mg_ws_reserve(ctx, pb));
    p.part = static_cast<float *>(ctx->ws);
  }
  p.q = q_dev;
  p.k = k_dev;
  p.v = v_dev;
  p.mask = bias_dev;
  p.y = y_dev;
  return mg_attn_run(ctx, p);
}

// --------------------------------------------------------------------------
// Convolution family.

namespace {

// Spatial axes are stored right-aligned in 3 slots (depth, height, width).
constexpr int kConvSlots = 3;

mg_status conv_common(const char *op, const int64_t *xs, int32_t xr, const int64_t *ws,
                      int32_t wr, const int64_t *strides, const int64_t *dil, int32_t group,
                      mg_conv_problem *p) {
  if (xr < 3 || xr > 5 || wr != xr || !shape_ok(xs, xr) || !shape_ok(ws, wr))
    return mg_fail(MG_INVALID_ARGUMENT,
                   std::string(op) + ": x and w must have the same rank, 3 to 5");
  if (group < 1) return mg_fail(MG_INVALID_ARGUMENT, std::string(op) + ": group must be >= 1");
  const int nd = xr - 2, o = kConvSlots - nd;
  for (int a = 0; a < nd; a++) {
    const int64_t s = strides ? strides[a] : 1, d = dil ? dil[a] : 1;
    if (s < 1 || d < 1)
      return mg_fail(MG_INVALID_ARGUMENT, std::string(op) + ": strides and dilations must be >= 1");
    if (ws[2 + a] < 1)
      return mg_fail(MG_INVALID_ARGUMENT, std::string(op) + ": empty kernel");
    p->in[o + a] = xs[2 + a];
    p->ker[o + a] = ws[2 + a];
    p->str[o + a] = s;
    p->dil[o + a] = d;
  }
  p->n = xs[0];
  p->c = xs[1];
  p->group = group;
  return MG_OK;
}

mg_status conv_limits(const char *op, const mg_conv_problem &p) {
  const int64_t lim = 0x7fffffff;
  int64_t in_sp = 1, out_sp = 1;
  for (int a = 0; a < kConvSlots; a++) {
    // The kernel forms o * str + kk * dil +- pad in 32 bits.
    if (p.in[a] > lim || p.out[a] > lim || p.ker[a] > lim || p.dil[a] > lim || p.str[a] > lim ||
        std::abs(p.pad[a]) > lim / 4 ||
        (double)p.out[a] * (double)p.str[a] + (double)p.ker[a] * (double)p.dil[a] +
                (double)std::abs(p.pad[a]) > (double)lim / 2)
      return mg_fail(MG_UNSUPPORTED, std::string(op) + ": spatial size too large");
    in_sp *= p.in[a];
    out_sp *= p.out[a];
  }
  if (in_sp > lim || out_sp > lim)
    return mg_fail(MG_UNSUPPORTED, std::string(op) + ": spatial size too large");
  // The kernel forms a window origin's offset in an input plane plus a tap's
  // shift in 32 bits (padding can put both outside the plane).
  auto span = [&](int a) {
    return (double)p.in[a] + (double)std::abs(p.pad[a]) + (double)p.str[a] +
           (double)p.ker[a] * (double)p.dil[a];
  };
  if ((span(0) * (double)p.in[1] + span(1)) * (double)p.in[2] + span(2) > (double)lim)
    return mg_fail(MG_UNSUPPORTED, std::string(op) + ": spatial size too large");
  // The kernel clamps out-of-range reads to element 0 of x, which must exist.
  if (in_sp == 0 && out_sp > 0 && p.n > 0 && p.m > 0 && p.cg > 0)
    return mg_fail(MG_UNSUPPORTED, std::string(op) + ": empty spatial input with padding");
  return MG_OK;
}

// Conv geometry (lib/src/onnx_nn_ops.dart:179-245 with _resolvePads :38-87):
// w [M, C/group, kernel...]; pads [begins..., ends...]; auto_pad 0 NOTSET,
// 1 SAME_UPPER, 2 SAME_LOWER, 3 VALID.  y_shape receives x_rank values.
mg_status plan_conv(const int64_t *xs, int32_t xr, const int64_t *ws, int32_t wr,
                    const int64_t *strides, const int64_t *pads, const int64_t *dil,
                    int32_t group, int32_t auto_pad, mg_conv_problem *p, int64_t *y_shape) {
  MG_TRY(conv_common("Conv", xs, xr, ws, wr, strides, dil, group, p));
  if (auto_pad < 0 || auto_pad > 3)
    return mg_fail(MG_INVALID_ARGUMENT, "Conv: auto_pad must be 0..3");
  const int nd = xr - 2, o = kConvSlots - nd;
  p->m = ws[0];
  p->cg = ws[1];
  if (p->cg * group != p->c)
    return mg_fail(MG_INVALID_ARGUMENT, "Conv: input channels must equal w.shape[1] * group");
  if (p->m % group != 0)
    return mg_fail(MG_INVALID_ARGUMENT, "Conv: output channels must be a multiple of group");
  p->mg = p->m / group;
  for (int a = 0; a < nd; a++) {
    const int64_t in = xs[2 + a], s = p->str[o + a];
    const int64_t window = p->dil[o + a] * (ws[2 + a] - 1) + 1;
    int64_t out, pb = 0;
    if (auto_pad == 1 || auto_pad == 2) {
      out = (in + s - 1) / s;
      const int64_t total = std::max<int64_t>(0, (out - 1) * s + window - in);
      const int64_t small = total / 2;
      pb = auto_pad == 1 ? small : total - small;  // SAME_UPPER: the extra at the end
    } else if (auto_pad == 3) {
      out = (in - window) / s + 1;  // truncating, as Dart's ~/
    } else {
      pb = pads ? pads[a] : 0;
      const int64_t pe = pads ? pads[nd + a] : 0;
      if (pb < 0 || pe < 0) return mg_fail(MG_INVALID_ARGUMENT, "Conv: negative pads");
      out = (in + pb + pe - window) / s + 1;
    }
    if (out < 0) return mg_fail(MG_INVALID_ARGUMENT, "Conv: kernel larger than padded input");
    p->out[o + a] = out;
    p->pad[o + a] = pb;
  }
  p->w_ms = p->cg * prod(ws, 2, wr);
  p->w_cs = prod(ws, 2, wr);
  p->w_gs = p->mg * p->w_ms;
  y_shape[0] = p->n;
  y_shape[1] = p->m;
  for (int a = 0; a < nd; a++) y_shape[2 + a] = p->out[o + a];
  return conv_limits("Conv", *p);
}

// ConvTranspose geometry (lib/src/onnx_nn_ops.dart:818-848, :976-995):
// w [C, M/group, kernel...]; full = (in - 1) s + d (k - 1) + 1 + output_padding;
// with output_shape (its last nd entries) the pads become total = full - out,
// end = total / 2, begin = total - end; else out = full - begin - end.
mg_status plan_conv_transpose(const int64_t *xs, int32_t xr, const int64_t *ws, int32_t wr,
                              const int64_t *strides, const int64_t *pads, const int64_t *dil,
                              const int64_t *out_pad, const int64_t *out_shape,
                              int32_t out_shape_len, int32_t group, mg_conv_problem *p,
                              int64_t *y_shape) {
  MG_TRY(conv_common("ConvTranspose", xs, xr, ws, wr, strides, dil, group, p));
  const int nd = xr - 2, o = kConvSlots - nd;
  if (out_shape && out_shape_len < nd)
    return mg_fail(MG_INVALID_ARGUMENT, "ConvTranspose: output_shape needs the spatial dims");
  if (p->c % group != 0)
    return mg_fail(MG_INVALID_ARGUMENT, "ConvTranspose: input channels must be a multiple of group");
  if (ws[0] != p->c)
    return mg_fail(MG_INVALID_ARGUMENT, "ConvTranspose: w.shape[0] must equal input channels");
  p->cg = p->c / group;
  p->mg = ws[1];
  p->m = p->mg * group;
  p->trans = 1;
  for (int a = 0; a < nd; a++)  // the kernel packs three stride remainders in 10 bits each
    if (p->str[o + a] >= 1024)
      return mg_fail(MG_UNSUPPORTED, "ConvTranspose: strides of 1024 or more");
  for (int a = 0; a < nd; a++) {
    const int64_t full =
        (xs[2 + a] - 1) * p->str[o + a] + p->dil[o + a] * (ws[2 + a] - 1) + 1 +
        (out_pad ? out_pad[a] : 0);
    int64_t out, pb;
    if (out_shape) {
      out = out_shape[out_shape_len - nd + a];
      const int64_t total = full - out;
      const int64_t pe = total / 2;  // truncating, as Dart's ~/
      pb = total - pe;
    } else {
      pb = pads ? pads[a] : 0;
      out = full - pb - (pads ? pads[nd + a] : 0);
    }
    if (out < 0) return mg_fail(MG_INVALID_ARGUMENT, "ConvTranspose: negative output size");
    p->out[o + a] = out;
    p->pad[o + a] = pb;
  }
  // W[g * cg + c][m][r]
  p->w_ms = prod(ws, 2, wr);
  p->w_cs = p->mg * p->w_ms;
  p->w_gs = p->cg * p->w_cs;
  y_shape[0] = p->n;
  y_shape[1] = p->m;
  for (int a = 0; a < nd; a++) y_shape[2 + a] = p->out[o + a];
  return conv_limits("ConvTranspose", *p);
}

int64_t conv_out_count(const mg_conv_problem &p) {
  return p.n * p.m * p.out[0] * p.out[1] * p.out[2];
}
int64_t conv_x_count(const mg_conv_problem &p) { return p.n * p.c * p.in[0] * p.in[1] * p.in[2]; }
int64_t conv_w_count(const mg_conv_problem &p) {
  return p.m * p.cg * p.ker[0] * p.ker[1] * p.ker[2];
}

// Per-channel integer parameters: weight zero points (scalar or [M]) as
// floats, and the requant multipliers x_scale * w_scale[m] / y_scale in
// double (lib/src/onnx_qlinear_ops.dart:371).
mg_status conv_int_params(const char *op, const mg_conv_problem &p, const int32_t *w_zp,
                          int64_t w_zp_len, const float *w_scale, int64_t w_scale_len,
                          float x_scale, float y_scale, bool requant, std::vector<float> *wz,
                          std::vector<double> *mult) {
  if (w_zp && w_zp_len != 1 && w_zp_len != p.m)
    return mg_fail(MG_UNSUPPORTED,
                   std::string(op) + ": weight zero point must be scalar or per-output-channel");
  if (requant && (!w_scale || (w_scale_len != 1 && w_scale_len != p.m)))
    return mg_fail(MG_UNSUPPORTED,
                   std::string(op) + ": weight scale must be scalar or per-output-channel");
  wz->assign((size_t)p.m, 0.f);
  if (w_zp)
    for (int64_t c = 0; c < p.m; c++) (*wz)[c] = (float)w_zp[w_zp_len == 1 ? 0 : c];
  if (requant) {
    mult->assign((size_t)p.m, 0.0);
    for (int64_t c = 0; c < p.m; c++)
      (*mult)[c] = (double)x_scale * (double)w_scale[w_scale_len == 1 ? 0 : c] / (double)y_scale;
  }
  return MG_OK;
}

// Runs p with operands already on the device; per-channel tables go into
// the workspace at wz_off / mult_off through the pinned staging, so the host
// tables may go away on return without a wait.
mg_status conv_launch(mg_ctx *ctx, mg_conv_problem p, const std::vector<float> &wz,
                      const std::vector<double> &mult, size_t wz_off, size_t mult_off,
                      size_t phase_off) {
  char *base = static_cast<char *>(ctx->ws);
  if (!wz.empty() && !mg_conv_int8_route(p)) {
    MG_TRY(mg_h2d_table(ctx, base + wz_off, wz.data(), wz.size() * 4));
    p.w_zp = reinterpret_cast<const float *>(base + wz_off);
  }
  if (!mult.empty()) {
    MG_TRY(mg_h2d_table(ctx, base + mult_off, mult.data(), mult.size() * 8));
    p.mult = reinterpret_cast<const double *>(base + mult_off);
  }
  return mg_conv_run(ctx, p, base + phase_off);
}

// Host-pointer call: stages x, w, bias and the tables, runs, copies y back.
mg_status conv_host(mg_ctx *ctx, mg_conv_problem p, const void *x, size_t x_el, const void *w,
                    size_t w_el, const void *bias, size_t bias_bytes, void *y, size_t y_el,
                    const std::vector<float> &wz, const std::vector<double> &mult) {
  const int64_t ny = conv_out_count(p);
  if (ny == 0) return MG_OK;
  const int64_t nx = conv_x_count(p), nw = conv_w_count(p);
  if ((!x && nx) || (!w && nw) || !y) return mg_fail(MG_INVALID_ARGUMENT, "conv: null buffer");
  MG_TRY(mg_use_device(ctx));
  Staging s;
  const size_t ox = s.take((size_t)nx * x_el), ow = s.take((size_t)nw * w_el),
               ob = s.take(bias ? bias_bytes : 0), oy = s.take((size_t)ny * y_el),
               oz = s.take(wz.size() * 4), om = s.take(mult.size() * 8),
               oph = s.take(mg_conv_ws_bytes(p));
  MG_TRY(mg_check_control(ctx, (int64_t)s.off));
  MG_TRY(mg_ws_reserve(ctx, s.off));
  char *base = static_cast<char *>(ctx->ws);
  hipStream_t st = ctx->stream;
  if (nx) MG_HIP(hipMemcpyAsync(base + ox, x, (size_t)nx * x_el, hipMemcpyHostToDevice, st));
  if (nw) MG_HIP(hipMemcpyAsync(base + ow, w, (size_t)nw * w_el, hipMemcpyHostToDevice, st));
  if (bias) MG_HIP(hipMemcpyAsync(base + ob, bias, bias_bytes, hipMemcpyHostToDevice, st));
  p.x = base + ox;
  p.w = base + ow;
  p.bias = bias ? base + ob : nullptr;
  p.y = base + oy;
  MG_TRY(conv_launch(ctx, p, wz, mult, oz, om, oph));
  MG_HIP(hipMemcpyAsync(y, base + oy, (size_t)ny * y_el, hipMemcpyDeviceToHost, st));
  MG_HIP(hipStreamSynchronize(st));
  return MG_OK;
}

// Device-pointer call: only the tables are staged.
mg_status conv_dev(mg_ctx *ctx, mg_conv_problem p, const void *x, const void *w,
                   const void *bias, void *y, const std::vector<float> &wz,
                   const std::vector<double> &mult) {
  if (conv_out_count(p) == 0) return MG_OK;
  MG_TRY(mg_use_device(ctx));
  Staging s;
  const size_t oz = s.take(wz.size() * 4), om = s.take(mult.size() * 8),
               oph = s.take(mg_conv_ws_bytes(p));
  MG_TRY(mg_check_control(ctx, (int64_t)s.off));
  if (s.off) MG_TRY(mg_ws_reserve(ctx, s.off));
  p.x = x;
  p.w = w;
  p.bias = bias;
  p.y = y;
  return conv_launch(ctx, p, wz, mult, oz, om, oph);
}

void conv_int_kinds(mg_conv_problem *p, int32_t x_signed, int32_t w_signed) {
  p->xk = x_signed ? MG_CONV_I8 : MG_CONV_U8;
  p->wk = w_signed ? MG_CONV_I8 : MG_CONV_U8;
}

}  // namespace

mg_status mg_conv_output_shape(const int64_t *x_shape, int32_t x_rank, const int64_t *w_shape,
                               const int64_t *strides, const int64_t *pads,
                               const int64_t *dilations, int32_t group, int32_t auto_pad,
                               int64_t *y_shape) {
  g_last_error.clear();
  if (!y_shape) return mg_fail(MG_INVALID_ARGUMENT, "mg_conv_output_shape: null y_shape");
  mg_conv_problem p;
  return plan_conv(x_shape, x_rank, w_shape, x_rank, strides, pads, dilations, group, auto_pad,
                   &p, y_shape);
}

mg_status mg_conv_f32(mg_ctx *ctx, const float *x, const int64_t *x_shape, int32_t x_rank,
                      const float *w, const int64_t *w_shape, const float *bias,
                      const int64_t *strides, const int64_t *pads, const int64_t *dilations,
                      int32_t group, int32_t auto_pad, float *y) {
  ProfScope prof_(ctx, "Conv");
  g_last_error.clear();
  if (!ctx) return mg_fail(MG_INVALID_ARGUMENT, "mg_conv_f32: null context");
  mg_conv_problem p;
  int64_t ys[5];
  MG_TRY(plan_conv(x_shape, x_rank, w_shape, x_rank, strides, pads, dilations, group, auto_pad,
                   &p, ys));
  return conv_host(ctx, p, x, 4, w, 4, bias, (size_t)p.m * 4, y, 4, {}, {});
}

mg_status mg_conv_f32_dev(mg_ctx *ctx, const float *x_dev, const int64_t *x_shape,
                          int32_t x_rank, const float *w_dev, const int64_t *w_shape,
                          const float *bias_dev, const int64_t *strides, const int64_t *pads,
                          const int64_t *dilations, int32_t group, int32_t auto_pad,
                          float *y_dev) {
  ProfScope prof_(ctx, "Conv");
  g_last_error.clear();
  if (!ctx) return mg_fail(MG_INVALID_ARGUMENT, "mg_conv_f32_dev: null context");
  mg_conv_problem p;
  int64_t ys[5];
  MG_TRY(plan_conv(x_shape, x_rank, w_shape, x_rank, strides, pads, dilations, group, auto_pad,
                   &p, ys));
  return conv_dev(ctx, p, x_dev, w_dev, bias_dev, y_dev, {}, {});
}

mg_status mg_conv_transpose_output_shape(const int64_t *x_shape, int32_t x_rank,
                                         const int64_t *w_shape, const int64_t *strides,
                                         const int64_t *pads, const int64_t *dilations,
                                         const int64_t *output_padding,
                                         const int64_t *output_shape, int32_t output_shape_len,
                                         int32_t group, int64_t *y_shape) {
  g_last_error.clear();
  if (!y_shape) return mg_fail(MG_INVALID_ARGUMENT, "mg_conv_transpose_output_shape: null y_shape");
  mg_conv_problem p;
  return plan_conv_transpose(x_shape, x_rank, w_shape, x_rank, strides, pads, dilations,
                             output_padding, output_shape, output_shape_len, group, &p, y_shape);
}

mg_status mg_conv_transpose_f32(mg_ctx *ctx, const float *x, const int64_t *x_shape,
                                int32_t x_rank, const float *w, const int64_t *w_shape,
                                const float *bias, const int64_t *strides, const int64_t *pads,
                                const int64_t *dilations, const int64_t *output_padding,
                                const int64_t *output_shape, int32_t output_shape_len,
                                int32_t group, float *y) {
  ProfScope prof_(ctx, "ConvTranspose");
  g_last_error.clear();
  if (!ctx) return mg_fail(MG_INVALID_ARGUMENT, "mg_conv_transpose_f32: null context");
  mg_conv_problem p;
  int64_t ys[5];
  MG_TRY(plan_conv_transpose(x_shape, x_rank, w_shape, x_rank, strides, pads, dilations,
                             output_padding, output_shape, output_shape_len, group, &p, ys));
  return conv_host(ctx, p, x, 4, w, 4, bias, (size_t)p.m * 4, y, 4, {}, {});
}

mg_status mg_conv_transpose_f32_dev(mg_ctx *ctx, const float *x_dev, const int64_t *x_shape,
                                    int32_t x_rank, const float *w_dev, const int64_t *w_shape,
                                    const float *bias_dev, const int64_t *strides,
                                    const int64_t *pads, const int64_t *dilations,
                                    const int64_t *output_padding, const int64_t *output_shape,
                                    int32_t output_shape_len, int32_t group, float *y_dev) {
  ProfScope prof_(ctx, "ConvTranspose");
  g_last_error.clear();
  if (!ctx) return mg_fail(MG_INVALID_ARGUMENT, "mg_conv_transpose_f32_dev: null context");
  mg_conv_problem p;
  int64_t ys[5];
  MG_TRY(plan_conv_transpose(x_shape, x_rank, w_shape, x_rank, strides, pads, dilations,
                             output_padding, output_shape, output_shape_len, group, &p, ys));
  return conv_dev(ctx, p, x_dev, w_dev, bias_dev, y_dev, {}, {});
}

mg_status mg_conv_integer(mg_ctx *ctx, const void *x, int32_t x_signed, const int64_t *x_shape,
                          int32_t x_rank, const void *w, int32_t w_signed,
                          const int64_t *w_shape, int32_t x_zp, const int32_t *w_zp,
                          int64_t w_zp_len, const int64_t *strides, const int64_t *pads,
                          const int64_t *dilations, int32_t group, int32_t *y) {
  ProfScope prof_(ctx, "ConvInteger");
  g_last_error.clear();
  if (!ctx) return mg_fail(MG_INVALID_ARGUMENT, "mg_conv_integer: null context");
  mg_conv_problem p;
  int64_t ys[5];
  MG_TRY(plan_conv(x_shape, x_rank, w_shape, x_rank, strides, pads, dilations, group, 0, &p, ys));
  conv_int_kinds(&p, x_signed, w_signed);
  p.w_zp_host = w_zp;
  p.w_zp_len = w_zp ? w_zp_len : 0;
  p.mode = MG_CONV_OUT_I32;
  p.x_zp = x_zp;
  std::vector<float> wz;
  std::vector<double> mult;
  MG_TRY(conv_int_params("ConvInteger", p, w_zp, w_zp_len, nullptr, 0, 0.f, 1.f, false, &wz,
                         &mult));
  return conv_host(ctx, p, x, 1, w, 1, nullptr, 0, y, 4, wz, mult);
}

mg_status mg_conv_integer_dev(mg_ctx *ctx, const void *x_dev, int32_t x_signed,
                              const int64_t *x_shape, int32_t x_rank, const void *w_dev,
                              int32_t w_signed, const int64_t *w_shape, int32_t x_zp,
                              const int32_t *w_zp, int64_t w_zp_len, const int64_t *strides,
                              const int64_t *pads, const int64_t *dilations, int32_t group,
                              int32_t *y_dev) {
  ProfScope prof_(ctx, "ConvInteger");
  g_last_error.clear();
  if (!ctx) return mg_fail(MG_INVALID_ARGUMENT, "mg_conv_integer_dev: null context");
  mg_conv_problem p;
  int64_t ys[5];
  MG_TRY(plan_conv(x_shape, x_rank, w_shape, x_rank, strides, pads, dilations, group, 0, &p, ys));
  conv_int_kinds(&p, x_signed, w_signed);
  p.w_zp_host = w_zp;
  p.w_zp_len = w_zp ? w_zp_len : 0;
  p.mode = MG_CONV_OUT_I32;
  p.x_zp = x_zp;
  std::vector<float> wz;
  std::vector<double> mult;
  MG_TRY(conv_int_params("ConvInteger", p, w_zp, w_zp_len, nullptr, 0, 0.f, 1.f, false, &wz,
                         &mult));
  return conv_dev(ctx, p, x_dev, w_dev, nullptr, y_dev, wz, mult);
}

mg_status mg_qlinear_conv(mg_ctx *ctx, const void *x, int32_t x_signed, const int64_t *x_shape,
                          int32_t x_rank, float x_scale, int32_t x_zp, const void *w,
                          int32_t w_signed, const int64_t *w_shape, const float *w_scale,
                          int64_t w_scale_len, const int32_t *w_zp, int64_t w_zp_len,
                          float y_scale, int32_t y_zp, const int32_t *bias,
                          const int64_t *strides, const int64_t *pads, const int64_t *dilations,
                          int32_t group, int32_t lo, int32_t hi, uint8_t *y) {
  ProfScope prof_(ctx, "QLinearConv");
  g_last_error.clear();
  if (!ctx) return mg_fail(MG_INVALID_ARGUMENT, "mg_qlinear_conv: null context");
  if (lo > hi) return mg_fail(MG_INVALID_ARGUMENT, "QLinearConv: lo > hi");
  mg_conv_problem p;
  int64_t ys[5];
  MG_TRY(plan_conv(x_shape, x_rank, w_shape, x_rank, strides, pads, dilations, group, 0, &p, ys));
  conv_int_kinds(&p, x_signed, w_signed);
  p.w_zp_host = w_zp;
  p.w_zp_len = w_zp ? w_zp_len : 0;
  p.mode = MG_CONV_OUT_Q8;
  p.x_zp = x_zp;
  p.y_zp = y_zp;
  p.lo = lo;
  p.hi = hi;
  std::vector<float> wz;
  std::vector<double> mult;
  MG_TRY(conv_int_params("QLinearConv", p, w_zp, w_zp_len, w_scale, w_scale_len, x_scale,
                         y_scale, true, &wz, &mult));
  return conv_host(ctx, p, x, 1, w, 1, bias, (size_t)p.m * 4, y, 1, wz, mult);
}

mg_status mg_qlinear_conv_dev(mg_ctx *ctx, const void *x_dev, int32_t x_signed,
                              const int64_t *x_shape, int32_t x_rank, float x_scale,
                              int32_t x_zp, const void *w_dev, int32_t w_signed,
                              const int64_t *w_shape, const float *w_scale, int64_t w_scale_len,
                              const int32_t *w_zp, int64_t w_zp_len, float y_scale,
                              int32_t y_zp, const int32_t *bias_dev, const int64_t *strides,
                              const int64_t *pads, const int64_t *dilations, int32_t group,
                              int32_t lo, int32_t hi, uint8_t *y_dev) {
  ProfScope prof_(ctx, "QLinearConv");
  g_last_error.clear();
  if (!ctx) return mg_fail(MG_INVALID_ARGUMENT, "mg_qlinear_conv_dev: null context");
  if (lo > hi) return mg_fail(MG_INVALID_ARGUMENT, "QLinearConv: lo > hi");
  mg_conv_problem p;
  int64_t ys[5];
  MG_TRY(plan_conv(x_shape, x_rank, w_shape, x_rank, strides, pads, dilations, group, 0, &p, ys));
  conv_int_kinds(&p, x_signed, w_signed);
  p.w_zp_host = w_zp;
  p.w_zp_len = w_zp ? w_zp_len : 0;
  p.mode = MG_CONV_OUT_Q8;
  p.x_zp = x_zp;
  p.y_zp = y_zp;
  p.lo = lo;
  p.hi = hi;
  std::vector<float> wz;
  std::vector<double> mult;
  MG_TRY(conv_int_params("QLinearConv", p, w_zp, w_zp_len, w_scale, w_scale_len, x_scale,
                         y_scale, true, &wz, &mult));
  return conv_dev(ctx, p, x_dev, w_dev, bias_dev, y_dev, wz, mult);
}

// --------------------------------------------------------------------------
// GroupQueryAttention (lib/src/onnx_ops.dart:1829-2012).

namespace {

struct GqaArgs {
  int64_t batch, seq, hidden, heads, kv, past, max_pos, half_rot;
  int32_t rotary, interleaved, bias_heads, has_bias, has_scale;
  float scale, softcap;
  int32_t local_window;
};

mg_status plan_gqa(const GqaArgs &a, mg_attn_problem *p, mg_gqa_prep *g) {
  // lib/src/onnx_ops.dart:1862-1866
  if (a.softcap != 0.f || a.local_window > 0)
    return mg_fail(MG_UNSUPPORTED, "GroupQueryAttention: softcap / local_window not supported");
  if (a.batch < 0 || a.seq < 0 || a.past < 0 || a.heads <= 0 || a.kv <= 0 ||
      a.heads % a.kv != 0 || a.hidden < 0 || a.hidden % a.heads != 0)
    return mg_fail(MG_INVALID_ARGUMENT,
                   "GroupQueryAttention: hidden must be a multiple of num_heads, and num_heads "
                   "of kv_num_heads");
  const int64_t hs = a.hidden / a.heads, group = a.heads / a.kv, total = a.past + a.seq;
  if (a.rotary && (a.half_rot < 1 || 2 * a.half_rot > hs || a.past + a.seq > a.max_pos))
    return mg_fail(MG_INVALID_ARGUMENT,
                   "GroupQueryAttention: cos/sin caches must be [>= past + seq, <= head_size / 2]");
  if (a.has_bias && a.bias_heads != 1 && a.bias_heads != a.heads)
    return mg_fail(MG_UNSUPPORTED, "GroupQueryAttention: bias heads must be 1 or num_heads");
  *g = mg_gqa_prep{};
  g->batch = a.batch;
  g->seq = a.seq;
  g->heads = a.heads;
  g->kv_heads = a.kv;
  g->hs = hs;
  g->past = a.past;
  g->half_rot = a.half_rot;
  g->rotary = a.rotary;
  g->interleaved = a.interleaved;
  *p = mg_attn_problem{};
  if (a.seq == 1) {
    // One query per head (a decode step): it sees every key, so the group's
    // query heads become the rows of one problem per (batch, KV head) and
    // read that KV head's keys once.
    p->nbd = 2;
    p->bdim[0] = a.batch;
    p->bdim[1] = a.kv;
    p->q_bs[0] = p->y_bs[0] = a.hidden;
    p->q_bs[1] = p->y_bs[1] = group * hs;
    p->k_bs[0] = p->v_bs[0] = a.kv * total * hs;
    p->k_bs[1] = p->v_bs[1] = total * hs;
    p->q_rs = p->y_rs = hs;
    p->q_cs = 1;
    p->k_ts = p->v_ts = hs;
    p->k_ds = p->v_ds = 1;
    if (a.has_bias) {
      const bool one = a.bias_heads == 1;
      p->m_bs[0] = a.bias_heads * total;
      p->m_bs[1] = one ? 0 : group * total;
      p->m_qs = one ? 0 : total;
      p->m_ts = 1;
    }
    p->S = (int)group;
    p->T = (int)total;
    p->D = p->DV = (int)hs;
    p->scale = a.has_scale ? a.scale : (float)(1.0 / std::sqrt((double)hs));
    if (total > 0x7fffffff || !fits_lane_offsets(*p))
      return mg_fail(MG_UNSUPPORTED, "GroupQueryAttention: dimensions too large");
    return MG_OK;
  }
  // Batch dims (batch, kv head, query head of the group): query head
  // h = kvh * group + j shares KV head kvh (stride 0 over j).
  p->nbd = 3;
  p->bdim[0] = a.batch;
  p->bdim[1] = a.kv;
  p->bdim[2] = group;
  p->q_bs[0] = p->y_bs[0] = a.seq * a.hidden;
  p->q_bs[1] = p->y_bs[1] = group * hs;
  p->q_bs[2] = p->y_bs[2] = hs;
  p->k_bs[0] = p->v_bs[0] = a.kv * total * hs;
  p->k_bs[1] = p->v_bs[1] = total * hs;
  p->k_bs[2] = p->v_bs[2] = 0;
  p->q_rs = p->y_rs = a.hidden;
  p->q_cs = 1;
  p->k_ts = p->v_ts = hs;
  p->k_ds = p->v_ds = 1;
  if (a.has_bias) {
    const bool one = a.bias_heads == 1;
    p->m_bs[0] = a.bias_heads * a.seq * total;
    p->m_bs[1] = one ? 0 : group * a.seq * total;
    p->m_bs[2] = one ? 0 : a.seq * total;
    p->m_qs = total;
    p->m_ts = 1;
  }
  p->S = (int)a.seq;
  p->T = (int)total;
  p->D = p->DV = (int)hs;
  p->scale = a.has_scale ? a.scale : (float)(1.0 / std::sqrt((double)hs));  // :1898
  p->causal = 1;
  p->causal_off = a.past;
  if (a.seq > 0x7fffffff || total > 0x7fffffff || !fits_lane_offsets(*p))
    return mg_fail(MG_UNSUPPORTED, "GroupQueryAttention: dimensions too large");
  return MG_OK;
}

mg_status gqa_run(mg_ctx *ctx, mg_attn_problem p, mg_gqa_prep g, const float *q, float *q_rot,
                  const float *bias, float *y) {
  g.q = q;
  g.q_rot = q_rot;
  MG_TRY(mg_gqa_prep_run(ctx, g));
  p.q = g.rotary ? q_rot : q;
  p.k = g.present_k;
  p.v = g.present_v;
  p.mask = bias;
  p.y = y;
  return mg_attn_run(ctx, p);
}

}  // namespace

mg_status mg_group_query_attention(
    mg_ctx *ctx, const float *q, const float *k, const float *v, int64_t batch, int64_t seq,
    int64_t hidden, int32_t num_heads, int32_t kv_num_heads, const float *past_key,
    const float *past_value, int64_t past_len, const float *cos_cache, const float *sin_cache,
    int64_t max_pos, int64_t half_rot, int32_t do_rotary, int32_t rotary_interleaved,
    const float *attention_bias, int32_t bias_heads, int32_t has_scale, float scale,
    float softcap, int32_t local_window, float *y, float *present_key, float *present_value) {
  ProfScope prof_(ctx, "GroupQueryAttention");
  g_last_error.clear();
  if (!ctx) return mg_fail(MG_INVALID_ARGUMENT, "mg_group_query_attention: null context");
  GqaArgs a{batch, seq, hidden, num_heads, kv_num_heads, past_len, max_pos, half_rot,
            do_rotary, rotary_interleaved, bias_heads, attention_bias != nullptr, has_scale,
            scale, softcap, local_window};
  mg_attn_problem p;
  mg_gqa_prep g;
  MG_TRY(plan_gqa(a, &p, &g));
  const int64_t hs = hidden / num_heads, total = past_len + seq;
  const int64_t nq = batch * seq * hidden, nkv = batch * seq * kv_num_heads * hs;
  const int64_t npast = batch * kv_num_heads * past_len * hs;
  const int64_t npres = batch * kv_num_heads * total * hs;
  const int64_t ncs = do_rotary ? max_pos * half_rot : 0;
  const int64_t nb = attention_bias ? batch * (int64_t)bias_heads * seq * total : 0;
  if ((!q && nq) || (!k && nkv) || (!v && nkv) || (past_len && (!past_key || !past_value)) ||
      (do_rotary && (!cos_cache || !sin_cache)) || (!y && nq) ||
      (npres && (!present_key || !present_value)))
    return mg_fail(MG_INVALID_ARGUMENT, "GroupQueryAttention: null buffer");
  if (nq + npres == 0) return MG_OK;
  MG_TRY(mg_use_device(ctx));
  Staging s;
  const size_t pb = mg_attn_plan_split(ctx, &p);
  const size_t opart = s.take(pb);
  const size_t oq = s.take(nq * 4), ok = s.take(nkv * 4), ov = s.take(nkv * 4),
               opk = s.take(npast * 4), opv = s.take(npast * 4), oc = s.take(ncs * 4),
               osn = s.take(ncs * 4), ob = s.take(nb * 4), oy = s.take(nq * 4),
               ork = s.take(npres * 4), orv = s.take(npres * 4),
               oqr = s.take(do_rotary ? nq * 4 : 0);
  MG_TRY(mg_check_control(ctx, (int64_t)s.off));
  MG_TRY(mg_ws_reserve(ctx, s.off));
  char *base = static_cast<char *>(ctx->ws);
  hipStream_t st = ctx->stream;
  auto up = [&](size_t off, const float *src, int64_t n) -> mg_status {
    if (n) MG_HIP(hipMemcpyAsync(base + off, src, (size_t)n * 4, hipMemcpyHostToDevice, st));
    return MG_OK;
  };
  MG_TRY(up(oq, q, nq));
  MG_TRY(up(ok, k, nkv));
  MG_TRY(up(ov, v, nkv));
  MG_TRY(up(opk, past_key, npast));
  MG_TRY(up(opv, past_value, npast));
  MG_TRY(up(oc, cos_cache, ncs));
  MG_TRY(up(osn, sin_cache, ncs));
  MG_TRY(up(ob, attention_bias, nb));
  auto at = [&](size_t off) { return reinterpret_cast<float *>(base + off); };
  if (pb) p.part = at(opart);
  g.k = at(ok);
  g.v = at(ov);
  g.past_k = at(opk);
  g.past_v = at(opv);
  g.cos = at(oc);
  g.sin = at(osn);
  g.present_k = at(ork);
  g.present_v = at(orv);
  MG_TRY(gqa_run(ctx, p, g, at(oq), at(oqr), attention_bias ? at(ob) : nullptr, at(oy)));
  if (nq) MG_HIP(hipMemcpyAsync(y, base + oy, (size_t)nq * 4, hipMemcpyDeviceToHost, st));
  if (npres) {
    MG_HIP(hipMemcpyAsync(present_key, base + ork, (size_t)npres * 4, hipMemcpyDeviceToHost, st));
    MG_HIP(hipMemcpyAsync(present_value, base + orv, (size_t)npres * 4, hipMemcpyDeviceToHost, st));
  }
  MG_HIP(hipStreamSynchronize(st));
  return MG_OK;
}

mg_status mg_group_query_attention_dev(
    mg_ctx *ctx, const float *q_dev, const float *k_dev, const float *v_dev, int64_t batch,
    int64_t seq, int64_t hidden, int32_t num_heads, int32_t kv_num_heads,
    const float *past_key_dev, const float *past_value_dev, int64_t past_len,
    const float *cos_cache_dev, const float *sin_cache_dev, int64_t max_pos, int64_t half_rot,
    int32_t do_rotary, int32_t rotary_interleaved, const float *attention_bias_dev,
    int32_t bias_heads, int32_t has_scale, float scale, float softcap, int32_t local_window,
    float *y_dev, float *present_key_dev, float *present_value_dev) {
  ProfScope prof_(ctx, "GroupQueryAttention");
  g_last_error.clear();
  if (!ctx) return mg_fail(MG_INVALID_ARGUMENT, "mg_group_query_attention_dev: null context");
  GqaArgs a{batch, seq, hidden, num_heads, kv_num_heads, past_len, max_pos, half_rot,
            do_rotary, rotary_interleaved, bias_heads, attention_bias_dev != nullptr, has_scale,
            scale, softcap, local_window};
  mg_attn_problem p;
  mg_gqa_prep g;
  MG_TRY(plan_gqa(a, &p, &g));
  const int64_t nq = batch * seq * hidden;
  const int64_t npres = batch * kv_num_heads * (past_len + seq) * (hidden / num_heads);
  if ((past_len && (!past_key_dev || !past_value_dev)) ||
      (do_rotary && (!cos_cache_dev || !sin_cache_dev)) ||
      (npres && (!present_key_dev || !present_value_dev)))
    return mg_fail(MG_INVALID_ARGUMENT, "GroupQueryAttention: null buffer");
  if (nq + npres == 0) return MG_OK;
  MG_TRY(mg_use_device(ctx));
  const size_t pb = mg_attn_plan_split(ctx, &p);
  const size_t qrot_bytes = do_rotary ? mg_align((size_t)nq * 4) : 0;
  MG_TRY(mg_check_control(ctx, (int64_t)(qrot_bytes + pb)));
  if (qrot_bytes + pb) MG_TRY(mg_ws_reserve(ctx, qrot_bytes + pb));
  if (pb) p.part = reinterpret_cast<float *>(static_cast<char *>(ctx->ws) + qrot_bytes);
  g.k = k_dev;
  g.v = v_dev;
  g.past_k = past_key_dev;
  g.past_v = past_value_dev;
  g.cos = cos_cache_dev;
  g.sin = sin_cache_dev;
  g.present_k = present_key_dev;
  g.present_v = present_value_dev;
  return gqa_run(ctx, p, g, q_dev, do_rotary ? static_cast<float *>(ctx->ws) : nullptr,
                 attention_bias_dev, y_dev);
}

// ------------------------------------------------------- elementwise ops

namespace {

// A shape as the reference prints a Dart List<int>: "[2, 3, 4]".
std::string dart_list(const int64_t *s, int32_t r) {
  std::string o = "[";
  for (int32_t i = 0; i < r; i++) o += (i ? ", " : "") + std::to_string(s[i]);
  return o + "]";
}

}  // namespace

extern "C" {

mg_status mg_binary_f32_dev(mg_ctx *ctx, int32_t op, const float *a_dev,
                            const int64_t *a_shape, int32_t a_rank, const float *b_dev,
                            const int64_t *b_shape, int32_t b_rank, float *y_dev) {
  static const char *names[] = {"Add", "Sub", "Mul", "Div"};
  ProfScope prof_(ctx, op >= 0 && op <= 3 ? names[op] : "Elementwise");
  g_last_error.clear();
  if (!ctx || op < 0 || op > 3 || !shape_ok(a_shape, a_rank) || !shape_ok(b_shape, b_rank))
    return mg_fail(MG_INVALID_ARGUMENT, "mg_binary_f32_dev: invalid argument");
  // Right-aligned broadcast (_broadcastShape).
  const int32_t rank = std::max(a_rank, b_rank);
  std::vector<int64_t> ad(rank), bd(rank), od(rank);
  for (int32_t k = 0; k < rank; k++) {
    ad[k] = k - (rank - a_rank) >= 0 ? a_shape[k - (rank - a_rank)] : 1;
    bd[k] = k - (rank - b_rank) >= 0 ? b_shape[k - (rank - b_rank)] : 1;
    if (ad[k] == bd[k]) od[k] = ad[k];
    else if (ad[k] == 1) od[k] = bd[k];
    else if (bd[k] == 1) od[k] = ad[k];
    else
      return mg_fail(MG_INVALID_ARGUMENT, "Cannot broadcast shapes " +
                                              dart_list(a_shape, a_rank) + " and " +
                                              dart_list(b_shape, b_rank));
  }
  int64_t n = 1;
  for (int32_t k = 0; k < rank; k++) n *= od[k];
  if (n == 0) return MG_OK;
  if (!a_dev || !b_dev || !y_dev)
    return mg_fail(MG_INVALID_ARGUMENT, "mg_binary_f32_dev: null buffer");
  MG_TRY(mg_use_device(ctx));
  MG_TRY(mg_check_control(ctx, 0));
  const bool same = ad == bd;
  mg_elem_bcast s{};
  if (!same) {
    // Row-major strides of each operand over the output dims (0 where it
    // broadcasts); size-1 output dims dropped, then neighbours merged while
    // both operands stay contiguous (or both broadcast) across them.
    std::vector<int64_t> dims, sa, sb;
    int64_t ra = 1, rb = 1;
    std::vector<int64_t> fa(rank), fb(rank);
    for (int32_t k = rank - 1; k >= 0; k--) {
      fa[k] = ad[k] == 1 ? 0 : ra;
      fb[k] = bd[k] == 1 ? 0 : rb;
      ra *= ad[k];
      rb *= bd[k];
    }
    for (int32_t k = 0; k < rank; k++) {
      if (od[k] == 1) continue;
      if (!dims.empty() && sa.back() == fa[k] * od[k] && sb.back() == fb[k] * od[k]) {
        dims.back() *= od[k];
        sa.back() = fa[k];
        sb.back() = fb[k];
      } else {
        dims.push_back(od[k]);
        sa.push_back(fa[k]);
        sb.push_back(fb[k]);
      }
    }
    s.rank = (int)dims.size();
    for (int k = 0; k < s.rank; k++) {
      s.dim[k] = dims[k];
      s.sa[k] = sa[k];
      s.sb[k] = sb[k];
    }
  }
  return mg_elem_binary(ctx, op, a_dev, b_dev, y_dev, n, same, s);
}

mg_status mg_sigmoid_f32_dev(mg_ctx *ctx, const float *x_dev, int64_t n, float *y_dev) {
  ProfScope prof_(ctx, "Sigmoid");
  g_last_error.clear();
  if (!ctx || n < 0 || (n > 0 && (!x_dev || !y_dev)))
    return mg_fail(MG_INVALID_ARGUMENT, "mg_sigmoid_f32_dev: invalid argument");
  if (n == 0) return MG_OK;
  MG_TRY(mg_use_device(ctx));
  MG_TRY(mg_check_control(ctx, 0));
  return mg_elem_sigmoid(ctx, x_dev, y_dev, n);
}

}  // extern "C"

namespace {

mg_status rms_common(mg_ctx *ctx, const char *what, const float *x_dev, const int64_t *shape,
                     int32_t rank, const float *gamma_dev, int64_t gamma_len, int64_t axis,
                     int64_t *outer, int64_t *dim, int64_t *inner) {
  if (!ctx || !shape_ok(shape, rank) || rank < 1)
    return mg_fail(MG_INVALID_ARGUMENT, std::string(what) + ": invalid argument");
  const int64_t ax = axis < 0 ? axis + rank : axis;
  if (ax < 0 || ax >= rank)
    return mg_fail(MG_INVALID_ARGUMENT, std::string(what) + ": axis out of range");
  if (gamma_len != shape[rank - 1])
    return mg_fail(MG_INVALID_ARGUMENT, "RMSNorm gamma length " + std::to_string(gamma_len) +
                                            " != last dim " + std::to_string(shape[rank - 1]));
  *outer = 1;
  *inner = 1;
  for (int64_t k = 0; k < ax; k++) *outer *= shape[k];
  for (int64_t k = ax + 1; k < rank; k++) *inner *= shape[k];
  *dim = shape[ax];
  if (*outer * *dim * *inner > 0 && (!x_dev || !gamma_dev))
    return mg_fail(MG_INVALID_ARGUMENT, std::string(what) + ": null buffer");
  if (*inner == 1 && *outer > INT32_MAX)
    return mg_fail(MG_UNSUPPORTED, std::string(what) + ": more than 2^31 rows");
  return MG_OK;
}

}  // namespace

extern "C" {

mg_status mg_rms_norm_f32_dev(mg_ctx *ctx, const float *x_dev, const int64_t *shape,
                              int32_t rank, const float *gamma_dev, int64_t gamma_len,
                              int64_t axis, double epsilon, float *y_dev) {
  ProfScope prof_(ctx, "RMSNorm");
  g_last_error.clear();
  int64_t outer, dim, inner;
  MG_TRY(rms_common(ctx, "mg_rms_norm_f32_dev", x_dev, shape, rank, gamma_dev, gamma_len, axis,
                    &outer, &dim, &inner));
  if (outer * dim * inner == 0) return MG_OK;
  if (!y_dev) return mg_fail(MG_INVALID_ARGUMENT, "mg_rms_norm_f32_dev: null buffer");
  MG_TRY(mg_use_device(ctx));
  MG_TRY(mg_check_control(ctx, 0));
  return mg_elem_rms_norm(ctx, x_dev, nullptr, gamma_dev, nullptr, epsilon, outer, dim, inner,
                          shape[rank - 1], y_dev, nullptr);
}

mg_status mg_skip_rms_norm_f32_dev(mg_ctx *ctx, const float *x_dev, const float *skip_dev,
                                   const int64_t *shape, int32_t rank, const float *gamma_dev,
                                   int64_t gamma_len, const float *bias_dev, double epsilon,
                                   float *y_dev, float *sum_dev) {
  ProfScope prof_(ctx, "SkipSimplifiedLayerNormalization");
  g_last_error.clear();
  int64_t outer, dim, inner;
  MG_TRY(rms_common(ctx, "mg_skip_rms_norm_f32_dev", x_dev, shape, rank, gamma_dev, gamma_len,
                    -1, &outer, &dim, &inner));
  if (outer * dim == 0) return MG_OK;
  if (!skip_dev || !y_dev)
    return mg_fail(MG_INVALID_ARGUMENT, "mg_skip_rms_norm_f32_dev: null buffer");
  MG_TRY(mg_use_device(ctx));
  MG_TRY(mg_check_control(ctx, 0));
  return mg_elem_rms_norm(ctx, x_dev, skip_dev, gamma_dev, bias_dev, epsilon, outer, dim, 1,
                          dim, y_dev, sum_dev);
}

// The producer of a decode GEMV's input that also writes its split
// activations (at most 16 rows of at most 8192 elements; block_size: that of
// the MatMulNBits weights that will read the split).
namespace {
mg_status split_rows(const char *what, const int64_t *shape, int32_t rank, int64_t block_size,
                     void *split, int64_t *rows, int64_t *d, int64_t *kpad) {
  if (!shape_ok(shape, rank) || rank < 1 || !split || block_size < 16 ||
      (block_size & (block_size - 1)))
    return mg_fail(MG_INVALID_ARGUMENT, std::string(what) + ": invalid argument");
  *d = shape[rank - 1];
  *rows = prod(shape, 0, rank - 1);
  if (*rows > 16 || *d > 8192)
    return mg_fail(MG_INVALID_ARGUMENT, std::string(what) +
                                            ": split activations need at most 16 rows of at "
                                            "most 8192 elements");
  *kpad = mg_nbits_kpad(std::max<int64_t>(*d, 1), block_size);
  return MG_OK;
}
}  // namespace

mg_status mg_skip_rms_norm_f32_split_dev(mg_ctx *ctx, const float *x_dev, const float *skip_dev,
                                         const int64_t *shape, int32_t rank,
                                         const float *gamma_dev, int64_t gamma_len,
                                         const float *bias_dev, double epsilon, float *y_dev,
                                         float *sum_dev, int64_t block_size, void *split_dev) {
  ProfScope prof_(ctx, skip_dev ? "SkipSimplifiedLayerNormalization" : "RMSNorm");
  g_last_error.clear();
  int64_t outer, dim, inner, rows, d, kpad;
  MG_TRY(rms_common(ctx, "mg_skip_rms_norm_f32_split_dev", x_dev, shape, rank, gamma_dev,
                    gamma_len, -1, &outer, &dim, &inner));
  MG_TRY(split_rows("mg_skip_rms_norm_f32_split_dev", shape, rank, block_size, split_dev, &rows,
                    &d, &kpad));
  if (outer * dim == 0) return MG_OK;
  if (!y_dev) return mg_fail(MG_INVALID_ARGUMENT, "mg_skip_rms_norm_f32_split_dev: null buffer");
  MG_TRY(mg_use_device(ctx));
  MG_TRY(mg_check_control(ctx, 0));
  return mg_elem_rms_norm_split(ctx, x_dev, skip_dev, gamma_dev, bias_dev, epsilon, rows, d,
                                y_dev, skip_dev ? sum_dev : nullptr, kpad, split_dev);
}

}  // extern "C"
