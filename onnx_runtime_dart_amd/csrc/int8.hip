// MatMulInteger / QLinearMatMul on gfx950 int8 MFMA.
//
// Reference semantics (lib/src/onnx_qlinear_ops.dart:32-108):
//   acc[m, n] = sum_k (A[m, k] - aZp) * (B[k, n] - bZp)       exact integers
//   QLinear:  q = roundHalfEven(fl32(acc * mult)) + yZp, clamped to [lo, hi],
//             mult = fl32(fl32(aS * bS) / yS).
//
// The MFMA multiplies signed bytes, so both operands are re-centred:
//   A' = A - oa, B' = B - ob with oa/ob = 128 for uint8 and 0 for int8, and
//   (A - aZp)(B - bZp) = (A' + ca)(B' + cb), ca = oa - aZp, cb = ob - bZp:
//   acc = sum A'B' + cb * rowsum(A') + ca * colsum(B') + K * ca * cb.
// Every term is int32 arithmetic; wrap-around cancels, so the result is exact
// whenever the true value fits int32 (always for K <= 33025).
//
// Fragment layouts (v_mfma_i32_16x16x64_i8; lane = 16*g + i):
//   A: [batch][m16][k64][lane][16 B]  lane holds row i, k = 64*k64 + 16*g + 0..15
//   B: [batch][n16][k64][lane][16 B]  lane holds col i, same k
// Both come from small prepack kernels (B once on upload for weights).
#include <hip/hip_runtime.h>

#include <cmath>

#include "mg_internal.h"

namespace {

typedef int int4v __attribute__((ext_vector_type(4)));

// A (u8 or i8, [rows, K] per batch with rows = M) -> fragments, ca, rowsum.
// One workgroup per (batch, 16-row subtile).
__global__ __launch_bounds__(256) void k_i8_prep_a(
    const uint8_t *__restrict__ a, int a_signed, int64_t M, int64_t K,
    int m16n, int kq, int za_scalar, const int32_t *__restrict__ za,
    int za_len, int4v *__restrict__ frag, int32_t *__restrict__ ca,
    int32_t *__restrict__ rowsum) {
  const int64_t bi = blockIdx.y;
  const int sub = blockIdx.x;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 15, g = lane >> 4;
  const int64_t row = (int64_t)sub * 16 + r;
  const uint8_t *arow = a + (bi * M + row) * K;
  const int flip = a_signed ? 0 : 0x80;
  int s = 0;
  for (int q = wave; q < kq; q += 4) {
    union { int4v v; int8_t b[16]; } u;
    for (int e = 0; e < 16; e++) {
      const int64_t k = (int64_t)q * 64 + 16 * g + e;
      int8_t v = 0;
      if (row < M && k < K) v = (int8_t)(arow[k] ^ flip);
      u.b[e] = v;
      s += v;
    }
    frag[(((bi * m16n + sub) * kq + q) * 64) + lane] = u.v;
  }
  __shared__ int red[4][64];
  red[wave][lane] = s;
  __syncthreads();
  if (threadIdx.x < 16) {
    int t = 0;
    for (int w = 0; w < 4; w++)
      for (int gg = 0; gg < 4; gg++) t += red[w][gg * 16 + threadIdx.x];
    const int64_t rr = (int64_t)sub * 16 + threadIdx.x;
    const int64_t slot = bi * m16n * 16 + rr;
    const int oa = a_signed ? 0 : 128;
    int z = za_scalar;
    if (za && za_len > 0) z = za[rr % za_len];
    ca[slot] = oa - z;
    rowsum[slot] = t;
  }
}

// B (u8 or i8, [K, N] per batch) -> fragments; one thread per 16-byte
// fragment slot.
__global__ __launch_bounds__(256) void k_i8_prep_b(
    const uint8_t *__restrict__ b, int b_signed, int64_t K, int64_t N,
    int n16n, int kq, int4v *__restrict__ frag) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t per_batch = (int64_t)n16n * kq * 64;
  const int64_t bi = blockIdx.y;
  if (idx >= per_batch) return;
  const int lane = (int)(idx & 63);
  const int64_t t = idx >> 6;
  const int q = (int)(t % kq);
  const int64_t sub = t / kq;
  const int c = lane & 15, g = lane >> 4;
  const int64_t col = sub * 16 + c;
  const uint8_t *bb = b + bi * K * N;
  const int flip = b_signed ? 0 : 0x80;
  union { int4v v; int8_t x[16]; } u;
  for (int e = 0; e < 16; e++) {
    const int64_t k = (int64_t)q * 64 + 16 * g + e;
    u.x[e] = (col < N && k < K) ? (int8_t)(bb[k * N + col] ^ flip) : (int8_t)0;
  }
  frag[bi * per_batch + idx] = u.v;
}

// Column sums of B' and cb per column; one thread per (batch, column).
__global__ __launch_bounds__(256) void k_i8_colsum(
    const uint8_t *__restrict__ b, int b_signed, int64_t K, int64_t N,
    int64_t npad, int zb_scalar, const int32_t *__restrict__ zb, int zb_len,
    int32_t *__restrict__ colsum, int32_t *__restrict__ cb) {
  const int64_t col = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t bi = blockIdx.y;
  if (col >= npad) return;
  const int flip = b_signed ? 0 : 0x80;
  int s = 0;
  if (col < N)
    for (int64_t k = 0; k < K; k++) s += (int8_t)(b[(bi * K + k) * N + col] ^ flip);
  colsum[bi * npad + col] = s;
  int z = zb_scalar;
  if (zb && zb_len > 0 && col < N) z = zb[col % zb_len];
  cb[bi * npad + col] = (b_signed ? 0 : 128) - z;
}

// y = sum A'B' + cb*rowsum + ca*colsum + K*ca*cb; REQ: requantise to bytes.
// Workgroup: 4 waves as 2 x 2; wave tile (16*WMS) x 64.
template <int WMS, int REQ>
__global__ __launch_bounds__(256) void k_i8_gemm(
    const int4v *__restrict__ afrag, const int32_t *__restrict__ ca,
    const int32_t *__restrict__ rowsum, const int4v *__restrict__ bfrag,
    const int32_t *__restrict__ colsum, const int32_t *__restrict__ cb,
    void *__restrict__ y, int64_t M, int64_t N, int64_t K, int m16n, int n16n,
    int kq, int64_t a_bstride, int64_t b_bstride, int64_t npad_b, float mult,
    int y_zp, int lo, int hi) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave & 1, wn = wave >> 1;
  const int64_t bz = blockIdx.z;
  const int sub0 = (blockIdx.y * 2 + wm) * WMS;
  const int nsub0 = (blockIdx.x * 2 + wn) * 4;
  const int4v *ab = afrag + bz * a_bstride;
  const int4v *bb = bfrag + bz * b_bstride;
  int4v acc[WMS][4];
#pragma unroll
  for (int i = 0; i < WMS; i++)
#pragma unroll
    for (int n = 0; n < 4; n++) acc[i][n] = (int4v){0, 0, 0, 0};
  for (int q = 0; q < kq; q++) {
    int4v bf[4];
#pragma unroll
    for (int n = 0; n < 4; n++) {
      const int ns = nsub0 + n;
      bf[n] = ns < n16n ? bb[((int64_t)ns * kq + q) * 64 + lane] : (int4v){0, 0, 0, 0};
    }
#pragma unroll
    for (int i = 0; i < WMS; i++) {
      const int ms = sub0 + i;
      const int4v af = ms < m16n ? ab[((int64_t)ms * kq + q) * 64 + lane] : (int4v){0, 0, 0, 0};
#pragma unroll
      for (int n = 0; n < 4; n++)
        acc[i][n] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af, bf[n], acc[i][n], 0, 0, 0);
    }
  }
  const int cl = lane & 15, lg = lane >> 4;
  const int64_t arow_base = bz * (a_bstride / ((int64_t)kq * 64)) * 16;  // rows of this batch's A
#pragma unroll
  for (int i = 0; i < WMS; i++) {
#pragma unroll
    for (int n = 0; n < 4; n++) {
      const int64_t col = (int64_t)(nsub0 + n) * 16 + cl;
      if (col >= N) continue;
      const int32_t cs = colsum[bz * npad_b * (b_bstride ? 1 : 0) + col];
      const int32_t cbv = cb[bz * npad_b * (b_bstride ? 1 : 0) + col];
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const int64_t row = (int64_t)(sub0 + i) * 16 + 4 * lg + r;
        if (row >= M) continue;
        const int64_t slot = arow_base + row;
        const int32_t cav = ca[slot];
        const uint32_t v = (uint32_t)acc[i][n][r] + (uint32_t)cbv * (uint32_t)rowsum[slot] +
                           (uint32_t)cav * (uint32_t)cs +
                           (uint32_t)K * (uint32_t)cav * (uint32_t)cbv;
        const int32_t vi = (int32_t)v;
        const int64_t o = (bz * M + row) * N + col;
        if (REQ) {
          const float p = (float)((double)vi * (double)mult);
          int qv = (int)rintf(p) + y_zp;
          qv = qv < lo ? lo : (qv > hi ? hi : qv);
          static_cast<uint8_t *>(y)[o] = (uint8_t)qv;
        } else {
          static_cast<int32_t *>(y)[o] = vi;
        }
      }
    }
  }
}

}  // namespace

// Weight arrays (bq fragments, colsum, cb) laid out in one allocation.
size_t mg_int8_weight_ws_bytes(int64_t K, int64_t N) {
  const int64_t kq = (K + 63) / 64, n16 = (N + 15) / 16;
  return mg_align((size_t)n16 * kq * 64 * 16) + 2 * mg_align((size_t)n16 * 16 * 4);
}

static void int8_carve(mg_weight *w, void *base) {
  const int64_t kq = (w->K + 63) / 64, n16 = (w->N + 15) / 16;
  char *p = static_cast<char *>(base);
  w->i8.kpad = kq * 64;
  w->i8.npad = n16 * 16;
  w->i8.bq = reinterpret_cast<int8_t *>(p);
  p += mg_align((size_t)n16 * kq * 64 * 16);
  w->i8.colsum = reinterpret_cast<int32_t *>(p);
  p += mg_align((size_t)n16 * 16 * 4);
  w->i8.cb = reinterpret_cast<int32_t *>(p);
}

// Prepacks B already in device memory.  b_zp is a host array.
mg_status mg_int8_prepack_dev(mg_ctx *ctx, mg_weight *w, const void *b_dev,
                              int32_t b_signed, const int32_t *b_zp,
                              int64_t b_zp_len, void *ws_weight) {
  int8_carve(w, ws_weight);
  w->i8.b_signed = b_signed;
  const int64_t K = w->K, N = w->N;
  const int kq = (int)(w->i8.kpad / 64), n16 = (int)(w->i8.npad / 16);
  hipStream_t st = ctx->stream;
  int zb_scalar = 0;
  const int32_t *zb_dev = nullptr;
  int zb_len = 0;
  if (b_zp && b_zp_len == 1) {
    zb_scalar = b_zp[0];
  } else if (b_zp && b_zp_len > 1) {
    // Per-column zero points travel through the tail of the cb array region:
    // write them into cb first, then the colsum kernel reads them back.
    MG_HIP(hipMemcpyAsync(w->i8.cb, b_zp, (size_t)b_zp_len * 4, hipMemcpyHostToDevice, st));
    zb_dev = w->i8.cb;
    zb_len = (int)b_zp_len;
  }
  const int64_t slots = (int64_t)n16 * kq * 64;
  hipLaunchKernelGGL(k_i8_prep_b, dim3((unsigned)((slots + 255) / 256), 1), dim3(256), 0, st,
                     static_cast<const uint8_t *>(b_dev), b_signed, K, N, n16, kq,
                     reinterpret_cast<int4v *>(w->i8.bq));
  MG_TRY(mg_launch_check("k_i8_prep_b"));
  hipLaunchKernelGGL(k_i8_colsum, dim3((unsigned)((w->i8.npad + 255) / 256), 1), dim3(256), 0,
                     st, static_cast<const uint8_t *>(b_dev), b_signed, K, N, w->i8.npad,
                     zb_scalar, zb_dev, zb_len, w->i8.colsum, w->i8.cb);
  return mg_launch_check("k_i8_colsum");
}

mg_status mg_int8_upload(mg_ctx *ctx, mg_weight *w, const void *b,
                         int32_t b_signed, const int32_t *b_zp,
                         int64_t b_zp_len) {
  const size_t bytes = mg_int8_weight_ws_bytes(w->K, w->N);
  void *base = nullptr;
  MG_HIP(hipMalloc(&base, bytes));
  w->device_bytes = (int64_t)bytes;
  void *raw = nullptr;
  const size_t raw_bytes = (size_t)(w->K * w->N);
  hipError_t e = hipMalloc(&raw, raw_bytes ? raw_bytes : 1);
  if (e != hipSuccess) {
    (void)hipFree(base);
    return mg_fail(MG_OUT_OF_MEMORY, "mg_weight_int8_create: staging allocation failed");
  }
  mg_status st = MG_OK;
  if (hipMemcpy(raw, b, raw_bytes, hipMemcpyHostToDevice) != hipSuccess)
    st = mg_fail(MG_DEVICE_ERROR, "mg_weight_int8_create: upload failed");
  if (st == MG_OK) st = mg_int8_prepack_dev(ctx, w, raw, b_signed, b_zp, b_zp_len, base);
  if (st == MG_OK && hipStreamSynchronize(ctx->stream) != hipSuccess)
    st = mg_fail(MG_DEVICE_ERROR, "mg_weight_int8_create: prepack failed");
  (void)hipFree(raw);
  if (st != MG_OK) (void)hipFree(base);
  return st;
}

void mg_int8_free(mg_weight *w) {
  if (w->i8.bq) (void)hipFree(w->i8.bq);
  w->i8 = mg_int8_dev{};
}

size_t mg_int8_ws_bytes(const mg_weight *w, int64_t rows) {
  const int64_t kq = w->i8.kpad / 64;
  const int64_t m16 = (rows + 15) / 16;
  return mg_align((size_t)m16 * kq * 64 * 16) + 2 * mg_align((size_t)m16 * 16 * 4) + 256;
}

// Shared launcher.  a_batch/b_batch: 1 or batch; rows per batch = M.
static mg_status int8_launch(mg_ctx *ctx, const int8_t *bq, const int32_t *colsum,
                             const int32_t *cb, int64_t npad, int64_t b_batch,
                             const void *a_dev, int32_t a_signed, int64_t a_batch,
                             int64_t M, int64_t N, int64_t K, const int32_t *a_zp,
                             int64_t a_zp_len, const mg_requant *rq, void *y_dev,
                             void *ws) {
  const int64_t kq = (K + 63) / 64, m16 = (M + 15) / 16, n16 = npad / 16;
  hipStream_t st = ctx->stream;
  char *p = static_cast<char *>(ws);
  int4v *afrag = reinterpret_cast<int4v *>(p);
  p += mg_align((size_t)a_batch * m16 * kq * 64 * 16);
  int32_t *ca = reinterpret_cast<int32_t *>(p);
  p += mg_align((size_t)a_batch * m16 * 16 * 4);
  int32_t *rowsum = reinterpret_cast<int32_t *>(p);
  p += mg_align((size_t)a_batch * m16 * 16 * 4);
  int32_t *za_dev = reinterpret_cast<int32_t *>(p);
  int za_scalar = 0, za_len = 0;
  if (a_zp && a_zp_len == 1) {
    za_scalar = a_zp[0];
  } else if (a_zp && a_zp_len > 1) {
    MG_HIP(hipMemcpyAsync(za_dev, a_zp, (size_t)a_zp_len * 4, hipMemcpyHostToDevice, st));
    za_len = (int)a_zp_len;
  }
  hipLaunchKernelGGL(k_i8_prep_a, dim3((unsigned)m16, (unsigned)a_batch), dim3(256), 0, st,
                     static_cast<const uint8_t *>(a_dev), a_signed, M, K, (int)m16, (int)kq,
                     za_scalar, za_len ? za_dev : nullptr, za_len, afrag, ca, rowsum);
  MG_TRY(mg_launch_check("k_i8_prep_a"));
  const int64_t batch = a_batch > b_batch ? a_batch : b_batch;
  const int wms = M <= 16 ? 1 : 2;
  const dim3 grid((unsigned)((n16 + 7) / 8), (unsigned)((m16 + 2 * wms - 1) / (2 * wms)),
                  (unsigned)batch);
  const int64_t a_bs = a_batch > 1 ? m16 * kq * 64 : 0;
  const int64_t b_bs = b_batch > 1 ? n16 * kq * 64 : 0;
  const float mult = rq ? rq->mult : 0.f;
  const int yz = rq ? rq->y_zp : 0, lo = rq ? rq->lo : 0, hi = rq ? rq->hi : 0;
#define MG_I8_ARGS                                                                  \
  afrag, ca, rowsum, reinterpret_cast<const int4v *>(bq), colsum, cb, y_dev, M, N, K, \
      (int)m16, (int)n16, (int)kq, a_bs, b_bs, npad, mult, yz, lo, hi
  if (wms == 1) {
    if (rq) hipLaunchKernelGGL((k_i8_gemm<1, 1>), grid, dim3(256), 0, st, MG_I8_ARGS);
    else hipLaunchKernelGGL((k_i8_gemm<1, 0>), grid, dim3(256), 0, st, MG_I8_ARGS);
  } else {
    if (rq) hipLaunchKernelGGL((k_i8_gemm<2, 1>), grid, dim3(256), 0, st, MG_I8_ARGS);
    else hipLaunchKernelGGL((k_i8_gemm<2, 0>), grid, dim3(256), 0, st, MG_I8_ARGS);
  }
#undef MG_I8_ARGS
  return mg_launch_check("k_i8_gemm");
}

mg_status mg_int8_run(mg_ctx *ctx, const mg_weight *w, const void *a_dev,
                      int32_t a_signed, int64_t rows, const int32_t *a_zp,
                      int64_t a_zp_len, const mg_requant *rq, void *y_dev,
                      void *ws) {
  return int8_launch(ctx, w->i8.bq, w->i8.colsum, w->i8.cb, w->i8.npad, 1, a_dev, a_signed, 1,
                     rows, w->N, w->K, a_zp, a_zp_len, rq, y_dev, ws);
}

// Runtime (non-weight) batched form: B already prepacked per batch into
// `bw` by mg_int8_prepack_batched.
mg_status mg_int8_run_batched(mg_ctx *ctx, const void *a_dev, int32_t a_signed,
                              int64_t a_batch, const void *b_dev,
                              int32_t b_signed, int64_t b_batch, int64_t M,
                              int64_t K, int64_t N, const int32_t *a_zp,
                              int64_t a_zp_len, const int32_t *b_zp,
                              int64_t b_zp_len, const mg_requant *rq,
                              void *y_dev, void *ws);

mg_status mg_int8_run_batched(mg_ctx *ctx, const void *a_dev, int32_t a_signed,
                              int64_t a_batch, const void *b_dev,
                              int32_t b_signed, int64_t b_batch, int64_t M,
                              int64_t K, int64_t N, const int32_t *a_zp,
                              int64_t a_zp_len, const int32_t *b_zp,
                              int64_t b_zp_len, const mg_requant *rq,
                              void *y_dev, void *ws) {
  const int64_t kq = (K + 63) / 64, n16 = (N + 15) / 16, npad = n16 * 16;
  hipStream_t st = ctx->stream;
  char *p = static_cast<char *>(ws);
  int8_t *bq = reinterpret_cast<int8_t *>(p);
  p += mg_align((size_t)b_batch * n16 * kq * 64 * 16);
  int32_t *colsum = reinterpret_cast<int32_t *>(p);
  p += mg_align((size_t)b_batch * npad * 4);
  int32_t *cb = reinterpret_cast<int32_t *>(p);
  p += mg_align((size_t)b_batch * npad * 4);
  int32_t *zb_dev = reinterpret_cast<int32_t *>(p);
  p += mg_align((size_t)(N + 1) * 4);
  int zb_scalar = 0, zb_len = 0;
  if (b_zp && b_zp_len == 1) {
    zb_scalar = b_zp[0];
  } else if (b_zp && b_zp_len > 1) {
    MG_HIP(hipMemcpyAsync(zb_dev, b_zp, (size_t)b_zp_len * 4, hipMemcpyHostToDevice, st));
    zb_len = (int)b_zp_len;
  }
  const int64_t slots = n16 * kq * 64;
  hipLaunchKernelGGL(k_i8_prep_b, dim3((unsigned)((slots + 255) / 256), (unsigned)b_batch),
                     dim3(256), 0, st, static_cast<const uint8_t *>(b_dev), b_signed, K, N,
                     (int)n16, (int)kq, reinterpret_cast<int4v *>(bq));
  MG_TRY(mg_launch_check("k_i8_prep_b"));
  hipLaunchKernelGGL(k_i8_colsum, dim3((unsigned)((npad + 255) / 256), (unsigned)b_batch),
                     dim3(256), 0, st, static_cast<const uint8_t *>(b_dev), b_signed, K, N,
                     npad, zb_scalar, zb_len ? zb_dev : nullptr, zb_len, colsum, cb);
  MG_TRY(mg_launch_check("k_i8_colsum"));
  return int8_launch(ctx, bq, colsum, cb, npad, b_batch, a_dev, a_signed, a_batch, M, N, K,
                     a_zp, a_zp_len, rq, y_dev, p);
}

size_t mg_int8_batched_ws_bytes(int64_t a_batch, int64_t b_batch, int64_t M,
                                int64_t K, int64_t N);
size_t mg_int8_batched_ws_bytes(int64_t a_batch, int64_t b_batch, int64_t M,
                                int64_t K, int64_t N) {
  const int64_t kq = (K + 63) / 64, n16 = (N + 15) / 16, npad = n16 * 16;
  const int64_t m16 = (M + 15) / 16;
  size_t b = mg_align((size_t)b_batch * n16 * kq * 64 * 16) + 2 * mg_align((size_t)b_batch * npad * 4) +
             mg_align((size_t)(N + 1) * 4);
  size_t a = mg_align((size_t)a_batch * m16 * kq * 64 * 16) + 2 * mg_align((size_t)a_batch * m16 * 16 * 4) +
             mg_align((size_t)(a_batch * M + 1) * 4);
  return b + a + 256;
}
