// DynamicQuantizeLinear on device (lib/src/onnx_ops.dart:3556-3583):
//   mn = min(0, min x), mx = max(0, max x)       (NaN never updates either)
//   scale = fl32((mx - mn) / 255)                 computed in f64
//   zp = roundHalfEven(clamp(fl32(-mn / scale), 0, 255))
//   y = clamp(roundHalfEven(fl32(x / scale)) + zp, 0, 255), or zp if scale==0
// fl32 of an f64 quotient of two floats equals the correctly rounded f32
// quotient, but the f64 form is kept to follow the reference literally.
// Two kernels: per-workgroup min/max partials, then every workgroup of the
// quantising kernel reduces the (few) partials itself and quantises its
// slice, so no host round trip sits between them.
#include <hip/hip_runtime.h>

#include <cmath>

#include "mg_internal.h"

namespace {

constexpr int DQL_PARTS = 512;

__global__ __launch_bounds__(256) void k_dql_partial(const float *__restrict__ x,
                                                     int64_t n, float *__restrict__ pmn,
                                                     float *__restrict__ pmx,
                                                     int *__restrict__ pbad) {
  float mn = 0.f, mx = 0.f;
  int bad = 0;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * 256) {
    const float v = x[i];
    if (v < mn) mn = v;
    if (v > mx) mx = v;
    if (!isfinite(v)) bad = 1;
  }
  __shared__ float smn[256], smx[256];
  __shared__ int sbad[256];
  smn[threadIdx.x] = mn;
  smx[threadIdx.x] = mx;
  sbad[threadIdx.x] = bad;
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if (threadIdx.x < s) {
      if (smn[threadIdx.x + s] < smn[threadIdx.x]) smn[threadIdx.x] = smn[threadIdx.x + s];
      if (smx[threadIdx.x + s] > smx[threadIdx.x]) smx[threadIdx.x] = smx[threadIdx.x + s];
      sbad[threadIdx.x] |= sbad[threadIdx.x + s];
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    pmn[blockIdx.x] = smn[0];
    pmx[blockIdx.x] = smx[0];
    pbad[blockIdx.x] = sbad[0];
  }
}

__device__ inline double round_even(double v) { return rint(v); }

__global__ __launch_bounds__(256) void k_dql_quant(
    const float *__restrict__ x, int64_t n, const float *__restrict__ pmn,
    const float *__restrict__ pmx, const int *__restrict__ pbad, int nparts,
    uint8_t *__restrict__ y, void *__restrict__ scale_zp) {
  __shared__ float smn[256], smx[256];
  __shared__ int sbad[256];
  float mn = 0.f, mx = 0.f;
  int bad = 0;
  for (int i = threadIdx.x; i < nparts; i += 256) {
    if (pmn[i] < mn) mn = pmn[i];
    if (pmx[i] > mx) mx = pmx[i];
    bad |= pbad[i];
  }
  smn[threadIdx.x] = mn;
  smx[threadIdx.x] = mx;
  sbad[threadIdx.x] = bad;
  __syncthreads();
  for (int s = 128; s > 0; s >>= 1) {
    if (threadIdx.x < s) {
      if (smn[threadIdx.x + s] < smn[threadIdx.x]) smn[threadIdx.x] = smn[threadIdx.x + s];
      if (smx[threadIdx.x + s] > smx[threadIdx.x]) smx[threadIdx.x] = smx[threadIdx.x + s];
      sbad[threadIdx.x] |= sbad[threadIdx.x + s];
    }
    __syncthreads();
  }
  const double dmn = smn[0], dmx = smx[0];
  const float scale_f = (float)((dmx - dmn) / 255.0);
  const double scale = scale_f;
  const float zpf = scale == 0.0 ? 0.f : (float)(-dmn / scale);
  double zc = zpf;
  zc = zc < 0.0 ? 0.0 : (zc > 255.0 ? 255.0 : zc);
  const int zp = (int)round_even(zc);
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * 256) {
    int q;
    if (scale == 0.0) {
      q = zp;
    } else {
      const float r = (float)((double)x[i] / scale);
      q = isfinite(r) ? (int)round_even((double)r) + zp : zp;
    }
    y[i] = (uint8_t)(q < 0 ? 0 : (q > 255 ? 255 : q));
  }
  if (blockIdx.x == 0 && threadIdx.x == 0) {
    float *sp = static_cast<float *>(scale_zp);
    int *ip = static_cast<int *>(scale_zp);
    sp[0] = scale_f;
    ip[1] = zp;
    ip[2] = (sbad[0] && scale != 0.0) ? 1 : 0;
  }
}

}  // namespace

size_t mg_dql_ws_bytes(int64_t) { return 3 * mg_align(DQL_PARTS * 4); }

mg_status mg_dql_run(mg_ctx *ctx, const float *x_dev, int64_t n,
                     uint8_t *y_dev, void *scale_zp_dev, void *ws) {
  char *p = static_cast<char *>(ws);
  float *pmn = reinterpret_cast<float *>(p);
  float *pmx = reinterpret_cast<float *>(p + mg_align(DQL_PARTS * 4));
  int *pbad = reinterpret_cast<int *>(p + 2 * mg_align(DQL_PARTS * 4));
  int64_t parts = (n + 255) / 256;
  if (parts > DQL_PARTS) parts = DQL_PARTS;
  if (parts < 1) parts = 1;
  hipLaunchKernelGGL(k_dql_partial, dim3((unsigned)parts), dim3(256), 0, ctx->stream, x_dev, n,
                     pmn, pmx, pbad);
  MG_TRY(mg_launch_check("k_dql_partial"));
  hipLaunchKernelGGL(k_dql_quant, dim3((unsigned)parts), dim3(256), 0, ctx->stream, x_dev, n,
                     pmn, pmx, pbad, (int)parts, y_dev, scale_zp_dev);
  return mg_launch_check("k_dql_quant");
}
