// fp32 MatMul / Gemm on gfx950 fp32 MFMA (v_mfma_f32_16x16x4_f32).
//
// Reference semantics: opMatMul (numpy broadcast, lib/src/onnx_ops.dart:
// 1710-1766) and opGemm (alpha * op(A) op(B) + beta * C,
// lib/src/onnx_ops.dart:2152-2172).  The MFMA multiplies fp32 operands exactly
// and accumulates in fp32, so results differ from the reference's sequential
// k-order sums only by accumulation order.
//
// Workgroup tile 64 x 64, four waves as 2 x 2 of 32 x 32 (2 x 2 MFMA
// subtiles).  Each k step of 16 is staged in LDS k-major, so the MFMA operand
// of lane (i = lane%16, g = lane/16) is As[k0 + g][row i] and Bs[k0 + g][col i].
// Batches run on grid.z with per-batch element offsets computed on the host
// (numpy broadcasting, lib/src/onnx_ops.dart:1742-1764).
#include <hip/hip_runtime.h>

#include "mg_internal.h"

namespace {

typedef float float4v __attribute__((ext_vector_type(4)));

constexpr int TM = 64, TN = 64, TK = 16;

__global__ __launch_bounds__(256) void k_f32_gemm(
    const float *__restrict__ A, const float *__restrict__ B,
    float *__restrict__ Y, int64_t M, int64_t N, int64_t K, int64_t lda,
    int64_t ldb, int trans_a, int trans_b, const int64_t *__restrict__ a_off,
    const int64_t *__restrict__ b_off, float alpha, float beta,
    const float *__restrict__ C, int64_t c_rs, int64_t c_cs) {
  __shared__ float As[TK][TM + 4];
  __shared__ float Bs[TK][TN + 4];
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave & 1, wn = wave >> 1;
  const int64_t bz = blockIdx.z;
  const float *Ab = A + (a_off ? a_off[bz] : 0);
  const float *Bb = B + (b_off ? b_off[bz] : 0);
  const int64_t r0 = (int64_t)blockIdx.y * TM, c0 = (int64_t)blockIdx.x * TN;
  const int li = lane & 15, lg = lane >> 4;

  float4v acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; i++)
#pragma unroll
    for (int j = 0; j < 2; j++) acc[i][j] = (float4v){0.f, 0.f, 0.f, 0.f};

  for (int64_t k0 = 0; k0 < K; k0 += TK) {
    // Stage A: 64 rows x 16 k.
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const int idx = tid + e * 256;
      int rr, kk;
      if (!trans_a) {
        rr = idx >> 4;
        kk = idx & 15;
      } else {
        kk = idx >> 6;
        rr = idx & 63;
      }
      const int64_t row = r0 + rr, k = k0 + kk;
      float v = 0.f;
      if (row < M && k < K) v = trans_a ? Ab[k * lda + row] : Ab[row * lda + k];
      As[kk][rr] = v;
    }
    // Stage B: 16 k x 64 cols.
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const int idx = tid + e * 256;
      int kk, cc;
      if (!trans_b) {
        kk = idx >> 6;
        cc = idx & 63;
      } else {
        cc = idx >> 4;
        kk = idx & 15;
      }
      const int64_t col = c0 + cc, k = k0 + kk;
      float v = 0.f;
      if (col < N && k < K) v = trans_b ? Bb[col * ldb + k] : Bb[k * ldb + col];
      Bs[kk][cc] = v;
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < TK; kk += 4) {
      float a[2], b[2];
#pragma unroll
      for (int i = 0; i < 2; i++) a[i] = As[kk + lg][wm * 32 + i * 16 + li];
#pragma unroll
      for (int j = 0; j < 2; j++) b[j] = Bs[kk + lg][wn * 32 + j * 16 + li];
#pragma unroll
      for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[i], b[j], acc[i][j], 0, 0, 0);
    }
    __syncthreads();
  }
  float *Yb = Y + bz * M * N;
#pragma unroll
  for (int i = 0; i < 2; i++)
#pragma unroll
    for (int j = 0; j < 2; j++) {
      const int64_t col = c0 + wn * 32 + j * 16 + li;
      if (col >= N) continue;
#pragma unroll
      for (int r = 0; r < 4; r++) {
        const int64_t row = r0 + wm * 32 + i * 16 + 4 * lg + r;
        if (row >= M) continue;
        float v = acc[i][j][r];
        if (alpha != 1.f) v = alpha * v;
        if (C) {
          float cv = C[row * c_rs + col * c_cs];
          if (beta != 1.f) cv = beta * cv;
          v = v + cv;
        }
        Yb[row * N + col] = v;
      }
    }
}

}  // namespace

mg_status mg_f32_run(mg_ctx *ctx, const mg_f32_problem &p, const float *a_dev,
                     const float *b_dev, float *y_dev) {
  if (p.M == 0 || p.N == 0 || p.batch == 0) return MG_OK;
  const dim3 grid((unsigned)((p.N + TN - 1) / TN), (unsigned)((p.M + TM - 1) / TM),
                  (unsigned)p.batch);
  hipLaunchKernelGGL(k_f32_gemm, grid, dim3(256), 0, ctx->stream, a_dev, b_dev, y_dev, p.M,
                     p.N, p.K, p.lda, p.ldb, p.trans_a, p.trans_b, p.a_off, p.b_off, p.alpha,
                     p.beta, p.c, p.c_rs, p.c_cs);
  return mg_launch_check("k_f32_gemm");
}
