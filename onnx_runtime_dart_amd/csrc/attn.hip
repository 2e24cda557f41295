// Fused attention in fp32: y = softmax(scale * Q K^T + mask) V per batch
// index, for the _FusedSDPA pattern (lib/src/onnx_ops.dart:2100-2149) and
// MultiHeadAttention (lib/src/onnx_ops.dart:2014-2098), whose per-head
// operands are strided views of [batch, seq, hidden] tensors.
//
// One wave per 32 query rows (a workgroup of 4 waves takes 128 rows of one
// batch index), streaming the keys in tiles of 32 with an online softmax:
//   * S^T tile (32 keys x 32 queries) = K . Q^T on v_mfma_f32_32x32x2_f32:
//     A operand lane l = key l % 32, dim 2s + l / 32 (read from K); B operand
//     lane l = query l % 32, dim 2s + l / 32 (the wave's Q, held in
//     registers for all tiles).  The result gives each lane one query and 16
//     keys t = 8 (v / 4) + 4 (l / 32) + v % 4 (the other 16 in lane l ^ 32).
//   * val = fma(S, scale, mask) (padding keys -inf); the running max m and
//     sum l per query (lane pair), p = exp(val - m_new), and the output and
//     sum rescaled by exp(m_old - m_new).
//   * O^T (32 dims x 32 queries, per 32-dim tile of V) += V^T . P^T: MFMA
//     step s pairs k slot l / 32 with key t(s, l / 32) = 8 (s / 4) +
//     4 (l / 32) + s % 4, so the B operand of step s is exactly the lane's
//     p[s] from the score layout (no data movement); the A operand lane l
//     reads V[t(s, l / 32)][32 j + l % 32].
//   * At the end y = O / l per query; a row whose every score is -inf is NaN
//     (the reference's exp(-inf - -inf)), and T = 0 gives zeros (an empty
//     product).
// fp32 throughout (the reference accumulates the products in f32 and the
// softmax in f64; results agree to fp32 rounding of the different order).
#include <hip/hip_runtime.h>

#include <cmath>

#include "mg_internal.h"

namespace {

typedef float float16v __attribute__((ext_vector_type(16)));

template <int DS, int DVT>
__global__ __launch_bounds__(256) void k_attn(const mg_attn_problem p) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int qtiles = (p.S + 127) / 128;
  const int64_t bi = blockIdx.x / qtiles;
  const int q0 = (int)(blockIdx.x % qtiles) * 128 + wave * 32;
  if (q0 >= p.S) return;  // no barriers below: idle waves may leave
  // Batch offsets of every operand.
  int64_t oq = 0, ok = 0, ov = 0, om = 0, oy = 0;
  {
    int64_t rem = bi;
    for (int d = p.nbd - 1; d >= 0; d--) {
      const int64_t c = rem % p.bdim[d];
      rem /= p.bdim[d];
      oq += c * p.q_bs[d];
      ok += c * p.k_bs[d];
      ov += c * p.v_bs[d];
      om += c * p.m_bs[d];
      oy += c * p.y_bs[d];
    }
  }
  const int r32 = lane & 31, h = lane >> 5;
  const int q = q0 + r32;  // this lane's query (B-operand column / result column)
  const bool qok = q < p.S;
  // Lane parts of the element offsets are 32-bit (the host checks the
  // strides); the uniform parts ride on the per-tile base pointers.
  const int kst = (int)p.k_ts, kds = (int)p.k_ds, vst = (int)p.v_ts, vds = (int)p.v_ds;
  const int mts = (int)p.m_ts;

  // Q^T fragments: step s holds dim 2s + h of query q.
  float qf[DS];
  {
    const float *qr = p.q + oq + (int64_t)(qok ? q : 0) * p.q_rs;
    const int qcs = (int)p.q_cs;
#pragma unroll
    for (int s = 0; s < DS; s++) {
      const int d = 2 * s + h;
      qf[s] = (qok && d < p.D) ? qr[d * qcs] : 0.f;
    }
  }
  float16v o[DVT];
#pragma unroll
  for (int j = 0; j < DVT; j++) o[j] = (float16v){};
  float m_run = -INFINITY, l_run = 0.f;
  const float *mrow = p.mask ? p.mask + om + (int64_t)(qok ? q : 0) * p.m_qs : nullptr;
  const int koff = r32 * kst + h * kds;  // key r32, dim h
  const int voff = 4 * h * vst;          // key offset 4h of every step

  for (int t0 = 0; t0 < p.T; t0 += 32) {
    const float *kt = p.k + ok + (int64_t)t0 * p.k_ts;
    const float *vt = p.v + ov + (int64_t)t0 * p.v_ts;
    // Scores S^T[t][q] for keys t0 .. t0 + 31.
    float16v sc = (float16v){};
    const bool tkok = t0 + r32 < p.T;
#pragma unroll
    for (int s = 0; s < DS; s++) {
      const bool dok = 2 * s + h < p.D;
      const float kv = (tkok && dok) ? kt[koff + 2 * s * kds] : 0.f;
      sc = __builtin_amdgcn_mfma_f32_32x32x2f32(kv, qf[s], sc, 0, 0, 0);
    }
    float pv[16];
    float tmax = -INFINITY;
#pragma unroll
    for (int v = 0; v < 16; v++) {
      const int tt = 8 * (v >> 2) + (v & 3);  // key of slot v in half 0
      float x = -INFINITY;
      if (t0 + tt + 4 * h < p.T)
        x = fmaf(sc[v], p.scale, mrow ? mrow[(int64_t)t0 * p.m_ts + (tt + 4 * h) * mts] : 0.f);
      pv[v] = x;
      tmax = fmaxf(tmax, x);
    }
    tmax = fmaxf(tmax, __shfl_xor(tmax, 32));
    const float m_new = fmaxf(m_run, tmax);
    float corr = 1.f;
    if (m_new == -INFINITY) {
#pragma unroll
      for (int v = 0; v < 16; v++) pv[v] = 0.f;
    } else {
      corr = __expf(m_run - m_new);  // 0 while nothing has been accumulated
      float ls = 0.f;
#pragma unroll
      for (int v = 0; v < 16; v++) {
        pv[v] = __expf(pv[v] - m_new);
        ls += pv[v];
      }
      l_run = l_run * corr + ls;
      m_run = m_new;
    }
#pragma unroll
    for (int j = 0; j < DVT; j++) {
#pragma unroll
      for (int v = 0; v < 16; v++) o[j][v] *= corr;
      const int dv = 32 * j + r32;
      const bool dvok = dv < p.DV;
      const int vl = voff + dv * vds;
#pragma unroll
      for (int s = 0; s < 16; s++) {
        const int tt = 8 * (s >> 2) + (s & 3);
        const float a = (dvok && t0 + tt + 4 * h < p.T) ? vt[vl + tt * vst] : 0.f;
        o[j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a, pv[s], o[j], 0, 0, 0);
      }
    }
  }

  const float l_tot = l_run + __shfl_xor(l_run, 32);
  if (!qok) return;
  float inv;
  if (p.T == 0)
    inv = 0.f;  // empty softmax: the product is a sum over no keys
  else if (m_run == -INFINITY)
    inv = __builtin_nanf("");
  else
    inv = 1.f / l_tot;
  float *yr = p.y + oy + (int64_t)q * p.y_rs;
#pragma unroll
  for (int j = 0; j < DVT; j++)
#pragma unroll
    for (int v = 0; v < 16; v++) {
      const int dv = 32 * j + 8 * (v >> 2) + 4 * h + (v & 3);
      if (dv < p.DV) yr[dv] = p.T == 0 ? 0.f : o[j][v] * inv;
    }
}

template <int DS>
void launch_dvt(const mg_attn_problem &p, dim3 grid, hipStream_t st) {
  if (p.DV <= 32)
    hipLaunchKernelGGL((k_attn<DS, 1>), grid, dim3(256), 0, st, p);
  else if (p.DV <= 64)
    hipLaunchKernelGGL((k_attn<DS, 2>), grid, dim3(256), 0, st, p);
  else
    hipLaunchKernelGGL((k_attn<DS, 4>), grid, dim3(256), 0, st, p);
}

}  // namespace

mg_status mg_attn_run(mg_ctx *ctx, const mg_attn_problem &p) {
  if (p.D > 128 || p.DV > 128)
    return mg_fail(MG_UNSUPPORTED, "attention: head sizes above 128 are not supported");
  if (p.nbd > MG_ATTN_MAX_BATCH_DIMS)
    return mg_fail(MG_UNSUPPORTED, "attention: more than 4 batch dimensions");
  int64_t nbatch = 1;
  for (int d = 0; d < p.nbd; d++) nbatch *= p.bdim[d];
  if (nbatch == 0 || p.S == 0 || p.DV == 0) return MG_OK;
  const int64_t wgs = nbatch * ((p.S + 127) / 128);
  if (wgs > 0x7fffffff) return mg_fail(MG_UNSUPPORTED, "attention: grid too large");
  const dim3 grid((unsigned)wgs);
  if (p.D <= 32)
    launch_dvt<16>(p, grid, ctx->stream);
  else if (p.D <= 64)
    launch_dvt<32>(p, grid, ctx->stream);
  else
    launch_dvt<64>(p, grid, ctx->stream);
  return mg_launch_check("k_attn");
}
