// Fused attention in fp32: y = softmax(scale * Q K^T + mask) V per batch
// index, for the _FusedSDPA pattern (lib/src/onnx_ops.dart:2100-2149) and
// MultiHeadAttention (lib/src/onnx_ops.dart:2014-2098), whose per-head
// operands are strided views of [batch, seq, hidden] tensors.
//
// One wave per 32 query rows (a workgroup of 4 waves takes 128 rows of one
// batch index), streaming the keys in tiles of 32 with an online softmax.
// The workgroup stages each K and V tile once in LDS (double-buffered; the
// next tile's loads are in flight while the current one is computed, one
// barrier per tile):
//   * S^T tile (32 keys x 32 queries) = K . Q^T on v_mfma_f32_32x32x2_f32:
//     A operand lane l = key l % 32, dim 2s + l / 32 (from the K tile); B operand
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
//     reads V[t(s, l / 32)][32 j + l % 32] from the V tile.
//   * At the end y = O / l per query; a row whose every score is -inf is NaN
//     (the reference's exp(-inf - -inf)), and T = 0 gives zeros (an empty
//     product).
// fp32 throughout (the reference accumulates the products in f32 and the
// softmax in f64; results agree to fp32 rounding of the different order).
#include <hip/hip_runtime.h>

#include <cmath>
#include <type_traits>

#include "mg_internal.h"

namespace {

typedef float float16v __attribute__((ext_vector_type(16)));

template <int DS, int DVT>
__global__ __launch_bounds__(256) void k_attn(const mg_attn_problem p) {
  constexpr int DP = 2 * DS + 1;     // LDS row pitch of a K tile (odd: no bank conflicts)
  constexpr int VP = 32 * DVT;       // LDS row pitch of a V tile
  constexpr int KE = 32 * 2 * DS / 256, VE = 32 * VP / 256;  // staged elements per thread
  __shared__ float ks[2][32 * DP];
  __shared__ float vs[2][32 * VP];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int qtiles = (p.S + 127) / 128;
  const int bi = (int)(blockIdx.x / qtiles);  // the host keeps the grid below 2^31
  const int q0 = (int)(blockIdx.x % qtiles) * 128 + wave * 32;
  const bool active = q0 < p.S;  // idle waves still stage tiles and meet the barriers
  // Batch offsets of every operand.
  int64_t oq = 0, ok = 0, ov = 0, om = 0, oy = 0;
  {
    int rem = bi;
    for (int d = p.nbd - 1; d >= 0; d--) {
      const int bd = (int)p.bdim[d];
      const int64_t c = rem % bd;
      rem /= bd;
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

  // Cooperative staging of key tile t0: element e of the thread's share is
  // (key, dim) chosen so that consecutive threads read consecutive addresses
  // of whichever index is contiguous in memory.  Out-of-range elements are 0.
  // The element offsets inside a tile are fixed per thread and 32-bit (the
  // host checks the strides); the tile base advances by 32 keys.
  const bool k_tmajor = p.k_ts == 1, v_tmajor = p.v_ts == 1;
  int kgo[KE], klo[KE], vgo[VE], vlo[VE];
  unsigned kd_ok = 0, vd_ok = 0;  // per element: dim in range
#pragma unroll
  for (int e = 0; e < KE; e++) {
    const int idx = tid + 256 * e;
    const int t = k_tmajor ? idx & 31 : idx / (2 * DS);
    const int d = k_tmajor ? idx >> 5 : idx % (2 * DS);
    kgo[e] = 4 * (t * (int)p.k_ts + d * (int)p.k_ds);  // bytes
    klo[e] = t * DP + d;
    if (d < p.D) kd_ok |= 1u << e;
  }
#pragma unroll
  for (int e = 0; e < VE; e++) {
    const int idx = tid + 256 * e;
    const int t = v_tmajor ? idx & 31 : idx / VP;
    const int dv = v_tmajor ? idx >> 5 : idx % VP;
    vgo[e] = 4 * (t * (int)p.v_ts + dv * (int)p.v_ds);  // bytes
    vlo[e] = t * VP + dv;
    if (dv < p.DV) vd_ok |= 1u << e;
  }
  // Raw loaded values: range selections happen when they are consumed (a
  // use at the load would make the wave wait for it right there).
  float kreg[KE], vreg[VE];
  unsigned kin = 0, vin = 0;  // per element: inside the tensor
  float mreg[16];  // the lane's mask values of the fetched tile (its query)
  // Loads address a uniform base plus a per-lane 32-bit byte offset.
  auto ldb = [](const float *base, unsigned bytes) {
    return *reinterpret_cast<const float *>(reinterpret_cast<const char *>(base) + bytes);
  };
  const float *mrow = p.mask ? p.mask + om + (int64_t)(qok ? q : 0) * p.m_qs : nullptr;
  const int mts = (int)p.m_ts;
  const unsigned mlane = 16u * h * mts;  // bytes of key offset 4h
  // full: the tile holds 32 keys (no clamping or range checks).
  auto fetch = [&](int t0, auto full) {
    constexpr bool F = decltype(full)::value;
    const int tl = p.T - t0;  // keys left from t0
    if (mrow && active) {
      const float *mt = mrow + (int64_t)t0 * p.m_ts;
#pragma unroll
      for (int v = 0; v < 16; v++) {
        // Unconditional loads (clamped in range) so that they batch; keys past
        // the end are excluded when the scores are formed.
        const int tu = 8 * (v >> 2) + (v & 3);
        if (F) {
          mreg[v] = ldb(mt + tu * mts, mlane);
        } else {
          const int tt = tu + 4 * h;
          mreg[v] = mt[min(tt, tl - 1) * mts];
        }
      }
    }
    const float *kt = p.k + ok + (int64_t)t0 * p.k_ts;
    const float *vt = p.v + ov + (int64_t)t0 * p.v_ts;
#pragma unroll
    for (int e = 0; e < KE; e++) {
      const int idx = tid + 256 * e;
      const int t = k_tmajor ? idx & 31 : idx / (2 * DS);
      const bool in = (F || t < tl) && ((kd_ok >> e) & 1);
      kin = in ? kin | (1u << e) : kin & ~(1u << e);
      kreg[e] = ldb(kt, in ? (unsigned)kgo[e] : 0u);
    }
#pragma unroll
    for (int e = 0; e < VE; e++) {
      const int idx = tid + 256 * e;
      const int t = v_tmajor ? idx & 31 : idx / VP;
      const bool in = (F || t < tl) && ((vd_ok >> e) & 1);
      vin = in ? vin | (1u << e) : vin & ~(1u << e);
      vreg[e] = ldb(vt, in ? (unsigned)vgo[e] : 0u);
    }
  };
  auto fetch_any = [&](int t0) {
    if (t0 + 32 <= p.T)
      fetch(t0, std::true_type{});
    else
      fetch(t0, std::false_type{});
  };
  auto stage = [&](int buf) {
#pragma unroll
    for (int e = 0; e < KE; e++) ks[buf][klo[e]] = ((kin >> e) & 1) ? kreg[e] : 0.f;
#pragma unroll
    for (int e = 0; e < VE; e++) vs[buf][vlo[e]] = ((vin >> e) & 1) ? vreg[e] : 0.f;
  };

  // Q^T fragments: step s holds dim 2s + h of query q.
  float qf[DS];
  {
    const float *qr = p.q + oq + (int64_t)(qok ? q : 0) * p.q_rs;
#pragma unroll
    for (int s = 0; s < DS; s++) {
      const int d = 2 * s + h;
      const bool in = qok && d < p.D;
      const float x = qr[in ? d * (int)p.q_cs : 0];
      qf[s] = in ? x : 0.f;
    }
  }
  float16v o[DVT];
#pragma unroll
  for (int j = 0; j < DVT; j++) o[j] = (float16v){};
  float m_run = -INFINITY, l_run = 0.f;
  float mcur[16];

  if (p.T > 0) {
    fetch_any(0);
    stage(0);
  }
  // Scores in the log2 domain: p = 2^(s * scale * log2 e + mask * log2 e - m).
  constexpr float kLog2e = 1.4426950408889634f;
  const float scale2 = p.scale * kLog2e;
  __syncthreads();
  for (int t0 = 0, it = 0; t0 < p.T; t0 += 32, it++) {
    const int buf = it & 1;
    const bool more = t0 + 32 < p.T;
#pragma unroll
    for (int v = 0; v < 16; v++) mcur[v] = mreg[v];
    if (more) fetch_any(t0 + 32);  // next tile's loads fly while this one is computed
    const bool full = t0 + 32 <= p.T;
    if (active) {
      const float *kl = &ks[buf][0];
      const float *vl = &vs[buf][0];
      // Scores S^T[t][q] for keys t0 .. t0 + 31.
      float16v sc = (float16v){};
#pragma unroll
      for (int s = 0; s < DS; s++)
        sc = __builtin_amdgcn_mfma_f32_32x32x2f32(kl[r32 * DP + 2 * s + h], qf[s], sc, 0, 0, 0);
      float pv[16];
      float tmax = -INFINITY;
#pragma unroll
      for (int v = 0; v < 16; v++) {
        const int tt = 8 * (v >> 2) + (v & 3) + 4 * h;  // key of slot v
        float x = fmaf(sc[v], scale2, mrow ? mcur[v] * kLog2e : 0.f);
        if (!full && t0 + tt >= p.T) x = -INFINITY;
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
        corr = __builtin_amdgcn_exp2f(m_run - m_new);  // 0 while nothing has been accumulated
        float ls = 0.f;
#pragma unroll
        for (int v = 0; v < 16; v++) {
          pv[v] = __builtin_amdgcn_exp2f(pv[v] - m_new);
          ls += pv[v];
        }
        l_run = l_run * corr + ls;
        m_run = m_new;
      }
#pragma unroll
      for (int j = 0; j < DVT; j++) {
#pragma unroll
        for (int v = 0; v < 16; v++) o[j][v] *= corr;
#pragma unroll
        for (int s = 0; s < 16; s++) {
          const int tt = 8 * (s >> 2) + (s & 3) + 4 * h;
          o[j] = __builtin_amdgcn_mfma_f32_32x32x2f32(vl[tt * VP + 32 * j + r32], pv[s], o[j], 0,
                                                      0, 0);
        }
      }
    }
    if (more) stage(buf ^ 1);  // the other buffer: its readers passed the last barrier
    __syncthreads();
  }

  const float l_tot = l_run + __shfl_xor(l_run, 32);
  if (!active || !qok) return;
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
  mg_attn_problem pp = p;
  if (p.D == 0) {  // no products: the kernel's (masked-off) Q and K loads read V instead
    pp.q = pp.k = p.v;
    pp.q_rs = pp.q_cs = pp.k_ts = pp.k_ds = 0;
    for (int d = 0; d < MG_ATTN_MAX_BATCH_DIMS; d++) pp.q_bs[d] = pp.k_bs[d] = 0;
  }
  if (p.D <= 32)
    launch_dvt<16>(pp, grid, ctx->stream);
  else if (p.D <= 64)
    launch_dvt<32>(pp, grid, ctx->stream);
  else
    launch_dvt<64>(pp, grid, ctx->stream);
  return mg_launch_check("k_attn");
}
