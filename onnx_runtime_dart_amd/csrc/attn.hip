// Fused attention in fp32: y = softmax(scale * Q K^T + mask) V per batch
// index, for the _FusedSDPA pattern (lib/src/onnx_ops.dart:2100-2149) and
// MultiHeadAttention (lib/src/onnx_ops.dart:2014-2098), whose per-head
// operands are strided views of [batch, seq, hidden] tensors.
//
// One wave per 32 query rows (a workgroup of 4 waves takes 128 rows of one
// batch index), streaming the keys in tiles of 32 with an online softmax.
// The workgroup stages each K and V tile once in LDS (double-buffered, one
// barrier per tile); its global loads are raw buffer loads issued two tiles
// ahead of use (two register sets), with out-of-range elements read as 0 by
// the hardware:
//   * S^T tile (32 keys x 32 queries) = K . Q^T on v_mfma_f32_32x32x2_f32:
//     step s gives lane l key l % 32 (A) or query l % 32 (B) at dim
//     DS (l / 32) + s, so a lane's K fragments of a tile are one contiguous
//     LDS run (16-byte reads); the Q fragments stay in registers.  The result
//     gives each lane one query and 16 keys t = 8 (v / 4) + 4 (l / 32) + v % 4
//     (the other 16 in lane l ^ 32).
//   * val = fma(S, scale, mask) (padding keys -inf); the running max m and
//     sum l per query (lane pair), p = exp(val - m_new), and the output and
//     sum rescaled by exp(m_old - m_new), all in the log2 domain.
//   * O^T (32 dims x 32 queries, per 32-dim tile of V) += V^T . P^T: MFMA
//     step s pairs k slot l / 32 with key t(s, l / 32) = 8 (s / 4) +
//     4 (l / 32) + s % 4, so the B operand of step s is exactly the lane's
//     p[s] from the score layout (no data movement); the A operand lane l
//     reads V[t(s, l / 32)][32 j + l % 32] from the transposed V tile, where
//     the keys of steps 4g .. 4g + 3 are adjacent (one 16-byte read).
//   * With causal masking (GroupQueryAttention) key t is -inf for query q
//     when t > q + causal_off, and a workgroup stops after the last key its
//     last query sees.
//   * At the end y = O / l per query; a row whose every score is -inf is NaN
//     (the reference's exp(-inf - -inf)), and T = 0 gives zeros (an empty
//     product).
// fp32 throughout (the reference accumulates the products in f32 and the
// softmax in f64; results agree to fp32 rounding of the different order).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <type_traits>

#include "mg_internal.h"

namespace {

typedef float float16v __attribute__((ext_vector_type(16)));

// Floats per query row of a key split's partials: the DV unnormalised
// outputs, the running max and the sum, padded to a multiple of four so
// that rows start 16-byte aligned (the merge reads four outputs at a time).
__host__ __device__ constexpr int64_t attn_part_row(int64_t dv) { return (dv + 5) & ~int64_t(3); }

template <int DS, int DVT>
__device__ __attribute__((always_inline)) void attn_tiles(const mg_attn_problem &p) {
  // Tiles prefetched ahead in registers: two for head size <= 32, one for the
  // larger heads (their fragments and accumulators need the registers; one
  // set keeps them at two waves per SIMD).
  constexpr int PD = (DS >= 32 || DVT >= 2) ? 1 : 2;
  // LDS tiles: K as [key][dim] with row pitch DP, V transposed as [dim][key]
  // with row pitch VT.  Both pitches are 4 (mod 64) floats: rows start on 16
  // bytes and the 16-byte reads of 16 consecutive rows fall in distinct bank
  // groups.
  constexpr int DP = 2 * DS + 4;
  constexpr int VT = 36;
  constexpr int KE = 32 * 2 * DS / 256, VE = 32 * 32 * DVT / 256;  // staged elements per thread
  __shared__ __attribute__((aligned(16))) float ks[2][32 * DP];
  __shared__ __attribute__((aligned(16))) float vs[2][32 * DVT * VT];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
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

  // Keys the workgroup visits: all T, or with causal masking only up to the
  // last key its last query sees (keys past it are -inf for every query).
  // With a key split (p.kc > 0) the workgroup takes keys [t_begin,
  // t_begin + kc) of split blockIdx.y and writes partial results.
  const int t_begin = p.kc > 0 ? (int)blockIdx.y * p.kc : 0;
  // (min() by value: a reference to a field of p would put p in scratch memory)
  int t_loop = p.kc > 0 ? min(p.T, t_begin + p.kc) : p.T;
  if (p.causal) {
    const int64_t q_last = (int64_t)(blockIdx.x % qtiles) * 128 + 127;
    t_loop = (int)std::min<int64_t>(t_loop, std::max<int64_t>(0, q_last + p.causal_off + 1));
  }
  if (p.part && t_loop <= t_begin) {
    // A split past the causal limit of every query of the tile: its partial
    // is that of no keys (zero O, max -inf, sum 0), written without loading
    // anything (the whole workgroup leaves here).
    if (!active || !qok) return;
    float *pr = p.part + (((int64_t)blockIdx.y * (gridDim.x / qtiles) + bi) * p.S + q) *
                             attn_part_row(p.DV);
#pragma unroll
    for (int j = 0; j < DVT; j++)
#pragma unroll
      for (int v = 0; v < 16; v++) {
        const int dv = 32 * j + 8 * (v >> 2) + 4 * h + (v & 3);
        if (dv < p.DV) pr[dv] = 0.f;
      }
    if (h == 0) pr[p.DV] = -INFINITY, pr[p.DV + 1] = 0.f;
    return;
  }

  // Cooperative staging of key tile t0: element e of the thread's share is
  // (key, dim) chosen so that consecutive threads read consecutive addresses
  // of whichever index is contiguous in memory.  Loads are raw buffer loads:
  // a tile base in the (uniform) resource plus a fixed 32-bit byte offset per
  // element; an element outside the tensor gets offset kOob, past the
  // resource's range, and the hardware returns 0 for it.  The host keeps the
  // in-range offsets below 2^31.
  constexpr unsigned kOob = 0x80000000u;
  const bool k_tmajor = p.k_ts == 1, v_tmajor = p.v_ts == 1;
  unsigned kgo[KE], vgo[VE];
#pragma unroll
  for (int e = 0; e < KE; e++) {
    const int idx = tid + 256 * e;
    const int t = k_tmajor ? idx & 31 : idx / (2 * DS);
    const int d = k_tmajor ? idx >> 5 : idx % (2 * DS);
    kgo[e] = d < p.D ? 4u * (unsigned)(t * (int)p.k_ts + d * (int)p.k_ds) : kOob;
  }
#pragma unroll
  for (int e = 0; e < VE; e++) {
    const int idx = tid + 256 * e;
    const int t = v_tmajor ? idx & 31 : idx / (32 * DVT);
    const int dv = v_tmajor ? idx >> 5 : idx % (32 * DVT);
    vgo[e] = dv < p.DV ? 4u * (unsigned)(t * (int)p.v_ts + dv * (int)p.v_ds) : kOob;
  }
  auto rsrc = [](const float *base) __attribute__((always_inline)) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(base), (short)0, 0x7ffffff0,
                                             0x00020000);
  };
  auto ldr = [](__amdgpu_buffer_rsrc_t r, unsigned off) __attribute__((always_inline)) {
    asm("" : "+v"(off));  // an opaque offset: the select stays a select, not a branch
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0));
  };
  // With two register sets tile i is fetched into set i % 2 two tiles ahead
  // of its use, so each load has two tiles of compute to arrive; with one it
  // is fetched one tile ahead.
  float kreg[PD][KE], vreg[PD][VE];
  float mreg[PD][16];  // the lane's mask values of a fetched tile (its query)
  // Mask rows of the wave's 32 queries: a wave-uniform base (row q0) and the
  // lane's row offset; rows past S read nothing.
  const float *mrow = p.mask ? p.mask + om + (int64_t)q0 * p.m_qs : nullptr;
  const unsigned mts4 = 4u * (unsigned)p.m_ts;
  const unsigned mq = qok ? 4u * (unsigned)(r32 * (int)p.m_qs) : kOob;
  // full: the tile holds 32 keys (no range checks on keys).
  auto fetch = [&](int t0, auto full, auto set) __attribute__((always_inline)) {
    constexpr bool F = decltype(full)::value;
    constexpr int R = decltype(set)::value;
    const int tl = p.T - t0;  // keys left from t0
    if (mrow && active) {
      const __amdgpu_buffer_rsrc_t rm = rsrc(mrow + (int64_t)t0 * p.m_ts);
#pragma unroll
      for (int v = 0; v < 16; v++) {
        const int tt = 8 * (v >> 2) + (v & 3) + 4 * h;  // key of slot v
        mreg[R][v] = ldr(rm, (F || tt < tl) && qok ? mq + (unsigned)tt * mts4 : kOob);
      }
    }
    const __amdgpu_buffer_rsrc_t rk = rsrc(p.k + ok + (int64_t)t0 * p.k_ts);
    const __amdgpu_buffer_rsrc_t rv = rsrc(p.v + ov + (int64_t)t0 * p.v_ts);
#pragma unroll
    for (int e = 0; e < KE; e++) {
      const int idx = tid + 256 * e;
      const int t = k_tmajor ? idx & 31 : idx / (2 * DS);
      kreg[R][e] = ldr(rk, F || t < tl ? kgo[e] : kOob);
    }
#pragma unroll
    for (int e = 0; e < VE; e++) {
      const int idx = tid + 256 * e;
      const int t = v_tmajor ? idx & 31 : idx / (32 * DVT);
      vreg[R][e] = ldr(rv, F || t < tl ? vgo[e] : kOob);
    }
  };
  auto fetch_any = [&](int t0, auto set) __attribute__((always_inline)) {
    if (t0 + 32 <= p.T)
      fetch(t0, std::true_type{}, set);
    else
      fetch(t0, std::false_type{}, set);
  };
  // Register set R -> LDS buffer L.  Element e of the thread's share sits
  // at a fixed LDS offset from the thread's first (256 divides the tile
  // rows), so the stores take immediate offsets and no index registers.
  const int kt0 = k_tmajor ? tid & 31 : tid / (2 * DS);
  const int kd0 = k_tmajor ? tid >> 5 : tid % (2 * DS);
  const int vt0 = v_tmajor ? tid & 31 : tid / (32 * DVT);
  const int vd0 = v_tmajor ? tid >> 5 : tid % (32 * DVT);
  float *const ks_t = &ks[0][kt0 * DP + kd0];
  float *const vs_t = &vs[0][vd0 * VT + vt0];
  auto stage = [&](auto set, auto buf) __attribute__((always_inline)) {
    constexpr int R = decltype(set)::value, L = decltype(buf)::value;
    float *const kw = ks_t + L * 32 * DP;
    float *const vw = vs_t + L * 32 * DVT * VT;
    if (k_tmajor) {
#pragma unroll
      for (int e = 0; e < KE; e++) kw[8 * e] = kreg[R][e];
    } else {
#pragma unroll
      for (int e = 0; e < KE; e++) kw[e * (256 / (2 * DS)) * DP] = kreg[R][e];
    }
    if (v_tmajor) {
#pragma unroll
      for (int e = 0; e < VE; e++) vw[8 * e * VT] = vreg[R][e];
    } else {
#pragma unroll
      for (int e = 0; e < VE; e++) vw[e * (8 / DVT)] = vreg[R][e];
    }
  };
  using I0 = std::integral_constant<int, 0>;
  using I1 = std::integral_constant<int, 1>;

  // Q^T fragments: step s holds dim DS h + s of query q (lane half h takes
  // one half of the dims, so its K fragments are one contiguous LDS run).
  float qf[DS];
  {
    const float *qr = p.q + oq + (int64_t)(qok ? q : 0) * p.q_rs;
    // Contiguous, 16-byte aligned query rows with D % 4 == 0: 16-byte loads
    // (a quad of dims is wholly inside D or past it).
    const bool qvec = p.q_cs == 1 && (p.q_rs & 3) == 0 && (p.D & 3) == 0 &&
                      (reinterpret_cast<uintptr_t>(p.q + oq) & 15) == 0;
    if (qvec) {
#pragma unroll
      for (int i = 0; i < DS / 4; i++) {
        const int d = DS * h + 4 * i;
        const bool in = qok && d < p.D;
        const float4 x = *reinterpret_cast<const float4 *>(qr + (in ? d : 0));
        qf[4 * i] = in ? x.x : 0.f, qf[4 * i + 1] = in ? x.y : 0.f;
        qf[4 * i + 2] = in ? x.z : 0.f, qf[4 * i + 3] = in ? x.w : 0.f;
      }
    } else {
#pragma unroll
      for (int s = 0; s < DS; s++) {
        const int d = DS * h + s;
        const bool in = qok && d < p.D;
        const float x = qr[in ? d * (int)p.q_cs : 0];
        qf[s] = in ? x : 0.f;
      }
    }
  }
  float16v o[DVT];
#pragma unroll
  for (int j = 0; j < DVT; j++) o[j] = (float16v){};
  float m_run = -INFINITY, l_run = 0.f;
  float mcur[16];

  if (t_loop > t_begin) {
    fetch_any(t_begin, I0{});
    if constexpr (PD == 2) {
      if (t_loop > t_begin + 32) fetch_any(t_begin + 32, I1{});
      stage(I0{}, I0{});
    } else {
      stage(I0{}, I0{});
#pragma unroll
      for (int v = 0; v < 16; v++) mcur[v] = mreg[0][v];
      if (t_loop > t_begin + 32) fetch_any(t_begin + 32, I0{});
    }
  }
  // Scores in the log2 domain: p = 2^(s * scale * log2 e + mask * log2 e - m).
  constexpr float kLog2e = 1.4426950408889634f;
  const float scale2 = p.scale * kLog2e;
  __syncthreads();
  // Tile at t0 (parity B): its K/V are in LDS buffer B.  Two register
  // sets: its mask is in set B, set B is then refilled with the tile at
  // t0 + 64, and set 1 - B (the tile at t0 + 32, fetched one tile ago) is
  // staged into buffer 1 - B after the scores.  One set: its mask is in
  // mcur and the set holds the tile at t0 + 32, staged after the scores;
  // the tile at t0 + 64 is fetched next.
  auto tile = [&](int t0, auto bsel) __attribute__((always_inline)) {
    constexpr int B = decltype(bsel)::value;
    using NB = std::integral_constant<int, 1 - B>;
    if constexpr (PD == 2) {
#pragma unroll
      for (int v = 0; v < 16; v++) mcur[v] = mreg[B][v];
      if (t0 + 64 < t_loop) fetch_any(t0 + 64, bsel);
    }
    const bool full = t0 + 32 <= p.T;
    if (active) {
      const float *kl = &ks[B][0];
      const float *vl = &vs[B][0];
      // Scores S^T[t][q] for keys t0 .. t0 + 31.  The lane's K fragments
      // (key r32, dims DS h ..) are read with 16-byte loads, KC at a time.
      constexpr int KC = DS < 16 ? DS : 16;
      float16v sc = (float16v){};
#pragma unroll
      for (int c = 0; c < DS; c += KC) {
        float kf[KC];
#pragma unroll
        for (int i = 0; i < KC / 4; i++) {
          const float4 x =
              *reinterpret_cast<const float4 *>(kl + r32 * DP + DS * h + c + 4 * i);
          kf[4 * i] = x.x, kf[4 * i + 1] = x.y, kf[4 * i + 2] = x.z, kf[4 * i + 3] = x.w;
        }
#pragma unroll
        for (int s = 0; s < KC; s++)
          sc = __builtin_amdgcn_mfma_f32_32x32x2f32(kf[s], qf[c + s], sc, 0, 0, 0);
      }
      float pv[16];
      float tmax = -INFINITY;
#pragma unroll
      for (int v = 0; v < 16; v++) {
        const int tt = 8 * (v >> 2) + (v & 3) + 4 * h;  // key of slot v
        float x = fmaf(sc[v], scale2, mrow ? mcur[v] * kLog2e : 0.f);
        if ((!full && t0 + tt >= p.T) || (p.causal && t0 + tt > q + p.causal_off)) x = -INFINITY;
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
        // V^T fragments of dim 32 j + r32: keys t(s, h) of steps 4g .. 4g + 3
        // are the 4 consecutive keys 8g + 4h .., one 16-byte read each.
        float vf[16];
#pragma unroll
        for (int g = 0; g < 4; g++) {
          const float4 x =
              *reinterpret_cast<const float4 *>(vl + (32 * j + r32) * VT + 8 * g + 4 * h);
          vf[4 * g] = x.x, vf[4 * g + 1] = x.y, vf[4 * g + 2] = x.z, vf[4 * g + 3] = x.w;
        }
#pragma unroll
        for (int v = 0; v < 16; v++) o[j][v] *= corr;
#pragma unroll
        for (int s = 0; s < 16; s++)
          o[j] = __builtin_amdgcn_mfma_f32_32x32x2f32(vf[s], pv[s], o[j], 0, 0, 0);
      }
    }
    if (t0 + 32 < t_loop) {  // buffer 1 - B: its readers passed the last barrier
      if constexpr (PD == 2) {
        stage(NB{}, NB{});
      } else {
        stage(I0{}, NB{});
#pragma unroll
        for (int v = 0; v < 16; v++) mcur[v] = mreg[0][v];
        if (t0 + 64 < t_loop) fetch_any(t0 + 64, I0{});
      }
    }
    __syncthreads();
  };
  for (int t0 = t_begin; t0 < t_loop; t0 += 64) {
    tile(t0, I0{});
    if (t0 + 32 < t_loop) tile(t0 + 32, I1{});
  }

  const float l_tot = l_run + __shfl_xor(l_run, 32);
  if (!active || !qok) return;
  if (p.part) {
    // Partial of this key split: unnormalised O, the running max (log2
    // domain) and the sum, [split][batch index][query][attn_part_row(DV)].
    float *pr = p.part + (((int64_t)blockIdx.y * (gridDim.x / qtiles) + bi) * p.S + q) *
                             attn_part_row(p.DV);
#pragma unroll
    for (int j = 0; j < DVT; j++)
#pragma unroll
      for (int v = 0; v < 16; v++) {
        const int dv = 32 * j + 8 * (v >> 2) + 4 * h + (v & 3);
        if (dv < p.DV) pr[dv] = o[j][v];
      }
    if (h == 0) pr[p.DV] = m_run, pr[p.DV + 1] = l_tot;
    return;
  }
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

// Head sizes whose fragments and accumulators fit 256 registers run at two
// waves per SIMD (k_attn_o2); the larger ones keep one (with two, the
// compiler would spill them to scratch memory).
template <int DS, int DVT>
constexpr bool attn_two_waves = DS <= 16 || (DS <= 32 && DVT <= 2);

template <int DS, int DVT>
__global__ __launch_bounds__(256) void k_attn(const mg_attn_problem p) {
  attn_tiles<DS, DVT>(p);
}

template <int DS, int DVT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2))) void k_attn_o2(
    const mg_attn_problem p) {
  attn_tiles<DS, DVT>(p);
}

// Decode-shaped attention: at most 16 queries per batch index (a decode
// step, or GroupQueryAttention's query heads of one KV head), where the
// products are too thin for MFMA tiles and the work is reading K and V.
// Workgroup = one batch index and one key split, walked in blocks of 64
// keys: the 256 threads stage the block's K ([key][dim], padded rows) and V
// ([key][dim]) in LDS with coalesced loads; wave w owns queries w, w + 4, ...
// For each block a wave
//   * scores the 64 keys against its queries, lane = key, reading its K row
//     from LDS (odd pitch: no bank conflicts) and Q as LDS broadcasts;
//   * runs the online softmax per query (block max across the wave; each
//     lane keeps its share of the sum) and puts p in LDS;
//   * accumulates O, lane = output dim (DL dims per lane), reading V rows
//     and p from LDS.
// It writes y, or with several key splits the partials k_attn_combine merges.
// DMAX: the largest head size (Q/K and V) the LDS tiles hold, 128 or 256
// (Gemma-style heads; 150 KB of LDS, one workgroup per CU).
constexpr int DEC_S = 16;
template <int DL, int DMAX>
__global__ __launch_bounds__(256) void k_attn_dec(const mg_attn_problem p) {
  constexpr int KB = 64, KP = DMAX + 1;  // keys per block, K row pitch
  __shared__ float qs[DEC_S * DMAX];
  __shared__ float ks[KB * KP];
  __shared__ float vs[KB * DMAX];
  __shared__ float pls[DEC_S * KB];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t bi = blockIdx.x;
  int64_t oq = 0, ok = 0, ov = 0, om = 0, oy = 0;
  {
    int rem = (int)bi;  // the host keeps the grid below 2^31
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
  const int S = p.S, D = p.D, DV = p.DV;
  const int t_begin = p.kc > 0 ? (int)blockIdx.y * p.kc : 0;
  const int t_end = p.kc > 0 ? min(p.T, t_begin + p.kc) : p.T;
  for (int e = tid; e < S * D; e += 256) {
    const int q = e / D, d = e % D;
    qs[q * DMAX + d] = p.q[oq + (int64_t)q * p.q_rs + (int64_t)d * p.q_cs];
  }
  // Staging order: consecutive threads take consecutive addresses of
  // whichever index is contiguous in memory.
  const bool k_key_fast = p.k_ts == 1, v_key_fast = p.v_ts == 1;
  // Rows of 16-byte aligned, contiguous dims (the KV-cache layout): 16-byte
  // loads, all issued before the first store (indices clamped in range,
  // padding keys zeroed at the store).
  const bool rows4 = p.k_ds == 1 && p.v_ds == 1 && D % 4 == 0 && DV % 4 == 0 &&
                     p.k_ts % 4 == 0 && p.v_ts % 4 == 0 &&
                     reinterpret_cast<uintptr_t>(p.k + ok) % 16 == 0 &&
                     reinterpret_cast<uintptr_t>(p.v + ov) % 16 == 0;
  constexpr float kLog2e = 1.4426950408889634f;
  const float scale2 = p.scale * kLog2e;
  constexpr int QW = DEC_S / 4;  // queries per wave
  float m[QW], l[QW], o[QW][DL];
#pragma unroll
  for (int i = 0; i < QW; i++) {
    m[i] = -INFINITY, l[i] = 0.f;
#pragma unroll
    for (int j = 0; j < DL; j++) o[i][j] = 0.f;
  }
  for (int tb = t_begin; tb < t_end; tb += KB) {
    const int nk = min(KB, t_end - tb);
    __syncthreads();  // the previous block's readers are done
    if (rows4) {
      constexpr int C4 = KB * DMAX / 4 / 256;  // float4 per thread at DMAX dims
      const int d4 = D / 4, dv4 = DV / 4;
      float4 kx[C4], vx[C4];
#pragma unroll
      for (int u = 0; u < C4; u++) {
        const int c = tid + 256 * u;
        const int key = min(c / d4, nk - 1), d = (c % d4) * 4;
        kx[u] = *reinterpret_cast<const float4 *>(p.k + ok + (int64_t)(tb + key) * p.k_ts + d);
        const int vkey = min(c / dv4, nk - 1), vd = (c % dv4) * 4;
        vx[u] = *reinterpret_cast<const float4 *>(p.v + ov + (int64_t)(tb + vkey) * p.v_ts + vd);
      }
#pragma unroll
      for (int u = 0; u < C4; u++) {
        const int c = tid + 256 * u;
        if (c < KB * d4) {
          const int key = c / d4, d = (c % d4) * 4;
          const float4 x = key < nk ? kx[u] : make_float4(0.f, 0.f, 0.f, 0.f);
          float *dst = ks + key * KP + d;
          dst[0] = x.x, dst[1] = x.y, dst[2] = x.z, dst[3] = x.w;
        }
        if (c < KB * dv4) {
          const int key = c / dv4, d = (c % dv4) * 4;
          const float4 x = key < nk ? vx[u] : make_float4(0.f, 0.f, 0.f, 0.f);
          *reinterpret_cast<float4 *>(vs + key * DMAX + d) = x;
        }
      }
    } else {
    for (int e = tid; e < KB * D; e += 256) {
      const int key = k_key_fast ? e % KB : e / D, d = k_key_fast ? e / KB : e % D;
      ks[key * KP + d] =
          key < nk ? p.k[ok + (int64_t)(tb + key) * p.k_ts + (int64_t)d * p.k_ds] : 0.f;
    }
    for (int e = tid; e < KB * DV; e += 256) {
      const int key = v_key_fast ? e % KB : e / DV, d = v_key_fast ? e / KB : e % DV;
      vs[key * DMAX + d] =
          key < nk ? p.v[ov + (int64_t)(tb + key) * p.v_ts + (int64_t)d * p.v_ds] : 0.f;
    }
    }
    __syncthreads();
    const int t = tb + lane;
    const bool tok = lane < nk;
    float sc[QW];
#pragma unroll
    for (int i = 0; i < QW; i++) sc[i] = 0.f;
#pragma unroll 8
    for (int d = 0; d < D; d++) {
      const float kv = ks[lane * KP + d];
#pragma unroll
      for (int i = 0; i < QW; i++) sc[i] = fmaf(qs[(wave + 4 * i) * DMAX + d], kv, sc[i]);
    }
#pragma unroll
    for (int i = 0; i < QW; i++) {
      const int q = wave + 4 * i;
      if (q >= S) break;
      float x = -INFINITY;
      if (tok && !(p.causal && t > q + p.causal_off)) {
        const float mk = p.mask ? p.mask[om + (int64_t)q * p.m_qs + (int64_t)t * p.m_ts] : 0.f;
        x = fmaf(sc[i], scale2, mk * kLog2e);
      }
      float bm = x;
#pragma unroll
      for (int w = 32; w >= 1; w >>= 1) bm = fmaxf(bm, __shfl_xor(bm, w));
      const float m_new = fmaxf(m[i], bm);
      float pv = 0.f, corr = 1.f;
      if (m_new != -INFINITY) {
        corr = __builtin_amdgcn_exp2f(m[i] - m_new);  // 0 while nothing has been accumulated
        pv = __builtin_amdgcn_exp2f(x - m_new);
        m[i] = m_new;
      }
      l[i] = fmaf(l[i], corr, pv);  // the lane's share of the sum
#pragma unroll
      for (int j = 0; j < DL; j++) o[i][j] *= corr;
      pls[q * KB + lane] = pv;
    }
    // p rows of this wave only: the wave's LDS writes complete in order.
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
    __builtin_amdgcn_wave_barrier();
#pragma unroll 8
    for (int j = 0; j < nk; j++) {
      float vv[DL];
#pragma unroll
      for (int k = 0; k < DL; k++) vv[k] = vs[j * DMAX + lane + 64 * k];
#pragma unroll
      for (int i = 0; i < QW; i++) {
        const int q = wave + 4 * i;
        if (q >= S) break;
        const float pj = pls[q * KB + j];
#pragma unroll
        for (int k = 0; k < DL; k++) o[i][k] = fmaf(pj, vv[k], o[i][k]);
      }
    }
  }
#pragma unroll
  for (int i = 0; i < QW; i++) {
    const int q = wave + 4 * i;
    if (q >= S) break;
    float ls = l[i];
#pragma unroll
    for (int w = 32; w >= 1; w >>= 1) ls += __shfl_xor(ls, w);
    if (p.part) {
      float *pr = p.part + (((int64_t)blockIdx.y * gridDim.x + bi) * S + q) * attn_part_row(DV);
#pragma unroll
      for (int k = 0; k < DL; k++)
        if (lane + 64 * k < DV) pr[lane + 64 * k] = o[i][k];
      if (lane == 0) pr[DV] = m[i], pr[DV + 1] = ls;
    } else {
      const float inv = p.T == 0 ? 0.f : (m[i] == -INFINITY ? __builtin_nanf("") : 1.f / ls);
#pragma unroll
      for (int k = 0; k < DL; k++)
        if (lane + 64 * k < DV)
          p.y[oy + (int64_t)q * p.y_rs + lane + 64 * k] = p.T == 0 ? 0.f : o[i][k] * inv;
    }
  }
}

// More than eight splits: eight per step with independent loads (a loop of
// one load per split would wait out the memory latency once per split), a
// pass for the maximum, then the ordered sum.
template <class Add>
__device__ inline void combine_many(const float *p0, int64_t cs, int nsplit, int dv, int DV,
                                    float &M, Add &add) {
  int c = 0;
  for (; c + 8 <= nsplit; c += 8) {
    float mm[8];
#pragma unroll
    for (int u = 0; u < 8; u++) mm[u] = p0[(c + u) * cs + DV];
#pragma unroll
    for (int u = 0; u < 8; u++) M = fmaxf(M, mm[u]);
  }
  for (; c < nsplit; c++) M = fmaxf(M, p0[c * cs + DV]);
  if (M == -INFINITY) return;
  c = 0;
  for (; c + 8 <= nsplit; c += 8) {
    float mm[8], oo[8], ll[8];
#pragma unroll
    for (int u = 0; u < 8; u++) {
      const float *pr = p0 + (c + u) * cs;
      mm[u] = pr[DV], oo[u] = pr[dv], ll[u] = pr[DV + 1];
    }
#pragma unroll
    for (int u = 0; u < 8; u++) add(mm[u], oo[u], ll[u]);
  }
  for (; c < nsplit; c++) {
    const float *pr = p0 + c * cs;
    add(pr[DV], pr[dv], pr[DV + 1]);
  }
}

// Merges the key splits of each (batch index, query): with M the largest
// split max, y = sum_c 2^(m_c - M) O_c / sum_c 2^(m_c - M) l_c; every score
// -inf gives NaN, as without splits.  One thread per output element.
__global__ __launch_bounds__(256) void k_attn_combine(const mg_attn_problem p, int nsplit,
                                                      int64_t nbatch) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t n = nbatch * p.S * p.DV;
  if (idx >= n) return;
  int dv, q;
  int64_t row, bi;  // row = bi * S + q
  if (n < ((int64_t)1 << 31)) {  // 32-bit divisions where the indices allow
    const unsigned i32 = (unsigned)idx, r32 = i32 / (unsigned)p.DV;
    dv = (int)(i32 - r32 * (unsigned)p.DV);
    q = (int)(r32 % (unsigned)p.S);
    row = r32;
    bi = r32 / (unsigned)p.S;
  } else {
    dv = (int)(idx % p.DV);
    row = idx / p.DV;
    q = (int)(row % p.S);
    bi = row / p.S;
  }
  const float *p0 = p.part + row * attn_part_row(p.DV);
  const int64_t cs = nbatch * p.S * attn_part_row(p.DV);  // stride between splits
  float M = -INFINITY, num = 0.f, den = 0.f;
  auto add = [&](float m, float o, float l) {
    const float w = m == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m - M);
    num = fmaf(w, o, num);
    den = fmaf(w, l, den);
  };
  if (nsplit <= 8) {
    // Every split's max, value and sum loaded at once (one memory round
    // trip); the same maximum and ordered sum as combine_many.
    float mm[8], oo[8], ll[8];
#pragma unroll
    for (int u = 0; u < 8; u++) {
      const float *pr = p0 + (u < nsplit ? u : 0) * cs;
      mm[u] = pr[p.DV], oo[u] = pr[dv], ll[u] = pr[p.DV + 1];
    }
#pragma unroll
    for (int u = 0; u < 8; u++)
      if (u < nsplit) M = fmaxf(M, mm[u]);
    if (M != -INFINITY) {
#pragma unroll
      for (int u = 0; u < 8; u++)
        if (u < nsplit) add(mm[u], oo[u], ll[u]);
    }
  } else {
    combine_many(p0, cs, nsplit, dv, (int)p.DV, M, add);
  }
  int64_t oy = 0;
  unsigned rem = (unsigned)bi;  // batch indices: below 2^31 (the host's grid bound)
  for (int d = p.nbd - 1; d >= 0; d--) {
    const unsigned bd = (unsigned)p.bdim[d];
    oy += (int64_t)(rem % bd) * p.y_bs[d];
    rem /= bd;
  }
  p.y[oy + (int64_t)q * p.y_rs + dv] = M == -INFINITY ? __builtin_nanf("") : num / den;
}

// k_attn_combine for four outputs of a row per thread (DV % 4 == 0 and
// 16-byte aligned output rows): each split's four values in one 16-byte
// load and its max and sum once for the four; per output the same maximum
// and ordered sum.
__global__ __launch_bounds__(256) void k_attn_combine4(const mg_attn_problem p, int nsplit,
                                                       int64_t nbatch) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t n = nbatch * p.S * (p.DV / 4);
  if (idx >= n) return;
  const int dq = (int)p.DV / 4;
  int dv, q;
  int64_t row, bi;
  if (n < ((int64_t)1 << 31)) {
    const unsigned i32 = (unsigned)idx, r32 = i32 / (unsigned)dq;
    dv = 4 * (int)(i32 - r32 * (unsigned)dq);
    q = (int)(r32 % (unsigned)p.S);
    row = r32;
    bi = r32 / (unsigned)p.S;
  } else {
    dv = 4 * (int)(idx % dq);
    row = idx / dq;
    q = (int)(row % p.S);
    bi = row / p.S;
  }
  const float *p0 = p.part + row * attn_part_row(p.DV);
  const int64_t cs = nbatch * p.S * attn_part_row(p.DV);
  float M = -INFINITY;
  float num[4] = {0.f, 0.f, 0.f, 0.f}, den = 0.f;
  auto add = [&](float m, const float4 &o, float l) {
    const float w = m == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m - M);
    num[0] = fmaf(w, o.x, num[0]);
    num[1] = fmaf(w, o.y, num[1]);
    num[2] = fmaf(w, o.z, num[2]);
    num[3] = fmaf(w, o.w, num[3]);
    den = fmaf(w, l, den);
  };
  for (int c0 = 0; c0 < nsplit; c0 += 8) {  // the maximum, eight splits' loads at once
    float mm[8];
#pragma unroll
    for (int u = 0; u < 8; u++) mm[u] = p0[(c0 + u < nsplit ? c0 + u : c0) * cs + p.DV];
#pragma unroll
    for (int u = 0; u < 8; u++)
      if (c0 + u < nsplit) M = fmaxf(M, mm[u]);
  }
  if (M != -INFINITY) {
    for (int c0 = 0; c0 < nsplit; c0 += 8) {
      float mm[8], ll[8];
      float4 oo[8];
#pragma unroll
      for (int u = 0; u < 8; u++) {
        const float *pr = p0 + (c0 + u < nsplit ? c0 + u : c0) * cs;
        mm[u] = pr[p.DV], ll[u] = pr[p.DV + 1];
        oo[u] = *reinterpret_cast<const float4 *>(pr + dv);
      }
#pragma unroll
      for (int u = 0; u < 8; u++)
        if (c0 + u < nsplit) add(mm[u], oo[u], ll[u]);
    }
  }
  int64_t oy = 0;
  unsigned rem = (unsigned)bi;
  for (int d = p.nbd - 1; d >= 0; d--) {
    const unsigned bd = (unsigned)p.bdim[d];
    oy += (int64_t)(rem % bd) * p.y_bs[d];
    rem /= bd;
  }
  float4 out;
  if (M == -INFINITY) {
    out = make_float4(__builtin_nanf(""), __builtin_nanf(""), __builtin_nanf(""),
                      __builtin_nanf(""));
  } else {
    out = make_float4(num[0] / den, num[1] / den, num[2] / den, num[3] / den);
  }
  *reinterpret_cast<float4 *>(p.y + oy + (int64_t)q * p.y_rs + dv) = out;
}

// The merge for many splits (9 .. 64) and value heads up to 128: one wave
// per query row, every load of the row in flight at once (split c's max and
// sum in lane c, its outputs in lane dv's registers), then the maximum and
// the ordered sum over splits read lane by lane: per output the same
// arithmetic in the same order as k_attn_combine, in one memory round trip
// instead of one per eight splits.
template <int DPL>
__global__ __launch_bounds__(256) void k_attn_combine_w(const mg_attn_problem p, int nsplit,
                                                        int64_t nbatch) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= nbatch * p.S) return;  // whole waves
  const int64_t bi = row / p.S;
  const int q = (int)(row % p.S);
  const float *p0 = p.part + row * attn_part_row(p.DV);
  const int64_t cs = nbatch * p.S * attn_part_row(p.DV);
  const int DV = (int)p.DV;
  const float mc = lane < nsplit ? p0[lane * cs + DV] : -INFINITY;
  const float lc = lane < nsplit ? p0[lane * cs + DV + 1] : 0.f;
  float o[DPL][64];
#pragma unroll
  for (int c = 0; c < 64; c++)
#pragma unroll
    for (int e = 0; e < DPL; e++) {
      const int dv = lane + 64 * e;
      o[e][c] = c < nsplit && dv < DV ? p0[c * cs + dv] : 0.f;
    }
  float M = -INFINITY;
#pragma unroll
  for (int c = 0; c < 64; c++)
    if (c < nsplit)
      M = fmaxf(M, __builtin_bit_cast(float,
                                      __builtin_amdgcn_readlane(__builtin_bit_cast(int, mc), c)));
  float num[DPL], den = 0.f;
#pragma unroll
  for (int e = 0; e < DPL; e++) num[e] = 0.f;
  if (M != -INFINITY) {
    const float w = mc == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mc - M);
#pragma unroll
    for (int c = 0; c < 64; c++) {
      if (c < nsplit) {
        const float wc = __builtin_bit_cast(
            float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, w), c));
        const float lcc = __builtin_bit_cast(
            float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, lc), c));
#pragma unroll
        for (int e = 0; e < DPL; e++) num[e] = fmaf(wc, o[e][c], num[e]);
        den = fmaf(wc, lcc, den);
      }
    }
  }
  int64_t oy = 0;
  unsigned rem = (unsigned)bi;
  for (int d = p.nbd - 1; d >= 0; d--) {
    const unsigned bd = (unsigned)p.bdim[d];
    oy += (int64_t)(rem % bd) * p.y_bs[d];
    rem /= bd;
  }
  float *yr = p.y + oy + (int64_t)q * p.y_rs;
#pragma unroll
  for (int e = 0; e < DPL; e++) {
    const int dv = lane + 64 * e;
    if (dv < DV) yr[dv] = M == -INFINITY ? __builtin_nanf("") : num[e] / den;
  }
}

// Launches the merge of nsplit key splits of the outputs of p.
mg_status launch_combine(const mg_attn_problem &p, int nsplit, int64_t nbatch, hipStream_t st) {
  bool v4 = p.DV % 4 == 0 && reinterpret_cast<uintptr_t>(p.y) % 16 == 0 && p.y_rs % 4 == 0;
  for (int d = 0; d < p.nbd; d++) v4 = v4 && p.y_bs[d] % 4 == 0;
  if (nsplit > 8 && nsplit <= 64 && p.DV <= 128) {
    const unsigned g = (unsigned)((nbatch * p.S + 3) / 4);
    if (p.DV <= 64)
      hipLaunchKernelGGL(k_attn_combine_w<1>, dim3(g), dim3(256), 0, st, p, nsplit, nbatch);
    else
      hipLaunchKernelGGL(k_attn_combine_w<2>, dim3(g), dim3(256), 0, st, p, nsplit, nbatch);
  } else if (v4) {
    const int64_t n = nbatch * p.S * (p.DV / 4);
    hipLaunchKernelGGL(k_attn_combine4, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, p,
                       nsplit, nbatch);
  } else {
    const int64_t n = nbatch * p.S * p.DV;
    hipLaunchKernelGGL(k_attn_combine, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, p,
                       nsplit, nbatch);
  }
  return mg_launch_check("k_attn_combine");
}

template <int DS, int DVT>
void launch_attn(const mg_attn_problem &p, dim3 grid, hipStream_t st) {
  if constexpr (attn_two_waves<DS, DVT>)
    hipLaunchKernelGGL((k_attn_o2<DS, DVT>), grid, dim3(256), 0, st, p);
  else
    hipLaunchKernelGGL((k_attn<DS, DVT>), grid, dim3(256), 0, st, p);
}

template <int DS>
void launch_dvt(const mg_attn_problem &p, dim3 grid, hipStream_t st) {
  if (p.DV <= 32) {
    launch_attn<DS, 1>(p, grid, st);
  } else if constexpr (DS > 64) {  // value chunks of 64 (mg_attn_run)
    launch_attn<DS, 2>(p, grid, st);
  } else {
    if (p.DV <= 64)
      launch_attn<DS, 2>(p, grid, st);
    else
      launch_attn<DS, 4>(p, grid, st);
  }
}

}  // namespace

mg_status mg_attn_run(mg_ctx *ctx, const mg_attn_problem &p) {
  if (p.D > 256 || p.DV > 256)
    return mg_fail(MG_UNSUPPORTED, "attention: head sizes above 256 are not supported");
  if (p.nbd > MG_ATTN_MAX_BATCH_DIMS)
    return mg_fail(MG_UNSUPPORTED, "attention: more than 4 batch dimensions");
  int64_t nbatch = 1;
  for (int d = 0; d < p.nbd; d++) nbatch *= p.bdim[d];
  if (nbatch == 0 || p.S == 0 || p.DV == 0) return MG_OK;
  const bool dec = p.S <= DEC_S;
  const int64_t wgs = dec ? nbatch : nbatch * ((p.S + 127) / 128);
  if (wgs > 0x7fffffff) return mg_fail(MG_UNSUPPORTED, "attention: grid too large");
  const int nsplit = p.kc > 0 ? (p.T + p.kc - 1) / p.kc : 1;
  if (p.kc > 0 && !p.part) return mg_fail(MG_INVALID_ARGUMENT, "attention: no partial buffer");
  const dim3 grid((unsigned)wgs, (unsigned)nsplit);
  if (dec) {
    if (p.D > 128 || p.DV > 128)
      hipLaunchKernelGGL((k_attn_dec<4, 256>), grid, dim3(256), 0, ctx->stream, p);
    else if (p.DV <= 64)
      hipLaunchKernelGGL((k_attn_dec<1, 128>), grid, dim3(256), 0, ctx->stream, p);
    else
      hipLaunchKernelGGL((k_attn_dec<2, 128>), grid, dim3(256), 0, ctx->stream, p);
    MG_TRY(mg_launch_check("k_attn_dec"));
    if (p.kc > 0) return launch_combine(p, nsplit, nbatch, ctx->stream);
    return MG_OK;
  }
  // Value heads above 128 (above 64 with query/key heads above 128, whose
  // 128 Q values per lane leave no registers for a fourth accumulator tile)
  // run as column chunks: each chunk computes the same scores in the same
  // order, so its softmax weights are bitwise those of the others.  A chunk's
  // partials use the front of the buffer planned for the whole head.
  const int chunk = p.D > 128 ? 64 : 128;
  for (int c0 = 0; c0 < p.DV; c0 += chunk) {
    mg_attn_problem pp = p;
    pp.v = p.v + (int64_t)c0 * p.v_ds;
    pp.y = p.y + c0;
    pp.DV = std::min(chunk, p.DV - c0);
    if (p.D == 0) {  // no products: the kernel's (masked-off) Q and K loads read V instead
      pp.q = pp.k = pp.v;
      pp.q_rs = pp.q_cs = pp.k_ts = pp.k_ds = 0;
      for (int d = 0; d < MG_ATTN_MAX_BATCH_DIMS; d++) pp.q_bs[d] = pp.k_bs[d] = 0;
    }
    if (p.D <= 32)
      launch_dvt<16>(pp, grid, ctx->stream);
    else if (p.D <= 64)
      launch_dvt<32>(pp, grid, ctx->stream);
    else if (p.D <= 128)
      launch_dvt<64>(pp, grid, ctx->stream);
    else
      launch_dvt<128>(pp, grid, ctx->stream);
    MG_TRY(mg_launch_check("k_attn"));
    if (p.kc > 0) MG_TRY(launch_combine(pp, nsplit, nbatch, ctx->stream));
  }
  return MG_OK;
}

// Key split for grids that leave the CUs idle (decode-like shapes: few
// queries, many keys): about two workgroups per CU,
// splits of at least 64 keys (a multiple of 32).  Sets p->kc and returns the
// bytes of the partial buffer the caller provides in p->part (0 = no split).
size_t mg_attn_plan_split(const mg_ctx *ctx, mg_attn_problem *p) {
  p->kc = 0;
  int64_t nbatch = 1;
  for (int d = 0; d < p->nbd; d++) nbatch *= p->bdim[d];
  // Decode-shaped problems (k_attn_dec) split in multiples of its 64-key
  // blocks, the tiled kernel in multiples of 32.
  const bool dec = p->S <= DEC_S;
  const int64_t gran = dec ? 64 : 32;
  const int64_t wgs = dec ? nbatch : nbatch * ((p->S + 127) / 128);
  if (wgs == 0 || p->T < 128 || p->DV == 0 || wgs >= ctx->num_cus) return 0;
  const int64_t want = std::min<int64_t>((2 * ctx->num_cus + wgs - 1) / wgs,
                                         (p->T + gran - 1) / gran);
  if (want < 2) return 0;
  const int64_t kc = ((p->T + want - 1) / want + gran - 1) / gran * gran;
  const int64_t nsplit = (p->T + kc - 1) / kc;
  if (nsplit < 2) return 0;
  p->kc = (int)kc;
  return (size_t)(nsplit * nbatch * p->S * attn_part_row(p->DV)) * 4;
}

// ------------------------------------------------------ GroupQueryAttention

namespace {

// RoPE of element d of one head row x (lib/src/onnx_ops.dart:2693-2716):
// computed in double and rounded once to f32, as the reference's
// Float32List stores of double expressions do.
__device__ inline float rope(const float *x, int64_t d, int64_t half_rot, const float *c,
                             const float *sn, int interleaved) {
  if (d >= 2 * half_rot) return x[d];
  if (interleaved) {
    const int64_t i = d >> 1;
    const double cc = c[i], ss = sn[i];
    return (d & 1) ? (float)((double)x[d] * cc + (double)x[d - 1] * ss)
                   : (float)((double)x[d] * cc - (double)x[d + 1] * ss);
  }
  if (d < half_rot) {
    const double cc = c[d], ss = sn[d];
    return (float)((double)x[d] * cc - (double)x[d + half_rot] * ss);
  }
  const int64_t i = d - half_rot;
  const double cc = c[i], ss = sn[i];
  return (float)((double)x[d] * cc + (double)x[i] * ss);
}

// rope() for the four elements d .. d + 3 (d % 4 == 0) of one head row with
// 16-byte loads of the row, its rotation partner and the cos / sin row
// (8-byte ones interleaved): half_rot % 4 == 0 (interleaved: % 2 == 0), so
// the four lie on one side of every boundary.  Per element the arithmetic
// of rope().
__device__ inline float4 rope4(const float *x, int64_t d, int64_t half_rot, const float *c,
                               const float *sn, int interleaved) {
  auto ld4 = [](const float *ptr) { return *reinterpret_cast<const float4 *>(ptr); };
  const float4 X = ld4(x + d);
  if (d >= 2 * half_rot) return X;
  if (interleaved) {
    const int64_t i = d >> 1;
    const float2 C = *reinterpret_cast<const float2 *>(c + i);
    const float2 S = *reinterpret_cast<const float2 *>(sn + i);
    return make_float4((float)((double)X.x * (double)C.x - (double)X.y * (double)S.x),
                       (float)((double)X.y * (double)C.x + (double)X.x * (double)S.x),
                       (float)((double)X.z * (double)C.y - (double)X.w * (double)S.y),
                       (float)((double)X.w * (double)C.y + (double)X.z * (double)S.y));
  }
  if (d < half_rot) {
    const float4 Y = ld4(x + d + half_rot), C = ld4(c + d), S = ld4(sn + d);
    return make_float4((float)((double)X.x * (double)C.x - (double)Y.x * (double)S.x),
                       (float)((double)X.y * (double)C.y - (double)Y.y * (double)S.y),
                       (float)((double)X.z * (double)C.z - (double)Y.z * (double)S.z),
                       (float)((double)X.w * (double)C.w - (double)Y.w * (double)S.w));
  }
  const int64_t i = d - half_rot;
  const float4 Y = ld4(x + i), C = ld4(c + i), S = ld4(sn + i);
  return make_float4((float)((double)X.x * (double)C.x + (double)Y.x * (double)S.x),
                     (float)((double)X.y * (double)C.y + (double)Y.y * (double)S.y),
                     (float)((double)X.z * (double)C.z + (double)Y.z * (double)S.z),
                     (float)((double)X.w * (double)C.w + (double)Y.w * (double)S.w));
}

// One thread per VEC consecutive elements (along the head dim) of present
// K/V (both written) and, when rotary, of the rotated Q.  Groups [0, nkv)
// are the caches, [nkv, nkv + nq) Q.  VEC = 4 needs head_size % 4 == 0 and
// 16-byte aligned tensors (checked by the host): the cache copies are then
// 16-byte loads and stores.  IX: the index type (32-bit where every element
// index fits, as divisions by the runtime sizes then cost a fraction of the
// 64-bit ones).  RQ (VEC = 4): the rotations and the new V rows by whole
// quads (rope4), with every operand 16-byte aligned.
template <int VEC, class IX, bool RQ>
__global__ __launch_bounds__(256) void k_gqa_prep(const mg_gqa_prep g, int64_t nkv, int64_t nq) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= nkv + nq) return;
  const IX total = (IX)(g.past + g.seq), hs = (IX)g.hs;
  if (idx < nkv) {
    const IX e = (IX)(idx * VEC);
    const IX d = e % hs, j = (e / hs) % total, bh = e / (hs * total);
    const IX kvh = bh % (IX)g.kv_heads, b = bh / (IX)g.kv_heads;
    if (j < g.past) {
      const int64_t src = (bh * g.past + j) * g.hs + d;
      if (VEC == 4) {
        *reinterpret_cast<float4 *>(g.present_k + e) = *reinterpret_cast<const float4 *>(g.past_k + src);
        *reinterpret_cast<float4 *>(g.present_v + e) = *reinterpret_cast<const float4 *>(g.past_v + src);
      } else {
        g.present_k[e] = g.past_k[src];
        g.present_v[e] = g.past_v[src];
      }
    } else {
      const int64_t s = j - g.past;
      const int64_t row = (b * g.seq + s) * g.kv_heads * g.hs + kvh * g.hs;
      const float *c = g.cos + (g.past + s) * g.half_rot, *sn = g.sin + (g.past + s) * g.half_rot;
      if constexpr (RQ) {
        *reinterpret_cast<float4 *>(g.present_k + e) =
            g.rotary ? rope4(g.k + row, d, g.half_rot, c, sn, g.interleaved)
                     : *reinterpret_cast<const float4 *>(g.k + row + d);
        *reinterpret_cast<float4 *>(g.present_v + e) =
            *reinterpret_cast<const float4 *>(g.v + row + d);
        return;
      }
#pragma unroll
      for (int u = 0; u < VEC; u++) {
        g.present_k[e + u] = g.rotary ? rope(g.k + row, d + u, g.half_rot, c, sn, g.interleaved)
                                      : g.k[row + d + u];
        g.present_v[e + u] = g.v[row + d + u];
      }
    }
    return;
  }
  const IX e = (IX)((idx - nkv) * VEC);  // rotated Q, [batch][seq][heads * hs]
  const IX d = e % hs, row = e - d;
  const IX s = (e / ((IX)g.heads * hs)) % (IX)g.seq;
  if constexpr (RQ) {
    *reinterpret_cast<float4 *>(g.q_rot + e) =
        rope4(g.q + row, d, g.half_rot, g.cos + (g.past + s) * g.half_rot,
              g.sin + (g.past + s) * g.half_rot, g.interleaved);
    return;
  }
#pragma unroll
  for (int u = 0; u < VEC; u++)
    g.q_rot[e + u] = rope(g.q + row, d + u, g.half_rot, g.cos + (g.past + s) * g.half_rot,
                          g.sin + (g.past + s) * g.half_rot, g.interleaved);
}

// The aligned, whole-quad case (RQ) by cache blocks: workgroup x < nbh * pbb
// takes block bh = x / pbb (batch x KV head, a scalar division) and 256
// consecutive quads of its present K and V rows (one per thread).  The past
// part of a block is one contiguous run, present[bh][0 .. past hs) =
// past[bh][0 .. past hs), so it needs no per-element index division; the
// new rows (RoPE'd K, raw V) follow.  Workgroups past nbh * pbb rotate Q,
// one quad per thread, as k_gqa_prep.
__global__ __launch_bounds__(256) void k_gqa_prep_blk(const mg_gqa_prep g, int nbh, int pbb,
                                                      int nq4) {
  const int xb = blockIdx.x;
  const int tid = threadIdx.x;
  const int hs4 = (int)g.hs / 4, past4 = (int)g.past * hs4, tot4 = (int)(g.past + g.seq) * hs4;
  if (xb < nbh * pbb) {
    const int bh = xb / pbb;
    const int x = (xb - bh * pbb) * 256 + tid;
    float4 *ok = reinterpret_cast<float4 *>(g.present_k) + (int64_t)bh * tot4;
    float4 *ov = reinterpret_cast<float4 *>(g.present_v) + (int64_t)bh * tot4;
    if (x < past4) {
      ok[x] = reinterpret_cast<const float4 *>(g.past_k)[(int64_t)bh * past4 + x];
      ov[x] = reinterpret_cast<const float4 *>(g.past_v)[(int64_t)bh * past4 + x];
    } else if (x < tot4) {
      const int r = x - past4, s = r / hs4, d = (r - s * hs4) * 4;
      const int b = bh / (int)g.kv_heads, kvh = bh - b * (int)g.kv_heads;
      const int64_t row = ((int64_t)b * g.seq + s) * g.kv_heads * g.hs + (int64_t)kvh * g.hs;
      const float *c = g.cos + (g.past + s) * g.half_rot, *sn = g.sin + (g.past + s) * g.half_rot;
      ok[x] = g.rotary ? rope4(g.k + row, d, g.half_rot, c, sn, g.interleaved)
                       : *reinterpret_cast<const float4 *>(g.k + row + d);
      ov[x] = *reinterpret_cast<const float4 *>(g.v + row + d);
    }
    return;
  }
  const int i4 = (xb - nbh * pbb) * 256 + tid;
  if (i4 >= nq4) return;
  const int64_t e = (int64_t)i4 * 4;  // rotated Q, [batch][seq][heads * hs]
  const int64_t d = e % g.hs, row = e - d;
  const int64_t s = (e / (g.heads * g.hs)) % g.seq;
  *reinterpret_cast<float4 *>(g.q_rot + e) =
      rope4(g.q + row, d, g.half_rot, g.cos + (g.past + s) * g.half_rot,
            g.sin + (g.past + s) * g.half_rot, g.interleaved);
}

}  // namespace

mg_status mg_gqa_prep_run(mg_ctx *ctx, const mg_gqa_prep &g) {
  auto al = [](const void *ptr) { return reinterpret_cast<uintptr_t>(ptr) % 16 == 0; };
  const bool v4 = g.hs % 4 == 0 && al(g.present_k) && al(g.present_v) &&
                  (g.past == 0 || (al(g.past_k) && al(g.past_v)));
  const int vec = v4 ? 4 : 1;
  const int64_t nkv = g.batch * g.kv_heads * (g.past + g.seq) * g.hs / vec;
  const int64_t nq = g.rotary ? g.batch * g.seq * g.heads * g.hs / vec : 0;
  if (nkv + nq == 0) return MG_OK;
  const int64_t blocks = (nkv + nq + 255) / 256;
  if (blocks > 0x7fffffff) return mg_fail(MG_UNSUPPORTED, "GroupQueryAttention: too large");
  const bool i32 = std::max(nkv, nq) * vec < ((int64_t)1 << 31);
  // Quads of the rotation: the rotated halves (interleaved: pairs) hold
  // whole quads, and the inputs, Q's output and the cos / sin rows are
  // aligned for 16-byte (interleaved cos / sin: 8-byte) loads.
  const bool rq =
      v4 && al(g.k) && al(g.v) && (!g.rotary || ((g.interleaved ? g.half_rot % 2 == 0
                                                                 : g.half_rot % 4 == 0) &&
                                                 al(g.q) && al(g.q_rot) &&
                                                 reinterpret_cast<uintptr_t>(g.cos) % 16 == 0 &&
                                                 reinterpret_cast<uintptr_t>(g.sin) % 16 == 0));
#ifndef MG_GQA_PREP_BLK
#define MG_GQA_PREP_BLK 1
#endif
  // (32-bit block indices: every block and the grid below 2^31.)
  const int64_t nbh = g.batch * g.kv_heads, tot4 = (g.past + g.seq) * g.hs / 4;
  const int64_t pbb = (tot4 + 255) / 256;
  const int64_t nq4 = g.rotary ? g.batch * g.seq * g.heads * g.hs / 4 : 0;
  const int64_t nblk = nbh * pbb + (nq4 + 255) / 256;
  if (MG_GQA_PREP_BLK && rq && nblk < 0x7fffffff && tot4 < 0x7fffffff && nq4 < 0x7fffffff) {
    hipLaunchKernelGGL(k_gqa_prep_blk, dim3((unsigned)nblk), dim3(256), 0, ctx->stream, g,
                       (int)nbh, (int)pbb, (int)nq4);
    return mg_launch_check("k_gqa_prep_blk");
  }
  const dim3 grid((unsigned)blocks);
  if (rq && i32)
    hipLaunchKernelGGL((k_gqa_prep<4, uint32_t, true>), grid, dim3(256), 0, ctx->stream, g, nkv,
                       nq);
  else if (rq)
    hipLaunchKernelGGL((k_gqa_prep<4, int64_t, true>), grid, dim3(256), 0, ctx->stream, g, nkv,
                       nq);
  else if (v4 && i32)
    hipLaunchKernelGGL((k_gqa_prep<4, uint32_t, false>), grid, dim3(256), 0, ctx->stream, g, nkv,
                       nq);
  else if (v4)
    hipLaunchKernelGGL((k_gqa_prep<4, int64_t, false>), grid, dim3(256), 0, ctx->stream, g, nkv,
                       nq);
  else if (i32)
    hipLaunchKernelGGL((k_gqa_prep<1, uint32_t, false>), grid, dim3(256), 0, ctx->stream, g, nkv,
                       nq);
  else
    hipLaunchKernelGGL((k_gqa_prep<1, int64_t, false>), grid, dim3(256), 0, ctx->stream, g, nkv,
                       nq);
  return mg_launch_check("k_gqa_prep");
}
