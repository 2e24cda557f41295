// fp32 MatMul / Gemm on gfx950 fp32 MFMA (v_mfma_f32_32x32x2_f32).
//
// Reference semantics: opMatMul (numpy broadcast, lib/src/onnx_ops.dart:
// 1710-1766) and opGemm (alpha * op(A) op(B) + beta * C,
// lib/src/onnx_ops.dart:2152-2172).  The MFMA multiplies fp32 operands exactly
// and accumulates in fp32, so results differ from the reference's sequential
// k-order sums only by accumulation order.
//
// Workgroup tile 128 x 128 (four waves as 2 x 2 of 64 x 64, i.e. 2 x 2 MFMA
// tiles of 32 x 32 each) with stages of 16 k or, when that grid would not
// fill the chip, 64 x 64 (one MFMA tile per wave) with stages of 32 k (16 k
// for grids beyond four workgroups per CU).  Each stage is double-buffered in
// LDS as Xs[row][k] (k contiguous, rows padded by 4 floats so 16-byte reads
// do not collide on banks) for both operands.
// Within a stage, MFMA step s gives lane l the k = 2 s + l / 32: LDS rows
// hold their even k, then their odd k, so each lane still reads its KS / 2
// k of a row with 16-byte LDS loads, and every output adds the k pairs in
// order whatever the stage size and tile (plans agree bit for bit).
// Operands may be stored k-contiguous ("RK": A [M][K], B^T [N][K]) or
// row-contiguous ("KR": A^T [K][M], B [K][N]); the stage loader reads 32
// bytes per thread either way and transposes KR tiles on their way into LDS.
// Where rows are 16-byte aligned and the contiguous extent is a multiple of
// 4 it uses raw buffer loads with out-of-range quads reading as zeros (no
// branches, so the loads of the next stage stay in flight across the current
// stage's products; the branchy form waited for them at once).
// Batches run on grid.z; each workgroup decodes its batch's operand offsets
// from the broadcast strides it receives as an argument (numpy broadcasting,
// lib/src/onnx_ops.dart:1742-1764).
//
// Tile order.  Workgroups are dealt to the chip's 8 XCDs round-robin
// (workgroup L runs on XCD L % 8) and each XCD has its own L2.  When the
// tile grid is large enough, it is cut into pr row bands x pc column bands
// (pr * pc = 8) and XCD j takes the tiles of rectangle j, so a row tile of A
// is fetched by pc XCDs and a column tile of B by pr, instead of both by
// all 8.  The host picks the cut that fetches the fewest bytes.
#include <hip/hip_runtime.h>

#include <algorithm>

#include "mg_internal.h"

namespace {

typedef float float16v __attribute__((ext_vector_type(16)));


// One operand's stage for a workgroup tile of T = 64 WT rows: rows
// [r0, r0 + T) x k [k0, k0 + KS) of X, E = KS T / 256 floats per thread,
// zero outside [R, K).  KR: X stored [K][R] (element (r, k) at k * ld + r),
// else [R][K] (r * ld + k).  In LDS a row holds KS floats padded to LDX.
template <int WT, int KS, bool KR>
struct Stage {
  static constexpr int T = 64 * WT, E = KS * T / 256, LDX = KS + 4;
  float v[E];

  // fast: the stage lies inside X and 16-byte loads are aligned (decided per
  // workgroup and stage, so the branch is uniform).
  __device__ inline void load(const float *__restrict__ X, bool fast, int64_t ld, int64_t R,
                              int64_t K, int64_t r0, int64_t k0, int t) {
    const int64_t r = KR ? r0 + (t % (T / E)) * E : r0 + t / (KS / E);
    const int64_t k = KR ? k0 + t / (T / E) : k0 + (t % (KS / E)) * E;
    const float *p = KR ? X + k * ld + r : X + r * ld + k;
    if (fast) {
#pragma unroll
      for (int q = 0; q < E / 4; q++) {
        const float4 x = *reinterpret_cast<const float4 *>(p + 4 * q);
        v[4 * q] = x.x; v[4 * q + 1] = x.y; v[4 * q + 2] = x.z; v[4 * q + 3] = x.w;
      }
    } else {
#pragma unroll
      for (int e = 0; e < E; e++)
        v[e] = (KR ? (k < K && r + e < R) : (r < R && k + e < K)) ? p[e] : 0.f;
    }
  }

  // Branch-free form (raw buffer loads): 16-byte quads of E / 4 consecutive
  // elements along the contiguous index; a quad past the tensor (row >= R or
  // k >= K) gets an offset past the resource and reads as zeros in hardware.
  // Needs 16-byte aligned rows and the contiguous extent (K, or R for KR) a
  // multiple of 4, so that a quad is wholly inside or outside, and byte
  // offsets below 2^31 (all checked by the host).
  __device__ inline void load_b(__amdgpu_buffer_rsrc_t rs, int64_t ld, int64_t R, int64_t K,
                                int64_t r0, int64_t k0, int t) {
    const int64_t r = KR ? r0 + (t % (T / E)) * E : r0 + t / (KS / E);
    const int64_t k = KR ? k0 + t / (T / E) : k0 + (t % (KS / E)) * E;
#pragma unroll
    for (int q = 0; q < E / 4; q++) {
      const bool ok = KR ? (k < K && r + 4 * q < R) : (r < R && k + 4 * q < K);
      const int64_t off = KR ? k * ld + r + 4 * q : r * ld + k + 4 * q;
      const unsigned bo = ok ? (unsigned)(off * 4) : 0x80000000u;
      const float4 x = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(rs, bo, 0, 0));
      v[4 * q] = x.x; v[4 * q + 1] = x.y; v[4 * q + 2] = x.z; v[4 * q + 3] = x.w;
    }
  }

  // In LDS a row holds its even k first, then its odd k (element k at
  // (k % 2) * KS / 2 + k / 2): MFMA step s then pairs k = 2 s (lane half 0)
  // with 2 s + 1 (half 1), so every output adds the pairs (0, 1), (2, 3), ...
  // in k order whatever the stage size and tile, and any tile plan (and any
  // column slice of a weight) gives bitwise the same results.
  __device__ inline void store(float *__restrict__ xs, int t) const {
    if (!KR) {
      // E consecutive k from a multiple of E: evens and odds are each E / 2
      // consecutive slots.
      const int k = (t % (KS / E)) * E;
      float *d0 = xs + (t / (KS / E)) * LDX + k / 2;
      float *d1 = d0 + KS / 2;
      if constexpr (E % 8 == 0) {
#pragma unroll
        for (int q = 0; q < E / 8; q++) {
          *reinterpret_cast<float4 *>(d0 + 4 * q) =
              make_float4(v[8 * q], v[8 * q + 2], v[8 * q + 4], v[8 * q + 6]);
          *reinterpret_cast<float4 *>(d1 + 4 * q) =
              make_float4(v[8 * q + 1], v[8 * q + 3], v[8 * q + 5], v[8 * q + 7]);
        }
      } else {
#pragma unroll
        for (int e = 0; e < E; e += 2) d0[e / 2] = v[e], d1[e / 2] = v[e + 1];
      }
    } else {
      const int k = t / (T / E);
      float *d = xs + (t % (T / E)) * E * LDX + (k & 1) * (KS / 2) + (k >> 1);
#pragma unroll
      for (int e = 0; e < E; e++) d[e * LDX] = v[e];
    }
  }
};

// WT = 2: 128 x 128 workgroup tile, each wave 64 x 64 (2 x 2 MFMA tiles);
// WT = 1: 64 x 64, each wave one 32 x 32 tile (for grids too small to fill
// the chip with the larger tile).  KS = k per LDS stage; a stage is
// KS / 2 MFMA steps per tile.  AKR / BKR: operand layouts (A transposed, B
// not transposed).
template <int WT, int KS, bool AKR, bool BKR, bool BV>
__global__ __launch_bounds__(256) void k_f32_gemm(
    const float *__restrict__ A, const float *__restrict__ B,
    float *__restrict__ Y, int64_t M, int64_t N, int64_t K, int64_t lda,
    int64_t ldb, int vec_a, int vec_b,
    const mg_f32_bcast bc, uint32_t z0, int nx, int pr, int pc, float alpha, float beta,
    const float *__restrict__ C, int64_t c_rs, int64_t c_cs, int64_t ldy, int sps) {
  constexpr int T = 64 * WT, LDX = KS + 4, NS = KS / 2;
  __shared__ float As[2][T * LDX];
  __shared__ float Bs[2][T * LDX];
  const int t = threadIdx.x;
  const int lane = t & 63, wave = t >> 6;
  const int wm = wave & 1, wn = wave >> 1;
  const int l32 = lane & 31, h = lane >> 5;
  // Tile of this workgroup (see the tile order above).  pr = 0: row-major.
  int tr, tc;
  {
    const int L = (int)blockIdx.x;
    if (pr == 0) {
      tr = L / nx;
      tc = L % nx;
    } else {
      const int ny = (int)((M + T - 1) / T);
      const int x = L & 7, i = L >> 3, br = x / pc, bcol = x % pc;
      const int rlo = br * ny / pr, rhi = (br + 1) * ny / pr;
      const int clo = bcol * nx / pc, chi = (bcol + 1) * nx / pc;
      const int w = chi - clo;
      if (i >= (rhi - rlo) * w) return;  // uniform: the whole workgroup leaves
      tr = rlo + i / w;
      tc = clo + i % w;
    }
  }
  const uint32_t bz = z0 + blockIdx.z;
  int64_t a_off, b_off;
  mg_f32_batch_offsets(bc, bz, &a_off, &b_off);
  const float *Ab = A + a_off;
  const float *Bb = B + b_off;
  const int64_t r0 = (int64_t)tr * T, c0 = (int64_t)tc * T;
  const bool a_in = vec_a && r0 + T <= M, b_in = vec_b && c0 + T <= N;

  float16v acc[WT][WT];
#pragma unroll
  for (int i = 0; i < WT; i++)
#pragma unroll
    for (int j = 0; j < WT; j++) acc[i][j] = (float16v){};

  const int nst = (int)((K + KS - 1) / KS);
  // K split (sps > 0): stages [s0, s1) of split blockIdx.y, whose raw sums
  // go to its own M x ldy block of Y (the partials).
  const int s0 = sps > 0 ? (int)blockIdx.y * sps : 0;
  const int s1 = sps > 0 ? min(nst, s0 + sps) : nst;
  Stage<WT, KS, AKR> sa;
  Stage<WT, KS, BKR> sb;
  // BV: every stage through the branch-free buffer loads.
  auto rsrc = [](const float *base) __attribute__((always_inline)) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(base), (short)0, 0x7ffffff0,
                                             0x00020000);
  };
  const __amdgpu_buffer_rsrc_t ra = rsrc(Ab), rb = rsrc(Bb);
  auto load = [&](int st) {
    const int64_t k0 = (int64_t)st * KS;
    if constexpr (BV) {
      sa.load_b(ra, lda, M, K, r0, k0, t);
      sb.load_b(rb, ldb, N, K, c0, k0, t);
    } else {
      const bool kin = k0 + KS <= K;
      sa.load(Ab, a_in && kin, lda, M, K, r0, k0, t);
      sb.load(Bb, b_in && kin, ldb, N, K, c0, k0, t);
    }
  };
  load(s0);
  sa.store(As[0], t);
  sb.store(Bs[0], t);
  __syncthreads();
  for (int st = s0; st < s1; st++) {
    const int buf = (st - s0) & 1;
    const bool more = st + 1 < s1;
    if (more) load(st + 1);
    float a[WT][NS], b[WT][NS];
#pragma unroll
    for (int i = 0; i < WT; i++) {
      const float *p = &As[buf][(wm * 32 * WT + i * 32 + l32) * LDX + NS * h];
#pragma unroll
      for (int q = 0; q < NS / 4; q++) {
        const float4 x = *reinterpret_cast<const float4 *>(p + 4 * q);
        a[i][4 * q] = x.x; a[i][4 * q + 1] = x.y; a[i][4 * q + 2] = x.z; a[i][4 * q + 3] = x.w;
      }
    }
#pragma unroll
    for (int j = 0; j < WT; j++) {
      const float *p = &Bs[buf][(wn * 32 * WT + j * 32 + l32) * LDX + NS * h];
#pragma unroll
      for (int q = 0; q < NS / 4; q++) {
        const float4 x = *reinterpret_cast<const float4 *>(p + 4 * q);
        b[j][4 * q] = x.x; b[j][4 * q + 1] = x.y; b[j][4 * q + 2] = x.z; b[j][4 * q + 3] = x.w;
      }
    }
#pragma unroll
    for (int s = 0; s < NS; s++)
#pragma unroll
      for (int i = 0; i < WT; i++)
#pragma unroll
        for (int j = 0; j < WT; j++)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i][s], b[j][s], acc[i][j], 0, 0, 0);
    if (more) {
      sa.store(As[buf ^ 1], t);
      sb.store(Bs[buf ^ 1], t);
    }
    __syncthreads();
  }

  // Lane l holds column l % 32 and rows 8 (v / 4) + 4 (l / 32) + v % 4 of
  // each 32 x 32 tile; 32 lanes write 128 contiguous bytes per store.  The
  // tile's C values are all loaded before the first store (one memory round
  // trip, not one per row).  BV: the stores are raw buffer stores, an output
  // past M or N getting an offset past the resource (dropped in hardware):
  // no branches, so the stores issue back to back (behind per-element
  // branches the compiler waited for each store before the next).
  float *Yb = Y + ((int64_t)bz + blockIdx.y) * M * ldy;  // blockIdx.y > 0 only for K splits
  const __amdgpu_buffer_rsrc_t ry = rsrc(Yb);
#pragma unroll
  for (int i = 0; i < WT; i++)
#pragma unroll
    for (int j = 0; j < WT; j++) {
      const int64_t col = c0 + wn * 32 * WT + j * 32 + l32;
      if (!BV && col >= N) continue;
      const int64_t rw = r0 + wm * 32 * WT + i * 32 + 4 * h;
      float cv[16];
      if (C) {
#pragma unroll
        for (int v = 0; v < 16; v++) {
          const int64_t row = rw + 8 * (v >> 2) + (v & 3);
          const bool ok = row < M && col < N;
          cv[v] = C[ok ? row * c_rs + col * c_cs : 0];
        }
      }
#pragma unroll
      for (int v = 0; v < 16; v++) {
        const int64_t row = rw + 8 * (v >> 2) + (v & 3);
        if (!BV && row >= M) continue;
        float y = acc[i][j][v];
        if (alpha != 1.f) y = alpha * y;
        if (C) {
          float c = cv[v];
          if (beta != 1.f) c = beta * c;
          y = y + c;
        }
        if constexpr (BV) {
          const bool ok = row < M && col < N;
          __builtin_amdgcn_raw_buffer_store_b32(
              __builtin_bit_cast(unsigned, y), ry,
              ok ? (unsigned)(row * ldy + col) * 4u : 0x80000000u, 0, 0);
        } else {
          Yb[row * ldy + col] = y;
        }
      }
    }
}

#ifndef MG_F32_BUFFER_LOADS
#define MG_F32_BUFFER_LOADS 1
#endif
template <int WT, int KS, bool BV>
void launch_f32_bv(const mg_f32_problem &p, dim3 grid, hipStream_t st, const float *a,
                   const float *b, float *y, int vec_a, int vec_b, uint32_t z0, int nx, int pr,
                   int pc, int sps) {
#define MG_F32_ARGS                                                                         \
  a, b, y, p.M, p.N, p.K, p.lda, p.ldb, vec_a, vec_b, p.bc, z0, nx, pr, pc, p.alpha, p.beta, \
      p.c, p.c_rs, p.c_cs, p.ldy ? p.ldy : p.N, sps
  const bool akr = p.trans_a != 0, bkr = p.trans_b == 0;
  if (!akr && !bkr)
    hipLaunchKernelGGL((k_f32_gemm<WT, KS, false, false, BV>), grid, dim3(256), 0, st,
                       MG_F32_ARGS);
  else if (!akr && bkr)
    hipLaunchKernelGGL((k_f32_gemm<WT, KS, false, true, BV>), grid, dim3(256), 0, st,
                       MG_F32_ARGS);
  else if (akr && !bkr)
    hipLaunchKernelGGL((k_f32_gemm<WT, KS, true, false, BV>), grid, dim3(256), 0, st,
                       MG_F32_ARGS);
  else
    hipLaunchKernelGGL((k_f32_gemm<WT, KS, true, true, BV>), grid, dim3(256), 0, st,
                       MG_F32_ARGS);
#undef MG_F32_ARGS
}

// The branch-free loads need aligned rows, quads that never straddle the
// contiguous extent, and every in-range byte offset of both operands and of
// the output (within one batch) below 2^31.
template <int WT, int KS>
void launch_f32(const mg_f32_problem &p, dim3 grid, hipStream_t st, const float *a,
                const float *b, float *y, int vec_a, int vec_b, uint32_t z0, int nx, int pr,
                int pc, int kspl = 1) {
  // Stages per split: a split covers a multiple of 32 k whatever the stage
  // size, so every tile plan splits K at the same k (bitwise equal sums).
  const int sps = kspl > 1 ? (int)(((p.K + kspl - 1) / kspl + 31) / 32 * (32 / KS)) : 0;
  const bool akr = p.trans_a != 0, bkr = p.trans_b == 0;
  const int64_t lim = ((int64_t)1 << 31) - 16;
  const bool bv =
      MG_F32_BUFFER_LOADS && vec_a && vec_b && (akr ? p.M % 4 == 0 : p.K % 4 == 0) &&
      (bkr ? p.N % 4 == 0 : p.K % 4 == 0) &&
      (akr ? p.K * p.lda : p.M * p.lda) * 4 < lim && (bkr ? p.K * p.ldb : p.N * p.ldb) * 4 < lim &&
      p.M * (p.ldy ? p.ldy : p.N) * 4 < lim;
  if (bv)
    launch_f32_bv<WT, KS, true>(p, grid, st, a, b, y, vec_a, vec_b, z0, nx, pr, pc, sps);
  else
    launch_f32_bv<WT, KS, false>(p, grid, st, a, b, y, vec_a, vec_b, z0, nx, pr, pc, sps);
}

// Sum of the kspl partials of one batch in split order, then the epilogue of
// k_f32_gemm (alpha, then beta C): one thread per output element.
__global__ __launch_bounds__(256) void k_f32_ksum(const float *__restrict__ part, int kspl,
                                                  int64_t M, int64_t N, float alpha, float beta,
                                                  const float *__restrict__ C, int64_t c_rs,
                                                  int64_t c_cs, float *__restrict__ Y,
                                                  int64_t ldy) {
  const int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (e >= M * N) return;
  const int64_t row = e / N, col = e - row * N;
  float y = part[e];
  for (int s = 1; s < kspl; s++) y += part[s * M * N + e];
  if (alpha != 1.f) y = alpha * y;
  if (C) {
    float c = C[row * c_rs + col * c_cs];
    if (beta != 1.f) c = beta * c;
    y = y + c;
  }
  Y[row * ldy + col] = y;
}

}  // namespace

int mg_f32_ksplit(int64_t M, int64_t K, int64_t batch) {
#ifndef MG_F32_KSPLIT
#define MG_F32_KSPLIT 2
#endif
#ifndef MG_F32_KSPLIT_MIN_K
#define MG_F32_KSPLIT_MIN_K 1024
#endif
  return batch == 1 && K >= MG_F32_KSPLIT_MIN_K && M <= 8192 ? MG_F32_KSPLIT : 1;
}

// The XCD cut of an ny x nx tile grid: pr row bands x pc column bands with
// pr * pc = 8, at least one tile per band, minimising the tiles fetched
// (ny * pc row tiles of A + nx * pr column tiles of B, equal sizes), then the
// largest rectangle.  Returns false (row-major order) for grids of fewer than
// 64 tiles or that no cut fits.
static bool mg_f32_xcd_cut(int64_t ny, int64_t nx, int *pr, int *pc, int64_t *per) {
  if (ny * nx < 64) return false;
  int64_t best = -1, best_per = 0;
  for (int r = 1; r <= 8; r *= 2) {
    const int c = 8 / r;
    if (r > ny || c > nx) continue;
    const int64_t cost = ny * c + nx * r;
    const int64_t rect = ((ny + r - 1) / r) * ((nx + c - 1) / c);
    if (best < 0 || cost < best || (cost == best && rect < best_per)) {
      best = cost;
      best_per = rect;
      *pr = r;
      *pc = c;
    }
  }
  if (best < 0) return false;
  *per = best_per;
  return true;
}

mg_status mg_f32_run(mg_ctx *ctx, const mg_f32_problem &p, const float *a_dev,
                     const float *b_dev, float *y_dev) {
  if (p.M == 0 || p.N == 0 || p.batch == 0) return MG_OK;
  // 16-byte operand loads need 16-byte aligned rows: the base pointers and,
  // for batches, every batch offset (the broadcast strides are multiples of
  // M*K resp. K*N elements, so checking the leading dimension and one batch
  // stride suffices).
  auto aligned = [](const float *ptr, int64_t ld, int64_t batch_stride) {
    return reinterpret_cast<uintptr_t>(ptr) % 16 == 0 && ld % 4 == 0 && batch_stride % 4 == 0;
  };
  const int vec_a = aligned(a_dev, p.lda, p.M * p.K) ? 1 : 0;
  const int vec_b = aligned(b_dev, p.ldb, p.K * p.N) ? 1 : 0;
  // The 128 x 128 tile when it still gives about two workgroups per CU,
  // else 64 x 64.
  const int64_t big = ((p.N + 127) / 128) * ((p.M + 127) / 128) * p.batch;
  const bool use_big = big >= 2 * (int64_t)ctx->num_cus;
  const int T = use_big ? 128 : 64;
  const int64_t nx = (p.N + T - 1) / T, ny = (p.M + T - 1) / T;
  int pr = 0, pc = 0;
  int64_t per = 0;
  const bool cut = mg_f32_xcd_cut(ny, nx, &pr, &pc, &per);
  if (!cut) pr = pc = 0;
  const unsigned gx = (unsigned)(cut ? 8 * per : nx * ny);
#ifndef MG_F32_KS_BIG
#define MG_F32_KS_BIG 16
#endif
#ifndef MG_F32_KS_SMALL
#define MG_F32_KS_SMALL 32
#endif
  // 64 x 64 tiles beyond four workgroups per CU take stages of 16 k: their
  // LDS (20 KB a workgroup against 36 KB) then holds every workgroup of the
  // grid at once instead of one and a half rounds (MiniLM FFN1 4096 x 384 x
  // 1536: 64.4 -> 59.6 us; with fewer tiles 32-k stages are faster).
  const bool small_ks16 = !use_big && nx * ny * p.batch > 4 * (int64_t)ctx->num_cus;
  if (p.kspl > 1 && p.part && p.batch == 1 && p.part_cols > 0 && p.N > p.part_cols) {
    // The partial buffer holds part_cols columns: column chunks, each the
    // same per-output arithmetic as the whole.
    const int64_t ldy = p.ldy ? p.ldy : p.N;
    for (int64_t n0 = 0; n0 < p.N; n0 += p.part_cols) {
      mg_f32_problem q = p;
      q.N = std::min(p.part_cols, p.N - n0);
      q.ldy = ldy;
      if (p.c) q.c = p.c + n0 * p.c_cs;
      const float *bq = p.trans_b ? b_dev + n0 * p.ldb : b_dev + n0;
      MG_TRY(mg_f32_run(ctx, q, a_dev, bq, y_dev + n0));
    }
    return MG_OK;
  }
  if (p.kspl > 1 && p.part && p.batch == 1) {
    // Raw sums of each K split into part, then k_f32_ksum.
    mg_f32_problem q = p;
    q.alpha = 1.f;
    q.c = nullptr;
    q.ldy = p.N;
    const dim3 grid(gx, (unsigned)p.kspl, 1);
    if (use_big)
      launch_f32<2, MG_F32_KS_BIG>(q, grid, ctx->stream, a_dev, b_dev, p.part, vec_a, vec_b, 0,
                                   (int)nx, pr, pc, p.kspl);
    else if (small_ks16)
      launch_f32<1, 16>(q, grid, ctx->stream, a_dev, b_dev, p.part, vec_a, vec_b, 0, (int)nx,
                        pr, pc, p.kspl);
    else
      launch_f32<1, MG_F32_KS_SMALL>(q, grid, ctx->stream, a_dev, b_dev, p.part, vec_a, vec_b, 0,
                                     (int)nx, pr, pc, p.kspl);
    MG_TRY(mg_launch_check("k_f32_gemm"));
    const int64_t tot = p.M * p.N;
    hipLaunchKernelGGL(k_f32_ksum, dim3((unsigned)((tot + 255) / 256)), dim3(256), 0,
                       ctx->stream, p.part, p.kspl, p.M, p.N, p.alpha, p.beta, p.c, p.c_rs,
                       p.c_cs, y_dev, p.ldy ? p.ldy : p.N);
    return mg_launch_check("k_f32_ksum");
  }
  // Batches in chunks of at most 65535 per launch (grid z).
  for (int64_t z0 = 0; z0 < p.batch; z0 += 65535) {
    const dim3 grid(gx, 1, (unsigned)std::min<int64_t>(65535, p.batch - z0));
    if (use_big)
      launch_f32<2, MG_F32_KS_BIG>(p, grid, ctx->stream, a_dev, b_dev, y_dev, vec_a, vec_b,
                                   (uint32_t)z0, (int)nx, pr, pc);
    else if (small_ks16)
      launch_f32<1, 16>(p, grid, ctx->stream, a_dev, b_dev, y_dev, vec_a, vec_b, (uint32_t)z0,
                        (int)nx, pr, pc);
    else
      launch_f32<1, MG_F32_KS_SMALL>(p, grid, ctx->stream, a_dev, b_dev, y_dev, vec_a, vec_b,
                                     (uint32_t)z0, (int)nx, pr, pc);
    MG_TRY(mg_launch_check("k_f32_gemm"));
  }
  return MG_OK;
}

// ------------------------------------------- MatMul on non-float operands
//
// opMatMul's fallback for operands that are not both Float32List
// (lib/src/onnx_ops.dart:1753-1762): each output is a double sum over k in
// order of a.getD * b.getD, rounded once to f32.  The operands arrive as
// doubles (getD's value: an int64 element converted to the nearest double,
// a float element exactly).  The products and sums are rounded separately
// (contraction into fused multiply-adds is switched off in the kernel: a
// product of two doubles is not exact, so a fused form would differ), so
// every output equals the reference's bit for bit.  One thread per output;
// batches decoded as the fp32 kernel decodes them.

namespace {

__global__ __launch_bounds__(256) void k_matmul_f64acc(const double *__restrict__ a,
                                                       const double *__restrict__ b,
                                                       float *__restrict__ y, int64_t M,
                                                       int64_t K, int64_t N,
                                                       const mg_f32_bcast bc, uint32_t z0) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= M * N) return;
  const uint32_t z = z0 + blockIdx.y;
  int64_t ao = 0, bo = 0;
  mg_f32_batch_offsets(bc, z, &ao, &bo);
  const int64_t r = i / N, c = i % N;
  const double *ar = a + ao + r * K;
  const double *bc_ = b + bo + c;
  double s = 0;
  {
#pragma clang fp contract(off)
    for (int64_t k = 0; k < K; k++) {
      const double p = ar[k] * bc_[k * N];
      s = s + p;
    }
  }
  y[(int64_t)z * M * N + i] = (float)s;
}

}  // namespace

mg_status mg_f64acc_run(mg_ctx *ctx, const mg_f32_problem &p, const double *a_dev,
                        const double *b_dev, float *y_dev) {
  if (p.M * p.N == 0 || p.batch == 0) return MG_OK;
  const unsigned gx = (unsigned)((p.M * p.N + 255) / 256);
  for (int64_t z0 = 0; z0 < p.batch; z0 += 65535) {  // grid y holds at most 65535
    const unsigned gy = (unsigned)std::min<int64_t>(65535, p.batch - z0);
    hipLaunchKernelGGL(k_matmul_f64acc, dim3(gx, gy), dim3(256), 0, ctx->stream, a_dev, b_dev,
                       y_dev, p.M, p.K, p.N, p.bc, (uint32_t)z0);
    MG_TRY(mg_launch_check("k_matmul_f64acc"));
  }
  return MG_OK;
}
