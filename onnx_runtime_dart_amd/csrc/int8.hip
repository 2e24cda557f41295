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
// v_mfma_i32_32x32x32_i8 operands: lane l holds row (A) or column (B) l % 32
// and 16 bytes along k; the 32x32 int32 result has lane l at column l % 32
// and rows 8 (v / 4) + 4 (l / 32) + v % 4, v < 16.  The sum over k does not
// care which 32 k a step covers as long as A and B agree, so within each
// 128-k stage step q gives lane l the k = 64 (l / 32) + 16 q + 0..15: a lane
// reads 64 contiguous bytes of its A row per stage (whole cache lines per
// workgroup) instead of four scattered 16-byte pieces.
//   B is prepacked once per weight in that order: bfrag[n32][4 stage + q]
//     [lane] (uint4), re-centred, zero outside [K, N]; N padded to 128 and
//     K to 256 (one LDS stage).
//   A is read in place from row-major [rows, K] when K % 256 == 0 and the
//     base is 16-byte aligned, else first copied into a padded [rows, kpad]
//     buffer whose pad bytes re-centre to zero.
// Workgroup tile: 128*WM rows x 128 columns, 4 waves, wave w owning rows
// [32*WM*w, +32*WM).  B moves global -> LDS directly (global_load_lds) in
// stages of 256 k, double buffered, one barrier per stage; its fragments are
// read from LDS a step ahead.  A goes straight to registers, each register
// reloaded four steps ahead right after its step; rowsum(A') is accumulated
// alongside with v_dot4_i32_i8.  The epilogue restages each 32-row tile in
// LDS and writes whole 16-byte row pieces.
#include <hip/hip_runtime.h>

#include <cmath>

#include "mg_internal.h"

namespace {

typedef int int4v __attribute__((ext_vector_type(4)));
typedef int int16v __attribute__((ext_vector_type(16)));

constexpr int TN = 128;  // workgroup tile columns
constexpr int QS = 8;    // 32-k MFMA steps per LDS stage (256 k)
constexpr int RA = 4;    // A register ring: steps loaded ahead of use
#ifndef KW_RA
#define KW_RA 4  // k_i8_gemm_kw: steps of loads in flight per wave
#endif

// B (u8 or i8, [K, N] per batch) -> fragments bfrag[batch][n32][q][lane]
// (lane l of fragment q holds column 32 n32 + l % 32, k = 128 (q / 4) +
// 64 (l / 32) + 16 (q % 4) .. +15, re-centred to signed).  Workgroup = one
// 32-column tile and one 128-k group (its four fragments q): the 128 x 32
// byte block is read row by row with 16-byte loads where the row piece is
// whole and aligned, staged in LDS, and each thread gathers its fragment's 16
// bytes of one column from there.  Bytes outside [K, N] are stored as the
// re-centring constant, so they come out as 0.  Grid: n32n * kqp / 4 per batch
// (kqp is a multiple of 8).
__global__ __launch_bounds__(256) void k_i8_prep_b(
    const uint8_t *__restrict__ b, int b_signed, int64_t K, int64_t N,
    int n32n, int kqp, int4v *__restrict__ frag) {
  __shared__ uint32_t tile[128][9];  // [k][32 columns as 8 words], one word of padding
  const int t = threadIdx.x;
  const int64_t bi = blockIdx.y;
  const int qgs = kqp / 4;
  const int n32 = (int)blockIdx.x / qgs, qg = (int)blockIdx.x % qgs;
  const uint32_t flip = b_signed ? 0u : 0x80u;
  {
    const int r = t >> 1, hh = t & 1;  // row of the block, 16-column half
    const int64_t k = (int64_t)qg * 128 + r;
    const int64_t c0 = (int64_t)n32 * 32 + 16 * hh;
    const uint8_t *src = b + (bi * K + (k < K ? k : 0)) * N + c0;
    uint32_t w[4];
    if (k < K && c0 + 16 <= N && (reinterpret_cast<uintptr_t>(src) & 15) == 0) {
      const uint4 x = *reinterpret_cast<const uint4 *>(src);
      w[0] = x.x, w[1] = x.y, w[2] = x.z, w[3] = x.w;
    } else {
#pragma unroll
      for (int q = 0; q < 4; q++) {
        uint32_t word = 0;
#pragma unroll
        for (int e = 0; e < 4; e++) {
          const int64_t c = c0 + 4 * q + e;
          const uint32_t by = (k < K && c < N) ? src[4 * q + e] : flip;
          word |= by << (8 * e);
        }
        w[q] = word;
      }
    }
#pragma unroll
    for (int q = 0; q < 4; q++) tile[r][4 * hh + q] = w[q];
  }
  __syncthreads();
  const int lane = t & 63, qq = t >> 6;
  const int col = lane & 31, kl = 64 * (lane >> 5) + 16 * qq;
  const uint32_t fl4 = flip * 0x01010101u;
  uint32_t o[4];
#pragma unroll
  for (int q = 0; q < 4; q++) {
    uint32_t word = 0;
#pragma unroll
    for (int e = 0; e < 4; e++) {
      const uint32_t by = (tile[kl + 4 * q + e][col >> 2] >> (8 * (col & 3))) & 0xFFu;
      word |= by << (8 * e);
    }
    o[q] = word ^ fl4;
  }
  const int64_t per_batch = (int64_t)n32n * kqp * 64;
  const int64_t idx = ((int64_t)n32 * kqp + qg * 4 + qq) * 64 + lane;
  frag[bi * per_batch + idx] = (int4v){(int)o[0], (int)o[1], (int)o[2], (int)o[3]};
}

// Column sums of B' and cb per column.  Workgroup = 64 columns of one batch
// (lane = column); its four waves take every fourth row k, each lane with 16
// row loads in flight, and the four partial sums meet in LDS (integer sums:
// exact in any order).
__global__ __launch_bounds__(256) void k_i8_colsum(
    const uint8_t *__restrict__ b, int b_signed, int64_t K, int64_t N,
    int64_t npad, int zb_scalar, const int32_t *__restrict__ zb, int zb_len,
    int32_t *__restrict__ colsum, int32_t *__restrict__ cb) {
  __shared__ int part[4][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t col = (int64_t)blockIdx.x * 64 + lane;
  const int64_t bi = blockIdx.y;
  const int flip = b_signed ? 0 : 0x80;
  const bool live = col < N;
  const uint8_t *bc = b + bi * K * N + (live ? col : 0);
  constexpr int U = 16;
  int s = 0;
  int64_t k = wave;
  for (; k + 4 * (U - 1) < K; k += 4 * U) {
    int x[U];
#pragma unroll
    for (int u = 0; u < U; u++) x[u] = bc[(k + 4 * u) * N];
#pragma unroll
    for (int u = 0; u < U; u++) s += (int8_t)(x[u] ^ flip);
  }
  for (; k < K; k += 4) s += (int8_t)(bc[k * N] ^ flip);
  part[wave][lane] = live ? s : 0;
  __syncthreads();
  if (wave != 0 || col >= npad) return;
  colsum[bi * npad + col] = part[0][lane] + part[1][lane] + part[2][lane] + part[3][lane];
  int z = zb_scalar;
  if (zb && zb_len > 0 && live) z = zb[col % zb_len];
  cb[bi * npad + col] = (b_signed ? 0 : 128) - z;
}

// B given transposed, bt [N, K] row-major (a convolution filter [M][C taps])
// -> the fragments of k_i8_prep_b: lane l of fragment q of column tile n32
// reads the 16 bytes of row 32 n32 + l % 32 at k = 128 (q / 4) + 64 (l / 32)
// + 16 (q % 4), one 16-byte load where the piece is whole and aligned.  One
// thread per fragment lane.
__global__ __launch_bounds__(256) void k_i8_prep_bt(const uint8_t *__restrict__ bt, int b_signed,
                                                    int64_t K, int64_t N, int n32n, int kqp,
                                                    int4v *__restrict__ frag) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (int64_t)n32n * kqp * 64) return;
  const int lane = (int)(idx & 63);
  const int64_t fq = idx >> 6;
  const int q = (int)(fq % kqp), n32 = (int)(fq / kqp);
  const int64_t n = (int64_t)n32 * 32 + (lane & 31);
  const int64_t k0 = (int64_t)(q / 4) * 128 + 64 * (lane >> 5) + 16 * (q % 4);
  const uint32_t flip = b_signed ? 0u : 0x80u;
  uint32_t w[4];
  const uint8_t *src = bt + (n < N ? n : 0) * K + k0;
  if (n < N && k0 + 16 <= K && (reinterpret_cast<uintptr_t>(src) & 15) == 0) {
    const uint4 x = *reinterpret_cast<const uint4 *>(src);
    w[0] = x.x, w[1] = x.y, w[2] = x.z, w[3] = x.w;
  } else {
#pragma unroll
    for (int j = 0; j < 4; j++) {
      uint32_t word = 0;
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const int64_t k = k0 + 4 * j + e;
        const uint32_t by = (n < N && k < K) ? src[4 * j + e] : flip;
        word |= by << (8 * e);
      }
      w[j] = word;
    }
  }
  const uint32_t fl4 = flip * 0x01010101u;
  frag[idx] = (int4v){(int)(w[0] ^ fl4), (int)(w[1] ^ fl4), (int)(w[2] ^ fl4), (int)(w[3] ^ fl4)};
}

// Column sums of B' from bt [N, K] (rows contiguous): one wave per column,
// 16-byte loads where the row allows, and cb per column as k_i8_colsum.
__global__ __launch_bounds__(256) void k_i8_colsum_t(
    const uint8_t *__restrict__ bt, int b_signed, int64_t K, int64_t N, int64_t npad,
    int zb_scalar, const int32_t *__restrict__ zb, int zb_len, int32_t *__restrict__ colsum,
    int32_t *__restrict__ cb) {
  const int lane = threadIdx.x & 63;
  const int64_t col = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (col >= npad) return;
  const bool live = col < N;
  int s = 0;
  if (live) {
    const uint8_t *row = bt + col * K;
    const bool vec = K % 16 == 0 && (reinterpret_cast<uintptr_t>(row) & 15) == 0;
    const int flip = b_signed ? 0 : 0x80;
    if (vec) {
      for (int64_t k = 16 * lane; k < K; k += 1024) {
        const uint4 x = *reinterpret_cast<const uint4 *>(row + k);
        const uint32_t wv[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
        for (int j = 0; j < 4; j++)
#pragma unroll
          for (int e = 0; e < 4; e++) s += (int8_t)(((wv[j] >> (8 * e)) & 0xFFu) ^ flip);
      }
    } else {
      for (int64_t k = lane; k < K; k += 64) s += (int8_t)(row[k] ^ flip);
    }
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) s += __shfl_xor(s, off);
  if (lane != 0) return;
  colsum[col] = s;
  int z = zb_scalar;
  if (zb && zb_len > 0 && live) z = zb[col % zb_len];
  cb[col] = (b_signed ? 0 : 128) - z;
}

// 16 bytes per lane global -> LDS (gfx950 global_load_lds_dwordx4): lane i's
// data lands at LDS byte address lds + 16 i (lds wave-uniform).  Issued as
// asm so that the compiler's own waits do not treat it as a write to every
// LDS location (it would otherwise wait for it before any LDS read); callers
// wait for it themselves (vmcnt) before the barrier that publishes the data.
__device__ inline void lds_copy16(const void *g, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %0\n\tglobal_load_lds_dwordx4 %1, off"
               :
               : "s"(lds), "v"(g)
               : "memory", "m0");
}

// A (u8 or i8, [M, K] per batch, row pitch lda) -> fragments
// afrag[batch][m32][q][lane] (the order the GEMM loads them: 1 KB per wave
// load), re-centred to signed, zero outside [M, K]; plus rowsum(A') and
// ca = oa - aZp per row.  One workgroup per (32-row tile, batch); its 16
// waves take every 16th k step, so that few row tiles still keep many
// loads in flight.
constexpr int PREP_A_WAVES = 16;
__global__ __launch_bounds__(64 * PREP_A_WAVES) void k_i8_prep_a(
    const uint8_t *__restrict__ a, int64_t lda, int64_t a_bs, int a_signed, int vec,
    int64_t M, int64_t K, int kqp, int m32n, int za_scalar, const int32_t *__restrict__ za,
    int za_len, int4v *__restrict__ afrag, int32_t *__restrict__ rowsum,
    int32_t *__restrict__ ca) {
  const int m32 = blockIdx.x;
  const int64_t bz = blockIdx.y;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int r = lane & 31, h = lane >> 5;
  const int64_t row = (int64_t)m32 * 32 + r;
  const uint8_t *ar = a + bz * a_bs + row * lda;
  const uint32_t flip = a_signed ? 0u : 0x80808080u;
  int4v *out = afrag + ((bz * m32n + m32) * (int64_t)kqp) * 64 + lane;
  int s = 0;
  for (int q = wave; q < kqp; q += PREP_A_WAVES) {
    const int64_t k0 = (int64_t)(q >> 2) * 128 + 64 * h + 16 * (q & 3);
    int4v v;
    if (row < M && vec && k0 + 16 <= K) {
      v = *reinterpret_cast<const int4v *>(ar + k0);
      v.x ^= flip; v.y ^= flip; v.z ^= flip; v.w ^= flip;
    } else {
      union { int4v v; uint8_t x[16]; } u;
#pragma unroll
      for (int e = 0; e < 16; e++)
        u.x[e] = (row < M && k0 + e < K) ? (uint8_t)(ar[k0 + e] ^ (flip & 0xff)) : (uint8_t)0;
      v = u.v;
    }
    s = __builtin_amdgcn_sdot4(v.x, 0x01010101, s, false);
    s = __builtin_amdgcn_sdot4(v.y, 0x01010101, s, false);
    s = __builtin_amdgcn_sdot4(v.z, 0x01010101, s, false);
    s = __builtin_amdgcn_sdot4(v.w, 0x01010101, s, false);
    out[(int64_t)q * 64] = v;
  }
  __shared__ int red[PREP_A_WAVES][64];
  red[wave][lane] = s;
  __syncthreads();
  if (t < 32) {
    int tot = 0;
#pragma unroll
    for (int w = 0; w < PREP_A_WAVES; w++) tot += red[w][t] + red[w][t + 32];
    const int64_t rr = (int64_t)m32 * 32 + t;
    const int64_t slot = bz * m32n * 32 + rr;
    rowsum[slot] = tot;
    const int z = (za && za_len > 0) ? za[rr % za_len] : za_scalar;
    ca[slot] = (a_signed ? 0 : 128) - z;
  }
}

struct I8Epi {
  const int32_t *colsum, *cb;  // [b batch?][npad]
  int64_t cs_bs;               // colsum/cb batch stride (0 = shared)
  const int32_t *rowsum, *ca;  // [a batch?][mpad]
  int64_t rs_bs;               // rowsum/ca batch stride (0 = shared)
  int K;
  int y_vec;  // output base 16-byte aligned (always for the partials)
  float mult;
  int y_zp, lo, hi;
  // Device-resident A scale (DynamicQuantizeLinear output): when set, the
  // multiplier is formed on the device from it, b_scale and y_scale.
  const float *a_scale_dev;
  float b_scale, y_scale;
};

// Requant multiplier fl32(fl32(aS * bS) / yS) with each step rounded to f32
// from a double product / quotient (lib/src/onnx_qlinear_ops.dart:95-98).
__device__ inline float i8_mult(const I8Epi &e) {
  if (!e.a_scale_dev) return e.mult;
  const float ab = (float)((double)e.a_scale_dev[0] * (double)e.b_scale);
  return (float)((double)ab / (double)e.y_scale);
}

// Final value of one output element and its store.
template <int REQ>
__device__ inline void i8_finish(void *y, int64_t o, int32_t acc, int32_t rs, int32_t cav,
                                 int32_t cs, int32_t cbv, const I8Epi &e) {
  const uint32_t v = (uint32_t)acc + (uint32_t)cbv * (uint32_t)rs + (uint32_t)cav * (uint32_t)cs +
                     (uint32_t)e.K * (uint32_t)cav * (uint32_t)cbv;
  const int32_t vi = (int32_t)v;
  if (REQ) {
    const float p = (float)((double)vi * (double)i8_mult(e));
    // Rounded values beyond +-65536 saturate alike after + y_zp and the
    // clamp (the reference's int is 64-bit; an int32 conversion of a larger
    // value would saturate and the + y_zp could wrap).
    int qv = (int)__builtin_amdgcn_fmed3f(rintf(p), -65536.f, 65536.f) + e.y_zp;
    qv = qv < e.lo ? e.lo : (qv > e.hi ? e.hi : qv);
    static_cast<uint8_t *>(y)[o] = (uint8_t)qv;
  } else {
    static_cast<int32_t *>(y)[o] = vi;
  }
}

// MODE 0: int32 output, 1: requantised bytes, 2: raw partial sums (split K,
// k_i8_reduce finishes).
// Grid: x = tiles in XCD-aware order (workgroup L runs on XCD L % 8; all row
// tiles of a column tile share L % 8, so its B stays in one L2), y = k
// splits of sps stages each, z = batch.
template <int WM, int MODE>
__global__ __launch_bounds__(256, 2) void k_i8_gemm(
    const int4v *__restrict__ afrag, int64_t a_bs, const int4v *__restrict__ bfrag,
    int64_t b_bs, void *__restrict__ y, I8Epi e, int M, int N, int kqp, int mtiles,
    int ntiles, int sps) {
  // B double buffer [2][n32][q][lane] (64 KB); afterwards the int32
  // epilogue stages, [32 rows][128 + 4 pad] per wave.
  constexpr int SROW = TN + 4;
  __shared__ int4v smem[4 * 32 * SROW / 4];
  int4v *bl0 = smem, *bl1 = smem + 4 * QS * 64;
  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int L = blockIdx.x;
  const int xcd = L & 7, qq = L >> 3;
  const int mt = qq % mtiles;
  const int nt = (qq / mtiles) * 8 + xcd;
  if (nt >= ntiles) return;
  const int64_t bz = blockIdx.z;
  const int nstage = kqp / QS;
  const int s0 = blockIdx.y * sps, s1 = min(nstage, s0 + sps);
  const int lc = lane & 31, lh = lane >> 5;

  const int4v *ap[WM];
#pragma unroll
  for (int mi = 0; mi < WM; mi++)
    ap[mi] = afrag + bz * a_bs + ((int64_t)(mt * 4 * WM + wave * WM + mi) * kqp) * 64 + lane;
  // B stage s -> LDS: 32 fragment blocks of 1 KB, 8 per wave.
  const int4v *bbase = bfrag + bz * b_bs + ((int64_t)nt * 4 * kqp) * 64 + lane;
  auto stage_b = [&](int s, int4v *dst) {
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const int u = wave + 4 * i;  // block = (n32 = u / QS, q = u % QS)
      lds_copy16(bbase + ((int64_t)(u / QS) * kqp + s * QS + (u % QS)) * 64,
                 (uint32_t)reinterpret_cast<uintptr_t>(&dst[u * 64]));
    }
  };

  int16v acc[WM][4];
#pragma unroll
  for (int mi = 0; mi < WM; mi++)
#pragma unroll
    for (int n = 0; n < 4; n++) acc[mi][n] = (int16v){};

  // ar[j % RA]: A of step j, reloaded with step j + RA right after use
  // (clamped to the split's last step; unused there).
  const int jlast = s1 * QS - 1;
  int4v ar[RA][WM];
  stage_b(s0, bl0);
#pragma unroll
  for (int j = 0; j < RA; j++)
#pragma unroll
    for (int mi = 0; mi < WM; mi++) ar[j][mi] = ap[mi][(int64_t)(s0 * QS + j) * 64];
  asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");

  // One stage: MFMAs on `cur` while the next stage's B is copied into `nxt`.
  auto run_stage = [&](int s, const int4v *cur, int4v *nxt) {
    if (s + 1 < s1) stage_b(s + 1, nxt);
    __builtin_amdgcn_sched_barrier(0);
    int4v b[4];
#pragma unroll
    for (int n = 0; n < 4; n++) b[n] = cur[(n * QS) * 64 + lane];
#pragma unroll
    for (int q = 0; q < QS; q++) {
      int4v bnx[4];
      if (q + 1 < QS) {
#pragma unroll
        for (int n = 0; n < 4; n++) bnx[n] = cur[(n * QS + q + 1) * 64 + lane];
      }
#pragma unroll
      for (int mi = 0; mi < WM; mi++)
#pragma unroll
        for (int n = 0; n < 4; n++)
          acc[mi][n] = __builtin_amdgcn_mfma_i32_32x32x32_i8(b[n], ar[q % RA][mi], acc[mi][n], 0, 0, 0);
      const int jn = min(s * QS + q + RA, jlast);
#pragma unroll
      for (int mi = 0; mi < WM; mi++) ar[q % RA][mi] = ap[mi][(int64_t)jn * 64];
      if (q + 1 < QS) {
#pragma unroll
        for (int n = 0; n < 4; n++) b[n] = bnx[n];
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    // The next stage's B (issued before this stage's 8 * WM A loads) has
    // landed in LDS once at most 8 * WM loads remain; then all waves meet.
    asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(8 * WM) : "memory");
  };
  for (int s = s0; s < s1; s += 2) {
    run_stage(s, bl0, bl1);
    if (s + 1 < s1) run_stage(s + 1, bl1, bl0);
  }

  // Epilogue.  With B as the MFMA's first operand each accumulator tile is
  // Y^T: lane l holds row l % 32 of the tile and, for g = 0..3, the four
  // consecutive columns 8 g + 4 (l / 32) + 0..3 (acc[..][4 g + i]).  Per
  // element v = acc + cb*(rowsum + K*ca) + ca*colsum in int32 wrap-around
  // (MODE 2: acc alone).  Requantised bytes (MODE 1) are stored from there;
  // int32 values go through the wave's LDS stage (rows padded by 16 bytes
  // against bank conflicts) and leave as whole 16-byte row pieces.
  const int64_t yb = (int64_t)bz * M;  // first output row of this batch
  const float mult = MODE == 1 ? i8_mult(e) : 0.f;
  const bool vec_ok = (N % 4) == 0 && e.y_vec;
  int32_t *stage = reinterpret_cast<int32_t *>(smem) + wave * (32 * SROW);
#pragma unroll
  for (int mi = 0; mi < WM; mi++) {
    const int rbase = (mt * 4 * WM + wave * WM + mi) * 32;
    const int row = rbase + lc;
    uint32_t rk = 0, cav = 0;
    if (MODE != 2) {
      const int32_t rs = e.rowsum[bz * e.rs_bs + row];
      cav = (uint32_t)e.ca[bz * e.rs_bs + row];
      rk = (uint32_t)rs + (uint32_t)e.K * cav;
    }
#pragma unroll
    for (int n = 0; n < 4; n++) {
#pragma unroll
      for (int g = 0; g < 4; g++) {
        const int cl = n * 32 + 8 * g + 4 * lh;  // column within the tile
        const int col = nt * TN + cl;           // < npad: arrays in bounds
        int4v v;
        if (MODE == 2) {
          v = (int4v){acc[mi][n][4 * g], acc[mi][n][4 * g + 1], acc[mi][n][4 * g + 2],
                      acc[mi][n][4 * g + 3]};
        } else {
          const int4v cbv = *reinterpret_cast<const int4v *>(&e.cb[bz * e.cs_bs + col]);
          const int4v csv = *reinterpret_cast<const int4v *>(&e.colsum[bz * e.cs_bs + col]);
#pragma unroll
          for (int i = 0; i < 4; i++)
            v[i] = (int32_t)((uint32_t)acc[mi][n][4 * g + i] + (uint32_t)cbv[i] * rk +
                             cav * (uint32_t)csv[i]);
        }
        if (MODE == 1) {
          if (row >= M || col >= N) continue;
          uint32_t pk = 0;
#pragma unroll
          for (int i = 0; i < 4; i++) {
            const float pf = (float)((double)v[i] * (double)mult);
            int qv = (int)__builtin_amdgcn_fmed3f(rintf(pf), -65536.f, 65536.f) + e.y_zp;
            qv = qv < e.lo ? e.lo : (qv > e.hi ? e.hi : qv);
            pk |= (uint32_t)(qv & 255) << (8 * i);
          }
          uint8_t *yp = static_cast<uint8_t *>(y) + (yb + row) * N + col;
          if (vec_ok && col + 3 < N) {
            *reinterpret_cast<uint32_t *>(yp) = pk;
          } else {
#pragma unroll
            for (int i = 0; i < 4; i++)
              if (col + i < N) yp[i] = (uint8_t)(pk >> (8 * i));
          }
        } else {
          *reinterpret_cast<int4v *>(&stage[lc * SROW + cl]) = v;
        }
      }
    }
    if (MODE != 1) {
      // Same-wave LDS traffic completes in order: no barrier between this
      // wave's stage writes and its reads.
      const int c4 = lane & 31;  // 4-column piece of the 128-column row
      const int col = nt * TN + 4 * c4;
      const bool full = vec_ok && col + 3 < N;
#pragma unroll 4
      for (int it = 0; it < 16; it++) {
        const int r = 2 * it + lh;
        const int rr = rbase + r;
        if (rr >= M) continue;
        const int4v v4 = *reinterpret_cast<const int4v *>(&stage[r * SROW + 4 * c4]);
        int32_t *yp = static_cast<int32_t *>(y) +
                      (MODE == 2 ? (int64_t)blockIdx.y * gridDim.z * M * N : 0) +
                      (yb + rr) * N + col;
        if (full) {
          __builtin_nontemporal_store(v4, reinterpret_cast<int4v *>(yp));
        } else {
#pragma unroll
          for (int i = 0; i < 4; i++)
            if (col + i < N) yp[i] = v4[i];
        }
      }
    }
  }
}

// The int8 GEMM for small grids (where the tile plan would split K over
// workgroups and finish with a reduction launch): a workgroup takes 32 rows x
// TN columns and its four waves take a quarter of the 32-k steps each,
// streaming A and B fragments straight into registers (no LDS stage, no
// barrier per step) with RA steps of loads in flight; the four partial tiles
// meet in LDS and are added (int32 wrap-around, so in any order the exact
// result), then the epilogue of k_i8_gemm: v = acc + cb*(rowsum + K*ca) +
// ca*colsum, stored as int32 (MODE 0) or requantised bytes (MODE 1).  Loads
// past a wave's last step go past their resources (zeros, no memory
// touched) instead of sitting under a branch.
template <int MODE>
__global__ __launch_bounds__(256, 2) void k_i8_gemm_kw(
    const int4v *__restrict__ afrag, int64_t a_bs, const int4v *__restrict__ bfrag,
    int64_t b_bs, void *__restrict__ y, I8Epi e, int M, int N, int kqp, int mt32, int ntiles) {
  __shared__ __align__(16) int32_t part[4][32 * TN];
  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int L = blockIdx.x;
  const int xcd = L & 7, qq = L >> 3;
  const int mt = qq % mt32;  // 32-row tile
  const int nt = (qq / mt32) * 8 + xcd;
  if (nt >= ntiles) return;
  const int64_t bz = blockIdx.z;
  const int lc = lane & 31, lh = lane >> 5;
  auto rsrc = [](const void *base) __attribute__((always_inline)) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, 0x7ffffff0,
                                             0x00020000);
  };
  // A fragments of row tile mt, step j: 1 KB at j; B of column tile nt,
  // n32 block n, step j: 1 KB at (n kqp + j).
  const __amdgpu_buffer_rsrc_t r_a = rsrc(afrag + bz * a_bs + (int64_t)mt * kqp * 64);
  const __amdgpu_buffer_rsrc_t r_b = rsrc(bfrag + bz * b_bs + (int64_t)nt * 4 * kqp * 64);
  // A resource with no records: loads of steps past the wave's last read
  // zeros through it and touch no memory (chosen with a scalar select, so
  // the lane offsets stay fixed registers).
  const __amdgpu_buffer_rsrc_t r_0 =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<int4v *>(afrag), (short)0, 0, 0x00020000);
  const unsigned vo = 16u * (unsigned)lane;
  const int kpw = (kqp + 3) >> 2;
  const int kb = min(kqp, wave * kpw), ke = min(kqp, kb + kpw);
  struct Step {
    int4v a, b[4];
  };
  auto load = [&](int j, Step &sp) __attribute__((always_inline)) {
    const bool live = j < ke;
    sp.a = __builtin_bit_cast(
        int4v, __builtin_amdgcn_raw_buffer_load_b128(live ? r_a : r_0, vo, j * 1024, 0));
#pragma unroll
    for (int n = 0; n < 4; n++)
      sp.b[n] = __builtin_bit_cast(int4v, __builtin_amdgcn_raw_buffer_load_b128(
                                              live ? r_b : r_0, vo, (n * kqp + j) * 1024, 0));
  };
  int16v acc[4];
#pragma unroll
  for (int n = 0; n < 4; n++) acc[n] = (int16v){};
  if (kb < ke) {
    Step ring[KW_RA];
#pragma unroll
    for (int r = 0; r < KW_RA; r++) load(kb + r, ring[r]);
    // Steps past ke (to a multiple of KW_RA) multiply zeros.
    for (int j0 = kb; j0 < ke; j0 += KW_RA) {
#pragma unroll
      for (int r = 0; r < KW_RA; r++) {
        // The slot is reloaded after its products are issued (a reload
        // before them would need a copy of the slot, whose wait would take
        // the loads in flight with it).
#pragma unroll
        for (int n = 0; n < 4; n++)
          acc[n] = __builtin_amdgcn_mfma_i32_32x32x32_i8(ring[r].b[n], ring[r].a, acc[n], 0, 0, 0);
        load(j0 + r + KW_RA, ring[r]);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  }
  // Partial tiles row-major [32 rows][TN] (lane: row lc, columns
  // 32 n + 8 g + 4 lh + i), then the sum over the waves.
  {
    int32_t *pw = part[wave];
#pragma unroll
    for (int n = 0; n < 4; n++)
#pragma unroll
      for (int g = 0; g < 4; g++)
        *reinterpret_cast<int4v *>(&pw[lc * TN + n * 32 + 8 * g + 4 * lh]) =
            (int4v){acc[n][4 * g], acc[n][4 * g + 1], acc[n][4 * g + 2], acc[n][4 * g + 3]};
  }
  __syncthreads();
  // Thread: row r = t / 8, columns c0 .. c0 + 15 (four quads).
  const int r = t >> 3, c0 = 16 * (t & 7);
  const int row = mt * 32 + r;
  if (row >= M) return;
  const int64_t yb = (int64_t)bz * M;
  const int32_t rs = e.rowsum[bz * e.rs_bs + row];
  const uint32_t cav = (uint32_t)e.ca[bz * e.rs_bs + row];
  const uint32_t rk = (uint32_t)rs + (uint32_t)e.K * cav;
  const float mult = MODE == 1 ? i8_mult(e) : 0.f;
  const bool vec_ok = (N % 4) == 0 && e.y_vec;
#pragma unroll
  for (int q4 = 0; q4 < 4; q4++) {
    const int cl = c0 + 4 * q4;
    const int col = nt * TN + cl;  // < npad: the tables are in bounds
    int4v v = *reinterpret_cast<const int4v *>(&part[0][r * TN + cl]);
#pragma unroll
    for (int w = 1; w < 4; w++) {
      const int4v x = *reinterpret_cast<const int4v *>(&part[w][r * TN + cl]);
#pragma unroll
      for (int i = 0; i < 4; i++) v[i] = (int32_t)((uint32_t)v[i] + (uint32_t)x[i]);
    }
    const int4v cbv = *reinterpret_cast<const int4v *>(&e.cb[bz * e.cs_bs + col]);
    const int4v csv = *reinterpret_cast<const int4v *>(&e.colsum[bz * e.cs_bs + col]);
#pragma unroll
    for (int i = 0; i < 4; i++)
      v[i] = (int32_t)((uint32_t)v[i] + (uint32_t)cbv[i] * rk + cav * (uint32_t)csv[i]);
    if (col >= N) continue;
    if (MODE == 1) {
      uint32_t pk = 0;
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const float pf = (float)((double)v[i] * (double)mult);
        int qv = (int)__builtin_amdgcn_fmed3f(rintf(pf), -65536.f, 65536.f) + e.y_zp;
        qv = qv < e.lo ? e.lo : (qv > e.hi ? e.hi : qv);
        pk |= (uint32_t)(qv & 255) << (8 * i);
      }
      uint8_t *yp = static_cast<uint8_t *>(y) + (yb + row) * N + col;
      if (vec_ok && col + 3 < N) {
        *reinterpret_cast<uint32_t *>(yp) = pk;
      } else {
#pragma unroll
        for (int i = 0; i < 4; i++)
          if (col + i < N) yp[i] = (uint8_t)(pk >> (8 * i));
      }
    } else {
      int32_t *yp = static_cast<int32_t *>(y) + (yb + row) * N + col;
      if (vec_ok && col + 3 < N) {
        __builtin_nontemporal_store(v, reinterpret_cast<int4v *>(yp));
      } else {
#pragma unroll
        for (int i = 0; i < 4; i++)
          if (col + i < N) yp[i] = v[i];
      }
    }
  }
}

// Split-K finish (and the K = 0 case, ks = 0): sums the partials of every
// split and applies the epilogue; one thread per output element.
template <int REQ>
__global__ __launch_bounds__(256) void k_i8_reduce(const int32_t *__restrict__ part,
                                                   void *__restrict__ y, I8Epi e, int64_t batch,
                                                   int64_t M, int64_t N, int ks) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t tot = batch * M * N;
  if (idx >= tot) return;
  const int64_t col = idx % N, brow = idx / N, bz = brow / M, row = brow % M;
  uint32_t s = 0;
  for (int k = 0; k < ks; k++) s += (uint32_t)part[(int64_t)k * tot + idx];
  const int64_t rslot = bz * e.rs_bs + row;
  i8_finish<REQ>(y, idx, (int32_t)s, e.rowsum[rslot], e.ca[rslot], e.colsum[bz * e.cs_bs + col],
                 e.cb[bz * e.cs_bs + col], e);
}

struct I8Plan {
  int wm, mtiles, m32n, ntiles, ks, sps, nstage;
  int64_t kpad, mpad;
  size_t off_a, off_rs, off_ca, off_za, off_part, total;
};

#ifndef MG_I8_AUTO_SMALL
#define MG_I8_AUTO_SMALL 1
#endif
#ifndef MG_I8_KWAVE
#define MG_I8_KWAVE 1
#endif


// a_batch: batches of A; batch: output batches (grid z).
I8Plan plan_i8(int64_t a_batch, int64_t batch, int64_t M, int64_t K, int64_t N,
               int max_ks = 0, bool small_tiles = false) {
  I8Plan p;
  p.kpad = (K + 255) / 256 * 256;
  p.nstage = (int)(p.kpad / 256);
  // 128-row tiles also where 256-row ones would leave CUs without a tile:
  // more workgroups and less K split (fewer partial sums to reduce); the
  // sums are exact integers, so the plan does not change the result.
  const int64_t big_tiles = (M + 255) / 256 * ((N + TN - 1) / TN) * batch;
  if (MG_I8_AUTO_SMALL && big_tiles < 256) small_tiles = true;
  p.wm = M > 128 && !small_tiles ? 2 : 1;
  p.mtiles = (int)((M + 128 * p.wm - 1) / (128 * p.wm));
  p.m32n = p.mtiles * 4 * p.wm;
  p.mpad = (int64_t)p.m32n * 32;
  p.ntiles = (int)((N + TN - 1) / TN);
  // Split K until ~2 workgroups per CU, keeping >= 2 stages per split.
  const int64_t tiles = (int64_t)p.mtiles * p.ntiles * batch;
  int ks = 1;
  while (tiles * ks * 2 <= 512 && p.nstage / (ks * 2) >= 2 && (max_ks <= 0 || ks * 2 <= max_ks))
    ks *= 2;
  p.sps = (p.nstage + ks - 1) / ks;
  p.ks = (p.nstage + p.sps - 1) / p.sps;
  p.off_a = 0;
  p.off_rs = mg_align(p.off_a + (size_t)a_batch * p.mpad * p.kpad);
  p.off_ca = mg_align(p.off_rs + (size_t)a_batch * p.mpad * 4);
  p.off_za = mg_align(p.off_ca + (size_t)a_batch * p.mpad * 4);
  p.off_part = mg_align(p.off_za + (size_t)(M + 1) * 4);
  p.total = mg_align(p.off_part + (p.ks > 1 ? (size_t)p.ks * batch * M * N * 4 : 0));
  return p;
}

}  // namespace

// Weight arrays (bq fragments, colsum, cb) laid out in one allocation.
size_t mg_int8_weight_ws_bytes(int64_t K, int64_t N) {
  const int64_t kqp = (K + 255) / 256 * 8, n32 = (N + 127) / 128 * 4;
  return mg_align((size_t)n32 * kqp * 64 * 16) + 2 * mg_align((size_t)n32 * 32 * 4);
}

static void int8_carve(mg_weight *w, void *base) {
  const int64_t kqp = (w->K + 255) / 256 * 8, n32 = (w->N + 127) / 128 * 4;
  char *p = static_cast<char *>(base);
  w->i8.kpad = kqp * 32;
  w->i8.npad = n32 * 32;
  w->i8.bq = reinterpret_cast<int8_t *>(p);
  p += mg_align((size_t)n32 * kqp * 64 * 16);
  w->i8.colsum = reinterpret_cast<int32_t *>(p);
  p += mg_align((size_t)n32 * 32 * 4);
  w->i8.cb = reinterpret_cast<int32_t *>(p);
}

// Prepacks B already in device memory.  b_zp is a host array.
mg_status mg_int8_prepack_dev(mg_ctx *ctx, mg_weight *w, const void *b_dev,
                              int32_t b_signed, const int32_t *b_zp,
                              int64_t b_zp_len, void *ws_weight) {
  int8_carve(w, ws_weight);
  w->i8.b_signed = b_signed;
  const int64_t K = w->K, N = w->N;
  const int kqp = (int)(w->i8.kpad / 32), n32 = (int)(w->i8.npad / 32);
  hipStream_t st = ctx->stream;
  int zb_scalar = 0;
  const int32_t *zb_dev = nullptr;
  int zb_len = 0;
  if (b_zp && b_zp_len == 1) {
    zb_scalar = b_zp[0];
  } else if (b_zp && b_zp_len > 1) {
    // Per-column zero points travel through the cb array: written there
    // first, then read back by the colsum kernel (one thread per column).
    MG_TRY(mg_h2d_table(ctx, w->i8.cb, b_zp, (size_t)b_zp_len * 4));
    zb_dev = w->i8.cb;
    zb_len = (int)b_zp_len;
  }
  const int64_t slots = (int64_t)n32 * kqp * 64;
  hipLaunchKernelGGL(k_i8_prep_b, dim3((unsigned)((slots + 255) / 256), 1), dim3(256), 0, st,
                     static_cast<const uint8_t *>(b_dev), b_signed, K, N, n32, kqp,
                     reinterpret_cast<int4v *>(w->i8.bq));
  MG_TRY(mg_launch_check("k_i8_prep_b"));
  hipLaunchKernelGGL(k_i8_colsum, dim3((unsigned)((w->i8.npad + 63) / 64), 1), dim3(256), 0,
                     st, static_cast<const uint8_t *>(b_dev), b_signed, K, N, w->i8.npad,
                     zb_scalar, zb_dev, zb_len, w->i8.colsum, w->i8.cb);
  return mg_launch_check("k_i8_colsum");
}

mg_status mg_int8_prepack_t_dev(mg_ctx *ctx, mg_weight *w, const void *bt_dev,
                                int32_t b_signed, const int32_t *b_zp, int64_t b_zp_len,
                                void *ws_weight) {
  int8_carve(w, ws_weight);
  w->i8.b_signed = b_signed;
  const int64_t K = w->K, N = w->N;
  const int kqp = (int)(w->i8.kpad / 32), n32 = (int)(w->i8.npad / 32);
  hipStream_t st = ctx->stream;
  int zb_scalar = 0;
  const int32_t *zb_dev = nullptr;
  int zb_len = 0;
  if (b_zp && b_zp_len == 1) {
    zb_scalar = b_zp[0];
  } else if (b_zp && b_zp_len > 1) {  // through the cb array, as mg_int8_prepack_dev
    MG_TRY(mg_h2d_table(ctx, w->i8.cb, b_zp, (size_t)b_zp_len * 4));
    zb_dev = w->i8.cb;
    zb_len = (int)b_zp_len;
  }
  const int64_t slots = (int64_t)n32 * kqp * 64;
  hipLaunchKernelGGL(k_i8_prep_bt, dim3((unsigned)((slots + 255) / 256)), dim3(256), 0, st,
                     static_cast<const uint8_t *>(bt_dev), b_signed, K, N, n32, kqp,
                     reinterpret_cast<int4v *>(w->i8.bq));
  MG_TRY(mg_launch_check("k_i8_prep_bt"));
  hipLaunchKernelGGL(k_i8_colsum_t, dim3((unsigned)((w->i8.npad + 3) / 4)), dim3(256), 0, st,
                     static_cast<const uint8_t *>(bt_dev), b_signed, K, N, w->i8.npad, zb_scalar,
                     zb_dev, zb_len, w->i8.colsum, w->i8.cb);
  return mg_launch_check("k_i8_colsum_t");
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

size_t mg_int8_ws_bytes(const mg_weight *w, int64_t rows, int max_ks) {
  return plan_i8(1, 1, rows, w->K, w->N, max_ks).total;
}

mg_i8_a_layout mg_int8_a_layout(int64_t rows, int64_t K, int64_t N, int max_ks,
                                bool small_tiles) {
  const I8Plan p = plan_i8(1, 1, rows, K, N, max_ks, small_tiles);
  mg_i8_a_layout l;
  l.off_a = p.off_a;
  l.off_rs = p.off_rs;
  l.off_ca = p.off_ca;
  l.m32n = p.m32n;
  l.kqp = p.nstage * QS;
  l.total = p.total;
  return l;
}

// Shared launcher.  a_batch/b_batch: 1 or batch; rows per batch = M.  bq,
// colsum, cb: prepacked B (b_batch copies, npad columns each).
static mg_status int8_launch(mg_ctx *ctx, const int8_t *bq, const int32_t *colsum,
                             const int32_t *cb, int64_t npad, int64_t b_batch,
                             const void *a_dev, int32_t a_signed, int64_t a_batch,
                             int64_t M, int64_t N, int64_t K, const int32_t *a_zp,
                             int64_t a_zp_len, const mg_requant *rq, void *y_dev,
                             void *ws, int max_ks = 0, bool a_ready = false,
                             bool small_tiles = false) {
  if (M == 0 || N == 0) return MG_OK;
  const int64_t batch = a_batch > b_batch ? a_batch : b_batch;
  const I8Plan p = plan_i8(a_batch, batch, M, K, N, max_ks, small_tiles);
  hipStream_t st = ctx->stream;
  char *base = static_cast<char *>(ws);
  int4v *afrag = reinterpret_cast<int4v *>(base + p.off_a);
  int32_t *rowsum = reinterpret_cast<int32_t *>(base + p.off_rs);
  int32_t *ca = reinterpret_cast<int32_t *>(base + p.off_ca);
  int za_scalar = 0, za_len = 0;
  const int32_t *za = nullptr;
  if (rq && rq->a_zp_dev) {
    za = rq->a_zp_dev;  // one int32 in device memory
    za_len = 1;
  } else if (a_zp && a_zp_len == 1) {
    za_scalar = a_zp[0];
  } else if (a_zp && a_zp_len > 1) {
    int32_t *zd = reinterpret_cast<int32_t *>(base + p.off_za);
    MG_TRY(mg_h2d_table(ctx, zd, a_zp, (size_t)a_zp_len * 4));
    za = zd;
    za_len = (int)a_zp_len;
  }
  const int kqp = p.nstage * QS;
  if (!a_ready) {  // else the caller wrote afrag, rowsum and ca (mg_int8_a_layout)
    const int vec = (reinterpret_cast<uintptr_t>(a_dev) % 16 == 0 && K % 16 == 0) ? 1 : 0;
    hipLaunchKernelGGL(k_i8_prep_a, dim3((unsigned)p.m32n, (unsigned)a_batch),
                       dim3(64 * PREP_A_WAVES), 0, st,
                       static_cast<const uint8_t *>(a_dev), K, M * K, a_signed, vec, M, K, kqp,
                       p.m32n, za_scalar, za, za_len, afrag, rowsum, ca);
    MG_TRY(mg_launch_check("k_i8_prep_a"));
  }
  I8Epi e{};
  e.colsum = colsum;
  e.cb = cb;
  e.cs_bs = b_batch > 1 ? npad : 0;
  e.rowsum = rowsum;
  e.ca = ca;
  e.rs_bs = a_batch > 1 ? p.mpad : 0;
  e.K = (int)K;
  const bool req = mg_requant_out(rq);
  if (req) {
    e.mult = rq->mult;
    e.y_zp = rq->y_zp;
    e.lo = rq->lo;
    e.hi = rq->hi;
    e.a_scale_dev = rq->a_scale_dev;
    e.b_scale = rq->b_scale;
    e.y_scale = rq->y_scale;
  }
  int32_t *part = reinterpret_cast<int32_t *>(base + p.off_part);
  const int mode = K == 0 ? 3 : (p.ks > 1 ? 2 : (req ? 1 : 0));
  // Where the plan splits K: 32-row tiles whose waves split K
  // (k_i8_gemm_kw, no reduction launch) when they give at least as many
  // workgroups with work as the split (row tiles x column tiles x splits).
  const int64_t mt32 = (M + 31) / 32;
  if (MG_I8_KWAVE && mode == 2 && mt32 >= (int64_t)p.mtiles * p.ks) {
    e.y_vec = reinterpret_cast<uintptr_t>(y_dev) % 16 == 0 ? 1 : 0;
    const int64_t a_bs = a_batch > 1 ? (int64_t)p.m32n * kqp * 64 : 0;
    const int64_t b_bs = b_batch > 1 ? (npad / 32) * kqp * 64 : 0;
    const dim3 grid((unsigned)(((p.ntiles + 7) / 8) * 8 * mt32), 1, (unsigned)batch);
#define MG_I8_KW_ARGS                                                                          afrag, a_bs, reinterpret_cast<const int4v *>(bq), b_bs, y_dev, e, (int)M, (int)N, kqp,         (int)mt32, p.ntiles
    if (req) hipLaunchKernelGGL(k_i8_gemm_kw<1>, grid, dim3(256), 0, st, MG_I8_KW_ARGS);
    else hipLaunchKernelGGL(k_i8_gemm_kw<0>, grid, dim3(256), 0, st, MG_I8_KW_ARGS);
#undef MG_I8_KW_ARGS
    return mg_launch_check("k_i8_gemm_kw");
  }
  e.y_vec = (mode == 2 || reinterpret_cast<uintptr_t>(y_dev) % 16 == 0) ? 1 : 0;
  if (mode != 3) {
    const int64_t a_bs = a_batch > 1 ? (int64_t)p.m32n * kqp * 64 : 0;
    const int64_t b_bs = b_batch > 1 ? (npad / 32) * kqp * 64 : 0;
    const unsigned gx = (unsigned)(((p.ntiles + 7) / 8) * 8 * p.mtiles);
    const dim3 grid(gx, (unsigned)p.ks, (unsigned)batch);
    void *yk = mode == 2 ? static_cast<void *>(part) : y_dev;
#define MG_I8_ARGS                                                                         \
  afrag, a_bs, reinterpret_cast<const int4v *>(bq), b_bs, yk, e, (int)M, (int)N, kqp, p.mtiles, \
      p.ntiles, p.sps
#define MG_I8_LAUNCH(WM_, MODE_) \
  hipLaunchKernelGGL((k_i8_gemm<WM_, MODE_>), grid, dim3(256), 0, st, MG_I8_ARGS)
    if (p.wm == 2) {
      if (mode == 0) MG_I8_LAUNCH(2, 0);
      else if (mode == 1) MG_I8_LAUNCH(2, 1);
      else MG_I8_LAUNCH(2, 2);
    } else {
      if (mode == 0) MG_I8_LAUNCH(1, 0);
      else if (mode == 1) MG_I8_LAUNCH(1, 1);
      else MG_I8_LAUNCH(1, 2);
    }
#undef MG_I8_LAUNCH
#undef MG_I8_ARGS
    MG_TRY(mg_launch_check("k_i8_gemm"));
  }
  if (mode >= 2) {  // split-K partials, or K == 0 (empty sums: the epilogue alone)
    const int64_t tot = batch * M * N;
    const unsigned blocks = (unsigned)((tot + 255) / 256);
    const int ks = mode == 3 ? 0 : p.ks;
    if (req)
      hipLaunchKernelGGL(k_i8_reduce<1>, dim3(blocks), dim3(256), 0, st, part, y_dev, e, batch,
                         M, N, ks);
    else
      hipLaunchKernelGGL(k_i8_reduce<0>, dim3(blocks), dim3(256), 0, st, part, y_dev, e, batch,
                         M, N, ks);
    MG_TRY(mg_launch_check("k_i8_reduce"));
  }
  return MG_OK;
}

mg_status mg_int8_run(mg_ctx *ctx, const mg_weight *w, const void *a_dev,
                      int32_t a_signed, int64_t rows, const int32_t *a_zp,
                      int64_t a_zp_len, const mg_requant *rq, void *y_dev,
                      void *ws, int max_ks) {
  return int8_launch(ctx, w->i8.bq, w->i8.colsum, w->i8.cb, w->i8.npad, 1, a_dev, a_signed, 1,
                     rows, w->N, w->K, a_zp, a_zp_len, rq, y_dev, ws, max_ks);
}

mg_status mg_int8_run_a_ready(mg_ctx *ctx, const mg_weight *w, int64_t rows,
                              const mg_requant *rq, void *y_dev, void *ws, int max_ks,
                              bool small_tiles) {
  return int8_launch(ctx, w->i8.bq, w->i8.colsum, w->i8.cb, w->i8.npad, 1, nullptr, 0, 1, rows,
                     w->N, w->K, nullptr, 0, rq, y_dev, ws, max_ks, true, small_tiles);
}

// Runtime (non-weight) batched form: B is prepacked per batch into the
// workspace first.
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
  const int64_t kqp = (K + 255) / 256 * 8, n32 = (N + 127) / 128 * 4, npad = n32 * 32;
  hipStream_t st = ctx->stream;
  char *p = static_cast<char *>(ws);
  int8_t *bq = reinterpret_cast<int8_t *>(p);
  p += mg_align((size_t)b_batch * n32 * kqp * 64 * 16);
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
    MG_TRY(mg_h2d_table(ctx, zb_dev, b_zp, (size_t)b_zp_len * 4));
    zb_len = (int)b_zp_len;
  }
  const int64_t slots = n32 * kqp * 64;
  hipLaunchKernelGGL(k_i8_prep_b, dim3((unsigned)((slots + 255) / 256), (unsigned)b_batch),
                     dim3(256), 0, st, static_cast<const uint8_t *>(b_dev), b_signed, K, N,
                     (int)n32, (int)kqp, reinterpret_cast<int4v *>(bq));
  MG_TRY(mg_launch_check("k_i8_prep_b"));
  hipLaunchKernelGGL(k_i8_colsum, dim3((unsigned)((npad + 63) / 64), (unsigned)b_batch),
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
  const int64_t kqp = (K + 255) / 256 * 8, n32 = (N + 127) / 128 * 4, npad = n32 * 32;
  const size_t b = mg_align((size_t)b_batch * n32 * kqp * 64 * 16) +
                   2 * mg_align((size_t)b_batch * npad * 4) + mg_align((size_t)(N + 1) * 4);
  return b + plan_i8(a_batch, a_batch > b_batch ? a_batch : b_batch, M, K, N).total;
}

// ------------------------------------------------------------ long K
//
// MatMulInteger accumulates in Dart's 64-bit int and returns Tensor.int64
// (lib/src/onnx_qlinear_ops.dart:55-80).  A k term is at most 255 * 255 in
// magnitude, so the int32 GEMM above is exact for K <= 33025.  Longer rows
// are cut into segments of MG_I8_SEG k: each segment runs the int32 GEMM
// (exact, |sum| <= 32768 * 65025 < 2^31) on contiguous copies of its A
// columns and B rows, and the segment sums are added in int64.  QLinearMatMul
// then requantises the int64 sum as the reference does: (double)acc * mult
// rounded to f32, round half to even, + y_zp, clamped (:100-106).

namespace {

constexpr int64_t MG_I8_SEG = 32768;

__global__ __launch_bounds__(256) void k_i64_accum(const int32_t *__restrict__ part,
                                                   int64_t *__restrict__ acc, int64_t n,
                                                   int first) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  acc[i] = first ? (int64_t)part[i] : acc[i] + (int64_t)part[i];
}

__global__ __launch_bounds__(256) void k_i64_requant(const int64_t *__restrict__ acc,
                                                     uint8_t *__restrict__ y, int64_t n,
                                                     float mult, int32_t y_zp, int32_t lo,
                                                     int32_t hi) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const float p = (float)((double)acc[i] * (double)mult);
  // Rounded values beyond +-65536 saturate alike after + y_zp and the clamp.
  int q = (int)__builtin_amdgcn_fmed3f(rintf(p), -65536.f, 65536.f) + y_zp;
  q = q < lo ? lo : (q > hi ? hi : q);
  y[i] = (uint8_t)q;
}

struct LongKLayout {
  int64_t seg, nseg;
  size_t off_a, off_b, off_part, off_acc, off_run, total;
};

LongKLayout long_k_layout(int64_t a_batch, int64_t b_batch, int64_t M, int64_t K, int64_t N,
                          bool requant) {
  LongKLayout l;
  const int64_t batch = a_batch > b_batch ? a_batch : b_batch;
  l.nseg = K <= MG_I8_SEG ? 1 : (K + MG_I8_SEG - 1) / MG_I8_SEG;
  l.seg = l.nseg == 1 ? K : MG_I8_SEG;
  const bool copy = l.nseg > 1;
  l.off_a = 0;
  l.off_b = l.off_a + (copy ? mg_align((size_t)(a_batch * M * l.seg)) : 0);
  l.off_part = l.off_b + (copy ? mg_align((size_t)(b_batch * l.seg * N)) : 0);
  l.off_acc = l.off_part + mg_align((size_t)(batch * M * N) * 4);
  l.off_run = l.off_acc + (requant ? mg_align((size_t)(batch * M * N) * 8) : 0);
  l.total = l.off_run + mg_int8_batched_ws_bytes(a_batch, b_batch, M, l.seg, N);
  return l;
}

}  // namespace

size_t mg_int8_long_k_ws_bytes(int64_t a_batch, int64_t b_batch, int64_t M, int64_t K, int64_t N,
                               bool requant) {
  return long_k_layout(a_batch, b_batch, M, K, N, requant).total;
}

mg_status mg_int8_run_long_k(mg_ctx *ctx, const void *a_dev, int32_t a_signed, int64_t a_batch,
                             const void *b_dev, int32_t b_signed, int64_t b_batch, int64_t M,
                             int64_t K, int64_t N, const int32_t *a_zp, int64_t a_zp_len,
                             const int32_t *b_zp, int64_t b_zp_len, const mg_requant *rq,
                             void *y_dev, void *ws) {
  const bool req = mg_requant_out(rq);
  const LongKLayout l = long_k_layout(a_batch, b_batch, M, K, N, req);
  const int64_t batch = a_batch > b_batch ? a_batch : b_batch;
  const int64_t tot = batch * M * N;
  if (tot == 0) return MG_OK;
  hipStream_t st = ctx->stream;
  char *base = static_cast<char *>(ws);
  int32_t *part = reinterpret_cast<int32_t *>(base + l.off_part);
  int64_t *acc = req ? reinterpret_cast<int64_t *>(base + l.off_acc)
                     : static_cast<int64_t *>(y_dev);
  const unsigned blocks = (unsigned)((tot + 255) / 256);
  for (int64_t s = 0; s < l.nseg; s++) {
    const int64_t k0 = s * l.seg, kn = std::min<int64_t>(l.seg, K - k0);
    const void *as = a_dev, *bs = b_dev;
    if (l.nseg > 1) {
      // A[:, :, k0:k0+kn] and B[:, k0:k0+kn, :] as contiguous operands.
      char *ad = base + l.off_a, *bd = base + l.off_b;
      MG_HIP(hipMemcpy2DAsync(ad, (size_t)kn, static_cast<const char *>(a_dev) + k0, (size_t)K,
                              (size_t)kn, (size_t)(a_batch * M), hipMemcpyDeviceToDevice, st));
      MG_HIP(hipMemcpy2DAsync(bd, (size_t)(kn * N),
                              static_cast<const char *>(b_dev) + k0 * N, (size_t)(K * N),
                              (size_t)(kn * N), (size_t)b_batch, hipMemcpyDeviceToDevice, st));
      as = ad;
      bs = bd;
    }
    MG_TRY(mg_int8_run_batched(ctx, as, a_signed, a_batch, bs, b_signed, b_batch, M, kn, N, a_zp,
                               a_zp_len, b_zp, b_zp_len, nullptr, part, base + l.off_run));
    hipLaunchKernelGGL(k_i64_accum, dim3(blocks), dim3(256), 0, st, part, acc, tot,
                       s == 0 ? 1 : 0);
    MG_TRY(mg_launch_check("k_i64_accum"));
  }
  if (req) {
    hipLaunchKernelGGL(k_i64_requant, dim3(blocks), dim3(256), 0, st, acc,
                       static_cast<uint8_t *>(y_dev), tot, rq->mult, rq->y_zp, rq->lo, rq->hi);
    MG_TRY(mg_launch_check("k_i64_requant"));
  }
  return MG_OK;
}
