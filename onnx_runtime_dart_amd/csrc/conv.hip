// Convolution family on gfx950 fp32 MFMA (v_mfma_f32_32x32x2_f32) as an
// implicit GEMM: no im2col buffer is written; the workgroup gathers its
// operand tiles straight from the NC* tensors into LDS.  ConvInteger and
// QLinearConv with one group take the int8 MFMA GEMM over a byte im2col
// instead (below); grouped integer convolutions stay on this kernel.
//
// Reference semantics:
//   Conv          lib/src/onnx_nn_ops.dart:179-817 (pads resolved by
//                 _resolvePads :38-87; 1-D runs as 2-D with height 1)
//   ConvTranspose lib/src/onnx_nn_ops.dart:818-1059
//   ConvInteger   lib/src/onnx_qlinear_ops.dart:232-337 (_convIntAcc)
//   QLinearConv   lib/src/onnx_qlinear_ops.dart:339-382
//
// Per (batch b, group g) the output is a GEMM Y[m][o] = sum_k W[m][k] X[k][o]
// with rows m = the group's output channels, columns o = output positions
// (depth, height, width flattened) and k = (input channel c of the group,
// kernel tap r).  X[k][o] is the input at the tap's position, 0 where that
// position is padding (or, transposed, where no input maps there):
//   Conv           i = o * str - pad + kk * dil
//   ConvTranspose  i = (o + pad - kk * dil) / str, only if the division is exact
// per spatial axis.  ConvTranspose thus gathers (each output sums its
// contributing inputs) instead of scattering, so no atomics are needed and
// the result is deterministic.
//
// Integer kinds (ConvInteger / QLinearConv): operands enter as the exact
// floats (x - x_zp) and (w - w_zp[m]), both in [-255, 255], so every MFMA
// product is exact and any partial sum of up to 256 of them is an integer
// below 2^24, also exact in fp32.  The accumulators are therefore moved into
// int32 every 256 k (and at the end): bit-exact int32 sums, like the
// reference's integer loop.  Requantisation (QLinearConv) is done in double:
// q = roundHalfEven((acc + bias) * mult[m]) + y_zp, clamped to [lo, hi], with
// mult = x_scale * w_scale[m] / y_scale formed in double, as the reference
// does.
//
// Tiles and MFMA core follow the fp32 GEMM: 128 x 128 workgroup tiles (2 x 2
// waves of 64 x 64) with 16-k stages, or 64 x 64 (one 32 x 32 tile per wave)
// with 32-k stages when the larger tile would not give two workgroups per CU
// (always for the integer kinds).  Stages are double-buffered in LDS as
// [row][k] with rows padded by 4 floats; step s of a stage gives lane l the
// k = (KS / 2)(l / 32) + s, so each lane reads its k run with 16-byte loads.
#include <hip/hip_runtime.h>

#include <cmath>

#include "mg_internal.h"

namespace {

typedef float float16v __attribute__((ext_vector_type(16)));
typedef int int16v __attribute__((ext_vector_type(16)));
typedef int int4v __attribute__((ext_vector_type(4)));

// Element e of a byte tensor as an integer (u8 or i8 by a uniform kind).
__device__ inline int load_int(const uint8_t *p, int64_t i, int kind) {
  const uint8_t b = p[i];
  return kind == MG_CONV_I8 ? (int)(int8_t)b : (int)b;
}

// Sub-pixel phases of a strided ConvTranspose with unit dilation.  Output
// position o along an axis reads input i = (o + pad - k) / str for the taps
// k with k == (o + pad) mod str; so the outputs of one phase ph = o mod str
// (o = ph + str * o') use only the taps k = r + str * k' with r = (ph + pad)
// mod str, and read i = o' + base - k' with base = (ph + pad - r) / str: a
// forward convolution of stride 1 and dilation -1 over a 1/str-sized kernel.
// Each phase then issues only its own taps, where the gather form issues all
// of them for every output.
// All phases run as one launch (grid z = phase); each workgroup takes its
// phase's geometry from this table.
constexpr int MG_CONV_MAX_PHASES = 16;
struct ConvPhases {
  int n;                            // phases (str0 * str1 * str2)
  int64_t off[MG_CONV_MAX_PHASES];  // first element of each phase's weights
  int64_t ker[MG_CONV_MAX_PHASES][3];
  int64_t out[MG_CONV_MAX_PHASES][3], pad[MG_CONV_MAX_PHASES][3], yb[MG_CONV_MAX_PHASES][3];
};

__host__ __device__ inline int64_t floor_mod(int64_t a, int64_t m) { return ((a % m) + m) % m; }

bool use_phases(const mg_conv_problem &p) {
  if (!p.trans || p.xk != MG_CONV_F32) return false;
  const int64_t np = p.str[0] * p.str[1] * p.str[2];
  return p.dil[0] == 1 && p.dil[1] == 1 && p.dil[2] == 1 && np > 1 && np <= MG_CONV_MAX_PHASES;
}

// Phase (pz, py, px) = index ((pz * s1) + py) * s2 + px: sub-kernel dims and
// weight offsets (weights laid out [phase][group][m][c][k']).
ConvPhases phase_table(const mg_conv_problem &p) {
  ConvPhases t{};
  t.n = (int)(p.str[0] * p.str[1] * p.str[2]);
  int64_t off = 0;
  for (int ph = 0; ph < t.n; ph++) {
    const int64_t pv[3] = {ph / (p.str[1] * p.str[2]), (ph / p.str[2]) % p.str[1],
                           ph % p.str[2]};
    int64_t kk = 1;
    for (int d = 0; d < 3; d++) {
      const int64_t r = floor_mod(pv[d] + p.pad[d], p.str[d]);
      t.ker[ph][d] = r < p.ker[d] ? (p.ker[d] - r + p.str[d] - 1) / p.str[d] : 0;
      kk *= t.ker[ph][d];
    }
    t.off[ph] = off;
    off += p.group * p.mg * p.cg * kk;
  }
  return t;
}

// BUF (float kinds, every element offset of x, w and y below 2^29): the
// gathered input taps and the bounds-checked weight runs are raw buffer
// loads, an element outside the tensor or in the padding getting an offset
// past the resource (read as zero in hardware), and the outputs raw buffer
// stores.  With a select on the
// loaded value instead, the compiler waits for the next stage's loads right
// after issuing them, and no stage overlaps its successor's loads.
template <int WT, int KS, bool TR, bool INT, bool BUF>
__global__ __launch_bounds__(256) void k_conv(const mg_conv_problem p0, int pix_tiles,
                                              const ConvPhases ph) {
  constexpr int T = 64 * WT, LDX = KS + 4, NS = KS / 2;
  constexpr int E = KS * T / 256;  // elements per thread and operand per stage
  constexpr int FLUSH = 256 / KS;  // stages per exact fp32 segment (integer kinds)
  __shared__ __attribute__((aligned(16))) float As[2][T * LDX];
  __shared__ __attribute__((aligned(16))) float Bs[2][T * LDX];
  const int t = threadIdx.x;
  const int lane = t & 63, wave = t >> 6;
  const int wm = wave & 1, wn = wave >> 1;
  const int l32 = lane & 31, h = lane >> 5;
  mg_conv_problem p = p0;
  if (p0.phased) {  // phase blockIdx.z of a strided ConvTranspose
    const int z3 = (int)blockIdx.z;
    const int64_t kk3 = ph.ker[z3][0] * ph.ker[z3][1] * ph.ker[z3][2];
    for (int d = 0; d < 3; d++) {
      p.out[d] = ph.out[z3][d];
      p.ker[d] = ph.ker[z3][d];
      p.pad[d] = ph.pad[z3][d];
      p.yb[d] = ph.yb[z3][d];
    }
    p.w = static_cast<const float *>(p0.w) + ph.off[z3];
    p.w_cs = kk3;
    p.w_ms = p.cg * kk3;
    p.w_gs = p.mg * p.cg * kk3;
    // The grid covers the largest phase: tiles past this one's outputs exit.
    if ((int64_t)(blockIdx.x % pix_tiles) * 64 * WT >= p.out[0] * p.out[1] * p.out[2]) return;
  }
  const int64_t z = blockIdx.x / pix_tiles;  // batch * group + g
  const int64_t b = z / p.group, g = z % p.group;
  const int64_t c0 = (int64_t)(blockIdx.x % pix_tiles) * T;  // first output position
  const int64_t r0 = (int64_t)blockIdx.y * T;                // first output channel of the group
  const int64_t K = p.cg * p.ker[0] * p.ker[1] * p.ker[2];
  const int kk = (int)(p.ker[0] * p.ker[1] * p.ker[2]), k12 = (int)(p.ker[1] * p.ker[2]);
  const int kw2 = (int)p.ker[2];
  const int64_t out_sp = p.out[0] * p.out[1] * p.out[2];
  const int64_t in_sp = p.in[0] * p.in[1] * p.in[2];
  const int o12 = (int)(p.out[1] * p.out[2]), o2 = (int)p.out[2];

  // A (weights): thread row ra, k run [ka, ka + E) of the stage.
  const int ra = t / (KS / E), ka = (t % (KS / E)) * E;
  const int64_t mrow = r0 + ra;
  const bool row_ok = mrow < p.mg;
  const int64_t wbase = g * p.w_gs + (row_ok ? mrow : 0) * p.w_ms;
  float wz = 0.f;
  if (INT && row_ok) wz = p.w_zp[g * p.mg + mrow];
  // B (input window): thread k kb, output run [nb, nb + E) of the stage.
  const int kb = t / (T / E), nb = (t % (T / E)) * E;
  const int64_t xbatch = (b * p.c + g * p.cg) * in_sp;  // channel 0 of the group
  // The thread's output positions are the same in every stage: for Conv
  // their window origins (o * str - pad per axis) and the origin's offset in
  // an input plane are computed once; a stage adds its tap's shift.
  // ConvTranspose: (o + pad) = q * str + rem per axis; a tap kk * dil =
  // kq * str + kr reaches input q - kq exactly when rem == kr.  q goes to
  // bz/by/bx and spe, the three remainders (each < 2^10) packed in rem3.
  int bz[E], by[E], bx[E], spe[E], rem3[E];
  bool nok[E];
  if (TR) {
    const int64_t n0 = c0 + nb;
    int oz = (int)(n0 / o12), oy = (int)((n0 % o12) / o2), ox = (int)(n0 % o2);
    const int sz = (int)p.str[0], sy = (int)p.str[1], sx = (int)p.str[2];
#pragma unroll
    for (int e = 0; e < E; e++) {
      nok[e] = n0 + e < out_sp;
      const int tz = oz + (int)p.pad[0], ty = oy + (int)p.pad[1], tx = ox + (int)p.pad[2];
      // floor division (t may be negative with negative pads)
      const int qz = tz >= 0 ? tz / sz : -((-tz + sz - 1) / sz);
      const int qy = ty >= 0 ? ty / sy : -((-ty + sy - 1) / sy);
      const int qx = tx >= 0 ? tx / sx : -((-tx + sx - 1) / sx);
      bz[e] = qz, by[e] = qy, bx[e] = qx;
      rem3[e] = (tz - qz * sz) | ((ty - qy * sy) << 10) | ((tx - qx * sx) << 20);
      spe[e] = (qz * (int)p.in[1] + qy) * (int)p.in[2] + qx;
      if (++ox == o2) {
        ox = 0;
        if (++oy == (int)p.out[1]) oy = 0, oz++;
      }
    }
  } else {
    const int64_t n0 = c0 + nb;
    int oz = (int)(n0 / o12), oy = (int)((n0 % o12) / o2), ox = (int)(n0 % o2);
#pragma unroll
    for (int e = 0; e < E; e++) {
      nok[e] = n0 + e < out_sp;
      bz[e] = oz * (int)p.str[0] - (int)p.pad[0];
      by[e] = oy * (int)p.str[1] - (int)p.pad[1];
      bx[e] = ox * (int)p.str[2] - (int)p.pad[2];
      spe[e] = (bz[e] * (int)p.in[1] + by[e]) * (int)p.in[2] + bx[e];
      if (++ox == o2) {
        ox = 0;
        if (++oy == (int)p.out[1]) oy = 0, oz++;
      }
    }
  }

  float va[E], vb[E];
  auto rsrc = [](const void *base) __attribute__((always_inline)) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, 0x7ffffff0,
                                             0x00020000);
  };
  const __amdgpu_buffer_rsrc_t rw = rsrc(p.w), rx = rsrc(p.x);
  constexpr unsigned kOob = 0x80000000u;
  auto ldb = [](__amdgpu_buffer_rsrc_t r, unsigned off) __attribute__((always_inline)) {
    return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 0));
  };
  auto load = [&](int st) __attribute__((always_inline)) {
    const int64_t k0 = (int64_t)st * KS;
    // Conv weights: an output channel's k run is contiguous (channel stride
    // = taps); whole aligned runs load as two 16-byte loads.
    if (!TR && !INT && row_ok && k0 + ka + E <= K && ((wbase + k0 + ka) & 3) == 0) {
      const float *wp = static_cast<const float *>(p.w) + wbase + k0 + ka;
#pragma unroll
      for (int q = 0; q < E / 4; q++) {
        const float4 x = *reinterpret_cast<const float4 *>(wp + 4 * q);
        va[4 * q] = x.x, va[4 * q + 1] = x.y, va[4 * q + 2] = x.z, va[4 * q + 3] = x.w;
      }
    } else if (!TR && INT && row_ok && k0 + ka + E <= K && ((wbase + k0 + ka) & 7) == 0) {
      // integer weights: the 8 bytes of the run in one load
      const uint2 x = *reinterpret_cast<const uint2 *>(static_cast<const uint8_t *>(p.w) + wbase +
                                                       k0 + ka);
#pragma unroll
      for (int e = 0; e < E; e++) {
        const uint32_t by = ((e < 4 ? x.x : x.y) >> (8 * (e & 3))) & 0xFFu;
        const int wv = p.wk == MG_CONV_I8 ? (int)(int8_t)by : (int)by;
        va[e] = (float)wv - wz;
      }
    } else {  // weights: taps of one output channel, k consecutive
      int64_t k = k0 + ka;
      int c = (int)(k / kk), r = (int)(k - (int64_t)c * kk);
#pragma unroll
      for (int e = 0; e < E; e++) {
        const bool ok = row_ok && k + e < K;
        const int64_t off = ok ? wbase + (int64_t)c * p.w_cs + r : 0;
        if constexpr (BUF) {
          va[e] = ldb(rw, ok ? (unsigned)off * 4u : kOob);
        } else {
          float v;
          if (INT)
            v = (float)load_int(static_cast<const uint8_t *>(p.w), off, p.wk) - wz;
          else
            v = static_cast<const float *>(p.w)[off];
          va[e] = ok ? v : 0.f;
        }
        if (++r == kk) r = 0, c++;
      }
    }
    {  // input window: one tap, E consecutive output positions
      const int64_t k = k0 + kb;
      const bool k_ok = k < K;
      const int c = k_ok ? (int)(k / kk) : 0;
      const int r = k_ok ? (int)(k - (int64_t)c * kk) : 0;
      const int kz = r / k12, ky = (r % k12) / kw2, kx = r % kw2;
      const int64_t xc = xbatch + (int64_t)c * in_sp;
      if (!TR) {
        const int shz = kz * (int)p.dil[0], shy = ky * (int)p.dil[1], shx = kx * (int)p.dil[2];
        const int tap = (shz * (int)p.in[1] + shy) * (int)p.in[2] + shx;
#pragma unroll
        for (int e = 0; e < E; e++) {
          const int iz = bz[e] + shz, iy = by[e] + shy, ix = bx[e] + shx;
          const bool ok = k_ok && nok[e] && (unsigned)iz < (unsigned)p.in[0] &&
                          (unsigned)iy < (unsigned)p.in[1] && (unsigned)ix < (unsigned)p.in[2];
          const int64_t off = ok ? xc + (spe[e] + tap) : 0;
          if constexpr (BUF) {
            vb[e] = ldb(rx, ok ? (unsigned)off * 4u : kOob);
            continue;
          }
          float v;
          if (INT)
            v = (float)(load_int(static_cast<const uint8_t *>(p.x), off, p.xk) - p.x_zp);
          else
            v = static_cast<const float *>(p.x)[off];
          vb[e] = ok ? v : 0.f;
        }
        return;
      }
      {
        const int sz = (int)p.str[0], sy = (int)p.str[1], sx = (int)p.str[2];
        const int dz = kz * (int)p.dil[0], dy = ky * (int)p.dil[1], dx = kx * (int)p.dil[2];
        const int kqz = dz / sz, kqy = dy / sy, kqx = dx / sx;
        const int kr3 = (dz - kqz * sz) | ((dy - kqy * sy) << 10) | ((dx - kqx * sx) << 20);
        const int tap = (kqz * (int)p.in[1] + kqy) * (int)p.in[2] + kqx;
#pragma unroll
        for (int e = 0; e < E; e++) {
          const int iz = bz[e] - kqz, iy = by[e] - kqy, ix = bx[e] - kqx;
          const bool ok = k_ok && nok[e] && rem3[e] == kr3 && (unsigned)iz < (unsigned)p.in[0] &&
                          (unsigned)iy < (unsigned)p.in[1] && (unsigned)ix < (unsigned)p.in[2];
          const int64_t off = ok ? xc + (spe[e] - tap) : 0;
          if constexpr (BUF) {
            vb[e] = ldb(rx, ok ? (unsigned)off * 4u : kOob);
            continue;
          }
          float v;
          if (INT)
            v = (float)(load_int(static_cast<const uint8_t *>(p.x), off, p.xk) - p.x_zp);
          else
            v = static_cast<const float *>(p.x)[off];
          vb[e] = ok ? v : 0.f;
        }
        return;
      }
    }
  };
  auto store = [&](int buf) __attribute__((always_inline)) {
    float *da = &As[buf][ra * LDX + ka];
#pragma unroll
    for (int q = 0; q < E / 4; q++)
      *reinterpret_cast<float4 *>(da + 4 * q) =
          make_float4(va[4 * q], va[4 * q + 1], va[4 * q + 2], va[4 * q + 3]);
    float *db = &Bs[buf][nb * LDX + kb];
#pragma unroll
    for (int e = 0; e < E; e++) db[e * LDX] = vb[e];
  };

  float16v acc[WT][WT];
  int16v iacc[WT][WT];
#pragma unroll
  for (int i = 0; i < WT; i++)
#pragma unroll
    for (int j = 0; j < WT; j++) acc[i][j] = (float16v){}, iacc[i][j] = (int16v){};

  const int nst = (int)((K + KS - 1) / KS);
  if (nst > 0) {
    load(0);
    store(0);
  }
  __syncthreads();
  for (int st = 0; st < nst; st++) {
    const int buf = st & 1;
    const bool more = st + 1 < nst;
    if (more) load(st + 1);
    float a[WT][NS], bf[WT][NS];
#pragma unroll
    for (int i = 0; i < WT; i++) {
      const float *q = &As[buf][(wm * 32 * WT + i * 32 + l32) * LDX + NS * h];
#pragma unroll
      for (int u = 0; u < NS / 4; u++) {
        const float4 x = *reinterpret_cast<const float4 *>(q + 4 * u);
        a[i][4 * u] = x.x, a[i][4 * u + 1] = x.y, a[i][4 * u + 2] = x.z, a[i][4 * u + 3] = x.w;
      }
    }
#pragma unroll
    for (int j = 0; j < WT; j++) {
      const float *q = &Bs[buf][(wn * 32 * WT + j * 32 + l32) * LDX + NS * h];
#pragma unroll
      for (int u = 0; u < NS / 4; u++) {
        const float4 x = *reinterpret_cast<const float4 *>(q + 4 * u);
        bf[j][4 * u] = x.x, bf[j][4 * u + 1] = x.y, bf[j][4 * u + 2] = x.z,
        bf[j][4 * u + 3] = x.w;
      }
    }
#pragma unroll
    for (int s = 0; s < NS; s++)
#pragma unroll
      for (int i = 0; i < WT; i++)
#pragma unroll
        for (int j = 0; j < WT; j++)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i][s], bf[j][s], acc[i][j], 0, 0, 0);
    if (INT && ((st + 1) % FLUSH == 0 || !more)) {
#pragma unroll
      for (int i = 0; i < WT; i++)
#pragma unroll
        for (int j = 0; j < WT; j++)
#pragma unroll
          for (int v = 0; v < 16; v++) {
            iacc[i][j][v] += (int)acc[i][j][v];  // an exact integer below 2^24
            acc[i][j][v] = 0.f;
          }
    }
    if (more) store(buf ^ 1);
    __syncthreads();
  }

    // Lane l holds output position l % 32 and channels 8 (v / 4) + 4 (l / 32)
  // + v % 4 of each 32 x 32 tile; 32 lanes write consecutive positions.  A
  // sub-pixel phase places its position o' at o' * ys + yb of the full
  // output.
  const int64_t y_sp = p.phased ? p.yo[0] * p.yo[1] * p.yo[2] : out_sp;
#pragma unroll
  for (int i = 0; i < WT; i++)
#pragma unroll
    for (int j = 0; j < WT; j++) {
      int64_t col = c0 + wn * 32 * WT + j * 32 + l32;
      const bool col_ok = col < out_sp;
      if (!BUF && !col_ok) continue;
      if (p.phased) {
        const int64_t oz = col / o12, oy = (col % o12) / o2, ox = col % o2;
        col = ((oz * p.ys[0] + p.yb[0]) * p.yo[1] + (oy * p.ys[1] + p.yb[1])) * p.yo[2] +
              (ox * p.ys[2] + p.yb[2]);
      }
      // The tile's biases, all loaded before the first store.
      float bv[16];
      if (!INT && p.bias) {
#pragma unroll
        for (int v = 0; v < 16; v++) {
          const int64_t row = r0 + wm * 32 * WT + i * 32 + 8 * (v >> 2) + 4 * h + (v & 3);
          bv[v] = static_cast<const float *>(p.bias)[g * p.mg + (row < p.mg ? row : 0)];
        }
      }
      if constexpr (BUF) {
        // Raw buffer stores, outputs past the tile's channels or positions
        // given an offset past the resource (dropped in hardware): no
        // branches, so the stores issue back to back (behind per-element
        // branches the compiler waited for each store before the next).
        const __amdgpu_buffer_rsrc_t ry = rsrc(p.y);
#pragma unroll
        for (int v = 0; v < 16; v++) {
          const int64_t row = r0 + wm * 32 * WT + i * 32 + 8 * (v >> 2) + 4 * h + (v & 3);
          const bool ok = col_ok && row < p.mg;
          const int64_t oi = (b * p.m + g * p.mg + row) * y_sp + col;
          float y = acc[i][j][v];
          if (p.bias) y += bv[v];
          __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, y), ry,
                                                ok ? (unsigned)oi * 4u : kOob, 0, 0);
        }
        continue;
      }
#pragma unroll
      for (int v = 0; v < 16; v++) {
        const int64_t row = r0 + wm * 32 * WT + i * 32 + 8 * (v >> 2) + 4 * h + (v & 3);
        if (row >= p.mg) continue;
        const int64_t ch = g * p.mg + row;
        const int64_t oi = (b * p.m + ch) * y_sp + col;
        if (!INT) {
          float y = acc[i][j][v];
          if (p.bias) y += bv[v];
          static_cast<float *>(p.y)[oi] = y;
        } else if (p.mode == MG_CONV_OUT_I32) {
          static_cast<int32_t *>(p.y)[oi] = iacc[i][j][v];
        } else {
          const int64_t s = (int64_t)iacc[i][j][v] +
                            (p.bias ? (int64_t) static_cast<const int32_t *>(p.bias)[ch] : 0);
          const double q = rint((double)s * p.mult[ch]) + (double)p.y_zp;  // half to even
          const double cl = fmin(fmax(q, (double)p.lo), (double)p.hi);
          static_cast<uint8_t *>(p.y)[oi] = (uint8_t)(int)cl;
        }
      }
    }
}

// One thread per weight element (group g, out channel m, in channel c, tap
// k): tap k belongs to the phases whose r == k mod str, i.e. ph == (k - pad)
// mod str, at sub-kernel tap k' = k / str.
__global__ __launch_bounds__(256) void k_conv_phase_weights(const mg_conv_problem p,
                                                            const ConvPhases t,
                                                            float *__restrict__ out) {
  const int64_t taps = p.ker[0] * p.ker[1] * p.ker[2];
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= p.group * p.mg * p.cg * taps) return;
  const int64_t tap = idx % taps, c = (idx / taps) % p.cg, m = (idx / (taps * p.cg)) % p.mg,
                g = idx / (taps * p.cg * p.mg);
  const int64_t k[3] = {tap / (p.ker[1] * p.ker[2]), (tap / p.ker[2]) % p.ker[1],
                        tap % p.ker[2]};
  int64_t ph = 0, kq[3];
  for (int d = 0; d < 3; d++) {
    ph = ph * p.str[d] + floor_mod(k[d] - p.pad[d], p.str[d]);
    kq[d] = k[d] / p.str[d];
  }
  const int64_t *kp = t.ker[ph];
  const int64_t kk = kp[0] * kp[1] * kp[2];
  const int64_t kl = (kq[0] * kp[1] + kq[1]) * kp[2] + kq[2];
  out[t.off[ph] + ((g * p.mg + m) * p.cg + c) * kk + kl] =
      static_cast<const float *>(p.w)[g * p.w_gs + m * p.w_ms + c * p.w_cs + tap];
}

#ifndef MG_CONV_BUFFER_LOADS
#define MG_CONV_BUFFER_LOADS 1
#endif
template <bool TR, bool INT>
void launch_conv(const mg_conv_problem &p, bool big, int64_t out_sp, hipStream_t st,
                 const ConvPhases &tb) {
  const int T = big ? 128 : 64;
  const int64_t pix_tiles = (out_sp + T - 1) / T;
  const dim3 grid((unsigned)(pix_tiles * p.n * p.group), (unsigned)((p.mg + T - 1) / T),
                  (unsigned)(p.phased ? tb.n : 1));
  if constexpr (!INT) {
    // Buffer loads need every element offset of x and w below 2^29 (bytes
    // below 2^31); phase weights hold as many elements as the filter.
    const int64_t taps = p.ker[0] * p.ker[1] * p.ker[2];
    const int64_t x_el = p.n * p.c * p.in[0] * p.in[1] * p.in[2];
    const int64_t w_el = p.group * p.mg * p.cg * taps;
    const int64_t y_el = p.n * p.m * (p.phased ? p.yo[0] * p.yo[1] * p.yo[2] : out_sp);
    const bool buf = MG_CONV_BUFFER_LOADS && x_el < ((int64_t)1 << 29) &&
                     w_el < ((int64_t)1 << 29) && y_el < ((int64_t)1 << 29);
    if (big && buf)
      hipLaunchKernelGGL((k_conv<2, 16, TR, INT, true>), grid, dim3(256), 0, st, p,
                         (int)pix_tiles, tb);
    else if (big)
      hipLaunchKernelGGL((k_conv<2, 16, TR, INT, false>), grid, dim3(256), 0, st, p,
                         (int)pix_tiles, tb);
    else if (buf)
      hipLaunchKernelGGL((k_conv<1, 32, TR, INT, true>), grid, dim3(256), 0, st, p,
                         (int)pix_tiles, tb);
    else
      hipLaunchKernelGGL((k_conv<1, 32, TR, INT, false>), grid, dim3(256), 0, st, p,
                         (int)pix_tiles, tb);
    return;
  }
  hipLaunchKernelGGL((k_conv<1, 32, TR, INT, false>), grid, dim3(256), 0, st, p, (int)pix_tiles,
                     tb);
}

// ------------------------------------- integer convolution on int8 MFMA
//
// ConvInteger / QLinearConv with one group (forward) run as MatMulInteger's
// int8 MFMA GEMM (int8.hip, exact int32 sums with the zero points taken out
// as row / column sum terms) over an im2col of the input, gathered straight
// into the GEMM's operand fragments:
//   A[b * O + o][k] = x[b][c][position of tap r at output o]  (k = c * taps + r)
//                     or the byte x_zp where the tap falls in the padding,
//   B[k][m]         = w[m][k]  (prepacked per call from the filter as laid out),
//   C[b * O + o][m] = sum_k (A - x_zp)(B - w_zp[m])   (int32),
// so a padded tap contributes (x_zp - x_zp) (w - w_zp) = 0, as in the
// reference's loop, which skips it.  The epilogue transposes C into
// y[b][m][o] through LDS and, for QLinearConv, requantises each sum as the
// fp32-MFMA kernel does (bias, double multiplier, round half to even).

// The GEMM's A operand gathered straight from the input, in the layout
// MatMulInteger's prepass (k_i8_prep_a) writes: per 32-row tile m32 and
// 32-k fragment q, lane l (row 32 m32 + l % 32) holds the 16 bytes at k =
// 128 (q / 4) + 64 (l / 32) + 16 (q % 4), re-centred to signed (u8 ^ 0x80),
// zero for k >= K or rows past the last; plus the row sums of those bytes
// over k < K and ca = (x signed ? 0 : 128) - x_zp.  A row is an output
// position (b, o); byte k = (channel c, tap r) is the input at the tap's
// position, or x_zp where that lies in the padding.
// Workgroup = 64 rows (two row tiles) and one of CONV_FRAG_GROUPS groups of
// 16-k chunks, 4 waves; thread = one row, and wave w of group g takes the
// chunks ch = 4 g + w (mod 4 CONV_FRAG_GROUPS), so the chunk's channel and
// tap offsets (from tab, built by k_conv_tab_i8) are the same for the
// whole wave (scalar loads); each thread stores
// its 16 bytes into its fragment's lane.  The row sums meet in LDS, then in
// rowsum by integer atomics (exact in any order; rowsum zeroed first by
// k_conv_tab_i8).  32-bit index arithmetic: the plan keeps every index
// below 2^31.
constexpr int CONV_FRAG_WAVES = 4, CONV_FRAG_GROUPS = 16;
__global__ __launch_bounds__(64 * CONV_FRAG_WAVES) void k_conv_frag_i8(
    const mg_conv_problem p, int K, int O, int rows, int rows_pad, int kqp,
    const int2 *__restrict__ tab, int4v *__restrict__ afrag, int32_t *__restrict__ rowsum,
    int32_t *__restrict__ ca) {
  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int grp = blockIdx.y;
  constexpr int STRIDE = CONV_FRAG_WAVES * CONV_FRAG_GROUPS;  // between a wave's chunks
  const int row = blockIdx.x * 64 + lane;
  const bool live = row < rows;
  const int b = live ? row / O : 0, o = live ? row - b * O : 0;
  const int out1 = (int)p.out[1], out2 = (int)p.out[2];
  const int oz = o / (out1 * out2), oy = (o / out2) % out1, ox = o % out2;
  const int in0 = (int)p.in[0], in1 = (int)p.in[1], in2 = (int)p.in[2];
  const int bz = oz * (int)p.str[0] - (int)p.pad[0], by0 = oy * (int)p.str[1] - (int)p.pad[1],
            bx = ox * (int)p.str[2] - (int)p.pad[2];
  const int in_sp = in0 * in1 * in2;
  // Taps whose input position lies inside this row's window (bit r of inw).
  const int kd = (int)p.ker[0], kh = (int)p.ker[1], kw = (int)p.ker[2];
  uint64_t inw = 0;
  for (int r = 0, kz = 0; kz < kd; kz++)
    for (int ky = 0; ky < kh; ky++)
      for (int kx = 0; kx < kw; kx++, r++) {
        const int iz = bz + kz * (int)p.dil[0], iy = by0 + ky * (int)p.dil[1],
                  ix = bx + kx * (int)p.dil[2];
        if ((unsigned)iz < (unsigned)in0 && (unsigned)iy < (unsigned)in1 &&
            (unsigned)ix < (unsigned)in2)
          inw |= 1ull << r;
      }
  if (!live) inw = 0;
  // Byte loads through a buffer resource over x: an offset past its end reads
  // 0 without a memory access (taps outside the window).
  const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<void *>(p.x), (short)0, (int)(p.n * p.c * in_sp), 0x00020000);
  const int org = b * (int)p.c * in_sp + (bz * in1 + by0) * in2 + bx;  // may lie outside
  const uint32_t flip = p.xk == MG_CONV_I8 ? 0u : 0x80u;
  const uint8_t zb = (uint8_t)((p.x_zp & 0xFF) ^ flip);
  const int nchunk = kqp * 2;  // 16-k chunks up to kpad
  int s = 0;
  // Two chunks per pass, all 32 byte loads issued before any is used.
  for (int ch0 = grp * CONV_FRAG_WAVES + wave; ch0 < nchunk; ch0 += 2 * STRIDE) {
    uint8_t raw[2][16];
    uint32_t okm[2] = {0u, 0u};
#pragma unroll
    for (int u = 0; u < 2; u++) {
      const int k0 = min((ch0 + u * STRIDE) * 16, nchunk * 16 - 16);  // wave-uniform
      int4 te[8];  // entries k0 .. k0 + 15 (the table runs to kpad)
#pragma unroll
      for (int j2 = 0; j2 < 8; j2++) te[j2] = reinterpret_cast<const int4 *>(tab + k0)[j2];
#pragma unroll
      for (int e = 0; e < 16; e++) {
        const int toff = (e & 1) ? te[e >> 1].z : te[e >> 1].x;
        const int tr = (e & 1) ? te[e >> 1].w : te[e >> 1].y;  // tap; 64 past K
        const bool ok = tr < 64 && ((inw >> (tr & 63)) & 1ull);
        raw[u][e] = (uint8_t)__builtin_amdgcn_raw_buffer_load_b8(
            rx, ok ? (unsigned)(org + toff) : 0x7ffffff0u, 0, 0);
        okm[u] |= (uint32_t)ok << e;
      }
    }
#pragma unroll
    for (int u = 0; u < 2; u++) {
      const int ch = ch0 + u * STRIDE;
      if (ch >= nchunk) break;
      const int k0 = ch * 16;
      uint32_t w[4] = {0u, 0u, 0u, 0u};
#pragma unroll
      for (int e = 0; e < 16; e++) {
        // in the window: the byte; in the padding (k < K): x_zp; k >= K or a dead row: 0
        const uint8_t v = ((okm[u] >> e) & 1u) ? (uint8_t)(raw[u][e] ^ flip)
                          : (live && k0 + e < K) ? zb : (uint8_t)0;
        w[e >> 2] |= (uint32_t)v << (8 * (e & 3));
      }
      const int4v v = (int4v){(int)w[0], (int)w[1], (int)w[2], (int)w[3]};
      s = __builtin_amdgcn_sdot4(v.x, 0x01010101, s, false);
      s = __builtin_amdgcn_sdot4(v.y, 0x01010101, s, false);
      s = __builtin_amdgcn_sdot4(v.z, 0x01010101, s, false);
      s = __builtin_amdgcn_sdot4(v.w, 0x01010101, s, false);
      if (row < rows_pad) {
        const int q = (k0 >> 7) * 4 + ((k0 >> 4) & 3), fl = (row & 31) + 32 * ((k0 >> 6) & 1);
        afrag[((int64_t)(row >> 5) * kqp + q) * 64 + fl] = v;
      }
    }
  }
  __shared__ int red[CONV_FRAG_WAVES][64];
  red[wave][lane] = s;
  __syncthreads();
  if (t < 64 && row < rows_pad) {
    int tot = 0;
#pragma unroll
    for (int wv = 0; wv < CONV_FRAG_WAVES; wv++) tot += red[wv][t];
    atomicAdd(&rowsum[row], tot);
    if (grp == 0) ca[row] = (p.xk == MG_CONV_I8 ? 0 : 128) - p.x_zp;
  }
}

// Tap table of the gather: tab[k] = {c * in_sp + (dz * in1 + dy) * in2 + dx,
// r} for k = (channel c, tap r = (kz, ky, kx)) < K, d* = k* * dilation, and
// {0, 64} for K <= k < kpad; and rowsum zeroed for the gather's atomics.
__global__ __launch_bounds__(256) void k_conv_tab_i8(const mg_conv_problem p, int K, int kpad,
                                                     int2 *__restrict__ tab,
                                                     int32_t *__restrict__ rowsum, int rows_pad) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < rows_pad) rowsum[i] = 0;
  if (i >= kpad) return;
  if (i >= K) {
    tab[i] = make_int2(0, 64);
    return;
  }
  const int kh = (int)p.ker[1], kw = (int)p.ker[2], k12 = kh * kw;
  const int taps = (int)p.ker[0] * k12;
  const int c = i / taps, r = i - c * taps;
  const int dz = (r / k12) * (int)p.dil[0], dy = ((r / kw) % kh) * (int)p.dil[1],
            dx = (r % kw) * (int)p.dil[2];
  const int in1 = (int)p.in[1], in2 = (int)p.in[2];
  const int in_sp = (int)p.in[0] * in1 * in2;
  tab[i] = make_int2(c * in_sp + (dz * in1 + dy) * in2 + dx, r);
}

// C [rows][M] int32 -> y [n][M][O] through a 64 x 64 LDS tile: reads along
// m, writes along o.  REQ: QLinearConv's requantisation, else the int32 sums.
template <bool REQ>
__global__ __launch_bounds__(256) void k_conv_i8_epi(const int32_t *__restrict__ c,
                                                     const mg_conv_problem p, int64_t O,
                                                     int64_t rows) {
  __shared__ int32_t tile[64][65];
  __shared__ double smult[64];
  __shared__ int64_t sbias[64];
  const int t = threadIdx.x, tx = t & 63, ty = t >> 6;
  const int64_t r0 = (int64_t)blockIdx.x * 64, m0 = (int64_t)blockIdx.y * 64;
  const int64_t M = p.m;
#pragma unroll
  for (int i = 0; i < 16; i++) {
    const int64_t r = r0 + 4 * i + ty, m = m0 + tx;
    tile[4 * i + ty][tx] = (r < rows && m < M) ? c[r * M + m] : 0;
  }
  if constexpr (REQ) {  // the tile's channel constants, loaded once
    if (t < 64 && m0 + t < M) {
      smult[t] = p.mult[m0 + t];
      sbias[t] = p.bias ? (int64_t) static_cast<const int32_t *>(p.bias)[m0 + t] : 0;
    }
  }
  __syncthreads();
  const int64_t r = r0 + tx;
  if (r >= rows) return;
  const int64_t b = r / O, o = r - b * O;  // once per thread: the tile row is fixed
#pragma unroll
  for (int i = 0; i < 16; i++) {
    const int64_t m = m0 + 4 * i + ty;
    if (m >= M) continue;
    const int32_t acc = tile[tx][4 * i + ty];
    const int64_t oi = (b * M + m) * O + o;
    if constexpr (REQ) {
      const int64_t sum = (int64_t)acc + sbias[m - m0];
      const double q = rint((double)sum * smult[m - m0]) + (double)p.y_zp;  // half to even
      const double cl = fmin(fmax(q, (double)p.lo), (double)p.hi);
      static_cast<uint8_t *>(p.y)[oi] = (uint8_t)(int)cl;
    } else {
      static_cast<int32_t *>(p.y)[oi] = acc;
    }
  }
}

// Sums of up to this many k stay exact in the int8 GEMM's int32 terms.
constexpr int64_t CONV_I8_MAX_K = 33025;
// Cap on the GEMM's K split (0: the int8 planner's choice).
#ifndef MG_CONV_I8_MAX_KS
#define MG_CONV_I8_MAX_KS 1
#endif

// 128-row GEMM tiles (the convolutions' C x taps x M products are narrow:
// the 256-row tiles leave most CUs idle), and no K split: measured on the
// ResNet-50 3 x 3 layer (6272 x 2304 x 256), the three-way split and its
// reduction cost 30 + 11.4 us against 22.9 us unsplit with 256-row tiles.
#ifndef MG_CONV_I8_SMALL_TILES
#define MG_CONV_I8_SMALL_TILES 1
#endif

struct ConvI8Plan {
  bool ok = false;
  int64_t K = 0, O = 0, rows = 0;
  mg_i8_a_layout a;
  size_t off_w = 0, off_c = 0, off_tab = 0, off_g = 0, total = 0;
};

ConvI8Plan conv_i8_plan(const mg_conv_problem &p) {
  ConvI8Plan q;
  if (p.xk == MG_CONV_F32 || p.trans || p.phased || p.group != 1) return q;
  const bool zp_byte = p.xk == MG_CONV_U8 ? (p.x_zp >= 0 && p.x_zp <= 255)
                                          : (p.x_zp >= -128 && p.x_zp <= 127);
  q.K = p.cg * p.ker[0] * p.ker[1] * p.ker[2];
  q.O = p.out[0] * p.out[1] * p.out[2];
  q.rows = p.n * q.O;
  const int64_t lim = (int64_t)1 << 31;
  // At most 64 taps (the gather's window mask), and x addressed with 32-bit offsets.
  const bool taps_ok = p.ker[0] * p.ker[1] * p.ker[2] <= 64;
  if (p.n * p.c * p.in[0] * p.in[1] * p.in[2] >= lim || !zp_byte || !taps_ok || q.K == 0 || q.K > CONV_I8_MAX_K || q.rows * q.K >= lim || q.K * p.m >= lim ||
      q.rows * p.m >= lim || (q.rows + 63) / 64 > 0x7fffffff || (p.m + 63) / 64 > 65535)
    return q;
  q.a = mg_int8_a_layout(q.rows, q.K, p.m, MG_CONV_I8_MAX_KS, MG_CONV_I8_SMALL_TILES);
  if ((int64_t)q.a.m32n * 32 * ((q.K + 255) / 256 * 256) >= lim) return q;
  q.off_w = 0;
  q.off_c = q.off_w + mg_align(mg_int8_weight_ws_bytes(q.K, p.m));
  q.off_tab = q.off_c + mg_align((size_t)(q.rows * p.m) * 4);
  q.off_g = q.off_tab + mg_align((size_t)((q.K + 255) / 256 * 256) * 8);
  q.total = q.off_g + mg_align(q.a.total);
  q.ok = true;
  return q;
}

mg_status conv_i8_run(mg_ctx *ctx, const mg_conv_problem &p, const ConvI8Plan &q, void *ws) {
  char *base = static_cast<char *>(ws);
  int32_t *c = reinterpret_cast<int32_t *>(base + q.off_c);
  char *g = base + q.off_g;
  hipStream_t st = ctx->stream;
  const int rows_pad = q.a.m32n * 32;
  int32_t *rowsum = reinterpret_cast<int32_t *>(g + q.a.off_rs);
  int2 *tab = reinterpret_cast<int2 *>(base + q.off_tab);
  const int kpad = q.a.kqp * 32;
  const int ntab = std::max(rows_pad, kpad);
  hipLaunchKernelGGL(k_conv_tab_i8, dim3((unsigned)((ntab + 255) / 256)), dim3(256), 0, st, p,
                     (int)q.K, kpad, tab, rowsum, rows_pad);
  MG_TRY(mg_launch_check("k_conv_tab_i8"));
  hipLaunchKernelGGL(k_conv_frag_i8, dim3((unsigned)((rows_pad + 63) / 64), CONV_FRAG_GROUPS),
                     dim3(64 * CONV_FRAG_WAVES), 0, st, p, (int)q.K, (int)q.O, (int)q.rows,
                     rows_pad, q.a.kqp, tab, reinterpret_cast<int4v *>(g + q.a.off_a),
                     reinterpret_cast<int32_t *>(g + q.a.off_rs),
                     reinterpret_cast<int32_t *>(g + q.a.off_ca));
  MG_TRY(mg_launch_check("k_conv_frag_i8"));
  // The filter [M][C taps] is B transposed: prepacked from it directly.
  mg_weight tw{};
  tw.kind = MG_W_INT8;
  tw.K = q.K;
  tw.N = p.m;
  // Per-channel zero points that are all equal go as one scalar (no table).
  int64_t zlen = p.w_zp_len;
  for (int64_t i = 1; i < zlen; i++)
    if (p.w_zp_host[i] != p.w_zp_host[0]) break;
    else if (i == zlen - 1) zlen = 1;
  MG_TRY(mg_int8_prepack_t_dev(ctx, &tw, p.w, p.wk == MG_CONV_I8, p.w_zp_host, zlen,
                               base + q.off_w));
  MG_TRY(mg_int8_run_a_ready(ctx, &tw, q.rows, nullptr, c, g, MG_CONV_I8_MAX_KS,
                             MG_CONV_I8_SMALL_TILES));
  const dim3 grid((unsigned)((q.rows + 63) / 64), (unsigned)((p.m + 63) / 64));
  if (p.mode == MG_CONV_OUT_I32)
    hipLaunchKernelGGL(k_conv_i8_epi<false>, grid, dim3(256), 0, st, c, p, q.O, q.rows);
  else
    hipLaunchKernelGGL(k_conv_i8_epi<true>, grid, dim3(256), 0, st, c, p, q.O, q.rows);
  return mg_launch_check("k_conv_i8_epi");
}

}  // namespace

bool mg_conv_int8_route(const mg_conv_problem &p) { return conv_i8_plan(p).ok; }

size_t mg_conv_ws_bytes(const mg_conv_problem &p) {
  const ConvI8Plan q = conv_i8_plan(p);
  if (q.ok) return q.total;
  if (!use_phases(p)) return 0;
  return mg_align((size_t)(p.group * p.mg * p.cg * p.ker[0] * p.ker[1] * p.ker[2]) * 4);
}

mg_status mg_conv_run(mg_ctx *ctx, const mg_conv_problem &p, void *ws);

namespace {
mg_status conv_launch_all(mg_ctx *ctx, const mg_conv_problem &p, int64_t out_sp,
                          const ConvPhases &tb);

// A strided ConvTranspose as forward convolutions, one per sub-pixel phase,
// in one launch.
mg_status conv_run_phases(mg_ctx *ctx, const mg_conv_problem &p, float *wph) {
  ConvPhases t = phase_table(p);
  const int64_t nw = p.group * p.mg * p.cg * p.ker[0] * p.ker[1] * p.ker[2];
  if (nw > 0) {
    hipLaunchKernelGGL(k_conv_phase_weights, dim3((unsigned)((nw + 255) / 256)), dim3(256), 0,
                       ctx->stream, p, t, wph);
    MG_TRY(mg_launch_check("k_conv_phase_weights"));
  }
  mg_conv_problem q = p;
  q.trans = 0;
  q.phased = 1;
  q.w = wph;
  int64_t max_sp = 0;
  for (int ph = 0; ph < t.n; ph++) {
    const int64_t pv[3] = {ph / (p.str[1] * p.str[2]), (ph / p.str[2]) % p.str[1],
                           ph % p.str[2]};
    int64_t sp = 1;
    for (int d = 0; d < 3; d++) {
      const int64_t r = floor_mod(pv[d] + p.pad[d], p.str[d]);
      t.pad[ph][d] = -((pv[d] + p.pad[d] - r) / p.str[d]);  // exact division
      t.out[ph][d] = p.out[d] > pv[d] ? (p.out[d] - pv[d] + p.str[d] - 1) / p.str[d] : 0;
      t.yb[ph][d] = pv[d];
      sp *= t.out[ph][d];
    }
    max_sp = std::max(max_sp, sp);
  }
  for (int d = 0; d < 3; d++) {
    q.str[d] = 1;
    q.dil[d] = -1;
    q.yo[d] = p.out[d];
    q.ys[d] = p.str[d];
    // The tile plan and grid follow the largest phase.
    q.out[d] = t.out[0][d];
    q.ker[d] = t.ker[0][d];
  }
  return conv_launch_all(ctx, q, max_sp, t);
}
}  // namespace

mg_status mg_conv_run(mg_ctx *ctx, const mg_conv_problem &p, void *ws) {
  const int64_t out_sp = p.out[0] * p.out[1] * p.out[2];
  if (p.n == 0 || p.m == 0 || out_sp == 0) return MG_OK;
  const ConvI8Plan q = conv_i8_plan(p);
  if (q.ok) return conv_i8_run(ctx, p, q, ws);
  if (use_phases(p)) return conv_run_phases(ctx, p, static_cast<float *>(ws));
  return conv_launch_all(ctx, p, out_sp, ConvPhases{});
}

namespace {
mg_status conv_launch_all(mg_ctx *ctx, const mg_conv_problem &p, int64_t out_sp,
                          const ConvPhases &tb) {
  const bool integer = p.xk != MG_CONV_F32;
  // The 128 x 128 tile when it still gives about two workgroups per CU and
  // at most a quarter of its rows are padding (64 output channels, as in a
  // ResNet stem, would waste half of its MFMA work).
  const int64_t nz = p.phased ? tb.n : 1;  // sub-pixel phases in grid z
  const int64_t big_wgs = ((out_sp + 127) / 128) * ((p.mg + 127) / 128) * p.n * p.group * nz;
  const bool big = !integer && big_wgs >= 2 * (int64_t)ctx->num_cus &&
                   3 * ((p.mg + 127) / 128 * 128) <= 4 * (int64_t)p.mg;
  const int64_t wgs = ((out_sp + (big ? 127 : 63)) / (big ? 128 : 64)) * p.n * p.group;
  if (wgs > 0x7fffffff || (p.mg + 63) / 64 > 65535)
    return mg_fail(MG_UNSUPPORTED, "conv: grid too large");
  if (!integer && !p.trans)
    launch_conv<false, false>(p, big, out_sp, ctx->stream, tb);
  else if (!integer)
    launch_conv<true, false>(p, big, out_sp, ctx->stream, tb);
  else if (!p.trans)
    launch_conv<false, true>(p, false, out_sp, ctx->stream, tb);
  else
    return mg_fail(MG_UNSUPPORTED, "conv: transposed integer convolution");
  return mg_launch_check("k_conv");
}
}  // namespace
