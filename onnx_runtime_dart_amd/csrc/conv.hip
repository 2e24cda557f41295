// Convolution family on gfx950 fp32 MFMA (v_mfma_f32_32x32x2_f32) as an
// implicit GEMM: no im2col buffer is written; the workgroup gathers its
// operand tiles straight from the NC* tensors into LDS.
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

template <int WT, int KS, bool TR, bool INT>
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
        float v;
        if (INT)
          v = (float)load_int(static_cast<const uint8_t *>(p.w), off, p.wk) - wz;
        else
          v = static_cast<const float *>(p.w)[off];
        va[e] = ok ? v : 0.f;
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
      if (col >= out_sp) continue;
      if (p.phased) {
        const int64_t oz = col / o12, oy = (col % o12) / o2, ox = col % o2;
        col = ((oz * p.ys[0] + p.yb[0]) * p.yo[1] + (oy * p.ys[1] + p.yb[1])) * p.yo[2] +
              (ox * p.ys[2] + p.yb[2]);
      }
#pragma unroll
      for (int v = 0; v < 16; v++) {
        const int64_t row = r0 + wm * 32 * WT + i * 32 + 8 * (v >> 2) + 4 * h + (v & 3);
        if (row >= p.mg) continue;
        const int64_t ch = g * p.mg + row;
        const int64_t oi = (b * p.m + ch) * y_sp + col;
        if (!INT) {
          float y = acc[i][j][v];
          if (p.bias) y += static_cast<const float *>(p.bias)[ch];
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

template <bool TR, bool INT>
void launch_conv(const mg_conv_problem &p, bool big, int64_t out_sp, hipStream_t st,
                 const ConvPhases &tb) {
  const int T = big ? 128 : 64;
  const int64_t pix_tiles = (out_sp + T - 1) / T;
  const dim3 grid((unsigned)(pix_tiles * p.n * p.group), (unsigned)((p.mg + T - 1) / T),
                  (unsigned)(p.phased ? tb.n : 1));
  if constexpr (!INT) {
    if (big) {
      hipLaunchKernelGGL((k_conv<2, 16, TR, INT>), grid, dim3(256), 0, st, p, (int)pix_tiles,
                         tb);
      return;
    }
  }
  hipLaunchKernelGGL((k_conv<1, 32, TR, INT>), grid, dim3(256), 0, st, p, (int)pix_tiles, tb);
}

}  // namespace

size_t mg_conv_ws_bytes(const mg_conv_problem &p) {
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
