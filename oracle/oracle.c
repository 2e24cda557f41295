/* CPU oracle for the matrix-multiply operator family (TEST INFRASTRUCTURE).
 * See oracle.h for the contract; every routine cites the reference routine it
 * restates.  Built with -ffp-contract=off so that each f32 multiply and add is
 * rounded separately, as the reference's Float32x4 lanes do. */
#include "oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ---------------------------------------------------------------- helpers */

int64_t orc_round_even(double v, int *err) {
  /* _roundEven: floor, compare the fraction against one half, ties to even. */
  if (!isfinite(v)) {
    if (err) *err = ORC_UNSUPPORTED;
    return 0;
  }
  double f = floor(v);
  double frac = v - f;
  int64_t i = (int64_t)f;
  if (frac > 0.5) return i + 1;
  if (frac < 0.5) return i;
  return (i % 2 == 0) ? i : i + 1;
}

/* ------------------------------------------------------------ fp32 kernel */

/* Panel width of _matmul4x16Direct (gemm_kernel_simd.dart:258-261): as many
 * columns as keep k*panel*4 bytes under 192 KiB, a multiple of 4, >= 4, <= n.
 * The panel loop never changes an element's k order, so it only shapes the
 * memory traffic of the CPU baseline. */
static int64_t panel_width(int64_t k, int64_t n) {
  int64_t panel = (192 * 1024) / (k > 0 ? k * 4 : 4);
  panel = (panel >> 2) << 2;
  if (panel < 4) panel = 4;
  if (panel > n) panel = n;
  return panel;
}

void orc_matmul_kernel(const float *a, const float *b, float *out, int64_t m,
                       int64_t k, int64_t n) {
  /* Columns computed in f32 lanes.  Only the m<4 paths (_gemvScalar,
   * _matmulSmallM) leave a scalar double tail beyond the last full lane; for
   * m==1 with n%4==0 the aligned GEMV covers every column (:459-475). */
  const int64_t f32_cols = (m < 4) ? (n & ~(int64_t)3) : n;
  if (k == 0) {
    memset(out, 0, sizeof(float) * (size_t)(m * n));
    return;
  }
  const int64_t panel = panel_width(k, n > 0 ? n : 1);
  for (int64_t p0 = 0; p0 < f32_cols; p0 += panel) {
    const int64_t pw = (p0 + panel <= f32_cols) ? panel : f32_cols - p0;
    int64_t i = 0;
    /* 4-row x 16-column register tiles (:264-340). */
    for (; i + 4 <= m; i += 4) {
      int64_t j = 0;
      for (; j + 16 <= pw; j += 16) {
        float c[4][16];
        memset(c, 0, sizeof c);
        const float *bp = b + p0 + j;
        for (int64_t kk = 0; kk < k; kk++, bp += n) {
          for (int r = 0; r < 4; r++) {
            const float v = a[(i + r) * k + kk];
            for (int q = 0; q < 16; q++) {
              const float prod = v * bp[q];
              c[r][q] = c[r][q] + prod;
            }
          }
        }
        for (int r = 0; r < 4; r++)
          memcpy(out + (i + r) * n + p0 + j, c[r], sizeof(float) * 16);
      }
      for (; j < pw; j++) {
        float c[4] = {0, 0, 0, 0};
        const float *bp = b + p0 + j;
        for (int64_t kk = 0; kk < k; kk++, bp += n) {
          for (int r = 0; r < 4; r++) {
            const float prod = a[(i + r) * k + kk] * bp[0];
            c[r] = c[r] + prod;
          }
        }
        for (int r = 0; r < 4; r++) out[(i + r) * n + p0 + j] = c[r];
      }
    }
    /* Remainder rows one at a time (:342-388). */
    for (; i < m; i++) {
      int64_t j = 0;
      for (; j + 16 <= pw; j += 16) {
        float c[16];
        memset(c, 0, sizeof c);
        const float *bp = b + p0 + j;
        const float *ar = a + i * k;
        for (int64_t kk = 0; kk < k; kk++, bp += n) {
          const float v = ar[kk];
          for (int q = 0; q < 16; q++) {
            const float prod = v * bp[q];
            c[q] = c[q] + prod;
          }
        }
        memcpy(out + i * n + p0 + j, c, sizeof(float) * 16);
      }
      for (; j < pw; j++) {
        float c = 0;
        for (int64_t kk = 0; kk < k; kk++) {
          const float prod = a[i * k + kk] * b[kk * n + p0 + j];
          c = c + prod;
        }
        out[i * n + p0 + j] = c;
      }
    }
  }
  /* Scalar double tails (:601-609, :665-673). */
  for (int64_t i = 0; i < m; i++) {
    for (int64_t j = f32_cols; j < n; j++) {
      double s = 0;
      for (int64_t kk = 0; kk < k; kk++)
        s += (double)a[i * k + kk] * (double)b[kk * n + j];
      out[i * n + j] = (float)s;
    }
  }
}

/* ------------------------------------------------------- GemmPool N-split */

/* The reference's isolate pool for f32 weights (lib/src/parallel_pool.dart:
 * 217-261 partition, :299-329 matmul): W workers, worker w owns columns
 * [start_w, start_w + count_w) with count_w = n / W + (w < n % W), as its own
 * contiguous [k x count_w] slice; a call sends every worker a copy of A, each
 * runs matmulKernel on its slice, and the slabs are stitched by column range.
 * Each column's arithmetic is that of the unsplit kernel (same k order), so
 * the result is bitwise the unsplit one.  Threads stand in for isolates. */
struct orc_pool {
  int workers;
  int64_t k, n;
  int64_t *start, *count;
  float **slice;
};

struct orc_pool_job {
  const struct orc_pool *p;
  int w;
  const float *a;
  int64_t m;
  float *slab;
};

static void *orc_pool_worker(void *arg) {
  struct orc_pool_job *j = (struct orc_pool_job *)arg;
  const struct orc_pool *p = j->p;
  const int64_t nw = p->count[j->w];
  /* The message copy of A (a Float32List sent to the isolate). */
  float *a = (float *)malloc(sizeof(float) * (size_t)(j->m * p->k + 1));
  memcpy(a, j->a, sizeof(float) * (size_t)(j->m * p->k));
  if (nw > 0) orc_matmul_kernel(a, p->slice[j->w], j->slab, j->m, p->k, nw);
  free(a);
  return NULL;
}

void *orc_pool_create(const float *b, int64_t k, int64_t n, int workers) {
  if (workers < 1 || k < 0 || n < 0) return NULL;
  struct orc_pool *p = (struct orc_pool *)calloc(1, sizeof *p);
  p->workers = workers;
  p->k = k;
  p->n = n;
  p->start = (int64_t *)calloc((size_t)workers, sizeof(int64_t));
  p->count = (int64_t *)calloc((size_t)workers, sizeof(int64_t));
  p->slice = (float **)calloc((size_t)workers, sizeof(float *));
  const int64_t base = n / workers, rem = n % workers;
  int64_t col = 0;
  for (int w = 0; w < workers; w++) {
    const int64_t nw = base + (w < rem ? 1 : 0);
    p->start[w] = col;
    p->count[w] = nw;
    p->slice[w] = (float *)malloc(sizeof(float) * (size_t)(k * nw + 1));
    for (int64_t r = 0; r < k; r++)
      memcpy(p->slice[w] + r * nw, b + r * n + col, sizeof(float) * (size_t)nw);
    col += nw;
  }
  return p;
}

int orc_pool_matmul(void *pool, const float *a, int64_t m, float *y) {
  struct orc_pool *p = (struct orc_pool *)pool;
  if (!p || m < 0) return ORC_INVALID_ARGUMENT;
  pthread_t *th = (pthread_t *)calloc((size_t)p->workers, sizeof(pthread_t));
  struct orc_pool_job *jobs =
      (struct orc_pool_job *)calloc((size_t)p->workers, sizeof(struct orc_pool_job));
  for (int w = 0; w < p->workers; w++) {
    jobs[w].p = p;
    jobs[w].w = w;
    jobs[w].a = a;
    jobs[w].m = m;
    jobs[w].slab = (float *)malloc(sizeof(float) * (size_t)(m * p->count[w] + 1));
    pthread_create(&th[w], NULL, orc_pool_worker, &jobs[w]);
  }
  for (int w = 0; w < p->workers; w++) {
    pthread_join(th[w], NULL);
    const int64_t nw = p->count[w], c0 = p->start[w];
    for (int64_t i = 0; i < m; i++)
      memcpy(y + i * p->n + c0, jobs[w].slab + i * nw, sizeof(float) * (size_t)nw);
    free(jobs[w].slab);
  }
  free(jobs);
  free(th);
  return ORC_OK;
}

void orc_pool_destroy(void *pool) {
  struct orc_pool *p = (struct orc_pool *)pool;
  if (!p) return;
  for (int w = 0; w < p->workers; w++) free(p->slice[w]);
  free(p->slice);
  free(p->start);
  free(p->count);
  free(p);
}

/* ------------------------------------------------------------- MatMul f32 */

static int broadcast_shape(const int64_t *x, int xr, const int64_t *y, int yr,
                           int64_t *out, int *outr) {
  int r = xr > yr ? xr : yr;
  for (int d = 0; d < r; d++) {
    int64_t xd = (d < r - xr) ? 1 : x[d - (r - xr)];
    int64_t yd = (d < r - yr) ? 1 : y[d - (r - yr)];
    if (xd != yd && xd != 1 && yd != 1) return ORC_INVALID_ARGUMENT;
    out[d] = (xd == 1) ? yd : xd;
  }
  *outr = r;
  return ORC_OK;
}

/* _flattenBroadcast: flat index into `shape` of the output coordinate
 * `coords` (right-aligned; size-1 dims read index 0). */
static int64_t flatten_broadcast(const int64_t *coords, int cr,
                                 const int64_t *shape, int sr) {
  int64_t idx = 0;
  for (int d = 0; d < sr; d++) {
    int64_t c = coords[d + (cr - sr)];
    idx = idx * shape[d] + (shape[d] == 1 ? 0 : c);
  }
  return idx;
}

int orc_matmul_f32(const float *a, const int64_t *a_shape, int a_rank,
                   const float *b, const int64_t *b_shape, int b_rank,
                   float *y) {
  if (a_rank < 2 || b_rank < 2 || a_rank > 8 || b_rank > 8)
    return ORC_INVALID_ARGUMENT;
  const int64_t m = a_shape[a_rank - 2], k = a_shape[a_rank - 1];
  const int64_t k2 = b_shape[b_rank - 2], n = b_shape[b_rank - 1];
  if (k != k2) return ORC_INVALID_ARGUMENT;
  int64_t ob[8];
  int obr = 0;
  if (broadcast_shape(a_shape, a_rank - 2, b_shape, b_rank - 2, ob, &obr))
    return ORC_INVALID_ARGUMENT;
  int64_t batch = 1, bbatch = 1;
  for (int d = 0; d < obr; d++) batch *= ob[d];
  for (int d = 0; d < b_rank - 2; d++) bbatch *= b_shape[d];
  /* Shared-weight collapse (onnx_ops.dart:1728-1735). */
  if (batch > 1 && bbatch == 1) {
    orc_matmul_kernel(a, b, y, batch * m, k, n);
    return ORC_OK;
  }
  int64_t coords[8] = {0};
  for (int64_t bi = 0; bi < batch; bi++) {
    int64_t rem = bi;
    for (int d = obr - 1; d >= 0; d--) {
      coords[d] = rem % ob[d];
      rem /= ob[d];
    }
    int64_t ai = flatten_broadcast(coords, obr, a_shape, a_rank - 2);
    int64_t bj = flatten_broadcast(coords, obr, b_shape, b_rank - 2);
    orc_matmul_kernel(a + ai * m * k, b + bj * k * n, y + bi * m * n, m, k, n);
  }
  return ORC_OK;
}

/* opMatMul's fallback when the operands are not both Float32List
 * (onnx_ops.dart:1753-1762): per batch (broadcast offsets :1742-1749), each
 * output is `double sum = 0; sum += a.getD(..) * b.getD(..)` over k in order,
 * stored into a Float32List (one rounding).  The operands arrive as the
 * getD doubles; this file is built with -ffp-contract=off, so each product
 * and sum is rounded on its own, as Dart's double arithmetic does. */
int orc_matmul_f64acc(const double *a, const int64_t *a_shape, int a_rank,
                      const double *b, const int64_t *b_shape, int b_rank,
                      float *y) {
  if (a_rank < 2 || b_rank < 2 || a_rank > 8 || b_rank > 8)
    return ORC_INVALID_ARGUMENT;
  const int64_t m = a_shape[a_rank - 2], k = a_shape[a_rank - 1];
  const int64_t k2 = b_shape[b_rank - 2], n = b_shape[b_rank - 1];
  if (k != k2) return ORC_INVALID_ARGUMENT;
  int64_t ob[8];
  int obr = 0;
  if (broadcast_shape(a_shape, a_rank - 2, b_shape, b_rank - 2, ob, &obr))
    return ORC_INVALID_ARGUMENT;
  int64_t batch = 1;
  for (int d = 0; d < obr; d++) batch *= ob[d];
  int64_t coords[8] = {0};
  for (int64_t bi = 0; bi < batch; bi++) {
    int64_t rem = bi;
    for (int d = obr - 1; d >= 0; d--) {
      coords[d] = rem % ob[d];
      rem /= ob[d];
    }
    const double *ab = a + flatten_broadcast(coords, obr, a_shape, a_rank - 2) * m * k;
    const double *bb = b + flatten_broadcast(coords, obr, b_shape, b_rank - 2) * k * n;
    float *yb = y + bi * m * n;
    for (int64_t i = 0; i < m; i++)
      for (int64_t j = 0; j < n; j++) {
        double sum = 0;
        for (int64_t kk = 0; kk < k; kk++) sum += ab[i * k + kk] * bb[kk * n + j];
        yb[i * n + j] = (float)sum;
      }
  }
  return ORC_OK;
}

int orc_gemm_f32(const float *a, const int64_t *a_shape, const float *b,
                 const int64_t *b_shape, const float *c, const int64_t *c_shape,
                 int c_rank, double alpha, double beta, int trans_a,
                 int trans_b, float *y) {
  const int64_t m = trans_a ? a_shape[1] : a_shape[0];
  const int64_t k = trans_a ? a_shape[0] : a_shape[1];
  const int64_t kb = trans_b ? b_shape[1] : b_shape[0];
  const int64_t n = trans_b ? b_shape[0] : b_shape[1];
  if (k != kb) return ORC_INVALID_ARGUMENT;
  /* opTranspose copies (onnx_ops.dart:2161-2162; the graph caches the
   * transB copy of an initializer, onnx_graph.dart:2159-2161). */
  float *at = NULL, *bt = NULL;
  const float *ap = a, *bp = b;
  if (trans_a) {
    at = (float *)malloc(sizeof(float) * (size_t)(m * k + 1));
    for (int64_t i = 0; i < m; i++)
      for (int64_t kk = 0; kk < k; kk++) at[i * k + kk] = a[kk * m + i];
    ap = at;
  }
  if (trans_b) {
    bt = (float *)malloc(sizeof(float) * (size_t)(k * n + 1));
    for (int64_t kk = 0; kk < k; kk++)
      for (int64_t j = 0; j < n; j++) bt[kk * n + j] = b[j * k + kk];
    bp = bt;
  }
  orc_matmul_kernel(ap, bp, y, m, k, n);
  free(at);
  free(bt);
  /* alpha in place: f32 element times a double, stored back as f32. */
  if (alpha != 1.0)
    for (int64_t i = 0; i < m * n; i++) y[i] = (float)((double)y[i] * alpha);
  if (c != NULL) {
    if (c_rank > 2) return ORC_INVALID_ARGUMENT;
    int64_t cs[2] = {1, 1};
    for (int d = 0; d < c_rank; d++) cs[2 - c_rank + d] = c_shape[d];
    if ((cs[0] != 1 && cs[0] != m) || (cs[1] != 1 && cs[1] != n))
      return ORC_INVALID_ARGUMENT;
    for (int64_t i = 0; i < m; i++)
      for (int64_t j = 0; j < n; j++) {
        float cv = c[(cs[0] == 1 ? 0 : i) * cs[1] + (cs[1] == 1 ? 0 : j)];
        if (beta != 1.0) cv = (float)((double)cv * beta);
        y[i * n + j] = y[i * n + j] + cv;
      }
  }
  return ORC_OK;
}

/* ------------------------------------------------------------ MatMulNBits */

float orc_nbits_weight(int64_t col, int64_t kk, int64_t k, int64_t block_size,
                       const uint8_t *b, const float *scales, int zp_kind,
                       const void *zp) {
  const int64_t nb = (k + block_size - 1) / block_size;
  const int64_t blob = block_size / 2;
  const int64_t zp_stride = (nb + 1) / 2;
  const int64_t blk = kk / block_size;
  const uint8_t byte = b[(col * nb + blk) * blob + (kk % block_size) / 2];
  const int q = (kk & 1) == 0 ? (byte & 15) : (byte >> 4);
  double z = 8;
  if (zp_kind == 1) {
    const uint8_t zb = ((const uint8_t *)zp)[col * zp_stride + blk / 2];
    z = (double)((blk & 1) == 0 ? (zb & 15) : (zb >> 4));
  } else if (zp_kind == 2) {
    z = (double)((const float *)zp)[col * nb + blk];
  }
  /* (q - zp) in double times the f32 scale, one rounding to f32. */
  return (float)(((double)q - z) * (double)scales[col * nb + blk]);
}

int orc_matmul_nbits(const float *a, int64_t m, int64_t k, int64_t n,
                     int64_t bits, int64_t block_size, const uint8_t *b,
                     const float *scales, int zp_kind, const void *zp,
                     const float *bias, float *y) {
  if (bits != 4) return ORC_UNSUPPORTED;
  if (k <= 0 || n <= 0 || block_size < 16 ||
      (block_size & (block_size - 1)) != 0)
    return ORC_INVALID_ARGUMENT;
  if (m == 0) return ORC_OK;
  if (m == 1) {
    /* Token decode: f64 accumulation in k order, + bias, one f32 rounding
     * (onnx_qlinear_ops.dart:194-205). */
    for (int64_t col = 0; col < n; col++) {
      double sum = 0;
      for (int64_t kk = 0; kk < k; kk++)
        sum += (double)a[kk] *
               (double)orc_nbits_weight(col, kk, k, block_size, b, scales,
                                        zp_kind, zp);
      y[col] = (float)(sum + (bias ? (double)bias[col] : 0.0));
    }
    return ORC_OK;
  }
  /* Multi-row: 32-column dequantized tiles through matmulKernel, then + bias
   * (onnx_qlinear_ops.dart:208-226). */
  const int64_t tile_cols = 32;
  float *bt = (float *)malloc(sizeof(float) * (size_t)(k * tile_cols));
  float *tile = (float *)malloc(sizeof(float) * (size_t)(m * tile_cols));
  for (int64_t start = 0; start < n; start += tile_cols) {
    const int64_t cols = (n - start < tile_cols) ? n - start : tile_cols;
    for (int64_t col = 0; col < cols; col++)
      for (int64_t kk = 0; kk < k; kk++)
        bt[kk * cols + col] = orc_nbits_weight(start + col, kk, k, block_size,
                                               b, scales, zp_kind, zp);
    orc_matmul_kernel(a, bt, tile, m, k, cols);
    for (int64_t row = 0; row < m; row++)
      for (int64_t col = 0; col < cols; col++)
        y[row * n + start + col] =
            (float)((double)tile[row * cols + col] +
                    (bias ? (double)bias[start + col] : 0.0));
  }
  free(bt);
  free(tile);
  return ORC_OK;
}

/* ----------------------------------------------- MatMulInteger / QLinear */

static inline int32_t load_q(const void *p, int is_signed, int64_t i) {
  return is_signed ? (int32_t)((const int8_t *)p)[i]
                   : (int32_t)((const uint8_t *)p)[i];
}

int orc_matmul_integer(const void *a, int a_signed, int64_t a_batch,
                       const void *b, int b_signed, int64_t b_batch, int64_t m,
                       int64_t k, int64_t n, const int32_t *a_zp,
                       int64_t a_zp_len, const int32_t *b_zp, int64_t b_zp_len,
                       int64_t *y) {
  if ((a_zp && a_zp_len != 1 && a_zp_len != m) ||
      (b_zp && b_zp_len != 1 && b_zp_len != n))
    return ORC_UNSUPPORTED;
  const int64_t az = (a_zp == NULL || a_zp_len != 1) ? 0 : a_zp[0];
  const int32_t *az_row = (a_zp && a_zp_len == m && m != 1) ? a_zp : NULL;
  const int64_t bz = (b_zp == NULL || b_zp_len != 1) ? 0 : b_zp[0];
  const int32_t *bz_col = (b_zp && b_zp_len == n && n != 1) ? b_zp : NULL;
  const int64_t batch = a_batch > b_batch ? a_batch : b_batch;
  if ((a_batch != batch && a_batch != 1) || (b_batch != batch && b_batch != 1))
    return ORC_INVALID_ARGUMENT;
  memset(y, 0, sizeof(int64_t) * (size_t)(batch * m * n));
  for (int64_t bb = 0; bb < batch; bb++) {
    const int64_t a_off = (a_batch == 1 ? 0 : bb) * m * k;
    const int64_t b_off = (b_batch == 1 ? 0 : bb) * k * n;
    int64_t *o = y + bb * m * n;
    for (int64_t i = 0; i < m; i++) {
      const int64_t azi = az_row ? az_row[i] : az;
      for (int64_t kk = 0; kk < k; kk++) {
        const int64_t av = load_q(a, a_signed, a_off + i * k + kk) - azi;
        if (av == 0) continue; /* zero contributions skipped (:61-62) */
        for (int64_t j = 0; j < n; j++) {
          const int64_t bv = load_q(b, b_signed, b_off + kk * n + j) -
                             (bz_col ? bz_col[j] : bz);
          o[i * n + j] += av * bv;
        }
      }
    }
  }
  return ORC_OK;
}

int orc_qlinear_matmul(const void *a, int a_signed, int64_t a_batch,
                       const void *b, int b_signed, int64_t b_batch, int64_t m,
                       int64_t k, int64_t n, float a_scale,
                       const int32_t *a_zp, int64_t a_zp_len, float b_scale,
                       const int32_t *b_zp, int64_t b_zp_len, float y_scale,
                       int32_t y_zp, int32_t lo, int32_t hi, int64_t *y) {
  int st = orc_matmul_integer(a, a_signed, a_batch, b, b_signed, b_batch, m, k,
                              n, a_zp, a_zp_len, b_zp, b_zp_len, y);
  if (st) return st;
  /* mult = fl32(fl32(aS*bS) / yS): each step rounded to f32 (:95-98). */
  const float ab = (float)((double)a_scale * (double)b_scale);
  const float mult = (float)((double)ab / (double)y_scale);
  const int64_t total = (a_batch > b_batch ? a_batch : b_batch) * m * n;
  for (int64_t i = 0; i < total; i++) {
    const float p = (float)((double)y[i] * (double)mult);
    int err = 0;
    int64_t q = orc_round_even((double)p, &err) + y_zp;
    if (err) return err;
    y[i] = q < lo ? lo : (q > hi ? hi : q);
  }
  return ORC_OK;
}

/* ------------------------------------------------ DynamicQuantizeLinear */

int orc_dynamic_quantize_linear(const float *x, int64_t n, uint8_t *y,
                                float *scale_out, int32_t *zp_out) {
  double mn = 0, mx = 0; /* the range always spans 0 */
  for (int64_t i = 0; i < n; i++) {
    const double v = x[i];
    if (v < mn) mn = v;
    if (v > mx) mx = v;
  }
  const float scale_f = (float)((mx - mn) / 255.0);
  const double scale = scale_f;
  const float zpf = scale == 0 ? 0.0f : (float)(-mn / scale);
  double zc = zpf;
  if (zc < 0) zc = 0;
  if (zc > 255) zc = 255;
  int err = 0;
  const int64_t zp = orc_round_even(zc, &err);
  if (err) return err;
  for (int64_t i = 0; i < n; i++) {
    int64_t q;
    if (scale == 0) {
      q = zp;
    } else {
      const float r = (float)((double)x[i] / scale);
      q = orc_round_even((double)r, &err) + zp;
      if (err) return err;
    }
    y[i] = (uint8_t)(q < 0 ? 0 : (q > 255 ? 255 : q));
  }
  *scale_out = scale_f;
  *zp_out = (int32_t)zp;
  return ORC_OK;
}

/* ------------------------------------------------------------ attention */

/* Scale, mask and row softmax of one score row in place, as opFusedSDPA
 * (lib/src/onnx_ops.dart:2123-2141) and opMultiHeadAttention (:2072-2089) do
 * it: val = s * scale + mask in double, stored rounded to f32, the max over
 * the unrounded doubles; e = exp(stored - max) in double, stored rounded,
 * summed in double; then divide by the sum (div = 1) or multiply by its
 * inverse (div = 0). */
static void softmax_row(float *row, int64_t t, double scale, const float *mask,
                        int64_t mask_stride, int div) {
  double mx = -INFINITY;
  for (int64_t j = 0; j < t; j++) {
    const double val = (double)row[j] * scale + (mask ? (double)mask[j * mask_stride] : 0.0);
    row[j] = (float)val;
    if (val > mx) mx = val;
  }
  double sum = 0;
  for (int64_t j = 0; j < t; j++) {
    const double e = exp((double)row[j] - mx);
    row[j] = (float)e;
    sum += e;
  }
  if (div) {
    for (int64_t j = 0; j < t; j++) row[j] = (float)((double)row[j] / sum);
  } else {
    const double inv = 1.0 / sum;
    for (int64_t j = 0; j < t; j++) row[j] = (float)((double)row[j] * inv);
  }
}

int orc_fused_sdpa(const float *a, const int64_t *a_shape, int a_rank,
                   const float *b, const int64_t *b_shape, int b_rank,
                   const float *v, const int64_t *v_shape, int v_rank,
                   const float *mask, const int64_t *mask_shape, int mask_rank,
                   double scale, float *y) {
  if (a_rank < 2 || b_rank < 2 || v_rank < 2 || a_rank > 8 || b_rank > 8 || v_rank > 8 ||
      mask_rank > 8)
    return ORC_INVALID_ARGUMENT;
  /* s = opMatMul(a, b) (:2107). */
  int64_t sb[8];
  int sbr = 0;
  if (broadcast_shape(a_shape, a_rank - 2, b_shape, b_rank - 2, sb, &sbr))
    return ORC_INVALID_ARGUMENT;
  const int64_t m = a_shape[a_rank - 2], t = b_shape[b_rank - 1];
  int64_t srows = m;
  for (int d = 0; d < sbr; d++) srows *= sb[d];
  float *s = (float *)malloc((size_t)(srows * t > 0 ? srows * t : 1) * sizeof(float));
  if (!s) return ORC_INVALID_ARGUMENT;
  int st = orc_matmul_f32(a, a_shape, a_rank, b, b_shape, b_rank, s);
  if (st) {
    free(s);
    return st;
  }
  /* Row loop with the mask broadcast (:2113-2146). */
  int64_t sshape[8];
  for (int d = 0; d < sbr; d++) sshape[d] = sb[d];
  sshape[sbr] = m;
  sshape[sbr + 1] = t;
  const int srank = sbr + 2;
  const int64_t mlast_stride = (mask_rank > 0 && mask_shape[mask_rank - 1] == t) ? 1 : 0;
  const int mrow_rank = mask_rank > 0 ? mask_rank - 1 : 0;
  int64_t coords[8] = {0};
  for (int64_t r = 0; r < srows; r++) {
    int64_t rem = r;
    for (int d = srank - 2; d >= 0; d--) {
      coords[d] = rem % sshape[d];
      rem /= sshape[d];
    }
    const int64_t mbase =
        mask_rank == 0 ? 0
                       : flatten_broadcast(coords, srank - 1, mask_shape, mrow_rank) *
                             mask_shape[mask_rank - 1];
    softmax_row(s + r * t, t, scale, mask + mbase, mlast_stride, 1);
  }
  /* opMatMul(s, v) (:2148). */
  sshape[sbr] = m;
  st = orc_matmul_f32(s, sshape, srank, v, v_shape, v_rank, y);
  free(s);
  return st;
}

int orc_multi_head_attention(const float *q, const float *k, const float *v,
                             int64_t batch, int64_t seq, int64_t kv_seq,
                             int64_t hidden, int64_t num_heads, const float *bias,
                             int64_t bias_heads, int has_scale, double scale, float *out) {
  if (num_heads <= 0 || hidden % num_heads) return ORC_INVALID_ARGUMENT;
  const int64_t hs = hidden / num_heads;
  const double s = has_scale ? scale : 1.0 / sqrt((double)hs); /* :2030 */
  float *qh = (float *)malloc((size_t)(seq * hs + 1) * sizeof(float));
  float *kt = (float *)malloc((size_t)(hs * kv_seq + 1) * sizeof(float));
  float *vh = (float *)malloc((size_t)(kv_seq * hs + 1) * sizeof(float));
  float *sc = (float *)malloc((size_t)(seq * kv_seq + 1) * sizeof(float));
  float *cx = (float *)malloc((size_t)(seq * hs + 1) * sizeof(float));
  if (!qh || !kt || !vh || !sc || !cx) {
    free(qh); free(kt); free(vh); free(sc); free(cx);
    return ORC_INVALID_ARGUMENT;
  }
  for (int64_t b = 0; b < batch; b++) {
    for (int64_t h = 0; h < num_heads; h++) {
      /* Gather Q [seq, hs], K^T [hs, kv_seq], V [kv_seq, hs] (:2047-2061). */
      for (int64_t i = 0; i < seq; i++)
        for (int64_t d = 0; d < hs; d++)
          qh[i * hs + d] = q[(b * seq + i) * hidden + h * hs + d];
      for (int64_t j = 0; j < kv_seq; j++)
        for (int64_t d = 0; d < hs; d++) {
          kt[d * kv_seq + j] = k[(b * kv_seq + j) * hidden + h * hs + d];
          vh[j * hs + d] = v[(b * kv_seq + j) * hidden + h * hs + d];
        }
      orc_matmul_kernel(qh, kt, sc, seq, hs, kv_seq); /* :2063-2064 */
      const int64_t bbase = bias ? (b * bias_heads + (h % bias_heads)) * seq * kv_seq : 0;
      for (int64_t i = 0; i < seq; i++)
        softmax_row(sc + i * kv_seq, kv_seq, s, bias ? bias + bbase + i * kv_seq : NULL, 1, 0);
      orc_matmul_kernel(sc, vh, cx, seq, kv_seq, hs); /* :2090-2091 */
      for (int64_t i = 0; i < seq; i++)
        for (int64_t d = 0; d < hs; d++)
          out[(b * seq + i) * hidden + h * hs + d] = cx[i * hs + d];
    }
  }
  free(qh); free(kt); free(vh); free(sc); free(cx);
  return ORC_OK;
}

/* ------------------------------------------------------------ convolution */

static double conv_elem(const void *p, int kind, int64_t i) {
  if (kind == 1) return (double)((const uint8_t *)p)[i];
  if (kind == 2) return (double)((const int8_t *)p)[i];
  return (double)((const float *)p)[i];
}

int orc_conv(const void *x, int x_kind, const void *w, int w_kind, int64_t n, int64_t c,
             int64_t m, int64_t group, const int64_t *in, const int64_t *ker,
             const int64_t *out, const int64_t *str, const int64_t *dil,
             const int64_t *pad, int trans, int32_t x_zp, const int32_t *w_zp,
             double *acc) {
  if (group < 1 || c % group || m % group) return ORC_INVALID_ARGUMENT;
  const int64_t cg = c / group, mg = m / group;
  const int64_t in_sp = in[0] * in[1] * in[2], out_sp = out[0] * out[1] * out[2];
  const int64_t taps = ker[0] * ker[1] * ker[2];
  const double xz = x_kind ? (double)x_zp : 0.0;
  for (int64_t i = 0; i < n * m * out_sp; i++) acc[i] = 0.0;
  if (!trans) {
    /* Gather per output element (_convIntAcc order: c, ky, kx). */
    for (int64_t b = 0; b < n; b++)
      for (int64_t om = 0; om < m; om++) {
        const int64_t g = om / mg;
        const double wz = (w_kind && w_zp) ? (double)w_zp[om] : 0.0;
        for (int64_t oz = 0; oz < out[0]; oz++)
          for (int64_t oy = 0; oy < out[1]; oy++)
            for (int64_t ox = 0; ox < out[2]; ox++) {
              double s = 0.0;
              for (int64_t cc = 0; cc < cg; cc++) {
                const int64_t xb = (b * c + g * cg + cc) * in_sp;
                const int64_t wb = (om * cg + cc) * taps;
                for (int64_t kz = 0; kz < ker[0]; kz++) {
                  const int64_t iz = oz * str[0] - pad[0] + kz * dil[0];
                  if (iz < 0 || iz >= in[0]) continue;
                  for (int64_t ky = 0; ky < ker[1]; ky++) {
                    const int64_t iy = oy * str[1] - pad[1] + ky * dil[1];
                    if (iy < 0 || iy >= in[1]) continue;
                    for (int64_t kx = 0; kx < ker[2]; kx++) {
                      const int64_t ix = ox * str[2] - pad[2] + kx * dil[2];
                      if (ix < 0 || ix >= in[2]) continue;
                      const double xv = conv_elem(x, x_kind, xb + (iz * in[1] + iy) * in[2] + ix) - xz;
                      const double wv = conv_elem(w, w_kind, wb + (kz * ker[1] + ky) * ker[2] + kx) - wz;
                      s += xv * wv;
                    }
                  }
                }
              }
              acc[((b * m + om) * out[0] + oz) * out[1] * out[2] + oy * out[2] + ox] = s;
            }
      }
    return ORC_OK;
  }
  /* Scatter per input element (opConvTranspose's generic path). */
  for (int64_t b = 0; b < n; b++)
    for (int64_t ci = 0; ci < c; ci++) {
      const int64_t g = ci / cg;
      for (int64_t iz = 0; iz < in[0]; iz++)
        for (int64_t iy = 0; iy < in[1]; iy++)
          for (int64_t ix = 0; ix < in[2]; ix++) {
            const double v = conv_elem(x, x_kind, ((b * c + ci) * in[0] + iz) * in[1] * in[2] +
                                                      iy * in[2] + ix) - xz;
            for (int64_t kz = 0; kz < ker[0]; kz++) {
              const int64_t oz = iz * str[0] + kz * dil[0] - pad[0];
              if (oz < 0 || oz >= out[0]) continue;
              for (int64_t ky = 0; ky < ker[1]; ky++) {
                const int64_t oy = iy * str[1] + ky * dil[1] - pad[1];
                if (oy < 0 || oy >= out[1]) continue;
                for (int64_t kx = 0; kx < ker[2]; kx++) {
                  const int64_t ox = ix * str[2] + kx * dil[2] - pad[2];
                  if (ox < 0 || ox >= out[2]) continue;
                  const int64_t r = (kz * ker[1] + ky) * ker[2] + kx;
                  for (int64_t mm = 0; mm < mg; mm++) {
                    const double wv = conv_elem(w, w_kind, (ci * mg + mm) * taps + r);
                    acc[((b * m + g * mg + mm) * out[0] + oz) * out[1] * out[2] + oy * out[2] +
                        ox] += v * wv;
                  }
                }
              }
            }
          }
    }
  return ORC_OK;
}

/* ------------------------------------------------------ GroupQueryAttention */

void orc_rotary_embedding(const float *x, int64_t batch, int64_t seq, int64_t heads,
                          int64_t hs, const int64_t *pos, const float *cos_cache,
                          const float *sin_cache, int64_t half_rot, int interleaved,
                          float *out) {
  const int64_t rot = 2 * half_rot;
  for (int64_t b = 0; b < batch; b++)
    for (int64_t s = 0; s < seq; s++) {
      const int64_t cb = pos[s] * half_rot;
      for (int64_t h = 0; h < heads; h++) {
        const int64_t base = (b * seq + s) * heads * hs + h * hs;
        if (interleaved) {
          for (int64_t i = 0; i < rot / 2; i++) {
            const double c = cos_cache[cb + i], sn = sin_cache[cb + i];
            const double x0 = x[base + 2 * i], x1 = x[base + 2 * i + 1];
            out[base + 2 * i] = (float)(x0 * c - x1 * sn);
            out[base + 2 * i + 1] = (float)(x1 * c + x0 * sn);
          }
        } else {
          const int64_t half = rot / 2;
          for (int64_t i = 0; i < half; i++) {
            const double c = cos_cache[cb + i], sn = sin_cache[cb + i];
            const double x0 = x[base + i], x1 = x[base + i + half];
            out[base + i] = (float)(x0 * c - x1 * sn);
            out[base + i + half] = (float)(x1 * c + x0 * sn);
          }
        }
        for (int64_t i = rot; i < hs; i++) out[base + i] = x[base + i];
      }
    }
}

int orc_group_query_attention(const float *q, const float *k, const float *v, int64_t batch,
                              int64_t seq, int64_t hidden, int64_t heads, int64_t kv_heads,
                              const float *past_k, const float *past_v, int64_t past_len,
                              const float *cos_cache, const float *sin_cache, int64_t half_rot,
                              int do_rotary, int interleaved, const float *bias,
                              int64_t bias_heads, int has_scale, double scale, float *out,
                              float *present_k, float *present_v) {
  if (heads <= 0 || kv_heads <= 0 || heads % kv_heads || hidden % heads)
    return ORC_INVALID_ARGUMENT;
  const int64_t hs = hidden / heads, group = heads / kv_heads, kvh_n = kv_heads * hs;
  const int64_t total = past_len + seq;
  float *qq = (float *)malloc((size_t)(batch * seq * hidden + 1) * sizeof(float));
  float *kk = (float *)malloc((size_t)(batch * seq * kvh_n + 1) * sizeof(float));
  int64_t *pos = (int64_t *)malloc((size_t)(seq + 1) * sizeof(int64_t));
  float *qh = (float *)malloc((size_t)(seq * hs + 1) * sizeof(float));
  float *kt = (float *)malloc((size_t)(hs * total + 1) * sizeof(float));
  float *sc = (float *)malloc((size_t)(seq * total + 1) * sizeof(float));
  float *cx = (float *)malloc((size_t)(seq * hs + 1) * sizeof(float));
  if (!qq || !kk || !pos || !qh || !kt || !sc || !cx) {
    free(qq); free(kk); free(pos); free(qh); free(kt); free(sc); free(cx);
    return ORC_INVALID_ARGUMENT;
  }
  memcpy(qq, q, sizeof(float) * (size_t)(batch * seq * hidden));
  memcpy(kk, k, sizeof(float) * (size_t)(batch * seq * kvh_n));
  if (do_rotary) { /* :1876-1896 */
    for (int64_t s = 0; s < seq; s++) pos[s] = past_len + s;
    orc_rotary_embedding(q, batch, seq, heads, hs, pos, cos_cache, sin_cache, half_rot,
                         interleaved, qq);
    orc_rotary_embedding(k, batch, seq, kv_heads, hs, pos, cos_cache, sin_cache, half_rot,
                         interleaved, kk);
  }
  const double s = has_scale ? scale : 1.0 / sqrt((double)hs);
  /* present K / V (:1907-1931) */
  for (int64_t b = 0; b < batch; b++)
    for (int64_t kvh = 0; kvh < kv_heads; kvh++) {
      const int64_t base = (b * kv_heads + kvh) * total * hs;
      for (int64_t j = 0; j < past_len; j++)
        for (int64_t d = 0; d < hs; d++) {
          const int64_t src = ((b * kv_heads + kvh) * past_len + j) * hs + d;
          present_k[base + j * hs + d] = past_k[src];
          present_v[base + j * hs + d] = past_v[src];
        }
      for (int64_t j = 0; j < seq; j++)
        for (int64_t d = 0; d < hs; d++) {
          const int64_t src = (b * seq + j) * kvh_n + kvh * hs + d;
          present_k[base + (past_len + j) * hs + d] = kk[src];
          present_v[base + (past_len + j) * hs + d] = v[src];
        }
    }
  for (int64_t b = 0; b < batch; b++)
    for (int64_t h = 0; h < heads; h++) {
      const int64_t kvh = h / group;
      const int64_t base = (b * kv_heads + kvh) * total * hs;
      for (int64_t i = 0; i < seq; i++)
        for (int64_t d = 0; d < hs; d++)
          qh[i * hs + d] = qq[(b * seq + i) * hidden + h * hs + d];
      for (int64_t j = 0; j < total; j++)
        for (int64_t d = 0; d < hs; d++) kt[d * total + j] = present_k[base + j * hs + d];
      orc_matmul_kernel(qh, kt, sc, seq, hs, total); /* :1952 */
      const int64_t bb = bias ? (b * bias_heads + (h % bias_heads)) * seq * total : 0;
      for (int64_t i = 0; i < seq; i++) { /* :1956-1981 */
        float *row = sc + i * total;
        const int64_t last = past_len + i;
        softmax_row(row, last + 1, s, bias ? bias + bb + i * total : NULL, 1, 0);
        for (int64_t j = last + 1; j < total; j++) row[j] = 0.f;
      }
      orc_matmul_kernel(sc, present_v + base, cx, seq, total, hs); /* :1985-1995 */
      for (int64_t i = 0; i < seq; i++)
        for (int64_t d = 0; d < hs; d++)
          out[(b * seq + i) * hidden + h * hs + d] = cx[i * hs + d];
    }
  free(qq); free(kk); free(pos); free(qh); free(kt); free(sc); free(cx);
  return ORC_OK;
}

/* ------------------------------------------------- elementwise (decoder) */

int orc_binary_f32(int op, const float *a, const int64_t *a_shape, int a_rank, const float *b,
                   const int64_t *b_shape, int b_rank, float *y, int64_t *out_shape) {
  enum { R = 16 };
  const int rank = a_rank > b_rank ? a_rank : b_rank;
  if (op < 0 || op > 3 || rank > R || a_rank < 0 || b_rank < 0) return ORC_INVALID_ARGUMENT;
  int64_t ad[R], bd[R], od[R];
  for (int k = 0; k < rank; k++) {
    const int ka = k - (rank - a_rank), kb = k - (rank - b_rank);
    ad[k] = ka >= 0 ? a_shape[ka] : 1;
    bd[k] = kb >= 0 ? b_shape[kb] : 1;
    if (ad[k] == bd[k]) od[k] = ad[k];
    else if (ad[k] == 1) od[k] = bd[k];
    else if (bd[k] == 1) od[k] = ad[k];
    else return ORC_INVALID_ARGUMENT;  /* "Cannot broadcast shapes" */
    out_shape[k] = od[k];
  }
  int64_t n = 1;
  for (int k = 0; k < rank; k++) n *= od[k];
  for (int64_t i = 0; i < n; i++) {
    /* coordinates of output element i, then the operands' row-major offsets */
    int64_t rem = i, ia = 0, ib = 0, sa = 1, sb = 1;
    for (int k = rank - 1; k >= 0; k--) {
      const int64_t c = rem % od[k];
      rem /= od[k];
      ia += (ad[k] == 1 ? 0 : c) * sa;
      ib += (bd[k] == 1 ? 0 : c) * sb;
      sa *= ad[k];
      sb *= bd[k];
    }
    const double x = a[ia], v = b[ib];
    double r;
    switch (op) {
      case 0: r = x + v; break;
      case 1: r = x - v; break;
      case 2: r = x * v; break;
      default: r = x / v; break;
    }
    y[i] = (float)r;
  }
  return ORC_OK;
}

void orc_sigmoid_f32(const float *x, int64_t n, float *y) {
  for (int64_t i = 0; i < n; i++) y[i] = (float)(1.0 / (1.0 + exp(-(double)x[i])));
}

int orc_rms_norm_f32(const float *x, const int64_t *shape, int rank, const float *gamma,
                     int64_t gamma_len, int64_t axis, double eps, float *y) {
  if (rank < 1) return ORC_INVALID_ARGUMENT;
  const int64_t ax = axis < 0 ? axis + rank : axis;
  if (ax < 0 || ax >= rank) return ORC_INVALID_ARGUMENT;
  const int64_t last = shape[rank - 1];
  if (gamma_len != last) return ORC_INVALID_ARGUMENT;  /* "RMSNorm gamma length" */
  int64_t outer = 1, inner = 1;
  for (int64_t k = 0; k < ax; k++) outer *= shape[k];
  for (int64_t k = ax + 1; k < rank; k++) inner *= shape[k];
  const int64_t dim = shape[ax];
  for (int64_t o = 0; o < outer; o++)
    for (int64_t i = 0; i < inner; i++) {
      const int64_t base = o * dim * inner + i;
      double ss = 0;
      for (int64_t j = 0; j < dim; j++) {
        const double v = x[base + j * inner];
        ss += v * v;
      }
      const double inv = 1.0 / sqrt(ss / (double)dim + eps);
      for (int64_t j = 0; j < dim; j++) {
        const int64_t idx = base + j * inner;
        y[idx] = (float)((double)x[idx] * inv * (double)gamma[idx % last]);
      }
    }
  return ORC_OK;
}
