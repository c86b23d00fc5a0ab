/*
 * oracle.c - CPU restatement of the FanarVSE search paths (throughput int8 engine and the trellis
 * latency engine) -- TEST INFRASTRUCTURE.
 *
 * This file is the checker, not the product: only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load it. Each function restates one reference function (cited
 * file:line under /root/reference) with the same canonical floating-point operation order as the
 * gfx950 kernels (include/fvs.h), so identical inputs give bit-identical outputs. Loops run over
 * queries with OpenMP; inside a query everything is sequential.
 *
 * Build: oracle/Makefile (gcc -O3 -march=x86-64-v3 -ffp-contract=off -fopenmp).
 */
#include <immintrin.h>
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define OR_MAXT 8

static inline float h2f(uint16_t h) { return _cvtsh_ss(h); }
static inline uint16_t f2h(float f) { return (uint16_t)_cvtss_sh(f, _MM_FROUND_TO_NEAREST_INT); }

/* ---------------------------------------------------------------- query code (a6)
 * throughput/enginei8.py:38  z = Qb @ Vr; qs = z.abs().amax(1).clamp(min=1e-12) / 127;
 *                            q8 = round(z / qs).clamp(-127, 127)   (R <= 1024)
 * throughput/enginei8.py:62  QC = Qb @ c
 */
static void project_row(const float *x, int d, const float *Vr, int R, float *z) {
  for (int j = 0; j < R; j++) z[j] = 0.f;
  for (int k = 0; k < d; k++) {
    const float xk = x[k];
    const float *v = Vr + (int64_t)k * R;
    for (int j = 0; j < R; j++) z[j] = fmaf(xk, v[j], z[j]);
  }
}

static void quant_row(const float *z, int R, int8_t *out8, float *outs) {
  float amax = 0.f;
  for (int j = 0; j < R; j++) amax = fmaxf(amax, fabsf(z[j]));
  const float a = fmaxf(amax, 1e-12f) / 127.0f;
  for (int j = 0; j < R; j++) {
    float q = rintf(z[j] / a);
    q = fminf(fmaxf(q, -127.0f), 127.0f);
    out8[j] = (int8_t)(int)q;
  }
  *outs = a;
}

/* 64 lane partial sums combined by the xor butterfly of a wave: lane[l] += lane[l ^ o], o = 32..1. */
static double butterfly64_d(double *lane) {
  for (int o = 32; o > 0; o >>= 1) {
    double t[64];
    for (int l = 0; l < 64; l++) t[l] = lane[l] + lane[l ^ o];
    memcpy(lane, t, sizeof(t));
  }
  return lane[0];
}

/* z = Q @ Vr with one sequential fmaf chain per output: the order of fvs_query_code's projection (the GPU's
 * query path) and of fvs_build_codes' residual projection, so the parity tests compare z bit for bit. */
void or_project(const float *Q, int64_t B, int d, const float *Vr, int R, float *z) {
#pragma omp parallel for schedule(static)
  for (int64_t q = 0; q < B; q++) project_row(Q + q * d, d, Vr, R, z + q * R);
}

void or_query_prep(const float *Q, int64_t B, int d, const float *z, int R, const float *c, int8_t *q8, float *qs,
                   float *qc, uint16_t *qh) {
#pragma omp parallel for schedule(static)
  for (int64_t q = 0; q < B; q++) {
    const float *x = Q + q * d;
    quant_row(z + q * R, R, q8 + q * R, qs + q);
    double lane[64];
    for (int l = 0; l < 64; l++) lane[l] = 0.0;
    for (int k = 0; k < d; k++) lane[k % 64] += (double)x[k] * (double)c[k];
    qc[q] = (float)butterfly64_d(lane);
    for (int k = 0; k < d; k++) qh[q * d + k] = f2h(x[k]);
  }
}

/* ---------------------------------------------------------------- base codes (a3)
 * throughput/enginei8.py:19-27  z = (x - means16[cell]) @ Vr, then as the query code.
 */
void or_build_codes(const uint16_t *X16, const int32_t *order, const int32_t *cell, int64_t N, int d,
                    const uint16_t *means16, const float *Vr, int R, int8_t *Z, float *zs) {
#pragma omp parallel for schedule(static)
  for (int64_t n = 0; n < N; n++) {
    float x[8192];
    const uint16_t *xr = X16 + (int64_t)order[n] * d;
    const uint16_t *mr = means16 + (int64_t)cell[n] * d;
    float z[1024];
    for (int k = 0; k < d; k++) x[k] = h2f(xr[k]) - h2f(mr[k]);
    project_row(x, d, Vr, R, z);
    quant_row(z, R, Z + n * R, zs + n);
  }
}

/* ---------------------------------------------------------------- fp16 products (CPU baseline only)
 * The reference computes QM = Qb.half() @ meansN.T (throughput/enginei8.py:67) and
 * Zq = Qb.half() @ VP16[:, :D] (throughput/s2lut.py:122) with a BLAS fp16 GEMM; here each output
 * is a sequential fmaf over k, rounded once to fp16.
 *   or_fp16_gemm_nt: out[m][n] = A[m,:] . Bt[n,:]      or_fp16_gemm_nn: out[m][n] = A[m,:] . Bm[:,n]
 */
void or_fp16_gemm_nt(const uint16_t *A, const uint16_t *Bt, int64_t M, int64_t Nn, int K, uint16_t *out) {
#pragma omp parallel for schedule(dynamic, 4)
  for (int64_t m = 0; m < M; m++) {
    float a[8192];
    for (int k = 0; k < K; k++) a[k] = h2f(A[m * K + k]);
    for (int64_t n = 0; n < Nn; n++) {
      const uint16_t *b = Bt + n * K;
      float acc = 0.f;
      for (int k = 0; k < K; k++) acc = fmaf(a[k], h2f(b[k]), acc);
      out[m * Nn + n] = f2h(acc);
    }
  }
}

void or_fp16_gemm_nn(const uint16_t *A, const uint16_t *Bm, int64_t M, int64_t Nn, int K, int ldb, uint16_t *out) {
#pragma omp parallel for schedule(dynamic, 4)
  for (int64_t m = 0; m < M; m++) {
    float acc[8192];
    for (int64_t n = 0; n < Nn; n++) acc[n] = 0.f;
    for (int k = 0; k < K; k++) {
      const float a = h2f(A[m * K + k]);
      const uint16_t *b = Bm + (int64_t)k * ldb;
      for (int64_t n = 0; n < Nn; n++) acc[n] = fmaf(a, h2f(b[n]), acc[n]);
    }
    for (int64_t n = 0; n < Nn; n++) out[m * Nn + n] = f2h(acc[n]);
  }
}

/* ---------------------------------------------------------------- ordering helpers */
static inline uint32_t ord32(float x) {
  uint32_t u;
  memcpy(&u, &x, 4);
  if (u == 0x80000000u) u = 0u;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
static inline uint32_t ord16(uint16_t u) {
  if (u == 0x8000u) u = 0u;
  return (u & 0x8000u) ? (uint32_t)((~u) & 0xffffu) : (uint32_t)(u | 0x8000u);
}
static int cmp_u64_desc(const void *a, const void *b) {
  const uint64_t x = *(const uint64_t *)a, y = *(const uint64_t *)b;
  return x < y ? 1 : (x > y ? -1 : 0);
}
static int cmp_u32_desc(const void *a, const void *b) {
  const uint32_t x = *(const uint32_t *)a, y = *(const uint32_t *)b;
  return x < y ? 1 : (x > y ? -1 : 0);
}

/* ---------------------------------------------------------------- routing (a7)
 * throughput/enginei8.py:67-68  probe = QM.topk(nprobe, 1).indices (sorted); ties: lower cell first.
 */
void or_route_topk(const uint16_t *QM, int64_t B, int NC, int np, int32_t *probe) {
#pragma omp parallel for schedule(static)
  for (int64_t q = 0; q < B; q++) {
    uint64_t *keys = (uint64_t *)malloc(sizeof(uint64_t) * NC);
    for (int c = 0; c < NC; c++) keys[c] = ((uint64_t)ord16(QM[q * NC + c]) << 16) | (uint64_t)(0xffffu - (uint32_t)c);
    qsort(keys, NC, sizeof(uint64_t), cmp_u64_desc);
    for (int i = 0; i < np; i++) probe[q * np + i] = (int32_t)(0xffffu - (uint32_t)(keys[i] & 0xffffu));
    free(keys);
  }
}

/* ---------------------------------------------------------------- int8 stage-1 estimate
 * throughput/ivf8c_kern.py:14,30  est = f32(q8 . Z) * qs * zs + qcp, with the last multiply-add fused.
 */
static inline float est_i8(const int8_t *qv, float qsv, const int8_t *zv, float zsv, float qcp, int R) {
  int32_t acc = 0;
  for (int j = 0; j < R; j++) acc += (int32_t)qv[j] * (int32_t)zv[j];
  const float t = (float)acc * qsv;
  return fmaf(t, zsv, qcp);
}
static inline int cell_blocks(const int32_t *off, int c) {
  const int s = off[c], e = off[c + 1];
  return e > s ? (e - 1) / 32 - s / 32 + 1 : 0;
}
static const float *g_qadd = NULL; /* per-query additive pair term of the projected-means variant */
static inline float pair_const(const uint16_t *QM, int64_t q, int NC, int c, const float *mnorm) {
  const float v = h2f(QM[q * NC + c]) * (mnorm ? mnorm[c] : 1.0f);  /* throughput/enginei8.py:14-15 */
  return g_qadd ? v + g_qadd[q] : v;  /* host_resident/space_x.py:33-36 */
}

/* First pass (a9), throughput/ivf8c_kern.py:2-16: block maxima over the first n1 probed cells.
 * bm[q][j][b] for b < blocks(cell); other entries are not written. */
/* An estimator of est(q, row) for one (query, cell) pair constant qcp. */
typedef float (*est_fn)(const void *ctx, int64_t q, int64_t row, float qcp);

typedef struct {
  const int8_t *q8;
  const float *qs;
  const int8_t *Z;
  const float *zs;
  int R;
} i8_ctx;

static float est_i8_cb(const void *ctx, int64_t q, int64_t r, float qcp) {
  const i8_ctx *c = (const i8_ctx *)ctx;
  return est_i8(c->q8 + q * c->R, c->qs[q], c->Z + r * c->R, c->zs[r], qcp, c->R);
}

/* First pass over the first n1 probed cells: maxima per (query, probe rank, block of the cell). */
static void first_pass_gen(est_fn f, const void *ctx, const int32_t *probe, int npr, int n1, const int32_t *off,
                           const uint16_t *QM, int NC, const float *mnorm, int64_t B, int MB, float *bm) {
#pragma omp parallel for schedule(dynamic, 1)
  for (int64_t q = 0; q < B; q++) {
    for (int j = 0; j < n1; j++) {
      const int c = probe[q * npr + j];
      const int cs = off[c], ce = off[c + 1];
      const float qcp = pair_const(QM, q, NC, c, mnorm);
      const int nb = cell_blocks(off, c);
      for (int b = 0; b < nb; b++) {
        const int blk = cs / 32 + b;
        float m = -1e30f;
        for (int r = blk * 32; r < blk * 32 + 32; r++) {
          if (r < cs || r >= ce) continue;
          m = fmaxf(m, f(ctx, q, r, qcp));
        }
        bm[((int64_t)q * n1 + j) * MB + b] = m;
      }
    }
  }
}

/* Emit: every probed row with est >= t0, kept in canonical order (est desc, row asc), first M stored. */
static void emit_gen(est_fn f, const void *ctx, const int32_t *probe, int npr, int np, const int32_t *off,
                     const uint16_t *QM, int NC, const float *mnorm, const float *t0, int64_t B, int M, int32_t *cnt,
                     float *bval, int32_t *bpos) {
#pragma omp parallel for schedule(dynamic, 1)
  for (int64_t q = 0; q < B; q++) {
    size_t cap = 1024, n = 0;
    uint64_t *keys = (uint64_t *)malloc(sizeof(uint64_t) * cap);
    const float th = t0[q];
    for (int j = 0; j < np; j++) {
      const int c = probe[q * npr + j];
      const float qcp = pair_const(QM, q, NC, c, mnorm);
      for (int r = off[c]; r < off[c + 1]; r++) {
        const float e = f(ctx, q, r, qcp);
        if (e >= th) {
          if (n == cap) {
            cap *= 2;
            keys = (uint64_t *)realloc(keys, sizeof(uint64_t) * cap);
          }
          keys[n++] = ((uint64_t)ord32(e) << 32) | (uint64_t)(0xffffffffu - (uint32_t)r);
        }
      }
    }
    qsort(keys, n, sizeof(uint64_t), cmp_u64_desc);
    cnt[q] = (int32_t)n;
    for (size_t i = 0; i < (size_t)M; i++) {
      if (i < n) {
        const uint32_t k = (uint32_t)(keys[i] >> 32);
        const uint32_t u = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
        memcpy(&bval[q * M + i], &u, 4);
        bpos[q * M + i] = (int32_t)(0xffffffffu - (uint32_t)(keys[i] & 0xffffffffu));
      } else {
        bval[q * M + i] = -1e30f;
        bpos[q * M + i] = 0;
      }
    }
    free(keys);
  }
}

void or_first_pass(const int8_t *q8, const float *qs, const int32_t *probe, int npr, int n1, const int32_t *off,
                   const int8_t *Z, const float *zs, int R, const uint16_t *QM, int NC, const float *mnorm, int64_t B,
                   int MB, float *bm) {
  const i8_ctx ctx = {q8, qs, Z, zs, R};
  first_pass_gen(est_i8_cb, &ctx, probe, npr, n1, off, QM, NC, mnorm, B, MB, bm);
}

/* A probe id outside [0, NC) is no cell (this build's guard, not a reference rule): it reads no offsets and
 * the query's t0 becomes 1e30, so its emit keeps nothing and its exactness flag is cleared. */
void or_threshold(const float *bm, const int32_t *probe, int npr, const int32_t *off, int NC, int64_t B, int n1,
                  int MB, int r, float *t0) {
#pragma omp parallel for schedule(static)
  for (int64_t q = 0; q < B; q++) {
    uint32_t *v = (uint32_t *)malloc(sizeof(uint32_t) * (size_t)n1 * MB);
    int nv = 0, bad = 0;
    for (int j = 0; j < n1; j++) {
      const int c = probe[q * npr + j];
      if (c < 0 || c >= NC) {
        bad = 1;
        continue;
      }
      const int nb = cell_blocks(off, c);
      for (int b = 0; b < nb; b++) v[nv++] = ord32(bm[((int64_t)q * n1 + j) * MB + b]);
    }
    int kk = r < n1 * MB ? r : n1 * MB;
    if (kk > nv) kk = nv;
    if (bad) kk = 0;
    if (kk == 0) {
      t0[q] = 1e30f;
    } else {
      qsort(v, nv, sizeof(uint32_t), cmp_u32_desc);
      const uint32_t k = v[kk - 1];
      const uint32_t u = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
      memcpy(&t0[q], &u, 4);
    }
    free(v);
  }
}

/* Emit (a11), throughput/ivf8c_kern.py:18-36: every probed row with est >= t0. The oracle keeps the
 * list in canonical order (est descending, row ascending), truncated to M; cnt is the full count. */
void or_emit(const int8_t *q8, const float *qs, const int32_t *probe, int npr, int np, const int32_t *off,
             const int8_t *Z, const float *zs, int R, const uint16_t *QM, int NC, const float *mnorm, const float *t0,
             int64_t B, int M, int32_t *cnt, float *bval, int32_t *bpos) {
  const i8_ctx ctx = {q8, qs, Z, zs, R};
  emit_gen(est_i8_cb, &ctx, probe, npr, np, off, QM, NC, mnorm, t0, B, M, cnt, bval, bpos);
}

/* Selection (a12) and the delta rule (a14), throughput/enginei8.py:60 (t = bval.topk(K); pos = bpos[t];
 * ok = K <= cnt <= M) and :87-88 (ncnt), with ties in est broken by the smaller position. */
void or_select(const float *bval, const int32_t *bpos, const int32_t *cnt, int64_t B, int M, int K, int kd, float delta,
               int32_t *pos, float *est1, uint8_t *ok, int32_t *ncnt) {
#pragma omp parallel for schedule(static)
  for (int64_t q = 0; q < B; q++) {
    const int n = cnt[q] < M ? cnt[q] : M;
    /* top-K of the first n entries in the canonical order (est descending, pos ascending) */
    uint64_t *keys = (uint64_t *)malloc(sizeof(uint64_t) * (n > 0 ? n : 1));
    for (int i = 0; i < n; i++)
      keys[i] = ((uint64_t)ord32(bval[q * M + i]) << 32) | (uint64_t)(0xffffffffu - (uint32_t)bpos[q * M + i]);
    qsort(keys, (size_t)n, sizeof(uint64_t), cmp_u64_desc);
    for (int i = 0; i < K; i++) {
      if (i < n) {
        const uint32_t k = (uint32_t)(keys[i] >> 32);
        const uint32_t u = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
        memcpy(&est1[q * K + i], &u, 4);
        pos[q * K + i] = (int32_t)(0xffffffffu - (uint32_t)(keys[i] & 0xffffffffu));
      } else {
        est1[q * K + i] = -1e30f;
        pos[q * K + i] = 0;
      }
    }
    free(keys);
    ok[q] = (uint8_t)(cnt[q] >= K && cnt[q] <= M);
    if (delta >= 0.f) {
      const float thr = est1[q * K + kd] - delta;
      int c = 0;
      for (int i = 0; i < K; i++) c += est1[q * K + i] >= thr;
      ncnt[q] = c;
    } else {
      ncnt[q] = K;
    }
  }
}

/* ---------------------------------------------------------------- routing-free dense scan
 * throughput/brute.py:46-47, :51-52   codes: a = max(max|z|, 1e-12) / 127, clamp(rint(z / a), -127, 127)
 * throughput/brute.py:16-17           est = (float)acc * qs[q] * (float)zs[n], two products left to right
 * throughput/brute.py:31-37           emit every (q, n) with est >= t0[q]
 * The emitted list is kept in canonical order (est descending, n ascending), truncated to M; cnt is the
 * full count. */
void or_quantize_rows(const float *z, int64_t n, int R, int8_t *q, float *scale) {
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < n; r++) quant_row(z + r * R, R, q + r * R, scale + r);
}

static inline int32_t dot_i8(const int8_t *a, const int8_t *b, int R) {
  int32_t acc = 0;
  for (int j = 0; j < R; j++) acc += (int32_t)a[j] * (int32_t)b[j];
  return acc;
}

static inline float dense_est(const int8_t *q, float qsv, const int8_t *z, uint16_t zsv, int R) {
  return ((float)dot_i8(q, z, R) * qsv) * h2f(zsv);
}

void or_dense_scores(const int8_t *Q, const float *qs, int64_t B, const int8_t *Z, const uint16_t *zs, int64_t N, int R,
                     float *out) {
#pragma omp parallel for schedule(static)
  for (int64_t q = 0; q < B; q++)
    for (int64_t n = 0; n < N; n++) out[q * N + n] = dense_est(Q + q * R, qs[q], Z + n * R, zs[n], R);
}

void or_dense_emit(const int8_t *Q, const float *qs, int64_t B, const int8_t *Z, const uint16_t *zs, int64_t N, int R,
                   const float *t0, int M, int32_t *cnt, float *bval, int32_t *bpos) {
#pragma omp parallel for schedule(dynamic, 1)
  for (int64_t q = 0; q < B; q++) {
    int cap = 1024, c = 0;
    uint64_t *keys = (uint64_t *)malloc(sizeof(uint64_t) * cap);
    for (int64_t n = 0; n < N; n++) {
      const float e = dense_est(Q + q * R, qs[q], Z + n * R, zs[n], R);
      if (e >= t0[q]) {
        if (c == cap) {
          cap *= 2;
          keys = (uint64_t *)realloc(keys, sizeof(uint64_t) * cap);
        }
        keys[c++] = ((uint64_t)ord32(e) << 32) | (uint64_t)(0xffffffffu - (uint32_t)n);
      }
    }
    qsort(keys, (size_t)c, sizeof(uint64_t), cmp_u64_desc);
    cnt[q] = c;
    for (int i = 0; i < M; i++) {
      if (i < c) {
        const uint32_t k = (uint32_t)(keys[i] >> 32);
        const uint32_t u = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
        memcpy(&bval[q * M + i], &u, 4);
        bpos[q * M + i] = (int32_t)(0xffffffffu - (uint32_t)(keys[i] & 0xffffffffu));
      } else {
        bval[q * M + i] = -1e30f;
        bpos[q * M + i] = 0;
      }
    }
    free(keys);
  }
}

/* ---------------------------------------------------------------- LUT build (a13)
 * throughput/s2lut.py:108-126  L[q, n*16+v] = sum_i Zq[q,4n+i] * bit_i(v), bit_i(v) = (v >> (3-i)) & 1;
 * qsum/qn2 per tier (throughput/s2lut.py:125). tiers: T x (start, end, bits). */
void or_lut_build(const uint16_t *Zq, int64_t B, int D, int T, const int32_t *tiers, int half, void *Lout, float *qsum,
                  float *qn2) {
  const int nn = D / 4;
  const int64_t LW = (int64_t)nn * 16;
#pragma omp parallel for schedule(static)
  for (int64_t q = 0; q < B; q++) {
    const uint16_t *zr = Zq + q * D;
    for (int n = 0; n < nn; n++) {
      float z[4];
      for (int i = 0; i < 4; i++) z[i] = h2f(zr[4 * n + i]);
      for (int v = 0; v < 16; v++) {
        float acc = 0.f;
        for (int i = 0; i < 4; i++) acc = fmaf(z[i], (float)((v >> (3 - i)) & 1), acc);
        if (half)
          ((uint16_t *)Lout)[q * LW + n * 16 + v] = f2h(acc);
        else
          ((float *)Lout)[q * LW + n * 16 + v] = acc;
      }
    }
    for (int t = 0; t < T; t++) {
      double l1[64], l2[64];
      for (int l = 0; l < 64; l++) l1[l] = l2[l] = 0.0;
      for (int i = tiers[3 * t]; i < tiers[3 * t + 1]; i++) {
        const double x = (double)h2f(zr[i]);
        const int l = (i - tiers[3 * t]) % 64;
        l1[l] += x;
        l2[l] += x * x;
      }
      qsum[(int64_t)t * B + q] = (float)butterfly64_d(l1);
      qn2[(int64_t)t * B + q] = (float)butterfly64_d(l2);
    }
  }
}

/* ---------------------------------------------------------------- LUT stage 2 (a15)
 * throughput/s2lut.py:48-106 over the packed records of src/tiered_fused.py:112-125:
 *   est = QC + sum_t scale_t * delta_t * (sum_p 2^(b-1-p) <q_t, plane_p> - mid_t * qsum_t)
 *   var = sum_t qn2_t * sig_t^2; slots m >= ncnt -> (-1e30, 0).
 * Plane sums are exact integers over the fixed-point table (scale 2^(24-s), see fvs.h). */
void or_lut_score(const int32_t *pos, const float *qc, const void *Lin, int half, int LW, const float *qsum,
                  const float *qn2, const uint8_t *rec, int RB, int soff, int T, const int32_t *tiers,
                  const float *deltas, const int32_t *toff, const int32_t *ncnt, int64_t B, int K, float *est,
                  float *sd) {
#pragma omp parallel for schedule(dynamic, 4)
  for (int64_t q = 0; q < B; q++) {
    int32_t *lut = (int32_t *)malloc(sizeof(int32_t) * LW);
    float m = 0.f;
    for (int i = 0; i < LW; i++) {
      const float v = half ? h2f(((const uint16_t *)Lin)[q * LW + i]) : ((const float *)Lin)[q * LW + i];
      m = fmaxf(m, fabsf(v));
    }
    int E = 0;
    (void)frexpf(m, &E);
    const int s = E - 3 > 0 ? E - 3 : 0;
    for (int i = 0; i < LW; i++) {
      const float v = half ? h2f(((const uint16_t *)Lin)[q * LW + i]) : ((const float *)Lin)[q * LW + i];
      lut[i] = (int32_t)rintf(ldexpf(v, 24 - s));
    }
    const int lim = ncnt ? (ncnt[q] < K ? ncnt[q] : K) : K;
    for (int mm = 0; mm < K; mm++) {
      const int64_t o = q * K + mm;
      if (mm >= lim) {
        est[o] = -1e30f;
        sd[o] = 0.f;
        continue;
      }
      const uint8_t *rp = rec + (int64_t)pos[o] * RB;
      float e = qc[q], var = 0.f;
      for (int t = 0; t < T; t++) {
        const int st = tiers[3 * t], en = tiers[3 * t + 1], b = tiers[3 * t + 2];
        const int kb = (en - st) / 8, loff = st * 4;
        int64_t A = 0;
        for (int p = 0; p < b; p++) {
          int64_t S = 0;
          const uint8_t *pl = rp + toff[t] + p * kb;
          for (int j = 0; j < kb; j++) {
            const int byte = pl[j];
            S += lut[loff + 32 * j + (byte >> 4)] + lut[loff + 32 * j + 16 + (byte & 15)];
          }
          A += S << (b - 1 - p);
        }
        const float mid = (float)((1 << b) - 1) * 0.5f;
        float a = ldexpf((float)A, s - 24);
        a = deltas[t] * fmaf(-mid, qsum[(int64_t)t * B + q], a);
        uint16_t sc16, sg16;
        memcpy(&sc16, rp + soff + 4 * t, 2);
        memcpy(&sg16, rp + soff + 4 * t + 2, 2);
        const float sc = h2f(sc16), sg = h2f(sg16);
        e = fmaf(a, sc, e);
        var = fmaf(qn2[(int64_t)t * B + q] * sg, sg, var);
      }
      est[o] = e;
      sd[o] = sqrtf(var);
    }
    free(lut);
  }
}

/* ---------------------------------------------------------------- classification + stage 3 (a16-a18)
 * throughput/enginei8.py:92-95; src/engine3.py:143-146; src/stage3_zc.py:11-27. */
static float exact_dot(const uint16_t *h, const float *qv, int d) {
  float lane[64];
  for (int l = 0; l < 64; l++) lane[l] = 0.f;
  for (int g = 0; g < d / 8; g++) {
    float *a = &lane[g % 64];
    for (int u = 0; u < 8; u++) *a = fmaf(h2f(h[8 * g + u]), qv[8 * g + u], *a);
  }
  for (int o = 32; o > 0; o >>= 1) {
    float t[64];
    for (int l = 0; l < 64; l++) t[l] = lane[l] + lane[l ^ o];
    memcpy(lane, t, sizeof(t));
  }
  return lane[0];
}

void or_refine(const float *est, const float *sd, const int32_t *pos, const int32_t *order, const uint16_t *H,
               const float *Q, int64_t B, int K, int d, float z, int k, int32_t *ids, int32_t *I, float *scores,
               int32_t *reads) {
#pragma omp parallel for schedule(dynamic, 4)
  for (int64_t q = 0; q < B; q++) {
    const float *e = est + q * K, *g = sd + q * K;
    float *lo = (float *)malloc(sizeof(float) * K), *hi = (float *)malloc(sizeof(float) * K);
    uint32_t *tmp = (uint32_t *)malloc(sizeof(uint32_t) * K);
    float *score = (float *)malloc(sizeof(float) * K);
    uint8_t *flag = (uint8_t *)malloc(K);
    uint64_t *keys = (uint64_t *)malloc(sizeof(uint64_t) * K);
    for (int i = 0; i < K; i++) {
      const float t = z * g[i];
      lo[i] = e[i] - t;
      hi[i] = e[i] + t;
    }
    for (int i = 0; i < K; i++) tmp[i] = ord32(hi[i]);
    qsort(tmp, K, sizeof(uint32_t), cmp_u32_desc);
    const uint32_t khk = tmp[k];
    for (int i = 0; i < K; i++) tmp[i] = ord32(lo[i]);
    qsort(tmp, K, sizeof(uint32_t), cmp_u32_desc);
    const uint32_t klk = tmp[k - 1];
    int namb = 0;
    for (int i = 0; i < K; i++) {
      /* compare through the order-preserving keys: a > b <=> ord(a) > ord(b) for non-NaN values */
      const int sure = ord32(lo[i]) > khk;
      const int amb = (ord32(hi[i]) >= klk) && !sure;
      const int32_t id = order[pos[q * K + i]];
      ids[q * K + i] = id;
      flag[i] = sure ? 1 : (amb ? 2 : 0);
      if (sure)
        score[i] = e[i] + 10.0f;
      else if (amb) {
        score[i] = exact_dot(H + (int64_t)id * d, Q + q * d, d);
        namb++;
      } else
        score[i] = -1e9f;
    }
    reads[q] = namb;
    for (int i = 0; i < K; i++) keys[i] = ((uint64_t)ord32(score[i]) << 32) | (uint64_t)(0xffffffffu - (uint32_t)i);
    qsort(keys, K, sizeof(uint64_t), cmp_u64_desc);
    for (int j = 0; j < k; j++) {
      const int slot = (int)(0xffffffffu - (uint32_t)(keys[j] & 0xffffffffu));
      I[q * k + j] = ids[q * K + slot];
      scores[q * k + j] = flag[slot] == 1 ? e[slot] : score[slot];
    }
    free(lo);
    free(hi);
    free(tmp);
    free(score);
    free(flag);
    free(keys);
  }
}

/* ================================================================ trellis engine (latency mode)
 * Bitshift trellis (k = 1 bit per coordinate, L-bit states), src/trellis.py:12-33,
 * src/trellis_scan.py:10-44, src/viterbi_fused.py:7-46. */

/* Viterbi over one vector (n = R coordinates): predecessors of s are (s >> 1) | (u << (L-1)); p1 is
 * taken only when its cost is strictly smaller (viterbi_fused.py:20); the final state is the smallest
 * index of minimum cost (:29-30). Costs in f32: d = x - tab[s]; cost = best + d * d. */
static void viterbi_row(const float *x, int R, const float *tab, int L, int32_t *path) {
  const int S = 1 << L, half = S >> 1;
  float *ca = (float *)malloc(sizeof(float) * S), *cb = (float *)malloc(sizeof(float) * S);
  uint8_t *back = (uint8_t *)malloc((size_t)(R - 1) * S);
  for (int s = 0; s < S; s++) {
    const float d = x[0] - tab[s];
    ca[s] = d * d;
  }
  for (int j = 1; j < R; j++) {
    for (int s = 0; s < S; s++) {
      const int p0 = s >> 1, p1 = p0 | half;
      const float c0 = ca[p0], c1 = ca[p1];
      const int take1 = c1 < c0;
      const float d = x[j] - tab[s];
      cb[s] = (take1 ? c1 : c0) + d * d;
      back[(size_t)(j - 1) * S + s] = (uint8_t)take1;
    }
    float *t = ca;
    ca = cb;
    cb = t;
  }
  int st = 0;
  for (int s = 1; s < S; s++)
    if (ca[s] < ca[st]) st = s;
  path[R - 1] = st;
  for (int j = R - 1; j > 0; j--) {
    const int u = back[(size_t)(j - 1) * S + st];
    st = (st >> 1) | (u << (L - 1));
    path[j - 1] = st;
  }
  free(ca);
  free(cb);
  free(back);
}

/* Encoder: paths, words (trellis_scan.py:10-18) and the fp16 scale (engine_cell.py:21-22) with the
 * canonical double sums (lane = j % 64, xor butterfly) of the GPU kernel. */
void or_trellis_encode(const float *Zs, const float *nz, int64_t n, int R, const float *tab, int L, int W,
                       uint32_t *words, uint16_t *scale1, int32_t *paths) {
#pragma omp parallel for schedule(dynamic, 4)
  for (int64_t v = 0; v < n; v++) {
    const float *x = Zs + v * R;
    int32_t *path = paths + v * R;
    viterbi_row(x, R, tab, L, path);
    for (int w = 0; w < W; w++) {
      uint32_t word = 0;
      for (int t = 0; t < 32; t++) {
        const int b = 32 * w + t;
        uint32_t bit = 0;
        if (b < L)
          bit = ((uint32_t)path[0] >> (L - 1 - b)) & 1u;
        else if (b < R + L - 1)
          bit = (uint32_t)path[b - L + 1] & 1u;
        word |= bit << (31 - t);
      }
      words[v * W + w] = word;
    }
    double l1[64], l2[64];
    for (int l = 0; l < 64; l++) l1[l] = l2[l] = 0.0;
    for (int j = 0; j < R; j++) {
      const double y = (double)tab[path[j]];
      l1[j % 64] += y * y;
      l2[j % 64] += (double)x[j] * y;
    }
    const float yn = sqrtf((float)butterfly64_d(l1));
    const float fip = (float)butterfly64_d(l2) / (yn * sqrtf((float)R));
    scale1[v] = f2h(nz[v] / (fip * yn));
  }
}

/* Decoded coordinate j of a word stream (trellis_scan.py:36-44). */
static inline uint32_t tr_window(const uint32_t *w, int W, int j, int L) {
  const int wi = j >> 5, off = j & 31;
  const uint64_t w0 = w[wi], w1 = wi + 1 < W ? w[wi + 1] : 0u;
  return (uint32_t)((((w0 << 32) | w1) >> (64 - L - off)) & ((1u << L) - 1u));
}

void or_trellis_decode(const uint32_t *words, int64_t n, int W, int R, int L, int32_t *states) {
  for (int64_t v = 0; v < n; v++)
    for (int j = 0; j < R; j++) states[v * R + j] = (int32_t)tr_window(words + v * W, W, j, L);
}

typedef struct {
  const float *Qr;
  const uint32_t *words;
  int W;
  const uint16_t *scale1;
  const float *tab;
  int L, R, half;
} tr_ctx;

/* est = fmaf(scale1, lo + hi, qcp); lo and hi are sequential fmaf chains over the two halves of
 * tab[state_j] * Qr[j] (src/s1cell.py:147-152 with a fixed summation order). half: both operands are first
 * rounded to fp16, as the reference's `.to(tl.float16)` before tl.dot does (src/s1cell.py:127,131-132);
 * half = 0 keeps the fp32 operands of its small-batch kernels (src/s1small_cell.py:17-20). */
static inline float tr_op(float x, int half) { return half ? h2f(f2h(x)) : x; }

static float est_tr_cb(const void *ctx, int64_t q, int64_t r, float qcp) {
  const tr_ctx *c = (const tr_ctx *)ctx;
  const float *qv = c->Qr + q * c->R;
  const uint32_t *w = c->words + r * c->W;
  float lo = 0.f, hi = 0.f;
  const int H = c->R / 2;
  for (int j = 0; j < H; j++)
    lo = fmaf(tr_op(c->tab[tr_window(w, c->W, j, c->L)], c->half), tr_op(qv[j], c->half), lo);
  for (int j = H; j < c->R; j++)
    hi = fmaf(tr_op(c->tab[tr_window(w, c->W, j, c->L)], c->half), tr_op(qv[j], c->half), hi);
  return fmaf(h2f(c->scale1[r]), lo + hi, qcp);
}

void or_tr_first_pass(const float *Qr, const int32_t *probe, int npr, int n1, const int32_t *off,
                      const uint32_t *words, int W, const uint16_t *scale1, const float *tab, int L, int R, int half,
                      const uint16_t *QM, int NC, const float *qadd, int64_t B, int MB, float *bm) {
  const tr_ctx ctx = {Qr, words, W, scale1, tab, L, R, half};
  g_qadd = qadd;
  first_pass_gen(est_tr_cb, &ctx, probe, npr, n1, off, QM, NC, NULL, B, MB, bm);
  g_qadd = NULL;
}

void or_tr_emit(const float *Qr, const int32_t *probe, int npr, int np, const int32_t *off, const uint32_t *words,
                int W, const uint16_t *scale1, const float *tab, int L, int R, int half, const uint16_t *QM, int NC,
                const float *qadd, const float *t0, int64_t B, int M, int32_t *cnt, float *bval, int32_t *bpos) {
  const tr_ctx ctx = {Qr, words, W, scale1, tab, L, R, half};
  g_qadd = qadd;
  emit_gen(est_tr_cb, &ctx, probe, npr, np, off, QM, NC, NULL, t0, B, M, cnt, bval, bpos);
  g_qadd = NULL;
}

/* Routing on fp32 keys (float)QM * scale (engine_cell.py:40-42), sorted by (key desc, cell asc). */
void or_route_topk_scaled(const uint16_t *QM, const float *scale, const float *qadd, int64_t B, int NC, int np,
                          int32_t *probe) {
#pragma omp parallel for schedule(static)
  for (int64_t q = 0; q < B; q++) {
    uint64_t *keys = (uint64_t *)malloc(sizeof(uint64_t) * NC);
    for (int c = 0; c < NC; c++)
      keys[c] = ((uint64_t)ord32(qadd ? (h2f(QM[q * NC + c]) + qadd[q]) * scale[c] : h2f(QM[q * NC + c]) * scale[c])
                 << 32) | (uint64_t)(0xffffffffu - (uint32_t)c);
    qsort(keys, NC, sizeof(uint64_t), cmp_u64_desc);
    for (int i = 0; i < np; i++) probe[q * np + i] = (int32_t)(0xffffffffu - (uint32_t)(keys[i] & 0xffffffffu));
    free(keys);
  }
}

/* Lloyd-Max tiered stage 2 (src/tiered_fused.py:47-72, packed records :112-125). cb: [T][256] levels. */
void or_tiered_score(const int32_t *pos, const float *qc, const float *Zq, int D, const uint8_t *rec, int RB,
                     int soff, int T, const int32_t *tiers, const int32_t *toff, const float *cb, const int32_t *ncnt,
                     int64_t B, int K, float *est, float *sd) {
#pragma omp parallel for schedule(dynamic, 4)
  for (int64_t q = 0; q < B; q++) {
    const float *zq = Zq + q * D;
    float qn2[OR_MAXT];
    for (int t = 0; t < T; t++) {
      double l2[64];
      for (int l = 0; l < 64; l++) l2[l] = 0.0;
      for (int k = 0; k < tiers[3 * t + 1] - tiers[3 * t]; k++) {
        const double z = (double)zq[tiers[3 * t] + k];
        l2[k % 64] += z * z;
      }
      qn2[t] = (float)butterfly64_d(l2);
    }
    const int nc = ncnt ? (ncnt[q] < K ? ncnt[q] : K) : K;
    for (int m = 0; m < K; m++) {
      if (m >= nc) {
        est[q * K + m] = -1e30f;
        sd[q * K + m] = 0.f;
        continue;
      }
      const uint8_t *r = rec + (int64_t)pos[q * K + m] * RB;
      float e = qc[q], var = 0.f;
      for (int t = 0; t < T; t++) {
        const int s = tiers[3 * t], d = tiers[3 * t + 1] - s, b = tiers[3 * t + 2], kb = d / 8;
        const uint8_t *pl = r + toff[t];
        float lane[64];
        for (int l = 0; l < 64; l++) lane[l] = 0.f;
        for (int k = 0; k < d; k++) {
          int code = 0;
          for (int p = 0; p < b; p++) code |= ((pl[p * kb + (k >> 3)] >> (7 - (k & 7))) & 1) << (b - 1 - p);
          lane[k % 64] = fmaf(cb[256 * t + code], zq[s + k], lane[k % 64]);
        }
        for (int o = 32; o > 0; o >>= 1) {
          float nl[64];
          for (int l = 0; l < 64; l++) nl[l] = lane[l] + lane[l ^ o];
          memcpy(lane, nl, sizeof(nl));
        }
        uint16_t ss[2];
        memcpy(ss, r + soff + 4 * t, 4);
        const float sc = h2f(ss[0]), sg = h2f(ss[1]);
        e = fmaf(lane[0], sc, e);
        var = fmaf(qn2[t] * sg, sg, var);
      }
      est[q * K + m] = e;
      sd[q * K + m] = sqrtf(var);
    }
  }
}
