// Projection + int8 quantisation (query code and base-set codes), the global-centre term and the
// fp16 query copy.
//
// One thread per output coordinate j (R = 256 threads per block), QB rows per block; every output
// is a sequential fmaf chain over k = 0..d-1, so the result does not depend on the tiling. The row
// tile is staged transposed in LDS (xs[k][row]) so each thread reads QB row values with wide
// broadcast reads, and Vr[k][j] is read once per block (coalesced across the block).
#include "fvs_common.h"

namespace {

constexpr int kR = 256;
constexpr int kKC = 32;  // k-chunk staged in LDS (double-buffered)

template <int QB, bool RESID>
__device__ __forceinline__ void stage_rows(float (*xs)[QB], const float *__restrict__ Q, const uint16_t *__restrict__ X16,
                                           const int32_t *__restrict__ order, const int32_t *__restrict__ cell,
                                           const uint16_t *__restrict__ M16, int64_t r0, int64_t nrows, int d, int k0) {
  for (int i = threadIdx.x; i < QB * kKC; i += 256) {
    const int rr = i / kKC, kk = i % kKC;
    const int64_t row = r0 + rr;
    const int k = k0 + kk;
    float x = 0.f;
    if (row < nrows && k < d) {
      if (RESID) {
        const int64_t id = order[row];
        const int64_t cc = cell[row];
        x = fvs_h2f(X16[id * d + k]) - fvs_h2f(M16[cc * d + k]);
      } else {
        x = Q[row * d + k];
      }
    }
    xs[kk][rr] = x;
  }
}

// RESID: rows are the cell residuals of the base set (index build). Otherwise rows are queries, and the block
// also writes the projection z itself (zout), qc = <Q, c> and the fp16 copy qh as k_query_code computes them.
template <int QB, bool RESID>
__global__ __launch_bounds__(256) void k_project(const float *__restrict__ Q, const uint16_t *__restrict__ X16,
                                                 const int32_t *__restrict__ order, const int32_t *__restrict__ cell,
                                                 const uint16_t *__restrict__ M16, int64_t nrows, int d,
                                                 const float *__restrict__ Vr, int8_t *__restrict__ out8,
                                                 float *__restrict__ outs, float *__restrict__ zout,
                                                 const float *__restrict__ c, float *__restrict__ qc,
                                                 uint16_t *__restrict__ qh) {
  __shared__ float xs[2][kKC][QB];
  __shared__ float red[QB][4];
  const int j = threadIdx.x;
  const int64_t r0 = (int64_t)blockIdx.x * QB;
  float acc[QB];
#pragma unroll
  for (int rr = 0; rr < QB; rr++) acc[rr] = 0.f;

  // software pipeline: chunk i+1 of the rows (LDS) and of Vr's column j (registers) is fetched while
  // chunk i is consumed
  float vcur[kKC], vnext[kKC];
  stage_rows<QB, RESID>(xs[0], Q, X16, order, cell, M16, r0, nrows, d, 0);
#pragma unroll
  for (int kk = 0; kk < kKC; kk++) vcur[kk] = kk < d ? Vr[(int64_t)kk * kR + j] : 0.f;
  __syncthreads();
  int buf = 0;
  for (int k0 = 0; k0 < d; k0 += kKC) {
    const int k1 = k0 + kKC;
    if (k1 < d) {
      stage_rows<QB, RESID>(xs[buf ^ 1], Q, X16, order, cell, M16, r0, nrows, d, k1);
#pragma unroll
      for (int kk = 0; kk < kKC; kk++) vnext[kk] = k1 + kk < d ? Vr[(int64_t)(k1 + kk) * kR + j] : 0.f;
    }
    const int kn = min(kKC, d - k0);
    if (kn == kKC) {
#pragma unroll
      for (int kk = 0; kk < kKC; kk++) {
#pragma unroll
        for (int rr = 0; rr < QB; rr++) acc[rr] = __builtin_fmaf(xs[buf][kk][rr], vcur[kk], acc[rr]);
      }
    } else {
#pragma unroll
      for (int kk = 0; kk < kKC; kk++) {
        if (kk < kn) {
#pragma unroll
          for (int rr = 0; rr < QB; rr++) acc[rr] = __builtin_fmaf(xs[buf][kk][rr], vcur[kk], acc[rr]);
        }
      }
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < kKC; kk++) vcur[kk] = vnext[kk];
    buf ^= 1;
  }

  // per-row max |z| over the 256 coordinates
  const int lane = threadIdx.x & 63, w = fvs_wave_id();
#pragma unroll
  for (int rr = 0; rr < QB; rr++) {
    const float m = fvs_wave_max(fabsf(acc[rr]));
    if (lane == 0) red[rr][w] = m;
  }
  __syncthreads();
#pragma unroll
  for (int rr = 0; rr < QB; rr++) {
    const int64_t row = r0 + rr;
    if (row >= nrows) continue;
    const float amax = fmaxf(fmaxf(red[rr][0], red[rr][1]), fmaxf(red[rr][2], red[rr][3]));
    const float a = fmaxf(amax, 1e-12f) / 127.0f;
    float qv = rintf(acc[rr] / a);
    qv = fminf(fmaxf(qv, -127.0f), 127.0f);
    out8[row * kR + j] = (int8_t)(int)qv;
    if (j == 0) outs[row] = a;
    if (!RESID) zout[row * kR + j] = acc[rr];
  }
  if constexpr (!RESID) {
    // qc and the fp16 copy, one wave per row: lane l sums the exact double products of coordinates
    // l, l + 64, ... in order, then the fixed xor butterfly (k_query_code's order)
    for (int rr = w; rr < QB; rr += 4) {
      const int64_t row = r0 + rr;
      if (row >= nrows) continue;
      const float *qr = Q + row * d;
      double sacc = 0.0;
      for (int k = lane; k < d; k += 64) {
        const float x = qr[k];
        qh[row * d + k] = fvs_f2h(x);
        sacc += (double)x * (double)c[k];
      }
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) sacc += fvs_xor_lane_d(sacc, o);
      if (lane == 0) qc[row] = (float)sacc;
    }
  }
}

// Query code from the projected query z (R = 256: four coordinates per lane), plus qc = <Q, c> and
// the fp16 copy of Q. One wave per query. qc: lane l sums the exact double products of coordinates
// l, l+64, ... in order, then a fixed xor butterfly combines the 64 lane sums.
__global__ __launch_bounds__(256) void k_query_code(const float *__restrict__ z, const float *__restrict__ Q, int64_t B,
                                                    int d, const float *__restrict__ c, int8_t *__restrict__ q8,
                                                    float *__restrict__ qs, float *__restrict__ qc,
                                                    uint16_t *__restrict__ qh) {
  const int64_t q = (int64_t)blockIdx.x * 4 + fvs_wave_id();
  if (q >= B) return;
  const int lane = threadIdx.x & 63;
  const float4 zz = reinterpret_cast<const float4 *>(z + q * kR)[lane];
  const float amax = fvs_wave_max(fmaxf(fmaxf(fabsf(zz.x), fabsf(zz.y)), fmaxf(fabsf(zz.z), fabsf(zz.w))));
  const float a = fmaxf(amax, 1e-12f) / 127.0f;
  const float zv[4] = {zz.x, zz.y, zz.z, zz.w};
  uint32_t packed = 0;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const float qv = fminf(fmaxf(rintf(zv[i] / a), -127.0f), 127.0f);
    packed |= ((uint32_t)(uint8_t)(int8_t)(int)qv) << (8 * i);
  }
  reinterpret_cast<uint32_t *>(q8 + q * kR)[lane] = packed;
  if (lane == 0) qs[q] = a;
  const float *qr = Q + q * d;
  double s = 0.0;
  for (int k = lane; k < d; k += 64) {
    const float x = qr[k];
    qh[q * d + k] = fvs_f2h(x);
    s += (double)x * (double)c[k];
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) s += fvs_xor_lane_d(s, o);
  if (lane == 0) qc[q] = (float)s;
}

// The three dense products of a small batch in one launch, one wave per output row:
//   rows [0, R):          Qr[b][j] = <Q[b], W1T[j]>            (f32)
//   rows [R, R + NC):     QM[b][c] = fp16(<fp16(Q[b]), M16[c]>) (fp16 inputs, f32 sum, one rounding)
//   rows [R + NC, +D):    Zq[b][t] = <Q[b], VPT[t]>            (f32)
//   row R + NC + D:       qc[b] = <Q[b], c>, the canonical double sum of k_query_code (lane l takes
//                         k = l, l + 64, ..., then the same xor butterfly), so it is the same value
// Each lane sums its 4-element slices of the row in k order for every query of the batch, then a fixed
// xor butterfly reduces the lanes. The products are the BLAS ones of a large batch, computed where
// three library launches would each cost more than the 24 MB they read.
constexpr int kDenseMaxB = 8;

__global__ __launch_bounds__(256) void k_dense_small(const float *__restrict__ Q, int B, int d,
                                                     const float *__restrict__ W1T, int R, float *__restrict__ Qr,
                                                     const uint16_t *__restrict__ M16, int NC,
                                                     uint16_t *__restrict__ QM, const float *__restrict__ VPT, int D,
                                                     float *__restrict__ Zq, const float *__restrict__ c,
                                                     float *__restrict__ qc) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + fvs_wave_id();
  if (row > R + NC + D) return;  // wave-uniform; no barrier below
  if (row == R + NC + D) {
    for (int b = 0; b < B; b++) {
      double sd = 0.0;
      for (int k = lane; k < d; k += 64) sd += (double)Q[(int64_t)b * d + k] * (double)c[k];
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) sd += fvs_xor_lane_d(sd, o);
      if (lane == 0) qc[b] = (float)sd;
    }
    return;
  }
  const int kind = row < R ? 0 : (row < R + NC ? 1 : 2);
  float acc[kDenseMaxB];
#pragma unroll
  for (int b = 0; b < kDenseMaxB; b++) acc[b] = 0.f;
  for (int i0 = 4 * lane; i0 < d; i0 += 256) {
    float x[4];
    if (kind == 1) {
      const uint2 h = *reinterpret_cast<const uint2 *>(M16 + (int64_t)(row - R) * d + i0);
      x[0] = fvs_h2f((uint16_t)(h.x & 0xffffu));
      x[1] = fvs_h2f((uint16_t)(h.x >> 16));
      x[2] = fvs_h2f((uint16_t)(h.y & 0xffffu));
      x[3] = fvs_h2f((uint16_t)(h.y >> 16));
    } else {
      const float *src = kind == 0 ? W1T + (int64_t)row * d : VPT + (int64_t)(row - R - NC) * d;
      const float4 v = *reinterpret_cast<const float4 *>(src + i0);
      x[0] = v.x;
      x[1] = v.y;
      x[2] = v.z;
      x[3] = v.w;
    }
#pragma unroll
    for (int b = 0; b < kDenseMaxB; b++) {
      if (b < B) {
        const float4 qv = *reinterpret_cast<const float4 *>(Q + (int64_t)b * d + i0);
        float q[4] = {qv.x, qv.y, qv.z, qv.w};
        if (kind == 1) {
#pragma unroll
          for (int u = 0; u < 4; u++) q[u] = fvs_h2f(fvs_f2h(q[u]));  // the fp16 copy of the query
        }
#pragma unroll
        for (int u = 0; u < 4; u++) acc[b] = __builtin_fmaf(q[u], x[u], acc[b]);
      }
    }
  }
#pragma unroll
  for (int b = 0; b < kDenseMaxB; b++) {
    if (b < B) {
      float v = acc[b];
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) v += fvs_xor_lane_f(v, o);
      if (lane == 0) {
        if (kind == 0)
          Qr[(int64_t)b * R + row] = v;
        else if (kind == 1)
          QM[(int64_t)b * NC + row - R] = fvs_f2h(v);
        else
          Zq[(int64_t)b * D + row - R - NC] = v;
      }
    }
  }
}

}  // namespace

extern "C" int fvs_dense_small(const float *Q, int64_t B, int32_t d, const float *W1T, int32_t R, float *Qr,
                               const uint16_t *M16, int32_t NC, uint16_t *QM, const float *VPT, int32_t D, float *Zq,
                               const float *c, float *qc, void *stream) {
  if (B < 0 || B > kDenseMaxB || d <= 0 || d % 4 != 0 || R < 0 || NC < 0 || D < 0) return FVS_E_ARG;
  if (B == 0) return FVS_OK;
  if (!Q || !c || !qc || (R && (!W1T || !Qr)) || (NC && (!M16 || !QM)) || (D && (!VPT || !Zq))) return FVS_E_ARG;
  const int64_t rows = (int64_t)R + NC + D + 1;
  hipLaunchKernelGGL(k_dense_small, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, (hipStream_t)stream, Q, (int)B, d,
                     W1T, R, Qr, M16, NC, QM, VPT, D, Zq, c, qc);
  return fvs_launch_status();
}

extern "C" int fvs_query_prep(const float *Q, int64_t B, int32_t d, const float *z, int32_t R, const float *c,
                              int8_t *q8, float *qs, float *qc, uint16_t *qh, void *stream) {
  if (R != kR) return FVS_E_SHAPE;
  if (B < 0 || d <= 0 || d % 8 != 0) return FVS_E_ARG;
  if (B == 0) return FVS_OK;
  if (!Q || !z || !c || !q8 || !qs || !qc || !qh) return FVS_E_ARG;
  hipLaunchKernelGGL(k_query_code, dim3((unsigned)((B + 3) / 4)), dim3(256), 0, (hipStream_t)stream, z, Q, B, d, c,
                     q8, qs, qc, qh);
  return fvs_launch_status();
}

extern "C" int fvs_build_codes(const uint16_t *X16, const int32_t *order, const int32_t *cell, int64_t N, int32_t d,
                               const uint16_t *means16, const float *Vr, int32_t R, int8_t *Z, float *zs,
                               void *stream) {
  if (R != kR) return FVS_E_SHAPE;
  if (N < 0 || d <= 0 || d % 8 != 0) return FVS_E_ARG;
  if (N == 0) return FVS_OK;
  if (!X16 || !order || !cell || !means16 || !Vr || !Z || !zs) return FVS_E_ARG;
  constexpr int QB = 64;
  const int64_t nb = (N + QB - 1) / QB;
  hipLaunchKernelGGL((k_project<QB, true>), dim3((unsigned)nb), dim3(256), 0, (hipStream_t)stream, nullptr, X16,
                     order, cell, means16, N, d, Vr, Z, zs, nullptr, nullptr, nullptr, nullptr);
  return fvs_launch_status();
}

extern "C" int fvs_query_code(const float *Q, int64_t B, int32_t d, const float *Vr, int32_t R, const float *c,
                              float *z, int8_t *q8, float *qs, float *qc, uint16_t *qh, void *stream) {
  if (R != kR) return FVS_E_SHAPE;
  if (B < 0 || d <= 0 || d % 8 != 0) return FVS_E_ARG;
  if (B == 0) return FVS_OK;
  if (!Q || !Vr || !c || !z || !q8 || !qs || !qc || !qh) return FVS_E_ARG;
  constexpr int QB = 8;  // 250 workgroups for a batch of 2000
  const int64_t nb = (B + QB - 1) / QB;
  hipLaunchKernelGGL((k_project<QB, false>), dim3((unsigned)nb), dim3(256), 0, (hipStream_t)stream, Q, nullptr,
                     nullptr, nullptr, nullptr, B, d, Vr, q8, qs, z, c, qc, qh);
  return fvs_launch_status();
}
