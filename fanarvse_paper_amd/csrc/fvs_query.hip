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
constexpr int kKC = 64;  // k-chunk staged in LDS

template <int QB, bool RESID>
__global__ __launch_bounds__(256) void k_project(const float *__restrict__ Q, const uint16_t *__restrict__ X16,
                                                 const int32_t *__restrict__ order, const int32_t *__restrict__ cell,
                                                 const uint16_t *__restrict__ M16, int64_t nrows, int d,
                                                 const float *__restrict__ Vr, int8_t *__restrict__ out8,
                                                 float *__restrict__ outs) {
  __shared__ float xs[kKC][QB];
  __shared__ float red[QB][4];
  const int j = threadIdx.x;
  const int64_t r0 = (int64_t)blockIdx.x * QB;
  float acc[QB];
#pragma unroll
  for (int rr = 0; rr < QB; rr++) acc[rr] = 0.f;

  for (int k0 = 0; k0 < d; k0 += kKC) {
    __syncthreads();
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
    __syncthreads();
    const int kn = min(kKC, d - k0);
    for (int kk = 0; kk < kn; kk++) {
      const float v = Vr[(int64_t)(k0 + kk) * kR + j];
#pragma unroll
      for (int rr = 0; rr < QB; rr++) acc[rr] = __builtin_fmaf(xs[kk][rr], v, acc[rr]);
    }
  }

  // per-row max |z| over the 256 coordinates
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
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
  }
}

// qc = <Q, c> (sequential double sum) and the fp16 copy of Q. One block per query.
__global__ __launch_bounds__(256) void k_qc_cast(const float *__restrict__ Q, int d, const float *__restrict__ c,
                                                 float *__restrict__ qc, uint16_t *__restrict__ qh) {
  const int64_t q = blockIdx.x;
  const float *qr = Q + q * d;
  for (int k = threadIdx.x; k < d; k += 256) qh[q * d + k] = fvs_f2h(qr[k]);
  if (threadIdx.x == 0) {
    double s = 0.0;
    for (int k = 0; k < d; k++) s += (double)qr[k] * (double)c[k];
    qc[q] = (float)s;
  }
}

}  // namespace

extern "C" int fvs_query_prep(const float *Q, int64_t B, int32_t d, const float *Vr, int32_t R, const float *c,
                              int8_t *q8, float *qs, float *qc, uint16_t *qh, void *stream) {
  if (R != kR) return FVS_E_SHAPE;
  if (B < 0 || d <= 0 || d % 8 != 0) return FVS_E_ARG;
  if (B == 0) return FVS_OK;
  if (!Q || !Vr || !c || !q8 || !qs || !qc || !qh) return FVS_E_ARG;
  hipStream_t st = (hipStream_t)stream;
  constexpr int QB = 8;
  const int64_t nb = (B + QB - 1) / QB;
  hipLaunchKernelGGL((k_project<QB, false>), dim3((unsigned)nb), dim3(256), 0, st, Q, nullptr, nullptr, nullptr,
                     nullptr, B, d, Vr, q8, qs);
  int e = fvs_launch_status();
  if (e) return e;
  hipLaunchKernelGGL(k_qc_cast, dim3((unsigned)B), dim3(256), 0, st, Q, d, c, qc, qh);
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
                     order, cell, means16, N, d, Vr, Z, zs);
  return fvs_launch_status();
}
