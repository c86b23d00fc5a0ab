// Threshold t0 from the first-pass block maxima, and the final stage-1 top-K selection.
#include "fvs_common.h"

namespace {

constexpr int kMaxK = 4096;     // LDS capacity of the sorted top-K (dynamic)
constexpr int kMaxN1 = 4096;
constexpr int kStageT = 8192;   // threshold keys (n1 x MB) staged in LDS once; more are read per pass

__device__ __forceinline__ int cell_blocks(const int32_t *off, int c) {
  const int s = off[c], e = off[c + 1];
  return e > s ? (e - 1) / 32 - s / 32 + 1 : 0;
}

// Batches of at most kSmallB queries run the per-query kernels below with 1024 threads per block: a batch
// of one query then spreads its radix passes over 16 waves instead of 4.
constexpr int kSmallB = 64;

// One block of NT threads per query. Valid values: bm[q][j][b], j < n1, b < blocks(probe[q][j]).
// A probe id outside [0, NC) reads no offsets: its cell counts as empty, and the query's t0 becomes 1e30,
// so its emit pass keeps nothing and its exactness flag (K <= cnt) is cleared. With `staged`, the n1 x MB
// keys are read from global memory once into LDS and the radix passes run over LDS.
template <int NT>
__global__ __launch_bounds__(NT) void k_threshold(const float *__restrict__ bm, const int32_t *__restrict__ probe,
                                                  int npr, const int32_t *__restrict__ off, int NC, int n1, int MB,
                                                  int r, int staged, float *__restrict__ t0, int32_t *__restrict__ cnt) {
  extern __shared__ uint32_t tdyn[];  // [n1] block counts, then [n1 x MB] keys when staged
  int *nb = reinterpret_cast<int *>(tdyn);
  uint32_t *keys = tdyn + n1;
  __shared__ int hist[256];
  __shared__ int sh[fvs_sh_ints(NT)];
  const int64_t q = blockIdx.x;
  int mine = 0, bad = 0;
  for (int j = threadIdx.x; j < n1; j += NT) {
    const int c = probe[q * npr + j];
    const bool in = (unsigned)c < (unsigned)NC;
    nb[j] = in ? cell_blocks(off, c) : 0;
    bad |= in ? 0 : 1;
    mine += nb[j];
  }
  const bool any_bad = __syncthreads_or(bad);
  // block sum of the valid counts
  const int tot = fvs_block_scan<NT>(mine, sh);
  if (threadIdx.x == NT - 1) sh[NT / 64 + 2] = tot;
  __syncthreads();
  const int nv = sh[NT / 64 + 2];
  __syncthreads();
  const int n = n1 * MB;
  const float *row = bm + q * (int64_t)n;
  auto key = [&](int i) -> uint32_t {
    const int j = i / MB, b = i - j * MB;
    return b < nb[j] ? fvs_ord32(row[i]) : 0u;
  };
  const int kk = any_bad ? 0 : min(min(r, n), nv);
  float out = 1e30f;
  if (kk > 0) {
    if (staged) {
      for (int i = threadIdx.x; i < n; i += NT) keys[i] = key(i);
      __syncthreads();
      out = fvs_unord32(fvs_block_kth<uint32_t, NT>([&](int i) { return keys[i]; }, n, kk, hist, sh));
    } else {
      out = fvs_unord32(fvs_block_kth<uint32_t, NT>(key, n, kk, hist, sh));
    }
  }
  if (threadIdx.x == 0) {
    t0[q] = out;
    if (cnt) cnt[q] = 0;  // the emit pass's counter, zeroed here instead of by a fill launch
  }
}

// One block per query: top-K of the first min(cnt, M) buffer entries by (est desc, pos asc).
// Buffers of up to kStage entries are staged once into LDS as 64-bit keys (vectorised loads) and the
// radix passes run over LDS; larger ones (the fallback's 65,536-entry buffers) are read from global.
constexpr int kStage = 4096;

template <int NT>
__global__ __launch_bounds__(NT) void k_select(const float *__restrict__ bval, const int32_t *__restrict__ bpos,
                                                const int32_t *__restrict__ cntp, int M, int K, int kd, float delta,
                                                int32_t *__restrict__ pos, float *__restrict__ est1,
                                                uint8_t *__restrict__ ok, int32_t *__restrict__ ncnt) {
  extern __shared__ uint64_t dyn64[];
  const int P = fvs_pow2_ceil(K);
  uint64_t *s = dyn64;           // [P] the sorted top-K
  uint64_t *keys = dyn64 + P;    // [min(M, kStage)] staged buffer
  __shared__ int hist[256];
  __shared__ int sh[fvs_sh_ints(NT)];
  __shared__ int gcnt;
  const int64_t q = blockIdx.x;
  const int cq = cntp[q];
  const int n = min(cq, M);
  const float *bv = bval + q * (int64_t)M;
  const int32_t *bp = bpos + q * (int64_t)M;
  auto gkey = [&](int i) -> uint64_t {
    return ((uint64_t)fvs_ord32(bv[i]) << 32) | (uint64_t)(0xffffffffu - (uint32_t)bp[i]);
  };
  const bool staged = n <= kStage;
  if (staged) {
    const bool vec = (M & 3) == 0;
    if (vec) {
      const float4 *bv4 = reinterpret_cast<const float4 *>(bv);
      const int4 *bp4 = reinterpret_cast<const int4 *>(bp);
#pragma unroll 4
      for (int i = threadIdx.x; i < (n + 3) / 4; i += NT) {
        const float4 v = bv4[i];
        const int4 p = bp4[i];
        const float vv[4] = {v.x, v.y, v.z, v.w};
        const int pp[4] = {p.x, p.y, p.z, p.w};
#pragma unroll
        for (int u = 0; u < 4; u++)
          if (4 * i + u < n) keys[4 * i + u] = ((uint64_t)fvs_ord32(vv[u]) << 32) | (uint64_t)(0xffffffffu - (uint32_t)pp[u]);
      }
    } else {
      for (int i = threadIdx.x; i < n; i += NT) keys[i] = gkey(i);
    }
    __syncthreads();
  }
  int have;
  if (n >= K) {
    if (staged)
      fvs_block_topk_u64<NT>([&](int i) { return keys[i]; }, n, K, s, hist, sh, &gcnt);
    else
      fvs_block_topk_u64<NT>(gkey, n, K, s, hist, sh, &gcnt);
    have = K;
  } else {
    const int Pn = fvs_pow2_ceil(n > 0 ? n : 1);
    for (int i = threadIdx.x; i < Pn; i += NT) s[i] = i < n ? (staged ? keys[i] : gkey(i)) : 0ull;
    __syncthreads();
    fvs_block_bitonic<uint64_t, true>(s, Pn);
    have = n;
  }
  float *e1 = est1 + q * (int64_t)K;
  int32_t *po = pos + q * (int64_t)K;
  for (int i = threadIdx.x; i < K; i += NT) {
    if (i < have) {
      const uint64_t x = s[i];
      e1[i] = fvs_unord32((uint32_t)(x >> 32));
      po[i] = (int32_t)(0xffffffffu - (uint32_t)(x & 0xffffffffu));
    } else {
      e1[i] = -1e30f;
      po[i] = 0;
    }
  }
  if (threadIdx.x == 0) ok[q] = (uint8_t)(cq >= K && cq <= M);
  if (delta >= 0.f) {
    auto est_at = [&](int i) -> float { return i < have ? fvs_unord32((uint32_t)(s[i] >> 32)) : -1e30f; };
    const float thr = est_at(kd) - delta;
    int mine = 0;
    for (int i = threadIdx.x; i < K; i += NT) mine += (est_at(i) >= thr) ? 1 : 0;
    const int tot = fvs_block_scan<NT>(mine, sh);
    if (threadIdx.x == NT - 1) ncnt[q] = tot;
  } else if (threadIdx.x == 0) {
    ncnt[q] = K;
  }
}

}  // namespace

extern "C" int fvs_threshold(const float *bm, const int32_t *probe, int32_t npr, const int32_t *off, int32_t NC,
                             int64_t B, int32_t n1, int32_t MB, int32_t r, float *t0, int32_t *cnt, void *stream) {
  if (B < 0 || NC <= 0 || n1 <= 0 || n1 > npr || MB <= 0 || r <= 0) return FVS_E_ARG;
  if (n1 > kMaxN1) return FVS_E_CAPACITY;
  if ((int64_t)n1 * MB > (int64_t)1 << 30) return FVS_E_ARG;
  if (B == 0) return FVS_OK;
  if (!bm || !probe || !off || !t0) return FVS_E_ARG;
  const int64_t n = (int64_t)n1 * MB;
  const int staged = n <= kStageT ? 1 : 0;
  const size_t shm = 4 * ((size_t)n1 + (staged ? (size_t)n : 0));
  if (B <= kSmallB)
    hipLaunchKernelGGL(k_threshold<1024>, dim3((unsigned)B), dim3(1024), shm, (hipStream_t)stream, bm, probe, npr, off,
                       NC, n1, MB, r, staged, t0, cnt);
  else
    hipLaunchKernelGGL(k_threshold<256>, dim3((unsigned)B), dim3(256), shm, (hipStream_t)stream, bm, probe, npr, off, NC,
                       n1, MB, r, staged, t0, cnt);
  return fvs_launch_status();
}

extern "C" int fvs_select(const float *bval, const int32_t *bpos, const int32_t *cnt, int64_t B, int32_t M, int32_t K,
                          int32_t kd, float delta, int32_t *pos, float *est1, uint8_t *ok, int32_t *ncnt,
                          void *stream) {
  if (B < 0 || M <= 0 || K <= 0 || kd < 0 || kd >= K) return FVS_E_ARG;
  if (K > kMaxK) return FVS_E_CAPACITY;
  if (B == 0) return FVS_OK;
  if (!bval || !bpos || !cnt || !pos || !est1 || !ok || !ncnt) return FVS_E_ARG;
  const size_t shm = 8 * ((size_t)fvs_pow2_ceil(K) + (size_t)(M < kStage ? M : kStage));
  if (B <= kSmallB)
    hipLaunchKernelGGL(k_select<1024>, dim3((unsigned)B), dim3(1024), shm, (hipStream_t)stream, bval, bpos, cnt, M, K,
                       kd, delta, pos, est1, ok, ncnt);
  else
    hipLaunchKernelGGL(k_select<256>, dim3((unsigned)B), dim3(256), shm, (hipStream_t)stream, bval, bpos, cnt, M, K,
                       kd, delta, pos, est1, ok, ncnt);
  return fvs_launch_status();
}
