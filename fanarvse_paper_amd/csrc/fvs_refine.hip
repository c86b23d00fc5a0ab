// Error-bar classification, exact scoring of the ambiguous candidates and the final top-k.
//
// One block (4 waves, or 16 for small batches) per query. est/sd are staged once into LDS as the
// lower/upper interval keys; the two order statistics (k+1-th largest upper bound, k-th largest lower
// bound) come from radix selects over LDS. Ambiguous slots and their ids are compacted in LDS and the
// waves take them in groups of four rows, so four fp16 rows (coalesced 16-byte lane loads, from HBM or pinned host
// memory over PCIe) are in flight per wave; each lane keeps its slice of the query in registers,
// and every row's partial sums are reduced with the same fixed butterfly.
#include "fvs_common.h"

namespace {

constexpr int kMaxK = 4096;
constexpr int kMaxk = 1024;
constexpr int kRows = 4;       // rows in flight per wave
constexpr int kMaxG = 8;       // 8-element groups per lane: d <= 8 * 64 * kMaxG = 4096
constexpr int kSmallB = 64;    // batches up to this size use 1024-thread blocks

struct RefineLds {  // fixed part; the per-slot arrays follow in dynamic LDS
  uint64_t s[kMaxk];
  int hist[512];
  int sh[fvs_sh_ints(1024)];
  int namb, gcnt;
};

template <int NG>
__device__ __forceinline__ void dot_rows(const uint16_t *__restrict__ H, int d, const int32_t *ids, const int16_t *slots,
                                         int a0, int na, const float (&qv)[NG][8], float *score, int lane) {
  // rows a0 .. a0+kRows-1 of the ambiguous list (guarded), lane l covers groups l, l+64, ...
  uint4 hv[kRows][NG];
#pragma unroll
  for (int r = 0; r < kRows; r++) {
    const int a = a0 + r;
    const int64_t id = a < na ? ids[a] : ids[a0];
    const uint4 *hr = reinterpret_cast<const uint4 *>(H + id * d);
#pragma unroll
    for (int g = 0; g < NG; g++) {
      const int gi = lane + 64 * g;
      hv[r][g] = gi * 8 < d ? hr[gi] : make_uint4(0, 0, 0, 0);
    }
  }
#pragma unroll
  for (int r = 0; r < kRows; r++) {
    float acc = 0.f;
#pragma unroll
    for (int g = 0; g < NG; g++) {
      if ((lane + 64 * g) * 8 < d) {
        const uint32_t hw[4] = {hv[r][g].x, hv[r][g].y, hv[r][g].z, hv[r][g].w};
#pragma unroll
        for (int u = 0; u < 4; u++) {
          acc = __builtin_fmaf(fvs_h2f((uint16_t)(hw[u] & 0xffffu)), qv[g][2 * u], acc);
          acc = __builtin_fmaf(fvs_h2f((uint16_t)(hw[u] >> 16)), qv[g][2 * u + 1], acc);
        }
      }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) acc += fvs_xor_lane_f(acc, o);
    if (lane == 0 && a0 + r < na) score[slots[a0 + r]] = acc;
  }
}

template <int NG, int NT>
__global__ __launch_bounds__(NT) void k_refine(const float *__restrict__ est, const float *__restrict__ sd,
                                                const int32_t *__restrict__ pos, const int32_t *__restrict__ order,
                                                const uint16_t *__restrict__ H, const float *__restrict__ Q, int K,
                                                int d, float z, int k, int32_t *__restrict__ ids,
                                                int32_t *__restrict__ Iout, float *__restrict__ scores,
                                                int32_t *__restrict__ reads) {
  __shared__ RefineLds L;
  extern __shared__ uint8_t dyn[];
  float *lo = reinterpret_cast<float *>(dyn);     // [K]
  float *hi = lo + K;                            // [K]
  float *score = hi + K;                         // [K]
  int32_t *sid = reinterpret_cast<int32_t *>(score + K);  // [K] ids of the slots
  int32_t *aid = sid + K;                        // [K] ids of the ambiguous slots
  int16_t *amb = reinterpret_cast<int16_t *>(aid + K);    // [K]
  uint8_t *flag = reinterpret_cast<uint8_t *>(amb + K);   // [K] 1 sure, 2 ambiguous

  const int64_t q = blockIdx.x;
  const int tid = threadIdx.x;
  const float *e = est + q * (int64_t)K;
  const float *g = sd + q * (int64_t)K;
  const int32_t *pq = pos + q * (int64_t)K;
  for (int i = tid; i < K; i += NT) {
    const float t = z * g[i];
    lo[i] = e[i] - t;
    hi[i] = e[i] + t;
    const int32_t id = order ? order[pq[i]] : pq[i];
    sid[i] = id;
    ids[q * (int64_t)K + i] = id;
  }
  if (tid == 0) L.namb = 0;
  __syncthreads();
  uint32_t hk1u, lku;  // the (k+1)-th largest upper bound and the k-th largest lower bound, in one set of passes
  fvs_block_kth2<uint32_t, NT>([&](int i) { return fvs_ord32(hi[i]); }, [&](int i) { return fvs_ord32(lo[i]); }, K,
                               k + 1, k, L.hist, L.sh, hk1u, lku);
  const float hk1 = fvs_unord32(hk1u), lk = fvs_unord32(lku);
  for (int i = tid; i < K; i += NT) {
    const bool sure = lo[i] > hk1;
    const bool am = (hi[i] >= lk) && !sure;
    flag[i] = sure ? 1 : (am ? 2 : 0);
    score[i] = sure ? e[i] + 10.0f : -1e9f;
    if (am) {
      const int a = atomicAdd(&L.namb, 1);
      amb[a] = (int16_t)i;
      aid[a] = sid[i];
    }
  }
  __syncthreads();

  // exact scores of the ambiguous candidates
  const int lane = tid & 63, w = fvs_wave_id();
  const int na = L.namb;
  if (na > 0) {
    float qv[NG][8];
    const float *qr = Q + q * (int64_t)d;
#pragma unroll
    for (int gg = 0; gg < NG; gg++) {
      const int gi = lane + 64 * gg;
#pragma unroll
      for (int u = 0; u < 8; u++) qv[gg][u] = gi * 8 < d ? qr[gi * 8 + u] : 0.f;
    }
    for (int a0 = w * kRows; a0 < na; a0 += (NT / 64) * kRows) dot_rows<NG>(H, d, aid, amb, a0, na, qv, score, lane);
  }
  __syncthreads();
  if (tid == 0) reads[q] = na;

  // final top-k by (score descending, slot ascending)
  auto key = [&](int i) -> uint64_t {
    return ((uint64_t)fvs_ord32(score[i]) << 32) | (uint64_t)(0xffffffffu - (uint32_t)i);
  };
  fvs_block_topk_u64<NT>(key, K, k, L.s, L.hist, L.sh, &L.gcnt);
  for (int j = tid; j < k; j += NT) {
    const int slot = (int)(0xffffffffu - (uint32_t)(L.s[j] & 0xffffffffu));
    Iout[q * (int64_t)k + j] = sid[slot];
    scores[q * (int64_t)k + j] = flag[slot] == 1 ? e[slot] : score[slot];
  }
}

// ---------------------------------------------------------------------------------- row tier split
// Stage 3 in two halves for rows that live outside GPU-visible memory (the NVMe row tier): the
// classification first, so the host knows which rows to read, then the exact scores from a buffer of
// those rows. Both halves follow k_refine step for step (same order statistics, same dot, same final
// top-k), so the results are bit-identical to fvs_refine over the same rows.

// One 256-thread block per query: ids, sure/ambiguous flags, and the ambiguous slots in ascending
// slot order.
__global__ __launch_bounds__(256) void k_classify(const float *__restrict__ est, const float *__restrict__ sd,
                                                  const int32_t *__restrict__ pos, const int32_t *__restrict__ order,
                                                  int K, float z, int k, int32_t *__restrict__ ids,
                                                  uint8_t *__restrict__ flag, int32_t *__restrict__ namb,
                                                  int32_t *__restrict__ aslot) {
  __shared__ int hist[512];
  __shared__ int sh[fvs_sh_ints(256)];
  extern __shared__ uint8_t dyn[];
  float *lo = reinterpret_cast<float *>(dyn);  // [K]
  float *hi = lo + K;                         // [K]
  const int64_t q = blockIdx.x;
  const int tid = threadIdx.x;
  const float *e = est + q * (int64_t)K;
  const float *g = sd + q * (int64_t)K;
  const int32_t *pq = pos + q * (int64_t)K;
  for (int i = tid; i < K; i += 256) {
    const float t = z * g[i];
    lo[i] = e[i] - t;
    hi[i] = e[i] + t;
    ids[q * (int64_t)K + i] = order ? order[pq[i]] : pq[i];
  }
  __syncthreads();
  uint32_t hk1u, lku;
  fvs_block_kth2<uint32_t>([&](int i) { return fvs_ord32(hi[i]); }, [&](int i) { return fvs_ord32(lo[i]); }, K, k + 1,
                           k, hist, sh, hk1u, lku);
  const float hk1 = fvs_unord32(hk1u), lk = fvs_unord32(lku);
  int base = 0;
  for (int i0 = 0; i0 < K; i0 += 256) {
    const int i = i0 + tid;
    bool am = false;
    if (i < K) {
      const bool sure = lo[i] > hk1;
      am = (hi[i] >= lk) && !sure;
      flag[q * (int64_t)K + i] = sure ? 1 : (am ? 2 : 0);
    }
    const int inc = fvs_block_scan256(am ? 1 : 0, sh);
    if (am) aslot[q * (int64_t)K + base + inc - 1] = i;
    if (tid == 255) sh[6] = inc;
    __syncthreads();
    base += sh[6];
    __syncthreads();
  }
  if (tid == 0) namb[q] = base;
}

// One block per query: rows[roff[q] + j] is the row of ambiguous slot aslot[q][j], j < namb[q].
template <int NG>
__global__ __launch_bounds__(256) void k_refine_rows(const float *__restrict__ est, const uint8_t *__restrict__ flag,
                                                     const int32_t *__restrict__ aslot,
                                                     const int32_t *__restrict__ namb,
                                                     const int64_t *__restrict__ roff,
                                                     const int32_t *__restrict__ ids,
                                                     const uint16_t *__restrict__ rows, const float *__restrict__ Q,
                                                     int K, int d, int k, int32_t *__restrict__ Iout,
                                                     float *__restrict__ scores, int32_t *__restrict__ reads) {
  __shared__ RefineLds L;
  extern __shared__ uint8_t dyn[];
  float *score = reinterpret_cast<float *>(dyn);           // [K]
  int32_t *aid = reinterpret_cast<int32_t *>(score + K);   // [K] row of the j-th ambiguous slot in `rows`
  int16_t *amb = reinterpret_cast<int16_t *>(aid + K);     // [K]
  const int64_t q = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, w = fvs_wave_id();
  const float *e = est + q * (int64_t)K;
  const uint8_t *fl = flag + q * (int64_t)K;
  const int na = namb[q];
  for (int i = tid; i < K; i += 256) score[i] = fl[i] == 1 ? e[i] + 10.0f : -1e9f;
  for (int j = tid; j < na; j += 256) {
    aid[j] = j;
    amb[j] = (int16_t)aslot[q * (int64_t)K + j];
  }
  __syncthreads();
  if (na > 0) {
    float qv[NG][8];
    const float *qr = Q + q * (int64_t)d;
#pragma unroll
    for (int gg = 0; gg < NG; gg++) {
      const int gi = lane + 64 * gg;
#pragma unroll
      for (int u = 0; u < 8; u++) qv[gg][u] = gi * 8 < d ? qr[gi * 8 + u] : 0.f;
    }
    const uint16_t *Hq = rows + roff[q] * (int64_t)d;
    for (int a0 = w * kRows; a0 < na; a0 += 4 * kRows) dot_rows<NG>(Hq, d, aid, amb, a0, na, qv, score, lane);
  }
  __syncthreads();
  if (tid == 0) reads[q] = na;
  auto key = [&](int i) -> uint64_t {
    return ((uint64_t)fvs_ord32(score[i]) << 32) | (uint64_t)(0xffffffffu - (uint32_t)i);
  };
  fvs_block_topk_u64(key, K, k, L.s, L.hist, L.sh, &L.gcnt);
  for (int j = tid; j < k; j += 256) {
    const int slot = (int)(0xffffffffu - (uint32_t)(L.s[j] & 0xffffffffu));
    Iout[q * (int64_t)k + j] = ids[q * (int64_t)K + slot];
    scores[q * (int64_t)k + j] = fl[slot] == 1 ? e[slot] : score[slot];
  }
}

}  // namespace

extern "C" int fvs_refine(const float *est, const float *sd, const int32_t *pos, const int32_t *order,
                          const uint16_t *H, const float *Q, int64_t B, int32_t K, int32_t d, float z, int32_t k,
                          int32_t *ids, int32_t *I, float *scores, int32_t *reads, void *stream) {
  if (B < 0 || k <= 0 || K <= k || d <= 0 || d % 8 != 0 || !(z >= 0.f)) return FVS_E_ARG;
  if (K > kMaxK || k > kMaxk || d > 8 * 64 * kMaxG) return FVS_E_CAPACITY;
  if (B == 0) return FVS_OK;
  if (!est || !sd || !pos || !H || !Q || !ids || !I || !scores || !reads) return FVS_E_ARG;
  const size_t shm = (size_t)K * (4 * 5 + 2 + 1);
  hipStream_t st = (hipStream_t)stream;
  const int ng = (d / 8 + 63) / 64;
  // batches of at most kSmallB queries: 1024 threads per query (16 waves, 64 rows in flight) when the
  // query slice fits the 128 registers a thread of such a block has (d <= 1536)
  const bool big = B <= kSmallB && ng <= 3;
#define FVS_REFINE_LAUNCH(NG, NT)                                                                                \
  hipLaunchKernelGGL((k_refine<NG, NT>), dim3((unsigned)B), dim3(NT), shm, st, est, sd, pos, order, H, Q, K, d, z, k, \
                     ids, I, scores, reads)
  if (ng <= 1) {
    if (big) FVS_REFINE_LAUNCH(1, 1024); else FVS_REFINE_LAUNCH(1, 256);
  } else if (ng <= 2) {
    if (big) FVS_REFINE_LAUNCH(2, 1024); else FVS_REFINE_LAUNCH(2, 256);
  } else if (ng <= 3) {
    if (big) FVS_REFINE_LAUNCH(3, 1024); else FVS_REFINE_LAUNCH(3, 256);
  } else if (ng <= 4) {
    FVS_REFINE_LAUNCH(4, 256);
  } else {
    FVS_REFINE_LAUNCH(8, 256);
  }
#undef FVS_REFINE_LAUNCH
  return fvs_launch_status();
}

extern "C" int fvs_classify(const float *est, const float *sd, const int32_t *pos, const int32_t *order, int64_t B,
                            int32_t K, float z, int32_t k, int32_t *ids, uint8_t *flag, int32_t *namb, int32_t *aslot,
                            void *stream) {
  if (B < 0 || k <= 0 || K <= k || !(z >= 0.f)) return FVS_E_ARG;
  if (K > kMaxK || k > kMaxk) return FVS_E_CAPACITY;
  if (B == 0) return FVS_OK;
  if (!est || !sd || !pos || !ids || !flag || !namb || !aslot) return FVS_E_ARG;
  hipLaunchKernelGGL(k_classify, dim3((unsigned)B), dim3(256), (size_t)K * 8, (hipStream_t)stream, est, sd, pos, order,
                     K, z, k, ids, flag, namb, aslot);
  return fvs_launch_status();
}

extern "C" int fvs_refine_rows(const float *est, const uint8_t *flag, const int32_t *aslot, const int32_t *namb,
                               const int64_t *roff, const int32_t *ids, const uint16_t *rows, const float *Q, int64_t B,
                               int32_t K, int32_t d, int32_t k, int32_t *I, float *scores, int32_t *reads,
                               void *stream) {
  if (B < 0 || k <= 0 || K <= k || d <= 0 || d % 8 != 0) return FVS_E_ARG;
  if (K > kMaxK || k > kMaxk || d > 8 * 64 * kMaxG) return FVS_E_CAPACITY;
  if (B == 0) return FVS_OK;
  if (!est || !flag || !aslot || !namb || !roff || !ids || !rows || !Q || !I || !scores || !reads) return FVS_E_ARG;
  const size_t shm = (size_t)K * (4 + 4 + 2);
  hipStream_t st = (hipStream_t)stream;
  const int ng = (d / 8 + 63) / 64;
#define FVS_ROWS_LAUNCH(NG)                                                                                       \
  hipLaunchKernelGGL(k_refine_rows<NG>, dim3((unsigned)B), dim3(256), shm, st, est, flag, aslot, namb, roff, ids, rows, \
                     Q, K, d, k, I, scores, reads)
  if (ng <= 1)
    FVS_ROWS_LAUNCH(1);
  else if (ng <= 2)
    FVS_ROWS_LAUNCH(2);
  else if (ng <= 3)
    FVS_ROWS_LAUNCH(3);
  else if (ng <= 4)
    FVS_ROWS_LAUNCH(4);
  else
    FVS_ROWS_LAUNCH(8);
#undef FVS_ROWS_LAUNCH
  return fvs_launch_status();
}
