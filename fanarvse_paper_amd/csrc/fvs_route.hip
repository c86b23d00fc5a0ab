// Routing (top-n_p cells per query) and the (query, cell) pair lists grouped by cell.
#include "fvs_common.h"

namespace {

constexpr int kMaxProbe = 4096;     // LDS capacity of the routing sort
constexpr int kMaxCellPairs = 16384;  // LDS capacity of the per-cell pair sort

// One block per query: radix-select the n_p-th largest key, gather the n_p keys above it and sort
// them. Key = (orderable fp16 score << 16) | (0xffff - cell): score descending, then cell ascending.
__global__ __launch_bounds__(256) void k_route_topk(const uint16_t *__restrict__ QM, int NC, int np,
                                                    int32_t *__restrict__ probe) {
  __shared__ uint64_t s[kMaxProbe];
  __shared__ int hist[256];
  __shared__ int sh[8];
  __shared__ int cnt;
  const int64_t q = blockIdx.x;
  const uint16_t *row = QM + q * NC;
  auto key = [&](int i) -> uint64_t {
    return ((uint64_t)fvs_ord16(row[i]) << 16) | (uint64_t)(0xffffu - (uint32_t)i);
  };
  fvs_block_topk_u64(key, NC, np, s, hist, sh, &cnt);
  for (int i = threadIdx.x; i < np; i += 256) probe[q * np + i] = (int32_t)(0xffffu - (uint32_t)(s[i] & 0xffffu));
}

__global__ void k_pairs_count(const int32_t *__restrict__ probe, int64_t B, int npr, int n, int32_t *__restrict__ ccnt) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= B * n) return;
  const int64_t q = t / n;
  const int r = (int)(t % n);
  atomicAdd(&ccnt[probe[q * npr + r]], 1);
}

// Exclusive prefix sum of ccnt into coff; clears fill. One block of 256 threads.
__global__ __launch_bounds__(256) void k_pairs_scan(const int32_t *__restrict__ ccnt, int NC, int32_t *__restrict__ coff,
                                                    int32_t *__restrict__ fill) {
  __shared__ int tmp[8];
  int run = 0;
  for (int base = 0; base < NC; base += 256) {
    const int c = base + (int)threadIdx.x;
    const int v = c < NC ? ccnt[c] : 0;
    const int inc = fvs_block_scan256(v, tmp);
    if (c < NC) {
      coff[c] = run + inc - v;
      fill[c] = 0;
    }
    if (threadIdx.x == 255) tmp[4] = inc;
    __syncthreads();
    run += tmp[4];
    __syncthreads();
  }
}

// Scatter each (q, r) pair into its cell's range; packs (q << 12 | r) into qid until the sort.
__global__ void k_pairs_scatter(const int32_t *__restrict__ probe, int64_t B, int npr, int n,
                                const int32_t *__restrict__ coff, int32_t *__restrict__ fill,
                                int32_t *__restrict__ qid) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= B * n) return;
  const int64_t q = t / n;
  const int r = (int)(t % n);
  const int c = probe[q * npr + r];
  const int slot = coff[c] + atomicAdd(&fill[c], 1);
  qid[slot] = (int32_t)(((uint32_t)q << 12) | (uint32_t)r);
}

// One block per cell: sort the cell's packed pairs by query (queries are unique within a cell, so
// the order equals the stable-sort order), unpack, and gather the pair constants.
__global__ __launch_bounds__(256) void k_pairs_sort(const int32_t *__restrict__ ccnt, const int32_t *__restrict__ coff,
                                                    const uint16_t *__restrict__ QM, const float *__restrict__ mnorm,
                                                    int NC, int32_t *__restrict__ qid, int32_t *__restrict__ qrank,
                                                    float *__restrict__ qcp) {
  __shared__ uint32_t s[kMaxCellPairs];
  const int c = blockIdx.x;
  const int cnt = ccnt[c];
  // cnt <= B <= kMaxCellPairs when probe rows hold distinct cells (as fvs_route_topk writes them);
  // a malformed probe with repeated cells is left unsorted rather than overrunning LDS.
  if (cnt == 0 || cnt > kMaxCellPairs) return;
  const int base = coff[c];
  const int P = fvs_pow2_ceil(cnt);
  for (int i = threadIdx.x; i < P; i += 256) s[i] = i < cnt ? (uint32_t)qid[base + i] : 0xffffffffu;
  __syncthreads();
  fvs_block_bitonic<uint32_t, false>(s, P);
  const float sc = mnorm ? mnorm[c] : 1.0f;
  for (int i = threadIdx.x; i < cnt; i += 256) {
    const uint32_t v = s[i];
    const int64_t q = v >> 12;
    qid[base + i] = (int32_t)q;
    qrank[base + i] = (int32_t)(v & 0xfffu);
    qcp[base + i] = fvs_h2f(QM[q * NC + c]) * sc;
  }
}

}  // namespace

extern "C" int fvs_route_topk(const uint16_t *QM, int64_t B, int32_t NC, int32_t nprobe, int32_t *probe, void *stream) {
  if (B < 0 || NC <= 0 || NC > 65536 || nprobe <= 0 || nprobe > NC) return FVS_E_ARG;
  if (nprobe > kMaxProbe) return FVS_E_CAPACITY;
  if (B == 0) return FVS_OK;
  if (!QM || !probe) return FVS_E_ARG;
  hipLaunchKernelGGL(k_route_topk, dim3((unsigned)B), dim3(256), 0, (hipStream_t)stream, QM, NC, nprobe, probe);
  return fvs_launch_status();
}

extern "C" int fvs_pairs(const int32_t *probe, int64_t B, int32_t npr, int32_t n, int32_t NC, const uint16_t *QM,
                         const float *mnorm, int32_t *ccnt, int32_t *coff, int32_t *fill, int32_t *qid,
                         int32_t *qrank, float *qcp, void *stream) {
  if (B < 0 || NC <= 0 || n <= 0 || n > npr || n > 4096) return FVS_E_ARG;
  if (B >= (1 << 20)) return FVS_E_ARG;
  if (B > kMaxCellPairs) return FVS_E_CAPACITY;  // a cell can be probed by every query
  if (!probe || !QM || !ccnt || !coff || !fill || !qid || !qrank || !qcp) return FVS_E_ARG;
  hipStream_t st = (hipStream_t)stream;
  int e = fvs_fill_u32(ccnt, NC, 0u, stream);
  if (e) return e;
  if (B == 0) {
    hipLaunchKernelGGL(k_pairs_scan, dim3(1), dim3(256), 0, st, ccnt, NC, coff, fill);
    return fvs_launch_status();
  }
  const int64_t tot = B * (int64_t)n;
  const unsigned g = (unsigned)((tot + 255) / 256);
  hipLaunchKernelGGL(k_pairs_count, dim3(g), dim3(256), 0, st, probe, B, npr, n, ccnt);
  if ((e = fvs_launch_status())) return e;
  hipLaunchKernelGGL(k_pairs_scan, dim3(1), dim3(256), 0, st, ccnt, NC, coff, fill);
  if ((e = fvs_launch_status())) return e;
  hipLaunchKernelGGL(k_pairs_scatter, dim3(g), dim3(256), 0, st, probe, B, npr, n, coff, fill, qid);
  if ((e = fvs_launch_status())) return e;
  hipLaunchKernelGGL(k_pairs_sort, dim3((unsigned)NC), dim3(256), 0, st, ccnt, coff, QM, mnorm, NC, qid, qrank, qcp);
  return fvs_launch_status();
}
