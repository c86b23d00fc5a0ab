// Error-bar classification, exact scoring of the ambiguous candidates and the final top-k.
//
// One block (4 waves) per query. The two order statistics (k+1-th largest upper bound, k-th
// largest lower bound) come from radix selects; the ambiguous slots are compacted in LDS and the
// waves take them round-robin, each wave reading one fp16 row (coalesced 16-byte lane loads, from
// HBM or from pinned host memory over PCIe) and reducing with a fixed butterfly.
#include "fvs_common.h"

namespace {

constexpr int kMaxK = 4096;
constexpr int kMaxk = 1024;

__global__ __launch_bounds__(256) void k_refine(const float *__restrict__ est, const float *__restrict__ sd,
                                                const int32_t *__restrict__ pos, const int32_t *__restrict__ order,
                                                const uint16_t *__restrict__ H, const float *__restrict__ Q, int K,
                                                int d, float z, int k, int32_t *__restrict__ ids,
                                                int32_t *__restrict__ Iout, float *__restrict__ scores,
                                                int32_t *__restrict__ reads) {
  __shared__ float score[kMaxK];
  __shared__ uint8_t flag[kMaxK];  // 1 sure, 2 ambiguous
  __shared__ int16_t amb[kMaxK];
  __shared__ uint64_t s[kMaxk];
  __shared__ int hist[256];
  __shared__ int sh[8];
  __shared__ int namb, gcnt;

  const int64_t q = blockIdx.x;
  const float *e = est + q * (int64_t)K;
  const float *g = sd + q * (int64_t)K;
  auto lo = [&](int i) -> float { return e[i] - z * g[i]; };
  auto hi = [&](int i) -> float { return e[i] + z * g[i]; };

  const float hk1 = fvs_unord32(fvs_block_kth<uint32_t>([&](int i) { return fvs_ord32(hi(i)); }, K, k + 1, hist, sh));
  const float lk = fvs_unord32(fvs_block_kth<uint32_t>([&](int i) { return fvs_ord32(lo(i)); }, K, k, hist, sh));

  if (threadIdx.x == 0) namb = 0;
  __syncthreads();
  for (int i = threadIdx.x; i < K; i += 256) {
    const float l = lo(i), h = hi(i);
    const bool sure = l > hk1;
    const bool am = (h >= lk) && !sure;
    flag[i] = sure ? 1 : (am ? 2 : 0);
    score[i] = sure ? e[i] + 10.0f : -1e9f;
    ids[q * (int64_t)K + i] = order[pos[q * (int64_t)K + i]];
    if (am) amb[atomicAdd(&namb, 1)] = (int16_t)i;
  }
  __syncthreads();

  // exact scores of the ambiguous candidates
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const float *qr = Q + q * (int64_t)d;
  const int ng = d / 8;
  for (int a = w; a < namb; a += 4) {
    const int slot = amb[a];
    const int64_t id = order[pos[q * (int64_t)K + slot]];
    const uint4 *hr = reinterpret_cast<const uint4 *>(H + id * d);
    float acc = 0.f;
    for (int gi = lane; gi < ng; gi += 64) {
      const uint4 hv = hr[gi];
      const uint32_t hw[4] = {hv.x, hv.y, hv.z, hv.w};
      const float *qg = qr + 8 * gi;
#pragma unroll
      for (int u = 0; u < 4; u++) {
        acc = __builtin_fmaf(fvs_h2f((uint16_t)(hw[u] & 0xffffu)), qg[2 * u], acc);
        acc = __builtin_fmaf(fvs_h2f((uint16_t)(hw[u] >> 16)), qg[2 * u + 1], acc);
      }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) acc += __shfl_xor(acc, o, FVS_WAVE);
    if (lane == 0) score[slot] = acc;
  }
  __syncthreads();
  if (threadIdx.x == 0) reads[q] = namb;

  // final top-k by (score descending, slot ascending)
  auto key = [&](int i) -> uint64_t {
    return ((uint64_t)fvs_ord32(score[i]) << 32) | (uint64_t)(0xffffffffu - (uint32_t)i);
  };
  fvs_block_topk_u64(key, K, k, s, hist, sh, &gcnt);
  for (int j = threadIdx.x; j < k; j += 256) {
    const int slot = (int)(0xffffffffu - (uint32_t)(s[j] & 0xffffffffu));
    Iout[q * (int64_t)k + j] = order[pos[q * (int64_t)K + slot]];
    scores[q * (int64_t)k + j] = flag[slot] == 1 ? e[slot] : score[slot];
  }
}

}  // namespace

extern "C" int fvs_refine(const float *est, const float *sd, const int32_t *pos, const int32_t *order,
                          const uint16_t *H, const float *Q, int64_t B, int32_t K, int32_t d, float z, int32_t k,
                          int32_t *ids, int32_t *I, float *scores, int32_t *reads, void *stream) {
  if (B < 0 || k <= 0 || K <= k || d <= 0 || d % 8 != 0 || !(z >= 0.f)) return FVS_E_ARG;
  if (K > kMaxK || k > kMaxk) return FVS_E_CAPACITY;
  if (B == 0) return FVS_OK;
  if (!est || !sd || !pos || !order || !H || !Q || !ids || !I || !scores || !reads) return FVS_E_ARG;
  hipLaunchKernelGGL(k_refine, dim3((unsigned)B), dim3(256), 0, (hipStream_t)stream, est, sd, pos, order, H, Q, K, d,
                     z, k, ids, I, scores, reads);
  return fvs_launch_status();
}
