// Routing (top-n_p cells per query) and the (query, cell) pair lists grouped by cell.
//
// Routing: one wave per query (NC <= 8192, n_p <= 2048, NC a multiple of 8). The query's scores are
// held in registers as orderable 16-bit keys (8 per 16-byte load, cell = (chunk * 64 + lane) * 8 + e);
// a 16-step bisection over the key space finds the n_p-th largest score v* (a wave-sum of per-lane
// counts per step); every cell above v* plus the lowest-numbered cells equal to v* are compacted into
// a wave-private LDS list with wave prefix sums in cell order; the n_p selected keys
// (score << 16 | 0xffff - cell) are sorted by a bitonic network held in registers (element
// lane * R + r; partners within a lane are registers, the others one lane shuffle away). The wave
// never waits at a block barrier. Larger rows take the block-per-query kernel below, which stages
// the keys in LDS, finds v* with two 8-bit histogram passes and sorts in LDS.
//
// Pairs: instead of a global counting sort (atomics on popular cells serialise), the probe lists are
// transposed into a cell-major rank matrix rank[c][q] (int16, -1 = not probed) in caller scratch.
// Each cell's block then reads its row once to count and once to compact its queries in ascending
// order -- the order of the reference's stable sort -- with no atomics and no per-cell sort.
#include "fvs_common.h"

namespace {

constexpr int kMaxProbe = 4096;  // LDS capacity of the routing sort
constexpr int kMaxNC = 16384;    // LDS capacity of the routing key row

__device__ __forceinline__ int wave_hist_sum(int (*hist)[256], int b) {
  return hist[0][b] + hist[1][b] + hist[2][b] + hist[3][b];
}

__device__ __forceinline__ int wave_sum_i32(int v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, FVS_WAVE);
  return __builtin_amdgcn_readfirstlane(v);
}

__device__ __forceinline__ int wave_incl_scan_i32(int v, int lane) {
#pragma unroll
  for (int o = 1; o < FVS_WAVE; o <<= 1) {
    const int t = __shfl_up(v, o, FVS_WAVE);
    if (lane >= o) v += t;
  }
  return v;
}

__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

constexpr int kRouteWaves = 4;  // queries per block

// C: 16-byte chunks of 8 scores per lane (NC <= 512 C); R: sorted keys per lane (n_p <= 64 R).
template <int C, int R>
__global__ __launch_bounds__(kRouteWaves * FVS_WAVE) void k_route_wave(const uint16_t *__restrict__ QM, int NC,
                                                                      int np, int64_t B,
                                                                      int32_t *__restrict__ probe) {
  __shared__ uint32_t sbuf[kRouteWaves][FVS_WAVE * R];
  const int lane = threadIdx.x & (FVS_WAVE - 1), wv = threadIdx.x >> 6;
  const int64_t q = (int64_t)blockIdx.x * kRouteWaves + wv;
  if (q >= B) return;  // wave-uniform, and no block barrier follows
  uint32_t *s = sbuf[wv];
  const uint4 *row = reinterpret_cast<const uint4 *>(QM + q * (int64_t)NC);

  // 1. keys; cells past NC get key 0 and are excluded below by their index
  uint32_t k[8 * C];
#pragma unroll
  for (int c = 0; c < C; c++) {
    const int ch = c * FVS_WAVE + lane;
    const uint4 v = ch * 8 < NC ? row[ch] : make_uint4(0, 0, 0, 0);
    const uint32_t w4[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int u = 0; u < 4; u++) {
      k[8 * c + 2 * u] = ch * 8 < NC ? fvs_ord16((uint16_t)(w4[u] & 0xffffu)) : 0u;
      k[8 * c + 2 * u + 1] = ch * 8 < NC ? fvs_ord16((uint16_t)(w4[u] >> 16)) : 0u;
    }
  }

  // 2. v* = the largest t with #{keys >= t} >= n_p (bit by bit from the top; candidates t >= 1 never
  //    count the padding, and t = 0 leaves all NC >= n_p cells)
  uint32_t vstar = 0;
#pragma unroll 1
  for (int bit = 15; bit >= 0; bit--) {
    const uint32_t cand = vstar | (1u << bit);
    int cnt = 0;
#pragma unroll
    for (int i = 0; i < 8 * C; i++) cnt += k[i] >= cand ? 1 : 0;
    if (wave_sum_i32(cnt) >= np) vstar = cand;
  }
  int gt = 0;
#pragma unroll
  for (int i = 0; i < 8 * C; i++) gt += k[i] > vstar ? 1 : 0;
  const int want = np - wave_sum_i32(gt);  // ties taken, lowest cells first

  // 3. compaction in cell order: (score << 16) | (0xffff - cell) for the n_p selected cells
  int sbase = 0, tbase = 0;
#pragma unroll
  for (int c = 0; c < C; c++) {
    const int ch = c * FVS_WAVE + lane;
    const bool ok = ch * 8 < NC;
    int nt = 0;
#pragma unroll
    for (int e = 0; e < 8; e++) nt += (ok && k[8 * c + e] == vstar) ? 1 : 0;
    const int tin = wave_incl_scan_i32(nt, lane);
    int tie = tbase + tin - nt;  // ties in lower cells
    uint32_t selm = 0;
#pragma unroll
    for (int e = 0; e < 8; e++) {
      const uint32_t x = k[8 * c + e];
      const bool eq = ok && x == vstar;
      const bool sel = ok && (x > vstar || (eq && tie < want));
      tie += eq ? 1 : 0;
      selm |= sel ? (1u << e) : 0u;
    }
    const int ns = __builtin_popcount(selm);
    const int sin = wave_incl_scan_i32(ns, lane);
    int at = sbase + sin - ns;
#pragma unroll
    for (int e = 0; e < 8; e++) {
      if (selm & (1u << e)) s[at++] = (k[8 * c + e] << 16) | (0xffffu - (uint32_t)(ch * 8 + e));
    }
    sbase += __builtin_amdgcn_readlane(sin, FVS_WAVE - 1);
    tbase += __builtin_amdgcn_readlane(tin, FVS_WAVE - 1);
  }
  for (int i = np + lane; i < FVS_WAVE * R; i += FVS_WAVE) s[i] = 0u;  // below every selected key
  wave_lds_sync();

  // 4. bitonic sort, descending, of element lane * R + r
  uint32_t x[R];
#pragma unroll
  for (int r = 0; r < R; r++) x[r] = s[lane * R + r];
#pragma unroll
  for (int kk = 2; kk <= FVS_WAVE * R; kk <<= 1) {
#pragma unroll
    for (int j = kk >> 1; j > 0; j >>= 1) {
      if (j >= R) {
        const int lo = lane * R;
        const bool desc = (lo & kk) == 0, first = (lo & j) == 0;
#pragma unroll
        for (int r = 0; r < R; r++) {
          const uint32_t y = __shfl_xor(x[r], j / R, FVS_WAVE);
          x[r] = (desc == first) ? max(x[r], y) : min(x[r], y);
        }
      } else {
#pragma unroll
        for (int r = 0; r < R; r++) {
          if ((r & j) == 0) {
            const bool desc = ((lane * R + r) & kk) == 0;
            const uint32_t a = x[r], b = x[r | j];
            const uint32_t hi = max(a, b), lo = min(a, b);
            x[r] = desc ? hi : lo;
            x[r | j] = desc ? lo : hi;
          }
        }
      }
    }
  }
  int32_t *out = probe + q * (int64_t)np;
#pragma unroll
  for (int r = 0; r < R; r++) {
    const int i = lane * R + r;
    if (i < np) out[i] = (int32_t)(0xffffu - (x[r] & 0xffffu));
  }
}

template <int C, int R>
int launch_route_wave(const uint16_t *QM, int64_t B, int NC, int np, int32_t *probe, hipStream_t st) {
  const unsigned grid = (unsigned)((B + kRouteWaves - 1) / kRouteWaves);
  hipLaunchKernelGGL((k_route_wave<C, R>), dim3(grid), dim3(kRouteWaves * FVS_WAVE), 0, st, QM, NC, np, B, probe);
  return fvs_launch_status();
}

template <int C>
int route_wave_r(const uint16_t *QM, int64_t B, int NC, int np, int32_t *probe, hipStream_t st) {
  if (np <= 64) return launch_route_wave<C, 1>(QM, B, NC, np, probe, st);
  if (np <= 128) return launch_route_wave<C, 2>(QM, B, NC, np, probe, st);
  if (np <= 256) return launch_route_wave<C, 4>(QM, B, NC, np, probe, st);
  if (np <= 512) return launch_route_wave<C, 8>(QM, B, NC, np, probe, st);
  if (np <= 1024) return launch_route_wave<C, 16>(QM, B, NC, np, probe, st);
  return launch_route_wave<C, 32>(QM, B, NC, np, probe, st);
}

__global__ __launch_bounds__(256) void k_route_topk(const uint16_t *__restrict__ QM, int NC, int np,
                                                    int32_t *__restrict__ probe) {
  __shared__ uint16_t v[kMaxNC];
  __shared__ uint32_t s[kMaxProbe];
  __shared__ int hist[4][256];
  __shared__ int sh[16];
  __shared__ int cnt;
  const int64_t q = blockIdx.x;
  const int tid = threadIdx.x, w = tid >> 6;
  const uint16_t *row = QM + q * NC;
  for (int i = tid; i < NC; i += 256) v[i] = (uint16_t)fvs_ord16(row[i]);
  int want = np;
  uint32_t prefix = 0;
  for (int pass = 0; pass < 2; pass++) {
    for (int i = tid; i < 4 * 256; i += 256) (&hist[0][0])[i] = 0;
    __syncthreads();
    for (int i = tid; i < NC; i += 256) {
      const uint32_t x = v[i];
      if (pass == 0)
        atomicAdd(&hist[w][x >> 8], 1);
      else if ((x >> 8) == prefix)
        atomicAdd(&hist[w][x & 255], 1);
    }
    __syncthreads();
    const int b = 255 - tid;
    const int h = wave_hist_sum(hist, b);
    const int inc = fvs_block_scan256(h, sh);
    const int exc = inc - h;
    if (exc < want && want <= inc) {
      sh[8] = b;
      sh[9] = want - exc;
    }
    __syncthreads();
    prefix = pass == 0 ? (uint32_t)sh[8] : ((prefix << 8) | (uint32_t)sh[8]);
    want = sh[9];
    __syncthreads();
  }
  const uint32_t vstar = prefix;  // the n_p-th largest key; `want` of its ties are taken
  if (tid == 0) cnt = 0;
  __syncthreads();
  int run = 0;  // ties already taken, in cell order
  for (int base = 0; base < NC; base += 256) {
    const int i = base + tid;
    const uint32_t x = i < NC ? (uint32_t)v[i] : 0u;
    const bool gt = i < NC && x > vstar;
    const bool eq = i < NC && x == vstar;
    if (gt) s[atomicAdd(&cnt, 1)] = (x << 16) | (0xffffu - (uint32_t)i);
    const int neq = __syncthreads_count(eq);
    if (neq > 0 && run < want) {
      const int rk = fvs_block_scan256(eq ? 1 : 0, sh) - 1;
      if (eq && run + rk < want) s[atomicAdd(&cnt, 1)] = (x << 16) | (0xffffu - (uint32_t)i);
    }
    run += neq;
  }
  __syncthreads();
  const int P = fvs_pow2_ceil(np);
  for (int i = np + tid; i < P; i += 256) s[i] = 0u;
  __syncthreads();
  fvs_block_bitonic<uint32_t, true>(s, P);
  for (int i = tid; i < np; i += 256) probe[q * np + i] = (int32_t)(0xffffu - (s[i] & 0xffffu));
}

// rank[c][q] = r for the first n probe columns (the matrix is pre-filled with 0xffff).
__global__ void k_rank_scatter(const int32_t *__restrict__ probe, int64_t B, int npr, int n, uint16_t *__restrict__ rank) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= B * n) return;
  const int64_t q = t / n;
  const int r = (int)(t % n);
  rank[(int64_t)probe[q * npr + r] * B + q] = (uint16_t)r;
}

// ccnt[c] = number of queries probing cell c.
__global__ __launch_bounds__(256) void k_cell_count(const uint16_t *__restrict__ rank, int64_t B,
                                                    int32_t *__restrict__ ccnt) {
  __shared__ int sh[8];
  const int c = blockIdx.x;
  const uint16_t *rr = rank + (int64_t)c * B;
  int m = 0;
  for (int64_t q = threadIdx.x; q < B; q += 256) m += rr[q] != 0xffffu;
  const int tot = fvs_block_scan256(m, sh);
  if (threadIdx.x == 255) ccnt[c] = tot;
}

// Exclusive prefix sum of ccnt into coff. One block of 256 threads.
__global__ __launch_bounds__(256) void k_cell_scan(const int32_t *__restrict__ ccnt, int NC, int32_t *__restrict__ coff) {
  __shared__ int tmp[8];
  int run = 0;
  for (int base = 0; base < NC; base += 256) {
    const int c = base + (int)threadIdx.x;
    const int v = c < NC ? ccnt[c] : 0;
    const int inc = fvs_block_scan256(v, tmp);
    if (c < NC) coff[c] = run + inc - v;
    if (threadIdx.x == 255) tmp[4] = inc;
    __syncthreads();
    run += tmp[4];
    __syncthreads();
  }
}

// One block per cell: its queries in ascending order, their probe ranks and pair constants.
__global__ __launch_bounds__(256) void k_cell_emit(const uint16_t *__restrict__ rank, int64_t B,
                                                   const int32_t *__restrict__ coff, const uint16_t *__restrict__ QM,
                                                   const float *__restrict__ mnorm, const float *__restrict__ qadd,
                                                   int NC, int32_t *__restrict__ qid,
                                                   int32_t *__restrict__ qrank, float *__restrict__ qcp) {
  __shared__ int sh[8];
  const int c = blockIdx.x;
  const uint16_t *rr = rank + (int64_t)c * B;
  const float sc = mnorm ? mnorm[c] : 1.0f;
  int run = coff[c];
  for (int64_t base = 0; base < B; base += 256) {
    const int64_t q = base + threadIdx.x;
    const uint16_t r = q < B ? rr[q] : (uint16_t)0xffffu;
    const bool f = r != 0xffffu;
    const int inc = fvs_block_scan256(f ? 1 : 0, sh);
    if (f) {
      const int o = run + inc - 1;
      qid[o] = (int32_t)q;
      qrank[o] = (int32_t)r;
      const float v = fvs_h2f(QM[q * NC + c]) * sc;
      qcp[o] = qadd ? v + qadd[q] : v;
    }
    if (threadIdx.x == 255) sh[6] = inc;
    __syncthreads();
    run += sh[6];
    __syncthreads();
  }
}

}  // namespace

extern "C" int fvs_route_topk(const uint16_t *QM, int64_t B, int32_t NC, int32_t nprobe, int32_t *probe, void *stream) {
  if (B < 0 || NC <= 0 || nprobe <= 0 || nprobe > NC) return FVS_E_ARG;
  if (nprobe > kMaxProbe || NC > kMaxNC) return FVS_E_CAPACITY;
  if (B == 0) return FVS_OK;
  if (!QM || !probe) return FVS_E_ARG;
  hipStream_t st = (hipStream_t)stream;
  if (NC % 8 == 0 && nprobe <= 2048 && (reinterpret_cast<uintptr_t>(QM) & 15) == 0) {
    if (NC <= 4096) return route_wave_r<8>(QM, B, NC, nprobe, probe, st);
    if (NC <= 8192) return route_wave_r<16>(QM, B, NC, nprobe, probe, st);
  }
  hipLaunchKernelGGL(k_route_topk, dim3((unsigned)B), dim3(256), 0, st, QM, NC, nprobe, probe);
  return fvs_launch_status();
}

extern "C" int64_t fvs_pairs_scratch_bytes(int64_t B, int32_t NC) {
  if (B < 0 || NC <= 0) return -1;
  return ((int64_t)NC * B * 2 + 255) / 256 * 256;
}

extern "C" int fvs_pairs(const int32_t *probe, int64_t B, int32_t npr, int32_t n, int32_t NC, const uint16_t *QM,
                         const float *mnorm, const float *qadd, int32_t *ccnt, int32_t *coff, void *scratch,
                         int64_t scratch_bytes,
                         int32_t *qid, int32_t *qrank, float *qcp, void *stream) {
  if (B < 0 || NC <= 0 || n <= 0 || n > npr || n > 65535) return FVS_E_ARG;
  if (scratch_bytes < fvs_pairs_scratch_bytes(B, NC)) return FVS_E_CAPACITY;
  if (!probe || !QM || !ccnt || !coff || !scratch || !qid || !qrank || !qcp) return FVS_E_ARG;
  hipStream_t st = (hipStream_t)stream;
  uint16_t *rank = reinterpret_cast<uint16_t *>(scratch);
  int e;
  if (B > 0) {
    if ((e = fvs_fill_u32(rank, ((int64_t)NC * B * 2 + 3) / 4, 0xffffffffu, stream))) return e;
    const int64_t tot = B * (int64_t)n;
    hipLaunchKernelGGL(k_rank_scatter, dim3((unsigned)((tot + 255) / 256)), dim3(256), 0, st, probe, B, npr, n, rank);
    if ((e = fvs_launch_status())) return e;
  }
  hipLaunchKernelGGL(k_cell_count, dim3((unsigned)NC), dim3(256), 0, st, rank, B, ccnt);
  if ((e = fvs_launch_status())) return e;
  hipLaunchKernelGGL(k_cell_scan, dim3(1), dim3(256), 0, st, ccnt, NC, coff);
  if ((e = fvs_launch_status())) return e;
  hipLaunchKernelGGL(k_cell_emit, dim3((unsigned)NC), dim3(256), 0, st, rank, B, coff, QM, mnorm, qadd, NC, qid, qrank, qcp);
  return fvs_launch_status();
}
