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
// the keys in LDS, finds v* with two 8-bit histogram passes and sorts in LDS. Routing on fp32 keys
// (fvs_route_topk_scaled, the trellis engine's scaled cell scores) follows the same two designs with
// 32-bit keys, a 32-step bisection and (key, cell) pairs sorted as 64-bit values.
//
// Pairs: instead of a global counting sort (atomics on popular cells serialise), the probe lists are
// transposed into a cell-major rank matrix rank[c][q] (int16, -1 = not probed) in caller scratch.
// The same pass copies each query's routing scores into a cell-major score matrix, so that the pair
// constants are read row-wise, and adds each tile's per-cell counts to the cell totals (one integer
// atomic per tile and cell). After a one-block scan of the totals, one wave per cell reads its rank and
// score rows once to compact its queries in ascending order -- the order of the reference's stable
// sort -- with no per-pair atomics, no per-cell sort and no column gathers. The first-pass list (the
// first n1 probe columns) and the full list come out of one matrix (fvs_pairs2).
#include <mutex>

#include "fvs_common.h"

// The allocation-free pair builder's scratch (fvs_pairs_noalloc): the rank and score matrices live in
// this file-scope device array instead of a caller buffer. Each device that runs the library holds its
// own copy until the process ends; host code reaches it only through the per-device address that
// hipGetSymbolAddress returns (the array's name is not a device address on the host).
static __device__ __align__(256) uint8_t scratch[FVS_PAIRS_NOALLOC_SCRATCH];

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
  const int lane = threadIdx.x & (FVS_WAVE - 1), wv = fvs_wave_id();
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
          const uint32_t y = fvs_xor_lane(x[r], j / R);
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

// ------------------------------------------------------------------------------------ routing
// Top-n_p cells by the fp32 key (float)QM[q][c] * scale[c] (or ((float)QM[q][c] + qadd[q]) * scale[c]),
// sorted by (key descending, cell ascending).
__global__ __launch_bounds__(256) void k_route_f32(const uint16_t *__restrict__ QM, const float *__restrict__ scale,
                                                   const float *__restrict__ qadd, int NC, int np,
                                                   int32_t *__restrict__ probe) {
  extern __shared__ uint64_t rk[];  // [NC] keys, then [pow2(np)] the sorted top
  __shared__ int hist[256];
  __shared__ int sh[8];
  __shared__ int gcnt;
  const int64_t q = blockIdx.x;
  uint64_t *top = rk + NC;
  const float add = qadd ? qadd[q] : 0.f;
  for (int i = threadIdx.x; i < NC; i += 256) {
    const float key = qadd ? (fvs_h2f(QM[q * NC + i]) + add) * scale[i] : fvs_h2f(QM[q * NC + i]) * scale[i];
    rk[i] = ((uint64_t)fvs_ord32(key) << 32) | (uint64_t)(0xffffffffu - (uint32_t)i);
  }
  __syncthreads();
  fvs_block_topk_u64([&](int i) { return rk[i]; }, NC, np, top, hist, sh, &gcnt);
  for (int i = threadIdx.x; i < np; i += 256) probe[q * np + i] = (int32_t)(0xffffffffu - (uint32_t)(top[i] & 0xffffffffu));
}

// The same selection with one wave per query (fvs_route_topk_scaled when NC % 8 == 0, NC <= 8192 and
// n_p <= 1024): 32-bit ordered keys in registers, v* = the n_p-th largest by bisection over the 32 bits,
// ties at v* taken lowest cells first, then a bitonic sort of the (key << 32 | ~cell) pairs, n_p <= 64 R.
template <int C, int R, bool ADD>
__global__ __launch_bounds__(kRouteWaves * FVS_WAVE) void k_route_wave_f32(const uint16_t *__restrict__ QM,
                                                                          const float *__restrict__ scale,
                                                                          const float *__restrict__ qadd, int NC,
                                                                          int np, int64_t B,
                                                                          int32_t *__restrict__ probe) {
  __shared__ uint64_t sbuf[kRouteWaves][FVS_WAVE * R];
  const int lane = threadIdx.x & (FVS_WAVE - 1), wv = fvs_wave_id();
  const int64_t q = (int64_t)blockIdx.x * kRouteWaves + wv;
  if (q >= B) return;  // wave-uniform, and no block barrier follows
  uint64_t *s = sbuf[wv];
  const uint4 *row = reinterpret_cast<const uint4 *>(QM + q * (int64_t)NC);
  const float4 *sc4 = reinterpret_cast<const float4 *>(scale);
  const float add = ADD ? qadd[q] : 0.f;

  // 1. keys, computed as in k_route_f32; cells past NC get key 0 and are excluded by their index
  uint32_t k[8 * C];
#pragma unroll
  for (int c = 0; c < C; c++) {
    const int ch = c * FVS_WAVE + lane;
    const bool ok = ch * 8 < NC;
    const uint4 v = ok ? row[ch] : make_uint4(0, 0, 0, 0);
    const float4 s0 = ok ? sc4[2 * ch] : make_float4(0.f, 0.f, 0.f, 0.f);
    const float4 s1 = ok ? sc4[2 * ch + 1] : make_float4(0.f, 0.f, 0.f, 0.f);
    const uint32_t w4[4] = {v.x, v.y, v.z, v.w};
    const float sc[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
#pragma unroll
    for (int e = 0; e < 8; e++) {
      float x = fvs_h2f((uint16_t)((e & 1) ? (w4[e >> 1] >> 16) : (w4[e >> 1] & 0xffffu)));
      if (ADD) x = x + add;
      x = x * sc[e];
      k[8 * c + e] = ok ? fvs_ord32(x) : 0u;
    }
  }

  // 2. v* = the largest t with #{keys >= t} >= n_p
  uint32_t vstar = 0;
#pragma unroll 1
  for (int bit = 31; bit >= 0; bit--) {
    const uint32_t cand = vstar | (1u << bit);
    int cnt = 0;
#pragma unroll
    for (int i = 0; i < 8 * C; i++) cnt += k[i] >= cand ? 1 : 0;
    if (wave_sum_i32(cnt) >= np) vstar = cand;
  }
  int gt = 0;
#pragma unroll
  for (int i = 0; i < 8 * C; i++) gt += k[i] > vstar ? 1 : 0;
  const int want = np - wave_sum_i32(gt);

  // 3. compaction in cell order
  int sbase = 0, tbase = 0;
#pragma unroll
  for (int c = 0; c < C; c++) {
    const int ch = c * FVS_WAVE + lane;
    const bool ok = ch * 8 < NC;
    int nt = 0;
#pragma unroll
    for (int e = 0; e < 8; e++) nt += (ok && k[8 * c + e] == vstar) ? 1 : 0;
    const int tin = wave_incl_scan_i32(nt, lane);
    int tie = tbase + tin - nt;
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
      if (selm & (1u << e))
        s[at++] = ((uint64_t)k[8 * c + e] << 32) | (uint64_t)(0xffffffffu - (uint32_t)(ch * 8 + e));
    }
    sbase += __builtin_amdgcn_readlane(sin, FVS_WAVE - 1);
    tbase += __builtin_amdgcn_readlane(tin, FVS_WAVE - 1);
  }
  for (int i = np + lane; i < FVS_WAVE * R; i += FVS_WAVE) s[i] = 0ull;  // below every selected pair
  wave_lds_sync();

  // 4. bitonic sort, descending, of element lane * R + r
  uint64_t x[R];
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
          const uint64_t y = fvs_shfl_xor_u64(x[r], j / R);
          x[r] = (desc == first) ? (x[r] > y ? x[r] : y) : (x[r] < y ? x[r] : y);
        }
      } else {
#pragma unroll
        for (int r = 0; r < R; r++) {
          if ((r & j) == 0) {
            const bool desc = ((lane * R + r) & kk) == 0;
            const uint64_t a = x[r], b = x[r | j];
            const uint64_t hi = a > b ? a : b, lo = a < b ? a : b;
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
    if (i < np) out[i] = (int32_t)(0xffffffffu - (uint32_t)(x[r] & 0xffffffffu));
  }
}

// The same selection with one 1024-thread block per query, for small batches (fvs_route_topk_scaled when
// NC % 8 == 0, NC <= 8192, n_p <= 1024 and B <= kRouteBlkMaxB). Thread t holds the keys of cells
// [KPT t, KPT t + KPT) in registers; v* = the n_p-th largest key comes from an MSD radix select over
// 8-bit digits with one LDS histogram per wave (so same-bucket atomics of different waves do not
// collide), stopped early when the chosen bucket is taken whole; ties at v* are taken lowest cells first
// by a block prefix sum in cell order. The n_p selected (key << 32 | ~cell) pairs are compacted into LDS
// and each is stored at its rank among them (a count of the larger pairs).
constexpr int kRouteBlk = 1024;
constexpr int kRouteBlkMaxB = 256;

template <int KPT, bool ADD>
__global__ __launch_bounds__(kRouteBlk) void k_route_blk_f32(const uint16_t *__restrict__ QM,
                                                            const float *__restrict__ scale,
                                                            const float *__restrict__ qadd, int NC, int np,
                                                            int32_t *__restrict__ probe) {
  constexpr int NW = kRouteBlk / FVS_WAVE;
  __shared__ int hist[NW][256];
  __shared__ uint64_t s[1024];
  __shared__ int wsum[NW];
  __shared__ int sh[4];
  const int tid = threadIdx.x, lane = tid & (FVS_WAVE - 1), wv = fvs_wave_id();
  const int64_t q = blockIdx.x;
  const int c0 = tid * KPT;
  const float add = ADD ? qadd[q] : 0.f;

  // 1. keys, computed as in k_route_f32; cells past NC get key 0 and are never selected
  uint32_t k[KPT];
  {
    uint16_t hv[KPT];
    float sc[KPT];
    if (c0 < NC) {
      if constexpr (KPT == 4) {
        const uint2 v = *reinterpret_cast<const uint2 *>(QM + q * (int64_t)NC + c0);
        const float4 f = *reinterpret_cast<const float4 *>(scale + c0);
        hv[0] = (uint16_t)(v.x & 0xffffu); hv[1] = (uint16_t)(v.x >> 16);
        hv[2] = (uint16_t)(v.y & 0xffffu); hv[3] = (uint16_t)(v.y >> 16);
        sc[0] = f.x; sc[1] = f.y; sc[2] = f.z; sc[3] = f.w;
      } else {
        const uint4 v = *reinterpret_cast<const uint4 *>(QM + q * (int64_t)NC + c0);
        const float4 f0 = *reinterpret_cast<const float4 *>(scale + c0);
        const float4 f1 = *reinterpret_cast<const float4 *>(scale + c0 + 4);
        const uint32_t w4[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int e = 0; e < 8; e++) hv[e] = (uint16_t)((e & 1) ? (w4[e >> 1] >> 16) : (w4[e >> 1] & 0xffffu));
        sc[0] = f0.x; sc[1] = f0.y; sc[2] = f0.z; sc[3] = f0.w;
        sc[4] = f1.x; sc[5] = f1.y; sc[6] = f1.z; sc[7] = f1.w;
      }
    }
#pragma unroll
    for (int e = 0; e < KPT; e++) {
      float x = c0 < NC ? fvs_h2f(hv[e]) : 0.f;
      if (ADD) x = x + add;
      x = x * (c0 < NC ? sc[e] : 0.f);
      k[e] = c0 < NC ? fvs_ord32(x) : 0u;
    }
  }

  // 2. radix select: after the loop, the selected keys are those with (key & mask) > prefix, plus, with
  //    (key & mask) == prefix, all of them (whole) or the `want` lowest cells
  uint32_t prefix = 0, mask = 0;
  int want = np;
  bool whole = false;
  for (int shift = 24; shift >= 0; shift -= 8) {
    for (int i = tid; i < NW * 256; i += kRouteBlk) (&hist[0][0])[i] = 0;
    __syncthreads();
#pragma unroll
    for (int e = 0; e < KPT; e++)
      if (c0 + e < NC && (k[e] & mask) == prefix) atomicAdd(&hist[wv][(k[e] >> shift) & 0xff], 1);
    __syncthreads();
    int h = 0, inc = 0;
    if (tid < 256) {  // thread order = descending digit 255 - tid; waves 0..3
#pragma unroll
      for (int j = 0; j < NW; j++) h += hist[j][255 - tid];
      inc = wave_incl_scan_i32(h, lane);
      if (lane == FVS_WAVE - 1) wsum[wv] = inc;
    }
    __syncthreads();
    if (tid < 256) {
      int before = 0;
      for (int j = 0; j < wv; j++) before += wsum[j];
      const int hi = before + inc, lo = hi - h;
      if (lo < want && want <= hi) {
        sh[0] = 255 - tid;
        sh[1] = want - lo;
        sh[2] = h;
      }
    }
    __syncthreads();
    prefix |= (uint32_t)sh[0] << shift;
    mask |= 0xffu << shift;
    want = sh[1];
    whole = sh[2] == want;
    if (whole) break;  // uniform: every thread read the same sh
  }

  // 3. ties in cell order (only when the last bucket is not taken whole)
  int tie0 = 0;
  if (!whole) {
    int nt = 0;
#pragma unroll
    for (int e = 0; e < KPT; e++) nt += (c0 + e < NC && k[e] == prefix) ? 1 : 0;
    const int inc = wave_incl_scan_i32(nt, lane);
    if (lane == FVS_WAVE - 1) wsum[wv] = inc;
    __syncthreads();
    int before = 0;
    for (int j = 0; j < wv; j++) before += wsum[j];
    tie0 = before + inc - nt;
  }

  // 4. compaction
  if (tid == 0) sh[3] = 0;
  __syncthreads();
#pragma unroll
  for (int e = 0; e < KPT; e++) {
    const uint32_t x = k[e] & mask;
    const bool eq = c0 + e < NC && x == prefix;
    const bool sel = c0 + e < NC && (x > prefix || (eq && (whole || tie0 < want)));
    tie0 += (eq && !whole) ? 1 : 0;
    if (sel) {
      const int slot = atomicAdd(&sh[3], 1);  // exactly n_p <= 1024 keys are selected
      if (slot < 1024) s[slot] = ((uint64_t)k[e] << 32) | (uint64_t)(0xffffffffu - (uint32_t)(c0 + e));
    }
  }
  __syncthreads();

  // 5. rank of each selected pair among them (keys are unique), one pair per thread
  if (tid < np) {
    const uint64_t mine = s[tid];
    int rank = 0;
    for (int j = 0; j < np; j++) rank += s[j] > mine ? 1 : 0;  // one address per wave: a broadcast read
    probe[q * (int64_t)np + rank] = (int32_t)(0xffffffffu - (uint32_t)(mine & 0xffffffffu));
  }
}

template <int C, int R>
int launch_route_wave_f32(const uint16_t *QM, const float *scale, const float *qadd, int64_t B, int NC, int np,
                          int32_t *probe, hipStream_t st) {
  const unsigned grid = (unsigned)((B + kRouteWaves - 1) / kRouteWaves);
  if (qadd)
    hipLaunchKernelGGL((k_route_wave_f32<C, R, true>), dim3(grid), dim3(kRouteWaves * FVS_WAVE), 0, st, QM, scale,
                       qadd, NC, np, B, probe);
  else
    hipLaunchKernelGGL((k_route_wave_f32<C, R, false>), dim3(grid), dim3(kRouteWaves * FVS_WAVE), 0, st, QM, scale,
                       qadd, NC, np, B, probe);
  return fvs_launch_status();
}

template <int C>
int route_wave_f32_r(const uint16_t *QM, const float *scale, const float *qadd, int64_t B, int NC, int np,
                     int32_t *probe, hipStream_t st) {
  if (np <= 64) return launch_route_wave_f32<C, 1>(QM, scale, qadd, B, NC, np, probe, st);
  if (np <= 128) return launch_route_wave_f32<C, 2>(QM, scale, qadd, B, NC, np, probe, st);
  if (np <= 256) return launch_route_wave_f32<C, 4>(QM, scale, qadd, B, NC, np, probe, st);
  if (np <= 512) return launch_route_wave_f32<C, 8>(QM, scale, qadd, B, NC, np, probe, st);
  return launch_route_wave_f32<C, 16>(QM, scale, qadd, B, NC, np, probe, st);
}

__global__ __launch_bounds__(256) void k_route_topk(const uint16_t *__restrict__ QM, int NC, int np,
                                                    int32_t *__restrict__ probe) {
  __shared__ uint16_t v[kMaxNC];
  __shared__ uint32_t s[kMaxProbe];
  __shared__ int hist[4][256];
  __shared__ int sh[16];
  __shared__ int cnt;
  const int64_t q = blockIdx.x;
  const int tid = threadIdx.x, w = fvs_wave_id();
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
// Rank and score matrices, row pitch Bp = B rounded up to 64 (one 128-byte line per 64 queries):
// rank[c * Bp + q] = rank of cell c in query q's probe row (first n columns), 0xffff when q does not probe
// c; score[c * Bp + q] = QM[q][c] (fp16 bits). One block per (64 queries, kTileC cells): the block's
// probe entries inside its cell range are scattered into an LDS rank tile and its scores are read
// row-wise into an LDS score tile (rows padded to 33 dwords, so neither the transposed writes nor the
// row reads conflict on banks); both tiles are then written out as whole 128-byte rows, and the tile's
// number of ranks below na (nb) per cell is added to ccnt_a (ccnt_b), which start at zero. Probe entries
// outside [0, NC) are ignored.
constexpr int kTileQ = 64;
constexpr int kTileC = 128;  // 33 KB of LDS per block, so blocks fit beside the scans of other batches
constexpr int kTileRow = kTileQ / 2 + 1;  // dwords per padded tile row

__global__ __launch_bounds__(512) void k_rank_build(const int32_t *__restrict__ probe, const uint16_t *__restrict__ QM,
                                                    int64_t B, int npr, int n, int NC, int64_t Bp,
                                                    uint16_t *__restrict__ rank, uint16_t *__restrict__ score,
                                                    uint32_t na, uint32_t nb, int32_t *__restrict__ ccnt_a,
                                                    int32_t *__restrict__ ccnt_b) {
  __shared__ uint32_t rt[kTileC * kTileRow];
  __shared__ uint32_t st[kTileC * kTileRow];
  const int64_t q0 = (int64_t)blockIdx.y * kTileQ;
  const int c0 = blockIdx.x * kTileC;
  const int tid = threadIdx.x;
  for (int i = tid; i < kTileC * kTileRow; i += 512) rt[i] = 0xffffffffu;
  // scores: thread reads QM[q0 + qq][c0 + cc] along cc (coalesced), 16 loads in flight, and writes the
  // transposed tile
  constexpr int kSU = 16;
  for (int i0 = 0; i0 < kTileQ * kTileC; i0 += 512 * kSU) {
    uint16_t h[kSU];
#pragma unroll
    for (int u = 0; u < kSU; u++) {
      const int i = i0 + u * 512 + tid;
      const int qq = i / kTileC, cc = i - qq * kTileC;
      const int64_t q = q0 + qq;
      h[u] = (i < kTileQ * kTileC && q < B && c0 + cc < NC) ? QM[q * NC + c0 + cc] : (uint16_t)0;
    }
#pragma unroll
    for (int u = 0; u < kSU; u++) {
      const int i = i0 + u * 512 + tid;
      const int qq = i / kTileC, cc = i - qq * kTileC;
      if (i < kTileQ * kTileC) reinterpret_cast<uint16_t *>(st)[2 * (cc * kTileRow) + qq] = h[u];
    }
  }
  __syncthreads();
  // ranks: one wave per query (8 at a time), its probe row read 64 entries per load with up to 16 loads in
  // flight; entries that fall in [c0, c0 + kTileC) are scattered into the tile
  constexpr int kPU = 16;
  const int lane = tid & (FVS_WAVE - 1), wv = fvs_wave_id();
  for (int qq = wv; qq < kTileQ; qq += 512 / FVS_WAVE) {
    if (q0 + qq >= B) break;
    const int32_t *pr = probe + (q0 + qq) * npr;
    for (int r0 = 0; r0 < n; r0 += kPU * FVS_WAVE) {
      int c[kPU];
#pragma unroll
      for (int u = 0; u < kPU; u++) {
        const int r = r0 + u * FVS_WAVE + lane;
        c[u] = r < n ? pr[r] : -1;
      }
#pragma unroll
      for (int u = 0; u < kPU; u++) {
        const unsigned cc = (unsigned)(c[u] - c0);
        if (cc < (unsigned)kTileC && c[u] < NC)
          reinterpret_cast<uint16_t *>(rt)[2 * (cc * kTileRow) + qq] = (uint16_t)(r0 + u * FVS_WAVE + lane);
      }
    }
  }
  __syncthreads();
  // the tile's share of each cell's counts: thread t < kTileC sums the ranks below na (and nb) in row t (the
  // odd row pitch keeps the 64 lanes' reads on distinct banks); one atomic per cell and list adds it to the
  // zeroed totals (integer sums: the result does not depend on their order)
  if (tid < kTileC && c0 + tid < NC) {
    int ma = 0, mb = 0;
    for (int j = 0; j < kTileRow - 1; j++) {
      const uint32_t v = rt[tid * kTileRow + j];
      ma += ((v & 0xffffu) < na) + ((v >> 16) < na);
      mb += ((v & 0xffffu) < nb) + ((v >> 16) < nb);
    }
    if (ma) atomicAdd(&ccnt_a[c0 + tid], ma);
    if (ccnt_b && mb) atomicAdd(&ccnt_b[c0 + tid], mb);
  }
  // out: 32 dwords per cell row, one row per 32 threads
  for (int i = tid; i < kTileC * 32; i += 512) {
    const int cc = i >> 5, j = i & 31;
    if (c0 + cc < NC) {
      const int64_t at = ((int64_t)(c0 + cc) * Bp + q0) / 2 + j;  // in dwords
      reinterpret_cast<uint32_t *>(rank)[at] = rt[cc * kTileRow + j];
      reinterpret_cast<uint32_t *>(score)[at] = st[cc * kTileRow + j];
    }
  }
}

// Entries of one 16-byte row piece (8 ranks) with rank < n.
__device__ __forceinline__ int below8(const uint4 v, uint32_t n) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
  int m = 0;
#pragma unroll
  for (int u = 0; u < 4; u++) m += ((w[u] & 0xffffu) < n) + ((w[u] >> 16) < n);
  return m;
}

constexpr int kCellWaves = 4;  // cells per block in the count and emit kernels (one wave per cell)

// ccnt_a[0, NC) = 0 (and ccnt_b): the totals k_rank_build adds its tiles' counts to.
__global__ __launch_bounds__(256) void k_cell_zero(int32_t *__restrict__ ccnt_a, int32_t *__restrict__ ccnt_b, int NC) {
  for (int c = blockIdx.x * 256 + threadIdx.x; c < NC; c += gridDim.x * 256) {
    ccnt_a[c] = 0;
    if (ccnt_b) ccnt_b[c] = 0;
  }
}

// Exclusive prefix sum of ccnt into coff (block y = list). Thread t scans a run of consecutive cells,
// then the run totals are scanned across the 1024 threads.
__global__ __launch_bounds__(1024) void k_cell_scan(const int32_t *__restrict__ ccnt_a, int32_t *__restrict__ coff_a,
                                                    const int32_t *__restrict__ ccnt_b, int32_t *__restrict__ coff_b,
                                                    int NC) {
  __shared__ int wsum[1024 / FVS_WAVE];
  const int32_t *ccnt = blockIdx.x ? ccnt_b : ccnt_a;
  int32_t *coff = blockIdx.x ? coff_b : coff_a;
  const int t = threadIdx.x, lane = t & (FVS_WAVE - 1), w = fvs_wave_id();
  const int per = (NC + 1023) / 1024;
  const int c0 = t * per, c1 = min(c0 + per, NC);
  int run = 0;
  for (int c = c0; c < c1; c++) run += ccnt[c];
  const int inc = wave_incl_scan_i32(run, lane);
  if (lane == FVS_WAVE - 1) wsum[w] = inc;
  __syncthreads();
  int base = 0;
  for (int i = 0; i < w; i++) base += wsum[i];
  int o = base + inc - run;
  for (int c = c0; c < c1; c++) {
    coff[c] = o;
    o += ccnt[c];
  }
}

struct PairList {
  int32_t *qid, *qrank;
  float *qcp;
  const int32_t *coff;
  uint32_t n;  // columns of the probe rows in this list
};

// One wave per cell: its queries in ascending order, their probe ranks and pair constants, for one or
// two lists. The rank and score rows are read kEmitU 16-byte pieces per lane at a time (2048 queries).
// For each round of one piece per lane (512 queries), wave prefix sums place each lane's pairs in the
// wave's LDS staging area in query order, and the wave then writes the round's pairs of each list out
// with consecutive lanes on consecutive slots (whole-line stores instead of one scattered store per
// pair and lane).
constexpr int kEmitU = 4;

template <bool TWO>
__global__ __launch_bounds__(kCellWaves * FVS_WAVE) void k_cell_emit(
    const uint16_t *__restrict__ rank, const uint16_t *__restrict__ score, int64_t Bp, const float *__restrict__ mnorm,
    const float *__restrict__ qadd, int NC, PairList la, PairList lb) {
  // a piece round's pairs of each list, in order: (query, rank << 16 | score bits)
  __shared__ uint2 stg[TWO ? 2 : 1][kCellWaves][8 * FVS_WAVE];
  const int lane = threadIdx.x & (FVS_WAVE - 1);
  const int wv = fvs_wave_id();
  const int c = blockIdx.x * kCellWaves + wv;
  if (c >= NC) return;
  const uint4 *rr = reinterpret_cast<const uint4 *>(rank + (int64_t)c * Bp);
  const uint4 *ss = reinterpret_cast<const uint4 *>(score + (int64_t)c * Bp);
  const float sc = mnorm ? mnorm[c] : 1.0f;
  const int64_t nv = Bp / 8;
  int runa = la.coff[c], runb = TWO ? lb.coff[c] : 0;
  auto flush = [&](const uint2 *st, int cnt, const PairList &l, int run) {
    for (int j = lane; j < cnt; j += FVS_WAVE) {
      const uint2 p = st[j];
      float x = fvs_h2f((uint16_t)(p.y & 0xffffu)) * sc;
      if (qadd) x = x + qadd[p.x];
      l.qid[run + j] = (int32_t)p.x;
      l.qrank[run + j] = (int32_t)(p.y >> 16);
      l.qcp[run + j] = x;
    }
  };
  for (int64_t base = 0; base < nv; base += kEmitU * FVS_WAVE) {
    uint4 v[kEmitU], sv[kEmitU];
#pragma unroll
    for (int u = 0; u < kEmitU; u++) {
      const int64_t i = base + u * FVS_WAVE + lane;
      v[u] = i < nv ? rr[i] : make_uint4(0xffffffffu, 0xffffffffu, 0xffffffffu, 0xffffffffu);
      sv[u] = i < nv ? ss[i] : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int u = 0; u < kEmitU; u++) {
      const int ma = below8(v[u], la.n);
      const int ia = wave_incl_scan_i32(ma, lane);
      const int ta = __builtin_amdgcn_readlane(ia, FVS_WAVE - 1);
      int oa = ia - ma, ob = 0, tb = 0;
      if (TWO) {
        const int mb = below8(v[u], lb.n);
        const int ib = wave_incl_scan_i32(mb, lane);
        tb = __builtin_amdgcn_readlane(ib, FVS_WAVE - 1);
        ob = ib - mb;
      }
      const uint32_t w[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
      const uint32_t hw[4] = {sv[u].x, sv[u].y, sv[u].z, sv[u].w};
#pragma unroll
      for (int e = 0; e < 8; e++) {
        const uint32_t r = (e & 1) ? (w[e >> 1] >> 16) : (w[e >> 1] & 0xffffu);
        const uint32_t h = (e & 1) ? (hw[e >> 1] >> 16) : (hw[e >> 1] & 0xffffu);
        const uint32_t q = (uint32_t)((base + u * FVS_WAVE + lane) * 8 + e);
        if (r < la.n) stg[0][wv][oa++] = make_uint2(q, (r << 16) | h);
        if (TWO && r < lb.n) stg[TWO ? 1 : 0][wv][ob++] = make_uint2(q, (r << 16) | h);
      }
      wave_lds_sync();
      flush(stg[0][wv], ta, la, runa);
      runa += ta;
      if (TWO) {
        flush(stg[TWO ? 1 : 0][wv], tb, lb, runb);
        runb += tb;
      }
      wave_lds_sync();
    }
  }
}

int64_t pairs_pitch(int64_t B) { return (B + kTileQ - 1) / kTileQ * kTileQ; }

int64_t matrix_bytes(int64_t B, int NC) { return ((int64_t)NC * pairs_pitch(B) * 2 + 255) / 256 * 256; }

// One or two pair lists (first na columns, and first nb columns when lb is given) from one rank matrix.
// Small batches (B <= kPairsSmallB, NC <= kPairsSmallNC): the whole builder in one workgroup. Each cell's queries
// are a 64-bit mask in LDS, one per list (atomic ORs over the probe rows); a block scan of their
// popcounts gives the offsets, and every pair then finds its slot at once: the cell's offset plus the
// number of lower queries in the cell's mask. That is the ascending query order of the matrix builder,
// bit for bit, in one launch instead of four. One workgroup runs out of memory parallelism as the batch
// grows: at 64 queries the four-launch builder is faster again, so batches above 16 use it.
constexpr int kPairsSmallB = 16;  // <= 64 (one mask bit per query)
constexpr int kPairsSmallNC = 4096;

__global__ __launch_bounds__(1024) void k_pairs_small(const int32_t *__restrict__ probe, int B, int npr, int NC,
                                                      const uint16_t *__restrict__ QM, const float *__restrict__ mnorm,
                                                      const float *__restrict__ qadd, int32_t *__restrict__ ccnt_a,
                                                      PairList la, int32_t *__restrict__ ccnt_b, PairList lb, int two) {
  __shared__ uint64_t qm[2][kPairsSmallNC];  // queries of each cell, per list
  __shared__ int off[2][kPairsSmallNC];      // each cell's first slot, per list
  __shared__ int wsum[2][1024 / FVS_WAVE];
  const int t = threadIdx.x, lane = t & (FVS_WAVE - 1), w = fvs_wave_id();
  for (int c = t; c < NC; c += 1024) {
    qm[0][c] = 0ull;
    qm[1][c] = 0ull;
  }
  __syncthreads();
  const int n = two ? (int)max(la.n, lb.n) : (int)la.n;
  for (int i = t; i < B * n; i += 1024) {
    const int q = i / n, r = i - q * n;
    const int c = probe[(int64_t)q * npr + r];
    if ((unsigned)c >= (unsigned)NC) continue;  // a probe id outside [0, NC) names no cell: no pair
    if (r < (int)la.n) atomicOr(&qm[0][c], 1ull << q);
    if (two && r < (int)lb.n) atomicOr(&qm[1][c], 1ull << q);
  }
  __syncthreads();
  // exclusive scans of the counts: thread t owns the run of cells [t * per, t * per + per)
  const int per = (NC + 1023) / 1024;
  const int c0 = t * per, c1 = min(c0 + per, NC);
  for (int l = 0; l < 1 + two; l++) {
    int run = 0;
    for (int c = c0; c < c1; c++) run += __popcll(qm[l][c]);
    const int inc = wave_incl_scan_i32(run, lane);
    if (lane == FVS_WAVE - 1) wsum[l][w] = inc;
    __syncthreads();
    int base = inc - run;
    for (int i = 0; i < w; i++) base += wsum[l][i];
    int32_t *ccnt = l ? ccnt_b : ccnt_a;
    int32_t *coff = const_cast<int32_t *>(l ? lb.coff : la.coff);
    for (int c = c0; c < c1; c++) {
      const int k = __popcll(qm[l][c]);
      ccnt[c] = k;
      coff[c] = base;
      off[l][c] = base;
      base += k;
    }
  }
  __syncthreads();
  for (int i = t; i < B * n; i += 1024) {
    const int q = i / n, r = i - q * n;
    const int c = probe[(int64_t)q * npr + r];
    if ((unsigned)c >= (unsigned)NC) continue;
    const uint64_t below = (1ull << q) - 1ull;  // q < 64
    float x = fvs_h2f(QM[(int64_t)q * NC + c]) * (mnorm ? mnorm[c] : 1.0f);
    if (qadd) x = x + qadd[q];
    if (r < (int)la.n) {
      const int o = off[0][c] + __popcll(qm[0][c] & below);
      la.qid[o] = q;
      la.qrank[o] = r;
      la.qcp[o] = x;
    }
    if (two && r < (int)lb.n) {
      const int o = off[1][c] + __popcll(qm[1][c] & below);
      lb.qid[o] = q;
      lb.qrank[o] = r;
      lb.qcp[o] = x;
    }
  }
}

int pairs_impl(const int32_t *probe, int64_t B, int npr, int NC, const uint16_t *QM, const float *mnorm,
               const float *qadd, void *scratch, int64_t scratch_bytes, int32_t *ccnt_a, PairList la,
               int32_t *ccnt_b, const PairList *lb, hipStream_t st) {
  if (scratch_bytes < 2 * matrix_bytes(B, NC)) return FVS_E_CAPACITY;
  if (NC > kMaxNC) return FVS_E_CAPACITY;
  if ((reinterpret_cast<uintptr_t>(scratch) & 15) != 0) return FVS_E_ARG;
  if (B > 0 && B <= kPairsSmallB && NC <= kPairsSmallNC) {
    const PairList lb_ = lb ? *lb : la;
    hipLaunchKernelGGL(k_pairs_small, dim3(1), dim3(1024), 0, st, probe, (int)B, npr, NC, QM, mnorm, qadd, ccnt_a, la,
                       lb ? ccnt_b : ccnt_a, lb_, lb ? 1 : 0);
    return fvs_launch_status();
  }
  const int64_t Bp = pairs_pitch(B);
  uint16_t *rank = reinterpret_cast<uint16_t *>(scratch);
  uint16_t *score = reinterpret_cast<uint16_t *>(reinterpret_cast<char *>(scratch) + matrix_bytes(B, NC));
  const int n = (int)max(la.n, lb ? lb->n : 0u);
  int e;
  hipLaunchKernelGGL(k_cell_zero, dim3((unsigned)((NC + 255) / 256)), dim3(256), 0, st, ccnt_a, lb ? ccnt_b : nullptr,
                     NC);
  if ((e = fvs_launch_status())) return e;
  if (B > 0) {
    const dim3 grid((unsigned)((NC + kTileC - 1) / kTileC), (unsigned)(Bp / kTileQ));
    hipLaunchKernelGGL(k_rank_build, grid, dim3(512), 0, st, probe, QM, B, npr, n, NC, Bp, rank, score, la.n,
                       lb ? lb->n : 0u, ccnt_a, lb ? ccnt_b : nullptr);
    if ((e = fvs_launch_status())) return e;
  }
  const unsigned cg = (unsigned)((NC + kCellWaves - 1) / kCellWaves);
  const dim3 cb(kCellWaves * FVS_WAVE);
  if (lb) {
    hipLaunchKernelGGL(k_cell_scan, dim3(2), dim3(1024), 0, st, ccnt_a, const_cast<int32_t *>(la.coff), ccnt_b,
                       const_cast<int32_t *>(lb->coff), NC);
    if ((e = fvs_launch_status())) return e;
    hipLaunchKernelGGL(k_cell_emit<true>, dim3(cg), cb, 0, st, rank, score, Bp, mnorm, qadd, NC, la, *lb);
  } else {
    hipLaunchKernelGGL(k_cell_scan, dim3(1), dim3(1024), 0, st, ccnt_a, const_cast<int32_t *>(la.coff), ccnt_a,
                       const_cast<int32_t *>(la.coff), NC);
    if ((e = fvs_launch_status())) return e;
    hipLaunchKernelGGL(k_cell_emit<false>, dim3(cg), cb, 0, st, rank, score, Bp, mnorm, qadd, NC, la, la);
  }
  return fvs_launch_status();
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

extern "C" int fvs_route_topk_scaled(const uint16_t *QM, const float *scale, const float *qadd, int64_t B, int32_t NC,
                                     int32_t nprobe, int32_t *probe, void *stream) {
  if (B < 0 || NC <= 0 || nprobe <= 0 || nprobe > NC) return FVS_E_ARG;
  if (NC > 8192 || nprobe > 4096) return FVS_E_CAPACITY;
  if (B == 0) return FVS_OK;
  if (!QM || !scale || !probe) return FVS_E_ARG;
  hipStream_t st = (hipStream_t)stream;
  if (NC % 8 == 0 && nprobe <= 1024 && ((reinterpret_cast<uintptr_t>(QM) | reinterpret_cast<uintptr_t>(scale)) & 15) == 0) {
    if (B <= kRouteBlkMaxB) {
      const dim3 g((unsigned)B), b(kRouteBlk);
      if (NC <= 4096) {
        if (qadd) hipLaunchKernelGGL((k_route_blk_f32<4, true>), g, b, 0, st, QM, scale, qadd, NC, nprobe, probe);
        else hipLaunchKernelGGL((k_route_blk_f32<4, false>), g, b, 0, st, QM, scale, qadd, NC, nprobe, probe);
      } else {
        if (qadd) hipLaunchKernelGGL((k_route_blk_f32<8, true>), g, b, 0, st, QM, scale, qadd, NC, nprobe, probe);
        else hipLaunchKernelGGL((k_route_blk_f32<8, false>), g, b, 0, st, QM, scale, qadd, NC, nprobe, probe);
      }
      return fvs_launch_status();
    }
    if (NC <= 4096) return route_wave_f32_r<8>(QM, scale, qadd, B, NC, nprobe, probe, st);
    return route_wave_f32_r<16>(QM, scale, qadd, B, NC, nprobe, probe, st);
  }
  const size_t shm = 8 * ((size_t)NC + (size_t)fvs_pow2_ceil(nprobe));
  hipLaunchKernelGGL(k_route_f32, dim3((unsigned)B), dim3(256), shm, st, QM, scale, qadd, NC, nprobe, probe);
  return fvs_launch_status();
}

namespace {
// out[q][c] = fp16(((float)QM[q][c] + qadd[q]) * scale[c]), each term only when its array is given (no "+ 0",
// which would turn -0 into +0). Four cells per thread.
template <bool ADD, bool MUL>
__global__ __launch_bounds__(256) void k_route_keys(const uint16_t *__restrict__ QM, const float *__restrict__ scale,
                                                    const float *__restrict__ qadd, int64_t B, int NC,
                                                    uint16_t *__restrict__ out) {
  const int64_t n = B * NC;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t q = i / NC;
    const int c = (int)(i - q * NC);
    float v = fvs_h2f(QM[i]);
    if (ADD) v = v + qadd[q];
    if (MUL) v = v * scale[c];
    out[i] = fvs_f2h(v);
  }
}
}  // namespace

extern "C" int fvs_route_keys(const uint16_t *QM, const float *scale, const float *qadd, int64_t B, int32_t NC,
                              uint16_t *out, void *stream) {
  if (B < 0 || NC <= 0) return FVS_E_ARG;
  if (B == 0) return FVS_OK;
  if (!QM || !out) return FVS_E_ARG;
  const int64_t n = B * NC;
  const unsigned grid = (unsigned)std::min<int64_t>((n + 255) / 256, 16384);
  hipStream_t st = (hipStream_t)stream;
  if (qadd && scale) hipLaunchKernelGGL((k_route_keys<true, true>), dim3(grid), dim3(256), 0, st, QM, scale, qadd, B, NC, out);
  else if (qadd) hipLaunchKernelGGL((k_route_keys<true, false>), dim3(grid), dim3(256), 0, st, QM, scale, qadd, B, NC, out);
  else if (scale) hipLaunchKernelGGL((k_route_keys<false, true>), dim3(grid), dim3(256), 0, st, QM, scale, qadd, B, NC, out);
  else hipLaunchKernelGGL((k_route_keys<false, false>), dim3(grid), dim3(256), 0, st, QM, scale, qadd, B, NC, out);
  return fvs_launch_status();
}

extern "C" int64_t fvs_pairs_scratch_bytes(int64_t B, int32_t NC) {
  if (B < 0 || NC <= 0) return -1;
  return 2 * matrix_bytes(B, NC);  // rank matrix, then score matrix
}

extern "C" int fvs_pairs(const int32_t *probe, int64_t B, int32_t npr, int32_t n, int32_t NC, const uint16_t *QM,
                         const float *mnorm, const float *qadd, int32_t *ccnt, int32_t *coff, void *scratch,
                         int64_t scratch_bytes,
                         int32_t *qid, int32_t *qrank, float *qcp, void *stream) {
  if (B < 0 || NC <= 0 || n <= 0 || n > npr || n > 65535) return FVS_E_ARG;
  if (!probe || !QM || !ccnt || !coff || !scratch || !qid || !qrank || !qcp) return FVS_E_ARG;
  const PairList la{qid, qrank, qcp, coff, (uint32_t)n};
  return pairs_impl(probe, B, npr, NC, QM, mnorm, qadd, scratch, scratch_bytes, ccnt, la, nullptr, nullptr,
                    (hipStream_t)stream);
}

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxDevices] = {};

// The device address of `scratch` on the current device, taken once per device.
int static_scratch(void **out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  if (dev < 0 || dev >= kMaxDevices) return FVS_E_CAPACITY;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void *p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return (int)e;
    if (!p) return FVS_E_ARG;
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return FVS_OK;
}

}  // namespace

extern "C" int fvs_pairs_noalloc(const int32_t *probe, int64_t B, int32_t npr, int32_t n, int32_t NC,
                                 const uint16_t *QM, const float *mnorm, const float *qadd, int32_t *ccnt,
                                 int32_t *coff, int32_t *qid, int32_t *qrank, float *qcp, void *stream) {
  if (B < 0 || NC <= 0 || n <= 0 || n > npr || n > 65535) return FVS_E_ARG;
  if (!probe || !QM || !ccnt || !coff || !qid || !qrank || !qcp) return FVS_E_ARG;
  if (NC > kMaxNC || 2 * matrix_bytes(B, NC) > (int64_t)FVS_PAIRS_NOALLOC_SCRATCH) return FVS_E_CAPACITY;
  void *buf = nullptr;
  const int e = static_scratch(&buf);
  if (e) return e;
  const PairList la{qid, qrank, qcp, coff, (uint32_t)n};
  return pairs_impl(probe, B, npr, NC, QM, mnorm, qadd, buf, FVS_PAIRS_NOALLOC_SCRATCH, ccnt, la, nullptr, nullptr,
                    (hipStream_t)stream);
}

extern "C" int fvs_pairs2(const int32_t *probe, int64_t B, int32_t npr, int32_t n1, int32_t NC, const uint16_t *QM,
                          const float *mnorm, const float *qadd, void *scratch, int64_t scratch_bytes,
                          int32_t *ccnt1, int32_t *coff1, int32_t *qid1, int32_t *qrank1, float *qcp1,
                          int32_t *ccnt, int32_t *coff, int32_t *qid, int32_t *qrank, float *qcp, void *stream) {
  if (B < 0 || NC <= 0 || n1 <= 0 || n1 > npr || npr > 65535) return FVS_E_ARG;
  if (!probe || !QM || !scratch || !ccnt1 || !coff1 || !qid1 || !qrank1 || !qcp1 || !ccnt || !coff || !qid ||
      !qrank || !qcp)
    return FVS_E_ARG;
  const PairList la{qid1, qrank1, qcp1, coff1, (uint32_t)n1};
  const PairList lb{qid, qrank, qcp, coff, (uint32_t)npr};
  return pairs_impl(probe, B, npr, NC, QM, mnorm, qadd, scratch, scratch_bytes, ccnt1, la, ccnt, &lb,
                    (hipStream_t)stream);
}
