// Device helpers shared by the libfvs kernels (gfx950, wave64).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/fvs.h"

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

#define FVS_WAVE 64

// Return the launch status of the kernel just enqueued (0 on success).
static inline int fvs_launch_status() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? 0 : (int)e;
}

__device__ __forceinline__ float fvs_h2f(uint16_t h) {
  return (float)__builtin_bit_cast(_Float16, h);
}
__device__ __forceinline__ uint16_t fvs_f2h(float f) {  // round to nearest even
  return __builtin_bit_cast(uint16_t, (_Float16)f);
}
__device__ __forceinline__ float fvs_round_h(float f) {  // f rounded to the nearest fp16 value (ties to even)
  return (float)(_Float16)f;
}

// Order-preserving maps to unsigned keys (larger float -> larger key); -0 is mapped like +0.
__device__ __forceinline__ uint32_t fvs_ord32(float x) {
  uint32_t u = __float_as_uint(x);
  if (u == 0x80000000u) u = 0u;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float fvs_unord32(uint32_t k) {
  uint32_t u = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
  return __uint_as_float(u);
}
__device__ __forceinline__ uint32_t fvs_ord16(uint16_t u) {
  if (u == 0x8000u) u = 0u;
  return (u & 0x8000u) ? (uint32_t)((~u) & 0xffffu) : (uint32_t)(u | 0x8000u);
}

// Compute units of the current device (queried once per device; up to 64 devices).
static inline int fvs_cu_count() {
  static int cus[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cus[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    cus[dev] = n;
  }
  return cus[dev];
}

// Workgroup barrier that orders LDS only: outstanding global loads stay in flight across it (a
// plain __syncthreads() also waits for every outstanding global access of the wave).
__device__ __forceinline__ void fvs_lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Index of the calling wave in its workgroup, as a value the compiler knows to be wave-uniform: branches
// and loops that depend on it compile to scalar code, and values carried through them stay in SGPRs.
__device__ __forceinline__ int fvs_wave_id() { return __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6); }

// Number of set bits of a wave mask below this lane.
__device__ __forceinline__ int fvs_lane_prefix(uint64_t mask) {
  return (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u));
}

// x of lane (lane ^ d) for a power of two d < 64, every lane of the wave active. With d known at compile
// time (unrolled loops) the exchange is a cross-lane move instead of an LDS permute: DPP quad permutations
// for 1 and 2, a rotation by 8 within 16-lane rows (which is lane ^ 8), ds_swizzle's xor mode within
// 32-lane groups for 4 and 16, and ds_bpermute for 32.
__device__ __forceinline__ uint32_t fvs_xor_lane(uint32_t x, int d) {
  switch (d) {
    case 1: return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0xb1, 0xf, 0xf, false);   // quad_perm 1,0,3,2
    case 2: return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x4e, 0xf, 0xf, false);   // quad_perm 2,3,0,1
    case 4: return (uint32_t)__builtin_amdgcn_ds_swizzle((int)x, 0x101f);                     // and 31, xor 4
    case 8: return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, 0x128, 0xf, 0xf, false);  // row_ror 8
    case 16: return (uint32_t)__builtin_amdgcn_ds_swizzle((int)x, 0x401f);                    // and 31, xor 16
    default: return (uint32_t)__shfl_xor((int)x, d, FVS_WAVE);
  }
}

__device__ __forceinline__ float fvs_xor_lane_f(float x, int d) { return __uint_as_float(fvs_xor_lane(__float_as_uint(x), d)); }

__device__ __forceinline__ double fvs_xor_lane_d(double x, int d) {
  const uint64_t u = (uint64_t)__double_as_longlong(x);
  const uint64_t r = ((uint64_t)fvs_xor_lane((uint32_t)(u >> 32), d) << 32) | fvs_xor_lane((uint32_t)u, d);
  return __longlong_as_double((long long)r);
}

__device__ __forceinline__ float fvs_wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, fvs_xor_lane_f(v, o));
  return v;
}

// Ints of LDS the block helpers below need for their `sh` argument with NT threads: NT / 64 for the scan,
// then up to six results.
__host__ __device__ constexpr int fvs_sh_ints(int NT) { return NT / 64 + 8; }

// Inclusive prefix sum over threadIdx.x for a block of NT threads (a multiple of 64). tmp: NT/64 ints.
template <int NT = 256>
__device__ __forceinline__ int fvs_block_scan(int v, int *tmp) {
  const int lane = threadIdx.x & 63, w = fvs_wave_id();
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    int t = __shfl_up(v, o, FVS_WAVE);
    if (lane >= o) v += t;
  }
  if (lane == 63) tmp[w] = v;
  __syncthreads();
  int add = 0;
  for (int i = 0; i < w; i++) add += tmp[i];
  __syncthreads();
  return v + add;
}
__device__ __forceinline__ int fvs_block_scan256(int v, int *tmp) { return fvs_block_scan<256>(v, tmp); }

// One radix pass's bucket choice, made by wave 0 alone: the 256 bins in descending order, four per lane,
// one wave prefix sum; the lane whose range holds the k-th key writes (bucket, k - keys above it, bucket
// size) to sh[R], sh[R + 1], sh[R + 2]. Every bin is zeroed as it is read, ready for the next pass.
template <int R>
__device__ __forceinline__ void fvs_pick_bucket(int *hist, int *sh, int k) {
  const int lane = threadIdx.x & 63;
  int h[4], s = 0;
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const int b = 255 - 4 * lane - j;
    h[j] = hist[b];
    hist[b] = 0;
    s += h[j];
  }
  int inc = s;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int t = __shfl_up(inc, o, FVS_WAVE);
    if (lane >= o) inc += t;
  }
  int e = inc - s;
#pragma unroll
  for (int j = 0; j < 4; j++) {
    if (e < k && k <= e + h[j]) {
      sh[R] = 255 - 4 * lane - j;
      sh[R + 1] = k - e;
      sh[R + 2] = h[j];
    }
    e += h[j];
  }
}

// k-th largest (1-based, counted with multiplicity) of n keys key(i), 1 <= k <= n, by an MSD radix
// select of 8 bits per pass: per pass a histogram of the keys that match the prefix so far, one
// barrier, the bucket choice by wave 0, one barrier. Block of NT >= 256 threads; hist: 256 ints of LDS,
// sh: fvs_sh_ints(NT) ints of LDS. Every thread returns the same key.
template <typename KT, int NT = 256, typename F>
__device__ KT fvs_block_kth(F key, int n, int k, int *hist, int *sh) {
  static_assert(NT >= 256 && NT % 64 == 0, "block of at least 256 threads");
  constexpr int R = NT / 64;
  KT prefix = 0, pmask = 0;
  if (threadIdx.x < 256) hist[threadIdx.x] = 0;
  __syncthreads();
  for (int shift = (int)sizeof(KT) * 8 - 8; shift >= 0; shift -= 8) {
    for (int i = threadIdx.x; i < n; i += NT) {
      KT x = key(i);
      if ((x & pmask) == prefix) atomicAdd(&hist[(int)((x >> shift) & 0xff)], 1);
    }
    __syncthreads();
    if (fvs_wave_id() == 0) fvs_pick_bucket<R>(hist, sh, k);
    __syncthreads();
    prefix |= (KT)sh[R] << shift;
    pmask |= (KT)0xff << shift;
    k = sh[R + 1];
  }
  __syncthreads();  // every thread has read sh before the caller reuses it
  return prefix;
}

// In-place bitonic sort of n (a power of two) keys in LDS, descending when DESC. Any block size.
template <typename KT, bool DESC>
__device__ void fvs_block_bitonic(KT *s, int n) {
  for (int k = 2; k <= n; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int i = threadIdx.x; i < n; i += blockDim.x) {
        const int ixj = i ^ j;
        if (ixj > i) {
          const KT a = s[i], b = s[ixj];
          const bool first = (i & k) == 0;  // this pair is ordered like the final order
          const bool swap = DESC ? (first ? a < b : a > b) : (first ? a > b : a < b);
          if (swap) {
            s[i] = b;
            s[ixj] = a;
          }
        }
      }
      __syncthreads();
    }
  }
}

__host__ __device__ __forceinline__ int fvs_pow2_ceil(int n) {
  int p = 1;
  while (p < n) p <<= 1;
  return p;
}

// Two k-th largest selections in the same passes: (the kA-th largest of keyA, the kB-th largest of keyB)
// over i < n, 1 <= kA, kB <= n. Waves 0 and 1 pick the two buckets of a pass concurrently, so both
// cost the barriers of one. hist: 512 ints of LDS. Block of NT >= 256 threads.
template <typename KT, int NT = 256, typename FA, typename FB>
__device__ void fvs_block_kth2(FA keyA, FB keyB, int n, int kA, int kB, int *hist, int *sh, KT &outA, KT &outB) {
  static_assert(NT >= 256 && NT % 64 == 0, "block of at least 256 threads");
  constexpr int R = NT / 64;
  KT pa = 0, pb = 0, pmask = 0;
  for (int i = threadIdx.x; i < 512; i += NT) hist[i] = 0;
  __syncthreads();
  for (int shift = (int)sizeof(KT) * 8 - 8; shift >= 0; shift -= 8) {
    for (int i = threadIdx.x; i < n; i += NT) {
      const KT a = keyA(i), b = keyB(i);
      if ((a & pmask) == pa) atomicAdd(&hist[(int)((a >> shift) & 0xff)], 1);
      if ((b & pmask) == pb) atomicAdd(&hist[256 + (int)((b >> shift) & 0xff)], 1);
    }
    __syncthreads();
    const int w = fvs_wave_id();
    if (w == 0) fvs_pick_bucket<R>(hist, sh, kA);
    if (w == 1) fvs_pick_bucket<R + 3>(hist + 256, sh, kB);
    __syncthreads();
    pa |= (KT)sh[R] << shift;
    pb |= (KT)sh[R + 3] << shift;
    pmask |= (KT)0xff << shift;
    kA = sh[R + 1];
    kB = sh[R + 4];
  }
  __syncthreads();
  outA = pa;
  outB = pb;
}

// A bound T with #{i : key(i) >= T} == kk for n UNIQUE keys, 1 <= kk <= n: the MSD radix select of
// fvs_block_kth, stopped as soon as the chosen bucket holds exactly the keys still wanted (then every
// key of the bucket is in and T is the bucket's smallest possible key). Block of NT >= 256 threads.
template <typename KT, int NT = 256, typename F>
__device__ KT fvs_block_kth_set(F key, int n, int k, int *hist, int *sh) {
  static_assert(NT >= 256 && NT % 64 == 0, "block of at least 256 threads");
  constexpr int R = NT / 64;
  KT prefix = 0, pmask = 0;
  if (threadIdx.x < 256) hist[threadIdx.x] = 0;
  __syncthreads();
  for (int shift = (int)sizeof(KT) * 8 - 8; shift >= 0; shift -= 8) {
    for (int i = threadIdx.x; i < n; i += NT) {
      KT x = key(i);
      if ((x & pmask) == prefix) atomicAdd(&hist[(int)((x >> shift) & 0xff)], 1);
    }
    __syncthreads();
    if (fvs_wave_id() == 0) fvs_pick_bucket<R>(hist, sh, k);
    __syncthreads();
    prefix |= (KT)sh[R] << shift;
    pmask |= (KT)0xff << shift;
    k = sh[R + 1];
    if (sh[R + 2] == k) break;  // the whole bucket is in (the same decision in every thread)
  }
  __syncthreads();  // every thread has read sh (and hist is zero) before the caller reuses them
  return prefix;
}

__device__ __forceinline__ uint64_t fvs_shfl_xor_u64(uint64_t x, int j) {
  const uint32_t lo = fvs_xor_lane((uint32_t)x, j);
  const uint32_t hi = fvs_xor_lane((uint32_t)(x >> 32), j);
  return ((uint64_t)hi << 32) | lo;
}

// Sorts s[0..kk) (unique 64-bit keys) descending in place, kk <= 2 NT, with blockDim.x == NT. Wave w sorts
// the run s[128 w, 128 w + 128) in registers (two keys per lane, element e * 64 + lane; a bitonic network
// whose exchanges within a lane are register moves and across lanes shuffles; missing keys are 0, which
// sorts last and equals any real key of 0, so the sorted values are the same either way) and writes it
// back in place. Each key's final index is then its index in its own run plus, for every other run, the
// number of that run's keys above it (a binary search in the sorted run).
template <int NT>
__device__ void fvs_block_sort_desc_u64(uint64_t *s, int kk) {
  const int lane = threadIdx.x & (FVS_WAVE - 1), w = threadIdx.x / FVS_WAVE;
  const int nreal = min(128, kk - 128 * w);  // keys in this wave's run (<= 0: no run)
  uint64_t v[2];
#pragma unroll
  for (int e = 0; e < 2; e++) v[e] = e * 64 + lane < nreal ? s[128 * w + e * 64 + lane] : 0ull;
  if (nreal > 0) {
#pragma unroll
    for (int k = 2; k <= 128; k <<= 1) {
#pragma unroll
      for (int j = k >> 1; j > 0; j >>= 1) {
        if (j == 64) {  // the pair (lane, 64 + lane): the lower index takes the larger key
          const uint64_t hi = v[0] > v[1] ? v[0] : v[1], lo = v[0] > v[1] ? v[1] : v[0];
          v[0] = hi;
          v[1] = lo;
        } else {
#pragma unroll
          for (int e = 0; e < 2; e++) {
            const uint64_t p = fvs_shfl_xor_u64(v[e], j);
            const int i = e * 64 + lane;
            // descending blocks where (i & k) == 0; the lower index of a pair holds the block's larger key
            const bool take_max = ((i & k) == 0) == ((i & j) == 0);
            const bool gt = v[e] > p;
            v[e] = take_max == gt ? v[e] : p;
          }
        }
      }
    }
  }
#pragma unroll
  for (int e = 0; e < 2; e++)
    if (e * 64 + lane < nreal) s[128 * w + e * 64 + lane] = v[e];
  __syncthreads();
  const int R = (kk + 127) / 128;
  int r[2];
#pragma unroll
  for (int e = 0; e < 2; e++) {
    const int i = e * 64 + lane;
    r[e] = i;
    if (i < nreal) {
      for (int w2 = 0; w2 < R; w2++) {
        if (w2 == w) continue;
        const uint64_t *run = s + 128 * w2;
        const int len = min(128, kk - 128 * w2);
        int idx = 0;  // keys of run w2 above v[e]: the run is descending
#pragma unroll
        for (int step = 128; step > 0; step >>= 1)
          if (idx + step <= len && run[idx + step - 1] > v[e]) idx += step;
        r[e] += idx;
      }
    }
  }
  __syncthreads();
#pragma unroll
  for (int e = 0; e < 2; e++)
    if (e * 64 + lane < nreal) s[r[e]] = v[e];
  __syncthreads();
}

// Top-kk of n unique 64-bit keys, sorted descending, into s[0..kk) (s holds pow2_ceil(kk) keys).
// Requires kk <= n. The kk keys above the radix bound are gathered, then sorted: by counting ranks up to
// 64 keys, as runs of 128 sorted in registers and merged by rank (fvs_block_sort_desc_u64) up to 2 NT, by
// a bitonic sort in LDS above.
// Block of NT threads; cnt: 1 int of LDS.
template <int NT = 256, typename F>
__device__ void fvs_block_topk_u64(F key, int n, int kk, uint64_t *s, int *hist, int *sh, int *cnt) {
  const int P = fvs_pow2_ceil(kk);
  const uint64_t kth = fvs_block_kth_set<uint64_t, NT>(key, n, kk, hist, sh);
  if (threadIdx.x == 0) *cnt = 0;
  for (int i = threadIdx.x; i < P; i += NT) s[i] = 0;
  __syncthreads();
  for (int i = threadIdx.x; i < n; i += NT) {
    const uint64_t x = key(i);
    if (x >= kth) {
      const int slot = atomicAdd(cnt, 1);
      if (slot < P) s[slot] = x;  // keys are unique, so exactly kk of them pass
    }
  }
  __syncthreads();
  if (kk <= 64) {
    // a few keys: each thread < kk places its key at its rank, a count of the larger keys (every lane
    // reads the same address per step: a broadcast)
    const uint64_t m0 = threadIdx.x < kk ? s[threadIdx.x] : 0ull;
    int r0 = 0;
    for (int t = 0; t < kk; t++) r0 += s[t] > m0 ? 1 : 0;
    __syncthreads();
    if (threadIdx.x < kk) s[r0] = m0;
    __syncthreads();
  } else if (kk <= 2 * NT) {
    fvs_block_sort_desc_u64<NT>(s, kk);
  } else {
    fvs_block_bitonic<uint64_t, true>(s, P);
  }
}
