// Routing-free int8 scan: the dense contraction of every query code with every stored code, with the
// reference's brute-force epilogue (throughput/brute.py:10-35, throughput/cbrute.py:22-64): a dense score
// pass (mode 0, for the threshold sample) and a threshold-and-emit pass (mode 1).
//
// Storage: a code matrix X [n, R] (int8) is kept in a fragment-tiled layout: block (rb, s) of rows
// 32 rb .. 32 rb + 31 and bytes 32 s .. 32 s + 31 is 1 KB at ((rb * R/32 + s) * 1024), holding 16 bytes
// per lane in the order lane = 32 h + li -> row 32 rb + li, bytes 32 s + 16 h .. + 15. That is exactly the
// MFMA operand of one v_mfma_i32_32x32x32_i8 step, so one 1 KB block moves from HBM into LDS with one
// contiguous direct-to-LDS load per wave (global_load_lds_dwordx4) and out of LDS with one contiguous
// ds_read_b128 per wave: no shuffles, no bank conflicts. Rows past n are zero.
//
// Scan: a workgroup computes 128 queries x 256 rows over the whole K dimension: four waves of 64 queries
// x 128 rows (8 MFMA tiles, 128 accumulators per lane). Operand blocks stream through three LDS stages of
// 2 K-steps (24 KB each); each wave requests a quarter of stage g + 2 while stage g is computed, one
// barrier per stage. Two workgroups share a CU (76 KB of LDS and at most 256 registers per lane each), so
// one workgroup's epilogue and barrier waits overlap the other's MFMAs. The grid is persistent and
// XCD-aware: the 64 workgroups of an XCD (workgroup b runs on XCD b % 8) process 64 consecutive tiles at a
// time, i.e. all 16 query tiles of 4 row tiles, so a row tile is read from HBM into one L2 and reused
// there 16 times. The pipeline runs across tile boundaries, so the next tile's first stages load under the
// current tile's epilogue.
//
// The LDS traffic bounds this layout: per 32 MFMAs a workgroup reads 24 KB of operands from LDS and writes
// 12 KB into it, about 140 bytes per clock per CU at the MFMA peak.
//
// Epilogue (canonical): est = ((float)acc * qs[q]) * (float)zs[n] (two products, left to right);
//   mode 0: out[q * N + n] = est;
//   mode 1: every (q, n) with est >= t0[q] is counted in cnt[q] and the first CAP of a query are stored at
//           bval/bpos[q * CAP + idx]. Each lane reserves the slots of its passing rows in a 16-row block with
//           one atomic add (the reference's MODE 3 reservation, throughput/brute.py:20-30).
#include "fvs_common.h"

namespace {

constexpr int kQT = 128;             // queries per workgroup tile
constexpr int kNT = 256;             // rows per workgroup tile
constexpr int kSS = 2;               // 32-byte K steps per LDS stage
constexpr int kWGCU = 2;             // workgroups resident per CU
constexpr int kNS = 3;               // LDS stages
constexpr int kQB = kQT / 32;        // query blocks per tile
constexpr int kRB = kNT / 32;        // row blocks per tile
constexpr int kBR = kQB + kRB;       // block rows of a tile: query blocks, then row blocks
constexpr int kDMA = kBR * kSS / 4;  // 1 KB blocks each wave requests per stage

__device__ __forceinline__ int acc_row(int v, int h) { return 8 * (v >> 2) + 4 * h + (v & 3); }

// Columns R .. 32 nsteps - 1 of the tiled copy are zero (R a multiple of 16, so a 16-byte chunk is all in or
// all out), which leaves every dot product unchanged.
__global__ __launch_bounds__(256) void k_dense_pack(const int8_t *__restrict__ X, int64_t n, int R, int nsteps,
                                                    int64_t nblk, int8_t *__restrict__ T) {
  const int64_t total = nblk * nsteps * 64;
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    const int lane = (int)(i & 63);
    const int64_t bs = i >> 6;
    const int64_t s = bs % nsteps, rb = bs / nsteps;
    const int64_t r = rb * 32 + (lane & 31);
    const int64_t col = 32 * s + 16 * (lane >> 5);
    v4i v = (v4i){0, 0, 0, 0};
    if (r < n && col < R) v = *reinterpret_cast<const v4i *>(X + r * R + col);
    reinterpret_cast<v4i *>(T)[i] = v;
  }
}

// Direct-to-LDS loads each wave issues with the first stage of a tile for the tile's row scales (waves 0, 1),
// query scales (waves 2, 3) and thresholds (waves 0, 1, emit pass only).
template <int MODE>
__device__ __forceinline__ int tile_requests(int w) {
  return (w < 2 && MODE == 1) ? 2 : 1;
}

template <int MODE>
__global__ __launch_bounds__(256, kWGCU) void k_dense_scan(const int8_t *__restrict__ Qt, const float *__restrict__ qs,
                                                       int B, const int8_t *__restrict__ Zt,
                                                       const uint16_t *__restrict__ zs16, int N, int nsteps, int ntq,
                                                       int ntiles, int m8, const float *__restrict__ t0,
                                                       int32_t *__restrict__ cnt, float *__restrict__ bval,
                                                       int32_t *__restrict__ bpos, int CAP, float *__restrict__ out) {
  // one array per stage (not one indexed array), so the compiler can tell that reading a stage does not
  // race with the direct-to-LDS loads of the others and needs no wait for them
  // stage layout: block row br (query blocks 0..3, then row blocks 0..7), K step s at [br][s]: the four K
  // steps of a block row are 4 KB contiguous, in LDS as in the tiled global layout, so one LDS base (M0)
  // and one global address serve all four loads with the same immediate offsets
  __shared__ __align__(16) v4i ls0[kBR][kSS][64], ls1[kBR][kSS][64], ls2[kBR][kSS][64];  // 24 KB each
  // per-tile constants, in three buffers by tile number mod 3: row scales (fp16 bits), query scales,
  // thresholds. Tile k + 2's constants are requested while other waves may still run tile k's epilogue
  // (with one stage per tile), so two buffers would not do.
  __shared__ __align__(16) uint16_t zsl[3][kNT];
  __shared__ __align__(16) float qsl[3][kQT], tsl[3][kQT];
  const int lane = threadIdx.x & 63, w = fvs_wave_id();
  const int h = lane >> 5, li = lane & 31;
  const int wq = w & 1, wn = w >> 1;  // this wave: queries 64 wq .. + 63, rows 128 wn .. + 127 of the tile
  const int nst = nsteps / kSS;
  const int x = blockIdx.x & 7, m = blockIdx.x >> 3;
  // tiles of this workgroup: tile k = (8 k + x) m8 + m for k < my_tiles
  int my_tiles = 0;
  if (m < m8) {
    const int base = x * m8 + m, step = 8 * m8;
    my_tiles = base < ntiles ? (ntiles - base + step - 1) / step : 0;
  }
  const int nstages = my_tiles * nst;
  const uint32_t blk_bytes = (uint32_t)nsteps * 1024;  // one 32-row block over the whole K dimension
  typedef __attribute__((address_space(3))) void *lds_ptr;

  // The request side, two stages ahead of the compute side: stage rst of the workgroup's tile rk. Wave w
  // loads block rows 3 w .. 3 w + 2 of the tile's 12 (query blocks 0..3, then row blocks 0..7), four K steps
  // of each per stage; the constants of a tile come with its first stage.
  int rk = 0, rst = 0, rpar = 0;
  const int8_t *rsrc[3] = {Qt, Qt, Qt};
  auto request = [&](v4i (&L)[kBR][kSS][64]) {
    if (rk >= my_tiles) return;
    if (rst == 0) {  // a new tile: its coordinates (one division per tile, not per stage) and operand bases
      const int tile = (rk * 8 + x) * m8 + m;
      const int tq = (int)((unsigned)tile % (unsigned)ntq), tn = (int)((unsigned)tile / (unsigned)ntq);
#pragma unroll
      for (int r = 0; r < 3; r++) {
        const int br = 3 * w + r;
        rsrc[r] = br < kQB ? Qt + (size_t)((unsigned)tq * kQB + br) * blk_bytes
                           : Zt + (size_t)((unsigned)tn * kRB + (br - kQB)) * blk_bytes;
      }
    }
    const uint32_t voff = (uint32_t)rst * (kSS * 1024) + (uint32_t)lane * 16;
#pragma unroll
    for (int r = 0; r < 3; r++) {
      const int8_t *src = rsrc[r] + voff;
      lds_ptr dst = (lds_ptr)&L[3 * w + r][0][0];
      static_assert(kSS == 2, "one load per K step of the stage");
      __builtin_amdgcn_global_load_lds(src, dst, 16, 0, 0);
      __builtin_amdgcn_global_load_lds(src, dst, 16, 1024, 0);
    }
    if (rst == 0) {
      const int tile = (rk * 8 + x) * m8 + m;
      const int tq = (int)((unsigned)tile % (unsigned)ntq), tn = (int)((unsigned)tile / (unsigned)ntq);
      if (w < 2) {  // rows 128 w .. 128 w + 127: 4 bytes (two fp16) per lane
        const char *src = reinterpret_cast<const char *>(zs16 + (size_t)tn * kNT + 128 * w) + 4 * lane;
        __builtin_amdgcn_global_load_lds(src, (lds_ptr)&zsl[rpar][128 * w], 4, 0, 0);
        if (MODE == 1)
          __builtin_amdgcn_global_load_lds(t0 + (size_t)tq * kQT + 64 * w + lane, (lds_ptr)&tsl[rpar][64 * w], 4, 0, 0);
      } else {
        __builtin_amdgcn_global_load_lds(qs + (size_t)tq * kQT + 64 * (w - 2) + lane, (lds_ptr)&qsl[rpar][64 * (w - 2)],
                                         4, 0, 0);
      }
    }
    if (++rst == nst) {
      rst = 0;
      ++rk;
      rpar = rpar == 2 ? 0 : rpar + 1;
    }
  };

  // Barrier of a stage: this wave's requests for the stage (and anything older) have landed, with only the
  // `pending` requests of the next stage still outstanding, and its LDS reads of the previous stage are
  // done. Written out instead of __syncthreads(), whose release fence would also wait for the requests
  // of the stage still ahead.
  auto stage_barrier = [&](int pending) {
    switch (pending) {
      case kDMA: asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(kDMA) : "memory"); break;
      case kDMA + 1: asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(kDMA + 1) : "memory"); break;
      case kDMA + 2: asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(kDMA + 2) : "memory"); break;
      default: asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory"); break;
    }
  };

  v16i acc[2][4];
  // the compute side: stage cst of the workgroup's tile ck
  int ck = 0, cst = 0, cpar = 0;
  auto epilogue = [&]() {
    const int tile = (ck * 8 + x) * m8 + m;
    const int tq = (int)((unsigned)tile % (unsigned)ntq), tn = (int)((unsigned)tile / (unsigned)ntq);
    const int par = cpar;
    const bool full = tn * kNT + kNT <= N && (N & 3) == 0;  // every row of the tile exists: no row checks
#pragma unroll
    for (int i = 0; i < 2; i++) {
      const int ql = 64 * wq + 32 * i + li;  // query in the tile
      const int q = tq * kQT + ql;
      const bool qv = q < B;
      const float qsv = qsl[par][ql];
      const float th = MODE == 1 ? tsl[par][ql] : 0.f;
#pragma unroll
      for (int rb = 0; rb < 4; rb++) {
        const int rl = 128 * wn + 32 * rb;  // first row of the block in the tile
        // est of the lane's 16 rows rl + 8 gq + 4 h + c (element 4 gq + c of the accumulator)
        float e[16];
#pragma unroll
        for (int gq = 0; gq < 4; gq++) {
          const uint2 z2 = *reinterpret_cast<const uint2 *>(&zsl[par][rl + 8 * gq + 4 * h]);
          const float zz[4] = {fvs_h2f((uint16_t)z2.x), fvs_h2f((uint16_t)(z2.x >> 16)), fvs_h2f((uint16_t)z2.y),
                               fvs_h2f((uint16_t)(z2.y >> 16))};
#pragma unroll
          for (int c = 0; c < 4; c++) e[4 * gq + c] = ((float)acc[i][rb][4 * gq + c] * qsv) * zz[c];
        }
        const int nb = tn * kNT + rl + 4 * h;  // row of element 0; element 4 gq + c is row nb + 8 gq + c
        if constexpr (MODE == 0) {
          if (qv) {
            float *o = out + (size_t)q * N + nb;
            if (full) {
#pragma unroll
              for (int gq = 0; gq < 4; gq++)
                *reinterpret_cast<float4 *>(o + 8 * gq) =
                    make_float4(e[4 * gq], e[4 * gq + 1], e[4 * gq + 2], e[4 * gq + 3]);
            } else {
#pragma unroll
              for (int j = 0; j < 16; j++)
                if (nb + 8 * (j >> 2) + (j & 3) < N) o[8 * (j >> 2) + (j & 3)] = e[j];
            }
          }
        } else {
          // rows that pass, one bit per element; one counter reservation per lane and block, then plain stores
          uint32_t pm = 0;
#pragma unroll
          for (int j = 0; j < 16; j++) pm |= (e[j] >= th ? 1u : 0u) << j;
          if (!qv) pm = 0;
          if (!full) {
#pragma unroll
            for (int j = 0; j < 16; j++)
              if (nb + 8 * (j >> 2) + (j & 3) >= N) pm &= ~(1u << j);
          }
          if (__ballot(pm != 0)) {
            if (pm) {
              int k = atomicAdd(&cnt[q], __popc(pm));
#pragma unroll
              for (int j = 0; j < 16; j++) {
                if ((pm >> j) & 1) {
                  if (k < CAP) {
                    bval[(size_t)q * CAP + k] = e[j];
                    bpos[(size_t)q * CAP + k] = nb + 8 * (j >> 2) + (j & 3);
                  }
                  ++k;
                }
              }
            }
          }
        }
      }
    }
  };

  // One stage: its operands in (LQ, LZ); the request side fills (NQ, NZ), the buffers of the stage before.
  // The last stage of a tile runs the tile's epilogue before that request, so the epilogue's global
  // accesses are older than every request still pending at the next barrier.
  auto stage = [&](v4i (&L)[kBR][kSS][64], v4i (&NL)[kBR][kSS][64]) {
    const bool last = cst == nst - 1;
    const bool more = !(last && ck == my_tiles - 1);  // a next stage exists: its requests are in flight
    stage_barrier(more ? kDMA + (last ? tile_requests<MODE>(w) : 0) : -1);
    if (cst == 0) {
#pragma unroll
      for (int i = 0; i < 2; i++)
#pragma unroll
        for (int rb = 0; rb < 4; rb++) acc[i][rb] = (v16i){0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
    }
    if (!last) request(NL);
    // operands of K step s + 1 are read from LDS while the MFMAs of step s run
    v4i za[2][4], qf[2][2];
    auto fetch = [&](int s, int b) {
#pragma unroll
      for (int rb = 0; rb < 4; rb++) za[b][rb] = L[kQB + 4 * wn + rb][s][lane];
#pragma unroll
      for (int i = 0; i < 2; i++) qf[b][i] = L[2 * wq + i][s][lane];
    };
    fetch(0, 0);
#pragma unroll
    for (int s = 0; s < kSS; s++) {
      if (s + 1 < kSS) fetch(s + 1, (s + 1) & 1);
#pragma unroll
      for (int i = 0; i < 2; i++)
#pragma unroll
        for (int rb = 0; rb < 4; rb++)
          acc[i][rb] = __builtin_amdgcn_mfma_i32_32x32x32_i8(za[s & 1][rb], qf[s & 1][i], acc[i][rb], 0, 0, 0);
    }
    if (last) {
      epilogue();
      request(NL);
      cst = 0;
      ++ck;
      cpar = cpar == 2 ? 0 : cpar + 1;
    } else {
      ++cst;
    }
  };
  request(ls0);
  request(ls1);
  for (int g = 0; g < nstages; g += 3) {
    stage(ls0, ls2);
    if (g + 1 < nstages) stage(ls1, ls0);
    if (g + 2 < nstages) stage(ls2, ls1);
  }
}

// t0[q] = the r-th largest of S[q][0 .. n) (the reference's topk(r).values[:, -1]); cnt[q] = 0 for the emit
// pass that follows. One workgroup per query, radix selection over order-preserving keys.
__global__ __launch_bounds__(256) void k_row_kth(const float *__restrict__ S, int n, int r, float *__restrict__ t0,
                                                 int32_t *__restrict__ cnt) {
  __shared__ int hist[256];
  __shared__ int sh[fvs_sh_ints(256)];
  const int64_t q = blockIdx.x;
  const float *row = S + q * (int64_t)n;
  const uint32_t k = fvs_block_kth<uint32_t, 256>([&](int i) { return fvs_ord32(row[i]); }, n, r, hist, sh);
  if (threadIdx.x == 0) {
    t0[q] = fvs_unord32(k);
    if (cnt) cnt[q] = 0;
  }
}

// The same selection for rows of at most 64 K values: one 1024-thread block per query loads the row once
// into registers (64 ordered keys per thread) and runs the four 8-bit radix passes over them, with one
// histogram per wave in LDS (fewer collisions on the busy bins), instead of re-reading the row from
// memory in every pass.
constexpr int kKthNT = 1024, kKthPer = 64;

__global__ __launch_bounds__(kKthNT) void k_row_kth_reg(const float *__restrict__ S, int n, int r,
                                                        float *__restrict__ t0, int32_t *__restrict__ cnt) {
  constexpr int NW = kKthNT / 64;
  __shared__ int hist[NW][256];
  __shared__ int tot[256];
  __shared__ int sh[fvs_sh_ints(kKthNT)];
  const int tid = threadIdx.x, w = fvs_wave_id();
  const int64_t q = blockIdx.x;
  const float *row = S + q * (int64_t)n;
  uint32_t key[kKthPer];
#pragma unroll
  for (int j = 0; j < kKthPer; j++) {
    const int i = j * kKthNT + tid;
    key[j] = i < n ? fvs_ord32(row[i]) : 0u;
  }
  uint32_t prefix = 0, pmask = 0;
  int k = r;
  for (int shift = 24; shift >= 0; shift -= 8) {
    for (int i = tid; i < NW * 256; i += kKthNT) (&hist[0][0])[i] = 0;
    __syncthreads();
#pragma unroll
    for (int j = 0; j < kKthPer; j++)
      if (j * kKthNT + tid < n && (key[j] & pmask) == prefix) atomicAdd(&hist[w][(key[j] >> shift) & 0xff], 1);
    __syncthreads();
    if (tid < 256) {
      int t = 0;
#pragma unroll
      for (int v = 0; v < NW; v++) t += hist[v][tid];
      tot[tid] = t;
    }
    __syncthreads();
    if (w == 0) fvs_pick_bucket<NW>(tot, sh, k);
    __syncthreads();
    prefix |= (uint32_t)sh[NW] << shift;
    pmask |= 0xffu << shift;
    k = sh[NW + 1];
    __syncthreads();  // every thread has read sh before the next pass's bucket choice rewrites it
  }
  if (tid == 0) {
    t0[q] = fvs_unord32(prefix);
    if (cnt) cnt[q] = 0;
  }
}

// int8 code of each row of z [n, R] (f32): scale = max(max_j |z[j]|, 1e-12f) / 127, code = clamp(rint(z / scale),
// -127, 127), the rule of throughput/brute.py:39-41 and :46-48 for any R. One wave per row.
__global__ __launch_bounds__(256) void k_quantize(const float *__restrict__ z, int64_t n, int R, int8_t *__restrict__ q,
                                                  float *__restrict__ scale, uint16_t *__restrict__ scale16) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + fvs_wave_id();
  if (row >= n) return;
  const float *zr = z + row * R;
  float mx = 0.f;
  for (int j = lane; j < R; j += 64) mx = fmaxf(mx, fabsf(zr[j]));
  mx = fvs_wave_max(mx);
  const float a = fmaxf(mx, 1e-12f) / 127.0f;
  for (int j = lane; j < R; j += 64) q[row * R + j] = (int8_t)fminf(fmaxf(rintf(zr[j] / a), -127.f), 127.f);
  if (lane == 0) {
    if (scale) scale[row] = a;
    if (scale16) scale16[row] = fvs_f2h(a);
  }
}

}  // namespace

extern "C" int fvs_dense_pack(const int8_t *X, int64_t n, int32_t R, int64_t npad, int32_t Rp, int8_t *T,
                              void *stream) {
  if (n < 0 || R <= 0 || R % 16 != 0 || Rp < R || Rp % 32 != 0 || npad < n || npad % 32 != 0) return FVS_E_ARG;
  if (npad == 0) return FVS_OK;
  if (!T || (n > 0 && !X)) return FVS_E_ARG;
  if ((reinterpret_cast<uintptr_t>(X) | reinterpret_cast<uintptr_t>(T)) & 15) return FVS_E_ARG;
  const int64_t nblk = npad / 32;
  const int64_t total = nblk * (Rp / 32) * 64;
  const unsigned grid = (unsigned)std::min<int64_t>((total + 255) / 256, 65536);
  hipLaunchKernelGGL(k_dense_pack, dim3(grid), dim3(256), 0, (hipStream_t)stream, X, n, (int)R, (int)(Rp / 32), nblk,
                     T);
  return fvs_launch_status();
}

extern "C" int fvs_dense_threshold(const float *S, int64_t B, int32_t n, int32_t r, float *t0, int32_t *cnt,
                                   void *stream) {
  if (B < 0 || n <= 0 || r <= 0 || r > n) return FVS_E_ARG;
  if (B == 0) return FVS_OK;
  if (!S || !t0) return FVS_E_ARG;
  if (n <= kKthNT * kKthPer)
    hipLaunchKernelGGL(k_row_kth_reg, dim3((unsigned)B), dim3(kKthNT), 0, (hipStream_t)stream, S, (int)n, (int)r, t0, cnt);
  else
    hipLaunchKernelGGL(k_row_kth, dim3((unsigned)B), dim3(256), 0, (hipStream_t)stream, S, (int)n, (int)r, t0, cnt);
  return fvs_launch_status();
}

extern "C" int fvs_dense_scan(int32_t mode, const int8_t *Qt, const float *qs, int64_t B, int64_t Bpad,
                              const int8_t *Zt, const uint16_t *zs, int64_t N, int64_t Npad, int32_t R, const float *t0,
                              int32_t *cnt, float *bval, int32_t *bpos, int32_t CAP, float *out, void *stream) {
  if (mode != 0 && mode != 1) return FVS_E_ARG;
  if (B < 0 || N < 0 || R <= 0 || R % (32 * kSS) != 0) return FVS_E_SHAPE;
  if (Bpad < B || Bpad % kQT != 0 || Npad < N || Npad % kNT != 0) return FVS_E_ARG;
  if (B == 0 || N == 0) return FVS_OK;
  if (!Qt || !qs || !Zt || !zs) return FVS_E_ARG;
  if ((reinterpret_cast<uintptr_t>(Qt) | reinterpret_cast<uintptr_t>(Zt)) & 15) return FVS_E_ARG;
  if (mode == 0 && !out) return FVS_E_ARG;
  if (mode == 1 && (!t0 || !cnt || !bval || !bpos || CAP <= 0)) return FVS_E_ARG;
  if (Bpad > (int64_t)1 << 24 || Npad > ((int64_t)1 << 31) - kNT) return FVS_E_CAPACITY;
  const int ntq = (int)(Bpad / kQT);
  const int64_t ntiles = (int64_t)ntq * (Npad / kNT);
  if (ntiles > ((int64_t)1 << 30)) return FVS_E_CAPACITY;
  const int cus = fvs_cu_count();
  const int m8 = std::max(1, kWGCU * cus / 8);  // workgroups per XCD
  const dim3 grid((unsigned)(8 * m8)), block(256);
  hipStream_t st = (hipStream_t)stream;
  if (mode == 0)
    hipLaunchKernelGGL(k_dense_scan<0>, grid, block, 0, st, Qt, qs, (int)B, Zt, zs, (int)N, (int)(R / 32), ntq, (int)ntiles, m8, t0,
                       cnt, bval, bpos, CAP, out);
  else
    hipLaunchKernelGGL(k_dense_scan<1>, grid, block, 0, st, Qt, qs, (int)B, Zt, zs, (int)N, (int)(R / 32), ntq, (int)ntiles, m8, t0,
                       cnt, bval, bpos, CAP, out);
  return fvs_launch_status();
}

extern "C" int fvs_quantize_i8(const float *z, int64_t n, int32_t R, int8_t *q, float *scale, uint16_t *scale16,
                               void *stream) {
  if (n < 0 || R <= 0) return FVS_E_ARG;
  if (n == 0) return FVS_OK;
  if (!z || !q) return FVS_E_ARG;
  hipLaunchKernelGGL(k_quantize, dim3((unsigned)((n + 3) / 4)), dim3(256), 0, (hipStream_t)stream, z, n, (int)R, q, scale,
                     scale16);
  return fvs_launch_status();
}
