// int8 stage-1 scans on gfx950 MFMA (v_mfma_i32_16x16x64_i8): the first pass (block maxima) and the
// threshold-and-emit pass.
//
// Work item = (cell, up to 128 consecutive rows of it from a first row r0), run by a workgroup of two waves,
// each wave holding 64 of the rows as four 16-row blocks. The first pass needs the reference's global
// 32-row blocks (its block maxima are per global block), so its items start on a multiple of 32; the emit
// pass, whose output does not depend on the grouping, takes items that start at the cell's first row (a
// cell of up to 128 rows is one item, with no block straddling the cell start). Each code byte is read from
// HBM once per pass: a wave keeps its code rows as MFMA operands in registers for the whole item, and the
// cell's queries stream through in tiles of 16:
//   * the item's pair list (query id, query scale, centre term, threshold or probe rank) and the row
//     scales of its rows are staged in LDS up front (kFMeta / kMetaE pairs at a time);
//   * a tile's query fragments are written straight into LDS by the vector memory unit (global_load_lds,
//     no registers), in MFMA-step order so that every fragment read is one contiguous 1 KB ds_read_b128 per
//     wave. The buffer is double-buffered and shared by the workgroup's waves: each wave requests its share
//     of tile t + 1 while tile t is computed, and one barrier per tile publishes it.
// Both passes are persistent: a workgroup loops over items (grid = resident workgroups), and the next
// item's pair ids, row scales and code rows are requested as soon as the current item's tile loop is done.
//
// Operand layout (16 x 16 x 64): for MFMA step s (64 bytes of the code), lane l holds the 16 bytes at
// 64 s + 16 (l >> 4) of row / column l & 15; both operands use the same assignment, so the contraction is
// exact for any internal k order. Accumulator element i of lane l is D[4 (l >> 4) + i][l & 15].
//
// The item's row scales sit in LDS; rows outside the cell get a NaN scale: their estimate is NaN,
// which never passes `est >= t0` and is ignored by fmaxf, so no per-element row mask is needed.
//
// The reference-signature seam (fvs_i8_scan_civf8, k_i8_civf8 at the end of this file) keeps its own
// one-block items on v_mfma_i32_32x32x32_i8.
#include <type_traits>

#include "fvs_common.h"

namespace {

constexpr int kR = 256;

// row of accumulator element v in the 32x32 layout, for lanes of half h = l / 32
__device__ __forceinline__ int acc_row(int v, int h) { return 8 * (v >> 2) + 4 * h + (v & 3); }

struct Meta {  // one (query, cell) pair of the item
  int qid;     // query
  float qs;    // query code scale
  float qcp;   // centre term of the pair
  float x;     // emit pass: threshold t0 of the query; first pass: probe rank (int bits)
};

// ------------------------------------------------------------------ the first pass (mode 0)
// A two-wave workgroup runs an item of up to four global 32-row blocks (128 rows from a multiple of 32):
// wave w keeps global blocks 2w and 2w + 1 as four 16-row blocks of v_mfma_i32_16x16x64_i8 A operands (the
// code rows; 64 VGPRs), and the cell's queries are the B operand, in tiles of 16 (4 KB, each wave requesting
// two of the four MFMA steps). Accumulator element i of lane l is row 4 (l >> 4) + i of the 16-row block
// against query l & 15 of the tile, so a lane reduces the 8 rows it holds of a global block in registers and
// two xor exchanges (lanes 16 and 32 apart) finish the block maximum of its query:
//   bm[(q * n1 + qrank[pair]) * MB + blk - cs/32] = max over the block's rows of fmaf((float)acc * qs, zs, qcp).
// Eight workgroups (sixteen waves) per CU: at most 128 VGPRs and 12.5 KB of LDS each. Against four-wave
// workgroups on 256-row items (three per CU) the scan has twice as many waves in flight to hide each item's
// dependent loads (its pair ids, their query scales, the first query tile), which is what bounds it.
constexpr int kFW = 2;            // waves per first-pass workgroup
constexpr int kFT = 64 * kFW;     // threads per first-pass workgroup
constexpr int kFRows = 64 * kFW;  // rows of a first-pass item
constexpr int kFMeta = 256;       // pairs staged in LDS at a time
constexpr int kFirstWG = 8;       // resident first-pass workgroups per CU

__global__ __launch_bounds__(kFT, 4) void k_i8_first(
    const int8_t *__restrict__ q8, const float *__restrict__ qs, const int32_t *__restrict__ qid,
    const int32_t *__restrict__ qrank, const int32_t *__restrict__ coff, const int32_t *__restrict__ ccnt,
    const int32_t *__restrict__ pcell, const int32_t *__restrict__ prow, const int32_t *__restrict__ ps,
    const int32_t *__restrict__ pe, int P, const int8_t *__restrict__ Z, const float *__restrict__ zs,
    const float *__restrict__ qcp, float *__restrict__ bm, int MB, int n1) {
  __shared__ __align__(16) Meta meta[kFMeta];
  __shared__ __align__(16) float zsl[kFRows];
  __shared__ __align__(16) v4i bsh[2][4 * 64];  // query tiles: [step s][lane], 16 B each
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = fvs_wave_id();
  const int g4 = lane >> 4, l16 = lane & 15;
  struct Item {
    int qn, qoff, r0, cs, ce;
  };
  auto item_at = [&](int p) {
    Item u{0, 0, 0, 0, 0};
    if (p < P) {
      const int c = pcell[p];
      u.r0 = prow[p];
      u.cs = ps[p];
      u.ce = min(u.r0 + kFRows, pe[p]);
      if (u.r0 < u.ce) {
        u.qn = ccnt[c];
        u.qoff = coff[c];
      }
    }
    return u;
  };
  int pq[kFMeta / kFT];
  float zr;
  v4i cb[4][4];  // this wave's code rows: 16-row block b, MFMA step s
  auto prefetch = [&](const Item &u) {
    if (u.qn == 0) return;
#pragma unroll
    for (int i = 0; i < kFMeta / kFT; i++) {
      const int j = tid + kFT * i;
      pq[i] = j < min(kFMeta, u.qn) ? qid[u.qoff + j] : 0;
    }
    {
      const int r = u.r0 + tid;
      zr = (r >= u.cs && r < u.ce) ? zs[r] : __builtin_nanf("");
    }
#pragma unroll
    for (int b = 0; b < 4; b++) {
      const int r = u.r0 + 64 * w + 16 * b + l16;
      const int64_t rr = r < u.ce ? r : u.ce - 1;  // rows past the cell carry a NaN scale
      const v4i *zp = reinterpret_cast<const v4i *>(Z + rr * kR + 16 * g4);
#pragma unroll
      for (int s = 0; s < 4; s++) cb[b][s] = zp[4 * s];
    }
  };

  const int stride = (int)gridDim.x;
  int p = blockIdx.x;
  Item cur = item_at(p);
  prefetch(cur);
  while (p < P) {
    const Item nxt = item_at(p + stride);
    if (cur.qn == 0) {
      prefetch(nxt);
      cur = nxt;
      p += stride;
      continue;
    }
    const int qn = cur.qn, qoff = cur.qoff, cs = cur.cs, row0 = cur.r0;
    zsl[tid] = zr;
    const int wrows = cur.ce - row0 - 64 * w;
    const int nact = wrows <= 0 ? 0 : min(4, (wrows + 15) >> 4);  // 16-row blocks with rows of the cell
    for (int c0 = 0; c0 < qn; c0 += kFMeta) {
      const int nq = min(kFMeta, qn - c0);
      if (c0 > 0) {
#pragma unroll
        for (int i = 0; i < kFMeta / kFT; i++) {
          const int j = tid + kFT * i;
          pq[i] = j < nq ? qid[qoff + c0 + j] : 0;
        }
      }
#pragma unroll
      for (int i = 0; i < kFMeta / kFT; i++) {
        const int j = tid + kFT * i;
        if (j < nq) {
          const int pidx = qoff + c0 + j;
          const int q = pq[i];
          Meta m;
          m.qid = q;
          m.qs = qs[q];
          m.qcp = qcp[pidx];
          m.x = __int_as_float(qrank[pidx]);
          meta[j] = m;
        }
      }
      __syncthreads();
      const int ntiles = (nq + 15) / 16;
      auto request = [&](int tile) {
        const int8_t *src = q8 + (int64_t)meta[min(tile * 16 + l16, nq - 1)].qid * kR + 16 * g4;
#pragma unroll
        for (int i = 0; i < 4 / kFW; i++) {
          const int s = (4 / kFW) * w + i;
          __builtin_amdgcn_global_load_lds(src + 64 * s, (__attribute__((address_space(3))) void *)&bsh[tile & 1][s * 64],
                                           16, 0, 0);
        }
      };
      auto published = [&]() {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
      };
      auto tiles = [&](auto NB_) {
        constexpr int NB = decltype(NB_)::value;
        for (int t = 0; t < ntiles; t++) {
          if (t + 1 < ntiles) request(t + 1);
          v4i qb[4];
#pragma unroll
          for (int s = 0; s < 4; s++) qb[s] = bsh[t & 1][s * 64 + lane];
          v4i A[NB];
#pragma unroll
          for (int s = 0; s < 4; s++)
#pragma unroll
            for (int b = 0; b < NB; b++)
              A[b] = __builtin_amdgcn_mfma_i32_16x16x64_i8(cb[b][s], qb[s], s == 0 ? (v4i){0, 0, 0, 0} : A[b], 0, 0, 0);
          const int jl = t * 16 + l16;
          const bool valid = jl < nq;
          const Meta m = meta[valid ? jl : nq - 1];
#pragma unroll
          for (int gb = 0; gb < (NB + 1) / 2; gb++) {
            float mx = -1e30f;
#pragma unroll
            for (int bb = 0; bb < 2; bb++) {
              const int b = 2 * gb + bb;
              if (b < NB) {
                const float4 z4 = *reinterpret_cast<const float4 *>(&zsl[64 * w + 16 * b + 4 * g4]);
                const float zz[4] = {z4.x, z4.y, z4.z, z4.w};
#pragma unroll
                for (int i = 0; i < 4; i++) mx = fmaxf(mx, __builtin_fmaf((float)A[b][i] * m.qs, zz[i], m.qcp));
              }
            }
            mx = fmaxf(mx, __shfl_xor(mx, 16, FVS_WAVE));
            mx = fmaxf(mx, __shfl_xor(mx, 32, FVS_WAVE));
            if (g4 == 0 && valid)
              bm[((int64_t)m.qid * n1 + __float_as_int(m.x)) * MB + ((row0 >> 5) + 2 * w + gb - (cs >> 5))] = mx;
          }
          published();
        }
      };
      request(0);
      published();
      switch (nact) {
        case 4: tiles(std::integral_constant<int, 4>{}); break;
        case 3: tiles(std::integral_constant<int, 3>{}); break;
        case 2: tiles(std::integral_constant<int, 2>{}); break;
        case 1: tiles(std::integral_constant<int, 1>{}); break;
        default:
          for (int t = 0; t < ntiles; t++) {
            if (t + 1 < ntiles) request(t + 1);
            published();
          }
      }
      __syncthreads();  // every wave is past meta before the next chunk restages it
    }
    prefetch(nxt);
    cur = nxt;
    p += stride;
  }
}

// ------------------------------------------------------------------ the emit pass (mode 1)
// The emit pass has the first pass's shape with the operands swapped: a workgroup of two waves takes a cell
// and up to 128 of its rows (64 per wave, as four 16-row blocks), and the cell's queries in tiles of 16, on
// v_mfma_i32_16x16x64_i8. Cells are skewed (a tenth hold under 16 rows), so 128-row items leave few waves
// without rows (about 4 % of the wave-steps, against 28 % for four-wave items of 256 rows), and 16-row
// blocks leave few empty rows in the blocks that are computed. The persistent grid walks the items in list
// order with a stride of the grid size; the engine's list (index.row_chunks(off, 128)) has about 6.5 items
// per workgroup at 1M rows, so the busiest workgroup runs 7.
//
// MFMA layout (16 x 16 x 64, int8): for step s (64 bytes of the code), lane l holds 16 bytes 64 s + 16 (l >> 4)
// .. + 15 of A row l & 15 (a query of the tile) and of B column l & 15 (a code row of the block); both use
// the same assignment, so the contraction is exact for any internal order. Accumulator element i of lane l is
// D[4 (l >> 4) + i][l & 15]: query 4 (l >> 4) + i of the tile against row l & 15 of the block. A wave ballot
// of one element covers 16 rows of four queries; passing rows cluster by query, so most ballots are empty.
// The tile's fragments (16 queries, 4 KB) go straight into LDS by the vector memory unit (global_load_lds),
// in MFMA-step order [s][lane], double-buffered; each wave requests two of the four steps of tile t + 1
// while tile t is computed, one barrier per tile.
//
// Per element the tile loop evaluates a conservative prefilter instead of the canonical estimate:
//   g = fmaf((float)acc, z, 2z) >= T[q],  T[q] = (t0 - qcp)/qs - 2^-20 (|t0| + |qcp|)/qs  (f32 ops).
// With u = 2^-24, |acc| <= 2^22 (any int8 operands: 256 * 128 * 128), qs > 0 and z >= 0:
// est = fmaf(RN(acc*qs), z, qcp) >= t0 implies acc*z >= (t0 - qcp)/qs - u|qcp|/qs - 3u|acc*z|
// >= (t0 - qcp)/qs - u|qcp|/qs - 0.75 z, while g >= acc*z + 2z - u|acc*z + 2z| >= acc*z + 1.74 z, and the
// rounding of T's three operations is far below its 2^-20 margin; so every element whose estimate passes
// also passes the prefilter. (A query with qs <= 0 or an overflowing T gets T = -inf, a row scale that is
// negative or infinite the addend +inf: the prefilter then admits every query of the chunk, and the exact
// test decides; the missing queries of a last partial tile have a NaN threshold, which nothing passes.) Per
// element that is a convert, an fma and a compare; the tests of two blocks (eight elements) are made before
// one branch on the OR of their ballots skips the group.
//
// The passing elements are staged as (accumulator, tag) in the wave's LDS region. The flush computes the
// canonical estimate of each, fmaf((float)acc * qs, zs, qcp), drops those below t0 (the few the
// prefilter admits in excess), numbers the rest per pair with LDS atomics, reserves each query's range
// with one global atomic per (item, query) and writes them out. So the emitted set and its estimates are
// exactly those of the canonical formula; their order in a query's buffer is unspecified.
//
// Six workgroups (twelve waves) per CU: at most 168 VGPRs and 23 KB of LDS each. An item's pairs are
// processed in chunks of up to kMetaE queries; a chunk whose candidates overflow a wave's region is dropped
// and scanned again with half as many queries, down to 8 queries, whose 8 x 64 = 512 candidates per wave
// always fit in its kCapE = 512 slots.
constexpr int kEW = 2;         // waves per emit workgroup
constexpr int kET = 64 * kEW;  // threads per emit workgroup
constexpr int kERows = 64 * kEW;  // rows of an emit item
constexpr int kTQ = 16;        // queries per tile
constexpr int kMetaE = 256;    // pairs staged in LDS at a time
constexpr int kCapE = 512;     // LDS candidate slots per wave
constexpr int kEmitWG = 6;     // resident emit workgroups per CU
static_assert(8 * 64 <= kCapE, "an 8-query chunk must fit a wave's region");

struct EmitStage {
  int acc[kEW][kCapE];       // dot products of the staged elements; the estimate after the exact test
  uint32_t tag[kEW][kCapE];  // row - first row of the item (bits 0-7) | pair index (8-19) | number (20-31)
  uint32_t lcnt[kMetaE];     // candidates of each pair in the item; then the pair's base in its query's buffer
  int n[kEW];
};

__device__ __forceinline__ float emit_prefilter_T(float th, float qc, float qsv) {
  if (!(qsv > 0.f)) return -__builtin_inff();
  const float b = (th - qc) / qsv;
  const float m = (fabsf(th) + fabsf(qc)) * (0x1p-20f / qsv);
  const float T = b - m;
  if (!(T < __builtin_inff())) return th == __builtin_inff() ? __builtin_inff() : -__builtin_inff();
  return T;
}

__global__ __launch_bounds__(kET, 3) void k_i8_emit(
    const int8_t *__restrict__ q8, const float *__restrict__ qs, const int32_t *__restrict__ qid,
    const int32_t *__restrict__ coff, const int32_t *__restrict__ ccnt, const int32_t *__restrict__ pcell,
    const int32_t *__restrict__ prow, const int32_t *__restrict__ ps, const int32_t *__restrict__ pe, int P,
    const int8_t *__restrict__ Z, const float *__restrict__ zs, const float *__restrict__ qcp,
    const float *__restrict__ t0, int32_t *__restrict__ cnt, float *__restrict__ bval, int32_t *__restrict__ bpos,
    int CAP) {
  __shared__ __align__(16) Meta meta[kMetaE];
  __shared__ __align__(16) float Tl[kMetaE + kTQ];
  __shared__ __align__(16) float zsl[kERows];
  __shared__ __align__(16) v4i bsh0[4 * 64];  // query tiles of even index: [step s][lane], 16 B each
  __shared__ __align__(16) v4i bsh1[4 * 64];  // query tiles of odd index
  __shared__ EmitStage S;
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = fvs_wave_id();
  const int g4 = lane >> 4, l16 = lane & 15;
  // item p: rows [lo, ce) with lo = max(prow, ps) and ce = min(prow + 128, pe), in 16-row blocks from prow;
  // qn = 0 marks an item without rows or queries
  struct Item {
    int qn, qoff, r0, lo, ce;
  };
  auto item_at = [&](int p) {
    Item u{0, 0, 0, 0, 0};
    if (p < P) {
      const int c = pcell[p];
      u.r0 = prow[p];
      u.lo = max(u.r0, ps[p]);
      u.ce = min(u.r0 + kERows, pe[p]);
      if (u.lo < u.ce) {
        u.qn = ccnt[c];
        u.qoff = coff[c];
      }
    }
    return u;
  };
  int pq[kMetaE / kET];  // pair ids of the item's first chunk
  float zr;              // this thread's row scale of the item (NaN outside the cell)
  v4i cb[4][4];          // this wave's code rows: block b (16 rows), MFMA step s (64 bytes)
  auto prefetch = [&](const Item &u) {
    if (u.qn == 0) return;
#pragma unroll
    for (int i = 0; i < kMetaE / kET; i++) {
      const int j = tid + kET * i;
      pq[i] = j < min(kMetaE, u.qn) ? qid[u.qoff + j] : 0;
    }
    {
      const int r = u.r0 + tid;
      zr = (r >= u.lo && r < u.ce) ? zs[r] : __builtin_nanf("");
    }
#pragma unroll
    for (int b = 0; b < 4; b++) {
      const int r = u.r0 + 64 * w + 16 * b + l16;
      const int64_t rr = r < u.ce ? r : u.ce - 1;  // rows past the cell carry a NaN scale
      const v4i *zp = reinterpret_cast<const v4i *>(Z + rr * kR + 16 * g4);
#pragma unroll
      for (int s = 0; s < 4; s++) cb[b][s] = zp[4 * s];
    }
  };

  const int stride = (int)gridDim.x;
  int p = blockIdx.x;
  Item cur = item_at(p);
  prefetch(cur);
  while (p < P) {
    const Item nxt = item_at(p + stride);
    if (cur.qn == 0) {
      prefetch(nxt);
      cur = nxt;
      p += stride;
      continue;
    }
    const int qn = cur.qn, qoff = cur.qoff;
    const int row0 = cur.r0;
    zsl[tid] = zr;
    int ebase = 0;  // wave-uniform: used slots of this wave's region (may exceed kCapE: overflow)
    int nq = 0;     // queries of the current pair chunk
    const int wrows = cur.ce - row0 - 64 * w;  // rows of this wave's 64 (<= 0: none)
    const int nact = wrows <= 0 ? 0 : min(4, (wrows + 15) >> 4);  // blocks with rows of the cell

    // the tile loop over the current chunk's nq pairs (staged in meta / Tl)
    auto scan = [&]() {
      const int ntiles = (nq + kTQ - 1) / kTQ;
      // tile t's fragments go to bsh0 (t even) or bsh1 (t odd): global_load_lds, 16 B per lane; wave w
      // requests steps 2w and 2w + 1
      // this lane's query in a tile; the tile loop reads it from LDS one tile ahead of the request, so the
      // LDS read is off the critical path of the request
      auto tile_q = [&](int tile) { return meta[min(tile * kTQ + l16, nq - 1)].qid; };
      auto request = [&](int q, v4i *buf) {
        const int8_t *src = q8 + (int64_t)q * kR + 16 * g4;
#pragma unroll
        for (int i = 0; i < 4 / kEW; i++) {
          const int s = (4 / kEW) * w + i;
          __builtin_amdgcn_global_load_lds(src + 64 * s, (__attribute__((address_space(3))) void *)&buf[s * 64], 16,
                                           0, 0);
        }
      };
      auto published = [&]() {  // this wave's requests have landed in LDS; every wave is past the reads
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
      };
      // this lane's row scale per block and the prefilter's addend; rows outside the cell have a NaN scale
      // and never pass
      float zl[4], nd[4];
#pragma unroll
      for (int b = 0; b < 4; b++) {
        const float z = zsl[64 * w + 16 * b + l16];
        const bool fin = z >= 0.f && z < __builtin_inff();
        zl[b] = fin || z != z ? z : 0.f;
        nd[b] = fin || z != z ? z + z : __builtin_inff();
      }
      // tile loop of a wave with NB blocks of rows: step t requests tile t + 1 into the other buffer (every
      // wave has passed the barrier that ended tile t - 1), computes tile t and waits for tile t + 1
      auto tiles = [&](auto NB_) {
        constexpr int NB = decltype(NB_)::value;
        v4i qa[4];
        int qn1 = tile_q(1);  // this lane's query of tile t + 1
        for (int t = 0; t < ntiles; t++) {
          const v4i *cur_t = (t & 1) ? bsh1 : bsh0;
          if (t + 1 < ntiles) request(qn1, (t & 1) ? bsh0 : bsh1);
          qn1 = tile_q(t + 2);
#pragma unroll
          for (int s = 0; s < 4; s++) qa[s] = cur_t[s * 64 + lane];
          v4i A[NB];
#pragma unroll
          for (int s = 0; s < 4; s++)
#pragma unroll
            for (int b = 0; b < NB; b++)
              A[b] = __builtin_amdgcn_mfma_i32_16x16x64_i8(qa[s], cb[b][s], s == 0 ? (v4i){0, 0, 0, 0} : A[b], 0, 0, 0);
          const float4 T4 = *reinterpret_cast<const float4 *>(&Tl[kTQ * t + 4 * g4]);
          const float Tv[4] = {T4.x, T4.y, T4.z, T4.w};
          const uint32_t tagt = (uint32_t)(kTQ * t + 4 * g4) << 8;
          // two blocks (eight tests) at a time: their tests issue back to back, and one branch on the OR of
          // the eight ballots skips the group
#pragma unroll
          for (int b0 = 0; b0 < NB; b0 += 2) {
            bool pass_[2][4];
            uint64_t bal[2][4];
            uint64_t anyb = 0;
#pragma unroll
            for (int bb = 0; bb < 2; bb++)
#pragma unroll
              for (int i = 0; i < 4; i++) {
                const int b = b0 + bb < NB ? b0 + bb : b0;
                pass_[bb][i] = b0 + bb < NB && __builtin_fmaf((float)A[b][i], zl[b], nd[b]) >= Tv[i];
                bal[bb][i] = __ballot(pass_[bb][i]);
                anyb |= bal[bb][i];
              }
            if (anyb) {
#pragma unroll
              for (int bb = 0; bb < 2; bb++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                  const int b = b0 + bb < NB ? b0 + bb : b0;
                  if (bal[bb][i]) {
                    const int pop = __popcll(bal[bb][i]);
                    if (ebase + pop <= kCapE && pass_[bb][i]) {
                      const int pre = fvs_lane_prefix(bal[bb][i]);
                      (S.acc[w] + ebase)[pre] = A[b][i];
                      (S.tag[w] + ebase)[pre] = ((uint32_t)(64 * w + 16 * b + l16) | tagt) + ((uint32_t)i << 8);
                    }
                    ebase += pop;
                  }
                }
            }
          }
          published();
        }
      };
      request(tile_q(0), bsh0);
      published();
      switch (nact) {
        case 4: tiles(std::integral_constant<int, 4>{}); break;
        case 3: tiles(std::integral_constant<int, 3>{}); break;
        case 2: tiles(std::integral_constant<int, 2>{}); break;
        case 1: tiles(std::integral_constant<int, 1>{}); break;
        default:  // a wave without rows of the cell: the same barriers and requests, no compute
          for (int t = 0; t < ntiles; t++) {
            if (t + 1 < ntiles) request(tile_q(t + 1), (t & 1) ? bsh0 : bsh1);
            published();
          }
      }
    };

    // flush of the current chunk: the exact estimate of every staged element; those at or above t0 take
    // their number among their pair's candidates (LDS atomic), one global atomic per (item, query) reserves
    // the query's range, and every candidate goes to base + number
    auto flush = [&]() {
#pragma unroll
      for (int ww = 0; ww < kEW; ww++) {
        const int nn = S.n[ww];
        for (int e = tid; e < nn; e += kET) {
          const uint32_t tg = S.tag[ww][e];
          const int j = (int)((tg >> 8) & 0xfffu);
          if (j >= nq) {  // not a pair of the chunk (cannot be staged: its threshold is NaN)
            S.tag[ww][e] = 0xffffffffu;
            continue;
          }
          const Meta m = meta[j];
          const float est = __builtin_fmaf((float)S.acc[ww][e] * m.qs, zsl[tg & 0xffu], m.qcp);
          if (est >= m.x) {
            const uint32_t num = atomicAdd(&S.lcnt[j], 1u);  // < 128 rows per item
            S.acc[ww][e] = __float_as_int(est);
            S.tag[ww][e] = tg | (num << 20);
          } else {
            S.tag[ww][e] = 0xffffffffu;  // admitted by the prefilter only
          }
        }
      }
      __syncthreads();
      for (int j = tid; j < nq; j += kET) {
        const int c = (int)S.lcnt[j];
        S.lcnt[j] = c ? (uint32_t)atomicAdd(&cnt[meta[j].qid], c) : 0u;
      }
      __syncthreads();
#pragma unroll
      for (int ww = 0; ww < kEW; ww++) {
        const int nn = S.n[ww];
        for (int e = tid; e < nn; e += kET) {
          const uint32_t tg = S.tag[ww][e];
          if (tg == 0xffffffffu) continue;
          const int j = (int)((tg >> 8) & 0xfffu);
          const int idx = (int)S.lcnt[j] + (int)(tg >> 20);
          if (idx < CAP) {
            const int64_t q = meta[j].qid;
            bval[q * CAP + idx] = __int_as_float(S.acc[ww][e]);
            bpos[q * CAP + idx] = row0 + (int)(tg & 0xffu);
          }
        }
      }
      __syncthreads();  // the flush has read meta and the regions before the next chunk restages them
    };

    // The item's pairs in chunks of csz queries (kMetaE at first), each staged, scanned and flushed. A chunk
    // whose candidates overflow a wave's region is dropped and scanned again with half as many queries, down
    // to 8, whose at most 8 x 64 = 512 candidates per wave always fit in kCapE = 512 slots.
    bool pq_ok = true;  // pq holds the first kMetaE pair ids of the item
    for (int c0 = 0, csz = kMetaE;;) {
      nq = min(csz, qn - c0);
      if (!(pq_ok && c0 == 0)) {
#pragma unroll
        for (int i = 0; i < kMetaE / kET; i++) {
          const int j = tid + kET * i;
          pq[i] = j < nq ? qid[qoff + c0 + j] : 0;
        }
      }
      pq_ok = false;
#pragma unroll
      for (int i = 0; i < kMetaE / kET; i++) {
        const int j = tid + kET * i;
        if (j < nq) {
          const int pidx = qoff + c0 + j;
          const int q = pq[i];
          Meta m;
          m.qid = q;
          m.qs = qs[q];
          m.qcp = qcp[pidx];
          m.x = t0[q];
          meta[j] = m;
          Tl[j] = emit_prefilter_T(m.x, m.qcp, m.qs);
          S.lcnt[j] = 0u;
        }
      }
      // the last tile's missing queries pass nothing: every compare with NaN is false, also for the +inf
      // prefilter value of a row whose scale is negative or infinite
      if (tid < kTQ) Tl[nq + tid] = __builtin_nanf("");
      ebase = 0;
      __syncthreads();
      scan();
      if (lane == 0) S.n[w] = ebase;
      __syncthreads();
      bool over = false;
#pragma unroll
      for (int ww = 0; ww < kEW; ww++) over = over || S.n[ww] > kCapE;
      if (over && csz > 8) {  // the same first pair again, with half the queries
        csz >>= 1;
        pq_ok = false;
        continue;
      }
      if (over) {
        // Unreachable: an 8-query chunk stages at most 8 x 64 = 512 <= kCapE elements per wave (the slots
        // past nq have a NaN threshold). Should it happen, the chunk's staged elements are dropped and bit
        // 30 of each of its queries' counts marks them (a count above any buffer: the query is flagged and
        // recomputed), and the scan goes on instead of halving below 8.
        for (int j = tid; j < nq; j += kET) atomicOr(&cnt[meta[j].qid], 1 << 30);
        __syncthreads();  // every thread has read the region counts
        if (tid < kEW) S.n[tid] = 0;
        __syncthreads();
      }
      if (c0 + nq >= qn) break;  // the last chunk is flushed after the next item's loads are issued
      flush();
      c0 += nq;
    }
    prefetch(nxt);  // the code rows are no longer needed: the next item's loads run under the flush
    flush();
    cur = nxt;
    p += stride;
  }
}

// ------------------------------------------------------------------ the reference's one-block work items
// civf8.launch semantics (throughput/civf8.py:89-91): one work item per (cell, global 32-row block) of
// src/s1cell.py:161-168, block maxima indexed by pair. One wave per item, four items per workgroup; the
// wave keeps the block's 32 code rows as the MFMA A operand (rows outside the cell clamped into it, their
// row scale NaN) and streams the cell's queries through as B in tiles of 32 (lane: query column l % 32,
// 16 rows of the block). No LDS and no barrier: the waves of a workgroup are independent.
//   mode 0: bmc[pair * MB + blk - cs / 32] = max over the block's rows in the cell (fmaxf from -1e30).
//   mode 1: a lane counts its query's passing rows, takes one atomic range of cnt[q] for them and writes
//           them in row order; the buffer's order is as unspecified as the reference's.
template <int MODE>
__global__ __launch_bounds__(256) void k_i8_civf8(
    const int8_t *__restrict__ q8, const float *__restrict__ qs, const int32_t *__restrict__ qid,
    const int32_t *__restrict__ coff, const int32_t *__restrict__ ccnt, const int32_t *__restrict__ pcell,
    const int32_t *__restrict__ pblk, const int32_t *__restrict__ ps, const int32_t *__restrict__ pe, int P,
    const int8_t *__restrict__ Z, const float *__restrict__ zs, const float *__restrict__ qcp,
    const float *__restrict__ t0, int32_t *__restrict__ cnt, float *__restrict__ bval, int32_t *__restrict__ bpos,
    float *__restrict__ bmc, int CAP, int MB) {
  const int lane = threadIdx.x & 63, w = fvs_wave_id();
  const int h = lane >> 5, li = lane & 31;
  const int p = blockIdx.x * 4 + w;
  if (p >= P) return;
  const int c = pcell[p];
  const int qn = ccnt[c];
  if (qn == 0) return;
  const int qoff = coff[c], blk = pblk[p], cs = ps[p], ce = pe[p];
  const int r0 = blk * 32;
  const int rr = min(max(r0 + li, cs), ce - 1);  // a row of the cell for every lane
  v4i a[8];
  const v4i *zp = reinterpret_cast<const v4i *>(Z + (int64_t)rr * kR + h * 16);
#pragma unroll
  for (int s = 0; s < 8; s++) a[s] = zp[2 * s];
  float zr[16];  // the scales of this lane's 16 rows: NaN outside the cell (never passes, ignored by fmaxf)
#pragma unroll
  for (int v = 0; v < 16; v++) {
    const int r = r0 + acc_row(v, h);
    zr[v] = (r >= cs && r < ce) ? zs[r] : __builtin_nanf("");
  }
  for (int j0 = 0; j0 < qn; j0 += 32) {
    const int j = j0 + li;
    const bool jv = j < qn;
    const int pidx = qoff + (jv ? j : qn - 1);
    const int q = qid[pidx];
    const v4i *src = reinterpret_cast<const v4i *>(q8 + (int64_t)q * kR + h * 16);
    v4i b[8];
#pragma unroll
    for (int s = 0; s < 8; s++) b[s] = src[2 * s];
    v16i acc = (v16i){0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
    for (int s = 0; s < 8; s++) acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[s], b[s], acc, 0, 0, 0);
    const float qsv = qs[q], qc = qcp[pidx];
    float ev[16];
#pragma unroll
    for (int v = 0; v < 16; v++) ev[v] = __builtin_fmaf((float)acc[v] * qsv, zr[v], qc);
    if constexpr (MODE == 0) {
      float mx = -1e30f;
#pragma unroll
      for (int v = 0; v < 16; v++) mx = fmaxf(mx, ev[v]);
      mx = fmaxf(mx, __shfl_xor(mx, 32, FVS_WAVE));
      if (h == 0 && jv) bmc[(int64_t)(qoff + j) * MB + (blk - cs / 32)] = mx;
    } else {
      const float th = jv ? t0[q] : __builtin_nanf("");  // NaN: an +inf estimate must not pass either
      uint32_t bits = 0;
#pragma unroll
      for (int v = 0; v < 16; v++) bits |= (ev[v] >= th ? 1u : 0u) << v;
      if (bits) {
        int idx = atomicAdd(&cnt[q], __builtin_popcount(bits));
#pragma unroll
        for (int v = 0; v < 16; v++) {
          if ((bits >> v) & 1u) {
            if (idx < CAP) {
              bval[(int64_t)q * CAP + idx] = ev[v];
              bpos[(int64_t)q * CAP + idx] = r0 + acc_row(v, h);
            }
            idx++;
          }
        }
      }
    }
  }
}

}  // namespace

extern "C" int fvs_i8_scan_civf8(int32_t mode, int32_t P, const int8_t *q8, const float *qs, const int32_t *qid,
                                 const int32_t *coff, const int32_t *ccnt, const int32_t *pcell, const int32_t *pblk,
                                 const int32_t *ps, const int32_t *pe, const int8_t *Z, const float *zs,
                                 const float *qcp, const float *t0, int32_t *cnt, float *bval, int32_t *bpos,
                                 float *bmc, int32_t CAP, int32_t MB, void *stream) {
  if (mode != 0 && mode != 1) return FVS_E_ARG;
  if (P < 0) return FVS_E_ARG;
  if (P == 0) return FVS_OK;
  if (!q8 || !qs || !qid || !coff || !ccnt || !pcell || !pblk || !ps || !pe || !Z || !zs || !qcp) return FVS_E_ARG;
  const dim3 grid((unsigned)((P + 3) / 4));
  hipStream_t st = (hipStream_t)stream;
  if (mode == 0) {
    if (!bmc || MB <= 0) return FVS_E_ARG;
    hipLaunchKernelGGL(k_i8_civf8<0>, grid, dim3(256), 0, st, q8, qs, qid, coff, ccnt, pcell, pblk, ps, pe, P, Z, zs,
                       qcp, t0, cnt, bval, bpos, bmc, CAP, MB);
  } else {
    if (!t0 || !cnt || !bval || !bpos || CAP <= 0) return FVS_E_ARG;
    hipLaunchKernelGGL(k_i8_civf8<1>, grid, dim3(256), 0, st, q8, qs, qid, coff, ccnt, pcell, pblk, ps, pe, P, Z, zs,
                       qcp, t0, cnt, bval, bpos, bmc, CAP, MB);
  }
  return fvs_launch_status();
}

extern "C" int fvs_i8_scan(int32_t mode, int32_t P, const int8_t *q8, const float *qs, const int32_t *qid,
                           const int32_t *qrank, const int32_t *coff, const int32_t *ccnt, const int32_t *pcell,
                           const int32_t *prow, const int32_t *ps, const int32_t *pe, const int8_t *Z,
                           const float *zs, int64_t N, int32_t R, const float *qcp, const float *t0, int32_t *cnt,
                           float *bval, int32_t *bpos, float *bm, int32_t CAP, int32_t MB, int32_t n1,
                           void *stream) {
  if (R != kR) return FVS_E_SHAPE;
  if (mode != 0 && mode != 1) return FVS_E_ARG;
  if (P < 0 || N <= 0) return FVS_E_ARG;
  if (P == 0) return FVS_OK;
  if (!q8 || !qs || !qid || !coff || !ccnt || !pcell || !prow || !ps || !pe || !Z || !zs || !qcp) return FVS_E_ARG;
  hipStream_t st = (hipStream_t)stream;
  // persistent grids: eight first-pass workgroups, six emit workgroups per CU
  if (mode == 0) {
    if (!qrank || !bm || MB <= 0 || n1 <= 0) return FVS_E_ARG;
    hipLaunchKernelGGL(k_i8_first, dim3((unsigned)min(P, kFirstWG * fvs_cu_count())), dim3(kFT), 0, st, q8, qs, qid,
                       qrank, coff, ccnt, pcell, prow, ps, pe, P, Z, zs, qcp, bm, MB, n1);
  } else {
    if (!t0 || !cnt || !bval || !bpos || CAP <= 0) return FVS_E_ARG;
    hipLaunchKernelGGL(k_i8_emit, dim3((unsigned)min(P, kEmitWG * fvs_cu_count())), dim3(kET), 0, st, q8, qs,
                       qid, coff, ccnt, pcell, prow, ps, pe, P, Z, zs, qcp, t0, cnt, bval, bpos, CAP);
  }
  return fvs_launch_status();
}
