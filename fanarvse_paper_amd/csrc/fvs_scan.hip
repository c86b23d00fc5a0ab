// int8 stage-1 scan on gfx950 MFMA (v_mfma_i32_32x32x32_i8).
//
// Work item = (cell, up to 256 consecutive rows of it from a first row r0); its 32-row blocks start at
// r0, r0 + 32, ... The first pass needs the reference's global 32-row blocks (its block maxima are per
// global block), so its items start on a multiple of 32; the emit pass, whose output does not depend on
// the grouping, takes items that start at the cell's first row (a cell of up to 256 rows is one item,
// with no block straddling the cell start). A 4-wave workgroup runs an item; wave w keeps blocks 2w and
// 2w+1 (64 code rows) as MFMA A operands in registers for the whole item, so each code byte is read from
// HBM once per pass. The cell's queries stream through as B operands in tiles of 32:
//   * the item's pair list (query id, query scale, centre term, threshold or probe rank) and the row
//     scales of its 256 rows are staged in LDS up front (kMeta pairs at a time);
//   * a tile's B fragments (its 32 query codes, 8 KB) are written straight into LDS by the vector memory
//     unit (global_load_lds, no registers), in MFMA-step order so that every fragment read is one
//     contiguous 1 KB ds_read_b128 per wave. The buffer is double-buffered and shared by the four waves:
//     each wave requests a quarter of tile t + 1 while tile t is computed, and one barrier per tile
//     publishes it.
// Two blocks per wave halve the B-fragment reads per MFMA. 168 VGPRs and 52 KB of LDS give three resident
// workgroups per CU. Both passes are persistent: a workgroup loops over items (grid = resident
// workgroups), and the next item's pair ids, row scales and code blocks are requested as soon as the
// current item's tile loop is done, under its flush.
//
// Operand layout: lane l holds row/column (l & 31) and, for MFMA step s (k-block of 32 bytes), the
// 16 bytes at 32*s + 16*(l >> 5); A and B use the same assignment, so the contraction is exact for
// any internal k order. Accumulator layout (32x32): lane l, element v holds row
// 8*(v/4) + 4*(l/32) + (v%4) and column (query) l%32, so each lane owns one query and 16 rows of a
// block; the epilogue needs only per-lane scalars for the query.
//
// The item's row scales sit in LDS; rows outside the cell get a NaN scale: their estimate is NaN,
// which never passes `est >= t0` and is ignored by fmaxf, so no per-element row mask is needed.
//
// Emit: for each accumulator element the wave takes a ballot of `est >= t0` (the compare's own lane
// mask). An empty ballot costs a scalar branch; otherwise the passing lanes, under the exec mask, take
// consecutive slots of the wave's own LDS region (a wave-uniform counter, no atomics, the overflow test
// scalar). If a wave's region overflows, the item's staged candidates are dropped and the item is redone
// on the direct path (one global atomic per candidate), which is also the path of cells probed by more
// than kMeta queries. At the end of the item every staged candidate takes its number among its pair's
// candidates with an LDS atomic, one global atomic per (item, query) reserves the query's buffer range,
// and every candidate is written out at base + number, with no per-candidate global atomics.
#include "fvs_common.h"

namespace {

constexpr int kR = 256;
constexpr int kNB = 2;       // 32-row blocks per wave
constexpr int kCB = 4 * kNB; // 32-row blocks per work item
constexpr int kMeta = 512;   // pairs staged in LDS at a time
constexpr int kCap = 768;    // LDS candidate slots per wave
constexpr bool kPersistEmit = true;  // the emit pass loops over items like the first pass

__device__ __forceinline__ int acc_row(int v, int h) { return 8 * (v >> 2) + 4 * h + (v & 3); }

struct Meta {  // one (query, cell) pair of the item
  int qid;     // query
  float qs;    // query code scale
  float qcp;   // centre term of the pair
  float x;     // mode 1: threshold t0 of the query; mode 0: probe rank (int bits)
};

struct EmitLds {
  float est[4][kCap];
  uint32_t tag[4][kCap];  // row - first row of the item (bits 0-7) | pair index in the cell (8-19) | number (20-31)
  uint32_t lcnt[kMeta];   // candidates of each pair in the item; then the pair's base in its query's buffer
  int n[4];
};

template <int MODE>
__global__ __launch_bounds__(256, 3) void k_i8_scan(
    const int8_t *__restrict__ q8, const float *__restrict__ qs, const int32_t *__restrict__ qid,
    const int32_t *__restrict__ qrank, const int32_t *__restrict__ coff, const int32_t *__restrict__ ccnt,
    const int32_t *__restrict__ pcell, const int32_t *__restrict__ prow, const int32_t *__restrict__ ps,
    const int32_t *__restrict__ pe, int P, const int8_t *__restrict__ Z, const float *__restrict__ zs, int64_t N,
    const float *__restrict__ qcp, const float *__restrict__ t0, int32_t *__restrict__ cnt,
    float *__restrict__ bval, int32_t *__restrict__ bpos, float *__restrict__ bm, int CAP, int MB, int n1) {
  __shared__ __align__(16) Meta meta[kMeta];
  __shared__ __align__(16) float zsl[32 * kCB];
  __shared__ __align__(16) v4i bsh[2][8 * 64];  // B tiles, double-buffered: [step s][half h][query li], 16 B each
  EmitLds *E = nullptr;
  if constexpr (MODE == 1) {
    __shared__ EmitLds Es;
    E = &Es;
  }
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = fvs_wave_id();
  const int h = lane >> 5, li = lane & 31;

  // Items p = blockIdx.x, blockIdx.x + gridDim.x, ...: right after an item's tile loop the next item's
  // pair ids, row scales and code blocks are requested, so their latency runs under the flush.
  struct Item {
    int p, c, qn, qoff, r0, cs, ce;  // r0: first row of the item
  };
  auto item_at = [&](int p) {
    Item it{p, 0, 0, 0, 0, 0, 0};
    if (p < P) {
      it.c = pcell[p];
      it.r0 = prow[p];
      it.cs = ps[p];
      it.ce = pe[p];
      it.qn = ccnt[it.c];
      it.qoff = coff[it.c];
    }
    return it;
  };
  int pq[kMeta / 256];  // pair ids of the item's first chunk
  float zr = 0.f;       // this thread's row scale of the item (thread < 32 * kCB)
  v4i a[kNB][8];        // this wave's blocks: the A operands
  auto prefetch = [&](const Item &it) {
    if (it.qn == 0) return;
#pragma unroll
    for (int i = 0; i < kMeta / 256; i++) {
      const int j = tid + 256 * i;
      pq[i] = j < min(kMeta, it.qn) ? qid[it.qoff + j] : 0;
    }
    if (tid < 32 * kCB) {
      const int r = it.r0 + tid;
      zr = (r >= it.cs && r < it.ce) ? zs[r] : __builtin_nanf("");
    }
#pragma unroll
    for (int u = 0; u < kNB; u++) {
      const int b0 = it.r0 + 32 * (kNB * w + u);  // first row of the block
      int64_t zr_ = (int64_t)b0 + li;
      if (b0 >= it.ce || zr_ > N - 1) zr_ = N - 1;  // rows past the cell carry a NaN scale
      const v4i *zp = reinterpret_cast<const v4i *>(Z + zr_ * kR + h * 16);
#pragma unroll
      for (int s = 0; s < 8; s++) a[u][s] = zp[2 * s];
    }
  };

  // Both passes loop over items (grid = resident workgroups, stride = grid): once an item's tile loop is
  // done (and the emit pass knows its regions did not overflow), the next item's pair ids, row scales and
  // code blocks are requested, so their latency runs under the flush.
  constexpr bool persist = MODE == 0 || kPersistEmit;
  const int stride = persist ? (int)gridDim.x : P;
  int p = blockIdx.x;
  Item cur = item_at(p);
  if constexpr (!persist) {
    if (cur.qn == 0) return;
  }
  prefetch(cur);
  while (p < P) {
    const Item nxt = persist ? item_at(p + stride) : Item{P, 0, 0, 0, 0, 0, 0};
    if (cur.qn == 0) {
      if constexpr (persist) prefetch(nxt);
      cur = nxt;
      p += stride;
      continue;
    }
    const int qn = cur.qn, qoff = cur.qoff, cs = cur.cs;
    const bool staged = MODE == 1 && qn <= kMeta;  // one pair chunk: meta holds the pairs until the flush
    const int row0 = cur.r0;  // first row of the item
    if (tid < 32 * kCB) zsl[tid] = zr;
    bool act[kNB];
#pragma unroll
    for (int u = 0; u < kNB; u++) act[u] = row0 + 32 * (kNB * w + u) < cur.ce;
    const bool any = act[0];
    int ebase = 0;  // wave-uniform: used slots of this wave's emit region (may exceed kCap: overflow)
    if constexpr (MODE == 1) {
      if (staged)
        for (int j = tid; j < qn; j += 256) E->lcnt[j] = 0u;
    }

    auto scan = [&](const bool direct, bool first) {
      for (int c0 = 0; c0 < qn; c0 += kMeta) {
        const int nq = min(kMeta, qn - c0);
        if (c0 > 0 || !first) {
#pragma unroll
          for (int i = 0; i < kMeta / 256; i++) {
            const int j = tid + 256 * i;
            pq[i] = j < nq ? qid[qoff + c0 + j] : 0;
          }
        }
#pragma unroll
        for (int i = 0; i < kMeta / 256; i++) {
          const int j = tid + 256 * i;
          if (j < nq) {
            const int pidx = qoff + c0 + j;
            const int q = pq[i];
            Meta m;
            m.qid = q;
            m.qs = qs[q];
            m.qcp = qcp[pidx];
            m.x = MODE == 0 ? __int_as_float(qrank[pidx]) : t0[q];
            meta[j] = m;
          }
        }
        __syncthreads();

        const int ntiles = (nq + 31) / 32;
        // B tile t: the fragments of the tile's 32 queries in MFMA step order, written straight into LDS by
        // the vector memory unit (global_load_lds, 16 B per lane at base + 16 * lane). Wave w requests steps
        // 2w and 2w + 1 of tile t + 1 while tile t is computed; one barrier per tile publishes it.
        auto request = [&](int tile) {
          const int jr = min(tile * 32 + li, nq - 1);
          const int8_t *src = q8 + (int64_t)meta[jr].qid * kR + h * 16;
#pragma unroll
          for (int k = 0; k < 2; k++) {
            const int s = 2 * w + k;
            __builtin_amdgcn_global_load_lds(src + 32 * s, (__attribute__((address_space(3))) void *)&bsh[tile & 1][s * 64],
                                             16, 0, 0);
          }
        };
        auto published = [&]() {
          asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's requests have landed in LDS
          __syncthreads();
        };
        {
          auto compute = [&](int t) {
            v4i b[8];
#pragma unroll
            for (int s = 0; s < 8; s++) b[s] = bsh[t & 1][s * 64 + lane];
            v16i acc[kNB];
#pragma unroll
            for (int u = 0; u < kNB; u++) {
              acc[u] = (v16i){0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
              if (act[u]) {
#pragma unroll
                for (int s = 0; s < 8; s++)
                  acc[u] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[u][s], b[s], acc[u], 0, 0, 0);
              }
            }
            const int jl = t * 32 + li;  // pair index inside the chunk
            const bool valid = jl < nq;
            const Meta m = meta[valid ? jl : nq - 1];
            const float th = MODE == 1 && valid ? m.x : __builtin_inff();
            const uint32_t tag0 = ((uint32_t)(c0 + jl) << 8) | (uint32_t)(64 * w + 4 * h);
#pragma unroll
            for (int u = 0; u < kNB; u++) {
              if (MODE == 0 && !act[u]) continue;
              // estimates of the block's 16 elements; the row scales are read from LDS up front
              float ev[16];
#pragma unroll
              for (int g = 0; g < 4; g++) {
                const float4 z4 = *reinterpret_cast<const float4 *>(&zsl[32 * (kNB * w + u) + 8 * g + 4 * h]);
                const float zz[4] = {z4.x, z4.y, z4.z, z4.w};
#pragma unroll
                for (int i = 0; i < 4; i++)
                  ev[4 * g + i] = __builtin_fmaf((float)acc[u][4 * g + i] * m.qs, zz[i], m.qcp);
              }
              if (MODE == 0) {
                float mx = -1e30f;
#pragma unroll
                for (int v = 0; v < 16; v++) mx = fmaxf(mx, ev[v]);
                mx = fmaxf(mx, __shfl_xor(mx, 32, FVS_WAVE));
                if (h == 0 && valid)
                  bm[((int64_t)m.qid * n1 + __float_as_int(m.x)) * MB + ((row0 >> 5) + kNB * w + u - (cs >> 5))] = mx;
              } else if (!direct) {
                // Per element: a wave ballot of est >= t0 (the compare's own mask). An empty ballot (about
                // half of them) is a scalar branch; otherwise the passing lanes, under the exec mask, take
                // consecutive slots of the wave's region. The region's fill is wave-uniform, so the
                // overflow test is scalar too; the count keeps growing past kCap so that the item end
                // sees the overflow and redoes the item on the direct path.
                float *est = E->est[w];
                uint32_t *tag = E->tag[w];
#pragma unroll
                for (int v = 0; v < 16; v++) {
                  const bool pass = ev[v] >= th;
                  const uint64_t bal = __ballot(pass);
                  if (bal) {
                    const int pop = __popcll(bal);
                    if (ebase + pop <= kCap && pass) {
                      // the region's fill is a scalar offset of the base; the lane adds its rank
                      const int pre = fvs_lane_prefix(bal);
                      (est + ebase)[pre] = ev[v];
                      (tag + ebase)[pre] = tag0 + (uint32_t)(32 * u + 8 * (v >> 2) + (v & 3));
                    }
                    ebase += pop;
                  }
                }
              } else {  // direct path
                // the lane's first row of the block; the empty asm keeps the compiler from hoisting the 16
                // per-element row ids out of the tile loop, where they would hold (and spill) 32 VGPRs
                int rb = row0 + 32 * (kNB * w + u) + 4 * h;
                asm volatile("" : "+v"(rb));
#pragma unroll
                for (int v = 0; v < 16; v++) {
                  if (ev[v] >= th) {
                    const int idx = atomicAdd(&cnt[m.qid], 1);
                    if (idx < CAP) {
                      bval[(int64_t)m.qid * CAP + idx] = ev[v];
                      bpos[(int64_t)m.qid * CAP + idx] = rb + 8 * (v >> 2) + (v & 3);
                    }
                  }
                }
              }
            }
          };
          request(0);
          published();
          for (int t = 0; t < ntiles; t++) {
            if (t + 1 < ntiles) request(t + 1);  // the other buffer: every wave has left tile t - 1
            if (any) compute(t);
            published();
          }
        }
      }
    };

    if constexpr (MODE == 0) {
      scan(true, true);
      prefetch(nxt);
    } else {
      scan(!staged, true);
      if (!staged) {
        prefetch(nxt);
      } else {
        // a wave whose region overflowed: drop the staged candidates and redo the item on the direct path
        if (lane == 0) E->n[w] = ebase;
        __syncthreads();
        if (E->n[0] > kCap || E->n[1] > kCap || E->n[2] > kCap || E->n[3] > kCap) {
          __syncthreads();
          scan(true, false);
          prefetch(nxt);
        } else {
          prefetch(nxt);  // the code blocks are no longer needed: the next item's loads run under the flush
          // flush: every staged candidate takes its number among its pair's candidates with an LDS atomic,
          // then one global atomic per (item, query) reserves the query's range, and every candidate goes
          // to base + number
#pragma unroll
          for (int ww = 0; ww < 4; ww++) {
            const int nn = E->n[ww];
            for (int k = tid; k < nn; k += 256) {
              const uint32_t tg = E->tag[ww][k];
              const uint32_t num = atomicAdd(&E->lcnt[(tg >> 8) & 0xfffu], 1u);  // < 256 rows per item
              E->tag[ww][k] = tg | (num << 20);
            }
          }
          __syncthreads();
          for (int j = tid; j < qn; j += 256) {
            const int c = (int)E->lcnt[j];
            E->lcnt[j] = c ? (uint32_t)atomicAdd(&cnt[meta[j].qid], c) : 0u;
          }
          __syncthreads();
#pragma unroll
          for (int ww = 0; ww < 4; ww++) {
            const int nn = E->n[ww];
            for (int k = tid; k < nn; k += 256) {
              const uint32_t tg = E->tag[ww][k];
              const int j = (tg >> 8) & 0xfffu;
              const int idx = (int)E->lcnt[j] + (int)(tg >> 20);
              if (idx < CAP) {
                const int64_t q = meta[j].qid;
                bval[q * CAP + idx] = E->est[ww][k];
                bpos[q * CAP + idx] = row0 + (int)(tg & 0xffu);
              }
            }
          }
        }
      }
      __syncthreads();  // the flush has read the LDS tables before the next item's staging rewrites them
    }
    if constexpr (!persist) break;
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
      const float th = jv ? t0[q] : __builtin_inff();
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
  // both passes: three resident workgroups per CU, each looping over items with the next item's loads in
  // flight during the current one
  const unsigned grid = (mode == 0 || kPersistEmit) ? (unsigned)min(P, 3 * fvs_cu_count()) : (unsigned)P;
  if (mode == 0) {
    if (!qrank || !bm || MB <= 0 || n1 <= 0) return FVS_E_ARG;
    hipLaunchKernelGGL(k_i8_scan<0>, dim3(grid), dim3(256), 0, st, q8, qs, qid, qrank, coff, ccnt, pcell, prow, ps,
                       pe, P, Z, zs, N, qcp, t0, cnt, bval, bpos, bm, CAP, MB, n1);
  } else {
    if (!t0 || !cnt || !bval || !bpos || CAP <= 0) return FVS_E_ARG;
    hipLaunchKernelGGL(k_i8_scan<1>, dim3(grid), dim3(256), 0, st, q8, qs, qid, qrank, coff, ccnt, pcell, prow, ps,
                       pe, P, Z, zs, N, qcp, t0, cnt, bval, bpos, bm, CAP, MB, n1);
  }
  return fvs_launch_status();
}
