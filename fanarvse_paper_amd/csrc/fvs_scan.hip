// int8 stage-1 scan on gfx950 MFMA (v_mfma_i32_32x32x32_i8).
//
// Work item = (cell, chunk of up to 8 consecutive global 32-row blocks of the cell), one 4-wave
// workgroup per item. Wave w keeps blocks 2w and 2w+1 of the chunk (64 code rows) as MFMA A operands
// in registers for the whole item, so each code byte is read from HBM once per pass. The cell's
// queries stream through as B operands in tiles of 32: a tile (32 x 256 B) is loaded once per item
// into LDS (row stride 272 B, so the 16-byte fragment reads of 8 consecutive lanes hit distinct
// banks) and read by all four waves; the next tile's global loads are issued before the current
// tile's MFMAs and stored to the other LDS buffer after them.
//
// Operand layout: lane l holds row/column (l & 31) and, for MFMA step s (k-block of 32 bytes), the
// 16 bytes at 32*s + 16*(l >> 5); A and B use the same assignment, so the contraction is exact for
// any internal k order. Accumulator layout (32x32): lane l, element v holds row
// 8*(v/4) + 4*(l/32) + (v%4) and column (query) l%32, so each lane owns one query and 16 rows of a
// block; the epilogue needs only per-lane scalars for the query.
//
// Rows of a block outside the cell get a NaN row scale: their estimate is NaN, which never passes
// `est >= t0` and is ignored by fmaxf, so no per-element row mask is needed.
#include "fvs_common.h"

namespace {

constexpr int kR = 256;
constexpr int kCB = 8;     // 32-row blocks per work item
constexpr int kRS = 272;   // LDS row stride of a query tile

__device__ __forceinline__ int acc_row(int v, int h) { return 8 * (v >> 2) + 4 * h + (v & 3); }

// One thread's share of a query tile in flight between global memory and LDS: thread t stages bytes
// 32*(t&7) .. +32 of the code of query row t>>3, and the threads with (t&7) == 0 its scalars. Loads
// are branch-free (indices clamped to the cell's last pair) so that the compiler can keep them in
// flight across the MFMA work of the current tile.
struct TileStage {
  v4i lo, hi;
  int qid, qrank;
  float qs, qcp, t0;
};

__device__ __forceinline__ int tile_pair(int tile, int qn, int qoff) {
  const int jq = tile * 32 + (int)(threadIdx.x >> 3);
  return qoff + (jq < qn ? jq : qn - 1);
}

// Issue the loads of one tile; q is qid[tile_pair(...)], loaded one iteration earlier.
template <int MODE>
__device__ __forceinline__ void tile_load(TileStage &st, int tile, int qn, int qoff, int q,
                                          const int8_t *__restrict__ q8, const float *__restrict__ qs,
                                          const int32_t *__restrict__ qrank, const float *__restrict__ qcp,
                                          const float *__restrict__ t0) {
  const int part = threadIdx.x & 7;
  const int pidx = tile_pair(tile, qn, qoff);
  const v4i *src = reinterpret_cast<const v4i *>(q8 + (int64_t)q * kR + part * 32);
  st.lo = src[0];
  st.hi = src[1];
  const bool valid = tile * 32 + (int)(threadIdx.x >> 3) < qn;
  st.qid = valid ? q : -1;
  st.qs = qs[q];
  st.qcp = qcp[pidx];
  if (MODE == 0) {
    st.qrank = qrank[pidx];
  } else {
    st.t0 = valid ? t0[q] : __builtin_inff();
  }
}

struct TileLds {
  int8_t q[2][32 * kRS];
  int qid[2][32];
  int qrank[2][32];
  float qs[2][32], qcp[2][32], t0[2][32];
};

// Emit staging: candidates that pass are collected in LDS for the whole item; at its end one global
// atomic per query reserves the query's buffer range, so the atomic round trip is paid once per item
// instead of once per query tile. Candidates beyond kES (or items of cells probed by more than kMaxQ
// queries) take the direct path: one global atomic per candidate.
constexpr int kES = 2048;
constexpr int kMaxQ = 2048;
struct EmitLds {
  float est[kES];
  int row[kES];
  uint16_t jq[kES];
  uint16_t rk[kES];
  int qcount[kMaxQ];
  int qbase[kMaxQ];
  int n;
};

template <int MODE>
__device__ __forceinline__ void tile_store(const TileStage &st, TileLds &L, int buf) {
  const int tid = threadIdx.x;
  const int row = tid >> 3, part = tid & 7;
  v4i *dst = reinterpret_cast<v4i *>(&L.q[buf][row * kRS + part * 32]);
  dst[0] = st.lo;
  dst[1] = st.hi;
  if (part == 0) {
    L.qid[buf][row] = st.qid;
    L.qs[buf][row] = st.qs;
    L.qcp[buf][row] = st.qcp;
    if (MODE == 0)
      L.qrank[buf][row] = st.qrank;
    else
      L.t0[buf][row] = st.t0;
  }
}

template <int MODE>
__global__ __launch_bounds__(256, 2) void k_i8_scan(
    const int8_t *__restrict__ q8, const float *__restrict__ qs, const int32_t *__restrict__ qid,
    const int32_t *__restrict__ qrank, const int32_t *__restrict__ coff, const int32_t *__restrict__ ccnt,
    const int32_t *__restrict__ pcell, const int32_t *__restrict__ pblk, const int32_t *__restrict__ ps,
    const int32_t *__restrict__ pe, const int8_t *__restrict__ Z, const float *__restrict__ zs, int64_t N,
    const float *__restrict__ qcp, const float *__restrict__ t0, int32_t *__restrict__ cnt,
    float *__restrict__ bval, int32_t *__restrict__ bpos, float *__restrict__ bm, int CAP, int MB, int n1) {
  __shared__ __align__(16) TileLds L;
  const int p = blockIdx.x;
  const int c = pcell[p];
  const int qn = ccnt[c];
  if (qn == 0) return;
  EmitLds *E = nullptr;
  if constexpr (MODE == 1) {
    __shared__ EmitLds Es;
    E = &Es;
    if (threadIdx.x == 0) Es.n = 0;
  }
  const bool staged = MODE == 1 && qn <= kMaxQ;
  const int qoff = coff[c];
  const int blk0 = pblk[p];
  const int cs = ps[p], ce = pe[p];
  const int lastblk = (ce - 1) / 32;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int h = lane >> 5, li = lane & 31;

  // this wave's two blocks: A operands and row scales
  int bk[2];
  bool act[2];
  v4i a[2][8];
  float zsv[2][16];
#pragma unroll
  for (int u = 0; u < 2; u++) {
    bk[u] = blk0 + 2 * w + u;
    act[u] = bk[u] <= lastblk && 2 * w + u < kCB;
    int64_t zr = (int64_t)bk[u] * 32 + li;
    if (!act[u] || zr > N - 1) zr = N - 1;
    const v4i *zp = reinterpret_cast<const v4i *>(Z + zr * kR + h * 16);
#pragma unroll
    for (int s = 0; s < 8; s++) a[u][s] = zp[2 * s];
#pragma unroll
    for (int v = 0; v < 16; v++) {
      const int64_t r = (int64_t)bk[u] * 32 + acc_row(v, h);
      zsv[u][v] = (act[u] && r >= cs && r < ce) ? zs[r] : __builtin_nanf("");
    }
  }
  const bool any = act[0] || act[1];

  // three-stage pipeline over query tiles: while tile t is multiplied, the codes of tile t+1 are in
  // flight to registers and the query ids of tile t+2 are being fetched
  const int ntiles = (qn + 31) / 32;
  TileStage st;
  int qnext = qid[tile_pair(0, qn, qoff)];
  tile_load<MODE>(st, 0, qn, qoff, qnext, q8, qs, qrank, qcp, t0);
  qnext = qid[tile_pair(1, qn, qoff)];
  tile_store<MODE>(st, L, 0);
  __syncthreads();
  int buf = 0;
  for (int t = 0; t < ntiles; t++) {
    const bool more = t + 1 < ntiles;
    tile_load<MODE>(st, t + 1, qn, qoff, qnext, q8, qs, qrank, qcp, t0);
    qnext = qid[tile_pair(t + 2, qn, qoff)];
    if (any) {
      v4i b[8];
      const int8_t *qrow = &L.q[buf][li * kRS + h * 16];
#pragma unroll
      for (int s = 0; s < 8; s++) b[s] = *reinterpret_cast<const v4i *>(qrow + 32 * s);
      v16i acc[2];
#pragma unroll
      for (int u = 0; u < 2; u++) {
        acc[u] = (v16i){0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
        if (act[u]) {
#pragma unroll
          for (int s = 0; s < 8; s++) acc[u] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[u][s], b[s], acc[u], 0, 0, 0);
        }
      }
      const int q = L.qid[buf][li];
      const float qsj = L.qs[buf][li];
      const float qcj = L.qcp[buf][li];
      if (MODE == 0) {
        const int rk = L.qrank[buf][li];
#pragma unroll
        for (int u = 0; u < 2; u++) {
          if (!act[u]) continue;
          float m = -1e30f;
#pragma unroll
          for (int v = 0; v < 16; v++) m = fmaxf(m, __builtin_fmaf((float)acc[u][v] * qsj, zsv[u][v], qcj));
          m = fmaxf(m, __shfl_xor(m, 32, FVS_WAVE));
          if (h == 0 && q >= 0) bm[((int64_t)q * n1 + rk) * MB + (bk[u] - cs / 32)] = m;
        }
      } else {
        const float th = L.t0[buf][li];
        float e[2][16];
        int nk = 0;
#pragma unroll
        for (int u = 0; u < 2; u++) {
#pragma unroll
          for (int v = 0; v < 16; v++) {
            e[u][v] = __builtin_fmaf((float)acc[u][v] * qsj, zsv[u][v], qcj);
            nk += (e[u][v] >= th) ? 1 : 0;
          }
        }
        if (nk) {
          int sp = staged ? atomicAdd(&E->n, nk) : kES;  // LDS slot range of this lane's candidates
          const uint16_t jq = (uint16_t)(t * 32 + li);
#pragma unroll
          for (int u = 0; u < 2; u++) {
#pragma unroll
            for (int v = 0; v < 16; v++) {
              if (e[u][v] >= th) {
                const int row = bk[u] * 32 + acc_row(v, h);
                if (sp < kES) {
                  E->est[sp] = e[u][v];
                  E->row[sp] = row;
                  E->jq[sp] = jq;
                } else {  // direct path
                  const int idx = atomicAdd(&cnt[q], 1);
                  if (idx < CAP) {
                    bval[(int64_t)q * CAP + idx] = e[u][v];
                    bpos[(int64_t)q * CAP + idx] = row;
                  }
                }
                sp++;
              }
            }
          }
        }
      }
    }
    if (more) tile_store<MODE>(st, L, buf ^ 1);
    __syncthreads();
    buf ^= 1;
  }

  if constexpr (MODE == 1) {
    // flush the staged candidates: rank within the query, one global reservation per query, write out
    if (!staged) return;
    const int n = min(E->n, kES);
    if (n == 0) return;
    for (int j = threadIdx.x; j < qn; j += 256) E->qcount[j] = 0;
    __syncthreads();
    for (int i = threadIdx.x; i < n; i += 256) E->rk[i] = (uint16_t)atomicAdd(&E->qcount[E->jq[i]], 1);
    __syncthreads();
    for (int j = threadIdx.x; j < qn; j += 256) {
      const int m = E->qcount[j];
      if (m) E->qbase[j] = atomicAdd(&cnt[qid[qoff + j]], m);
    }
    __syncthreads();
    for (int i = threadIdx.x; i < n; i += 256) {
      const int j = E->jq[i];
      const int idx = E->qbase[j] + E->rk[i];
      if (idx < CAP) {
        const int64_t q = qid[qoff + j];
        bval[q * CAP + idx] = E->est[i];
        bpos[q * CAP + idx] = E->row[i];
      }
    }
  }
}

}  // namespace

extern "C" int fvs_i8_scan(int32_t mode, int32_t P, const int8_t *q8, const float *qs, const int32_t *qid,
                           const int32_t *qrank, const int32_t *coff, const int32_t *ccnt, const int32_t *pcell,
                           const int32_t *pblk, const int32_t *ps, const int32_t *pe, const int8_t *Z,
                           const float *zs, int64_t N, int32_t R, const float *qcp, const float *t0, int32_t *cnt,
                           float *bval, int32_t *bpos, float *bm, int32_t CAP, int32_t MB, int32_t n1,
                           void *stream) {
  if (R != kR) return FVS_E_SHAPE;
  if (mode != 0 && mode != 1) return FVS_E_ARG;
  if (P < 0 || N <= 0) return FVS_E_ARG;
  if (P == 0) return FVS_OK;
  if (!q8 || !qs || !qid || !coff || !ccnt || !pcell || !pblk || !ps || !pe || !Z || !zs || !qcp) return FVS_E_ARG;
  hipStream_t st = (hipStream_t)stream;
  if (mode == 0) {
    if (!qrank || !bm || MB <= 0 || n1 <= 0) return FVS_E_ARG;
    hipLaunchKernelGGL(k_i8_scan<0>, dim3((unsigned)P), dim3(256), 0, st, q8, qs, qid, qrank, coff, ccnt, pcell,
                       pblk, ps, pe, Z, zs, N, qcp, t0, cnt, bval, bpos, bm, CAP, MB, n1);
  } else {
    if (!t0 || !cnt || !bval || !bpos || CAP <= 0) return FVS_E_ARG;
    hipLaunchKernelGGL(k_i8_scan<1>, dim3((unsigned)P), dim3(256), 0, st, q8, qs, qid, qrank, coff, ccnt, pcell,
                       pblk, ps, pe, Z, zs, N, qcp, t0, cnt, bval, bpos, bm, CAP, MB, n1);
  }
  return fvs_launch_status();
}
