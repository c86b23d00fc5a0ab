// int8 stage-1 scan on gfx950 MFMA (v_mfma_i32_32x32x32_i8).
//
// One wave per static (cell, 32-row block) item. The block's 32 code rows are the MFMA A operand
// (M = rows) and stay in registers for the whole item; the cell's queries stream through as the
// B operand (N = queries) in tiles of 32, so each code byte is read from HBM once per pass while
// the query codes (B x 256 B, L2-resident) are re-read per block.
//
// Operand layout: lane l holds row/column (l & 31) and, for MFMA step s (k-block of 32 bytes),
// the 16 bytes at 32*s + 16*(l >> 5); A and B use the same assignment, so the contraction is
// exact for any internal k order. Accumulator layout (32x32): lane l, element v holds row
// 8*(v/4) + 4*(l/32) + (v%4) and column (query) l%32, so every lane owns one query and 16 rows;
// the epilogue needs only per-lane scalars for the query (qs, qcp, t0).
//
// Rows of the block outside the cell get a NaN row scale: their estimate is NaN, which never
// passes `est >= t0` and is ignored by fmaxf, so no per-element row mask is needed.
#include "fvs_common.h"

namespace {

constexpr int kR = 256;

__device__ __forceinline__ int acc_row(int v, int h) { return 8 * (v >> 2) + 4 * h + (v & 3); }

template <int MODE>
__global__ __launch_bounds__(64) void k_i8_scan(
    const int8_t *__restrict__ q8, const float *__restrict__ qs, const int32_t *__restrict__ qid,
    const int32_t *__restrict__ qrank, const int32_t *__restrict__ coff, const int32_t *__restrict__ ccnt,
    const int32_t *__restrict__ pcell, const int32_t *__restrict__ pblk, const int32_t *__restrict__ ps,
    const int32_t *__restrict__ pe, const int8_t *__restrict__ Z, const float *__restrict__ zs, int64_t N,
    const float *__restrict__ qcp, const float *__restrict__ t0, int32_t *__restrict__ cnt,
    float *__restrict__ bval, int32_t *__restrict__ bpos, float *__restrict__ bm, int CAP, int MB, int n1) {
  const int p = blockIdx.x;
  const int lane = threadIdx.x;
  const int c = pcell[p];
  const int qn = ccnt[c];
  if (qn == 0) return;
  const int qoff = coff[c];
  const int blk = pblk[p];
  const int cs = ps[p], ce = pe[p];
  const int64_t row0 = (int64_t)blk * 32;
  const int h = lane >> 5, li = lane & 31;

  // A operand: the block's code rows (rows past the end of Z are clamped; they are masked below)
  int64_t zr = row0 + li;
  if (zr > N - 1) zr = N - 1;
  const v4i *zp = reinterpret_cast<const v4i *>(Z + zr * kR + h * 16);
  v4i a[8];
#pragma unroll
  for (int s = 0; s < 8; s++) a[s] = zp[2 * s];

  float zsv[16];
#pragma unroll
  for (int v = 0; v < 16; v++) {
    const int64_t r = row0 + acc_row(v, h);
    zsv[v] = (r >= cs && r < ce) ? zs[r] : __builtin_nanf("");
  }
  const int blocal = blk - cs / 32;

  for (int t = 0; t < qn; t += 32) {
    const int jq = t + li;
    const bool qv = jq < qn;
    const int pidx = qoff + (qv ? jq : qn - 1);
    const int q = qid[pidx];
    const v4i *qp = reinterpret_cast<const v4i *>(q8 + (int64_t)q * kR + h * 16);
    v4i b[8];
#pragma unroll
    for (int s = 0; s < 8; s++) b[s] = qp[2 * s];
    v16i acc = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
    for (int s = 0; s < 8; s++) acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[s], b[s], acc, 0, 0, 0);
    const float qsj = qs[q];
    const float qcj = qcp[pidx];
    if (MODE == 0) {
      float m = -1e30f;
#pragma unroll
      for (int v = 0; v < 16; v++) m = fmaxf(m, __builtin_fmaf((float)acc[v] * qsj, zsv[v], qcj));
      m = fmaxf(m, __shfl_xor(m, 32, FVS_WAVE));
      if (h == 0 && qv) bm[((int64_t)q * n1 + qrank[pidx]) * MB + blocal] = m;
    } else {
      const float th = qv ? t0[q] : __builtin_inff();
      float e[16];
      int nk = 0;
#pragma unroll
      for (int v = 0; v < 16; v++) {
        e[v] = __builtin_fmaf((float)acc[v] * qsj, zsv[v], qcj);
        nk += (e[v] >= th) ? 1 : 0;
      }
      if (nk) {
        int idx = atomicAdd(&cnt[q], nk);
        float *bv = bval + (int64_t)q * CAP;
        int32_t *bp = bpos + (int64_t)q * CAP;
#pragma unroll
        for (int v = 0; v < 16; v++) {
          if (e[v] >= th) {
            if (idx < CAP) {
              bv[idx] = e[v];
              bp[idx] = (int32_t)(row0 + acc_row(v, h));
            }
            idx++;
          }
        }
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
    hipLaunchKernelGGL(k_i8_scan<0>, dim3((unsigned)P), dim3(64), 0, st, q8, qs, qid, qrank, coff, ccnt, pcell, pblk,
                       ps, pe, Z, zs, N, qcp, t0, cnt, bval, bpos, bm, CAP, MB, n1);
  } else {
    if (!t0 || !cnt || !bval || !bpos || CAP <= 0) return FVS_E_ARG;
    hipLaunchKernelGGL(k_i8_scan<1>, dim3((unsigned)P), dim3(64), 0, st, q8, qs, qid, qrank, coff, ccnt, pcell, pblk,
                       ps, pe, Z, zs, N, qcp, t0, cnt, bval, bpos, bm, CAP, MB, n1);
  }
  return fvs_launch_status();
}
