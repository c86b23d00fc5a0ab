// The trellis cell-residual engine of the latency mode: bitshift-trellis encoder (Viterbi), stage-1
// scan over the decoded codes and the Lloyd-Max tiered stage 2 (its fp32-key routing is in fvs_route.hip).
//
// Trellis code (L-bit states, one bit per coordinate): a vector's bit stream is the L bits of its
// first state (MSB first) followed by the newest bit of every later state; state_j is the window
// bits[j .. j+L) read MSB first and the decoded coordinate j is tab[state_j]. The stream is stored
// as W = ceil((R + L - 1) / 32) 32-bit words, first bit in the most significant position.
#include <algorithm>
#include <mutex>

#include "fvs_common.h"

namespace {

constexpr int kTrR = 256;      // coordinates per trellis code
constexpr int kMaxL = 12;      // largest state width the encoder's LDS holds (4096 states)
constexpr int kMaxT = FVS_MAX_TIERS;

// ------------------------------------------------------------------------------------ encoder
// One workgroup (256 threads) per vector. Path costs ping-pong in LDS; backpointers are one bit per
// state per step (ballots), all in LDS; the backtrack, the words and the scale follow in the same
// workgroup. Canonical arithmetic (shared with the CPU checker):
//   cost_0(s) = d*d, d = x_0 - tab[s];  cost_j(s) = min(cost(p0), cost(p1)) + d*d, d = x_j - tab[s],
//   with p0 = s >> 1, p1 = p0 | 2^(L-1), taking p1 only when cost(p1) < cost(p0) (strictly);
//   the final state is the smallest index of minimum cost.
template <int S>
__global__ __launch_bounds__(256) void k_trellis_encode(const float *__restrict__ Zs, const float *__restrict__ nz,
                                                        int L, const float *__restrict__ tab, int W,
                                                        uint32_t *__restrict__ words, uint16_t *__restrict__ scale1,
                                                        int32_t *__restrict__ paths) {
  __shared__ float x[kTrR];
  __shared__ float vals[S];
  __shared__ float cost[2][S];
  __shared__ uint32_t back[kTrR - 1][S / 32];
  __shared__ int path[kTrR];
  __shared__ unsigned long long best;
  const int64_t v = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, w = fvs_wave_id();
  for (int i = tid; i < S; i += 256) vals[i] = tab[i];
  x[tid] = Zs[v * kTrR + tid];
  if (tid == 0) best = ~0ull;
  __syncthreads();
  constexpr int PER = S / 256;
#pragma unroll
  for (int i = 0; i < PER; i++) {
    const int s = tid + 256 * i;
    const float d = x[0] - vals[s];
    cost[0][s] = d * d;
  }
  __syncthreads();
  const int half = S >> 1;
  for (int j = 1; j < kTrR; j++) {
    const float *cp = cost[(j - 1) & 1];
    float *cn = cost[j & 1];
    const float xj = x[j];
#pragma unroll
    for (int i = 0; i < PER; i++) {
      const int s = tid + 256 * i;
      const int p0 = s >> 1, p1 = p0 | half;
      const float c0 = cp[p0], c1 = cp[p1];
      const bool take1 = c1 < c0;
      const float d = xj - vals[s];
      cn[s] = (take1 ? c1 : c0) + d * d;
      const uint64_t bal = __ballot(take1);
      if (lane == 0) {
        back[j - 1][(256 * i + 64 * w) >> 5] = (uint32_t)bal;
        back[j - 1][((256 * i + 64 * w) >> 5) + 1] = (uint32_t)(bal >> 32);
      }
    }
    __syncthreads();
  }
  // smallest index of minimum cost (costs are non-negative: their bit patterns order like the values)
  const float *cf = cost[(kTrR - 1) & 1];
  unsigned long long mine = ~0ull;
#pragma unroll
  for (int i = 0; i < PER; i++) {
    const int s = tid + 256 * i;
    const unsigned long long k = ((unsigned long long)__float_as_uint(cf[s]) << 32) | (unsigned)s;
    mine = k < mine ? k : mine;
  }
  for (int o = 32; o > 0; o >>= 1) {
    const unsigned long long t = __shfl_xor(mine, o, FVS_WAVE);
    mine = t < mine ? t : mine;
  }
  if (lane == 0) atomicMin(&best, mine);
  __syncthreads();
  if (tid == 0) {
    int st = (int)(best & 0xffffffffu);
    path[kTrR - 1] = st;
    for (int j = kTrR - 1; j > 0; j--) {
      const int u = (int)((back[j - 1][st >> 5] >> (st & 31)) & 1u);
      st = (st >> 1) | (u << (L - 1));
      path[j - 1] = st;
    }
  }
  __syncthreads();
  if (paths) paths[v * kTrR + tid] = path[tid];
  // words: bit b of the stream is (b < L) ? bit L-1-b of path[0] : lowest bit of path[b - L + 1]
  if (tid < W) {
    uint32_t word = 0;
    for (int t = 0; t < 32; t++) {
      const int b = 32 * tid + t;
      uint32_t bit = 0;
      if (b < L)
        bit = ((uint32_t)path[0] >> (L - 1 - b)) & 1u;
      else if (b < kTrR + L - 1)
        bit = (uint32_t)path[b - L + 1] & 1u;
      word |= bit << (31 - t);
    }
    words[v * W + tid] = word;
  }
  // scale = |z| / (<Zs, Y> / (|Y| sqrt(R)) * |Y|), Y = tab[path]; sums in double, lane = j % 64
  if (w == 0) {
    double yy = 0.0, zy = 0.0;
    for (int j = lane; j < kTrR; j += 64) {
      const double y = (double)vals[path[j]];
      yy += y * y;
      zy += (double)x[j] * y;
    }
    for (int o = 32; o > 0; o >>= 1) {
      yy += __shfl_xor(yy, o, FVS_WAVE);
      zy += __shfl_xor(zy, o, FVS_WAVE);
    }
    if (lane == 0) {
      const float yn = sqrtf((float)yy);
      const float fip = (float)zy / (yn * sqrtf((float)kTrR));
      scale1[v] = fvs_f2h(nz[v] / (fip * yn));
    }
  }
}

// ------------------------------------------------------------------------------------ stage 1
// One wave per static (cell, 32-row block) item, four items per workgroup. Lane l decodes row l % 32,
// coordinates [128 h, 128 h + 128) with h = l / 32, into registers; for each query of the cell it
// forms the half dot product as a sequential fmaf chain and adds the two halves:
//   est = fmaf(scale1, lo + hi, qcp),  lo / hi = sum over j < 128 / j >= 128 of tab[state_j] * Qr[j].
// half != 0: both operands are first rounded to fp16 (the table once, each query element as it is staged),
// as the reference's tensor-core dot takes them; their products are exact in fp32.
// mode 0: bm[(q*n1 + qrank)*MB + blk - cs/32] = max over the block's rows in the cell.
// mode 1: every (q, row) with est >= t0[q] is appended to the query's buffer (one atomic each).
// words and scale1 hold rows row0 .. of the index (a staged chunk, or the whole index with row0 = 0).
// A launch over few items (a staged chunk of the host-resident engine) splits each item's queries into
// nsplit consecutive parts, one wave each, so that the launch still fills the GPU; a (query, row) pair is
// computed by exactly one wave either way, with the same arithmetic.
template <int MODE>
__global__ __launch_bounds__(256) void k_tr_scan(const float *__restrict__ Qr, const int32_t *__restrict__ qid,
                                                 const int32_t *__restrict__ qrank, const int32_t *__restrict__ coff,
                                                 const int32_t *__restrict__ ccnt, const int32_t *__restrict__ pcell,
                                                 const int32_t *__restrict__ pblk, const int32_t *__restrict__ ps,
                                                 const int32_t *__restrict__ pe, int P, const uint32_t *__restrict__ words,
                                                 int64_t row0, int W, const uint16_t *__restrict__ scale1,
                                                 const float *__restrict__ tab,
                                                 int L, int half, const float *__restrict__ qcp,
                                                 const float *__restrict__ t0,
                                                 int32_t *__restrict__ cnt, float *__restrict__ bval,
                                                 int32_t *__restrict__ bpos, float *__restrict__ bm, int CAP, int MB, int n1,
                                                 int nsplit) {
  __shared__ float stab[1 << kMaxL];
  __shared__ float4 qbuf[4][kTrR / 4];  // per wave: the query vector of the current step
  __shared__ uint32_t rows_s[4][32 * 10];  // per wave: the words of its item's rows (W <= 10)
  const int tid = threadIdx.x, lane = tid & 63, w = fvs_wave_id();
  const int S = 1 << L;
  for (int i = tid; i < S; i += 256) stab[i] = half ? fvs_round_h(tab[i]) : tab[i];
  __syncthreads();
  const int64_t u = (int64_t)blockIdx.x * 4 + w;  // work unit: item p, part `part` of its queries
  if (u >= (int64_t)P * nsplit) return;
  const int p = (int)(u / nsplit), part = (int)(u - (int64_t)p * nsplit);
  const int c = pcell[p];
  const int qcell = ccnt[c];
  const int qlo = (int)((int64_t)qcell * part / nsplit), qhi = (int)((int64_t)qcell * (part + 1) / nsplit);
  const int qn = qhi - qlo;
  if (qn <= 0) return;
  const int qoff = coff[c] + qlo;  // this part's pairs: qoff .. qoff + qn - 1
  const int blk = pblk[p], cs = ps[p], ce = pe[p];
  const int h = lane >> 5, li = lane & 31;
  const int r = blk * 32 + li;
  const bool valid = r >= cs && r < ce;
  // The item's rows r_lo .. r_hi - 1 are one contiguous run of words: the wave reads it with consecutive
  // lanes on consecutive dwords (every byte fetched once, which matters when the words are read
  // zero-copy from pinned host memory over PCIe) and stages it in LDS for the per-row decode.
  const int r_lo = max(blk * 32, cs), r_hi = min(blk * 32 + 32, ce);
  const int rr = valid ? r : r_lo;  // padding lanes decode a staged row (their results are dropped)
  {
    const int nw = max(r_hi - r_lo, 0) * W;  // <= 32 * 10
    const uint32_t *src = words + ((int64_t)r_lo - row0) * W;
    uint32_t tmp[5];
#pragma unroll
    for (int k = 0; k < 5; k++) {
      const int i = lane + 64 * k;
      tmp[k] = i < nw ? src[i] : 0u;
    }
#pragma unroll
    for (int k = 0; k < 5; k++) {
      const int i = lane + 64 * k;
      if (i < nw) rows_s[w][i] = tmp[k];
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }
  // coordinates [128 h, 128 h + 128) need words 4h .. 4h + 4 of the stream
  uint32_t ww[5];
#pragma unroll
  for (int k = 0; k < 5; k++) {
    const int i = 4 * h + k;
    ww[k] = i < W ? rows_s[w][(rr - r_lo) * W + i] : 0u;
  }
  float v[128];
  const uint32_t mask = (uint32_t)S - 1u;
#pragma unroll
  for (int i = 0; i < 128; i++) {
    const uint64_t comb = ((uint64_t)ww[i >> 5] << 32) | (uint64_t)ww[(i >> 5) + 1];
    v[i] = stab[(uint32_t)(comb >> (64 - L - (i & 31))) & mask];
  }
  const float s1 = valid ? fvs_h2f(scale1[(int64_t)rr - row0]) : 0.f;
  // The query vectors (kTrR floats = one float4 per lane) are read one step ahead and staged in LDS, so
  // a step waits for one LDS round trip instead of a chain of global ones.
  const float4 *Qr4 = reinterpret_cast<const float4 *>(Qr);
  float4 nxt = Qr4[(int64_t)__builtin_amdgcn_readfirstlane(qid[qoff]) * (kTrR / 4) + lane];
  for (int i = 0; i < qn; i++) {
    const int pidx = qoff + i;
    const int q = __builtin_amdgcn_readfirstlane(qid[pidx]);  // one query per wave and step
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");  // the previous step's reads of qbuf are issued
    __builtin_amdgcn_wave_barrier();
    qbuf[w][lane] = half ? make_float4(fvs_round_h(nxt.x), fvs_round_h(nxt.y), fvs_round_h(nxt.z), fvs_round_h(nxt.w))
                         : nxt;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    if (i + 1 < qn) nxt = Qr4[(int64_t)__builtin_amdgcn_readfirstlane(qid[pidx + 1]) * (kTrR / 4) + lane];
    const float4 *qv = &qbuf[w][32 * h];
    float acc = 0.f;
#pragma unroll
    for (int g = 0; g < 32; g++) {
      const float4 x4 = qv[g];
      acc = __builtin_fmaf(v[4 * g + 0], x4.x, acc);
      acc = __builtin_fmaf(v[4 * g + 1], x4.y, acc);
      acc = __builtin_fmaf(v[4 * g + 2], x4.z, acc);
      acc = __builtin_fmaf(v[4 * g + 3], x4.w, acc);
    }
    const float other = __shfl_xor(acc, 32, FVS_WAVE);
    const float est = __builtin_fmaf(s1, acc + other, qcp[pidx]);
    if (MODE == 0) {
      float m = valid ? est : -__builtin_inff();
#pragma unroll
      for (int o = 16; o > 0; o >>= 1) m = fmaxf(m, fvs_xor_lane_f(m, o));
      if (lane == 0) bm[((int64_t)q * n1 + qrank[pidx]) * MB + (blk - cs / 32)] = m;
    } else {
      // one counter update per wave: slot = base + rank of the lane among the passing lanes
      const bool pass = h == 0 && valid && est >= t0[q];
      const uint64_t m = __ballot(pass);
      if (m) {
        const int lead = __builtin_ctzll(m);
        int base = 0;
        if (lane == lead) base = atomicAdd(&cnt[q], __builtin_popcountll(m));
        base = __builtin_amdgcn_readlane(base, lead);
        const int idx = base + __builtin_popcountll(m & ((1ull << lane) - 1ull));
        if (pass && idx < CAP) {
          bval[(int64_t)q * CAP + idx] = est;
          bpos[(int64_t)q * CAP + idx] = r;
        }
      }
    }
  }
}


// ------------------------------------------------------------------------------------ stage 2
struct LmTiers {
  int T;
  int start[kMaxT], width[kMaxT], bits[kMaxT], toff[kMaxT];
};

// A query's K candidates are split over `nchunk` workgroups of 4 waves; workgroup (q, c) takes candidates
// 4*cpw*c .. 4*cpw*(c+1)-1 and each wave one candidate at a time, so a batch of one query still fills the
// chip while a large batch keeps one staging of Zq and the codebooks per 4*cpw candidates. Canonical arithmetic:
//   a_t = (xor butterfly over 64 lanes of) the lane sums, lane l summing fmaf(cb_t[code_k], Zq[s_t + k], .)
//   over the tier's coordinates k = l, l + 64, ... in order;
//   est = fmaf(a_t, scale_t, est) and var = fmaf(qn2_t * sig_t, sig_t, var) for t = 0..T-1 from
//   est = qc[q], var = 0; sd = sqrtf(var). qn2_t = (float) of the double sum of Zq^2 over the tier
//   (lane = offset in the tier % 64, then the butterfly).
__global__ __launch_bounds__(256) void k_tiered_score(const int32_t *__restrict__ pos, const float *__restrict__ qc,
                                                      const float *__restrict__ Zq, int D, const uint8_t *__restrict__ rec,
                                                      int RB, int soff, LmTiers tiers, const float *__restrict__ cb,
                                                      const int32_t *__restrict__ ncnt, int K, int nchunk, int cpw,
                                                      float *__restrict__ est, float *__restrict__ sd) {
  extern __shared__ __align__(16) uint8_t dyn[];
  float *zq = reinterpret_cast<float *>(dyn);                  // [D]
  float *cbs = zq + D;                                         // [T][256]
  uint8_t *recs = reinterpret_cast<uint8_t *>(cbs + 256 * tiers.T);  // [4][RB]
  __shared__ float qn2[kMaxT];
  const int64_t q = blockIdx.x / nchunk;
  const int m0 = (int)(blockIdx.x % nchunk) * 4 * cpw, m1 = min(K, m0 + 4 * cpw);
  const int tid = threadIdx.x, lane = tid & 63, w = fvs_wave_id();
  for (int i = tid; i < D; i += 256) zq[i] = Zq[q * D + i];
  for (int i = tid; i < 256 * tiers.T; i += 256) cbs[i] = cb[i];
  __syncthreads();
  if (w == 0) {
#pragma unroll
    for (int t = 0; t < kMaxT; t++) {
      if (t >= tiers.T) break;
      double a = 0.0;
      for (int k = lane; k < tiers.width[t]; k += 64) {
        const double z = (double)zq[tiers.start[t] + k];
        a += z * z;
      }
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) a += fvs_xor_lane_d(a, o);
      if (lane == 0) qn2[t] = (float)a;
    }
  }
  __syncthreads();
  const int nc = ncnt ? min(ncnt[q], K) : K;
  uint8_t *rw = recs + w * RB;
  for (int m = m0 + w; m < m1; m += 4) {
    if (m >= nc) {
      if (lane == 0) {
        est[q * K + m] = -1e30f;
        sd[q * K + m] = 0.f;
      }
      continue;
    }
    const int64_t row = pos[q * K + m];
    const uint4 *src = reinterpret_cast<const uint4 *>(rec + row * RB);
    for (int i = lane; i < RB / 16; i += 64) reinterpret_cast<uint4 *>(rw)[i] = src[i];
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
    float e = qc[q], var = 0.f;
#pragma unroll
    for (int t = 0; t < kMaxT; t++) {
      if (t >= tiers.T) break;
      const int d = tiers.width[t], b = tiers.bits[t], kb = d >> 3;
      const uint8_t *pl = rw + tiers.toff[t];
      const float *cbt = cbs + 256 * t;
      const float *zt = zq + tiers.start[t];
      float acc = 0.f;
      for (int k = lane; k < d; k += 64) {
        int code = 0;
        for (int pp = 0; pp < b; pp++) code |= (((int)pl[pp * kb + (k >> 3)] >> (7 - (k & 7))) & 1) << (b - 1 - pp);
        acc = __builtin_fmaf(cbt[code], zt[k], acc);
      }
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) acc += fvs_xor_lane_f(acc, o);
      const uint16_t *ss = reinterpret_cast<const uint16_t *>(rw + soff + 4 * t);
      const float sc = fvs_h2f(ss[0]), sg = fvs_h2f(ss[1]);
      e = __builtin_fmaf(acc, sc, e);
      var = __builtin_fmaf(qn2[t] * sg, sg, var);
    }
    if (lane == 0) {
      est[q * K + m] = e;
      sd[q * K + m] = sqrtf(var);
    }
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
  }
}

}  // namespace

extern "C" int fvs_trellis_encode(const float *Zs, const float *nz, int64_t n, int32_t R, const float *tab, int32_t L,
                                  uint32_t *words, int32_t W, uint16_t *scale1, int32_t *paths, void *stream) {
  if (R != kTrR) return FVS_E_SHAPE;
  if (L < 8 || L > kMaxL || n < 0) return FVS_E_ARG;
  if (W != (R + L - 1 + 31) / 32) return FVS_E_ARG;
  if (n == 0) return FVS_OK;
  if (!Zs || !nz || !tab || !words || !scale1) return FVS_E_ARG;
  hipStream_t st = (hipStream_t)stream;
  if (L == 8)
    hipLaunchKernelGGL(k_trellis_encode<256>, dim3((unsigned)n), dim3(256), 0, st, Zs, nz, L, tab, W, words, scale1, paths);
  else if (L == 9)
    hipLaunchKernelGGL(k_trellis_encode<512>, dim3((unsigned)n), dim3(256), 0, st, Zs, nz, L, tab, W, words, scale1, paths);
  else if (L == 10)
    hipLaunchKernelGGL(k_trellis_encode<1024>, dim3((unsigned)n), dim3(256), 0, st, Zs, nz, L, tab, W, words, scale1, paths);
  else
    return FVS_E_SHAPE;  // 11 and 12 exceed the encoder's LDS budget
  return fvs_launch_status();
}

extern "C" int fvs_tr_scan(int32_t mode, int32_t P, const float *Qr, const int32_t *qid, const int32_t *qrank,
                           const int32_t *coff, const int32_t *ccnt, const int32_t *pcell, const int32_t *pblk,
                           const int32_t *ps, const int32_t *pe, const uint32_t *words, int64_t row0, int32_t W,
                           const uint16_t *scale1,
                           const float *tab, int32_t L, int32_t R, int32_t half, const float *qcp, const float *t0,
                           int32_t *cnt, float *bval, int32_t *bpos, float *bm, int32_t CAP, int32_t MB, int32_t n1,
                           int32_t nsplit, void *stream) {
  if (R != kTrR) return FVS_E_SHAPE;
  if (nsplit < 1 || nsplit > 64) return FVS_E_ARG;
  if (mode != 0 && mode != 1) return FVS_E_ARG;
  if (half != 0 && half != 1) return FVS_E_ARG;
  if (L < 2 || L > kMaxL || W != (R + L - 1 + 31) / 32 || W > 10 || P < 0 || row0 < 0) return FVS_E_ARG;
  if (P == 0) return FVS_OK;
  if (!Qr || !qid || !coff || !ccnt || !pcell || !pblk || !ps || !pe || !words || !scale1 || !tab || !qcp)
    return FVS_E_ARG;
  hipStream_t st = (hipStream_t)stream;
  const dim3 grid((unsigned)(((int64_t)P * nsplit + 3) / 4));
  if (mode == 0) {
    if (!qrank || !bm || MB <= 0 || n1 <= 0) return FVS_E_ARG;
    hipLaunchKernelGGL(k_tr_scan<0>, grid, dim3(256), 0, st, Qr, qid, qrank, coff, ccnt, pcell, pblk, ps, pe, P, words,
                       row0, W, scale1, tab, L, half, qcp, t0, cnt, bval, bpos, bm, CAP, MB, n1, nsplit);
  } else {
    if (!t0 || !cnt || !bval || !bpos || CAP <= 0) return FVS_E_ARG;
    hipLaunchKernelGGL(k_tr_scan<1>, grid, dim3(256), 0, st, Qr, qid, qrank, coff, ccnt, pcell, pblk, ps, pe, P, words,
                       row0, W, scale1, tab, L, half, qcp, t0, cnt, bval, bpos, bm, CAP, MB, n1, nsplit);
  }
  return fvs_launch_status();
}

namespace {

// Events that order one streamed pass (start, ready[2], done[2]), created once per device.
hipError_t streamed_events(hipEvent_t *&ev) {
  static std::mutex mu;
  static hipEvent_t evs[64][5];
  static bool made[64] = {false};
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= 64) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(mu);
  if (!made[dev]) {
    for (int k = 0; k < 5; k++) {
      e = hipEventCreateWithFlags(&evs[dev][k], hipEventDisableTiming);
      if (e != hipSuccess) return e;
    }
    made[dev] = true;
  }
  ev = evs[dev];
  return hipSuccess;
}

}  // namespace

extern "C" int fvs_tr_scan_streamed(int32_t mode, int32_t nchunks, const int64_t *chunks, const uint8_t *stage_h,
                                    uint8_t *slot0, uint8_t *slot1, int64_t slot_bytes, void *side, const float *Qr,
                                    const int32_t *qid, const int32_t *qrank, const int32_t *coff, const int32_t *ccnt,
                                    const int32_t *pcell, const int32_t *pblk, const int32_t *ps, const int32_t *pe,
                                    int32_t W, const float *tab, int32_t L, int32_t R, int32_t half, const float *qcp,
                                    const float *t0, int32_t *cnt, float *bval, int32_t *bpos, float *bm, int32_t CAP,
                                    int32_t MB, int32_t n1, int32_t nsplit, void *stream) {
  if (nchunks < 0) return FVS_E_ARG;
  if (nchunks == 0) return FVS_OK;
  if (!chunks || !stage_h || !slot0 || !slot1 || !pcell || !pblk || !ps || !pe || W <= 0) return FVS_E_ARG;
  // every chunk's block fits a slot, and its items are a range of the work list, before anything is queued
  for (int i = 0; i < nchunks; i++) {
    const int64_t *c = chunks + 5 * (int64_t)i;
    const int64_t n = c[1] - c[0];
    if (n <= 0 || c[0] < 0 || c[2] < 0 || c[3] < c[2] || c[4] < 0) return FVS_E_ARG;
    if (n * 4 * W + (2 * n + 15) / 16 * 16 > slot_bytes) return FVS_E_CAPACITY;
  }
  hipEvent_t *ev = nullptr;
  hipError_t e = streamed_events(ev);
  if (e != hipSuccess) return (int)e;
  hipStream_t st = (hipStream_t)stream, sd = (hipStream_t)side;
  // the slots' previous contents have been read by the work already queued on `stream`
  if ((e = hipEventRecord(ev[0], st)) != hipSuccess) return (int)e;
  if ((e = hipStreamWaitEvent(sd, ev[0], 0)) != hipSuccess) return (int)e;
  for (int i = 0; i < nchunks; i++) {
    const int64_t *c = chunks + 5 * (int64_t)i;
    const int64_t r0 = c[0], n = c[1] - c[0];
    const int i0 = (int)c[2], np = (int)(c[3] - c[2]);
    const int slot = i & 1;
    uint8_t *buf = slot ? slot1 : slot0;
    const size_t nb = (size_t)(n * 4 * W + (2 * n + 15) / 16 * 16);
    if (i >= 2 && (e = hipStreamWaitEvent(sd, ev[3 + slot], 0)) != hipSuccess) return (int)e;  // scan i-2 done
    if ((e = hipMemcpyAsync(buf, stage_h + c[4], nb, hipMemcpyHostToDevice, sd)) != hipSuccess) return (int)e;
    if ((e = hipEventRecord(ev[1 + slot], sd)) != hipSuccess) return (int)e;
    if ((e = hipStreamWaitEvent(st, ev[1 + slot], 0)) != hipSuccess) return (int)e;
    const int rc = fvs_tr_scan(mode, np, Qr, qid, qrank, coff, ccnt, pcell + i0, pblk + i0, ps + i0, pe + i0,
                               reinterpret_cast<const uint32_t *>(buf), r0, W,
                               reinterpret_cast<const uint16_t *>(buf + n * 4 * W), tab, L, R, half, qcp, t0, cnt,
                               bval, bpos, bm, CAP, MB, n1, nsplit, stream);
    if (rc != FVS_OK) return rc;
    if ((e = hipEventRecord(ev[3 + slot], st)) != hipSuccess) return (int)e;
  }
  return FVS_OK;
}

extern "C" int fvs_tiered_score(const int32_t *pos, const float *qc, const float *Zq, int32_t D, const uint8_t *rec,
                                int64_t N, int32_t RB, int32_t soff, int32_t T, const int32_t *tiers, const int32_t *toff,
                                const float *cb, const int32_t *ncnt, int64_t B, int32_t K, float *est, float *sd,
                                void *stream) {
  if (B < 0 || K <= 0 || D <= 0 || N <= 0 || RB <= 0 || RB % 16 != 0) return FVS_E_ARG;
  if (T <= 0 || T > kMaxT) return FVS_E_SHAPE;
  if (B == 0) return FVS_OK;
  if (!pos || !qc || !Zq || !rec || !tiers || !toff || !cb || !est || !sd) return FVS_E_ARG;
  LmTiers ta{};
  ta.T = T;
  for (int t = 0; t < T; t++) {
    const int s = tiers[3 * t], e = tiers[3 * t + 1], b = tiers[3 * t + 2];
    if (s < 0 || e > D || e <= s || (e - s) % 8 != 0 || b < 1 || b > 8) return FVS_E_SHAPE;
    if (toff[t] < 0 || toff[t] + b * (e - s) / 8 > soff || soff + 4 * T > RB) return FVS_E_SHAPE;
    ta.start[t] = s;
    ta.width[t] = e - s;
    ta.bits[t] = b;
    ta.toff[t] = toff[t];
  }
  const size_t shm = 4 * (size_t)D + 4 * 256 * (size_t)T + 4 * (size_t)RB;
  if (shm > 160 * 1024) return FVS_E_CAPACITY;
  // about 2048 workgroups when the batch is small, one per query when it is large
  const int groups = (K + 3) / 4;
  const int nchunk = (int)std::min<int64_t>(groups, std::max<int64_t>(1, (2048 + B - 1) / B));
  const int cpw = (groups + nchunk - 1) / nchunk;
  if (B * nchunk > 0x7fffffff) return FVS_E_CAPACITY;
  hipLaunchKernelGGL(k_tiered_score, dim3((unsigned)(B * nchunk)), dim3(256), shm, (hipStream_t)stream, pos, qc, Zq,
                     D, rec, RB, soff, ta, cb, ncnt, K, nchunk, cpw, est, sd);
  return fvs_launch_status();
}
