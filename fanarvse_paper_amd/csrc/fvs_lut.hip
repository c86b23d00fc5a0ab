// Uniform tiered refinement code: nibble lookup tables and the LUT stage-2 scorer with error bars.
//
// Scorer mapping: one block (2 waves) per query. The query's LUT is converted once into 32-bit
// fixed point in LDS, so every plane sum is an exact integer and the result does not depend on the
// summation order (any lane/tile mapping gives the same bits). Each lane scores one candidate:
// it streams the candidate's packed record (128 B in flight per iteration), looks up two LUT
// entries per code byte, and folds the per-tier integer sums into the f32 estimate in tier order.
// A per-dword descriptor table in LDS (LUT base, plane weight, end-of-tier flag) is shared by all
// lanes, so control flow is uniform across the wave.
#include "fvs_common.h"

namespace {

struct TierArgs {
  int T;
  int toff[FVS_MAX_TIERS];   // byte offset of the tier's first plane in the record
  int kb[FVS_MAX_TIERS];     // bytes per plane = d_t / 8
  int bits[FVS_MAX_TIERS];
  int loff[FVS_MAX_TIERS];   // LUT offset of the tier = start * 4
  float delta[FVS_MAX_TIERS];
  float mid[FVS_MAX_TIERS];  // (2^b - 1) / 2
};

template <bool HALF>
__global__ __launch_bounds__(256) void k_lut_build(const uint16_t *__restrict__ Zq, int D, void *__restrict__ Lout,
                                                   TierArgs ta, float *__restrict__ qsum, float *__restrict__ qn2,
                                                   int64_t B) {
  const int64_t q = blockIdx.x;
  const int nn = D / 4;
  const int64_t LW = (int64_t)nn * 16;
  const uint16_t *zr = Zq + q * D;
  for (int n = threadIdx.x; n < nn; n += 256) {
    float z[4];
#pragma unroll
    for (int i = 0; i < 4; i++) z[i] = fvs_h2f(zr[4 * n + i]);
    float o[16];
#pragma unroll
    for (int v = 0; v < 16; v++) {
      float acc = 0.f;
#pragma unroll
      for (int i = 0; i < 4; i++) acc = __builtin_fmaf(z[i], (float)((v >> (3 - i)) & 1), acc);
      o[v] = acc;
    }
    if (HALF) {
      uint16_t *L = reinterpret_cast<uint16_t *>(Lout) + q * LW + (int64_t)n * 16;
      uint32_t w[8];
#pragma unroll
      for (int v = 0; v < 8; v++) w[v] = (uint32_t)fvs_f2h(o[2 * v]) | ((uint32_t)fvs_f2h(o[2 * v + 1]) << 16);
      uint4 *L4 = reinterpret_cast<uint4 *>(L);
      L4[0] = make_uint4(w[0], w[1], w[2], w[3]);
      L4[1] = make_uint4(w[4], w[5], w[6], w[7]);
    } else {
      float *L = reinterpret_cast<float *>(Lout) + q * LW + (int64_t)n * 16;
      float4 *L4 = reinterpret_cast<float4 *>(L);
#pragma unroll
      for (int v = 0; v < 4; v++) L4[v] = make_float4(o[4 * v], o[4 * v + 1], o[4 * v + 2], o[4 * v + 3]);
    }
  }
  // per-tier sums, one thread per tier (the unrolled loop keeps the argument-struct index uniform)
#pragma unroll
  for (int t = 0; t < FVS_MAX_TIERS; t++) {
    if (t < ta.T && (int)threadIdx.x == t) {
      const int i0 = ta.loff[t] / 4, i1 = i0 + 8 * ta.kb[t];
      double s1 = 0.0, s2 = 0.0;
      for (int i = i0; i < i1; i++) {
        const double x = (double)fvs_h2f(zr[i]);
        s1 += x;
        s2 += x * x;
      }
      qsum[(int64_t)t * B + q] = (float)s1;
      qn2[(int64_t)t * B + q] = (float)s2;
    }
  }
}

constexpr int kScoreThreads = 128;

template <bool HALF>
__global__ __launch_bounds__(kScoreThreads) void k_lut_score(
    const int32_t *__restrict__ pos, const float *__restrict__ qc, const void *__restrict__ Lin, int LW,
    const float *__restrict__ qsum, const float *__restrict__ qn2, const uint8_t *__restrict__ rec, int RB, int soff,
    TierArgs ta, const int32_t *__restrict__ ncnt, int64_t N, int64_t B, int K, float *__restrict__ est,
    float *__restrict__ sdo) {
  extern __shared__ int32_t smem[];
  int32_t *lut = smem;                                               // [LW]
  uint32_t *meta = reinterpret_cast<uint32_t *>(smem + LW);          // [nw]
  const int nw = soff / 4;
  float *tf = reinterpret_cast<float *>(meta + nw);                  // [T][4]: delta, mid, qsum, qn2
  uint32_t *ssw = reinterpret_cast<uint32_t *>(tf + 4 * FVS_MAX_TIERS);  // [threads][8]
  __shared__ float red[2];
  __shared__ int sexp;

  const int64_t q = blockIdx.x;
  const int tid = threadIdx.x;

  // 1. fixed-point exponent of this query's table
  float m = 0.f;
  if (HALF) {
    const uint16_t *L = reinterpret_cast<const uint16_t *>(Lin) + q * LW;
    for (int i = tid; i < LW; i += kScoreThreads) m = fmaxf(m, fabsf(fvs_h2f(L[i])));
  } else {
    const float *L = reinterpret_cast<const float *>(Lin) + q * LW;
    for (int i = tid; i < LW; i += kScoreThreads) m = fmaxf(m, fabsf(L[i]));
  }
  m = fvs_wave_max(m);
  if ((tid & 63) == 0) red[tid >> 6] = m;
  __syncthreads();
  if (tid == 0) {
    int E = 0;
    (void)frexpf(fmaxf(red[0], red[1]), &E);
    sexp = max(0, E - 3);
  }
  __syncthreads();
  const int s = sexp;

  // 2. integer LUT, per-dword descriptors, per-tier constants
  if (HALF) {
    const uint16_t *L = reinterpret_cast<const uint16_t *>(Lin) + q * LW;
    for (int i = tid; i < LW; i += kScoreThreads) lut[i] = (int32_t)rintf(ldexpf(fvs_h2f(L[i]), 24 - s));
  } else {
    const float *L = reinterpret_cast<const float *>(Lin) + q * LW;
    for (int i = tid; i < LW; i += kScoreThreads) lut[i] = (int32_t)rintf(ldexpf(L[i], 24 - s));
  }
  for (int w = tid; w < nw; w += kScoreThreads) {
    const int byte = 4 * w;
    uint32_t d = 0;
    for (int t = 0; t < ta.T; t++) {
      const int len = ta.bits[t] * ta.kb[t];
      if (byte >= ta.toff[t] && byte < ta.toff[t] + len) {
        const int rel = byte - ta.toff[t];
        const int p = rel / ta.kb[t];
        const int j0 = rel - p * ta.kb[t];
        const uint32_t base = (uint32_t)(ta.loff[t] + 32 * j0);
        const uint32_t shift = (uint32_t)(ta.bits[t] - 1 - p);
        const uint32_t last = (byte + 4 == ta.toff[t] + len) ? 1u : 0u;
        d = base | (shift << 16) | (last << 19) | ((uint32_t)t << 20);
      }
    }
    meta[w] = d;
  }
#pragma unroll
  for (int t = 0; t < FVS_MAX_TIERS; t++) {
    if (t < ta.T && tid == t) {
      tf[4 * t + 0] = ta.delta[t];
      tf[4 * t + 1] = ta.mid[t];
      tf[4 * t + 2] = qsum[(int64_t)t * B + q];
      tf[4 * t + 3] = qn2[(int64_t)t * B + q];
    }
  }
  __syncthreads();

  const int lim = ncnt ? min(ncnt[q], K) : K;
  const float qcq = qc[q];
  const int nchunk = RB / 16;
  for (int mm = tid; mm < K; mm += kScoreThreads) {
    const int64_t o = q * (int64_t)K + mm;
    if (mm >= lim) {
      est[o] = -1e30f;
      sdo[o] = 0.f;
      continue;
    }
    const int64_t row = min(max((int64_t)pos[o], (int64_t)0), N - 1);  // positions come from fvs_select
    const uint8_t *rp = rec + row * RB;
    const uint32_t *rp32 = reinterpret_cast<const uint32_t *>(rp);
    const uint4 *rp16 = reinterpret_cast<const uint4 *>(rp);
    for (int t = 0; t < ta.T; t++) ssw[tid * 8 + t] = rp32[soff / 4 + t];
    int64_t acc = 0;
    float e = qcq, var = 0.f;
    for (int w0 = 0; w0 < nw; w0 += 32) {
      uint4 ch[8];
#pragma unroll
      for (int u = 0; u < 8; u++) {
        const int ci = w0 / 4 + u;
        ch[u] = ci < nchunk ? rp16[ci] : make_uint4(0, 0, 0, 0);
      }
#pragma unroll
      for (int u = 0; u < 8; u++) {
        const uint32_t xs[4] = {ch[u].x, ch[u].y, ch[u].z, ch[u].w};
#pragma unroll
        for (int ee = 0; ee < 4; ee++) {
          const int w = w0 + 4 * u + ee;
          if (w < nw) {
            const uint32_t mt = meta[w];
            const int base = (int)(mt & 0xffffu);
            const uint32_t x = xs[ee];
            const int part = lut[base + ((x >> 4) & 15)] + lut[base + 16 + (x & 15)] +
                             lut[base + 32 + ((x >> 12) & 15)] + lut[base + 48 + ((x >> 8) & 15)] +
                             lut[base + 64 + ((x >> 20) & 15)] + lut[base + 80 + ((x >> 16) & 15)] +
                             lut[base + 96 + (x >> 28)] + lut[base + 112 + ((x >> 24) & 15)];
            acc += (int64_t)part << ((mt >> 16) & 7);
            if (mt & (1u << 19)) {
              const int t = (int)(mt >> 20);
              float a = ldexpf((float)acc, s - 24);
              a = tf[4 * t] * __builtin_fmaf(-tf[4 * t + 1], tf[4 * t + 2], a);
              const uint32_t sw = ssw[tid * 8 + t];
              const float sc = fvs_h2f((uint16_t)(sw & 0xffffu)), sg = fvs_h2f((uint16_t)(sw >> 16));
              e = __builtin_fmaf(a, sc, e);
              var = __builtin_fmaf(tf[4 * t + 3] * sg, sg, var);
              acc = 0;
            }
          }
        }
      }
    }
    est[o] = e;
    sdo[o] = sqrtf(var);
  }
}

int fill_tiers(int T, const int32_t *tiers, const float *deltas, const int32_t *toff, TierArgs *ta, int D_limit) {
  if (T <= 0 || T > FVS_MAX_TIERS || !tiers) return FVS_E_SHAPE;
  ta->T = T;
  int prev_end = 0;
  for (int t = 0; t < T; t++) {
    const int s = tiers[3 * t], e = tiers[3 * t + 1], b = tiers[3 * t + 2];
    if (s != prev_end || e <= s || (e - s) % 32 != 0 || b < 1 || b > 8 || e > D_limit) return FVS_E_SHAPE;
    prev_end = e;
    ta->kb[t] = (e - s) / 8;
    ta->bits[t] = b;
    ta->loff[t] = s * 4;
    ta->toff[t] = toff ? toff[t] : 0;
    ta->delta[t] = deltas ? deltas[t] : 0.f;
    ta->mid[t] = (float)((1 << b) - 1) * 0.5f;
  }
  return FVS_OK;
}

}  // namespace

extern "C" int fvs_lut_build(const uint16_t *Zq, int64_t B, int32_t D, int32_t T, const int32_t *tiers, int32_t half,
                             void *L, float *qsum, float *qn2, void *stream) {
  if (B < 0 || D <= 0 || D % 32 != 0) return FVS_E_ARG;
  TierArgs ta;
  int e = fill_tiers(T, tiers, nullptr, nullptr, &ta, D);
  if (e) return e;
  if (tiers[3 * (T - 1) + 1] != D) return FVS_E_SHAPE;
  if (B == 0) return FVS_OK;
  if (!Zq || !L || !qsum || !qn2) return FVS_E_ARG;
  hipStream_t st = (hipStream_t)stream;
  if (half)
    hipLaunchKernelGGL(k_lut_build<true>, dim3((unsigned)B), dim3(256), 0, st, Zq, D, L, ta, qsum, qn2, B);
  else
    hipLaunchKernelGGL(k_lut_build<false>, dim3((unsigned)B), dim3(256), 0, st, Zq, D, L, ta, qsum, qn2, B);
  return fvs_launch_status();
}

extern "C" int fvs_lut_score(const int32_t *pos, const float *qc, const void *L, int32_t half, int32_t LW,
                             const float *qsum, const float *qn2, const uint8_t *rec, int64_t N, int32_t RB,
                             int32_t soff, int32_t T, const int32_t *tiers, const float *deltas, const int32_t *toff,
                             const int32_t *ncnt, int64_t B, int32_t K, float *est, float *sd, void *stream) {
  if (B < 0 || K <= 0 || N <= 0 || LW <= 0 || LW > 16384 || LW % 16 != 0) return FVS_E_ARG;
  if (RB <= 0 || RB % 16 != 0 || soff <= 0 || soff % 4 != 0) return FVS_E_ARG;
  if (!toff || !deltas) return FVS_E_ARG;
  TierArgs ta;
  int e = fill_tiers(T, tiers, deltas, toff, &ta, LW / 4);
  if (e) return e;
  // planes must tile [0, soff) in tier order and the (scale, sigma) pairs must fit in the record
  int at = 0;
  for (int t = 0; t < T; t++) {
    if (ta.toff[t] != at) return FVS_E_SHAPE;
    at += ta.bits[t] * ta.kb[t];
  }
  if (at != soff || soff + 4 * T > RB) return FVS_E_SHAPE;
  if (B == 0) return FVS_OK;
  if (!pos || !qc || !L || !qsum || !qn2 || !rec || !est || !sd) return FVS_E_ARG;
  const size_t shm = (size_t)LW * 4 + (size_t)(soff / 4) * 4 + 4 * FVS_MAX_TIERS * 4 + kScoreThreads * 8 * 4;
  if (shm > 160 * 1024 - 64) return FVS_E_CAPACITY;
  hipStream_t st = (hipStream_t)stream;
  if (half)
    hipLaunchKernelGGL(k_lut_score<true>, dim3((unsigned)B), dim3(kScoreThreads), shm, st, pos, qc, L, LW, qsum, qn2,
                       rec, RB, soff, ta, ncnt, N, B, K, est, sd);
  else
    hipLaunchKernelGGL(k_lut_score<false>, dim3((unsigned)B), dim3(kScoreThreads), shm, st, pos, qc, L, LW, qsum,
                       qn2, rec, RB, soff, ta, ncnt, N, B, K, est, sd);
  return fvs_launch_status();
}
