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
  // per-tier sums, one wave per tier: lane l sums coordinates start+l, start+l+64, ... in double,
  // then a fixed xor butterfly (the unrolled tier loop keeps the argument-struct index uniform)
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
#pragma unroll
  for (int t = 0; t < FVS_MAX_TIERS; t++) {
    if (t < ta.T && (t & 3) == wv) {
      const int i0 = ta.loff[t] / 4, i1 = i0 + 8 * ta.kb[t];
      double s1 = 0.0, s2 = 0.0;
      for (int i = i0 + lane; i < i1; i += 64) {
        const double x = (double)fvs_h2f(zr[i]);
        s1 += x;
        s2 += x * x;
      }
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) {
        s1 += __shfl_xor(s1, o, FVS_WAVE);
        s2 += __shfl_xor(s2, o, FVS_WAVE);
      }
      if (lane == 0) {
        qsum[(int64_t)t * B + q] = (float)s1;
        qn2[(int64_t)t * B + q] = (float)s2;
      }
    }
  }
}

constexpr int kScoreThreads = 128;
constexpr int kUnit = 16;  // 16-byte chunks per pipeline unit (256 bytes of a record)

// Per-dword descriptors (LDS): planes carry the LUT byte offset, the plane weight, an end-of-tier flag
// and the tier; the dwords after the planes carry the (scale, sigma) pair of tier t.
constexpr uint32_t kMetaLast = 1u << 24;
constexpr uint32_t kMetaScale = 1u << 25;

struct RecUnit {
  uint4 c[kUnit];
};

__device__ __forceinline__ void load_unit(RecUnit &b, const uint8_t *__restrict__ rec, int64_t row, int RB, int u,
                                          int nchunk, bool live) {
  const uint4 *rp = reinterpret_cast<const uint4 *>(rec + row * RB) + u * kUnit;
#pragma unroll
  for (int c = 0; c < kUnit; c++) b.c[c] = (live && u * kUnit + c < nchunk) ? rp[c] : make_uint4(0, 0, 0, 0);
}

template <bool HALF>
__global__ __launch_bounds__(kScoreThreads) void k_lut_score(
    const int32_t *__restrict__ pos, const float *__restrict__ qc, const void *__restrict__ Lin, int LW,
    const float *__restrict__ qsum, const float *__restrict__ qn2, const uint8_t *__restrict__ rec, int RB, int soff,
    TierArgs ta, const int32_t *__restrict__ ncnt, int64_t N, int64_t B, int K, float *__restrict__ est,
    float *__restrict__ sdo) {
  extern __shared__ int32_t smem[];
  int32_t *lut = smem;                                                 // [LW] fixed-point table
  const int nw = soff / 4;
  uint32_t *meta = reinterpret_cast<uint32_t *>(smem + LW);            // [nw + T], padded to even
  float *tf = reinterpret_cast<float *>(meta + ((nw + FVS_MAX_TIERS + 1) & ~1));  // [T][4]: delta, mid, qsum, qn2
  uint32_t *ssw = reinterpret_cast<uint32_t *>(tf + 4 * FVS_MAX_TIERS);  // [threads][T] (scale, sigma)
  int64_t *acct = reinterpret_cast<int64_t *>(ssw + kScoreThreads * FVS_MAX_TIERS);  // [threads][T]
  int32_t *rows = reinterpret_cast<int32_t *>(acct + kScoreThreads * FVS_MAX_TIERS);  // [K]
  __shared__ float red[2];
  __shared__ int sexp;

  const int64_t q = blockIdx.x;
  const int tid = threadIdx.x;
  const int T = ta.T;

  // 1. fixed-point exponent of this query's table (vectorised passes over the table)
  float m = 0.f;
  if (HALF) {
    const uint4 *L4 = reinterpret_cast<const uint4 *>(reinterpret_cast<const uint16_t *>(Lin) + q * LW);
#pragma unroll 8
    for (int i = tid; i < LW / 8; i += kScoreThreads) {
      const uint4 v = L4[i];
      const uint32_t w4[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int u = 0; u < 4; u++)
        m = fmaxf(m, fmaxf(fabsf(fvs_h2f((uint16_t)(w4[u] & 0xffffu))), fabsf(fvs_h2f((uint16_t)(w4[u] >> 16)))));
    }
  } else {
    const float4 *L4 = reinterpret_cast<const float4 *>(reinterpret_cast<const float *>(Lin) + q * LW);
#pragma unroll 8
    for (int i = tid; i < LW / 4; i += kScoreThreads) {
      const float4 v = L4[i];
      m = fmaxf(m, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
    }
  }
  m = fvs_wave_max(m);
  if ((tid & 63) == 0) red[tid >> 6] = m;
  // candidate rows of this query, staged while the reduction settles
  const int lim = ncnt ? min(ncnt[q], K) : K;
  for (int i = tid; i < K; i += kScoreThreads) rows[i] = (int32_t)min(max((int64_t)pos[q * (int64_t)K + i], (int64_t)0), N - 1);
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
    const uint4 *L4 = reinterpret_cast<const uint4 *>(reinterpret_cast<const uint16_t *>(Lin) + q * LW);
#pragma unroll 8
    for (int i = tid; i < LW / 8; i += kScoreThreads) {
      const uint4 v = L4[i];
      const uint32_t w4[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int u = 0; u < 4; u++) {
        lut[8 * i + 2 * u] = (int32_t)rintf(ldexpf(fvs_h2f((uint16_t)(w4[u] & 0xffffu)), 24 - s));
        lut[8 * i + 2 * u + 1] = (int32_t)rintf(ldexpf(fvs_h2f((uint16_t)(w4[u] >> 16)), 24 - s));
      }
    }
  } else {
    const float4 *L4 = reinterpret_cast<const float4 *>(reinterpret_cast<const float *>(Lin) + q * LW);
#pragma unroll 8
    for (int i = tid; i < LW / 4; i += kScoreThreads) {
      const float4 v = L4[i];
      lut[4 * i + 0] = (int32_t)rintf(ldexpf(v.x, 24 - s));
      lut[4 * i + 1] = (int32_t)rintf(ldexpf(v.y, 24 - s));
      lut[4 * i + 2] = (int32_t)rintf(ldexpf(v.z, 24 - s));
      lut[4 * i + 3] = (int32_t)rintf(ldexpf(v.w, 24 - s));
    }
  }
  for (int w = tid; w < nw + T; w += kScoreThreads) {
    uint32_t d = 0;
    if (w >= nw) {
      d = kMetaScale | (uint32_t)(w - nw);
    } else {
      const int byte = 4 * w;
      for (int t = 0; t < T; t++) {
        const int len = ta.bits[t] * ta.kb[t];
        if (byte >= ta.toff[t] && byte < ta.toff[t] + len) {
          const int rel = byte - ta.toff[t];
          const int p = rel / ta.kb[t];
          const int j0 = rel - p * ta.kb[t];
          const uint32_t base = (uint32_t)(ta.loff[t] + 32 * j0) * 4u;  // byte offset in the table
          const uint32_t shift = (uint32_t)(ta.bits[t] - 1 - p);
          const uint32_t last = (byte + 4 == ta.toff[t] + len) ? kMetaLast : 0u;
          d = base | (shift << 17) | last | ((uint32_t)t << 20);
        }
      }
    }
    meta[w] = d;
  }
#pragma unroll
  for (int t = 0; t < FVS_MAX_TIERS; t++) {
    if (t < T && tid == t) {
      tf[4 * t + 0] = ta.delta[t];
      tf[4 * t + 1] = ta.mid[t];
      tf[4 * t + 2] = qsum[(int64_t)t * B + q];
      tf[4 * t + 3] = qn2[(int64_t)t * B + q];
    }
  }
  __syncthreads();

  // 3. candidates: lane `tid` scores slots tid, tid + 128, ...; the record stream is cut into units of
  //    256 bytes and double-buffered in registers, so the next unit is in flight while one is summed
  const int nchunk = (soff + 4 * T + 15) / 16;  // chunks holding planes and (scale, sigma) pairs
  const int U = (nchunk + kUnit - 1) / kUnit;
  const int nround = (K + kScoreThreads - 1) / kScoreThreads;
  const int S = nround * U;
  const char *lutb = reinterpret_cast<const char *>(lut);
  const float qcq = qc[q];
  RecUnit ub0, ub1;
  int64_t acc = 0;
  // one pipeline step: `cur` holds unit sq, `nxt` receives unit sq + 1
  auto step = [&](int sq, const RecUnit &cur, RecUnit &nxt) {
    const int i = sq / U, u = sq - i * U;
    const int mm = tid + kScoreThreads * i;
    const bool live = mm < lim;
    if (sq + 1 < S) {
      const int i1 = (sq + 1) / U, u1 = (sq + 1) - i1 * U;
      const int m1 = tid + kScoreThreads * i1;
      load_unit(nxt, rec, m1 < lim ? rows[m1] : 0, RB, u1, nchunk, m1 < lim);
    }
    if (live) {
#pragma unroll
      for (int c = 0; c < kUnit; c++) {
        const uint32_t xs[4] = {cur.c[c].x, cur.c[c].y, cur.c[c].z, cur.c[c].w};
#pragma unroll
        for (int ee = 0; ee < 4; ee++) {
          const int w = (u * kUnit + c) * 4 + ee;
          if (w < nw) {
            const uint32_t mt = meta[w];
            const char *lb = lutb + (mt & 0x1ffffu);
            const uint32_t x = xs[ee];
            const uint32_t xh = (x >> 2) & 0x3c3c3c3cu, xl = (x << 2) & 0x3c3c3c3cu;  // nibble * 4 per byte
            int part = 0;
#pragma unroll
            for (int j = 0; j < 4; j++) {
              part += *reinterpret_cast<const int32_t *>(lb + 128 * j + ((xh >> (8 * j)) & 0xffu));
              part += *reinterpret_cast<const int32_t *>(lb + 128 * j + 64 + ((xl >> (8 * j)) & 0xffu));
            }
            acc += (int64_t)part << ((mt >> 17) & 7u);
            if (mt & kMetaLast) {
              acct[tid * FVS_MAX_TIERS + ((mt >> 20) & 7u)] = acc;
              acc = 0;
            }
          } else if (w < nw + T) {
            ssw[tid * FVS_MAX_TIERS + (w - nw)] = xs[ee];
          }
        }
      }
    }
    if (u == U - 1 && mm < K) {
      const int64_t o = q * (int64_t)K + mm;
      if (!live) {
        est[o] = -1e30f;
        sdo[o] = 0.f;
      } else {
        float e = qcq, var = 0.f;
        for (int t = 0; t < T; t++) {
          float a = ldexpf((float)acct[tid * FVS_MAX_TIERS + t], s - 24);
          a = tf[4 * t] * __builtin_fmaf(-tf[4 * t + 1], tf[4 * t + 2], a);
          const uint32_t sw = ssw[tid * FVS_MAX_TIERS + t];
          const float sc = fvs_h2f((uint16_t)(sw & 0xffffu)), sg = fvs_h2f((uint16_t)(sw >> 16));
          e = __builtin_fmaf(a, sc, e);
          var = __builtin_fmaf(tf[4 * t + 3] * sg, sg, var);
        }
        est[o] = e;
        sdo[o] = sqrtf(var);
      }
    }
  };
  load_unit(ub0, rec, tid < lim ? rows[tid] : 0, RB, 0, nchunk, tid < lim);
  for (int sq = 0; sq < S; sq += 2) {
    step(sq, ub0, ub1);
    if (sq + 1 < S) step(sq + 1, ub1, ub0);
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
  if (K > 4096) return FVS_E_CAPACITY;
  const size_t shm = (size_t)LW * 4 + (size_t)((soff / 4 + FVS_MAX_TIERS + 1) & ~1) * 4 + 4 * FVS_MAX_TIERS * 4 +
                     (size_t)kScoreThreads * FVS_MAX_TIERS * (4 + 8) + (size_t)K * 4;
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
