// Uniform tiered refinement code: nibble lookup tables and the LUT stage-2 scorer with error bars.
//
// Scorer mapping: one block (4 waves) per query. The query's LUT is converted once into 32-bit
// fixed point in LDS, so every plane sum is an exact integer and the result does not depend on the
// summation order (any lane/tile mapping gives the same bits). Each lane scores one candidate:
// it streams the candidate's packed record in 128-byte units (the next unit in flight while one is
// summed), looks up two LUT entries per code byte, and folds the per-tier integer sums into the f32
// estimate in tier order. All lanes of a wave process the same record dword at the same time, so the
// per-dword descriptor (LUT base, plane weight, end-of-tier flag) is wave-uniform: it is read from a
// lane register into a scalar register, the lookups of one dword hit one 64-byte table (no LDS bank
// conflicts), and the only branch, at a tier's end, is uniform.
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
  const int lane = threadIdx.x & 63, wv = fvs_wave_id();
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

constexpr int kScoreThreads = 256;
constexpr int kUnit = 8;             // 16-byte chunks per pipeline unit (128 bytes of a record)
constexpr int kUD = kUnit * 4;       // dwords per unit; lane l of a wave holds the descriptor of dword l % kUD
constexpr int kZeroBytes = 512;      // zero table after the LUT: dwords past the planes look up zeros

// Per-dword descriptors (LDS, one per dword of every unit): the LUT byte offset of the dword's first table,
// the plane weight (shift), the tier, an end-of-tier flag, and a flag for the (scale, sigma) dword of tier t.
constexpr uint32_t kMetaLast = 1u << 24;
constexpr uint32_t kMetaPair = 1u << 25;

struct RecUnit {
  uint4 c[kUnit];
};

// Unit u of record `row`. Every lane loads (dead lanes read row 0) and chunks past the record are clamped
// to its last chunk, so the loads are unconditional and the pipeline's wait counts stay exact.
__device__ __forceinline__ void load_unit(RecUnit &b, const uint8_t *__restrict__ rec, int64_t row, int RB16, int u) {
  const uint4 *rp = reinterpret_cast<const uint4 *>(rec) + row * RB16;
#pragma unroll
  for (int c = 0; c < kUnit; c++) b.c[c] = rp[min(u * kUnit + c, RB16 - 1)];
}

__device__ __forceinline__ uint32_t unit_word(const RecUnit &b, int k) {
  const uint4 &c = b.c[k >> 2];
  return (k & 3) == 0 ? c.x : (k & 3) == 1 ? c.y : (k & 3) == 2 ? c.z : c.w;
}

// The 8 LUT entries of one record dword: byte j's high nibble indexes the table at lb + 128 j, its low
// nibble the table at lb + 128 j + 64 (tables of 16 int32 = 64 bytes, nibble * 4 = byte offset).
__device__ __forceinline__ void lookup8(const char *lutb, uint32_t x, uint32_t lb, int32_t (&v)[8]) {
  uint32_t xh = (x >> 2) & 0x3c3c3c3cu, xl = (x << 2) & 0x3c3c3c3cu;
  // opaque to the optimiser, so each byte stays a byte-select operand of the address add (SDWA) instead
  // of being refolded into a shift and a mask per lookup
  asm("" : "+v"(xh), "+v"(xl));
#pragma unroll
  for (int j = 0; j < 4; j++) {
    v[2 * j] = *reinterpret_cast<const int32_t *>(lutb + (lb + __builtin_amdgcn_ubfe(xh, 8 * j, 8)) + 128 * j);
    v[2 * j + 1] = *reinterpret_cast<const int32_t *>(lutb + (lb + __builtin_amdgcn_ubfe(xl, 8 * j, 8)) + 128 * j + 64);
  }
}

template <bool HALF>
__global__ __launch_bounds__(kScoreThreads) void k_lut_score(
    const int32_t *__restrict__ pos, const float *__restrict__ qc, const void *__restrict__ Lin, int LW,
    const float *__restrict__ qsum, const float *__restrict__ qn2, const uint8_t *__restrict__ rec, int RB, int soff,
    TierArgs ta, const int32_t *__restrict__ ncnt, int64_t N, int64_t B, int K, float *__restrict__ est,
    float *__restrict__ sdo) {
  extern __shared__ int32_t smem[];
  int32_t *lut = smem;                                                  // [LW] fixed-point table + zero table
  const int nw = soff / 4;                                              // plane dwords
  const int U = (nw + ta.T + kUD - 1) / kUD;                            // units per record (planes + pairs)
  uint32_t *meta = reinterpret_cast<uint32_t *>(smem + LW + kZeroBytes / 4);  // [U * kUD]
  float *tf = reinterpret_cast<float *>(meta + U * kUD);                // [T][4]: delta, mid, qsum, qn2
  int64_t *acct = reinterpret_cast<int64_t *>(tf + 4 * FVS_MAX_TIERS);  // [T][threads] tier sums
  uint32_t *ssw = reinterpret_cast<uint32_t *>(acct + ta.T * kScoreThreads);  // [T][threads] (scale, sigma)
  int32_t *rows = reinterpret_cast<int32_t *>(ssw + ta.T * kScoreThreads);  // [K]
  __shared__ float red[kScoreThreads / FVS_WAVE];
  __shared__ int sexp;

  const int64_t q = blockIdx.x;
  const int tid = threadIdx.x;
  const int T = ta.T;

  // 1. fixed-point exponent of this query's table (vectorised passes over the table)
  float m = 0.f;
  if (HALF) {
    const uint4 *L4 = reinterpret_cast<const uint4 *>(reinterpret_cast<const uint16_t *>(Lin) + q * LW);
#pragma unroll 4
    for (int i = tid; i < LW / 8; i += kScoreThreads) {
      const uint4 v = L4[i];
      const uint32_t w4[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int u = 0; u < 4; u++)
        m = fmaxf(m, fmaxf(fabsf(fvs_h2f((uint16_t)(w4[u] & 0xffffu))), fabsf(fvs_h2f((uint16_t)(w4[u] >> 16)))));
    }
  } else {
    const float4 *L4 = reinterpret_cast<const float4 *>(reinterpret_cast<const float *>(Lin) + q * LW);
#pragma unroll 4
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
    float mm = red[0];
#pragma unroll
    for (int w = 1; w < kScoreThreads / FVS_WAVE; w++) mm = fmaxf(mm, red[w]);
    int E = 0;
    (void)frexpf(mm, &E);
    sexp = max(0, E - 3);
  }
  __syncthreads();
  const int s = sexp;

  // 2. integer LUT, zero table, per-dword descriptors, per-tier constants
  if (HALF) {
    const uint4 *L4 = reinterpret_cast<const uint4 *>(reinterpret_cast<const uint16_t *>(Lin) + q * LW);
#pragma unroll 4
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
#pragma unroll 4
    for (int i = tid; i < LW / 4; i += kScoreThreads) {
      const float4 v = L4[i];
      lut[4 * i + 0] = (int32_t)rintf(ldexpf(v.x, 24 - s));
      lut[4 * i + 1] = (int32_t)rintf(ldexpf(v.y, 24 - s));
      lut[4 * i + 2] = (int32_t)rintf(ldexpf(v.z, 24 - s));
      lut[4 * i + 3] = (int32_t)rintf(ldexpf(v.w, 24 - s));
    }
  }
  for (int i = tid; i < kZeroBytes / 4; i += kScoreThreads) lut[LW + i] = 0;
  for (int w = tid; w < U * kUD; w += kScoreThreads) {
    uint32_t d = (uint32_t)LW * 4u;  // past the planes: the zero table, weight 1, never the end of a tier
    if (w >= nw && w < nw + T) d |= kMetaPair | ((uint32_t)(w - nw) << 20);
    if (w < nw) {
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

  // 3. candidates: lane `tid` scores slots tid, tid + threads, ...; each record is streamed in units of
  //    kUnit 16-byte chunks, double-buffered in registers, and the lookups of dword k + 1 are issued
  //    before the entries of dword k are summed
  const int RB16 = RB / 16;
  const int nround = (K + kScoreThreads - 1) / kScoreThreads;
  const int S = nround * U;
  const char *lutb = reinterpret_cast<const char *>(lut);
  const float qcq = qc[q];
  const int lane = tid & (FVS_WAVE - 1);
  RecUnit ub0, ub1;
  int64_t acc = 0;
  // every step issues the same unconditional loads (the last one reloads its own unit), so the wait
  // before a unit is summed never has to drain the prefetch of the next one
  auto row_of = [&](int m) {
    const int r = rows[min(m, K - 1)];
    return m < lim ? r : 0;
  };
  auto step = [&](int sq, const RecUnit &cur, RecUnit &nxt) {
    const int i = sq / U, u = sq - i * U;
    const int mm = tid + kScoreThreads * i;
    const uint32_t mv = meta[u * kUD + (lane & (kUD - 1))];
    {
      const int sq1 = min(sq + 1, S - 1);
      const int i1 = sq1 / U, u1 = sq1 - i1 * U;
      load_unit(nxt, rec, row_of(tid + kScoreThreads * i1), RB16, u1);
    }
    // wave-uniform: skip waves whose lanes are all past the candidate list
    if (kScoreThreads * i + (tid & ~(FVS_WAVE - 1)) < lim) {
      int32_t va[8], vb[8];
      lookup8(lutb, unit_word(cur, 0), __builtin_amdgcn_readlane(mv, 0) & 0x1ffffu, va);
#pragma unroll
      for (int k = 0; k < kUD; k++) {
        int32_t(&vc)[8] = (k & 1) ? vb : va;
        int32_t(&vn)[8] = (k & 1) ? va : vb;
        if (k + 1 < kUD) lookup8(lutb, unit_word(cur, k + 1), __builtin_amdgcn_readlane(mv, k + 1) & 0x1ffffu, vn);
        const uint32_t mt = __builtin_amdgcn_readlane(mv, k);
        const int32_t part = vc[0] + vc[1] + vc[2] + vc[3] + vc[4] + vc[5] + vc[6] + vc[7];
        acc += (int64_t)part << ((mt >> 17) & 7u);
        if (mt & kMetaLast) {
          acct[((mt >> 20) & 7u) * kScoreThreads + tid] = acc;
          acc = 0;
        }
        if (mt & kMetaPair) ssw[((mt >> 20) & 7u) * kScoreThreads + tid] = unit_word(cur, k);
      }
    }
    if (u == U - 1 && mm < K) {
      const int64_t o = q * (int64_t)K + mm;
      if (mm >= lim) {
        est[o] = -1e30f;
        sdo[o] = 0.f;
      } else {
        float e = qcq, var = 0.f;
#pragma unroll
        for (int t = 0; t < FVS_MAX_TIERS; t++) {
          if (t < T) {
            float a = ldexpf((float)acct[t * kScoreThreads + tid], s - 24);
            a = tf[4 * t] * __builtin_fmaf(-tf[4 * t + 1], tf[4 * t + 2], a);
            const uint32_t sw = ssw[t * kScoreThreads + tid];
            const float sc = fvs_h2f((uint16_t)(sw & 0xffffu)), sg = fvs_h2f((uint16_t)(sw >> 16));
            e = __builtin_fmaf(a, sc, e);
            var = __builtin_fmaf(tf[4 * t + 3] * sg, sg, var);
          }
        }
        est[o] = e;
        sdo[o] = sqrtf(var);
      }
    }
  };
  load_unit(ub0, rec, row_of(tid), RB16, 0);
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
  const int units = (soff / 4 + T + kUD - 1) / kUD;
  const size_t shm = (size_t)LW * 4 + kZeroBytes + (size_t)units * kUD * 4 + 4 * FVS_MAX_TIERS * 4 +
                     (size_t)kScoreThreads * T * (8 + 4) + (size_t)K * 4;
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
