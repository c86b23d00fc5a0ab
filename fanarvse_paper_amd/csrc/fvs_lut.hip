// Uniform tiered refinement code: nibble lookup tables and the LUT stage-2 scorer with error bars.
//
// Scorer mapping: one block (4 waves) per query. The query's LUT is converted once into 32-bit
// fixed point in LDS, so every plane sum is an exact integer and the result does not depend on the
// summation order (any lane/tile mapping gives the same bits). Each lane scores one candidate:
// it streams the candidate's packed record in 128-byte units (the next unit in flight while one is
// summed), looks up two LUT entries per code byte, and folds the per-tier integer sums into the f32
// estimate in tier order. All lanes of a wave process the same record dword at the same time, so the
// per-dword descriptor (LUT base, end-of-plane, end-of-tier and pair flags) is wave-uniform: the host
// builds these descriptors once per record layout and passes them as a kernel argument, so they reach
// scalar registers through the scalar cache; the lookups of one dword hit one 64-byte table (no LDS
// bank conflicts), and the only branches, at a plane's or tier's end or a pair, are uniform.
#include <type_traits>

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
        s1 += fvs_xor_lane_d(s1, o);
        s2 += fvs_xor_lane_d(s2, o);
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
constexpr int kUD = kUnit * 4;       // dwords per unit
constexpr int kZeroBytes = 512;      // zero table after the LUT: dwords past the planes look up zeros
constexpr int kSchedMax = 512;       // record dwords (whole units) the schedule covers: records up to 2 KiB
constexpr int kSetupVec = 16;        // 16-byte table vectors per thread in the one-pass set-up (LW <= 16384)
constexpr int kSetupPos = 4;         // FUSED: 4-coordinate table groups per thread (D <= 4096)

// Schedule: one descriptor per record dword, the same for every record and query, built on the host and
// passed as a kernel argument. Kernel arguments are read through the scalar cache, so a dword's descriptor
// arrives in a scalar register with no vector instruction.
//   bit 0      ends a plane that is not its tier's last: the tier sum is doubled after this dword
//   bit 6      the dword ends a plane or tier or is a (scale, sigma) pair: the one flag the summing loop tests
//   bit 7      ends a tier
//   bit 8      is the (scale, sigma) pair of the next tier in order
//   bits 9-16  byte offset of the dword's 512-byte table group in LDS (the zero table past the planes)
// A tier's planes come most significant first, so its sum sum_p 2^(b-1-p) S_p is formed by Horner's rule:
// every dword adds its entries unshifted and the sum doubles at each plane end but the last.
constexpr uint32_t kSchedDouble = 1u << 0;
constexpr uint32_t kSchedSpecial = 1u << 6;
constexpr uint32_t kSchedLast = 1u << 7;
constexpr uint32_t kSchedPair = 1u << 8;
constexpr uint32_t kSchedBase = 0x1fe00u;
struct ScoreSched {
  uint32_t d[kSchedMax];
};

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

// The 8 LUT entries of one record dword x whose 512-byte table group starts at byte lb: byte j's high
// nibble indexes the table at lb + 128 j, its low nibble the table at lb + 128 j + 64 (tables of 16 int32
// = 64 bytes, nibble * 4 = byte offset).
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

// FUSED: the kernel builds the query's table and tier sums itself from its rotated query Zq (fp16 [B, D]), with
// k_lut_build's operations (the same entries, fp16-rounded when HALF, and the same double sums), instead of
// reading the table L and the sums qsum / qn2 that k_lut_build wrote; the results are the same bits.
template <bool HALF, int TT, bool FUSED>
__global__ __launch_bounds__(kScoreThreads) void k_lut_score(
    const int32_t *__restrict__ pos, const float *__restrict__ qc, const void *__restrict__ Lin, int LW,
    const float *__restrict__ qsum, const float *__restrict__ qn2, const uint16_t *__restrict__ Zq, int D,
    const uint8_t *__restrict__ rec, int RB, int U, TierArgs ta, ScoreSched sched, const int32_t *__restrict__ ncnt,
    int64_t N, int64_t B, int K, float *__restrict__ est, float *__restrict__ sdo) {
  // the table comes first in LDS (no static LDS), so a schedule offset is an LDS address as it stands
  extern __shared__ int32_t smem[];
  int32_t *lut = smem;                                                  // [LW] fixed-point tables + zero table
  float *tf = reinterpret_cast<float *>(smem + LW + kZeroBytes / 4);    // [T][4]: delta, mid, qsum, qn2
  float *red = tf + 4 * FVS_MAX_TIERS;                                  // [waves] exponent reduction
  int32_t *rows = reinterpret_cast<int32_t *>(red + kScoreThreads / FVS_WAVE);  // [K]

  const int64_t q = blockIdx.x;
  const int tid = threadIdx.x;
  const int T = ta.T;

  // 1. every global read of the set-up is issued at once: the query's table (one pass, held in registers),
  //    its candidate rows, its tier constants, and the first unit of this lane's first record
  const int nvec = HALF ? LW / 8 : LW / 4;  // 16-byte vectors of the table: 8 halves or 4 floats each
  uint4 lv[FUSED ? 1 : kSetupVec];
  uint2 zv[FUSED ? kSetupPos : 1];  // FUSED: the four query coordinates of each of this thread's table groups
  if constexpr (FUSED) {
    const uint2 *Z2 = reinterpret_cast<const uint2 *>(Zq + q * (int64_t)D);
#pragma unroll
    for (int c = 0; c < kSetupPos; c++)
      if (tid + kScoreThreads * c < D / 4) zv[c] = Z2[tid + kScoreThreads * c];
  } else {
    const uint4 *L4 = reinterpret_cast<const uint4 *>(Lin) + q * nvec;
#pragma unroll
    for (int c = 0; c < kSetupVec; c++)
      if (tid + kScoreThreads * c < nvec) lv[c] = L4[tid + kScoreThreads * c];
  }
  const int lim = ncnt ? min(ncnt[q], K) : K;
  for (int i = tid; i < K; i += kScoreThreads)
    rows[i] = (int32_t)min(max((int64_t)pos[q * (int64_t)K + i], (int64_t)0), N - 1);
  float tq0 = 0.f, tq1 = 0.f;
  if (!FUSED && tid < T) {
    tq0 = qsum[(int64_t)tid * B + q];
    tq1 = qn2[(int64_t)tid * B + q];
  }
  const int RB16 = RB / 16;
  RecUnit ub0, ub1;
  {
    const int64_t r0 = tid < lim ? min(max((int64_t)pos[q * (int64_t)K + tid], (int64_t)0), N - 1) : 0;
    load_unit(ub0, rec, r0, RB16, 0);
  }

  // 2. fixed-point exponent of the table, then the integer table, zero table and per-tier constants
  constexpr int kPer = HALF ? 8 : 4;  // entries per vector
  auto entry = [&](const uint4 &v, int u) {  // entry u of a vector (u static)
    const int d = HALF ? u >> 1 : u;
    const uint32_t x = d == 0 ? v.x : d == 1 ? v.y : d == 2 ? v.z : v.w;
    return HALF ? fvs_h2f((uint16_t)((u & 1) ? x >> 16 : x & 0xffffu)) : __uint_as_float(x);
  };
  float m = 0.f;
  float ov[FUSED ? kSetupPos : 1][16];  // FUSED: this thread's table entries (group tid + 256 c, nibble v)
  if constexpr (FUSED) {
    // entries as k_lut_build computes them: sum over i of fmaf(z_i, bit (3 - i) of v, .) in i order, then
    // fp16-rounded when HALF
#pragma unroll
    for (int c = 0; c < kSetupPos; c++) {
      if (tid + kScoreThreads * c < D / 4) {
        const float z[4] = {fvs_h2f((uint16_t)(zv[c].x & 0xffffu)), fvs_h2f((uint16_t)(zv[c].x >> 16)),
                            fvs_h2f((uint16_t)(zv[c].y & 0xffffu)), fvs_h2f((uint16_t)(zv[c].y >> 16))};
#pragma unroll
        for (int v = 0; v < 16; v++) {
          float a = 0.f;
#pragma unroll
          for (int i = 0; i < 4; i++) a = __builtin_fmaf(z[i], (float)((v >> (3 - i)) & 1), a);
          ov[c][v] = HALF ? fvs_round_h(a) : a;
          m = fmaxf(m, fabsf(ov[c][v]));
        }
      }
    }
    // the tier sums as k_lut_build forms them: wave t & 3 sums tier t, lane l the coordinates start + l,
    // start + l + 64, ... in double, then a fixed xor butterfly
    const int lane = tid & 63, wv = fvs_wave_id();
    const uint16_t *zr = Zq + q * (int64_t)D;
#pragma unroll
    for (int t = 0; t < FVS_MAX_TIERS; t++) {
      if (t < T && (t & 3) == wv) {
        const int i0 = ta.loff[t] / 4, i1 = i0 + 8 * ta.kb[t];
        double s1 = 0.0, s2 = 0.0;
        for (int i = i0 + lane; i < i1; i += 64) {
          const double x = (double)fvs_h2f(zr[i]);
          s1 += x;
          s2 += x * x;
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
          s1 += fvs_xor_lane_d(s1, o);
          s2 += fvs_xor_lane_d(s2, o);
        }
        if (lane == 0) {
          tf[4 * t + 2] = (float)s1;
          tf[4 * t + 3] = (float)s2;
        }
      }
    }
  } else {
#pragma unroll
    for (int c = 0; c < kSetupVec; c++)
      if (tid + kScoreThreads * c < nvec) {
#pragma unroll
        for (int u = 0; u < kPer; u++) m = fmaxf(m, fabsf(entry(lv[c], u)));
      }
  }
  m = fvs_wave_max(m);
  if ((tid & 63) == 0) red[tid >> 6] = m;
  __syncthreads();
  int s;
  {
    float mm = red[0];
#pragma unroll
    for (int w = 1; w < kScoreThreads / FVS_WAVE; w++) mm = fmaxf(mm, red[w]);
    int E = 0;
    (void)frexpf(mm, &E);
    s = max(0, E - 3);
  }
  if constexpr (FUSED) {
#pragma unroll
    for (int c = 0; c < kSetupPos; c++) {
      const int n = tid + kScoreThreads * c;
      if (n < D / 4) {
        int32_t w[16];
#pragma unroll
        for (int v = 0; v < 16; v++) w[v] = (int32_t)rintf(ldexpf(ov[c][v], 24 - s));
        int4 *dst = reinterpret_cast<int4 *>(lut + 16 * n);
#pragma unroll
        for (int v = 0; v < 4; v++) dst[v] = make_int4(w[4 * v], w[4 * v + 1], w[4 * v + 2], w[4 * v + 3]);
      }
    }
  } else {
#pragma unroll
    for (int c = 0; c < kSetupVec; c++) {
      const int i = tid + kScoreThreads * c;
      if (i < nvec) {
#pragma unroll
        for (int u = 0; u < kPer; u++) lut[kPer * i + u] = (int32_t)rintf(ldexpf(entry(lv[c], u), 24 - s));
      }
    }
  }
  for (int i = tid; i < kZeroBytes / 4; i += kScoreThreads) lut[LW + i] = 0;
#pragma unroll
  for (int t = 0; t < FVS_MAX_TIERS; t++) {
    if (t < T && tid == t) {
      tf[4 * t + 0] = ta.delta[t];
      tf[4 * t + 1] = ta.mid[t];
      if (!FUSED) {
        tf[4 * t + 2] = tq0;
        tf[4 * t + 3] = tq1;
      }
    }
  }
  __syncthreads();

  // 3. candidates: lane `tid` scores slots tid, tid + 256, ...; each record is streamed in units of kUnit
  //    16-byte chunks, double-buffered in registers, and the lookups of dword k + 1 are issued before the
  //    entries of dword k are summed. The tier sums and (scale, sigma) words stay in registers: tiers end,
  //    and their pairs come, in tier order, so each is shifted into a register queue of TT entries, where
  //    tier t ends up at position TT - 1 - t.
  const int nround = (K + kScoreThreads - 1) / kScoreThreads;
  const char *lutb = reinterpret_cast<const char *>(lut);
  const float qcq = qc[q];
  int64_t acc = 0;
  int64_t tsum[TT];
  uint32_t tss[TT];
#pragma unroll
  for (int t = 0; t < TT; t++) {
    tsum[t] = 0;
    tss[t] = 0u;
  }
  // every step issues the same unconditional loads (the last one reloads its own unit), so the wait
  // before a unit is summed never has to drain the prefetch of the next one
  auto row_of = [&](int mm) {
    const int r = rows[min(mm, K - 1)];
    return mm < lim ? r : 0;
  };
  // step (i, u): sum unit u of the record of slot tid + 256 i; (ni, nu): the next step, prefetched
  auto step = [&](int i, int u, int ni, int nu, const RecUnit &cur, RecUnit &nxt) {
    const int mm = tid + kScoreThreads * i;
    // the unit's descriptors, fetched together: one scalar-load wait per unit (it also waits for LDS)
    uint32_t sd[kUD];
#pragma unroll
    for (int k = 0; k < kUD; k++) sd[k] = sched.d[u * kUD + k];
#pragma unroll
    for (int k = 0; k < kUD; k++) asm volatile("" : "+s"(sd[k]));
    load_unit(nxt, rec, row_of(tid + kScoreThreads * ni), RB16, nu);
    // wave-uniform: skip waves whose lanes are all past the candidate list
    if (kScoreThreads * i + (tid & ~(FVS_WAVE - 1)) < lim) {
      int32_t va[8], vb[8];
      // an even dword that is not special (no plane, tier or pair end) shares its plane with the next
      // dword: its entries are carried in `pk` and added to the tier sum with the next dword's, so the
      // 64-bit add happens once per pair. |entry| < 2^27 (the fixed-point exponent), so 16 entries fit
      // in 32 bits.
      int32_t pk = 0;
      lookup8(lutb, unit_word(cur, 0), sd[0] & kSchedBase, va);
#pragma unroll
      for (int k = 0; k < kUD; k++) {
        int32_t(&vc)[8] = (k & 1) ? vb : va;
        int32_t(&vn)[8] = (k & 1) ? va : vb;
        if (k + 1 < kUD) lookup8(lutb, unit_word(cur, k + 1), sd[k + 1] & kSchedBase, vn);
        const uint32_t dk = sd[k];
        const int32_t part = vc[0] + vc[1] + vc[2] + vc[3] + vc[4] + vc[5] + vc[6] + vc[7] + ((k & 1) ? pk : 0);
        if ((k & 1) == 0) pk = part;
        if ((k & 1) || (dk & kSchedSpecial)) acc += (int64_t)part;
        if (dk & kSchedSpecial) {
          if ((k & 1) == 0) pk = 0;
          if (dk & kSchedDouble) acc <<= 1;
          if (dk & kSchedLast) {
#pragma unroll
            for (int t = TT - 1; t > 0; t--) tsum[t] = tsum[t - 1];
            tsum[0] = acc;
            acc = 0;
          }
          if (dk & kSchedPair) {
#pragma unroll
            for (int t = TT - 1; t > 0; t--) tss[t] = tss[t - 1];
            tss[0] = unit_word(cur, k);
          }
        }
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
        for (int t = 0; t < TT; t++) {  // tier t sits at queue position TT - 1 - t
          float a = ldexpf((float)tsum[TT - 1 - t], s - 24);
          a = tf[4 * t] * __builtin_fmaf(-tf[4 * t + 1], tf[4 * t + 2], a);
          const uint32_t sw = tss[TT - 1 - t];
          const float sc = fvs_h2f((uint16_t)(sw & 0xffffu)), sg = fvs_h2f((uint16_t)(sw >> 16));
          e = __builtin_fmaf(a, sc, e);
          var = __builtin_fmaf(tf[4 * t + 3] * sg, sg, var);
        }
        est[o] = e;
        sdo[o] = sqrtf(var);
      }
    }
  };
  const int S = nround * U;
  int ci = 0, cu = 0;  // the step about to run
  auto advance = [&](int &i, int &u) {
    if (++u == U) {
      u = 0;
      ++i;
    }
  };
  for (int sq = 0; sq < S; sq += 2) {
    int ni = ci, nu = cu;
    advance(ni, nu);
    if (sq + 1 >= S) {  // the last step reloads its own unit
      ni = ci;
      nu = cu;
    }
    step(ci, cu, ni, nu, ub0, ub1);
    if (sq + 1 < S) {
      int mi = ni, mu = nu;
      advance(mi, mu);
      if (sq + 2 >= S) {
        mi = ni;
        mu = nu;
      }
      step(ni, nu, mi, mu, ub1, ub0);
      ci = mi;
      cu = mu;
    }
  }
}

// The schedule of a record layout (see ScoreSched): plane dwords look up their tier's tables and mark the
// ends of planes and tiers; the T (scale, sigma) dwords after the planes and the padding up to whole units
// look up the zero table.
int build_sched(const TierArgs &ta, int nw, int U, int LW, ScoreSched *sc) {
  if (U * kUD > kSchedMax) return FVS_E_CAPACITY;
  const uint32_t zero = (uint32_t)LW * 4u;
  if ((zero & ~kSchedBase) != 0) return FVS_E_SHAPE;
  for (int w = 0; w < U * kUD; w++) {
    uint32_t d = zero;
    if (w >= nw && w < nw + ta.T) d |= kSchedSpecial | kSchedPair;
    if (w < nw) {
      const int byte = 4 * w;
      for (int t = 0; t < ta.T; t++) {
        const int len = ta.bits[t] * ta.kb[t];
        if (byte >= ta.toff[t] && byte < ta.toff[t] + len) {
          const int rel = byte - ta.toff[t];
          const int p = rel / ta.kb[t];
          const int j0 = rel - p * ta.kb[t];
          const uint32_t base = (uint32_t)(ta.loff[t] + 32 * j0) * 4u;  // byte offset of the dword's table group
          if ((base & ~kSchedBase) != 0) return FVS_E_SHAPE;
          d = base;
          if (byte + 4 == ta.toff[t] + len) d |= kSchedSpecial | kSchedLast;
          else if (j0 + 4 == ta.kb[t]) d |= kSchedSpecial | kSchedDouble;
        }
      }
    }
    sc->d[w] = d;
  }
  for (int w = U * kUD; w < kSchedMax; w++) sc->d[w] = zero;
  return FVS_OK;
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

namespace {

// Checks, schedule and launch shared by fvs_lut_score (table L and sums qsum / qn2 from fvs_lut_build) and
// fvs_lut_score_zq (the kernel builds them from the rotated queries Zq: fused = true).
int lut_score_impl(const int32_t *pos, const float *qc, const void *L, int32_t half, int32_t LW, const float *qsum,
                   const float *qn2, const uint16_t *Zq, int32_t D, bool fused, const uint8_t *rec, int64_t N,
                   int32_t RB, int32_t soff, int32_t T, const int32_t *tiers, const float *deltas,
                   const int32_t *toff, int32_t nt, const int32_t *ncnt, int64_t B, int32_t K, float *est, float *sd,
                   void *stream) {
  // LW = 16 entries per 4 coordinates, in whole 512-byte table groups (tiers are whole 32-coordinate blocks)
  if (B < 0 || K <= 0 || N <= 0 || LW <= 0 || LW > 16384 || LW % 128 != 0) return FVS_E_ARG;
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
  // a partial estimate scores the leading nt tiers: the schedule then covers their planes and pairs only
  // (the other dwords look up the zero table), and the tier queues hold nt entries
  if (nt < 0 || nt > T) return FVS_E_ARG;
  if (nt > 0) ta.T = nt;
  if (B == 0) return FVS_OK;
  if (!pos || !qc || !rec || !est || !sd) return FVS_E_ARG;
  if (fused ? !Zq : (!L || !qsum || !qn2)) return FVS_E_ARG;
  if (K > 4096) return FVS_E_CAPACITY;
  const int units = (soff / 4 + T + kUD - 1) / kUD;
  ScoreSched sched;
  e = build_sched(ta, soff / 4, units, LW, &sched);
  if (e) return e;
  const size_t shm = (size_t)LW * 4 + kZeroBytes + 4 * FVS_MAX_TIERS * 4 + kScoreThreads / FVS_WAVE * 4 +
                     (size_t)K * 4;
  if (shm > 160 * 1024 - 64) return FVS_E_CAPACITY;
  hipStream_t st = (hipStream_t)stream;
  // one instantiation per tier count, so the tier queues have a static size
  auto launch = [&](auto HALF_, auto TT_, auto FUSED_) {
    hipLaunchKernelGGL((k_lut_score<decltype(HALF_)::value, decltype(TT_)::value, decltype(FUSED_)::value>),
                       dim3((unsigned)B), dim3(kScoreThreads), shm, st, pos, qc, L, LW, qsum, qn2, Zq, D, rec, RB,
                       units, ta, sched, ncnt, N, B, K, est, sd);
  };
  auto by_t = [&](auto HALF_, auto FUSED_) {
    switch (ta.T) {
      case 1: launch(HALF_, std::integral_constant<int, 1>{}, FUSED_); break;
      case 2: launch(HALF_, std::integral_constant<int, 2>{}, FUSED_); break;
      case 3: launch(HALF_, std::integral_constant<int, 3>{}, FUSED_); break;
      case 4: launch(HALF_, std::integral_constant<int, 4>{}, FUSED_); break;
      case 5: launch(HALF_, std::integral_constant<int, 5>{}, FUSED_); break;
      case 6: launch(HALF_, std::integral_constant<int, 6>{}, FUSED_); break;
      case 7: launch(HALF_, std::integral_constant<int, 7>{}, FUSED_); break;
      default: launch(HALF_, std::integral_constant<int, 8>{}, FUSED_); break;
    }
  };
  if (fused) {
    if (half)
      by_t(std::true_type{}, std::true_type{});
    else
      by_t(std::false_type{}, std::true_type{});
  } else {
    if (half)
      by_t(std::true_type{}, std::false_type{});
    else
      by_t(std::false_type{}, std::false_type{});
  }
  return fvs_launch_status();
}

}  // namespace

extern "C" int fvs_lut_score(const int32_t *pos, const float *qc, const void *L, int32_t half, int32_t LW,
                             const float *qsum, const float *qn2, const uint8_t *rec, int64_t N, int32_t RB,
                             int32_t soff, int32_t T, const int32_t *tiers, const float *deltas, const int32_t *toff,
                             int32_t nt, const int32_t *ncnt, int64_t B, int32_t K, float *est, float *sd,
                             void *stream) {
  return lut_score_impl(pos, qc, L, half, LW, qsum, qn2, nullptr, 0, false, rec, N, RB, soff, T, tiers, deltas, toff,
                        nt, ncnt, B, K, est, sd, stream);
}

extern "C" int fvs_lut_score_zq(const int32_t *pos, const float *qc, const uint16_t *Zq, int32_t D, int32_t half,
                                const uint8_t *rec, int64_t N, int32_t RB, int32_t soff, int32_t T,
                                const int32_t *tiers, const float *deltas, const int32_t *toff, int32_t nt,
                                const int32_t *ncnt, int64_t B, int32_t K, float *est, float *sd, void *stream) {
  // the table covers the D coordinates of the tiers: 16 entries per 4 coordinates; the last tier ends at D
  if (D <= 0 || D % 32 != 0 || D > 4 * kScoreThreads * kSetupPos) return FVS_E_ARG;
  if (T <= 0 || T > FVS_MAX_TIERS || !tiers || tiers[3 * (T - 1) + 1] != D) return FVS_E_SHAPE;
  return lut_score_impl(pos, qc, nullptr, half, D / 4 * 16, nullptr, nullptr, Zq, D, true, rec, N, RB, soff, T,
                        tiers, deltas, toff, nt, ncnt, B, K, est, sd, stream);
}
