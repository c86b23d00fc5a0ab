// Version, error strings, a graph-capturable fill and the matrix-core calibration kernel.
#include "fvs_common.h"

namespace {

__global__ void k_fill_u32(uint32_t *__restrict__ dst, int64_t n, uint32_t value) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) dst[i] = value;
}

// The achievable int8 matrix-core rate of the device for the emit scan's instruction mix: per round each wave
// runs four independent 4-step accumulation chains of v_mfma_i32_16x16x64_i8 (16 MFMAs, each chain started
// from a fresh accumulator, as the scan's tiles are) on register operands, with no memory access in the loop,
// and folds one element of each result into a checksum that lane 0 writes to out[wave], so that the work is
// kept. One round is 16 x 16 x 16 x 64 multiply-adds per wave.
__global__ __launch_bounds__(256) void k_calib_mfma(int iters, int32_t *__restrict__ out) {
  const int tid = threadIdx.x;
  const int lane = tid & (FVS_WAVE - 1);
  v4i a[4], b[4];
#pragma unroll
  for (int s = 0; s < 4; s++) {
    a[s] = (v4i){(lane + s) * 0x01010101, (lane + 1) * 0x01010101, (lane + 2) * 0x01010101, (lane + 3) * 0x01010101};
    b[s] = (v4i){0x01020304 ^ (lane + s), 0x05060708 ^ lane, 0x090a0b0c, 0x0d0e0f10};
  }
  int32_t sum = 0;
  for (int i = 0; i < iters; i++) {
    v4i c[4];
#pragma unroll
    for (int s = 0; s < 4; s++)
#pragma unroll
      for (int j = 0; j < 4; j++)
        c[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[s], b[(s + j) & 3], s == 0 ? (v4i){i, 0, 0, 0} : c[j], 0, 0, 0);
#pragma unroll
    for (int j = 0; j < 4; j++) sum ^= c[j][j];
  }
  if (lane == 0) out[(int64_t)blockIdx.x * (256 / FVS_WAVE) + (tid >> 6)] = sum;
}

// [ok | ids] of each query as int64: out[q * (k + 1)] = ok[q], out[q * (k + 1) + 1 + j] = I[q * k + j].
__global__ void k_pack_ids(const uint8_t *__restrict__ ok, const int32_t *__restrict__ I, int64_t B, int k,
                           int64_t *__restrict__ out) {
  const int64_t n = B * (k + 1);
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
    const int64_t q = i / (k + 1);
    const int j = (int)(i - q * (k + 1));
    out[i] = j == 0 ? (int64_t)ok[q] : (int64_t)I[q * k + j - 1];
  }
}

}  // namespace

extern "C" int fvs_abi_version(void) { return FVS_ABI_VERSION; }

extern "C" const char *fvs_error_string(int code) {
  switch (code) {
    case FVS_OK: return "ok";
    case FVS_E_ARG: return "argument out of range";
    case FVS_E_SHAPE: return "unsupported shape";
    case FVS_E_CAPACITY: return "per-workgroup capacity exceeded";
    default: return code > 0 ? hipGetErrorString((hipError_t)code) : "unknown error";
  }
}

extern "C" int fvs_fill_u32(void *dst, int64_t n, uint32_t value, void *stream) {
  if (n < 0) return FVS_E_ARG;
  if (n == 0) return FVS_OK;
  if (!dst) return FVS_E_ARG;
  int64_t blocks = (n + 255) / 256;
  if (blocks > 8192) blocks = 8192;
  hipLaunchKernelGGL(k_fill_u32, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, (uint32_t *)dst, n, value);
  return fvs_launch_status();
}

extern "C" int fvs_calib_mfma(int32_t blocks, int32_t iters, int32_t *out, void *stream) {
  if (blocks <= 0 || iters <= 0) return FVS_E_ARG;
  if (!out) return FVS_E_ARG;
  hipLaunchKernelGGL(k_calib_mfma, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, (int)iters, out);
  return fvs_launch_status();
}

extern "C" int fvs_pack_ids(const uint8_t *ok, const int32_t *I, int64_t B, int32_t k, int64_t *out, void *stream) {
  if (B < 0 || k <= 0) return FVS_E_ARG;
  if (B == 0) return FVS_OK;
  if (!ok || !I || !out) return FVS_E_ARG;
  int64_t blocks = (B * (k + 1) + 255) / 256;
  if (blocks > 8192) blocks = 8192;
  hipLaunchKernelGGL(k_pack_ids, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, ok, I, B, (int)k, out);
  return fvs_launch_status();
}
