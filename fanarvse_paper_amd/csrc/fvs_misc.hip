// Version, error strings and a graph-capturable fill.
#include "fvs_common.h"

namespace {

__global__ void k_fill_u32(uint32_t *__restrict__ dst, int64_t n, uint32_t value) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) dst[i] = value;
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

extern "C" int fvs_pack_ids(const uint8_t *ok, const int32_t *I, int64_t B, int32_t k, int64_t *out, void *stream) {
  if (B < 0 || k <= 0) return FVS_E_ARG;
  if (B == 0) return FVS_OK;
  if (!ok || !I || !out) return FVS_E_ARG;
  int64_t blocks = (B * (k + 1) + 255) / 256;
  if (blocks > 8192) blocks = 8192;
  hipLaunchKernelGGL(k_pack_ids, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream, ok, I, B, (int)k, out);
  return fvs_launch_status();
}
