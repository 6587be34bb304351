// libsdv: status strings, ABI version and the device E4M3FN encoder entry point.
#include "sdv_internal.h"

namespace sdv {

__global__ __launch_bounds__(256) void fp8_encode_kernel(const float* __restrict__ in, uint8_t* __restrict__ out,
                                                         int64_t n) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride)
    out[i] = (uint8_t)e4m3fn_encode(in[i]);
}

}  // namespace sdv

using namespace sdv;

extern "C" int sdv_fp8_encode(const float* in, uint8_t* out, int64_t n, void* stream) {
  if (!in || !out) return SDV_ERR_NULL;
  if (n < 0) return SDV_ERR_SHAPE;
  if (!aligned(in, 4)) return SDV_ERR_ALIGN;
  if (n == 0) return SDV_OK;
  const int64_t want = (n + 255) / 256;
  const unsigned blocks = (unsigned)(want < 65536 ? want : 65536);
  hipLaunchKernelGGL(fp8_encode_kernel, dim3(blocks), dim3(256), 0, static_cast<hipStream_t>(stream), in, out, n);
  return hipGetLastError() == hipSuccess ? SDV_OK : SDV_ERR_HIP;
}

extern "C" const char* sdv_status_string(int status) {
  switch (status) {
    case SDV_OK: return "ok";
    case SDV_ERR_NULL: return "a required pointer argument is NULL";
    case SDV_ERR_SHAPE: return "a size argument is out of range or inconsistent";
    case SDV_ERR_UNSUPPORTED: return "unsupported configuration (head_dim must be 64 or 128, group_size == head_dim)";
    case SDV_ERR_WORKSPACE: return "workspace is NULL, too small or not 256-byte aligned";
    case SDV_ERR_ALIGN: return "a tensor pointer or layer stride is not aligned as required";
    case SDV_ERR_HIP: return "the HIP runtime reported an error at kernel launch";
    default: return "unknown status";
  }
}

extern "C" int sdv_abi_version(void) { return SDV_ABI_VERSION; }
