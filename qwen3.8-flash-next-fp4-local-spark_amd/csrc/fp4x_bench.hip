// A plain coalesced read, the reference point the GEMVs' times are compared
// with: one launch reads `bytes` of HBM with 16-byte loads, U of them in
// flight per thread, over wgs_per_cu workgroups of 256 threads per CU.  The
// benchmark sweeps U and the grid and keeps the fastest, so its time is the
// measured ceiling of a one-shot read of that size on this GPU.
#include <hip/hip_runtime.h>
#include <string>

#include "../../include/fp4x.h"

namespace fp4x {
void set_error(const std::string& msg);
int check_launch(const char* what);
int device_cus();

template <int U>
__global__ __launch_bounds__(256) void read_stream_kernel(const uint4* __restrict__ src, int64_t n, uint32_t* sink) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  uint32_t acc = 0;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += U * stride) {
    uint4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) v[u] = i + u * stride < n ? src[i + u * stride] : make_uint4(0, 0, 0, 0);
#pragma unroll
    for (int u = 0; u < U; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  }
  // keeps the loads live; the data would have to fold to this exact word
  if (acc == 0x9e3779b9u) sink[0] = acc;
}
}  // namespace fp4x

using namespace fp4x;

extern "C" {

int fp4x_read_ceiling(const void* src, int64_t bytes, int unroll, int wgs_per_cu, uint32_t* sink, void* stream) {
  if (bytes <= 0 || bytes % 16 || (reinterpret_cast<uintptr_t>(src) & 15) || !sink || wgs_per_cu < 1 ||
      wgs_per_cu > 32) {
    set_error("read_ceiling: need 16-byte aligned src, bytes a positive multiple of 16, 1 <= wgs_per_cu <= 32");
    return FP4X_ERR_ARG;
  }
  const int64_t n = bytes / 16;
  const dim3 grid((unsigned)(device_cus() * wgs_per_cu)), block(256);
  const uint4* p = static_cast<const uint4*>(src);
  hipStream_t st = (hipStream_t)stream;
  switch (unroll) {
    case 2: hipLaunchKernelGGL(read_stream_kernel<2>, grid, block, 0, st, p, n, sink); break;
    case 4: hipLaunchKernelGGL(read_stream_kernel<4>, grid, block, 0, st, p, n, sink); break;
    case 8: hipLaunchKernelGGL(read_stream_kernel<8>, grid, block, 0, st, p, n, sink); break;
    case 16: hipLaunchKernelGGL(read_stream_kernel<16>, grid, block, 0, st, p, n, sink); break;
    default: set_error("read_ceiling: unroll must be 2, 4, 8 or 16"); return FP4X_ERR_ARG;
  }
  return check_launch("read_ceiling");
}

}  // extern "C"
