// A plain coalesced read, the reference point the GEMVs' times are compared
// with: one launch reads `bytes` of HBM with 16-byte loads, U of them in
// flight per thread, over wgs_per_cu workgroups of 256 threads per CU.  The
// benchmark sweeps U and the grid and keeps the fastest, so its time is the
// measured ceiling of a one-shot read of that size on this GPU.
// Also a kernel that holds CUs for a fixed time, with which a test makes
// another kernel's workgroups start late.
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

// Holds a CU for `ticks` of the constant wall clock: the workgroup's dynamic
// LDS keeps other workgroups that need LDS off its CU.  The loop also ends
// after max_iter sleeps, so it ends even if the clock were to stop.
__global__ __launch_bounds__(64) void hold_cu_kernel(uint64_t ticks, int max_iter, uint32_t* sink) {
  const uint64_t t0 = wall_clock64();
  int it = 0;
  while (wall_clock64() - t0 < ticks && it < max_iter) {
    __builtin_amdgcn_s_sleep(32);
    ++it;
  }
  if (it == 0x7fffffff) sink[0] = 1;                 // never true: keeps the loop
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

int fp4x_hold_cus(int wgs, int64_t microseconds, int lds_kb, uint32_t* sink, void* stream) {
  if (wgs < 1 || wgs > 4096 || microseconds < 0 || microseconds > 100000 || lds_kb < 1 || lds_kb > 160 || !sink) {
    set_error("hold_cus: need 1 <= wgs <= 4096, 0 <= microseconds <= 100000, 1 <= lds_kb <= 160");
    return FP4X_ERR_ARG;
  }
  int khz = 0;
  if (hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, 0) != hipSuccess || khz <= 0) {
    set_error("hold_cus: no wall clock rate");
    return FP4X_ERR_LAUNCH;
  }
  const size_t lds = (size_t)lds_kb * 1024;
  if (lds > 64 * 1024 && hipFuncSetAttribute(reinterpret_cast<const void*>(hold_cu_kernel),
                                             hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess) {
    (void)hipGetLastError();
    set_error("hold_cus: the LDS size was refused");
    return FP4X_ERR_LAUNCH;
  }
  const uint64_t ticks = (uint64_t)microseconds * (uint64_t)khz / 1000;
  // a sleep of 32 x 64 cycles is at least about 0.5 us: 2 per microsecond bounds the loop above its time
  const int max_iter = (int)(microseconds * 2 + 1000);
  hipLaunchKernelGGL(hold_cu_kernel, dim3(wgs), dim3(64), lds, (hipStream_t)stream, ticks, max_iter, sink);
  return check_launch("hold_cus");
}

}  // extern "C"
