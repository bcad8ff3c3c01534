// The fast head's coarse stage (fp4x_int2_topk) for callers that cannot
// allocate device memory: code under HIP graph capture, tight serving loops.
// Its one scratch buffer, the top-k's slice maxima, lives in a file-scope
// device array instead of a caller's workspace.
//
//   * Size: a row's slice maxima take at most 32768 u16 (the top-k keeps the
//     slices of a row at or below 32768 by lengthening them), i.e. 64 KiB, and
//     the GEMV takes at most 16 rows: 1 MiB covers every call.  Larger
//     requests are rejected.
//   * Every GPU the library runs on holds its own copy of the array until the
//     process ends.  Its address is looked up once per device (the first call
//     on that device, with it current) with hipGetSymbolAddress and kept;
//     host code passes that address, never the array's name, to the kernels.
//   * The slice maxima need no initial contents: every entry the select reads
//     is written first by the same call.  Calls on one device share the
//     array, so calls that overlap in time (different streams) race.
#include <hip/hip_runtime.h>
#include <mutex>
#include <string>

#include "../../include/fp4x.h"

namespace fp4x {
void set_error(const std::string& msg);
}

namespace {

constexpr int64_t kScratchBytes = 1 << 20;
constexpr int kMaxDevices = 64;

__device__ __align__(256) uint8_t scratch[kScratchBytes];

std::mutex g_mu;
void* g_ptr[kMaxDevices] = {};

// The array's device address on the current device (nullptr and an error
// message on failure).
void* scratch_on_current_device() {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    (void)hipGetLastError();
    fp4x::set_error("int2_topk_noalloc: no current HIP device (or more than 64 devices)");
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(g_mu);
  if (!g_ptr[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      (void)hipGetLastError();
      fp4x::set_error(std::string("int2_topk_noalloc: hipGetSymbolAddress of the static workspace failed: ") +
                      hipGetErrorString(e));
      return nullptr;
    }
    g_ptr[dev] = p;
  }
  return g_ptr[dev];
}

}  // namespace

extern "C" {

int64_t fp4x_int2_topk_noalloc_limit(void) { return kScratchBytes; }

int fp4x_int2_topk_noalloc(const void* x, int64_t x_stride, const void* P, const void* S, int s_fmt, const float* rs,
                           void* coarse, int coarse_dtype, int64_t coarse_stride, int M, int N, int K, int G, int C,
                           int64_t* idx_out, int set_only, void* stream) {
  const int64_t need = fp4x_topk_workspace_size(M, N);
  if (need > kScratchBytes) {
    fp4x::set_error("int2_topk_noalloc: M rows of N logits need " + std::to_string(need) +
                    " bytes of slice maxima, above the static workspace's " + std::to_string(kScratchBytes));
    return FP4X_ERR_ARG;
  }
  void* ws = scratch_on_current_device();
  if (!ws) return FP4X_ERR_LAUNCH;
  return fp4x_int2_topk(x, x_stride, P, S, s_fmt, rs, coarse, coarse_dtype, coarse_stride, M, N, K, G, C, idx_out,
                        set_only, ws, kScratchBytes, stream);
}

}  // extern "C"
