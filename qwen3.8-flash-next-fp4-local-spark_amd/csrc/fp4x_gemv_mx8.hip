// Explicit GEMV instantiations (one translation unit per weight format, so
// the library compiles in parallel).
#include "fp4x_kernels.h"

namespace fp4x {
template int launch_gemv<FmtMX8, EpiStore, 1>(const GemvLaunch&, int, hipStream_t);
}  // namespace fp4x
