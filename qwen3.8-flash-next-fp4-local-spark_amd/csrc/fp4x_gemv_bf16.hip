// Explicit GEMV instantiations (one translation unit per weight format, so
// the library compiles in parallel).
#include "fp4x_mfma.h"

namespace fp4x {
template int launch_gemv_mfma<FmtBF16, EpiStore>(const GemvLaunch&, int, hipStream_t);
}  // namespace fp4x
