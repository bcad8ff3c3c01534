// Explicit GEMV instantiations (one translation unit per weight format, so
// the library compiles in parallel).
#include "fp4x_mfma.h"

namespace fp4x {
template int launch_gemv_mfma<FmtInt2<true, 16>, EpiStore>(const GemvLaunch&, int, hipStream_t);
template int launch_gemv_mfma<FmtInt2<true, 32>, EpiStore>(const GemvLaunch&, int, hipStream_t);
template int launch_gemv_mfma<FmtInt2<true, 0>, EpiStore>(const GemvLaunch&, int, hipStream_t);
}  // namespace fp4x
