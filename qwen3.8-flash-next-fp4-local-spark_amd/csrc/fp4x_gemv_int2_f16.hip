// Explicit GEMV instantiations (one translation unit per weight format, so
// the library compiles in parallel).
#include "fp4x_mfma.h"
#include "fp4x_stream.h"

namespace fp4x {
template int launch_gemv_mfma<FmtInt2<false, 16>, EpiStore>(const GemvLaunch&, int, hipStream_t);
template int launch_gemv_mfma<FmtInt2<false, 32>, EpiStore>(const GemvLaunch&, int, hipStream_t);
template int launch_gemv_mfma<FmtInt2<false, 0>, EpiStore>(const GemvLaunch&, int, hipStream_t);
bool launch_int2_stream_f16(GemvLaunch p, hipStream_t st) {
  return p.pa.G == 32 ? launch_int2_stream<false, 32>(p, st) : launch_int2_stream<false, 16>(p, st);
}
}  // namespace fp4x
