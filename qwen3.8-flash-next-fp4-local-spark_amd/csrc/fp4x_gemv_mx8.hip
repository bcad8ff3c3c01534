// Explicit GEMV instantiations (one translation unit per weight format, so
// the library compiles in parallel).
#include "fp4x_stream.h"

namespace fp4x {
template int launch_gemv_mfma<FmtMX8, EpiStore>(const GemvLaunch&, int, hipStream_t);
bool launch_mx8_stream_entry(GemvLaunch p, hipStream_t st) { return launch_mx8_stream(p, st); }
bool launch_mx8_stream_tile_entry(GemvLaunch p, hipStream_t st) {
  return launch_stream_tile_per_wg<StreamMX8>(p, switches().mx8_stream, st);
}
}  // namespace fp4x
