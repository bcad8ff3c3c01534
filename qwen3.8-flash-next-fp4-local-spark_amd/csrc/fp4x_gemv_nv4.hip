// Explicit GEMV instantiations (one translation unit per weight format, so
// the library compiles in parallel).
#include "fp4x_stream.h"

namespace fp4x {
template int launch_gemv_mfma<FmtNV4, EpiStore>(const GemvLaunch&, int, hipStream_t);
bool launch_nv4_stream_entry(GemvLaunch p, hipStream_t st) { return launch_nv4_stream(p, st); }
bool launch_nv4_stream_tile_entry(GemvLaunch p, hipStream_t st) {
  return launch_stream_tile_per_wg<StreamNV4>(p, switches().nv4_stream, st);
}
bool launch_nv4_stream_one_entry(GemvLaunch p, hipStream_t st) { return launch_nv4_stream_one(p, st); }
}  // namespace fp4x
