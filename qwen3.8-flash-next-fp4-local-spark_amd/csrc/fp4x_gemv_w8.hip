// Explicit GEMV instantiations (one translation unit per weight format, so
// the library compiles in parallel).
#include "fp4x_mfma.h"
#include "fp4x_stream.h"

namespace fp4x {
template int launch_gemv_mfma<FmtW8<false>, EpiStore>(const GemvLaunch&, int, hipStream_t);
template int launch_gemv_mfma<FmtW8<true>, EpiStore>(const GemvLaunch&, int, hipStream_t);
template bool launch_w8_stream<false>(GemvLaunch, int, hipStream_t);
template bool launch_w8_stream<true>(GemvLaunch, int, hipStream_t);
template bool launch_w8_ktile<false, EpiStore>(GemvLaunch, hipStream_t);
template bool launch_w8_ktile<true, EpiStore>(GemvLaunch, hipStream_t);
bool launch_w8_single_stream_f16(GemvLaunch p, hipStream_t st) { return launch_w8_single_stream<StreamW8H>(p, st); }
bool launch_w8_single_stream_f32(GemvLaunch p, hipStream_t st) { return launch_w8_single_stream<StreamW8F>(p, st); }
}  // namespace fp4x
