// Dense decode GEMVs (MXFP8, W8 g64, W6 g32, NVFP4, INT2 coarse head), the
// layer-batched W8 launch, and the dequant kernels, behind a C ABI.
#include "fp4x_mfma.h"
#include "fp4x_rows.h"
#include "../../include/fp4x.h"
#include <cstdio>
#include <cstdlib>

namespace fp4x {

// GEMV launches are instantiated in the fp4x_gemv_*.hip translation units.
extern template int launch_gemv_mfma<FmtBF16, EpiStore>(const GemvLaunch&, int, hipStream_t);
extern template int launch_gemv_mfma<FmtMX8, EpiStore>(const GemvLaunch&, int, hipStream_t);
extern template int launch_gemv_mfma<FmtW8<false>, EpiStore>(const GemvLaunch&, int, hipStream_t);
extern template int launch_gemv_mfma<FmtW8<true>, EpiStore>(const GemvLaunch&, int, hipStream_t);
template <bool F16S> bool launch_w8_stream(GemvLaunch p, int batch, hipStream_t st);
extern template bool launch_w8_stream<false>(GemvLaunch, int, hipStream_t);
extern template bool launch_w8_stream<true>(GemvLaunch, int, hipStream_t);
bool launch_int2_stream_f16(GemvLaunch p, hipStream_t st);
bool launch_int2_stream_e4m3(GemvLaunch p, hipStream_t st);
bool launch_nv4_stream_entry(GemvLaunch p, hipStream_t st);
bool launch_w6_stream_entry(GemvLaunch p, hipStream_t st);
bool launch_mx8_stream_entry(GemvLaunch p, hipStream_t st);
bool launch_nv4_stream_one_entry(GemvLaunch p, hipStream_t st);
bool launch_w6_stream_one_entry(GemvLaunch p, hipStream_t st);
bool launch_w6_stream_tile_entry(GemvLaunch p, hipStream_t st);
bool launch_nv4_stream_tile_entry(GemvLaunch p, hipStream_t st);
bool launch_mx8_stream_tile_entry(GemvLaunch p, hipStream_t st);
bool launch_w8_single_stream_f16(GemvLaunch p, hipStream_t st);
bool launch_w8_single_stream_f32(GemvLaunch p, hipStream_t st);
int topk_check(const void* logits, int dtype, int64_t stride, int M, int V, int C, void* workspace,
               int64_t ws_bytes);
int topk_launch(const void* lg, int dtype, int64_t stride, int M, int V, int C, int64_t* idx_out, uint16_t* smax,
                bool have_smax, bool set_only, hipStream_t st);
int topk_slice_len(int V);
int64_t topk_smax_stride(int V);
template <bool F16S, class Epi> bool launch_w8_ktile(GemvLaunch p, hipStream_t st);
extern template bool launch_w8_ktile<false, EpiStore>(GemvLaunch, hipStream_t);
extern template bool launch_w8_ktile<true, EpiStore>(GemvLaunch, hipStream_t);
extern template int launch_gemv_mfma<FmtW6, EpiStore>(const GemvLaunch&, int, hipStream_t);
extern template int launch_gemv_mfma<FmtNV4, EpiStore>(const GemvLaunch&, int, hipStream_t);
extern template int launch_gemv_mfma<FmtInt2<false, 16>, EpiStore>(const GemvLaunch&, int, hipStream_t);
extern template int launch_gemv_mfma<FmtInt2<false, 32>, EpiStore>(const GemvLaunch&, int, hipStream_t);
extern template int launch_gemv_mfma<FmtInt2<false, 0>, EpiStore>(const GemvLaunch&, int, hipStream_t);
extern template int launch_gemv_mfma<FmtInt2<true, 16>, EpiStore>(const GemvLaunch&, int, hipStream_t);
extern template int launch_gemv_mfma<FmtInt2<true, 32>, EpiStore>(const GemvLaunch&, int, hipStream_t);
extern template int launch_gemv_mfma<FmtInt2<true, 0>, EpiStore>(const GemvLaunch&, int, hipStream_t);

static thread_local std::string g_err;

int device_cus() {
  static int cus = 0;
  if (!cus) {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) == hipSuccess && hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0)
      cus = n;
    else
      cus = 256;
  }
  return cus;
}

static Switches g_switches;
static bool g_switches_read = false;

void reload_switches() {
  auto on = [](const char* name) {
    const char* e = getenv(name);
    return !(e && e[0] == '0');
  };
  Switches w;
  w.w8_stream = on("FP4X_W8_STREAM");
  w.int2_stream = on("FP4X_INT2_STREAM");
  w.nv4_stream = on("FP4X_NV4_STREAM");
  w.w6_stream = on("FP4X_W6_STREAM");
  w.mx8_stream = on("FP4X_MX8_STREAM");
  w.hc_mix = on("FP4X_HC_MIX");
  w.rows = on("FP4X_ROWS");
  w.hc_xcd = on("FP4X_HC_XCD");
  const char* e = getenv("FP4X_WAVES_PER_CU");
  const int v = e ? atoi(e) : 0;
  w.waves_per_cu = v >= 1 && v <= 64 ? v : 0;
  const char* sp = getenv("FP4X_HC_SPIN_LIMIT");
  const long spin = sp ? atol(sp) : -1;
  w.hc_spin_limit = spin >= 0 && spin <= (1 << 22) ? (int)spin : 1 << 22;
  g_switches = w;
  g_switches_read = true;
}

const Switches& switches() {
  if (!g_switches_read) reload_switches();
  return g_switches;
}

int waves_per_cu_cap() { return switches().waves_per_cu; }
void set_error(const std::string& msg) { g_err = msg; }

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error(std::string(what) + ": launch failed: " + hipGetErrorString(e));
    return FP4X_ERR_LAUNCH;
  }
  return FP4X_OK;
}

static int fail(int code, const char* fmt, long long a = 0, long long b = 0, long long c = 0) {
  char buf[256];
  snprintf(buf, sizeof buf, fmt, a, b, c);
  set_error(buf);
  return code;
}

static bool aligned(const void* p, int n) { return (reinterpret_cast<uintptr_t>(p) & (n - 1)) == 0; }

struct FmtInfo {
  int kpc;      // weights per 16-byte chunk
  int kmult;    // K must be a multiple of this
};

static FmtInfo fmt_info(int fmt) {
  switch (fmt) {
    case FP4X_FMT_MX8: return {16, 32};
    case FP4X_FMT_W8_F32: case FP4X_FMT_W8_F16: return {16, 64};
    case FP4X_FMT_W6: return {32, 32};
    case FP4X_FMT_NV4: return {32, 32};
    case FP4X_FMT_INT2_F16: case FP4X_FMT_INT2_E4M3: return {64, 64};
    case FP4X_FMT_BF16: return {16, 16};
    default: return {0, 0};
  }
}

// Shared validation of shapes, split and activation layout.
static int validate(int fmt, const void* x, int64_t x_stride, int M, int N, int K, int ksplit,
                    const float* part, const int* tickets) {
  const FmtInfo fi = fmt_info(fmt);
  if (!fi.kpc) return fail(FP4X_ERR_ARG, "unknown weight format %lld", fmt);
  if (M < 0 || M > 16) return fail(FP4X_ERR_ARG, "M=%lld outside [0, 16]", M);
  if (N < 0 || K <= 0) return fail(FP4X_ERR_ARG, "bad shape N=%lld K=%lld", N, K);
  if (K % fi.kmult) return fail(FP4X_ERR_ARG, "K=%lld must be a multiple of %lld", K, fi.kmult);
  if (ksplit < 1 || ksplit > 64 || K % ksplit || (K / ksplit) % fi.kpc)
    return fail(FP4X_ERR_ARG, "ksplit=%lld must divide K=%lld into multiples of %lld", ksplit, K, fi.kpc);
  if (ksplit > 1 && (!part || !tickets)) return fail(FP4X_ERR_ARG, "ksplit=%lld needs split-K scratch", ksplit);
  if (M > 0 && (!aligned(x, 16) || x_stride % 8 || x_stride < K))
    return fail(FP4X_ERR_ARG, "x must be 16-byte aligned with a row stride (%lld) that is a multiple of 8 and >= K (%lld)",
                x_stride, K);
  return FP4X_OK;
}

static GemvLaunch base_launch(int fmt, const void* x, int64_t x_stride, void* out, int out_dtype, int64_t out_stride,
                              int M, int N, int K, int ksplit, float* part, int* tickets) {
  GemvLaunch p{};
  p.x = static_cast<const uint16_t*>(x);
  p.x_stride = x_stride;
  p.out = out;
  p.out_dtype = out_dtype;
  p.out_stride = out_stride;
  p.gs = 1.0f;
  p.M = M;
  p.N = N;
  p.ksplit = ksplit;
  const int chunks = (K / ksplit) / fmt_info(fmt).kpc;
  p.lpr = layout_lpr(chunks);
  p.cpl = (chunks + p.lpr - 1) / p.lpr;
  p.part = part;
  p.tickets = tickets;
  p.pa.K = K;
  p.pa.G = 0;
  return p;
}

}  // namespace fp4x

using namespace fp4x;

extern "C" {

const char* fp4x_last_error(void) { return g_err.c_str(); }

int fp4x_abi_version(void) { return FP4X_ABI_VERSION; }

int fp4x_layout(int fmt, int k_slice, int* lpr, int* cpl) {
  const FmtInfo fi = fmt_info(fmt);
  if (!fi.kpc || k_slice <= 0 || k_slice % fi.kpc) return fail(FP4X_ERR_ARG, "bad layout query fmt=%lld k=%lld", fmt, k_slice);
  const int chunks = k_slice / fi.kpc;
  *lpr = layout_lpr(chunks);
  *cpl = (chunks + *lpr - 1) / *lpr;
  return FP4X_OK;
}

int fp4x_splitk_sizes(int fmt, int M, int N, int K, int ksplit, int batch, int64_t* part_floats, int64_t* n_tickets) {
  const FmtInfo fi = fmt_info(fmt);
  if (!fi.kpc || ksplit < 1 || K % ksplit || (K / ksplit) % fi.kpc) return fail(FP4X_ERR_ARG, "bad split-K query");
  (void)M;
  *part_floats = (int64_t)batch * ksplit * 16 * N;     // one 16-row slot tile per K slice
  *n_tickets = (int64_t)batch * ((N + 15) / 16);       // one ticket per 16-row tile
  return FP4X_OK;
}

int fp4x_mx8_linear(const void* x, int64_t x_stride, const void* w, const void* s, void* out, int out_dtype,
                    int M, int N, int K, int ksplit, float* part, int* tickets, void* stream) {
  int rc = validate(FP4X_FMT_MX8, x, x_stride, M, N, K, ksplit, part, tickets);
  if (rc) return rc;
  if (!aligned(w, 16)) return fail(FP4X_ERR_ARG, "mx8: weight rows must be 16-byte aligned");
  if (M == 0 || N == 0) return FP4X_OK;
  GemvLaunch p = base_launch(FP4X_FMT_MX8, x, x_stride, out, out_dtype, N, M, N, K, ksplit, part, tickets);
  p.pa.w0 = static_cast<const uint8_t*>(w);
  p.pa.s = static_cast<const uint8_t*>(s);
  if (launch_rows_wide<FmtMX8>(p, (hipStream_t)stream)) return check_launch("mx8_rows");    // 16-20 rows per CU, M = 1
  if (launch_mx8_stream_entry(p, (hipStream_t)stream)) return check_launch("mx8_stream");   // many tiles
  if (launch_rows_gemv<FmtMX8>(p, 1, (hipStream_t)stream)) return check_launch("mx8_rows");  // fewer rows
  if (launch_mx8_stream_tile_entry(p, (hipStream_t)stream)) return check_launch("mx8_stream"); // 1/2-1 tile per CU
  return launch_gemv_mfma<FmtMX8, EpiStore>(p, 1, (hipStream_t)stream);
}

int fp4x_bf16_linear(const void* x, int64_t x_stride, const void* w, void* out, int out_dtype, int M, int N, int K,
                     int ksplit, float* part, int* tickets, void* stream) {
  int rc = validate(FP4X_FMT_BF16, x, x_stride, M, N, K, ksplit, part, tickets);
  if (rc) return rc;
  if (!aligned(w, 16)) return fail(FP4X_ERR_ARG, "bf16: weight rows must be 16-byte aligned");
  if (M == 0 || N == 0) return FP4X_OK;
  GemvLaunch p = base_launch(FP4X_FMT_BF16, x, x_stride, out, out_dtype, N, M, N, K, ksplit, part, tickets);
  p.pa.w0 = static_cast<const uint8_t*>(w);
  if (launch_rows_gemv<FmtBF16>(p, 1, (hipStream_t)stream)) return check_launch("bf16_rows");
  return launch_gemv_mfma<FmtBF16, EpiStore>(p, 1, (hipStream_t)stream);
}

int fp4x_w8_linear_layers(const void* x, int64_t x_stride, int64_t x_lstride, const void* q, int64_t q_lstride,
                          const void* s, int s_dtype, int64_t s_lstride, void* out, int out_dtype, int64_t out_lstride,
                          int layers, int M, int N, int K, int ksplit, float* part, int* tickets, void* stream) {
  const int fmt = s_dtype == FP4X_DT_F16 ? FP4X_FMT_W8_F16 : FP4X_FMT_W8_F32;
  if (s_dtype != FP4X_DT_F16 && s_dtype != FP4X_DT_F32) return fail(FP4X_ERR_ARG, "w8: scale dtype %lld", s_dtype);
  int rc = validate(fmt, x, x_stride, M, N, K, ksplit, part, tickets);
  if (rc) return rc;
  if (layers < 0) return fail(FP4X_ERR_ARG, "w8: layers=%lld", layers);
  if (!aligned(q, 16) || (layers > 1 && (q_lstride % 16 || x_lstride % 8)))
    return fail(FP4X_ERR_ARG, "w8: weight (and per-layer strides) must be 16-byte aligned");
  if (!aligned(s, s_dtype == FP4X_DT_F16 ? 2 : 4)) return fail(FP4X_ERR_ARG, "w8: misaligned scales");
  if (M == 0 || N == 0 || layers == 0) return FP4X_OK;
  GemvLaunch p = base_launch(fmt, x, x_stride, out, out_dtype, N, M, N, K, ksplit, part, tickets);
  p.x_bstride = x_lstride;
  p.pa.w0 = static_cast<const uint8_t*>(q);
  p.pa.s = static_cast<const uint8_t*>(s);
  p.w0_bstride = q_lstride;
  p.s_bstride = s_lstride * (s_dtype == FP4X_DT_F16 ? 2 : 4);
  p.out_bstride = out_lstride;
  // long runs of tiles (layer-batched gates) stream through LDS; split-K calls of
  // few tiles spread each tile's K over several workgroups (or over the waves
  // of one workgroup), the mixer's down projection taking the same path; other
  // matrices of few rows (a router gate) or of short rows take the few-rows
  // kernels; other single matrices of at least half a tile per CU stream
  // through LDS; other shapes use the MFMA core
  hipStream_t st = (hipStream_t)stream;
  if (fmt == FP4X_FMT_W8_F16) {
    if (launch_w8_stream<true>(p, layers, st)) return check_launch("w8_stream");
    if (layers == 1 && launch_w8_ktile<true, EpiStore>(p, st)) return check_launch("w8_ktile");
    if (launch_rows_gemv<FmtW8<true>>(p, layers, st)) return check_launch("w8_rows");   // few rows (a router gate)
    if (layers == 1 && launch_w8_single_stream_f16(p, st)) return check_launch("w8_single_stream");
    return launch_gemv_mfma<FmtW8<true>, EpiStore>(p, layers, st);
  }
  if (launch_w8_stream<false>(p, layers, st)) return check_launch("w8_stream");
  if (layers == 1 && launch_w8_ktile<false, EpiStore>(p, st)) return check_launch("w8_ktile");
  if (launch_rows_gemv<FmtW8<false>>(p, layers, st)) return check_launch("w8_rows");
  if (layers == 1 && launch_w8_single_stream_f32(p, st)) return check_launch("w8_single_stream");
  return launch_gemv_mfma<FmtW8<false>, EpiStore>(p, layers, st);
}

int fp4x_w8_linear(const void* x, int64_t x_stride, const void* q, const void* s, int s_dtype, void* out, int out_dtype,
                   int M, int N, int K, int ksplit, float* part, int* tickets, void* stream) {
  return fp4x_w8_linear_layers(x, x_stride, 0, q, 0, s, s_dtype, 0, out, out_dtype, 0, 1, M, N, K, ksplit, part,
                               tickets, stream);
}

int fp4x_w6_linear(const void* x, int64_t x_stride, const void* L, const void* H, const void* S, void* out,
                   int out_dtype, int M, int N, int K, int ksplit, float* part, int* tickets, void* stream) {
  int rc = validate(FP4X_FMT_W6, x, x_stride, M, N, K, ksplit, part, tickets);
  if (rc) return rc;
  if (!aligned(L, 16) || !aligned(H, 8) || !aligned(S, 2)) return fail(FP4X_ERR_ARG, "w6: misaligned planes");
  if (M == 0 || N == 0) return FP4X_OK;
  GemvLaunch p = base_launch(FP4X_FMT_W6, x, x_stride, out, out_dtype, N, M, N, K, ksplit, part, tickets);
  p.pa.w0 = static_cast<const uint8_t*>(L);
  p.pa.w1 = static_cast<const uint8_t*>(H);
  p.pa.s = static_cast<const uint8_t*>(S);
  if (launch_rows_wide<FmtW6>(p, (hipStream_t)stream)) return check_launch("w6_rows");       // many rows, M = 1
  if (launch_w6_stream_entry(p, (hipStream_t)stream)) return check_launch("w6_stream");     // many tiles
  if (launch_rows_gemv<FmtW6>(p, 1, (hipStream_t)stream)) return check_launch("w6_rows");    // fewer rows
  if (launch_w6_stream_one_entry(p, (hipStream_t)stream)) return check_launch("w6_stream");  // 1-2 tiles per CU
  if (launch_w6_stream_tile_entry(p, (hipStream_t)stream)) return check_launch("w6_stream"); // 1/2-1 tile per CU
  return launch_gemv_mfma<FmtW6, EpiStore>(p, 1, (hipStream_t)stream);
}

int fp4x_nv4_linear(const void* x, int64_t x_stride, const void* P, const void* S, float gs, void* out, int out_dtype,
                    int M, int N, int K, int ksplit, float* part, int* tickets, void* stream) {
  int rc = validate(FP4X_FMT_NV4, x, x_stride, M, N, K, ksplit, part, tickets);
  if (rc) return rc;
  if (!aligned(P, 16) || !aligned(S, 2)) return fail(FP4X_ERR_ARG, "nv4: misaligned planes");
  if (M == 0 || N == 0) return FP4X_OK;
  GemvLaunch p = base_launch(FP4X_FMT_NV4, x, x_stride, out, out_dtype, N, M, N, K, ksplit, part, tickets);
  p.pa.w0 = static_cast<const uint8_t*>(P);
  p.pa.s = static_cast<const uint8_t*>(S);
  p.gs = gs;
  if (launch_nv4_stream_entry(p, (hipStream_t)stream)) return check_launch("nv4_stream");   // many tiles
  if (launch_rows_gemv<FmtNV4>(p, 1, (hipStream_t)stream)) return check_launch("nv4_rows");  // fewer rows
  if (launch_nv4_stream_one_entry(p, (hipStream_t)stream)) return check_launch("nv4_stream"); // 1-2 tiles per CU
  if (launch_nv4_stream_tile_entry(p, (hipStream_t)stream)) return check_launch("nv4_stream"); // 1/2-1 tile per CU
  return launch_gemv_mfma<FmtNV4, EpiStore>(p, 1, (hipStream_t)stream);
}

}  // extern "C"

namespace fp4x {
// INT2 coarse logits [M, N] at out (row stride out_stride); with smax set, the
// streaming kernel also writes the 16-element slice maxima of the stored
// logits and the function returns 1 (0 when another kernel ran and smax was
// not written), or a negative error.
static int int2_coarse(const void* x, int64_t x_stride, const void* P, const void* S, int s_fmt, const float* rs,
                       void* out, int out_dtype, int64_t out_stride, int M, int N, int K, int G, uint16_t* smax,
                       int64_t smax_stride, hipStream_t st) {
  const int fmt = s_fmt == FP4X_DT_E4M3 ? FP4X_FMT_INT2_E4M3 : FP4X_FMT_INT2_F16;
  if (s_fmt != FP4X_DT_E4M3 && s_fmt != FP4X_DT_F16) return fail(FP4X_ERR_ARG, "int2: scale format %lld", s_fmt);
  int rc = validate(fmt, x, x_stride, M, N, K, 1, nullptr, nullptr);
  if (rc) return rc;
  if (!(G == 16 || G == 32 || (G >= 64 && G % 64 == 0)) || K % G)
    return fail(FP4X_ERR_ARG, "int2: group size G=%lld must be 16, 32 or a multiple of 64 dividing K=%lld", G, K);
  if (!aligned(P, 16) || !aligned(S, s_fmt == FP4X_DT_E4M3 ? (G == 16 ? 4 : 1) : (G == 16 ? 8 : 2)))
    return fail(FP4X_ERR_ARG, "int2: misaligned planes");
  if (M == 0 || N == 0) return 0;
  GemvLaunch p = base_launch(fmt, x, x_stride, out, out_dtype, out_stride, M, N, K, 1, nullptr, nullptr);
  p.pa.w0 = static_cast<const uint8_t*>(P);
  p.pa.s = static_cast<const uint8_t*>(S);
  p.pa.G = G;
  p.rs = rs;
  p.smax = smax;
  p.smax_stride = smax_stride;
  if (fmt == FP4X_FMT_INT2_F16) {
    if ((G == 16 || G == 32) && launch_int2_stream_f16(p, st)) {   // large heads
      rc = check_launch("int2_stream");
      return rc ? rc : (smax ? 1 : 0);
    }
    p.smax = nullptr;
    return G == 16   ? launch_gemv_mfma<FmtInt2<false, 16>, EpiStore>(p, 1, st)
           : G == 32 ? launch_gemv_mfma<FmtInt2<false, 32>, EpiStore>(p, 1, st)
                     : launch_gemv_mfma<FmtInt2<false, 0>, EpiStore>(p, 1, st);
  }
  if (G == 16 && launch_int2_stream_e4m3(p, st)) {     // large heads
    rc = check_launch("int2_stream");
    return rc ? rc : (smax ? 1 : 0);
  }
  p.smax = nullptr;
  if (G == 16) return launch_gemv_mfma<FmtInt2<true, 16>, EpiStore>(p, 1, st);
  if (G == 32) return launch_gemv_mfma<FmtInt2<true, 32>, EpiStore>(p, 1, st);
  return launch_gemv_mfma<FmtInt2<true, 0>, EpiStore>(p, 1, st);
}
}  // namespace fp4x

extern "C" {

int fp4x_int2_logits(const void* x, int64_t x_stride, const void* P, const void* S, int s_fmt, const float* rs,
                     void* out, int out_dtype, int M, int N, int K, int G, void* stream) {
  const int rc = int2_coarse(x, x_stride, P, S, s_fmt, rs, out, out_dtype, N, M, N, K, G, nullptr, 0,
                             (hipStream_t)stream);
  return rc < 0 ? rc : FP4X_OK;
}

int fp4x_int2_topk(const void* x, int64_t x_stride, const void* P, const void* S, int s_fmt, const float* rs,
                   void* coarse, int coarse_dtype, int64_t coarse_stride, int M, int N, int K, int G, int C,
                   int64_t* idx_out, int set_only, void* workspace, int64_t ws_bytes, void* stream) {
  int rc = topk_check(coarse, coarse_dtype, coarse_stride, M, N, C, workspace, ws_bytes);
  if (rc) return rc;
  if (M == 0) return FP4X_OK;
  hipStream_t st = (hipStream_t)stream;
  uint16_t* smax = static_cast<uint16_t*>(workspace);
  // the streaming kernel's per-tile maxima (of the bf16-rounded logits, also
  // for fp32 coarse logits) are the top-k's slices when they are 16 elements
  const bool fuse = topk_slice_len(N) == 16;
  rc = int2_coarse(x, x_stride, P, S, s_fmt, rs, coarse, coarse_dtype, coarse_stride, M, N, K, G,
                   fuse ? smax : nullptr, topk_smax_stride(N), st);
  if (rc < 0) return rc;
  return topk_launch(coarse, coarse_dtype, coarse_stride, M, N, C, idx_out, smax, rc == 1, set_only != 0, st);
}

}  // extern "C"

// ----------------------------------------------------------------------------
// Dequant kernels: the bf16 operand each GEMV feeds to its dot (same device
// decode functions), and the fp32 MXFP8 dequant (x/fp4x_kernels.py:261-267).
namespace fp4x {

template <class F>
__global__ __launch_bounds__(256) void dequant_bf16_kernel(PlaneArgs pa, int N, uint16_t* out) {
  const int cpr = pa.K / F::KPC;
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= (int64_t)N * cpr) return;
  const int64_t row = t / cpr;
  const int c = (int)(t - row * cpr);
  const typename F::Chunk ch = F::load(pa, row, c);
#pragma unroll
  for (int sub = 0; sub < F::SUB; ++sub) {
    uint32_t w[8];
    F::deq16(ch, sub, w);
    uint4* o = reinterpret_cast<uint4*>(out + row * pa.K + c * F::KPC + sub * 16);
    o[0] = make_uint4(w[0], w[1], w[2], w[3]);
    o[1] = make_uint4(w[4], w[5], w[6], w[7]);
  }
}

__global__ __launch_bounds__(256) void mx8_dequant_f32_kernel(const uint8_t* w, const uint8_t* s, int N, int K,
                                                              float* out) {
  const int cpr = K / 16;
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= (int64_t)N * cpr) return;
  const int64_t row = t / cpr;
  const int c = (int)(t - row * cpr);
  const uint4 q = ld_u128(w + row * K + c * 16);
  const float sc = e8m0_to_f32(ld_u8(s + row * (K / 32) + (c >> 1)));
  const uint32_t d[4] = {q.x, q.y, q.z, q.w};
  float4* o = reinterpret_cast<float4*>(out + row * K + c * 16);
  const bool inf_scale = ld_u8(s + row * (K / 32) + (c >> 1)) == 255u;   // exp2(128) = +inf (see FmtMX8)
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f32x2_t a = fp8x2_to_f32x2<false>(d[i], sc), b = fp8x2_to_f32x2<true>(d[i], sc);
    if (inf_scale) {
      const float v[4] = {__uint_as_float(FmtMX8::inf_bf16(d[i] & 0xffu) << 16),
                          __uint_as_float(FmtMX8::inf_bf16((d[i] >> 8) & 0xffu) << 16),
                          __uint_as_float(FmtMX8::inf_bf16((d[i] >> 16) & 0xffu) << 16),
                          __uint_as_float(FmtMX8::inf_bf16(d[i] >> 24) << 16)};
      a = f32x2_t{v[0], v[1]};
      b = f32x2_t{v[2], v[3]};
    }
    o[i] = make_float4(a.x, a.y, b.x, b.y);
  }
}

}  // namespace fp4x

extern "C" {

int fp4x_reload_env(void) {
  reload_switches();
  return FP4X_OK;
}

int fp4x_dequant_bf16(int fmt, const void* w0, const void* w1, const void* s, int N, int K, int G, void* out,
                      void* stream) {
  const FmtInfo fi = fmt_info(fmt);
  if (!fi.kpc || N < 0 || K <= 0 || K % fi.kmult) return fail(FP4X_ERR_ARG, "dequant: bad format/shape");
  if ((fmt == FP4X_FMT_INT2_F16 || fmt == FP4X_FMT_INT2_E4M3) &&
      (!(G == 16 || G == 32 || (G >= 64 && G % 64 == 0)) || K % G))
    return fail(FP4X_ERR_ARG, "dequant: bad INT2 group size %lld", G);
  if (!aligned(w0, 16) || !aligned(out, 16)) return fail(FP4X_ERR_ARG, "dequant: misaligned buffers");
  if (N == 0) return FP4X_OK;
  PlaneArgs pa{static_cast<const uint8_t*>(w0), static_cast<const uint8_t*>(w1), static_cast<const uint8_t*>(s), K, G};
  const int64_t threads = (int64_t)N * (K / fi.kpc);
  dim3 grid((unsigned)((threads + 255) / 256));
  hipStream_t st = (hipStream_t)stream;
  uint16_t* o = static_cast<uint16_t*>(out);
  switch (fmt) {
    case FP4X_FMT_MX8: hipLaunchKernelGGL(dequant_bf16_kernel<FmtMX8>, grid, dim3(256), 0, st, pa, N, o); break;
    case FP4X_FMT_W8_F32: hipLaunchKernelGGL(dequant_bf16_kernel<FmtW8<false>>, grid, dim3(256), 0, st, pa, N, o); break;
    case FP4X_FMT_W8_F16: hipLaunchKernelGGL(dequant_bf16_kernel<FmtW8<true>>, grid, dim3(256), 0, st, pa, N, o); break;
    case FP4X_FMT_W6: hipLaunchKernelGGL(dequant_bf16_kernel<FmtW6>, grid, dim3(256), 0, st, pa, N, o); break;
    case FP4X_FMT_NV4: hipLaunchKernelGGL(dequant_bf16_kernel<FmtNV4>, grid, dim3(256), 0, st, pa, N, o); break;
    case FP4X_FMT_BF16: hipLaunchKernelGGL(dequant_bf16_kernel<FmtBF16>, grid, dim3(256), 0, st, pa, N, o); break;
    case FP4X_FMT_INT2_F16:
      if (G == 16) hipLaunchKernelGGL((dequant_bf16_kernel<FmtInt2<false, 16>>), grid, dim3(256), 0, st, pa, N, o);
      else if (G == 32) hipLaunchKernelGGL((dequant_bf16_kernel<FmtInt2<false, 32>>), grid, dim3(256), 0, st, pa, N, o);
      else hipLaunchKernelGGL((dequant_bf16_kernel<FmtInt2<false, 0>>), grid, dim3(256), 0, st, pa, N, o);
      break;
    default:
      if (G == 16) hipLaunchKernelGGL((dequant_bf16_kernel<FmtInt2<true, 16>>), grid, dim3(256), 0, st, pa, N, o);
      else if (G == 32) hipLaunchKernelGGL((dequant_bf16_kernel<FmtInt2<true, 32>>), grid, dim3(256), 0, st, pa, N, o);
      else hipLaunchKernelGGL((dequant_bf16_kernel<FmtInt2<true, 0>>), grid, dim3(256), 0, st, pa, N, o);
      break;
  }
  return check_launch("dequant_bf16");
}

int fp4x_mx8_dequant(const void* w, const void* s, int N, int K, float* out, void* stream) {
  if (N < 0 || K <= 0 || K % 32) return fail(FP4X_ERR_ARG, "mx8_dequant: K=%lld must be a multiple of 32", K);
  if (!aligned(w, 16) || !aligned(out, 16)) return fail(FP4X_ERR_ARG, "mx8_dequant: misaligned buffers");
  if (N == 0) return FP4X_OK;
  const int64_t threads = (int64_t)N * (K / 16);
  hipLaunchKernelGGL(mx8_dequant_f32_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0,
                     (hipStream_t)stream, static_cast<const uint8_t*>(w), static_cast<const uint8_t*>(s), N, K, out);
  return check_launch("mx8_dequant");
}

}  // extern "C"
