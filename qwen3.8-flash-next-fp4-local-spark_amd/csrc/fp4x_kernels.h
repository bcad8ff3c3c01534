// Kernel templates shared by the dense, mixer and head translation units.
#pragma once
#include "fp4x_gemv.h"
#include <string>

namespace fp4x {

struct GemvLaunch {
  const uint16_t* x;     // bf16 activations
  int64_t x_stride;      // elements between rows of x
  int64_t x_bstride;     // elements between batch entries of x
  PlaneArgs pa;
  int64_t w0_bstride, w1_bstride, s_bstride;  // bytes between batch entries
  void* out;
  int out_dtype;
  int64_t out_stride;    // elements between output rows (m)
  int64_t out_bstride;   // elements between batch entries of out
  float gs;              // scale applied to every dot product (NVFP4 global scale)
  const float* rs;       // optional per-row scale (INT2 row-scale variant)
  int M, N, ksplit, lpr, cpl;  // cpl = chunks per lane per K slice
  int J, nb;             // MFMA core: chunks per lane per tile, register batches per tile
  int batch, per_wg;     // MFMA core: batch entries, (entry, tile) items per workgroup
  int xbufs;             // streaming W8 kernel: activation buffers staged in LDS
  uint16_t* smax;        // streaming INT2 head: per-tile maximum order key of each row m (or null)
  int64_t smax_stride;   //   elements between rows m of smax
  float* part;           // split-K slots [batch][ksplit][MT][N]
  int* tickets;          // split-K tickets [batch][tiles], zero between calls
  int tstride = 1;       //   ints between consecutive tickets (the single-launch mixer: one 128-byte line each)
  // mixer-down epilogue
  void* out2;
  int lr, hc;
};

// Reads the launch fields the streaming kernels use in one round of scalar
// loads at kernel entry.  Left to itself the compiler loads the arguments in
// several rounds, each behind a branch or a first use, and every round waits
// out the argument memory's latency before the first weight load can issue.
__device__ __forceinline__ void load_launch_once(const GemvLaunch& p) {
  asm volatile("" ::"s"(p.x), "s"(p.x_stride), "s"(p.x_bstride), "s"(p.pa.w0), "s"(p.pa.w1), "s"(p.pa.s),
               "s"(p.pa.K), "s"(p.w0_bstride), "s"(p.w1_bstride), "s"(p.s_bstride), "s"(p.out), "s"(p.out_dtype),
               "s"(p.out_stride), "s"(p.out_bstride), "s"(p.gs), "s"(p.rs), "s"(p.M), "s"(p.N), "s"(p.batch),
               "s"(p.per_wg), "s"(p.xbufs));
}

// Plain store: out[b][m * out_stride + row] = cast(v)
struct EpiStore {
  __device__ static void apply(const GemvLaunch& p, int b, int m, int64_t row, float v) {
    if (p.rs) v = v * p.rs[row];
    store_out(p.out, b * p.out_bstride + m * p.out_stride + row, p.out_dtype, v);
  }
};

// Mixer bottleneck activation silu(bf16(d / hc)) rounded to bf16, from the
// bf16 down-projection value d (x/fp4x_kernels.py:461-464).
__device__ __forceinline__ uint16_t hc_scaled_silu(float d_bf16, int hc) {
  const float sc = round_bf16(d_bf16 / (float)hc);
  return f32_to_bf16(sc * sigmoid_f32(sc));
}

// Mixer down epilogue: DI = bf16(v); BOT = scaled silu for rows < lr.
struct EpiHcDown {
  __device__ static void apply(const GemvLaunch& p, int, int m, int64_t row, float v) {
    const uint16_t d = f32_to_bf16(v);
    reinterpret_cast<uint16_t*>(p.out)[m * p.out_stride + row] = d;
    if (row < p.lr)
      reinterpret_cast<uint16_t*>(p.out2)[(int64_t)m * p.lr + row] = hc_scaled_silu(bf16_to_f32(d), p.hc);
  }
};

// The same epilogue for the single-launch mixer: BOT is stored device-coherently,
// since other workgroups of the same launch read it.
struct EpiHcDownShared {
  __device__ static void apply(const GemvLaunch& p, int, int m, int64_t row, float v) {
    const uint16_t d = f32_to_bf16(v);
    reinterpret_cast<uint16_t*>(p.out)[m * p.out_stride + row] = d;
    if (row < p.lr)
      __hip_atomic_store(reinterpret_cast<uint16_t*>(p.out2) + (int64_t)m * p.lr + row,
                         hc_scaled_silu(bf16_to_f32(d), p.hc), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
};

// Host-side launch plumbing ---------------------------------------------------
void set_error(const std::string& msg);
int check_launch(const char* what);

// Path switches, read from the environment when first needed and again by
// fp4x_reload_env(), never per launch.  "0" turns a streaming path or the
// single-launch mixer off (the MFMA core or the two-call mixer runs instead):
// FP4X_W8_STREAM, FP4X_INT2_STREAM, FP4X_NV4_STREAM, FP4X_W6_STREAM,
// FP4X_MX8_STREAM, FP4X_HC_MIX, FP4X_ROWS (the few-rows kernel of small
// matrices), FP4X_HC_XCD (the single-launch mixer's XCD-local down
// partials).  FP4X_WAVES_PER_CU (1..64) caps the MFMA
// core's resident waves per CU (0: no cap).  FP4X_HC_SPIN_LIMIT (>= 0)
// bounds the single-launch mixer's flag wait (reads, default 2^22, about a
// second); 0 makes every wait that is not already satisfied give up, which
// lets tests exercise the give-up path from the host.
struct Switches {
  bool w8_stream = true, int2_stream = true, nv4_stream = true, w6_stream = true, mx8_stream = true;
  bool hc_mix = true, rows = true, hc_xcd = true;
  int waves_per_cu = 0;
  int hc_spin_limit = 1 << 22;
};
const Switches& switches();
void reload_switches();

inline int mt_of(int M) { return M <= 4 ? M : M <= 8 ? 8 : 16; }

}  // namespace fp4x
