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
  float* part;           // split-K slots [batch][ksplit][MT][N]
  int* tickets;          // split-K tickets [batch][tiles], zero between calls
  // mixer-down epilogue
  void* out2;
  int lr, hc;
};

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

template <class F, int MT, int RPL, bool XL, class Epi>
__global__ __launch_bounds__(kThreads) void gemv_kernel(GemvLaunch p) {
  extern __shared__ __align__(16) uint16_t lds_x[];
  const int b = blockIdx.z, split = blockIdx.y;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int lpr = p.lpr, lrow = lane & (lpr - 1), slot = lane / lpr, spw = 64 / lpr;
  const int tile_rows = kWaves * spw * RPL;
  const int64_t row_base = (int64_t)blockIdx.x * tile_rows + wave * spw * RPL + slot;
  int64_t rows[RPL];
#pragma unroll
  for (int r = 0; r < RPL; ++r) {
    const int64_t rr = row_base + r * spw;
    rows[r] = rr < p.N ? rr : -1;
  }
  PlaneArgs pa = p.pa;
  pa.w0 += b * p.w0_bstride;
  if (pa.w1) pa.w1 += b * p.w1_bstride;
  pa.s += b * p.s_bstride;
  const int ks = pa.K / p.ksplit, k0 = split * ks, c0 = k0 / F::KPC, cend = c0 + ks / F::KPC;
  const uint16_t* xg = p.x + b * p.x_bstride;

  float acc[RPL][MT];
#pragma unroll
  for (int r = 0; r < RPL; ++r)
#pragma unroll
    for (int m = 0; m < MT; ++m) acc[r][m] = 0.0f;

  for (int jb = 0; jb < p.cpl; jb += kCplBatch) {
    ChunkBatch<F, RPL> cb;
    load_batch<F, RPL>(cb, pa, rows, c0, cend, lrow, lpr, jb, p.cpl);
    if constexpr (XL) {
      if (jb == 0) {
        stage_x<MT>(lds_x, xg, p.x_stride, p.M, k0, ks);
        __syncthreads();
      }
      compute_batch<F, MT, RPL>(cb, (const uint16_t*)lds_x, ks, k0, MT, c0, cend, lrow, lpr, jb, p.cpl, acc);
    } else {
      compute_batch<F, MT, RPL>(cb, xg, (int)p.x_stride, 0, p.M, c0, cend, lrow, lpr, jb, p.cpl, acc);
    }
  }
#pragma unroll
  for (int r = 0; r < RPL; ++r)
#pragma unroll
    for (int m = 0; m < MT; ++m) acc[r][m] = group_allreduce(acc[r][m], lpr);

  if (p.ksplit == 1) {
    if (lrow == 0) {
#pragma unroll
      for (int r = 0; r < RPL; ++r)
        if (rows[r] >= 0)
#pragma unroll
          for (int m = 0; m < MT; ++m)
            if (m < p.M) Epi::apply(p, b, m, rows[r], acc[r][m] * p.gs);
    }
    return;
  }
  // split-K: the tile's partials go through LDS to wave 0, which writes the
  // slice's slot; the last workgroup of the tile sums slots 0..ks-1 in order.
  __shared__ float tile_part[kWaves * 64 * RPL * MT];
  const int nrow = tile_rows;                       // rows of this tile
  if (lrow == 0) {
#pragma unroll
    for (int r = 0; r < RPL; ++r)
#pragma unroll
      for (int m = 0; m < MT; ++m)
        tile_part[m * nrow + wave * spw * RPL + r * spw + slot] = acc[r][m] * p.gs;
  }
  __syncthreads();
  float* part = p.part + (int64_t)b * p.ksplit * MT * p.N;
  const int64_t tile0 = (int64_t)blockIdx.x * tile_rows;
  if (threadIdx.x < 64) {
    for (int i = threadIdx.x; i < p.M * nrow; i += 64) {
      const int m = i / nrow;
      const int64_t row = tile0 + (i - m * nrow);
      if (row < p.N) part[((int64_t)split * MT + m) * p.N + row] = tile_part[i];
    }
  }
  const int tiles = gridDim.x;
  int* ticket = p.tickets + (int64_t)b * tiles + blockIdx.x;
  if (!splitk_arrive(ticket, p.ksplit)) return;
  for (int i = threadIdx.x; i < p.M * nrow; i += blockDim.x) {
    const int m = i / nrow;
    const int64_t row = tile0 + (i - m * nrow);
    if (row >= p.N) continue;
    const float* src = part + (int64_t)m * p.N + row;
    const int64_t sstride = (int64_t)MT * p.N;
    float tot = 0.0f;
    for (int s0 = 0; s0 < p.ksplit; s0 += 8) {
      float v[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] = s0 + j < p.ksplit ? src[(s0 + j) * sstride] : 0.0f;
#pragma unroll
      for (int j = 0; j < 8; ++j)
        if (s0 + j < p.ksplit) tot = s0 + j == 0 ? v[j] : tot + v[j];
    }
    Epi::apply(p, b, m, row, tot);
  }
  if (threadIdx.x == 0) ticket_reset(ticket);
}

// Host-side launch plumbing ---------------------------------------------------
void set_error(const std::string& msg);
int check_launch(const char* what);

template <class F, int MT, int RPL, class Epi>
int launch_gemv_mt(const GemvLaunch& p, int batch, hipStream_t st) {
  const int spw = 64 / p.lpr;
  const int tile_rows = kWaves * spw * RPL;
  const int tiles = (p.N + tile_rows - 1) / tile_rows;
  dim3 grid(tiles, p.ksplit, batch);
  const int ks = p.pa.K / p.ksplit;
  const size_t lds = (size_t)MT * ks * 2;
  if (lds <= (size_t)kLdsXBytes) {
    hipLaunchKernelGGL((gemv_kernel<F, MT, RPL, true, Epi>), grid, dim3(kThreads), lds, st, p);
  } else {
    hipLaunchKernelGGL((gemv_kernel<F, MT, RPL, false, Epi>), grid, dim3(kThreads), 0, st, p);
  }
  return check_launch("gemv");
}

template <class F, class Epi, int RPL = 1>
int launch_gemv(const GemvLaunch& p, int batch, hipStream_t st) {
  switch (p.M <= 4 ? p.M : p.M <= 8 ? 8 : 16) {
    case 1: return launch_gemv_mt<F, 1, RPL, Epi>(p, batch, st);
    case 2: return launch_gemv_mt<F, 2, RPL, Epi>(p, batch, st);
    case 3: return launch_gemv_mt<F, 3, RPL, Epi>(p, batch, st);
    case 4: return launch_gemv_mt<F, 4, RPL, Epi>(p, batch, st);
    case 8: return launch_gemv_mt<F, 8, RPL, Epi>(p, batch, st);
    default: return launch_gemv_mt<F, 16, RPL, Epi>(p, batch, st);
  }
}

inline int mt_of(int M) { return M <= 4 ? M : M <= 8 ? 8 : 16; }

}  // namespace fp4x
