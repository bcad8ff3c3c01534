// MFMA GEMV core for gfx950: y[m, n] = sum_k x[m, k] * w[n, k], M <= 16.
//
// One workgroup owns a tile of 16 weight rows (the n dimension of
// v_mfma_f32_16x16x32_bf16; the M <= 16 activation rows pad the m dimension)
// and loops over tiles grid-stride.  Its KW waves split the K slice: lane
// (n = lane & 15, g = lane >> 4) of wave w streams 16-byte chunks
// c = w*4 + g + j*4*KW of row n (four lane groups read four consecutive
// chunks of each row), dequantizes them in registers to the bf16 operand and
// feeds 8 k-values per MFMA step; the activation fragment of lane (m, g)
// carries x[m] at the same k.  The KW partial 16x16 tiles are summed in wave
// order through LDS.
//
// Split-K (ksplit > 1) and the epilogue functors are those of the VALU core
// (fp4x_kernels.h): one slot per K slice, the last-arriving workgroup sums
// the slots in slice order.
#pragma once
#include "fp4x_kernels.h"

namespace fp4x {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int kJ = 4;   // chunks per lane held in registers per batch

// Waves per tile for a K slice of `chunks` 16-byte chunks: at most four
// chunks per lane where 8 waves allow it.
__host__ __device__ inline int mfma_kw(int chunks) {
  int want = (chunks + 15) / 16, kw = 1;
  while (kw < want && kw < 8) kw <<= 1;
  return kw;
}

__device__ __forceinline__ f32x4_t mfma16(uint4 a, uint4 b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b), c,
                                                 0, 0, 0);
}

template <class F>
struct MfmaBatch {
  typename F::Chunk ch[kJ];
};

// Chunk c of this lane for batch slot j: c = c0 + cw + j * cstep.
template <class F>
__device__ __forceinline__ void mfma_load(MfmaBatch<F>& b, const PlaneArgs& a, int64_t row, int c0, int cend, int cw,
                                          int cstep, int jb, int J) {
  const typename F::Row r = F::row(a, row < 0 ? 0 : row);
#pragma unroll
  for (int j = 0; j < kJ; ++j) {
    const int c = c0 + cw + (jb + j) * cstep;
    if (jb + j < J && row >= 0 && c < cend) b.ch[j] = F::load_row(r, c);
    else b.ch[j] = F::zero();
  }
}

// MFMA steps over one batch.  xs: x[m][k] at xs[m * xstride + k - kx0] for
// m < M (LDS or global); lanes with m >= M feed zeros.
template <class F, class XPtr>
__device__ __forceinline__ void mfma_compute(const MfmaBatch<F>& b, XPtr xs, int xstride, int kx0, int M, bool wrow,
                                             int c0, int cend, int cw, int cstep, int jb, int J, f32x4_t& acc) {
  const int lane = threadIdx.x & 63;
  const int xm = lane & 15;
#pragma unroll
  for (int j = 0; j < kJ; ++j) {
    if (jb + j >= J) break;
    const int c = c0 + cw + (jb + j) * cstep;
    const bool live = c < cend;                     // lane group's chunk exists (uniform per 16 lanes)
#pragma unroll
    for (int sub = 0; sub < F::SUB; ++sub) {
      uint32_t w[8];
      F::deq16(b.ch[j], sub, w);
      const int k = c * F::KPC + sub * 16;
      uint4 xa = make_uint4(0, 0, 0, 0), xb = xa;
      if (live && xm < M) {
        const uint4* xp = reinterpret_cast<const uint4*>(xs + (int64_t)xm * xstride + (k - kx0));
        xa = xp[0];
        xb = xp[1];
      }
      uint4 wa = make_uint4(w[0], w[1], w[2], w[3]), wb = make_uint4(w[4], w[5], w[6], w[7]);
      if (!live || !wrow) { wa = make_uint4(0, 0, 0, 0); wb = wa; }
      acc = mfma16(xa, wa, acc);
      acc = mfma16(xb, wb, acc);
    }
  }
}

// Sum the KW waves' 16x16 tiles in wave order; the result is valid in wave 0.
template <int KWMAX>
__device__ __forceinline__ f32x4_t mfma_wave_reduce(f32x4_t acc, int KW, float* red) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (KW == 1) return acc;
  if (wave > 0) reinterpret_cast<f32x4_t*>(red)[(wave - 1) * 64 + lane] = acc;
  __syncthreads();
  if (wave == 0) {
    for (int w = 1; w < KW; ++w) {
      const f32x4_t o = reinterpret_cast<const f32x4_t*>(red)[(w - 1) * 64 + lane];
      acc[0] += o[0]; acc[1] += o[1]; acc[2] += o[2]; acc[3] += o[3];
    }
  }
  __syncthreads();
  return acc;
}

// LDS layout: [x: M x ks bf16 (XL only)] [red: (KW-1) x 64 x 4 fp32] [slot tile: 16 x 16 fp32]
__host__ __device__ inline size_t mfma_lds_bytes(int M, int ks, int KW, bool xl) {
  size_t x = xl ? (size_t)M * ks * 2 : 0;
  x = (x + 15) & ~(size_t)15;
  return x + (size_t)(KW > 1 ? KW - 1 : 0) * 64 * 16 + 16 * 16 * 4;
}

template <class F, bool XL, class Epi>
__global__ __launch_bounds__(512) void gemv_mfma_kernel(GemvLaunch p) {
  extern __shared__ __align__(16) uint16_t lds[];
  const int b = blockIdx.z, split = blockIdx.y;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int KW = blockDim.x >> 6;
  const int n = lane & 15, g = lane >> 4;
  PlaneArgs pa = p.pa;
  pa.w0 += b * p.w0_bstride;
  if (pa.w1) pa.w1 += b * p.w1_bstride;
  pa.s += b * p.s_bstride;
  const int ks = pa.K / p.ksplit, k0 = split * ks, c0 = k0 / F::KPC, cend = c0 + ks / F::KPC;
  const int cw = wave * 4 + g, cstep = 4 * KW;
  const int J = (ks / F::KPC + cstep - 1) / cstep;     // chunks per lane per tile
  const uint16_t* xg = p.x + b * p.x_bstride;
  size_t xbytes = XL ? (((size_t)p.M * ks * 2 + 15) & ~(size_t)15) : 0;
  float* red = reinterpret_cast<float*>(reinterpret_cast<char*>(lds) + xbytes);
  float* slot = red + (KW > 1 ? KW - 1 : 0) * 64 * 4;
  const int tiles = (p.N + 15) / 16;
  int t = blockIdx.x;
  if (t >= tiles) return;

  if constexpr (XL) {
    // stage x[0:M, k0:k0+ks]
    const int per_row = ks / 8;
    for (int i = threadIdx.x; i < p.M * per_row; i += blockDim.x) {
      const int m = i / per_row, q = i - m * per_row;
      reinterpret_cast<uint4*>(lds + m * ks)[q] = *reinterpret_cast<const uint4*>(xg + m * p.x_stride + k0 + q * 8);
    }
    __syncthreads();
  }

  for (; t < tiles; t += gridDim.x) {
    const int64_t row = (int64_t)t * 16 + n;
    const bool wrow = row < p.N;
    f32x4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int jb = 0; jb < J; jb += kJ) {
      MfmaBatch<F> cur;
      mfma_load<F>(cur, pa, wrow ? row : -1, c0, cend, cw, cstep, jb, J);
      if constexpr (XL) mfma_compute<F>(cur, (const uint16_t*)lds, ks, k0, p.M, wrow, c0, cend, cw, cstep, jb, J, acc);
      else mfma_compute<F>(cur, xg, (int)p.x_stride, 0, p.M, wrow, c0, cend, cw, cstep, jb, J, acc);
    }
    acc = mfma_wave_reduce<8>(acc, KW, red);
    // lane holds D[m = g*4 + i][n]
    if (p.ksplit == 1) {
      if (wave == 0 && wrow) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (g * 4 + i < p.M) Epi::apply(p, b, g * 4 + i, row, acc[i] * p.gs);
      }
      continue;
    }
    // split-K: wave 0 writes this slice's slot tile, the last workgroup reduces
    float* part = p.part + (int64_t)b * p.ksplit * 16 * p.N;
    const int64_t tile0 = (int64_t)t * 16;
    if (wave == 0) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int m = g * 4 + i;
        if (m < p.M && wrow) part[((int64_t)split * 16 + m) * p.N + row] = acc[i] * p.gs;
      }
    }
    int* ticket = p.tickets + (int64_t)b * tiles + t;
    if (splitk_arrive(ticket, p.ksplit)) {
      for (int i = threadIdx.x; i < p.M * 16; i += blockDim.x) {
        const int m = i >> 4;
        const int64_t r = tile0 + (i & 15);
        if (r >= p.N) continue;
        const float* src = part + (int64_t)m * p.N + r;
        const int64_t sstride = (int64_t)16 * p.N;
        float tot = 0.0f;
        for (int s0 = 0; s0 < p.ksplit; s0 += 8) {
          float v[8];
#pragma unroll
          for (int jj = 0; jj < 8; ++jj) v[jj] = s0 + jj < p.ksplit ? src[(s0 + jj) * sstride] : 0.0f;
#pragma unroll
          for (int jj = 0; jj < 8; ++jj)
            if (s0 + jj < p.ksplit) tot = s0 + jj == 0 ? v[jj] : tot + v[jj];
        }
        Epi::apply(p, b, m, r, tot);
      }
      if (threadIdx.x == 0) ticket_reset(ticket);
    }
    __syncthreads();
  }
  (void)slot;
}

// Workgroups to launch so that each CU holds about 16 waves of KW-wave groups.
int mfma_grid_target(int kw);

template <class F, class Epi>
int launch_gemv_mfma(const GemvLaunch& p0, int batch, hipStream_t st) {
  GemvLaunch p = p0;
  const int ks = p.pa.K / p.ksplit;
  const int chunks = ks / F::KPC;
  const int KW = mfma_kw(chunks);
  const int tiles = (p.N + 15) / 16;
  const int per_batch = (mfma_grid_target(KW) + batch * p.ksplit - 1) / (batch * p.ksplit);
  const int gx = tiles < per_batch ? tiles : (per_batch < 1 ? 1 : per_batch);
  const bool xl = mfma_lds_bytes(p.M, ks, KW, true) <= 96 * 1024;
  const size_t lds = mfma_lds_bytes(p.M, ks, KW, xl);
  dim3 grid(gx, p.ksplit, batch), block(64 * KW);
  if (xl) hipLaunchKernelGGL((gemv_mfma_kernel<F, true, Epi>), grid, block, lds, st, p);
  else hipLaunchKernelGGL((gemv_mfma_kernel<F, false, Epi>), grid, block, lds, st, p);
  return check_launch("gemv_mfma");
}

}  // namespace fp4x
