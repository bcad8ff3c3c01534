// Few-rows GEMV: matrices of so few rows that 16-row tiles would leave most
// CUs idle (a router gate's 512 x 2560 is 32 tiles on 256 CUs).  A
// workgroup owns whole weight rows, so no row's sum spans two workgroups: no
// cross-workgroup reduction, no scratch, no tickets.  Each kernel takes a
// compact argument block read in one round of scalar loads at its start, and
// issues every memory load before using any, so a lane waits for one memory
// round trip.  Two kernels:
//
//   * M <= 4 (rows_fma_kernel): R = 1, 2 or 4 weight rows per workgroup,
//     thread c owning chunk c (the format's 16-byte unit of the main plane,
//     with its scale) of each row, or, for the 32-weight chunks of W6 and
//     NVFP4, half c & 1 of chunk c >> 1 (half the serial dequant work per
//     lane); dequantized to the bf16 operand and multiplied with the M
//     activation rows by v_dot2_f32_bf16 (two bf16 products and the running
//     fp32 sum per step: half the instructions of an fma per product, which
//     took the 512 x 2560 gate at M = 3 from 3.3 to 3.0 us).  Each wave sums
//     its partials with DPP steps, lane 63 stores the wave's sums, and thread
//     r M + m adds the waves' sums of row r in wave order.
//   * 4 < M <= 16 (rows_mfma_kernel): R <= 4 weight rows per workgroup,
//     products on v_mfma_f32_4x4x4bf16_1k: 16 independent blocks of
//     D[4 x 4] += A[4 x 4] B[4 x 4].  Lane 4b + q of a wave holds, for block
//     b, A row q (activation row m = 4g + q over 4 consecutive k) and B column
//     q (weight row q over the same 4 k); D[m][q] lands in lane 4b + q,
//     element m.  Each lane dequantizes CPL chunks of one weight row and feeds
//     the bf16 pairs and the bf16 activations to the MFMA as they are; two DPP
//     row rotations add the 4 blocks of each 16-lane row, and thread (q, m)
//     adds the rows' sums of every wave in a fixed order.
//
// Both orders are fixed, so results repeat bit for bit.  At M <= 4 the fma
// kernel's extra VALU work costs less than the MFMA kernel's 4-lane
// replication of every chunk's loads (measured on the 512 x 2560 gate:
// 3.0 against 3.4 us at M = 1); at M = 16 the MFMA kernel is faster
// (5.6 against 6.8 us).
#pragma once
#include "fp4x_mfma.h"
#include <type_traits>

namespace fp4x {

// The few-rows kernels' arguments: only what they read, 80 bytes.
struct RowsLaunch {
  PlaneArgs pa;
  const uint16_t* x;     // bf16 activations [M][x_stride]
  void* out;             // [M][out_stride]
  int x_stride, out_stride;
  int N, M, R, out_dtype;
  float gs;              // applied to every sum (NVFP4 global scale; 1 otherwise)
};

// ------------------------------------------------------------------ M <= 4

constexpr int kRowsFmaMaxThreads = 256;              // K up to 256 chunks (4096 int8, 8192 NVFP4 weights)
constexpr int kRowsMultiMaxThreads = 512;            // several rows, or half chunks, per workgroup: 512 lanes
constexpr int rows_fma_max_threads(int R, int LPC) {
  return R == 1 && LPC == 1 ? kRowsFmaMaxThreads : kRowsMultiMaxThreads;
}

// Sum over each row of 16 lanes, every lane of the row receiving it: DPP
// xor-partner additions with partners 1, 2 (quad permutes), 4 (half-row
// mirror, within the already uniform quads) and 8 (row mirror).
__device__ __forceinline__ float row16_sum(float v) {
  v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, false));   // quad_perm [1,0,3,2]
  v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xF, 0xF, false));   // quad_perm [2,3,0,1]
  v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x141, 0xF, 0xF, false));  // row_half_mirror
  v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x140, 0xF, 0xF, false));  // row_mirror
  return v;
}

// Wave sum, complete in lane 63: the four row sums s0..s3 of row16_sum added
// as (s3 + s2) + (s1 + s0) by two DPP broadcasts (row_bcast:15 adds each
// even row's sum into the next row, row_bcast:31 adds row 1 into rows 2
// and 3; rows outside the row mask add the +0 of `old`).
__device__ __forceinline__ float wave_sum_lane63(float v) {
  v = row16_sum(v);
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x142, 0xA, 0xF, false));  // row_bcast:15
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x143, 0xC, 0xF, false));  // row_bcast:31
  return v;
}

// c + (the two bf16 products of a and b) in fp32, one v_dot2_f32_bf16 (the
// two products' sum is not always rounded once; the few-rows sums are checked
// against the accumulation bound, and repeat bit for bit)
__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a), __builtin_bit_cast(bf16x2_t, b), c, false);
}

template <class F, int MT, int R, int LPC>
__global__ __launch_bounds__(rows_fma_max_threads(R, LPC)) void rows_fma_kernel(
    RowsLaunch p) {
  extern __shared__ float red[];                       // [waves][R][MT]
  // every argument read up front (the empty asm needs each value in a
  // register), so no scalar load waits between the main loads and the store
  const PlaneArgs pa = p.pa;
  const uint16_t* const xg = p.x;
  void* const out = p.out;
  const int xs = p.x_stride, os = p.out_stride, N = p.N, M = p.M, odt = p.out_dtype;
  const float gs = p.gs;
  asm volatile("" ::"s"(pa.w0), "s"(pa.w1), "s"(pa.s), "s"(pa.K), "s"(pa.G), "s"(xg), "s"(out), "s"(xs), "s"(os),
               "s"(N), "s"(M), "s"(odt), "s"(gs));
  // LPC lanes per chunk: with 2, lane c takes half c & 1 (16 weights) of
  // chunk c >> 1, loaded as the sub-0 half of a chunk
  static_assert(LPC == 1 || (LPC == 2 && F::SUB == 2), "half chunks of two-half formats only");
  constexpr int SUBL = LPC == 2 ? 1 : F::SUB;          // 16-weight halves per lane
  const int nch = pa.K / F::KPC, nl = nch * LPC;
  const int c = threadIdx.x;
  const int64_t row0 = (int64_t)blockIdx.x * R;
  // Lanes past the row's chunks load the last one (their sums are zeroed
  // below), rows past N load row N - 1 (never stored); loads under a branch
  // would each be waited for at its join.
  const int cl = c < nl ? c : nl - 1;
  const int cc = cl / LPC, hf = LPC == 2 ? (cl & 1) : 0;
  auto load_row = [&](int64_t row) {
    if constexpr (LPC == 2) return F::load_half(pa, row, cc, hf);
    else return F::load(pa, row, cc);
  };
  typename F::Chunk ch[R];
  uint4 xr[SUBL][MT][2];
  auto load_x = [&]() {
#pragma unroll
    for (int sub = 0; sub < SUBL; ++sub)
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        const uint4* xp = reinterpret_cast<const uint4*>(xg + (int64_t)m * xs + cc * F::KPC + (hf + sub) * 16);
        xr[sub][m][0] = xp[0];
        xr[sub][m][1] = xp[1];
      }
  };
  if constexpr (R == 1) {
    ch[0] = load_row(row0);
    load_x();
  } else {
    // the activations first, then the rows in order, so that row r's sums
    // wait only for the loads up to its own
    load_x();
#pragma unroll
    for (int r = 0; r < R; ++r) ch[r] = load_row(row0 + r < N ? row0 + r : (int64_t)N - 1);
  }
  __builtin_amdgcn_sched_barrier(0);                   // every load above issues before any use below
  float acc[R][MT];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int m = 0; m < MT; ++m) acc[r][m] = 0.0f;
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int sub = 0; sub < SUBL; ++sub) {
      uint32_t w[8];
      F::deq16(ch[r], sub, w);
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        const uint4 xa = xr[sub][m][0], xb = xr[sub][m][1];
        const uint32_t xv[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
        float t = acc[r][m];
#pragma unroll
        for (int i = 0; i < 8; ++i) t = dot2_bf16(w[i], xv[i], t);
        acc[r][m] = t;
      }
    }
  if (c >= nl) {
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int m = 0; m < MT; ++m) acc[r][m] = 0.0f;
  }
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nwaves = (nl + 63) >> 6;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    float sums[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m) sums[m] = wave_sum_lane63(acc[r][m]);
    if (lane == 63) {
#pragma unroll
      for (int m = 0; m < MT; ++m) red[(wave * R + r) * MT + m] = sums[m];
    }
  }
  __syncthreads();
  const int o = threadIdx.x;
  if (o < R * MT) {
    const int r = o / MT, m = o % MT;
    float v = red[r * MT + m];
    for (int j = 1; j < nwaves; ++j) v += red[(j * R + r) * MT + m];
    const int64_t row = row0 + r;
    if (row < N) store_out(out, (int64_t)m * os + row, odt, v * gs);
  }
}

// ------------------------------------------------------------------ 4 < M <= 16

typedef short rows_s16x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f32x4_t mfma4(uint32_t a0, uint32_t a1, uint32_t b0, uint32_t b1, f32x4_t c) {
  const uint2 a = make_uint2(a0, a1), b = make_uint2(b0, b1);
  return __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(__builtin_bit_cast(rows_s16x4, a), __builtin_bit_cast(rows_s16x4, b),
                                                c, 0, 0, 0);
}

// v + the same lane's value 4 and then 8 lanes round its row of 16 (DPP
// row_ror): every lane ends with the sum over the 4 blocks of its row for
// its column q = lane % 4.
__device__ __forceinline__ float row_blocks_sum(float v) {
  v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x124, 0xF, 0xF, false));  // row_ror:4
  v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x128, 0xF, 0xF, false));  // row_ror:8
  return v;
}

// The MFMA few-rows decomposition of rows of nch chunks at M activation
// rows: MG groups of 4 activation rows, CPL chunks per lane, `waves` waves.
// CPL aims at about 5 waves (fewer chunks per lane leave more fixed cost per
// chunk, more leave longer waits on each wave's slowest load), within the
// registers that hold every activation load of a lane (CPL MG SUB <= 16).
struct RowsPlan {
  int MG, cpl, waves;
};

template <class F>
inline bool rows_mfma_plan(int nch, int M, RowsPlan& pl) {
  if (nch < 1 || M < 1 || M > 16) return false;
  pl.MG = M <= 4 ? 1 : M <= 8 ? 2 : 4;
  int cpl = (nch + 79) / 80;
  while (cpl > 1 && cpl * pl.MG * F::SUB > 16) --cpl;
  if (cpl > 8) cpl = 8;
  pl.cpl = cpl;
  pl.waves = (nch + 16 * cpl - 1) / (16 * cpl);
  return pl.waves <= 8;
}

// One workgroup's R <= 4 rows [row0, row0 + R) of the MFMA few-rows GEMV
// (MG groups of 4 activation rows, CPL chunks per lane) on its first `waves`
// waves; the other waves only meet the barrier.  store(m, row, v) receives
// every sum of a row below N.  red: LDS of waves * 4 * 4 MG * 4 floats.
template <class F, int MG, int CPL, class Store>
__device__ __forceinline__ void rows_mfma_item(const PlaneArgs& pa, const uint16_t* xg, int xs, int N, int M, int R,
                                               int64_t row0, int waves, float* red, Store store) {
  const int nch = pa.K / F::KPC;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int q = lane & 3;
  if (wave < waves) {
    // Every load goes out unconditionally, before any is used, so a lane
    // waits for one memory round trip: columns q >= R load row R - 1 (the
    // same lines as column R - 1, so no extra traffic; never stored), rows
    // past N load row N - 1, activation rows past M load row 0 (never
    // stored), and chunks past the row's end load its last chunk (their B
    // operand is zeroed below).  Lane chunk t of wave w is chunk
    // (CPL w + t) 16 + block: each load instruction reads 16 consecutive
    // chunks of every row.
    int64_t wr = row0 + (q < R ? q : R - 1);
    if (wr >= N) wr = N - 1;
    typename F::Chunk ch[CPL];
    uint4 xr[CPL][MG][F::SUB][2];
#pragma unroll
    for (int t = 0; t < CPL; ++t) {
      const int c = (wave * CPL + t) * 16 + (lane >> 2);
      const int cc = c < nch ? c : nch - 1;
      ch[t] = F::load(pa, wr, cc);
#pragma unroll
      for (int g = 0; g < MG; ++g) {
        const int m = 4 * g + q;
        const uint4* xp = reinterpret_cast<const uint4*>(xg + (int64_t)(m < M ? m : 0) * xs + cc * F::KPC);
#pragma unroll
        for (int sub = 0; sub < F::SUB; ++sub) {
          xr[t][g][sub][0] = xp[2 * sub];
          xr[t][g][sub][1] = xp[2 * sub + 1];
        }
      }
    }
    __builtin_amdgcn_sched_barrier(0);                 // every load above issues before any use below
    f32x4_t acc[MG];
#pragma unroll
    for (int g = 0; g < MG; ++g) acc[g] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int t = 0; t < CPL; ++t) {
      const bool live = (wave * CPL + t) * 16 + (lane >> 2) < nch;
#pragma unroll
      for (int sub = 0; sub < F::SUB; ++sub) {
        uint32_t w[8];
        F::deq16(ch[t], sub, w);
        if (!live) {
#pragma unroll
          for (int i = 0; i < 8; ++i) w[i] = 0u;
        }
#pragma unroll
        for (int g = 0; g < MG; ++g) {
          const uint4 xa = xr[t][g][sub][0], xb = xr[t][g][sub][1];
          acc[g] = mfma4(xa.x, xa.y, w[0], w[1], acc[g]);
          acc[g] = mfma4(xa.z, xa.w, w[2], w[3], acc[g]);
          acc[g] = mfma4(xb.x, xb.y, w[4], w[5], acc[g]);
          acc[g] = mfma4(xb.z, xb.w, w[6], w[7], acc[g]);
        }
      }
    }
    // block sums per 16-lane row, stored by lanes 0-3 of the row as
    // red[wave * 4 + row][m][q]
    const int slot = wave * 4 + (lane >> 4);
#pragma unroll
    for (int g = 0; g < MG; ++g)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float v = row_blocks_sum(acc[g][e]);
        if ((lane & 12) == 0) red[(slot * (4 * MG) + 4 * g + e) * 4 + q] = v;
      }
  }
  __syncthreads();
  const int o = threadIdx.x;
  if (o < R * M) {
    const int j = o / M, m = o % M;
    // every row sum read at once (slots past the workgroup's waves read slot
    // 0 and add nothing), then added in slot order
    float t[32];
#pragma unroll
    for (int s2 = 0; s2 < 32; ++s2) t[s2] = red[((s2 < waves * 4 ? s2 : 0) * (4 * MG) + m) * 4 + j];
    float v = t[0];
#pragma unroll
    for (int s2 = 1; s2 < 32; ++s2) v += s2 < waves * 4 ? t[s2] : 0.0f;
    const int64_t row = row0 + j;
    if (row < N) store(m, row, v);
  }
}

template <class F, int MG, int CPL>
__global__ __launch_bounds__(512) void rows_mfma_kernel(RowsLaunch p) {
  extern __shared__ float red[];
  // every argument read up front (the empty asm needs each value in a
  // register), so no scalar load waits between the main loads and the store
  const PlaneArgs pa = p.pa;
  const uint16_t* const xg = p.x;
  void* const out = p.out;
  const int xs = p.x_stride, os = p.out_stride, N = p.N, M = p.M, R = p.R, odt = p.out_dtype;
  const float gs = p.gs;
  asm volatile("" ::"s"(pa.w0), "s"(pa.w1), "s"(pa.s), "s"(pa.K), "s"(pa.G), "s"(xg), "s"(out), "s"(xs), "s"(os),
               "s"(N), "s"(M), "s"(R), "s"(odt), "s"(gs));
  rows_mfma_item<F, MG, CPL>(pa, xg, xs, N, M, R, (int64_t)blockIdx.x * R, (int)(blockDim.x >> 6), red,
                             [&](int m, int64_t row, float v) { store_out(out, (int64_t)m * os + row, odt, v * gs); });
}

// Rows per workgroup of an MFMA few-rows launch: the fewest (<= 4) that keep
// the grid within the CUs; 0 when N needs more.
inline int rows_per_wg(int N, int cus) {
  for (int r = 1; r <= 4; ++r)
    if ((N + r - 1) / r <= cus) return r;
  return 0;
}

// Launch rows_mfma_item's kernel for plan pl.
template <class F, int MG, int CPL>
inline void rows_mfma_launch1(const RowsLaunch& a, const RowsPlan& pl, hipStream_t st) {
  const size_t lds = (size_t)pl.waves * 4 * (4 * MG) * 4 * sizeof(float);
  hipLaunchKernelGGL((rows_mfma_kernel<F, MG, CPL>), dim3((unsigned)((a.N + a.R - 1) / a.R)),
                     dim3((unsigned)(64 * pl.waves)), lds, st, a);
}

// Dispatch over the (MG, CPL) instances rows_mfma_plan can produce: MG 1
// with CPL 1..8, MG 2 with 1..8, MG 4 with 1..4 (SUB 1) or 1..2 (SUB 2).
template <class F, class Body>
inline bool rows_dispatch(const RowsPlan& pl, Body body) {
#define FP4X_ROWS_C(G, C)                                        \
  if constexpr (C * G * F::SUB <= 16) {                          \
    if (pl.MG == G && pl.cpl == C) {                             \
      body.template run<G, C>();                                 \
      return true;                                               \
    }                                                            \
  }
  FP4X_ROWS_C(1, 1) FP4X_ROWS_C(1, 2) FP4X_ROWS_C(1, 3) FP4X_ROWS_C(1, 4)
  FP4X_ROWS_C(1, 5) FP4X_ROWS_C(1, 6) FP4X_ROWS_C(1, 7) FP4X_ROWS_C(1, 8)
  FP4X_ROWS_C(2, 1) FP4X_ROWS_C(2, 2) FP4X_ROWS_C(2, 3) FP4X_ROWS_C(2, 4)
  FP4X_ROWS_C(2, 5) FP4X_ROWS_C(2, 6) FP4X_ROWS_C(2, 7) FP4X_ROWS_C(2, 8)
  FP4X_ROWS_C(4, 1) FP4X_ROWS_C(4, 2) FP4X_ROWS_C(4, 3) FP4X_ROWS_C(4, 4)
#undef FP4X_ROWS_C
  return false;
}

template <class F>
struct RowsGemvBody {
  const RowsLaunch& a;
  const RowsPlan& pl;
  hipStream_t st;
  template <int G, int C>
  void run() const { rows_mfma_launch1<F, G, C>(a, pl, st); }
};

// The few-rows shapes: one matrix of so few rows that the MFMA core's 16-row
// tiles fill under half of the CUs, at most 4 rows per workgroup.
inline bool rows_shape_ok(int N, int M, int cus) {
  const int tiles = (N + 15) / 16;
  return M >= 1 && M <= 16 && N >= 1 && tiles * 2 < cus && rows_per_wg(N, cus) > 0;
}

// Workgroups of rows_fma_kernel<F, MT, R, LPC> of `threads` threads one CU
// holds at once (its registers decide: the NVFP4 and W6 kernels at M >= 3
// hold fewer).
template <class F, int MT, int R, int LPC>
int rows_fma_resident(int threads) {
  static int cache[kRowsMultiMaxThreads / 64 + 1];
  const int key = threads / 64;
  int occ = cache[key];
  if (occ <= 0) {
    const size_t lds = (size_t)key * R * MT * sizeof(float);
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
            &occ, reinterpret_cast<const void*>(rows_fma_kernel<F, MT, R, LPC>), threads, lds) != hipSuccess ||
        occ < 1)
      occ = 1;
    cache[key] = occ;
  }
  return occ;
}

template <class F, int R, int LPC>
int rows_fma_resident_m(int M, int threads) {
  return M == 1   ? rows_fma_resident<F, 1, R, LPC>(threads)
         : M == 2 ? rows_fma_resident<F, 2, R, LPC>(threads)
         : M == 3 ? rows_fma_resident<F, 3, R, LPC>(threads)
                  : rows_fma_resident<F, 4, R, LPC>(threads);
}

// The fma kernel beyond few-rows shapes: wider matrices of short rows (the MTP
// shared expert's [1280 x 2560] and its down projection [2560 x 640]), whose
// tiles leave the MFMA core and the streaming kernels one memory round trip
// per tile with few loads in flight, while one row per workgroup puts every
// load of the matrix in flight at once.  Three limits: at most 2^17 fp32
// products per lane slot of a CU (N * threads * M * KPC / CUs), beyond which
// the dot work outlasts the loads; every workgroup resident in one round; and
// at most 32 waves per CU whatever the occupancy, so that the mixer's up
// projection [10240 x 320 or 640] (one wave per row, 40 per CU) stays on the
// MFMA core, whose sums the single-launch mixer's up tiles reproduce bit for
// bit.  (Two resident rounds were faster for W8 [4096 x 2560] at M = 1, 4.6
// against 6.1 us, but would take that projection.)  Measured as graph replays
// from HBM, this kernel against the path the shape takes without it, us at
// M = 1 / 2 / 3 / 4: W8 [2560 x 2560] 3.8 /
// 4.4 / 4.9 / 5.5 against 5.5 / 5.8 / 6.0 / 6.3 (streaming); W8 [8192 x 640]
// 4.0 / 4.3 / 4.9 / 5.4 against 5.9 / 6.0 / 6.1 / 6.3 (MFMA core); MXFP8
// [2048 x 2560] 3.4 / 3.9 / 4.3 / 4.7 against 6.3 / 6.5 / 6.7 / 6.9; W6 [2048
// x 2560] 3.9 / 4.6 / 5.4 / 6.1 against 7.1 / 7.2 / 7.4 / 8.0; NVFP4 [4096 x
// 2560] 4.5 / 6.0 against 6.3 / 6.4 at M = 1 / 2, and 7.5 against 6.5 at
// M = 3, past the limit.
constexpr int64_t kRowsFmaProductsPerCu = int64_t(1) << 17;

template <class F, int LPC>
bool rows_fma_shape_ok(int N, int M, int threads, int cus) {
  if (M < 1 || M > 4 || N < 1 || threads > rows_fma_max_threads(1, LPC)) return false;
  if (rows_shape_ok(N, M, cus)) return true;
  if ((int64_t)N * threads * M * F::KPC / LPC > kRowsFmaProductsPerCu * cus) return false;
  if ((int64_t)N * (threads / 64) / LPC > 32 * (int64_t)cus) return false;
  return N <= (int64_t)rows_fma_resident_m<F, 1, LPC>(M, threads) * cus;
}

// Rows per workgroup R of the fma kernel for a matrix of M <= 4 activation
// rows that is not a few-rows shape, or 0 for none.  With R > 1 a workgroup
// loads its activations once and then every chunk of its R rows, so the
// activation reads (M * K * 2 bytes per workgroup, from L2) shrink R-fold,
// at R times the registers and 1/R of the workgroups.  Only for rows longer
// than one wave's chunks (the mixer's up projection, 20 or 40 chunks, stays
// on the MFMA core) and of at most 512 chunks, with every workgroup resident
// in one round:
//   * M >= 2 and N >= 8 rows per CU: R = 2;
//   * else R = 1 where rows_fma_shape_ok takes the matrix (at M = 1, and
//     for under 8 rows per CU, the one-row kernel's extra workgroups pay
//     more than its activation reads cost);
//   * else R = 2 (rows of over 256 chunks, or past the one-row limits).
// Measured as graph replays from HBM (us at M = 1 / 2 / 3 / 4; one lane per
// chunk, before W6 and NVFP4 split chunks over two lanes), R = 1 / 2:
// W6 [2048 x 2560] 3.9 / 4.6 / 5.4 / 6.1 against 4.2 / 4.5 / 5.0 / 5.4;
// NVFP4 [2048 x 2560] 3.5 / 4.3 / 5.0 / 5.8 against 3.6 / 4.0 / 4.4 / 4.7;
// W8 [2560 x 2560] 3.8 / 4.4 / 5.0 / 5.5 against 4.0 / 4.4 / 4.7 / 5.1;
// MXFP8 [2048 x 2560] 3.5 / 3.9 / 4.3 / 4.8 against 3.8 / 4.0 / 4.4 / 4.8;
// W6 [1280 x 2560] 3.4 / 3.9 / 4.4 / 4.9 against 3.9 / 4.3 / 4.7 / 5.1.  Against
// the path these shapes took before (MFMA core, or W8's single-matrix
// stream): W6 [2560 x 6144] (the attention output projection) 5.4 (R = 1) /
// 6.7 / 8.1 / 9.5 against 14.0 / 14.3 / 14.6 / 16.2 (R = 4 at M = 2..4: 7.6
// / 8.7 / 9.7; R = 8: 9.8 / 11.1 / 12.4); NVFP4 [2560 x 6144] 4.7 / 5.7 / 7.1
// / 8.6 against 10.7 / 11.0 / 11.3 / 12.7; MXFP8, W8 and bf16 [2560 x 6144]
// (384 chunks, past the one-row kernel, R = 2): 5.5 / 6.5 / 7.5 / 8.4, 5.6 /
// 6.6 / 7.6 / 8.4 and 7.8 / 7.9 / 8.7 / 9.6 against 11.7 / 12.0 / 12.3 / 13.6,
// 7.9 / 8.3 / 8.7 / 14.3 and 12.5 / 12.6 / 12.8 / 14.3; W6 [4096 x 2560] 5.1
// / 6.0 / 6.7 / 7.6 against 7.5 / 7.6 / 7.8 / 8.3; NVFP4 [8192 x 2560] 5.9 /
// 7.2 at M = 1 / 2 against 7.6 / 7.8.  Larger matrices stay on the streaming
// kernels or the MFMA core (W6 [8192 x 2560] at M = 3: 7.4 streaming against
// 10.5 / 9.9 at R = 2 / 4).
template <class F, int LPC>
int rows_fma_pick(int N, int M, int nch, int threads, int cus) {
  if (M < 1 || M > 4 || N < 1) return 0;
  if (rows_shape_ok(N, M, cus)) return threads <= rows_fma_max_threads(1, LPC) ? 1 : 0;
  const bool r2 = nch > 64 && threads <= kRowsMultiMaxThreads &&
                  (N + 1) / 2 <= (int64_t)rows_fma_resident_m<F, 2, LPC>(M, threads) * cus;
  if (M >= 2 && N >= 8 * cus && r2) return 2;
  if (rows_fma_shape_ok<F, LPC>(N, M, threads, cus)) return 1;
  return r2 ? 2 : 0;
}

template <class F, int R, int LPC>
inline bool rows_fma_launch(const RowsLaunch& a, int threads, hipStream_t st) {
  const size_t lds = (size_t)(threads / 64) * R * a.M * sizeof(float);
  const dim3 grid((unsigned)((a.N + R - 1) / R)), block((unsigned)threads);
  switch (a.M) {
    case 1: hipLaunchKernelGGL((rows_fma_kernel<F, 1, R, LPC>), grid, block, lds, st, a); return true;
    case 2: hipLaunchKernelGGL((rows_fma_kernel<F, 2, R, LPC>), grid, block, lds, st, a); return true;
    case 3: hipLaunchKernelGGL((rows_fma_kernel<F, 3, R, LPC>), grid, block, lds, st, a); return true;
    case 4: hipLaunchKernelGGL((rows_fma_kernel<F, 4, R, LPC>), grid, block, lds, st, a); return true;
  }
  return false;
}

// The few-rows launch block of a call, false when the call's layout does not
// fit the few-rows kernels (several matrices, a per-row scale, strides past
// int32, K not a whole number of chunks, FP4X_ROWS=0).
inline bool rows_launch_args(const GemvLaunch& p, int batch, int kpc, RowsLaunch& a) {
  if (!switches().rows || batch != 1 || p.rs) return false;
  if (p.x_stride > INT32_MAX || p.out_stride > INT32_MAX || p.pa.K % kpc) return false;
  a.pa = p.pa;
  a.x = p.x;
  a.out = p.out;
  a.x_stride = (int)p.x_stride;
  a.out_stride = (int)p.out_stride;
  a.N = p.N;
  a.M = p.M;
  a.R = 1;
  a.out_dtype = p.out_dtype;
  a.gs = p.gs;
  return true;
}

template <class F, int LPC>
inline bool rows_fma_go(RowsLaunch& a, int R, int threads, hipStream_t st) {
  a.R = R;
  switch (R) {
    case 1: return rows_fma_launch<F, 1, LPC>(a, threads, st);
    case 2: return rows_fma_launch<F, 2, LPC>(a, threads, st);
    case 4: return rows_fma_launch<F, 4, LPC>(a, threads, st);
  }
  return false;
}

// Launch a few-rows kernel when the call fits one: one matrix, no per-row
// scale, strides within int32, and either the fma kernel (M <= 4, R rows per
// workgroup as rows_fma_pick decides) or, for a few-rows shape, an MFMA plan
// of at most 8 waves; false (nothing launched) otherwise, or when
// FP4X_ROWS=0.  The split count of the call is a shape precondition only:
// these kernels sum each row over its whole K inside one workgroup, in a
// fixed order.  W6 and NVFP4 split each chunk over two lanes, measured
// against one lane per chunk (us at M = 1 / 3): W6 [1280 x 2560] 3.3 / 3.8
// against 3.4 / 4.5; [2560 x 640] 3.0 / 3.4 against 3.3 / 4.2; [640 x 2560]
// 3.0 / 3.4 against 3.1 / 3.7; [4096 x 2560] 4.8 / 6.1 against 5.1 / 6.7;
// [2560 x 6144] at M = 3 7.7 against 8.1 (at M = 1 5.6 against 5.4, so rows
// of over 128 chunks keep one lane per chunk at M = 1); NVFP4 [2560 x 640]
// 2.8 / 3.3 against 3.0 / 3.9; [4096 x 2560] 4.2 / 5.4 against 4.5 / 5.9.
template <class F>
bool launch_rows_gemv(const GemvLaunch& p, int batch, hipStream_t st) {
  RowsLaunch a;
  if (!rows_launch_args(p, batch, F::KPC, a)) return false;
  const int cus = device_cus();
  if constexpr (std::is_same<F, FmtMX8>::value || std::is_same<F, FmtNV4>::value) {
    // MXFP8 and NVFP4 from 10 rows per CU at M >= 3 with rows of K >= 4096,
    // and at M = 4 with any K, stream instead (one tile per workgroup): the
    // two-row workgroups then read the activations more often than they
    // save.  Graph replays from HBM, us, streaming against this kernel:
    // MXFP8 [2560 x 6144] M = 3 / 4 7.15 / 7.34 against 7.59 / 8.48,
    // [2560 x 2560] M = 4 4.87 against 5.25; NVFP4 [2560 x 6144] 6.40 / 6.60
    // against 6.75 / 7.81, [2560 x 2560] M = 4 4.58 against 4.97, [4096 x
    // 2560] M = 4 5.78 against 6.04 (at M = 3 and K = 2560 this kernel ties or
    // wins: MXFP8 [2048 x 2560] 4.39 against 4.69).
    if (p.M >= 3 && p.N >= 10 * cus && (p.pa.K >= 4096 || p.M >= 4)) return false;
  }
  const int nch = p.pa.K / F::KPC;
  if constexpr (F::SUB == 2) {
    // W6 and NVFP4 chunks (32 weights) split over two lanes: at M >= 2, and
    // at M = 1 for rows of up to 128 chunks
    if (p.M >= 2 || 2 * nch <= kRowsFmaMaxThreads) {
      const int lanes = (2 * nch + 63) / 64 * 64;
      const int R = rows_fma_pick<F, 2>(p.N, p.M, nch, lanes, cus);
      if (R) return rows_fma_go<F, 2>(a, R, lanes, st);
    }
  }
  const int lanes = (nch + 63) / 64 * 64;
  const int R = rows_fma_pick<F, 1>(p.N, p.M, nch, lanes, cus);
  if (R) return rows_fma_go<F, 1>(a, R, lanes, st);
  if (!rows_shape_ok(p.N, p.M, cus)) return false;
  RowsPlan pl;
  if (!rows_mfma_plan<F>(nch, p.M, pl)) return false;
  a.R = rows_per_wg(p.N, cus);
  return rows_dispatch<F>(pl, RowsGemvBody<F>{a, pl, st});
}

// MXFP8 matrices of 16 to 20 rows per CU at M = 1 (shapes its streaming
// kernel takes): the fma kernel with 2 rows per workgroup, when every
// workgroup is resident.  Measured as graph replays from HBM, us, this
// against the streaming kernel: [4096 x 2560] 4.44 against 4.66 at M = 1.
// Since the streaming kernel's five-wave geometry it is the other way round
// at M = 2 ([4096 x 2560] 5.09 against 4.95) and for more rows ([6144 x 2560]
// 5.60-5.74 against 5.51-5.54 at M = 1, [8192 x 2560] 6.15-6.41 against
// 6.06-6.12), so those stream.
//
// W6 at M = 1 from 32 to 52 rows per CU (shapes its streaming kernel takes):
// 2 rows per workgroup with two lanes per chunk, in as many rounds as it
// takes, ahead of the streaming kernel (us, two runs: [8192 x 2560] 6.9-7.1
// against 7.2; [10240 x 2560] 7.7-8.2 against 9.6; [13312 x 2560] 9.6-9.9
// against 9.9; [16384 x 2560] 11.4 against 10.4-11.0, so larger matrices
// stream).
template <class F>
bool launch_rows_wide(const GemvLaunch& p, hipStream_t st) {
  RowsLaunch a;
  if constexpr (std::is_same<F, FmtW6>::value) {
    if (p.M != 1 || !rows_launch_args(p, 1, F::KPC, a)) return false;
    const int cus = device_cus();
    const int lanes = (2 * (p.pa.K / F::KPC) + 63) / 64 * 64;
    if (p.N < 32 * cus || p.N > 52 * cus || lanes > kRowsMultiMaxThreads) return false;
    return rows_fma_go<F, 2>(a, 2, lanes, st);
  }
  if (p.M != 1 || !rows_launch_args(p, 1, F::KPC, a)) return false;
  const int cus = device_cus();
  const int nch = p.pa.K / F::KPC;
  const int threads = (nch + 63) / 64 * 64;
  if (p.N < 16 * cus || p.N > 20 * cus || nch <= 64 || threads > kRowsMultiMaxThreads) return false;
  if ((p.N + 1) / 2 > (int64_t)rows_fma_resident_m<F, 2, 1>(p.M, threads) * cus) return false;
  return rows_fma_go<F, 1>(a, 2, threads, st);
}

}  // namespace fp4x
