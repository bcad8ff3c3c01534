// MFMA GEMV core for gfx950: y[m, n] = sum_k x[m, k] * w[n, k], M <= 16.
//
// One workgroup of KW waves works on tiles of 16 weight rows (the n dimension
// of v_mfma_f32_16x16x32_bf16; the M <= 16 activation rows pad the m
// dimension).  The K slice of a row is cut into 16-byte chunks (KPC weights
// each) taken in pairs: lane (n = lane & 15, g = lane >> 4) of wave w holds
// pair slots p = w*4 + g + j*4*KW of row n, i.e. chunks 2p and 2p + 1, so the
// four lane groups of a wave read 128 contiguous bytes of each of 16 rows per
// pair of load instructions, and one scale (or auxiliary-plane) load serves
// both chunks.  Chunks are dequantized in registers to the bf16 operand and
// fed 8 k-values per MFMA step; the activation fragment of lane (m, g)
// carries x[m] at the same k, read from LDS.  The KW partial 16x16 tiles are
// summed in wave order through LDS.
//
// Instruction economy: KW is a template parameter, so a lane's chunks sit at
// compile-time strides from one base pointer per weight plane (F::Lane) and
// from one activation address; every load and LDS read of a batch uses a
// constant offset.
//
// Latency hiding: KW is chosen so that a lane's share of a tile (J pair
// slots) fills whole register batches of NJ slots, all of a batch's loads
// are in flight together, and the launch keeps as many workgroups resident
// as the register and LDS budget allows (each with the same number of
// tiles), so the memory latency of one workgroup overlaps the work of the
// others.  The first batch's loads go out before the activations are staged.
//
// Split-K (ksplit > 1): one fp32 slot tile per K slice; the last-arriving
// workgroup of a tile (agent-scope ticket, see splitk_arrive) sums the slots
// in slice order and applies the epilogue, which keeps results independent
// of the arrival order.
#pragma once
#include "fp4x_kernels.h"

namespace fp4x {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int kMaxKW = 8;     // waves per workgroup at most

// A lane's register batch holds NJ slots of CPS chunks each: CPS = 1, or 2
// for the pair layout (32 contiguous bytes per lane and one scale load shared
// by both chunks).  Measured on MI355X: pairs pay off for W8 slices of at
// least 128 chunks (K = 2560 router gates); single chunks win everywhere
// else (MXFP8, W6, NVFP4, INT2, and the K = 640 mixer slices).
constexpr int kNJ = 5;
template <class F> struct MfmaTune { static constexpr bool PAIRS = false; };

// Formats whose MFMA operand is produced in a permuted k order within each
// 16-element block (F::deq16t) declare XPERM; their activations are staged
// with the same permutation.
template <class F, class = void> struct HasXPerm { static constexpr bool value = false; };
template <class F> struct HasXPerm<F, decltype(void(F::XPERM))> { static constexpr bool value = F::XPERM; };
template <bool F16S> struct MfmaTune<FmtW8<F16S>> { static constexpr bool PAIRS = true; };

template <class F>
__host__ __device__ inline int mfma_cps(int chunks) { return MfmaTune<F>::PAIRS && chunks >= 128 ? 2 : 1; }

// Waves per tile for a K slice of `chunks` chunks: the fewest (a power of
// two, at most kMaxKW) that keep a lane's share within one batch.
__host__ __device__ inline int mfma_kw(int chunks, int cps) {
  const int slots = (chunks + cps - 1) / cps;
  int kw = 1;
  while (kw < kMaxKW && (slots + 4 * kw - 1) / (4 * kw) > kNJ) kw <<= 1;
  return kw;
}

// True when every lane of every wave gets exactly J slots in whole batches
// (the constant-offset path); other slices take the general path.
__host__ __device__ inline bool mfma_full(int chunks, int kw, int cps) {
  const int dp = 4 * kw;
  return chunks % (cps * dp) == 0 && (chunks / (cps * dp)) % kNJ == 0;
}

__device__ __forceinline__ f32x4_t mfma16(uint4 a, uint4 b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b), c,
                                                 0, 0, 0);
}

// Barrier for LDS hand-offs between the waves of a workgroup.  Only LDS
// accesses are ordered: outstanding global memory operations (the epilogue's
// stores) are not waited for.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

template <class F, int CPS>
struct MfmaBatch {
  typename F::Chunk ch[kNJ][CPS];
};

// Full path: the NJ slots of a batch at constant offsets from L (L at the
// slot-0 chunk CPS*p, DP = 4*KW slots between a lane's slots).
template <class F, int DP, int CPS>
__device__ __forceinline__ void mfma_load_full(MfmaBatch<F, CPS>& b, const typename F::Lane& L) {
#pragma unroll
  for (int j = 0; j < kNJ; ++j) {
    if constexpr (CPS == 2) F::template pair<2 * DP>(L, j, b.ch[j][0], b.ch[j][1]);
    else b.ch[j][0] = F::template at<DP>(L, j);
  }
}

// General path: chunk (slot j, half h) is c0 + CPS * (cw + (jb + j) * DP) + h
// when it is inside the slice (jb + j < J and the chunk index < nch); other
// chunks read chunk c0 of the same row, which is in bounds, and are
// multiplied as zeros.
template <class F, int DP, int CPS>
__device__ __forceinline__ void mfma_load_general(MfmaBatch<F, CPS>& b, const PlaneArgs& a, int64_t row, int c0,
                                                  int cw, int jb, int J, int nch) {
#pragma unroll
  for (int j = 0; j < kNJ; ++j)
#pragma unroll
    for (int h = 0; h < CPS; ++h) {
      const int jj = jb + j, c = CPS * (cw + jj * DP) + h;
      const bool live = jj < J && c < nch;
      b.ch[j][h] = F::template at<CPS * DP>(F::lane(a, row, live ? c0 + c : c0), 0);
    }
}

// MFMA steps over one batch.  xl points at x[m][k] of this lane's slot-0
// chunk (LDS or global, m = lane & 15, or a valid row for m >= M); slot j's
// activations are CPS*DP*KPC elements further, chunk h of a slot h*KPC
// further.
//
// Output row m of the 16x16 tile depends only on activation row m, and
// column n only on weight row n.  Lanes of rows m >= M and of weight rows
// past N therefore feed whatever their (valid, in-bounds) addresses hold:
// their outputs are never stored.  Only dead chunks of the general path
// (outside the K slice) would reach stored outputs, so only they are zeroed.
// Every chunk is consumed, so no path leaves a batch load outstanding past
// its compute.
template <class F, int DP, int CPS, bool FULL, bool XP, class XPtr>
__device__ __forceinline__ void mfma_compute(const MfmaBatch<F, CPS>& b, XPtr xl, int jb, int J, int cw, int nch,
                                             f32x4_t& acc) {
#pragma unroll
  for (int j = 0; j < kNJ; ++j)
#pragma unroll
    for (int h = 0; h < CPS; ++h) {
      const bool live = FULL || (jb + j < J && CPS * (cw + (jb + j) * DP) + h < nch);   // uniform per 16 lanes
#pragma unroll
      for (int sub = 0; sub < F::SUB; ++sub) {
        uint32_t w[8];
        if constexpr (XP) F::deq16t(b.ch[j][h], sub, w);
        else F::deq16(b.ch[j][h], sub, w);
        uint4 wa = make_uint4(w[0], w[1], w[2], w[3]), wb = make_uint4(w[4], w[5], w[6], w[7]);
        uint4 xa, xb;
        if constexpr (FULL) {
          const uint4* xp = reinterpret_cast<const uint4*>(xl + (j * CPS * DP + h) * F::KPC + sub * 16);
          xa = xp[0];
          xb = xp[1];
        } else {
          xa = make_uint4(0, 0, 0, 0);
          xb = xa;
          if (live) {
            const uint4* xp = reinterpret_cast<const uint4*>(xl + (j * CPS * DP + h) * F::KPC + sub * 16);
            xa = xp[0];
            xb = xp[1];
          } else {
            wa = xa;
            wb = xa;
          }
        }
        acc = mfma16(xa, wa, acc);
        acc = mfma16(xb, wb, acc);
      }
    }
}

// Sum the KW waves' 16x16 tiles in wave order; the result is valid in wave 0
// (wave: the index within the tile's group of KW waves, red: the group's
// reduction buffer).  Every wave of the workgroup takes part in the barriers.
template <int KW>
__device__ __forceinline__ f32x4_t mfma_wave_reduce(f32x4_t acc, float* red, int wave) {
  const int lane = threadIdx.x & 63;
  if constexpr (KW == 1) return acc;
  if (wave > 0) reinterpret_cast<f32x4_t*>(red)[(wave - 1) * 64 + lane] = acc;
  lds_barrier();
  if (wave == 0) {
#pragma unroll
    for (int w = 1; w < KW; ++w) {
      const f32x4_t o = reinterpret_cast<const f32x4_t*>(red)[(w - 1) * 64 + lane];
      acc[0] += o[0]; acc[1] += o[1]; acc[2] += o[2]; acc[3] += o[3];
    }
  }
  lds_barrier();
  return acc;
}

// Activation rows in LDS are padded by 16 bytes so that the 16 rows of an
// MFMA fragment fall into different banks.
__host__ __device__ inline int mfma_xstride(int ks) { return ks + 8; }

// LDS layout: [x: M x xstride bf16 (XL only)] [red: G x (KW-1) x 64 x 4 fp32]
__host__ __device__ inline size_t mfma_lds_bytes(int M, int ks, int KW, bool xl, int G = 1) {
  size_t x = xl ? (size_t)M * mfma_xstride(ks) * 2 : 0;
  x = (x + 15) & ~(size_t)15;
  return x + (size_t)G * (KW > 1 ? KW - 1 : 0) * 64 * 16;
}

// Finish tile t: wave reduce, then the epilogue (ksplit == 1) or the split-K
// slot write and last-arrival reduction.
// With several tile groups per workgroup (ksplit == 1 only), wave is the index
// within the group and live is false for a group's padding round.
template <int KW, class Epi>
__device__ __forceinline__ void mfma_finish(const GemvLaunch& p, int b, int split, int t, f32x4_t acc, float* red,
                                            int wave, bool live) {
  const int lane = threadIdx.x & 63;
  const int n = lane & 15, g = lane >> 4;
  const int64_t row = (int64_t)t * 16 + n;
  const bool wrow = row < p.N && live;
  acc = mfma_wave_reduce<KW>(acc, red, wave);
  // lane of wave 0 holds D[m = g*4 + i][n]
  if (p.ksplit == 1) {
    if (wave == 0 && wrow) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (g * 4 + i < p.M) Epi::apply(p, b, g * 4 + i, row, acc[i] * p.gs);
    }
    return;
  }
  float* part = p.part + (int64_t)b * p.ksplit * 16 * p.N;
  if (wave == 0) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int m = g * 4 + i;
      if (m < p.M && wrow)
        __hip_atomic_store(part + ((int64_t)split * 16 + m) * p.N + row, acc[i] * p.gs, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  const int tiles = (p.N + 15) / 16;
  int* ticket = p.tickets + (int64_t)b * tiles + t;
  if (splitk_arrive(ticket, p.ksplit)) {
    const int64_t tile0 = (int64_t)t * 16;
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
        for (int jj = 0; jj < 8; ++jj) v[jj] = s0 + jj < p.ksplit ? ld_coherent(src + (s0 + jj) * sstride) : 0.0f;
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

// Activation staging in two halves around the weight batch loads: the first
// round's global loads (up to four 16-byte pieces per thread) go out before
// the weights, so that the wait for them before their LDS writes leaves the
// younger weight loads in flight (the wait counter counts in issue order).
// Rows of x and of the stage are 16-byte aligned (strides and k0 are
// multiples of 8 elements).
typedef uint32_t xs_u32x4 __attribute__((ext_vector_type(4)));
// XR: 16-byte pieces per thread in the first round (plain layout; the 4x4
// transposed layout takes XR / 2 blocks of two pieces).
template <int XR>
struct XStage {
  xs_u32x4 v[XR];
};
__device__ __forceinline__ xs_u32x4 xs_ld(const uint4* p) { return *reinterpret_cast<const xs_u32x4*>(p); }
__device__ __forceinline__ uint4 xs_u4(xs_u32x4 v) { return make_uint4(v.x, v.y, v.z, v.w); }
template <int XR>
__device__ __forceinline__ void mfma_xfirst_load(XStage<XR>& r, const uint16_t* xg, int64_t x_stride, int M, int k0,
                                                 int ks, bool t4) {
  const uint4* xg4 = reinterpret_cast<const uint4*>(xg + k0);
  const int64_t xrow4 = x_stride / 8;
  if (!t4) {
    const int per_row = ks / 8, total = M * per_row;
#pragma unroll
    for (int h = 0; h < XR; ++h) {
      const int i = threadIdx.x + h * blockDim.x, j = i < total ? i : total - 1;
      r.v[h] = xs_ld(xg4 + (j / per_row) * xrow4 + j % per_row);
    }
  } else {
    const int per_row = ks / 16, total = M * per_row;
#pragma unroll
    for (int h = 0; h < XR / 2; ++h) {
      const int i = threadIdx.x + h * blockDim.x, j = i < total ? i : total - 1;
      const int m = j / per_row, q = j - m * per_row;
      r.v[2 * h] = xs_ld(xg4 + m * xrow4 + 2 * q);
      r.v[2 * h + 1] = xs_ld(xg4 + m * xrow4 + 2 * q + 1);
    }
  }
}
__device__ __forceinline__ void mfma_x_t4_pack(uint4 a, uint4 b, uint4& o, uint4& r) {
  o.x = perm_b32(a.z, a.x, 0x05040100u);   // x0, x4
  o.y = perm_b32(b.z, b.x, 0x05040100u);   // x8, x12
  o.z = perm_b32(a.z, a.x, 0x07060302u);   // x1, x5
  o.w = perm_b32(b.z, b.x, 0x07060302u);   // x9, x13
  r.x = perm_b32(a.w, a.y, 0x05040100u);   // x2, x6
  r.y = perm_b32(b.w, b.y, 0x05040100u);   // x10, x14
  r.z = perm_b32(a.w, a.y, 0x07060302u);   // x3, x7
  r.w = perm_b32(b.w, b.y, 0x07060302u);   // x11, x15
}
// Store the first round, then stage the remaining rounds (loads and stores).
template <int XR>
__device__ __forceinline__ void mfma_xrest(const XStage<XR>& r, uint16_t* lds, const uint16_t* xg, int64_t x_stride,
                                           int M, int k0, int ks, int xs, bool t4) {
  const uint4* xg4 = reinterpret_cast<const uint4*>(xg + k0);
  const int64_t xrow4 = x_stride / 8;
  uint4* lds4 = reinterpret_cast<uint4*>(lds);
  const int lrow4 = xs / 8;
  if (!t4) {
    const int per_row = ks / 8, total = M * per_row;
#pragma unroll
    for (int h = 0; h < XR; ++h) {
      const int i = threadIdx.x + h * blockDim.x;
      if (i < total) lds4[(i / per_row) * lrow4 + i % per_row] = xs_u4(r.v[h]);
    }
    for (int i = threadIdx.x + XR * blockDim.x; i < total; i += blockDim.x)
      lds4[(i / per_row) * lrow4 + i % per_row] = xg4[(i / per_row) * xrow4 + i % per_row];
  } else {
    const int per_row = ks / 16, total = M * per_row;
#pragma unroll
    for (int h = 0; h < XR / 2; ++h) {
      const int i = threadIdx.x + h * blockDim.x;
      if (i < total) {
        const int m = i / per_row, q = i - m * per_row;
        uint4 o, rr;
        mfma_x_t4_pack(xs_u4(r.v[2 * h]), xs_u4(r.v[2 * h + 1]), o, rr);
        lds4[m * lrow4 + 2 * q] = o;
        lds4[m * lrow4 + 2 * q + 1] = rr;
      }
    }
    for (int i = threadIdx.x + (XR / 2) * blockDim.x; i < total; i += blockDim.x) {
      const int m = i / per_row, q = i - m * per_row;
      uint4 o, rr;
      mfma_x_t4_pack(xg4[m * xrow4 + 2 * q], xg4[m * xrow4 + 2 * q + 1], o, rr);
      lds4[m * lrow4 + 2 * q] = o;
      lds4[m * lrow4 + 2 * q + 1] = rr;
    }
  }
}

// Work items are (batch entry, 16-row tile) pairs, numbered entry-major;
// workgroup x of K slice y takes items [x * per_wg, (x + 1) * per_wg).  The
// host sizes per_wg so that every workgroup of the launch is resident at once
// and all carry the same number of items.  The activations of an entry are
// staged once per run of items of that entry.  p.J: chunks per lane per
// tile (slots), p.nb: register batches per tile.
//
// G > 1 (single matrix, ksplit == 1): the workgroup's waves form G groups of
// KW that work on G items at once, sharing one activation stage: for large
// M * K the stage limits a CU to one workgroup, whose tiles would otherwise
// run one after another, each with its memory latency exposed.  Every group
// runs the same number of rounds; a round past the workgroup's items
// recomputes its last item and stores nothing.
template <class F, int KW, int CPS, bool FULL, bool XL, class Epi, int G = 1>
__global__ __launch_bounds__(64 * KW * G) void gemv_mfma_kernel(GemvLaunch p) {
  constexpr int DP = 4 * KW;                // slots between a lane's consecutive slots
  constexpr int NJ = kNJ;
  extern __shared__ __align__(16) uint16_t lds[];
  const int split = blockIdx.y;
  const int lane = threadIdx.x & 63, wave_all = threadIdx.x >> 6;
  const int grp = G > 1 ? wave_all / KW : 0, wave = wave_all - grp * KW;
  const int n = lane & 15, g = lane >> 4;
  const int tiles = (p.N + 15) / 16, items = p.batch * tiles;
  const int it0 = blockIdx.x * p.per_wg;
  const int iend = it0 + p.per_wg < items ? it0 + p.per_wg : items;
  if (it0 >= iend) return;
  const int ks = p.pa.K / p.ksplit, k0 = split * ks, nch = ks / F::KPC, c0 = k0 / F::KPC;
  const int cw = wave * 4 + g;              // this lane's first slot within the slice
  const int J = p.J, nb = p.nb;
  const int xs = mfma_xstride(ks);
  const size_t xbytes = XL ? (((size_t)p.M * xs * 2 + 15) & ~(size_t)15) : 0;
  float* red = reinterpret_cast<float*>(reinterpret_cast<char*>(lds) + xbytes) + grp * (KW > 1 ? KW - 1 : 0) * 256;
  const bool xon = n < p.M;
  const int xrow = xon ? n : 0;
  int cur_b = -1;
  for (int it = it0 + grp; it - grp < iend; it += G) {
    const bool live = it < iend;
    const int itc = live ? it : iend - 1;
    const int b = itc / tiles, t = itc - b * tiles;
    PlaneArgs pa = p.pa;
    pa.w0 += b * p.w0_bstride;
    if (pa.w1) pa.w1 += b * p.w1_bstride;
    pa.s += b * p.s_bstride;
    const int64_t row = (int64_t)t * 16 + n;
    const int64_t rowc = row < p.N ? row : p.N - 1;     // rows past N read row N-1 (in bounds) as zeros
    const uint16_t* xg = p.x + b * p.x_bstride;
    const uint16_t* xl0 = XL ? lds + xrow * xs + CPS * cw * F::KPC : xg + xrow * p.x_stride + k0 + CPS * cw * F::KPC;
    f32x4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
    // The activations' first round of loads goes out ahead of the first weight
    // batch of every item (unconditionally: a load under a branch would be
    // waited for at the branch's join), and is written to LDS, for a new batch
    // entry, while the weights are in flight.
    {
      // first-round pieces per thread: 12 with tile groups (chosen for large
      // activation stages: M = 16, K = 2560 in one round of 8 waves), else 4
      XStage<(G > 1 ? 12 : 4)> xr;
      if constexpr (XL) {
        mfma_xfirst_load(xr, xg, p.x_stride, p.M, k0, ks, HasXPerm<F>::value);
        asm volatile("" ::: "memory");                  // keep the issue order: activations, then weights
      }
      MfmaBatch<F, CPS> A;
      if constexpr (FULL) mfma_load_full<F, DP, CPS>(A, F::lane(pa, rowc, c0 + CPS * cw));
      else mfma_load_general<F, DP, CPS>(A, pa, rowc, c0, cw, 0, J, nch);
      if constexpr (XL) {
        if (b != cur_b) {
          if (cur_b >= 0) __syncthreads();               // every wave is done with the previous entry's x
          mfma_xrest(xr, lds, xg, p.x_stride, p.M, k0, ks, xs, HasXPerm<F>::value);
          __syncthreads();
          cur_b = b;
        }
      }
      mfma_compute<F, DP, CPS, FULL, XL && HasXPerm<F>::value>(A, xl0, 0, J, cw, nch, acc);
    }
    for (int bi = 1; bi < nb; ++bi) {
      MfmaBatch<F, CPS> A;
      if constexpr (FULL) mfma_load_full<F, DP, CPS>(A, F::lane(pa, rowc, c0 + CPS * (cw + bi * NJ * DP)));
      else mfma_load_general<F, DP, CPS>(A, pa, rowc, c0, cw, bi * NJ, J, nch);
      mfma_compute<F, DP, CPS, FULL, XL && HasXPerm<F>::value>(A, xl0 + bi * NJ * CPS * DP * F::KPC, bi * NJ, J, cw,
                                                                nch, acc);
    }
    mfma_finish<KW, Epi>(p, b, split, t, acc, red, wave, live);
  }
}

// Compute units of the current device (cached).
int device_cus();
// Optional cap on resident waves per CU from FP4X_WAVES_PER_CU (0: none).
int waves_per_cu_cap();

template <class F, int KW, int CPS, bool FULL, bool XL, class Epi, int G = 1>
void launch_mfma_kw(GemvLaunch p, int batch, size_t lds, hipStream_t st) {
  auto kern = gemv_mfma_kernel<F, KW, CPS, FULL, XL, Epi, G>;
  // resident workgroups per CU for this kernel and LDS size (cached per LDS size)
  static int occ_cache[97];
  const int key = (int)((lds + 1023) / 1024);
  int occ = key < 97 ? occ_cache[key] : 0;
  if (occ <= 0) {
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, reinterpret_cast<const void*>(kern), 64 * KW * G, lds) !=
            hipSuccess || occ < 1)
      occ = 1;
    if (key < 97) occ_cache[key] = occ;
  }
  const int cap = waves_per_cu_cap();
  if (cap > 0 && occ * KW * G > cap) occ = cap / (KW * G) > 0 ? cap / (KW * G) : 1;
  const int tiles = (p.N + 15) / 16;
  const int64_t items = (int64_t)batch * tiles;
  int64_t slots = (int64_t)device_cus() * occ / p.ksplit;
  if (slots < 1) slots = 1;
  const int64_t per = (items + slots - 1) / slots;
  p.batch = batch;
  p.per_wg = (int)per;
  const int gx = (int)((items + per - 1) / per);
  hipLaunchKernelGGL(kern, dim3(gx, p.ksplit, 1), dim3(64 * KW * G), lds, st, p);
}

// Tile groups (see gemv_mfma_kernel): single matrix, ksplit == 1, full slots,
// single chunks, activations staged in LDS.
// At most 8 waves per workgroup (KW * G <= 8): 16-wave groupings spill.
template <class F, class Epi>
void launch_mfma_grouped(const GemvLaunch& p, int KW, int G, size_t lds, hipStream_t st) {
  if (G == 4) {
    if (KW == 1) launch_mfma_kw<F, 1, 1, true, true, Epi, 4>(p, 1, lds, st);
    else launch_mfma_kw<F, 2, 1, true, true, Epi, 4>(p, 1, lds, st);
  } else {
    if (KW == 1) launch_mfma_kw<F, 1, 1, true, true, Epi, 2>(p, 1, lds, st);
    else if (KW == 2) launch_mfma_kw<F, 2, 1, true, true, Epi, 2>(p, 1, lds, st);
    else launch_mfma_kw<F, 4, 1, true, true, Epi, 2>(p, 1, lds, st);
  }
}

template <class F, int KW, int CPS, bool FULL, class Epi>
void launch_mfma_xl(const GemvLaunch& p, int batch, size_t lds, bool xl, hipStream_t st) {
  if (xl) launch_mfma_kw<F, KW, CPS, FULL, true, Epi>(p, batch, lds, st);
  else launch_mfma_kw<F, KW, CPS, FULL, false, Epi>(p, batch, lds, st);
}

template <class F, int CPS, class Epi>
void launch_mfma_full(const GemvLaunch& p, int KW, int batch, size_t lds, bool xl, hipStream_t st) {
  switch (KW) {
    case 1: launch_mfma_xl<F, 1, CPS, true, Epi>(p, batch, lds, xl, st); break;
    case 2: launch_mfma_xl<F, 2, CPS, true, Epi>(p, batch, lds, xl, st); break;
    case 4: launch_mfma_xl<F, 4, CPS, true, Epi>(p, batch, lds, xl, st); break;
    default: launch_mfma_xl<F, 8, CPS, true, Epi>(p, batch, lds, xl, st); break;
  }
}

// Pair loads of the full path read 16-byte main-plane pieces and
// F::AUX_ALIGN-byte scale pieces: every plane base (and batch stride) must
// allow them, else the general path runs.
template <class F>
bool mfma_pair_aligned(const GemvLaunch& p, int batch) {
  auto al = [](const void* q, int n) { return (reinterpret_cast<uintptr_t>(q) & (uintptr_t)(n - 1)) == 0; };
  bool ok = al(p.pa.w0, 16) && al(p.pa.s, F::AUX_ALIGN) && (!p.pa.w1 || al(p.pa.w1, 16));
  if (batch > 1)
    ok = ok && p.w0_bstride % 16 == 0 && p.s_bstride % F::AUX_ALIGN == 0 && (!p.pa.w1 || p.w1_bstride % 16 == 0);
  return ok;
}

template <class F, class Epi>
int launch_gemv_mfma(const GemvLaunch& p0, int batch, hipStream_t st) {
  GemvLaunch p = p0;
  const int ks = p.pa.K / p.ksplit;
  const int chunks = ks / F::KPC;
  const int cps = mfma_cps<F>(chunks) == 2 && mfma_pair_aligned<F>(p, batch) ? 2 : 1;
  int KW = mfma_kw(chunks, cps);
  const bool full = mfma_full(chunks, KW, cps);
  if (!full) KW = kMaxKW;                               // general path (single chunks): one instantiation
  const int cpsu = full ? cps : 1;
  p.J = ((chunks + cpsu - 1) / cpsu + 4 * KW - 1) / (4 * KW);
  p.nb = (p.J + kNJ - 1) / kNJ;
  const bool xl = mfma_lds_bytes(p.M, ks, KW, true) <= 96 * 1024;
  // Tile groups when the activation stage leaves room for one workgroup per
  // CU and the tiles outnumber the CUs: G tiles at once, G <= 4, KW * G <= 8.
  int G = 1;
  if (full && xl && cps == 1 && batch == 1 && p.ksplit == 1 && mfma_lds_bytes(p.M, ks, KW, true) > 80 * 1024) {
    const int64_t tiles = (p.N + 15) / 16, cus = device_cus();
    const int64_t per_cu = (tiles + cus - 1) / cus;
    while (G < 4 && 2 * G <= per_cu && KW * 2 * G <= 8 && mfma_lds_bytes(p.M, ks, KW, true, 2 * G) <= 160 * 1024)
      G *= 2;
  }
  const size_t lds = mfma_lds_bytes(p.M, ks, KW, xl, G);
  if (G > 1) {
    launch_mfma_grouped<F, Epi>(p, KW, G, lds, st);
    return check_launch("gemv_mfma");
  }
  if (!full) launch_mfma_xl<F, kMaxKW, 1, false, Epi>(p, batch, lds, xl, st);
  else if constexpr (MfmaTune<F>::PAIRS) {
    if (cps == 2) launch_mfma_full<F, 2, Epi>(p, KW, batch, lds, xl, st);
    else launch_mfma_full<F, 1, Epi>(p, KW, batch, lds, xl, st);
  } else {
    launch_mfma_full<F, 1, Epi>(p, KW, batch, lds, xl, st);
  }
  return check_launch("gemv_mfma");
}

}  // namespace fp4x
