// Streaming W8 g64 GEMV for long runs of 16-row tiles (the layer-batched
// router gates: many independent [N, K] int8 matrices, one launch).
//
// y[m, n] = sum_k x[m, k] * bf16(q[n, k] * s[n, k / 64]), fp32 accumulation,
// the semantics of the plugin's _w8 kernel (x/fp4x_kernels.py:116-135).
//
// Design (one workgroup per CU, every tile of the launch in one pass):
//   * A workgroup runs T tile slots x KW waves.  The KW waves of a slot split
//     the K range of their 16-row tile into KW contiguous parts; a part is a
//     sequence of "units" of 128 bytes of each of the 16 rows.
//   * Each wave streams its units through a private ring of D unit buffers in
//     LDS, filled by direct global->LDS loads (global_load_lds_dwordx4 /
//     _dword, which need no registers): per unit two 16-byte loads per lane
//     (8 rows x one full 128-byte line each) and one 4-byte load per lane for
//     the unit's group scales.  The wave waits on its own load counter for the
//     oldest unit, computes it, and refills that buffer with the unit D ahead,
//     so about D units per wave are always in flight while it computes.
//   * All LDS accesses after the first direct load are inline assembly: the
//     compiler cannot tell the ring from other LDS data and would otherwise
//     wait for every outstanding direct load before each LDS access.  Each
//     asm read block ends with its own LDS wait, so no use of a loaded
//     register can be scheduled before the data arrives.  vmcnt waits count
//     at most the loads issued after the awaited unit, so stores or other
//     memory operations in between only make a wait stricter.
//   * Dequant: v_cvt_f32_i32 with a sign-extended byte select (SDWA), the fp32
//     product q * s (the reference's rounding), packed to bf16 with RNE; MFMA
//     v_mfma_f32_16x16x32_bf16 accumulates one tile part per wave.
//   * The KW parts of a tile are summed in part order through LDS, then stored.
//   * The activations of the one or two batch entries a workgroup touches
//     are staged once into LDS by direct loads of 1 KB rows pieces.
#pragma once
#include <cstdlib>
#include "fp4x_mfma.h"

namespace fp4x {

typedef __attribute__((address_space(3))) void* lds_ptr_t;

__device__ __forceinline__ uint32_t lds_addr(const void* p) { return (uint32_t)(uintptr_t)(lds_ptr_t)p; }

// Direct global -> LDS loads: lane l writes its bytes at l * size from the
// (wave-uniform) LDS address.
__device__ __forceinline__ void dma_b128(const void* g, void* l) {
  __builtin_amdgcn_global_load_lds(g, (lds_ptr_t)l, 16, 0, 0);
}
__device__ __forceinline__ void dma_b32(const void* g, void* l) {
  __builtin_amdgcn_global_load_lds(g, (lds_ptr_t)l, 4, 0, 0);
}

// Wait until at most N vector memory operations of this wave are outstanding.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
// Workgroup barrier without a memory fence (LDS data is waited for by the
// asm blocks that produce it).
__device__ __forceinline__ void wg_barrier_raw() { asm volatile("s_barrier" ::: "memory"); }

__device__ __forceinline__ void lds_put_f32x4(uint32_t a, f32x4_t v) {
  asm volatile("ds_write_b128 %0, %1\n\ts_waitcnt lgkmcnt(0)" ::"v"(a), "v"(v) : "memory");
}

// acc += the N partial sums at LDS byte addresses a + 1024 h (h = 0 .. N - 1),
// added in h order.  The reads are ordinary LDS loads, so every one issues
// before the first add waits (one LDS round trip, not N).
template <int N>
__device__ __forceinline__ void lds_add_parts(uint32_t a, f32x4_t& acc) {
  typedef const __attribute__((address_space(3))) f32x4_t* lds_f32x4_ptr;
  f32x4_t o[N];
#pragma unroll
  for (int h = 0; h < N; ++h) o[h] = *reinterpret_cast<lds_f32x4_ptr>((uintptr_t)(a + h * 1024));
#pragma unroll
  for (int h = 0; h < N; ++h) {
    acc[0] += o[h][0]; acc[1] += o[h][1]; acc[2] += o[h][2]; acc[3] += o[h][3];
  }
}

// One unit's operands for lane (n, g): weight chunks g and g + 4 of row n (at
// wa, wb), the two scale dwords (sa, sa + 64), and the activations of both
// chunks (xa: 32 bytes of chunk g; chunk g + 4 is 128 bytes further).
__device__ __forceinline__ void stream_read_unit(uint32_t wa, uint32_t wb, uint32_t sa, uint32_t xa, uint4& q0,
                                                 uint4& q1, uint32_t& s0, uint32_t& s1, uint4& x0a, uint4& x0b,
                                                 uint4& x1a, uint4& x1b) {
  asm volatile(
      "ds_read_b128 %0, %8\n\t"
      "ds_read_b128 %1, %9\n\t"
      "ds_read_b32 %2, %10\n\t"
      "ds_read_b32 %3, %10 offset:64\n\t"
      "ds_read_b128 %4, %11\n\t"
      "ds_read_b128 %5, %11 offset:16\n\t"
      "ds_read_b128 %6, %11 offset:128\n\t"
      "ds_read_b128 %7, %11 offset:144\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(q0), "=&v"(q1), "=&v"(s0), "=&v"(s1), "=&v"(x0a), "=&v"(x0b), "=&v"(x1a), "=&v"(x1b)
      : "v"(wa), "v"(wb), "v"(sa), "v"(xa)
      : "memory");
}

// bf16(q * s) for 16 int8 weights; q * s is the fp32 product, then RNE.
__device__ __forceinline__ uint32_t w8_pair_bf16(uint32_t d, int sh, float s) {
  const float a = (float)(int8_t)(d >> sh), b = (float)(int8_t)(d >> (sh + 8));
  return pack_bf16x2(a * s, b * s);
}
__device__ __forceinline__ void w8_chunk_bf16(uint4 q, float s, uint32_t (&w)[8]) {
  w[0] = w8_pair_bf16(q.x, 0, s); w[1] = w8_pair_bf16(q.x, 16, s);
  w[2] = w8_pair_bf16(q.y, 0, s); w[3] = w8_pair_bf16(q.y, 16, s);
  w[4] = w8_pair_bf16(q.z, 0, s); w[5] = w8_pair_bf16(q.z, 16, s);
  w[6] = w8_pair_bf16(q.w, 0, s); w[7] = w8_pair_bf16(q.w, 16, s);
}

constexpr int kStreamUnit = 2048 + 256;     // LDS bytes of one unit: 16 rows x 128 B + scale dwords

// Geometry shared by host and device.
struct StreamGeom {
  int T, KW, D;
  __host__ __device__ static int xrow_bytes(int K) { return mfma_xstride(K) * 2; }
  __host__ __device__ static int xbuf_bytes(int M, int K) { return (M * xrow_bytes(K) + 15) & ~15; }
};

template <bool F16S, int T, int KW, int D, class Epi>
__global__ __launch_bounds__(64 * T * KW) void w8_stream_kernel(GemvLaunch p) {
  constexpr int NW = T * KW;
  extern __shared__ __align__(16) uint16_t lds[];
  char* base = reinterpret_cast<char*>(lds);
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int slot = wave / KW, part = wave - slot * KW;
  const int n = lane & 15, g = lane >> 4;
  const int tiles = (p.N + 15) / 16, items = p.batch * tiles;
  const int K = p.pa.K, JW = K / 128 / KW;           // units per wave per tile
  const int xrow = StreamGeom::xrow_bytes(K), xbuf = StreamGeom::xbuf_bytes(p.M, K);
  const int wg0 = blockIdx.x * p.per_wg;
  const int wgend = wg0 + p.per_wg < items ? wg0 + p.per_wg : items;
  if (wg0 >= wgend) return;
  const int R = (wgend - wg0 + T - 1) / T;           // rounds of T tiles
  const int b0 = wg0 / tiles, nbuf = (wgend - 1) / tiles - b0 + 1;
  char* part_base = base + p.xbufs * xbuf;
  char* ring = part_base + T * (KW - 1) * 1024 + wave * D * kStreamUnit;

  // Activations of the workgroup's batch entries: 1 KB pieces of each row.
  const int bpr = K * 2 / 1024, nblk = nbuf * p.M * bpr;
  for (int i = wave; i < nblk; i += NW) {
    const int bi = i / (p.M * bpr), r = i - bi * (p.M * bpr), m = r / bpr, blk = r - m * bpr;
    const uint16_t* xg = p.x + (int64_t)(b0 + bi) * p.x_bstride + (int64_t)m * p.x_stride + blk * 512 + lane * 8;
    dma_b128(xg, base + bi * xbuf + m * xrow + blk * 1024);
  }

  // DMA lane l of weight load h reads row 8h + (l >> 3) of the tile, chunk
  // (l & 7) ^ (row >> 1) of the unit: 8 lanes cover one 128-byte line, and the
  // XOR makes the 16 lanes of a quarter-wave read 16 different LDS bank
  // groups when the operands are read back.
  const int dr = lane >> 3, dc = lane & 7;
  const int cA = dc ^ (dr >> 1), cB = dc ^ (4 + (dr >> 1));
  // Scale lane: fp32, row n, group 2j + ((l >> 4) & 1); fp16, row n, the
  // dword holding groups 2j and 2j + 1.
  const int sg = F16S ? 0 : (lane >> 4) & 1;
  const int U = R * JW;
  int ir = 0, ij = 0, is = 0, issued = 0;
  const uint8_t* iw = nullptr;
  const uint8_t* isb = nullptr;
  uint32_t o0 = 0, o1 = 0, os = 0;
  auto set_tile = [&](int rr) {
    int it = wg0 + rr * T + slot;
    if (it >= wgend) it = wgend - 1;                 // idle slot of the last round: reload a valid tile
    const int b = it / tiles, t = it - b * tiles;
    const int lim = p.N - 1 - t * 16;                // rows past N read row N - 1
    iw = p.pa.w0 + b * p.w0_bstride + (int64_t)t * 16 * K + part * JW * 128;
    isb = p.pa.s + b * p.s_bstride + ((int64_t)t * 16 * (K / 64) + part * JW * 2) * (F16S ? 2 : 4);
    const int rA = dr < lim ? dr : lim, rB = dr + 8 < lim ? dr + 8 : lim, rS = n < lim ? n : lim;
    o0 = (uint32_t)(rA * K + cA * 16);
    o1 = (uint32_t)(rB * K + cB * 16);
    os = (uint32_t)((rS * (K / 64) + sg) * (F16S ? 2 : 4));
  };
  set_tile(0);
  auto issue_next = [&]() {
    char* l = ring + is * kStreamUnit;
    const uint8_t* u0 = iw + ij * 128;
    dma_b128(u0 + o0, l);
    dma_b128(u0 + o1, l + 1024);
    dma_b32(isb + ij * (F16S ? 4 : 8) + os, l + 2048);
    if (++is == D) is = 0;
    ++issued;
    if (++ij == JW) {
      ij = 0;
      if (++ir < R) set_tile(ir);
    }
  };
  const int pro = U < D ? U : D;
  for (int u = 0; u < pro; ++u) issue_next();
  // the activation loads went out first: wait for them only
  if (pro == D) wait_vmcnt<3 * D>();
  else wait_vmcnt<0>();
  wg_barrier_raw();

  const int xr = n < p.M ? n : 0;                    // rows m >= M: never stored
  const uint32_t rl = lds_addr(ring);
  const uint32_t wlA = rl + n * 128 + ((g ^ (n >> 1)) * 16), wlB = rl + n * 128 + (((g + 4) ^ (n >> 1)) * 16);
  const uint32_t sl = rl + 2048 + n * 4;
  const uint32_t pl = lds_addr(part_base) + slot * (KW - 1) * 1024 + lane * 16;
  int cs = 0, u = 0;
  for (int r = 0; r < R; ++r) {
    const int it = wg0 + r * T + slot;
    const int itc = it < wgend ? it : wgend - 1;
    const int b = itc / tiles, t = itc - b * tiles;
    const uint32_t xl = lds_addr(base + (b - b0) * xbuf) + xr * xrow + part * JW * 256 + g * 32;
    f32x4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int j = 0; j < JW; ++j, ++u) {
      if (issued - 1 - u >= D - 1) wait_vmcnt<3 * (D - 1)>();
      else wait_vmcnt<0>();
      uint4 q0, q1, x0a, x0b, x1a, x1b;
      uint32_t s0, s1;
      const uint32_t so = cs * kStreamUnit;
      stream_read_unit(wlA + so, wlB + so, sl + so, xl + j * 256, q0, q1, s0, s1, x0a, x0b, x1a, x1b);
      float sc0, sc1;
      if constexpr (F16S) {
        sc0 = f16_to_f32((uint16_t)s0);
        sc1 = f16_to_f32((uint16_t)(s0 >> 16));
      } else {
        sc0 = __uint_as_float(s0);
        sc1 = __uint_as_float(s1);
      }
      uint32_t w[8];
      w8_chunk_bf16(q0, sc0, w);
      acc = mfma16(x0a, make_uint4(w[0], w[1], w[2], w[3]), acc);
      acc = mfma16(x0b, make_uint4(w[4], w[5], w[6], w[7]), acc);
      w8_chunk_bf16(q1, sc1, w);
      acc = mfma16(x1a, make_uint4(w[0], w[1], w[2], w[3]), acc);
      acc = mfma16(x1b, make_uint4(w[4], w[5], w[6], w[7]), acc);
      if (++cs == D) cs = 0;
      if (issued < U) issue_next();
    }
    if constexpr (KW > 1) {
      if (part > 0) lds_put_f32x4(pl + (part - 1) * 1024, acc);
      wg_barrier_raw();
      if (part == 0) lds_add_parts<KW - 1>(pl, acc);
      wg_barrier_raw();
    }
    if (part == 0 && it < wgend) {
      const int64_t row = (int64_t)t * 16 + n;       // lane (n, g) holds D[m = 4g + i][n]
      if (row < p.N) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (g * 4 + i < p.M) Epi::apply(p, b, g * 4 + i, row, acc[i] * p.gs);
      }
    }
  }
}

// The activations of one unit for lane (n, g): 32 bytes of chunk g and 32 of
// chunk g + 4 (128 bytes further).
__device__ __forceinline__ void stream_read_x(uint32_t xa, uint4& x0a, uint4& x0b, uint4& x1a, uint4& x1b) {
  asm volatile(
      "ds_read_b128 %0, %4\n\t"
      "ds_read_b128 %1, %4 offset:16\n\t"
      "ds_read_b128 %2, %4 offset:128\n\t"
      "ds_read_b128 %3, %4 offset:144\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(x0a), "=&v"(x0b), "=&v"(x1a), "=&v"(x1b)
      : "v"(xa)
      : "memory");
}

// Split-K W8 GEMV of few 16-row tiles (the mixer's down projection, N = 640,
// K = 10240): C workgroups per tile, each of WPG waves owning JW units of 128
// K values (so C = K / (128 * WPG * JW)), which spreads a 40-tile matrix over
// C x 40 CUs.  A CU streams only some 20 GB/s of its own, so the CU count, not
// the depth of one CU's queue, bounds a GEMV this small.
//   * Every wave issues its weight and scale loads (lane (n, g): chunks g and
//     g + 4 of row n per unit, and the unit's scale dword) right after the
//     workgroup's activation slice, waits once, and computes from registers.
//   * The WPG wave parts are summed in wave order through LDS; wave 0 stores
//     the workgroup's [M x 16] partial to slot c of the tile with agent-scope
//     (device-coherent) stores, waits for them to complete, and takes a ticket
//     on the tile; the workgroup drawing ticket C - 1 reads the C slots with
//     agent-scope loads, sums them in slot order (so the result does not
//     depend on arrival order), runs the epilogue and re-arms the ticket.
//     Ordering comes from the explicit completion wait between the slot
//     stores and the ticket, and from the loads depending on the ticket value;
//     no cache-wide write-back or invalidate is needed because every access to
//     the slots and the ticket is device-coherent.
//
// XCD-local slots (LOCAL, the single-launch mixer): when the caller places
// every item of a tile on one XCD (workgroups whose indices are congruent
// mod 8: the dispatcher hands consecutive workgroups to the XCDs in turn), the
// partials are stored plainly, with no completion wait and no ticket (their
// lines stay within the XCD that reads them).  The tile's closer is
// its last part (c = C - 1, the highest workgroup index of the tile, so every
// other part was dispatched before it and none of them waits on anything).
// Parts c < C - 1 store their [M x 16] partials as 64-bit (value, tag) pairs,
// each pair in one store, and end; the tag is the complement of the call's
// count, which every workgroup of every call counts in a word of its own
// (*call_count).  The closer reads the pairs until every
// tag is its call's (back to back, at most spin_limit reads: the
// caller's flag limit, but never under 65,536), adds them in slot order with its
// own partial last and runs the epilogue.  That replaces the
// slot stores' completion wait, the device-scope ticket and a separate read
// of the slots (the served mixer 9.43 -> 9.06 us, the 640-row one 11.91 ->
// 11.83).  A closer whose reads reach spin_limit (a part that ran on
// another XCD, so its pairs are in another L2, or one that never got a CU)
// writes NaN for the tile and sets bit 1 of *status; the next call starts
// clean.
struct SplitLocal {
  uint64_t* pairs;     // [tiles][C][M][16] (partial, tag) pairs
  int* status;
  int spin_limit;      // the closer's reads of the other parts' pairs before it gives up
};

// Seven (value, tag) pairs, device-scope loads (sc1), all issued before one
// wait.  Measured on the mixer: workgroup-scope (sc0) loads kept returning the
// first value a CU had read, even after a vector L1 invalidate, so the
// closer never saw a late part; atomic ORs of zero saw it but made the mixer
// 0.8-1.5 us slower; these loads see it and cost least.  A pair counts only
// when its tag is this call's, whatever path its line took.
__device__ __forceinline__ void read_pairs_7(const uint64_t* const (&a)[7], uint64_t (&v)[7]) {
  asm volatile(
      "global_load_dwordx2 %0, %7, off sc1\n\t"
      "global_load_dwordx2 %1, %8, off sc1\n\t"
      "global_load_dwordx2 %2, %9, off sc1\n\t"
      "global_load_dwordx2 %3, %10, off sc1\n\t"
      "global_load_dwordx2 %4, %11, off sc1\n\t"
      "global_load_dwordx2 %5, %12, off sc1\n\t"
      "global_load_dwordx2 %6, %13, off sc1\n\t"
      "s_waitcnt vmcnt(0)"
      : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), "=&v"(v[3]), "=&v"(v[4]), "=&v"(v[5]), "=&v"(v[6])
      : "v"(a[0]), "v"(a[1]), "v"(a[2]), "v"(a[3]), "v"(a[4]), "v"(a[5]), "v"(a[6])
      : "memory");
}

// w8_splitk_item runs one (tile t, part c) item with the workgroup's WPG waves
// and LDS at base; it returns true in the wave that ran the tile's epilogue
// (wave 0 of the last-arriving workgroup), false elsewhere.
template <bool F16S, int WPG, int JW, class Epi, bool LOCAL = false>
__device__ __forceinline__ bool w8_splitk_item(const GemvLaunch& p, int C, int t, int c, char* base,
                                               const SplitLocal& loc = SplitLocal{}, const int* call_count = nullptr) {
  constexpr int UW = WPG * JW;                       // units per workgroup
  constexpr int XR = UW * 256 + 64;                  // LDS bytes per activation row
  static_assert(UW % 4 == 0, "activation slice in whole 1 KB pieces");
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n = lane & 15, g = lane >> 4;
  const int K = p.pa.K;
  char* part_base = base + ((p.M * XR + 15) & ~15);

  // activation slice [M, c * UW * 128, + UW * 128): 1 KB pieces
  constexpr int PPR = UW / 4;                        // pieces per row
  for (int i = wave; i < p.M * PPR; i += WPG) {
    const int m = i / PPR, u = i - m * PPR;
    dma_b128(p.x + (int64_t)m * p.x_stride + (int64_t)(c * UW + u * 4) * 128 + lane * 8, base + m * XR + u * 1024);
  }
  const int lim = p.N - 1 - t * 16;                  // rows past N read row N - 1
  const int64_t row = (int64_t)t * 16 + (n < lim ? n : lim);
  const int u0 = c * UW + wave * JW;
  const uint8_t* wr = p.pa.w0 + row * K + u0 * 128 + g * 16;
  const uint8_t* sr = p.pa.s + (row * (K / 64) + u0 * 2) * (F16S ? 2 : 4);
  typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
  u32x4_t qa[JW], qb[JW];
  uint32_t sa[JW], sb[JW];
#pragma unroll
  for (int j = 0; j < JW; ++j) {
    qa[j] = *reinterpret_cast<const u32x4_t*>(wr + j * 128);
    qb[j] = *reinterpret_cast<const u32x4_t*>(wr + j * 128 + 64);
    if constexpr (F16S) {
      sa[j] = *reinterpret_cast<const uint32_t*>(sr + j * 4);
      sb[j] = 0;
    } else {
      sa[j] = *reinterpret_cast<const uint32_t*>(sr + j * 8);
      sb[j] = *reinterpret_cast<const uint32_t*>(sr + j * 8 + 4);
    }
  }
  wait_vmcnt<0>();
  wg_barrier_raw();

  const int xr = n < p.M ? n : 0;                    // rows m >= M: never stored
  const uint32_t xl = lds_addr(base) + xr * XR + wave * JW * 256 + g * 32;
  f32x4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int j = 0; j < JW; ++j) {
    uint4 x0a, x0b, x1a, x1b;
    stream_read_x(xl + j * 256, x0a, x0b, x1a, x1b);
    float sc0, sc1;
    if constexpr (F16S) {
      sc0 = f16_to_f32((uint16_t)sa[j]);
      sc1 = f16_to_f32((uint16_t)(sa[j] >> 16));
    } else {
      sc0 = __uint_as_float(sa[j]);
      sc1 = __uint_as_float(sb[j]);
    }
    uint32_t w[8];
    w8_chunk_bf16(make_uint4(qa[j].x, qa[j].y, qa[j].z, qa[j].w), sc0, w);
    acc = mfma16(x0a, make_uint4(w[0], w[1], w[2], w[3]), acc);
    acc = mfma16(x0b, make_uint4(w[4], w[5], w[6], w[7]), acc);
    w8_chunk_bf16(make_uint4(qb[j].x, qb[j].y, qb[j].z, qb[j].w), sc1, w);
    acc = mfma16(x1a, make_uint4(w[0], w[1], w[2], w[3]), acc);
    acc = mfma16(x1b, make_uint4(w[4], w[5], w[6], w[7]), acc);
  }
  if constexpr (WPG > 1) {
    const uint32_t pl = lds_addr(part_base) + lane * 16;
    if (wave > 0) lds_put_f32x4(pl + (wave - 1) * 1024, acc);
    wg_barrier_raw();
    if (wave > 0) return false;
    lds_add_parts<WPG - 1>(pl, acc);
  }
  // wave 0: slot c of tile t holds [M][16] fp32 partials
  float* slots = p.part + (int64_t)t * C * p.M * 16;
  if constexpr (LOCAL) {
    // slot c of tile t: [M][16] 64-bit pairs (partial bits, tag), each
    // stored in one single-copy-atomic store; the tag is the complement of
    // the call's count (*call_count, in LDS, one more every call on every
    // workgroup of the grid), so no pair of an earlier call, whatever its
    // shape, and no zero word passes for this call's (and, as a float, it is
    // a negative NaN pattern, which no float slot of the two-launch path
    // holds).  The closer is the tile's last part, which reads the others'
    // pairs until every tag is this call's and adds its own partial last
    // (slot order)
    const uint32_t tag = ~(uint32_t)__builtin_amdgcn_readfirstlane(*call_count);
    uint64_t* pairs = loc.pairs + (int64_t)t * C * p.M * 16;
    if (c != C - 1) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (g * 4 + i < p.M)
          __hip_atomic_store(pairs + (c * p.M + g * 4 + i) * 16 + n,
                             ((uint64_t)tag << 32) | __float_as_uint(acc[i]), __ATOMIC_RELAXED,
                             __HIP_MEMORY_SCOPE_WORKGROUP);
      return false;
    }
    bool ok = true;
    for (int e0 = 0; e0 < p.M * 16; e0 += 64) {
      const int e = e0 + lane;
      const int ec = e < p.M * 16 ? e : 0, m = ec >> 4, nn = ec & 15;
      // this part's own partial of element ec: lane nn + 16 (m >> 2), component m & 3
      const int src = (nn + 16 * (m >> 2)) << 2;
      float own = 0.0f;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float v = __int_as_float(__builtin_amdgcn_ds_bpermute(src, __float_as_int(acc[i])));
        if ((m & 3) == i) own = v;
      }
      const uint64_t* a[7];
#pragma unroll
      for (int cc = 0; cc < 7; ++cc) a[cc] = pairs + ((cc < C - 1 ? cc : 0) * p.M + m) * 16 + nn;
      uint64_t v[7] = {0, 0, 0, 0, 0, 0, 0};
      for (int it = 0;; ++it) {
        if (!ok) break;
        read_pairs_7(a, v);
        bool have = true;
#pragma unroll
        for (int cc = 0; cc < 7; ++cc)
          if (cc < C - 1 && (uint32_t)(v[cc] >> 32) != tag) have = false;
        if (__ballot(!have) == 0) break;
        // no sleep between reads: they are served by this XCD's L2 and load
        // nothing that other workgroups wait on (synthetic mixer 11.33 ->
        // 11.13 us, served 8.92 -> 8.86 against one s_sleep unit)
        if (it >= loc.spin_limit) ok = false;        // (a part ran on another XCD, or never ran)
      }
      float tot = __uint_as_float((uint32_t)v[0]);
#pragma unroll
      for (int cc = 1; cc < 7; ++cc)
        if (cc < C - 1) tot += __uint_as_float((uint32_t)v[cc]);
      tot = C > 1 ? tot + own : own;
      const int64_t orow = (int64_t)t * 16 + nn;
      if (e < p.M * 16 && orow < p.N) Epi::apply(p, 0, m, orow, ok ? tot * p.gs : __builtin_nanf(""));
    }
    if (lane == 0 && !ok) __hip_atomic_fetch_or(loc.status, 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return true;
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (g * 4 + i < p.M)
        __hip_atomic_store(slots + (c * p.M + g * 4 + i) * 16 + n, acc[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  wait_vmcnt<0>();                                   // the slot stores have completed
  int tk = 0;
  int* const ticket = p.tickets + (int64_t)t * p.tstride;
  if (lane == 0) tk = __hip_atomic_fetch_add(ticket, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  tk = __builtin_amdgcn_readfirstlane(tk);
  if (tk != C - 1) return false;
  for (int e = lane; e < p.M * 16; e += 64) {        // e = m * 16 + n
    const float* src = slots + e;
    float tot = ld_coherent(src);
    for (int cc = 1; cc < C; ++cc) tot += ld_coherent(src + cc * p.M * 16);
    const int64_t orow = (int64_t)t * 16 + (e & 15);
    if (orow < p.N) Epi::apply(p, 0, e >> 4, orow, tot * p.gs);
  }
  if (lane == 0) ticket_reset(ticket);
  return true;
}

template <bool F16S, int WPG, int JW, class Epi>
__global__ __launch_bounds__(64 * WPG) void w8_splitk_kernel(GemvLaunch p, int C) {
  extern __shared__ __align__(16) uint16_t lds[];
  const int t = blockIdx.x / C, c = blockIdx.x - t * C;
  w8_splitk_item<F16S, WPG, JW, Epi>(p, C, t, c, reinterpret_cast<char*>(lds));
}

template <bool F16S, int WPG, int JW, class Epi>
bool launch_w8_splitk(GemvLaunch p, int C, size_t lds, int gx, hipStream_t st) {
  auto kern = w8_splitk_kernel<F16S, WPG, JW, Epi>;
  static bool attr_set = false;
  if (!attr_set) {
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                            160 * 1024) != hipSuccess) {
      (void)hipGetLastError();
      return false;
    }
    attr_set = true;
  }
  hipLaunchKernelGGL(kern, dim3(gx), dim3(64 * WPG), lds, st, p, C);
  return true;
}

template <bool F16S, int T, int KW, int D, class Epi>
bool launch_w8_stream_cfg(GemvLaunch p, size_t lds, int gx, hipStream_t st) {
  auto kern = w8_stream_kernel<F16S, T, KW, D, Epi>;
  static bool attr_set = false;
  if (!attr_set) {
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                            160 * 1024) != hipSuccess) {
      (void)hipGetLastError();
      return false;
    }
    attr_set = true;
  }
  hipLaunchKernelGGL(kern, dim3(gx), dim3(64 * T * KW), lds, st, p);
  return true;
}

// Launch the streaming kernel when the call fits it; returns false (and
// launches nothing) otherwise, or when the environment sets FP4X_W8_STREAM=0.
// Conditions: no split-K, K a multiple of 512
// (whole 1 KB activation pieces and whole units per part), scales and their
// batch stride 4-byte aligned, enough tiles for a full round on every CU, and
// the LDS plan within the CU's 160 KB.
struct StreamW8H;
struct StreamW8F;
template <class U, int T, int KW, int D>
bool launch_dense_stream(GemvLaunch p, int batch, bool on, hipStream_t st, int64_t min_items = -1);

template <bool F16S>
bool launch_w8_stream(GemvLaunch p, int batch, hipStream_t st) {
  constexpr int T = 6, KW = 2, D = 3;
  if (!switches().w8_stream) return false;            // FP4X_W8_STREAM=0: always the MFMA core
  // 256-K units (five loads per 256 K values instead of six).  The 48
  // layer-batched gates [512 x 2560] at M = 3 with fp16 scales, measured back
  // to back on one GPU: (T, KW, D) = (6, 2, 2) 15.2 us against 15.5 for this
  // kernel's 128-K units; (6, 1, 3) 16.2, (3, 2, 3) 16.6, (2, 5, 2) 16.8.
  // With fp32 scales (StreamW8F, one 4-byte scale load per lane) at M = 3 /
  // 1: 16.2-16.7 / 15.6-15.8 us against 17.0-17.5 / 16.3-16.6 on the 128-K
  // kernel (two interleaved pairs of runs on one box).  Calls whose LDS plan
  // does not fit (M >= 5 with two batch entries per workgroup) take the 128-K
  // kernel below.
  if constexpr (F16S) {
    if (launch_dense_stream<StreamW8H, 6, 2, 2>(p, batch, true, st)) return true;
  } else {
    if (launch_dense_stream<StreamW8F, 6, 2, 2>(p, batch, true, st)) return true;
  }
  const int K = p.pa.K, tiles = (p.N + 15) / 16;
  if (p.ksplit != 1 || K % 512 != 0 || p.M > 16 || (K / 128) % KW != 0) return false;
  if ((reinterpret_cast<uintptr_t>(p.pa.s) & 3) || (batch > 1 && (p.s_bstride & 3))) return false;
  const int64_t items = (int64_t)batch * tiles;
  const int cus = device_cus();
  if (items < (int64_t)cus * T) return false;
  const int64_t per = (items + (int64_t)cus * T - 1) / ((int64_t)cus * T) * T;
  // batch entries one workgroup can span: its first and last tile
  const int64_t span = (per + tiles - 1) / tiles + 1;
  if (span > 2) return false;
  const size_t lds = (size_t)span * StreamGeom::xbuf_bytes(p.M, K) + (size_t)T * (KW - 1) * 1024 +
                     (size_t)T * KW * D * kStreamUnit;
  if (lds > 160 * 1024) return false;
  p.batch = batch;
  p.per_wg = (int)per;
  p.xbufs = (int)span;
  const int gx = (int)((items + per - 1) / per);
  return launch_w8_stream_cfg<F16S, T, KW, D, EpiStore>(p, lds, gx, st);
}

// Split-K W8 GEMVs of few tiles (the mixer's down projection, N = 640,
// K = 10240).  The caller's ksplit > 1 selects split-K (whatever its value);
// this library picks the decomposition from (M, N, K, ksplit) alone, so every
// entry point deciding on the same shape takes the same path, which keeps the
// fused mixer bit-identical to the unfused GEMV + epilogue kernels:
//   * w8_splitk_kernel when K is a multiple of 2048 (8 waves x 2 units per
//     workgroup, C = K / 2048 >= 2 workgroups per tile) and the caller's
//     scratch (ksplit x 16 x N floats, one ticket per tile) holds the
//     tiles x C x M x 16 partial slots;
//   * else the ring kernel with one workgroup per tile whose KW = 16 waves
//     split K and sum in part order through LDS (no scratch), when K / 128 is
//     a multiple of 16 with at least 2 units per wave and the activations fit
//     in LDS beside the rings (M <= 3 at K = 10240).
// Both need at most two tiles per CU.  Returns false otherwise (or with
// FP4X_W8_STREAM=0), launching nothing.
constexpr int kSplitWaves = 8, kSplitUnits = 2;     // w8_splitk_kernel: waves per workgroup, units per wave

// The split-over-workgroups plan of a W8 split-K call: true with C (workgroups
// per tile) and the LDS bytes when w8_splitk_kernel takes it.
inline bool w8_splitk_plan(const GemvLaunch& p, int& C, size_t& lds) {
  constexpr int SU = kSplitWaves * kSplitUnits;
  if (!switches().w8_stream) return false;
  const int K = p.pa.K, tiles = (p.N + 15) / 16, units = K / 128;
  if (p.ksplit < 2 || K % 512 != 0 || p.M > 16) return false;
  if (reinterpret_cast<uintptr_t>(p.pa.s) & 3) return false;
  if (tiles > 2 * device_cus() || units % SU != 0 || units / SU < 2 || !p.part || !p.tickets) return false;
  C = units / SU;
  const int64_t slots = (int64_t)tiles * C * p.M * 16, have = (int64_t)p.ksplit * 16 * p.N;
  lds = (size_t)((p.M * (SU * 256 + 64) + 15) & ~15) + (size_t)(kSplitWaves - 1) * 1024;
  return slots <= have && lds <= 160 * 1024;
}

template <bool F16S, class Epi>
bool launch_w8_ktile(GemvLaunch p, hipStream_t st) {
  constexpr int KW = 16, D = 2;
  if (!switches().w8_stream) return false;
  const int K = p.pa.K, tiles = (p.N + 15) / 16;
  if (p.ksplit < 2 || K % 512 != 0 || p.M > 16) return false;
  if (reinterpret_cast<uintptr_t>(p.pa.s) & 3) return false;
  if (tiles > 2 * device_cus()) return false;
  const int units = K / 128;
  p.batch = 1;
  p.per_wg = 1;
  p.xbufs = 1;
  int C = 0;
  size_t slds = 0;
  if (w8_splitk_plan(p, C, slds))
    return launch_w8_splitk<F16S, kSplitWaves, kSplitUnits, Epi>(p, C, slds, tiles * C, st);
  if (units % KW != 0 || units / KW < D) return false;
  const size_t lds = (size_t)StreamGeom::xbuf_bytes(p.M, K) + (size_t)(KW - 1) * 1024 + (size_t)KW * D * kStreamUnit;
  if (lds > 160 * 1024) return false;
  p.ksplit = 1;                                      // one slice per workgroup: the parts live in its waves
  return launch_w8_stream_cfg<F16S, 1, KW, D, Epi>(p, lds, tiles, st);
}

}  // namespace fp4x

namespace fp4x {

// ---------------------------------------------------------------------------
// Streaming INT2 coarse head (2-bit codes, one fp16 or e4m3 scale per 16 K
// values): logits[m, n] = sum_k x[m, k] * bf16((code - 1.5) * s)
// (x/fp4x_kernels.py:304-325), optionally times rs[n] (the e4m3 form's row scale).
//
// One wave per 16-row tile, no cross-wave reduction: the tiles of the matrix
// are split into contiguous, equal (+-1) ranges over every wave of the grid
// (one workgroup of W waves per CU), and each wave streams its tiles' units
// through a private LDS ring of D buffers.  A unit is 128 bytes of codes
// (512 weights) and the 64 (fp16, G = 16) or 32 (e4m3 with G = 16, fp16 with
// G = 32: a compact scale row, C32) bytes of their scales, for each of the 16
// rows: two 16-byte direct loads per lane for the codes (the W8 lane pattern)
// and one for the scales (64-byte rows: lane l: row l >> 2, 16-byte piece
// (l & 3) ^ ((row >> 2) & 3), so that the 8-byte scale reads of a quarter-wave
// hit distinct banks; 32-byte rows: lanes 0..31, row l >> 1, piece (l & 1) ^
// (row >> 3), so that the 4-byte scale reads of a wave hit 64 distinct
// banks).  A 64-weight chunk's scales are 4 bytes of a compact row either way
// (four e4m3 group scales, or two fp16 ones).  The activations are staged
// once per workgroup in the 4x4-transposed k order of FmtInt2::deq16t (one
// byte permute per weight).
template <bool C32>
struct Int2Unit {
  static constexpr int scale_row = C32 ? 32 : 64;     // scale bytes of one row in a unit
  static constexpr int bytes = 2048 + 16 * scale_row;
};

__device__ __forceinline__ void int2_read_unit(uint32_t wa, uint32_t wb, uint32_t sa, uint32_t sb, uint4& q0,
                                               uint4& q1, uint2& s0, uint2& s1) {
  asm volatile(
      "ds_read_b128 %0, %4\n\t"
      "ds_read_b128 %1, %5\n\t"
      "ds_read_b64 %2, %6\n\t"
      "ds_read_b64 %3, %7\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(q0), "=&v"(q1), "=&v"(s0), "=&v"(s1)
      : "v"(wa), "v"(wb), "v"(sa), "v"(sb)
      : "memory");
}
// The activations of one 64-weight chunk: 4 sub-blocks x 2 operand halves.
__device__ __forceinline__ void int2_read_x(uint32_t xa, uint4 (&x)[8]) {
  asm volatile(
      "ds_read_b128 %0, %8\n\t"
      "ds_read_b128 %1, %8 offset:16\n\t"
      "ds_read_b128 %2, %8 offset:32\n\t"
      "ds_read_b128 %3, %8 offset:48\n\t"
      "ds_read_b128 %4, %8 offset:64\n\t"
      "ds_read_b128 %5, %8 offset:80\n\t"
      "ds_read_b128 %6, %8 offset:96\n\t"
      "ds_read_b128 %7, %8 offset:112\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(x[0]), "=&v"(x[1]), "=&v"(x[2]), "=&v"(x[3]), "=&v"(x[4]), "=&v"(x[5]), "=&v"(x[6]), "=&v"(x[7])
      : "v"(xa)
      : "memory");
}
// One unit's weights and scales plus both halves' activations in one go:
// waits only for the first 12 reads (LDS operations of a wave complete in
// order), so the second half's 8 activation reads stay in flight while the
// first half computes; int2_wait_x then releases them.
typedef uint32_t i2x_u32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ void int2_read_unit_x(uint32_t wa, uint32_t wb, uint32_t sa, uint32_t sb, uint32_t xa,
                                                 uint4& q0, uint4& q1, uint2& s0, uint2& s1, i2x_u32x4 (&x)[8],
                                                 i2x_u32x4 (&y)[8]) {
  asm volatile(
      "ds_read_b128 %0, %20\n\t"
      "ds_read_b128 %1, %21\n\t"
      "ds_read_b64 %2, %22\n\t"
      "ds_read_b64 %3, %23\n\t"
      "ds_read_b128 %4, %24\n\t"
      "ds_read_b128 %5, %24 offset:16\n\t"
      "ds_read_b128 %6, %24 offset:32\n\t"
      "ds_read_b128 %7, %24 offset:48\n\t"
      "ds_read_b128 %8, %24 offset:64\n\t"
      "ds_read_b128 %9, %24 offset:80\n\t"
      "ds_read_b128 %10, %24 offset:96\n\t"
      "ds_read_b128 %11, %24 offset:112\n\t"
      "ds_read_b128 %12, %24 offset:512\n\t"
      "ds_read_b128 %13, %24 offset:528\n\t"
      "ds_read_b128 %14, %24 offset:544\n\t"
      "ds_read_b128 %15, %24 offset:560\n\t"
      "ds_read_b128 %16, %24 offset:576\n\t"
      "ds_read_b128 %17, %24 offset:592\n\t"
      "ds_read_b128 %18, %24 offset:608\n\t"
      "ds_read_b128 %19, %24 offset:624\n\t"
      "s_waitcnt lgkmcnt(8)"
      : "=&v"(q0), "=&v"(q1), "=&v"(s0), "=&v"(s1), "=&v"(x[0]), "=&v"(x[1]), "=&v"(x[2]), "=&v"(x[3]),
        "=&v"(x[4]), "=&v"(x[5]), "=&v"(x[6]), "=&v"(x[7]), "=&v"(y[0]), "=&v"(y[1]), "=&v"(y[2]), "=&v"(y[3]),
        "=&v"(y[4]), "=&v"(y[5]), "=&v"(y[6]), "=&v"(y[7])
      : "v"(wa), "v"(wb), "v"(sa), "v"(sb), "v"(xa)
      : "memory");
}
// int2_read_unit_x with compact scale rows: 4 bytes per half (s0.y, s1.y untouched).
__device__ __forceinline__ void int2_read_unit_x_c32(uint32_t wa, uint32_t wb, uint32_t sa, uint32_t sb,
                                                      uint32_t xa, uint4& q0, uint4& q1, uint32_t& s0, uint32_t& s1,
                                                      i2x_u32x4 (&x)[8], i2x_u32x4 (&y)[8]) {
  asm volatile(
      "ds_read_b128 %0, %20\n\t"
      "ds_read_b128 %1, %21\n\t"
      "ds_read_b32 %2, %22\n\t"
      "ds_read_b32 %3, %23\n\t"
      "ds_read_b128 %4, %24\n\t"
      "ds_read_b128 %5, %24 offset:16\n\t"
      "ds_read_b128 %6, %24 offset:32\n\t"
      "ds_read_b128 %7, %24 offset:48\n\t"
      "ds_read_b128 %8, %24 offset:64\n\t"
      "ds_read_b128 %9, %24 offset:80\n\t"
      "ds_read_b128 %10, %24 offset:96\n\t"
      "ds_read_b128 %11, %24 offset:112\n\t"
      "ds_read_b128 %12, %24 offset:512\n\t"
      "ds_read_b128 %13, %24 offset:528\n\t"
      "ds_read_b128 %14, %24 offset:544\n\t"
      "ds_read_b128 %15, %24 offset:560\n\t"
      "ds_read_b128 %16, %24 offset:576\n\t"
      "ds_read_b128 %17, %24 offset:592\n\t"
      "ds_read_b128 %18, %24 offset:608\n\t"
      "ds_read_b128 %19, %24 offset:624\n\t"
      "s_waitcnt lgkmcnt(8)"
      : "=&v"(q0), "=&v"(q1), "=&v"(s0), "=&v"(s1), "=&v"(x[0]), "=&v"(x[1]), "=&v"(x[2]), "=&v"(x[3]),
        "=&v"(x[4]), "=&v"(x[5]), "=&v"(x[6]), "=&v"(x[7]), "=&v"(y[0]), "=&v"(y[1]), "=&v"(y[2]), "=&v"(y[3]),
        "=&v"(y[4]), "=&v"(y[5]), "=&v"(y[6]), "=&v"(y[7])
      : "v"(wa), "v"(wb), "v"(sa), "v"(sb), "v"(xa)
      : "memory");
}
// The second half's activations are in registers after this (tied to them so
// that no use moves above the wait, and to the accumulator so that the first
// half's MFMAs stay above it).
__device__ __forceinline__ void int2_wait_x(i2x_u32x4 (&y)[8], f32x4_t& acc) {
  asm volatile("s_waitcnt lgkmcnt(0)"
               : "+v"(y[0]), "+v"(y[1]), "+v"(y[2]), "+v"(y[3]), "+v"(y[4]), "+v"(y[5]), "+v"(y[6]), "+v"(y[7]),
                 "+v"(acc)
               :
               : "memory");
}
__device__ __forceinline__ void lds_put_u128(uint32_t a, uint4 v) {
  typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
  const u32x4_t w = {v.x, v.y, v.z, v.w};
  asm volatile("ds_write_b128 %0, %1" ::"v"(a), "v"(w) : "memory");
}
__device__ __forceinline__ void wait_lgkm0_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

template <bool E4M3, int GC, int W, int D>
__global__ __launch_bounds__(64 * W) void int2_stream_kernel(GemvLaunch p) {
  static_assert(GC == 16 || (GC == 32 && !E4M3), "G = 16, or fp16 scales at G = 32");
  constexpr bool C32 = E4M3 || GC == 32;               // 32 scale bytes per row and unit
  using F = FmtInt2<E4M3, GC>;
  using U = Int2Unit<C32>;
  extern __shared__ __align__(16) uint16_t lds[];
  char* base = reinterpret_cast<char*>(lds);
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int n = lane & 15, g = lane >> 4;
  const int K = p.pa.K, J = K / 512;                 // units per tile
  const int64_t tiles = (p.N + 15) / 16;
  // The workgroup's tiles [T0, T1) go to its waves as they free up: wave w
  // starts on tile T0 + w and takes each further one from a counter in LDS.
  // (Contiguous equal ranges per wave left the waves of one SIMD finishing
  // one after another - the SIMD favours its oldest wave - so the last
  // quarter of the kernel ran on a quarter of the waves.)
  // A wave whose first tile T0 + w is past T1 (a workgroup of fewer tiles
  // than waves) issues and computes nothing; it only helps stage the
  // activations.
  const int64_t nw = (int64_t)gridDim.x * W, g0 = (int64_t)blockIdx.x * W;
  const int T0 = (int)(g0 * tiles / nw), T1 = (int)((g0 + W) * tiles / nw);   // T1 - T0 >= W / 2 - 1 (host condition)
  const bool act = T0 + wave < T1;
  __shared__ int s_next;
  if (threadIdx.x == 0) s_next = T0 + W;              // (visible after the staging barrier below)
  const int xrow = StreamGeom::xrow_bytes(K), xbuf = StreamGeom::xbuf_bytes(p.M, K);
  char* ring = base + xbuf + wave * D * U::bytes;
  const int cb = K / 4, sbr = K / 16 * (C32 ? 1 : 2);    // code and scale bytes per row

  // DMA lanes (codes as in the W8 kernel; scales: row l >> 2, piece (l & 3) ^ ((row >> 2) & 3))
  const int dr = lane >> 3, dc = lane & 7;
  const int cA = dc ^ (dr >> 1), cB = dc ^ (4 + (dr >> 1));
  const int sr = C32 ? lane >> 1 : lane >> 2;
  const int sp = C32 ? (lane & 1) ^ (sr >> 3) : (lane & 3) ^ ((sr >> 2) & 3);
  // issuer: the tile whose units go out (ij: next unit; a new tile is taken
  // when its first unit is issued, never before the staging barrier since
  // D <= J), the tiles taken so far (ngot), the last two of them (fifo)
  int ij = 0, is = 0, issued = 0, ngot = act ? 1 : 0;
  bool need = false, idone = !act;
  int fifo[2] = {T0 + wave, 0};
  const uint8_t* iw = nullptr;
  const uint8_t* isb = nullptr;
  uint32_t o0 = 0, o1 = 0, os = 0;
  auto set_tile = [&](int t) {
    const int64_t lim64 = (int64_t)p.N - 1 - (int64_t)t * 16;
    const int lim = (int)(lim64 < 15 ? lim64 : 15);
    iw = p.pa.w0 + (int64_t)t * 16 * cb;
    isb = p.pa.s + (int64_t)t * 16 * sbr;
    const int rA = dr < lim ? dr : lim, rB = dr + 8 < lim ? dr + 8 : lim, rS = sr < lim ? sr : lim;
    o0 = (uint32_t)(rA * cb + cA * 16);
    o1 = (uint32_t)(rB * cb + cB * 16);
    os = (uint32_t)(rS * sbr + sp * 16);
  };
  set_tile(act ? T0 + wave : T0);
  auto issue_next = [&]() {
    if (need) {
      int t = 0;
      if (lane == 0) t = atomicAdd(&s_next, 1);
      t = __builtin_amdgcn_readfirstlane(t);
      need = false;
      if (t >= T1) {
        idone = true;
        return;
      }
      fifo[ngot & 1] = t;
      ++ngot;
      set_tile(t);
    }
    char* l = ring + is * U::bytes;
    dma_b128(iw + ij * 128 + o0, l);
    dma_b128(iw + ij * 128 + o1, l + 1024);
    if (!C32 || lane < 32) dma_b128(isb + ij * U::scale_row + os, l + 2048);
    if (++is == D) is = 0;
    ++issued;
    if (++ij == J) {
      ij = 0;
      need = true;
    }
  };
  // D units of the first tile go out first, then the activations are staged
  // while they fly.
  if (act) {
#pragma unroll
    for (int u = 0; u < D; ++u) issue_next();
  }
  {
    const int per_row = K / 16, total = p.M * per_row;
    const uint4* xg4 = reinterpret_cast<const uint4*>(p.x);
    const int64_t xrow4 = p.x_stride / 8;
    const uint32_t xl0 = lds_addr(base);
    for (int i = threadIdx.x; i < total; i += 64 * W) {
      const int m = i / per_row, qb = i - m * per_row;
      const uint4 a = xg4[m * xrow4 + 2 * qb], b = xg4[m * xrow4 + 2 * qb + 1];   // elements 0-7, 8-15
      uint4 o, r;
      o.x = perm_b32(a.z, a.x, 0x05040100u);   // x0, x4
      o.y = perm_b32(b.z, b.x, 0x05040100u);   // x8, x12
      o.z = perm_b32(a.z, a.x, 0x07060302u);   // x1, x5
      o.w = perm_b32(b.z, b.x, 0x07060302u);   // x9, x13
      r.x = perm_b32(a.w, a.y, 0x05040100u);   // x2, x6
      r.y = perm_b32(b.w, b.y, 0x05040100u);   // x10, x14
      r.z = perm_b32(a.w, a.y, 0x07060302u);   // x3, x7
      r.w = perm_b32(b.w, b.y, 0x07060302u);   // x11, x15
      const uint32_t la = xl0 + m * xrow + qb * 32;
      lds_put_u128(la, o);
      lds_put_u128(la + 16, r);
    }
    wait_lgkm0_barrier();
  }
  const int xr = n < p.M ? n : 0;
  const uint32_t rl = lds_addr(ring);
  const uint32_t wlA = rl + n * 128 + ((g ^ (n >> 1)) * 16), wlB = rl + n * 128 + (((g + 4) ^ (n >> 1)) * 16);
  // lane (n, g): the scales of chunks g (A) and g + 4 (B) of row n
  const int sx = C32 ? n >> 3 : (n >> 2) & 3;
  const uint32_t slA = C32 ? rl + 2048 + n * 32 + (sx * 16) + g * 4
                           : rl + 2048 + n * 64 + (((g >> 1) ^ sx) * 16) + (g & 1) * 8;
  const uint32_t slB = C32 ? rl + 2048 + n * 32 + ((1 ^ sx) * 16) + g * 4
                           : rl + 2048 + n * 64 + (((2 + (g >> 1)) ^ sx) * 16) + (g & 1) * 8;
  const uint32_t xl = lds_addr(base) + xr * xrow + g * 128;   // chunk g of unit 0
  int cs = 0, u = 0;
  for (int q = 0; q < ngot; ++q) {                   // (ngot grows while tiles are taken)
    const int64_t tq = fifo[q & 1];
    f32x4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int j = 0; j < J; ++j, ++u) {
      if (issued - 1 - u >= D - 1) wait_vmcnt<3 * (D - 1)>();
      else wait_vmcnt<0>();
      const uint32_t so = cs * U::bytes;
      typename F::Chunk ch[2];
      i2x_u32x4 xh[2][8];
      if constexpr (C32) {
        ch[0].s.y = ch[1].s.y = 0;
        int2_read_unit_x_c32(wlA + so, wlB + so, slA + so, slB + so, xl + j * 1024, ch[0].q, ch[1].q, ch[0].s.x,
                              ch[1].s.x, xh[0], xh[1]);
      } else {
        int2_read_unit_x(wlA + so, wlB + so, slA + so, slB + so, xl + j * 1024, ch[0].q, ch[1].q, ch[0].s, ch[1].s,
                         xh[0], xh[1]);
      }
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        if (h == 1) int2_wait_x(xh[1], acc);
#pragma unroll
        for (int sub = 0; sub < 4; ++sub) {
          uint32_t w[8];
          F::deq16t(ch[h], sub, w);
          const i2x_u32x4 a0 = xh[h][2 * sub], a1 = xh[h][2 * sub + 1];
          acc = mfma16(make_uint4(a0.x, a0.y, a0.z, a0.w), make_uint4(w[0], w[1], w[2], w[3]), acc);
          acc = mfma16(make_uint4(a1.x, a1.y, a1.z, a1.w), make_uint4(w[4], w[5], w[6], w[7]), acc);
        }
      }
      if (++cs == D) cs = 0;
      if (!idone) issue_next();
    }
    const int64_t row = tq * 16 + n;                 // lane (n, g) holds D[m = 4g + i][n]
    if (row < p.N) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (g * 4 + i < p.M) EpiStore::apply(p, 0, g * 4 + i, row, acc[i] * p.gs);
    }
    if (p.smax) {
      // the largest order key of the tile's 16 stored (bf16) logits of each row m:
      // the 16-element slice maxima of the top-k (rows past N: key 0, below all)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float v = acc[i] * p.gs;
        if (p.rs) v = v * p.rs[row < p.N ? row : p.N - 1];
        uint32_t key = row < p.N ? tk_key(f32_to_bf16(v)) : 0u;
        // maximum over the 16 lanes n of this g (one DPP row): quad swaps, half mirror, mirror
        key = max(key, (uint32_t)__builtin_amdgcn_mov_dpp((int)key, 0xB1, 0xF, 0xF, false));
        key = max(key, (uint32_t)__builtin_amdgcn_mov_dpp((int)key, 0x4E, 0xF, 0xF, false));
        key = max(key, (uint32_t)__builtin_amdgcn_mov_dpp((int)key, 0x141, 0xF, 0xF, false));
        key = max(key, (uint32_t)__builtin_amdgcn_mov_dpp((int)key, 0x140, 0xF, 0xF, false));
        if (n == 0 && g * 4 + i < p.M) p.smax[(int64_t)(g * 4 + i) * p.smax_stride + tq] = (uint16_t)key;
      }
    }
  }
  wait_vmcnt<0>();                                   // no load of the prologue outlives the wave
}

// The INT2 head (G = 16 with fp16 or e4m3 scales, G = 32 with fp16 ones) through the streaming kernel
// when the matrix has at least one tile per two waves of the grid and a tile's
// units fill the ring (the 65k-token draft subset: 4075 tiles over 16 waves
// per CU); false otherwise (or when FP4X_INT2_STREAM=0).  16 waves per CU
// (ring depth 3) when the staged activations leave room, else 8 waves with
// the deepest ring that fits.
constexpr int kInt2DynLds = 160 * 1024 - 256;      // room for the kernel's static LDS (the tile counter)

template <bool E4M3, int GC, int W, int D>
bool launch_int2_stream_wd(GemvLaunch p, size_t lds, hipStream_t st) {
  auto kern = int2_stream_kernel<E4M3, GC, W, D>;
  static bool attr_set = false;
  if (!attr_set) {
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                            kInt2DynLds) != hipSuccess) {
      (void)hipGetLastError();
      return false;
    }
    attr_set = true;
  }
  hipLaunchKernelGGL(kern, dim3(device_cus()), dim3(64 * W), lds, st, p);
  return true;
}

template <bool E4M3, int GC>
inline bool launch_int2_stream(GemvLaunch p, hipStream_t st) {
  if (!switches().int2_stream) return false;
  const int K = p.pa.K;
  if (p.pa.G != GC || K % 512 != 0 || p.M > 16 || p.ksplit != 1) return false;
  if ((reinterpret_cast<uintptr_t>(p.pa.w0) & 15) || (reinterpret_cast<uintptr_t>(p.pa.s) & 15)) return false;
  const int64_t tiles = (p.N + 15) / 16;
  const size_t xb = (size_t)StreamGeom::xbuf_bytes(p.M, K);
  const int64_t cus = device_cus();
  constexpr size_t ub = Int2Unit<E4M3 || GC == 32>::bytes;
  auto fits = [&](int W, int D) {
    return xb + (size_t)W * D * ub <= (size_t)kInt2DynLds && K / 512 >= D && 2 * tiles >= cus * W;
  };
  if (fits(16, 3)) return launch_int2_stream_wd<E4M3, GC, 16, 3>(p, xb + 16 * 3 * ub, st);
  if (fits(8, 6)) return launch_int2_stream_wd<E4M3, GC, 8, 6>(p, xb + 8 * 6 * ub, st);
  if (fits(8, 4)) return launch_int2_stream_wd<E4M3, GC, 8, 4>(p, xb + 8 * 4 * ub, st);
  if (fits(8, 3)) return launch_int2_stream_wd<E4M3, GC, 8, 3>(p, xb + 8 * 3 * ub, st);
  return false;
}

}  // namespace fp4x

namespace fp4x {

// ---------------------------------------------------------------------------
// Streaming dense GEMVs for a single matrix of many 16-row tiles (NVFP4 N =
// 16384, W6 N = 8192, MXFP8 N = 4096 and the 248,320-row MXFP8 head, K =
// 2560): the W8 streaming design, with a per-format unit policy U.
//   * A unit is U::UK K values (128 or 256) of the tile's 16 rows; lane (n, g)
//     consumes K values [g UK / 4, (g + 1) UK / 4) of row n as chunks of the
//     format's core dequant (FmtMX8, FmtNV4, FmtW6), four MFMAs per 32 K
//     values, reading UK / 2 bytes of activations.
//   * U::issue puts a unit into LDS with U::NDMA direct loads per lane; the
//     16-byte pieces of each row are XOR-swizzled so that the 16 lanes of a
//     quarter-wave, one per row, read distinct LDS bank groups.  Lanes of a
//     4-byte scale load past the unit's scales repeat them into an unread
//     tail.
//   * T tile slots x KW waves per workgroup, each wave with a ring of D
//     units; the KW parts of a tile are summed in part order through LDS; gs
//     multiplies the sum, as in the core kernel.

// MXFP8 unit: 16 rows x 128 bytes of e4m3 codes (two 16-byte loads of 8 rows
// each; row r's piece p at position p ^ ((r >> 1) & 7)), then 16 rows x 4
// e8m0 scales (lanes 0..15 of a 4-byte load).
struct StreamMX8 {
  static constexpr int UK = 128, BYTES = 2048 + 256, NDMA = 3;
  const uint8_t* w;
  const uint8_t* s;
  uint32_t oa, ob, os;
  static constexpr int XG = 64;                       // activation bytes between lane groups g
  static constexpr bool BATCHED = false;              // single matrices only
  __device__ void set(const GemvLaunch& p, int K, int b, int64_t t, int k128, int lane, int lim) {
    const int ra = lane >> 3, rb = ra + 8, pp = lane & 7, sr = lane & 15;
    w = p.pa.w0 + b * p.w0_bstride + t * 16 * K + k128 * 128;
    s = p.pa.s + b * p.s_bstride + t * 16 * (K / 32) + k128 * 4;
    oa = (uint32_t)((ra < lim ? ra : lim) * K + (pp ^ ((ra >> 1) & 7)) * 16);
    ob = (uint32_t)((rb < lim ? rb : lim) * K + (pp ^ ((rb >> 1) & 7)) * 16);
    os = (uint32_t)((sr < lim ? sr : lim) * (K / 32));
  }
  __device__ void issue(char* d, int ij) const {
    dma_b128(w + ij * 128 + oa, d);
    dma_b128(w + ij * 128 + ob, d + 1024);
    dma_b32(s + ij * 4 + os, d + 2048);
  }
  __device__ static void consume(uint32_t u, uint32_t xa, int n, int g, f32x4_t& acc) {
    FmtMX8::Chunk a, b;
    uint4 x0, x1, x2, x3;
    const int f = (n >> 1) & 7;
    asm volatile(
        "ds_read_b128 %0, %7\n\t"
        "ds_read_b128 %1, %8\n\t"
        "ds_read_u8 %2, %9\n\t"
        "ds_read_b128 %3, %10\n\t"
        "ds_read_b128 %4, %10 offset:16\n\t"
        "ds_read_b128 %5, %10 offset:32\n\t"
        "ds_read_b128 %6, %10 offset:48\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(a.q), "=&v"(b.q), "=&v"(a.e), "=&v"(x0), "=&v"(x1), "=&v"(x2), "=&v"(x3)
        : "v"(u + n * 128 + (((2 * g) ^ f) * 16)), "v"(u + n * 128 + (((2 * g + 1) ^ f) * 16)),
          "v"(u + 2048 + n * 4 + g), "v"(xa)
        : "memory");
    b.e = a.e;
    uint32_t w[8];
    FmtMX8::deq16(a, 0, w);
    acc = mfma16(x0, make_uint4(w[0], w[1], w[2], w[3]), acc);
    acc = mfma16(x1, make_uint4(w[4], w[5], w[6], w[7]), acc);
    FmtMX8::deq16(b, 0, w);
    acc = mfma16(x2, make_uint4(w[0], w[1], w[2], w[3]), acc);
    acc = mfma16(x3, make_uint4(w[4], w[5], w[6], w[7]), acc);
  }
};

// W6 unit of 256 K values: 16 rows x 128 bytes of L (two 16-byte loads of 8
// rows, pieces swizzled by (row >> 1) & 7), 16 rows x 64 bytes of H (one
// 16-byte load, pieces swizzled by (row >> 2) & 3), 16 rows x 8 fp16 scales
// (one 4-byte load): four loads per 256 K values instead of eight.  Lane (n,
// g) takes chunks 2g and 2g + 1 of row n, K values [64 g, 64 g + 64).
struct StreamW6 {
  static constexpr int UK = 256, BYTES = 2048 + 1024 + 256, NDMA = 4;
  const uint8_t* l;
  const uint8_t* h;
  const uint8_t* s;
  uint32_t ola, olb, oh, os;
  static constexpr int XG = 128;
  static constexpr bool BATCHED = false;
  __device__ void set(const GemvLaunch& p, int K, int b, int64_t t, int ku, int lane, int lim) {
    const int ra = lane >> 3, rb = ra + 8, pp = lane & 7;
    const int hr = lane >> 2, hp = (lane & 3) ^ ((hr >> 2) & 3);
    l = p.pa.w0 + b * p.w0_bstride + t * 16 * (K / 2) + ku * 128;
    h = p.pa.w1 + b * p.w1_bstride + t * 16 * (K / 4) + ku * 64;
    s = p.pa.s + b * p.s_bstride + t * 16 * (K / 16) + ku * 16;
    ola = (uint32_t)((ra < lim ? ra : lim) * (K / 2) + (pp ^ ((ra >> 1) & 7)) * 16);
    olb = (uint32_t)((rb < lim ? rb : lim) * (K / 2) + (pp ^ ((rb >> 1) & 7)) * 16);
    oh = (uint32_t)((hr < lim ? hr : lim) * (K / 4) + hp * 16);
    os = (uint32_t)((hr < lim ? hr : lim) * (K / 16) + (lane & 3) * 4);
  }
  __device__ void issue(char* d, int ij) const {
    dma_b128(l + ij * 128 + ola, d);
    dma_b128(l + ij * 128 + olb, d + 1024);
    dma_b128(h + ij * 64 + oh, d + 2048);
    dma_b32(s + ij * 16 + os, d + 3072);
  }
  __device__ static void consume(uint32_t u, uint32_t xa, int n, int g, f32x4_t& acc) {
    uint4 la, lb, hh, x[8];
    uint32_t sc;
    const int f = (n >> 1) & 7;
    asm volatile(
        "ds_read_b128 %0, %12\n\t"
        "ds_read_b128 %1, %13\n\t"
        "ds_read_b128 %2, %14\n\t"
        "ds_read_b32 %3, %15\n\t"
        "ds_read_b128 %4, %16\n\t"
        "ds_read_b128 %5, %16 offset:16\n\t"
        "ds_read_b128 %6, %16 offset:32\n\t"
        "ds_read_b128 %7, %16 offset:48\n\t"
        "ds_read_b128 %8, %16 offset:64\n\t"
        "ds_read_b128 %9, %16 offset:80\n\t"
        "ds_read_b128 %10, %16 offset:96\n\t"
        "ds_read_b128 %11, %16 offset:112\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(la), "=&v"(lb), "=&v"(hh), "=&v"(sc), "=&v"(x[0]), "=&v"(x[1]), "=&v"(x[2]), "=&v"(x[3]),
          "=&v"(x[4]), "=&v"(x[5]), "=&v"(x[6]), "=&v"(x[7])
        : "v"(u + n * 128 + (((2 * g) ^ f) * 16)), "v"(u + n * 128 + (((2 * g + 1) ^ f) * 16)),
          "v"(u + 2048 + n * 64 + ((g ^ ((n >> 2) & 3)) * 16)), "v"(u + 3072 + n * 16 + g * 4), "v"(xa)
        : "memory");
    FmtW6::Chunk c0, c1;
    c0.lo = la; c0.hi = make_uint2(hh.x, hh.y); c0.s = sc & 0xffffu;
    c1.lo = lb; c1.hi = make_uint2(hh.z, hh.w); c1.s = sc >> 16;
    uint32_t w[8];
    FmtW6::deq16(c0, 0, w);
    acc = mfma16(x[0], make_uint4(w[0], w[1], w[2], w[3]), acc);
    acc = mfma16(x[1], make_uint4(w[4], w[5], w[6], w[7]), acc);
    FmtW6::deq16(c0, 1, w);
    acc = mfma16(x[2], make_uint4(w[0], w[1], w[2], w[3]), acc);
    acc = mfma16(x[3], make_uint4(w[4], w[5], w[6], w[7]), acc);
    FmtW6::deq16(c1, 0, w);
    acc = mfma16(x[4], make_uint4(w[0], w[1], w[2], w[3]), acc);
    acc = mfma16(x[5], make_uint4(w[4], w[5], w[6], w[7]), acc);
    FmtW6::deq16(c1, 1, w);
    acc = mfma16(x[6], make_uint4(w[0], w[1], w[2], w[3]), acc);
    acc = mfma16(x[7], make_uint4(w[4], w[5], w[6], w[7]), acc);
  }
};

// NVFP4 unit of 256 K values: 16 rows x 128 bytes of codes (two 16-byte
// loads of 8 rows, pieces swizzled by (row >> 1) & 7), 16 rows x 16 e4m3
// scales (one 4-byte load).  Lane (n, g) takes chunks 2g and 2g + 1 of row n.
struct StreamNV4 {
  static constexpr int UK = 256, BYTES = 2048 + 256, NDMA = 3;
  const uint8_t* w;
  const uint8_t* s;
  uint32_t oa, ob, os;
  static constexpr int XG = 128;
  static constexpr bool BATCHED = false;
  __device__ void set(const GemvLaunch& p, int K, int b, int64_t t, int ku, int lane, int lim) {
    const int ra = lane >> 3, rb = ra + 8, pp = lane & 7, sr = lane >> 2;
    w = p.pa.w0 + b * p.w0_bstride + t * 16 * (K / 2) + ku * 128;
    s = p.pa.s + b * p.s_bstride + t * 16 * (K / 16) + ku * 16;
    oa = (uint32_t)((ra < lim ? ra : lim) * (K / 2) + (pp ^ ((ra >> 1) & 7)) * 16);
    ob = (uint32_t)((rb < lim ? rb : lim) * (K / 2) + (pp ^ ((rb >> 1) & 7)) * 16);
    os = (uint32_t)((sr < lim ? sr : lim) * (K / 16) + (lane & 3) * 4);
  }
  __device__ void issue(char* d, int ij) const {
    dma_b128(w + ij * 128 + oa, d);
    dma_b128(w + ij * 128 + ob, d + 1024);
    dma_b32(s + ij * 16 + os, d + 2048);
  }
  __device__ static void consume(uint32_t u, uint32_t xa, int n, int g, f32x4_t& acc) {
    uint4 qa, qb, x[8];
    uint32_t sc;
    const int f = (n >> 1) & 7;
    asm volatile(
        "ds_read_b128 %0, %11\n\t"
        "ds_read_b128 %1, %12\n\t"
        "ds_read_b32 %2, %13\n\t"
        "ds_read_b128 %3, %14\n\t"
        "ds_read_b128 %4, %14 offset:16\n\t"
        "ds_read_b128 %5, %14 offset:32\n\t"
        "ds_read_b128 %6, %14 offset:48\n\t"
        "ds_read_b128 %7, %14 offset:64\n\t"
        "ds_read_b128 %8, %14 offset:80\n\t"
        "ds_read_b128 %9, %14 offset:96\n\t"
        "ds_read_b128 %10, %14 offset:112\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(qa), "=&v"(qb), "=&v"(sc), "=&v"(x[0]), "=&v"(x[1]), "=&v"(x[2]), "=&v"(x[3]), "=&v"(x[4]),
          "=&v"(x[5]), "=&v"(x[6]), "=&v"(x[7])
        : "v"(u + n * 128 + (((2 * g) ^ f) * 16)), "v"(u + n * 128 + (((2 * g + 1) ^ f) * 16)),
          "v"(u + 2048 + n * 16 + g * 4), "v"(xa)
        : "memory");
    FmtNV4::Chunk c0, c1;
    c0.q = qa; c0.s = sc & 0xffffu;
    c1.q = qb; c1.s = sc >> 16;
    uint32_t w[8];
    FmtNV4::deq16(c0, 0, w);
    acc = mfma16(x[0], make_uint4(w[0], w[1], w[2], w[3]), acc);
    acc = mfma16(x[1], make_uint4(w[4], w[5], w[6], w[7]), acc);
    FmtNV4::deq16(c0, 1, w);
    acc = mfma16(x[2], make_uint4(w[0], w[1], w[2], w[3]), acc);
    acc = mfma16(x[3], make_uint4(w[4], w[5], w[6], w[7]), acc);
    FmtNV4::deq16(c1, 0, w);
    acc = mfma16(x[4], make_uint4(w[0], w[1], w[2], w[3]), acc);
    acc = mfma16(x[5], make_uint4(w[4], w[5], w[6], w[7]), acc);
    FmtNV4::deq16(c1, 1, w);
    acc = mfma16(x[6], make_uint4(w[0], w[1], w[2], w[3]), acc);
    acc = mfma16(x[7], make_uint4(w[4], w[5], w[6], w[7]), acc);
  }
};

// W8 g64 unit of 256 K values with fp16 scales: 16 rows x 256 bytes of int8
// (four 16-byte loads of 4 rows; row r's piece p at position p ^ (r & 15)),
// then 16 rows x 4 fp16 scales (lanes 0..31 of a 4-byte load).  Lane (n, g)
// takes the 16-value chunks g, g + 4, g + 8, g + 12 of row n, chunk g + 4i in
// g64 group i, with the activations of K values [16 c, 16 c + 16).
struct StreamW8H {
  static constexpr int UK = 256, BYTES = 4096 + 256, NDMA = 5, XG = 32;
  static constexpr bool BATCHED = true;               // layer-batched calls (the 48 gates)
  const uint8_t* w;
  const uint8_t* s;
  uint32_t o[4], os;
  __device__ void set(const GemvLaunch& p, int K, int b, int64_t t, int ku, int lane, int lim) {
    const int sr = (lane & 31) >> 1;
    w = p.pa.w0 + b * p.w0_bstride + t * 16 * K + ku * 256;
    s = p.pa.s + b * p.s_bstride + (t * 16 * (K / 64) + ku * 4) * 2;
#pragma unroll
    for (int h = 0; h < 4; ++h) {
      const int r = 4 * h + (lane >> 4);
      o[h] = (uint32_t)((r < lim ? r : lim) * K + ((lane & 15) ^ r) * 16);
    }
    os = (uint32_t)((sr < lim ? sr : lim) * (K / 64) * 2 + (lane & 1) * 4);
  }
  __device__ void issue(char* d, int ij) const {
#pragma unroll
    for (int h = 0; h < 4; ++h) dma_b128(w + ij * 256 + o[h], d + h * 1024);
    dma_b32(s + ij * 8 + os, d + 4096);
  }
  __device__ static void consume(uint32_t u, uint32_t xa, int n, int g, f32x4_t& acc) {
    uint4 q[4], x[8];
    uint2 sc;
    asm volatile(
        "ds_read_b128 %0, %13\n\t"
        "ds_read_b128 %1, %14\n\t"
        "ds_read_b128 %2, %15\n\t"
        "ds_read_b128 %3, %16\n\t"
        "ds_read_b64 %4, %17\n\t"
        "ds_read_b128 %5, %18\n\t"
        "ds_read_b128 %6, %18 offset:16\n\t"
        "ds_read_b128 %7, %18 offset:128\n\t"
        "ds_read_b128 %8, %18 offset:144\n\t"
        "ds_read_b128 %9, %18 offset:256\n\t"
        "ds_read_b128 %10, %18 offset:272\n\t"
        "ds_read_b128 %11, %18 offset:384\n\t"
        "ds_read_b128 %12, %18 offset:400\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(q[0]), "=&v"(q[1]), "=&v"(q[2]), "=&v"(q[3]), "=&v"(sc), "=&v"(x[0]), "=&v"(x[1]), "=&v"(x[2]),
          "=&v"(x[3]), "=&v"(x[4]), "=&v"(x[5]), "=&v"(x[6]), "=&v"(x[7])
        : "v"(u + n * 256 + ((g ^ n) * 16)), "v"(u + n * 256 + (((g + 4) ^ n) * 16)),
          "v"(u + n * 256 + (((g + 8) ^ n) * 16)), "v"(u + n * 256 + (((g + 12) ^ n) * 16)),
          "v"(u + 4096 + n * 8), "v"(xa)
        : "memory");
    const float s0 = f16_to_f32((uint16_t)sc.x), s1 = f16_to_f32((uint16_t)(sc.x >> 16));
    const float s2 = f16_to_f32((uint16_t)sc.y), s3 = f16_to_f32((uint16_t)(sc.y >> 16));
    uint32_t w[8];
    w8_chunk_bf16(q[0], s0, w);
    acc = mfma16(x[0], make_uint4(w[0], w[1], w[2], w[3]), acc);
    acc = mfma16(x[1], make_uint4(w[4], w[5], w[6], w[7]), acc);
    w8_chunk_bf16(q[1], s1, w);
    acc = mfma16(x[2], make_uint4(w[0], w[1], w[2], w[3]), acc);
    acc = mfma16(x[3], make_uint4(w[4], w[5], w[6], w[7]), acc);
    w8_chunk_bf16(q[2], s2, w);
    acc = mfma16(x[4], make_uint4(w[0], w[1], w[2], w[3]), acc);
    acc = mfma16(x[5], make_uint4(w[4], w[5], w[6], w[7]), acc);
    w8_chunk_bf16(q[3], s3, w);
    acc = mfma16(x[6], make_uint4(w[0], w[1], w[2], w[3]), acc);
    acc = mfma16(x[7], make_uint4(w[4], w[5], w[6], w[7]), acc);
  }
};

// W8 g64 unit with fp32 scales (the reference's _w8 layout): StreamW8H's
// 16 rows x 256 bytes of int8, then 16 rows x 4 fp32 scales, lane l loading
// the scale of row l >> 2, group l & 3 (one 4-byte load), so row r's four
// scales are the 16 bytes at 4096 + 16 r.
struct StreamW8F {
  static constexpr int UK = 256, BYTES = 4096 + 256, NDMA = 5, XG = 32;
  static constexpr bool BATCHED = true;
  const uint8_t* w;
  const uint8_t* s;
  uint32_t o[4], os;
  __device__ void set(const GemvLaunch& p, int K, int b, int64_t t, int ku, int lane, int lim) {
    const int sr = lane >> 2;
    w = p.pa.w0 + b * p.w0_bstride + t * 16 * K + ku * 256;
    s = p.pa.s + b * p.s_bstride + (t * 16 * (K / 64) + ku * 4) * 4;
#pragma unroll
    for (int h = 0; h < 4; ++h) {
      const int r = 4 * h + (lane >> 4);
      o[h] = (uint32_t)((r < lim ? r : lim) * K + ((lane & 15) ^ r) * 16);
    }
    os = (uint32_t)((sr < lim ? sr : lim) * (K / 64) * 4 + (lane & 3) * 4);
  }
  __device__ void issue(char* d, int ij) const {
#pragma unroll
    for (int h = 0; h < 4; ++h) dma_b128(w + ij * 256 + o[h], d + h * 1024);
    dma_b32(s + ij * 16 + os, d + 4096);
  }
  __device__ static void consume(uint32_t u, uint32_t xa, int n, int g, f32x4_t& acc) {
    uint4 q[4], x[8], sc;
    asm volatile(
        "ds_read_b128 %0, %13\n\t"
        "ds_read_b128 %1, %14\n\t"
        "ds_read_b128 %2, %15\n\t"
        "ds_read_b128 %3, %16\n\t"
        "ds_read_b128 %4, %17\n\t"
        "ds_read_b128 %5, %18\n\t"
        "ds_read_b128 %6, %18 offset:16\n\t"
        "ds_read_b128 %7, %18 offset:128\n\t"
        "ds_read_b128 %8, %18 offset:144\n\t"
        "ds_read_b128 %9, %18 offset:256\n\t"
        "ds_read_b128 %10, %18 offset:272\n\t"
        "ds_read_b128 %11, %18 offset:384\n\t"
        "ds_read_b128 %12, %18 offset:400\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(q[0]), "=&v"(q[1]), "=&v"(q[2]), "=&v"(q[3]), "=&v"(sc), "=&v"(x[0]), "=&v"(x[1]), "=&v"(x[2]),
          "=&v"(x[3]), "=&v"(x[4]), "=&v"(x[5]), "=&v"(x[6]), "=&v"(x[7])
        : "v"(u + n * 256 + ((g ^ n) * 16)), "v"(u + n * 256 + (((g + 4) ^ n) * 16)),
          "v"(u + n * 256 + (((g + 8) ^ n) * 16)), "v"(u + n * 256 + (((g + 12) ^ n) * 16)),
          "v"(u + 4096 + n * 16), "v"(xa)
        : "memory");
    uint32_t w[8];
    w8_chunk_bf16(q[0], __uint_as_float(sc.x), w);
    acc = mfma16(x[0], make_uint4(w[0], w[1], w[2], w[3]), acc);
    acc = mfma16(x[1], make_uint4(w[4], w[5], w[6], w[7]), acc);
    w8_chunk_bf16(q[1], __uint_as_float(sc.y), w);
    acc = mfma16(x[2], make_uint4(w[0], w[1], w[2], w[3]), acc);
    acc = mfma16(x[3], make_uint4(w[4], w[5], w[6], w[7]), acc);
    w8_chunk_bf16(q[2], __uint_as_float(sc.z), w);
    acc = mfma16(x[4], make_uint4(w[0], w[1], w[2], w[3]), acc);
    acc = mfma16(x[5], make_uint4(w[4], w[5], w[6], w[7]), acc);
    w8_chunk_bf16(q[3], __uint_as_float(sc.w), w);
    acc = mfma16(x[6], make_uint4(w[0], w[1], w[2], w[3]), acc);
    acc = mfma16(x[7], make_uint4(w[4], w[5], w[6], w[7]), acc);
  }
};

template <class U, int T, int KW, int D, int KC>
__global__ __launch_bounds__(64 * T * KW) void dense_stream_kernel(GemvLaunch p) {
  load_launch_once(p);
  constexpr int NW = T * KW;
  extern __shared__ __align__(16) uint16_t lds[];
  char* base = reinterpret_cast<char*>(lds);
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int slot = wave / KW, part = wave - slot * KW;
  const int n = lane & 15, g = lane >> 4;
  // items: (batch entry, tile); single-matrix policies compile the batch terms away
  const int tiles = (p.N + 15) / 16, items = (U::BATCHED ? p.batch : 1) * tiles;
  const int K = KC ? KC : p.pa.K, JW = K / U::UK / KW;   // units per wave per tile
  const int xrow = StreamGeom::xrow_bytes(K), xbuf = StreamGeom::xbuf_bytes(p.M, K);
  const int wg0 = blockIdx.x * p.per_wg;
  const int wgend = wg0 + p.per_wg < items ? wg0 + p.per_wg : items;
  if (wg0 >= wgend) return;
  const int R = (wgend - wg0 + T - 1) / T;           // rounds of T tiles
  const int b0 = U::BATCHED ? wg0 / tiles : 0;
  const int nbuf = U::BATCHED ? (wgend - 1) / tiles - b0 + 1 : 1;   // nbuf <= p.xbufs
  char* part_base = base + (U::BATCHED ? p.xbufs : 1) * xbuf;
  char* ring = part_base + T * (KW - 1) * 1024 + wave * D * U::BYTES;

  // activations of the workgroup's batch entries: 1 KB pieces of each row
  const int bpr = K * 2 / 1024;
  if constexpr (U::BATCHED) {
    const int nblk = nbuf * p.M * bpr;
    for (int i = wave; i < nblk; i += NW) {
      const int bi = i / (p.M * bpr), r = i - bi * (p.M * bpr), m = r / bpr, blk = r - m * bpr;
      dma_b128(p.x + (int64_t)(b0 + bi) * p.x_bstride + (int64_t)m * p.x_stride + blk * 512 + lane * 8,
               base + bi * xbuf + m * xrow + blk * 1024);
    }
  } else {
    const int nblk = p.M * bpr;
    for (int i = wave; i < nblk; i += NW) {
      const int m = i / bpr, blk = i - m * bpr;
      dma_b128(p.x + (int64_t)m * p.x_stride + blk * 512 + lane * 8, base + m * xrow + blk * 1024);
    }
  }

  const int U_ = R * JW;
  int ir = 0, ij = 0, is = 0, issued = 0;
  U unit;
  auto set_tile = [&](int rr) {
    int it = wg0 + rr * T + slot;
    if (it >= wgend) it = wgend - 1;                 // idle slot of the last round: reload a valid tile
    const int b = U::BATCHED ? it / tiles : 0, t = it - b * tiles;
    unit.set(p, K, b, t, part * JW, lane, p.N - 1 - t * 16);   // rows past N read row N - 1
  };
  set_tile(0);
  auto issue_next = [&]() {
    unit.issue(ring + is * U::BYTES, ij);
    if (++is == D) is = 0;
    ++issued;
    if (++ij == JW) {
      ij = 0;
      if (++ir < R) set_tile(ir);
    }
  };
  const int pro = U_ < D ? U_ : D;
  for (int u = 0; u < pro; ++u) issue_next();
  // the activation loads went out first: wait for them only
  if (pro == D) wait_vmcnt<U::NDMA * D>();
  else wait_vmcnt<0>();
  wg_barrier_raw();

  const int xr = n < p.M ? n : 0;                    // rows m >= M: never stored
  const uint32_t rl = lds_addr(ring);
  const uint32_t pl = lds_addr(part_base) + slot * (KW - 1) * 1024 + lane * 16;
  const uint32_t xl0 = lds_addr(base) + xr * xrow + part * JW * U::UK * 2 + g * U::XG;
  int cs = 0, u = 0;
  for (int r = 0; r < R; ++r) {
    const int it = wg0 + r * T + slot;
    const int itc = it < wgend ? it : wgend - 1;
    const int b = U::BATCHED ? itc / tiles : 0, t = itc - b * tiles;
    const uint32_t xl = U::BATCHED ? xl0 + (b - b0) * xbuf : xl0;
    f32x4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int j = 0; j < JW; ++j, ++u) {
      if (issued - 1 - u >= D - 1) wait_vmcnt<U::NDMA * (D - 1)>();
      else wait_vmcnt<0>();
      U::consume(rl + cs * U::BYTES, xl + j * U::UK * 2, n, g, acc);
      if (++cs == D) cs = 0;
      if (issued < U_) issue_next();
    }
    if constexpr (KW > 1) {
      if (part > 0) lds_put_f32x4(pl + (part - 1) * 1024, acc);
      wg_barrier_raw();
      if (part == 0) lds_add_parts<KW - 1>(pl, acc);
      wg_barrier_raw();
    }
    if (part == 0 && it < wgend) {
      const int64_t row = (int64_t)t * 16 + n;       // lane (n, g) holds D[m = 4g + i][n]
      if (row < p.N) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (g * 4 + i < p.M) EpiStore::apply(p, b, g * 4 + i, row, acc[i] * p.gs);
      }
    }
  }
  wait_vmcnt<0>();                                   // no load of the prologue outlives the wave
}

// The model's hidden size, the K of every dense decode GEMV: the streaming
// kernels compile it as a constant (their address and activation-staging
// arithmetic then folds; measured 0.1-0.6 us per call), other K take the
// instantiation that reads K at run time.
constexpr int kStreamKc = 2560;

template <class U, int T, int KW, int D, int KC>
bool dense_stream_ready() {
  static bool attr_set = false;
  if (!attr_set) {
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(dense_stream_kernel<U, T, KW, D, KC>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024) != hipSuccess) {
      (void)hipGetLastError();
      return false;
    }
    attr_set = true;
  }
  return true;
}

// Workgroups of dense_stream_kernel<U, T, KW, D, KC> with `lds` bytes of LDS
// one CU holds at once, at most 2 (cached per LDS size).
template <class U, int T, int KW, int D, int KC>
int dense_stream_resident(size_t lds) {
  static size_t keys[16];
  static int vals[16];
  for (int i = 0; i < 16 && keys[i]; ++i)
    if (keys[i] == lds) return vals[i];
  int occ = 1;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(
          &occ, reinterpret_cast<const void*>(dense_stream_kernel<U, T, KW, D, KC>), 64 * T * KW, lds) !=
          hipSuccess ||
      occ < 1) {
    (void)hipGetLastError();
    occ = 1;
  }
  occ = occ < 2 ? occ : 2;
  for (int i = 0; i < 16; ++i)
    if (!keys[i]) {
      keys[i] = lds;
      vals[i] = occ;
      break;
    }
  return occ;
}

template <class U, int T, int KW, int D, int KC>
bool launch_dense_stream_k(GemvLaunch p, int64_t items, size_t lds, bool batched, hipStream_t st) {
  if (!dense_stream_ready<U, T, KW, D, KC>()) return false;
  // One round of T tiles per workgroup where two workgroups fit a CU (a
  // single matrix), instead of rounds of T tiles in one workgroup per CU:
  // the second workgroup's loads overlap the first's dequant and epilogue.
  // Measured as graph replays, us at M = 1 / 3: W6 [13312 x 2560] 10.0 /
  // 10.3 against 10.7-11.1 / 11.0; W6 [16384 x 2560] 10.6 / 11.1 against
  // 11.0 / 11.4; MXFP8 [8192 x 2560] 6.4 / 6.8 against 6.3-6.5 / 7.2;
  // MXFP8 [16384 x 2560] 9.9 / 10.2 against 10.0-10.3 / 10.8 (three rounds
  // of one tile, or one workgroup per tile when more than two would share a
  // CU, were slower).
  const int64_t cus = device_cus();
  const int occ = batched ? 1 : dense_stream_resident<U, T, KW, D, KC>(lds);
  const int64_t per = (items + cus * T * occ - 1) / (cus * T * occ) * T;
  p.per_wg = (int)per;
  const unsigned gx = (unsigned)((items + per - 1) / per);
  hipLaunchKernelGGL((dense_stream_kernel<U, T, KW, D, KC>), dim3(gx), dim3(64 * T * KW), lds, st, p);
  return true;
}

// Launch U's streaming kernel when the call fits it (no split-K, M <= 16, K a
// multiple of 512, 16-byte aligned code planes and 4-byte aligned scale /
// high-bit planes, at least T tiles per CU, the LDS plan within 160 KB);
// false (and nothing launched) otherwise, or when `env` is set to 0.  (The
// second weight plane, W6's H, must be 16-byte aligned.)
template <class U, int T, int KW, int D>
bool launch_dense_stream(GemvLaunch p, int batch, bool on, hipStream_t st, int64_t min_items) {
  if (!on) return false;                              // the format's switch is off: the MFMA core runs
  const int K = p.pa.K, tiles = (p.N + 15) / 16;
  if (p.ksplit != 1 || K % 512 != 0 || p.M > 16 || (K / U::UK) % KW != 0 || batch < 1) return false;
  if (!U::BATCHED && batch != 1) return false;
  if ((reinterpret_cast<uintptr_t>(p.pa.w0) & 15) || (reinterpret_cast<uintptr_t>(p.pa.s) & 3) ||
      (reinterpret_cast<uintptr_t>(p.pa.w1) & 15))
    return false;
  if (batch > 1 && ((p.w0_bstride & 15) || (p.w1_bstride & 15) || (p.s_bstride & 3))) return false;
  const int64_t cus = device_cus(), items = (int64_t)batch * tiles;
  if (items < (min_items >= 0 ? min_items : cus * T)) return false;
  const int64_t per = (items + cus * T - 1) / (cus * T) * T;
  // batch entries one workgroup can span (its first and last item), each with its activations
  const int64_t span = batch > 1 ? (per + tiles - 1) / tiles + 1 : 1;
  if (span > 2) return false;
  const size_t lds = (size_t)span * StreamGeom::xbuf_bytes(p.M, K) + (size_t)T * (KW - 1) * 1024 +
                     (size_t)T * KW * D * U::BYTES;
  if (lds > 160 * 1024) return false;
  p.batch = batch;
  p.xbufs = (int)span;
  // layer-batched calls keep one workgroup per CU (their activation buffers
  // are planned for that many items per workgroup)
  return K == kStreamKc ? launch_dense_stream_k<U, T, KW, D, kStreamKc>(p, items, lds, batch > 1, st)
                        : launch_dense_stream_k<U, T, KW, D, 0>(p, items, lds, batch > 1, st);
}

// Shapes measured as graph replays (T slots, KW waves per tile, D units per
// ring -> us at M = 1 / 3 / 16).
// NVFP4 16384 x 2560, 256-K units: (4, 2, 2) 8.2 / 8.5 / 9.2; (4, 2, 3) 8.5 /
// 8.6 / 9.8; (4, 1, 3) 8.8 / 8.7 / 10.1; (2, 5, 2) 8.7 / 9.4 / 10.3.  With
// 128-K units (two loads each): (4, 2, 3) 8.8 / 8.9 / 9.9; (4, 4, 3) 9.5 / 9.4
// / 10.6; (2, 4, 3) 9.0 / 9.2 / 10.1; (2, 5, 2) 9.1 / 9.5 / 10.5; (1, 10, 2)
// 10.2 / 10.8 / 11.9.  The core: 10.5 / 11.1 / 14.7.  With two workgroups
// of one round per CU (2, 2, 2) is faster at M <= 5 (us at M = 1 / 2 / 3 / 4
// / 5 / 8: 7.3 / 7.4 / 7.6 / 7.8 / 8.0 / 8.5 against 7.7 / 7.7 / 7.8 / 8.0 /
// 8.1 / 8.3; M = 16: 10.0 against 8.9), and it takes matrices of 2 to 4
// tiles per CU, which (4, 2, 2) cannot: [8192 x 2560] 5.7 / 5.7 / 5.9 / 6.2 /
// 6.1 / 6.4 against 5.8 / 7.1 / 8.0 / 8.6 / 9.4 / 10.0 on the few-rows kernel
// (M <= 2) or the core; [13312 x 2560] 7.0 / 7.2 / 7.4 / 7.6 / 7.8 / 8.1
// against the core's 10.0 / 10.4 / 10.9 / 11.9 / 12.8 / 13.3.  Rechecked with
// the K = 2560 instantiation (us at M = 1 / 3 / 16): 16384 x 2560 (2, 2, 2)
// 7.4 / 7.7 / 9.1 against (1, 5, 2) 8.1 / 8.3 / 10.1, (1, 10, 2) 8.7 / 9.0 /
// 10.2, (2, 5, 2) 9.8 / 10.8 / 9.7; 13312 x 2560 7.1 / 7.4 / 9.8 against
// (1, 5, 2) 7.9 / 8.1 / 9.9; only at exactly two tiles per CU, one round of
// one tile per workgroup, does (1, 5, 2) gain a little (8192 x 2560 5.5 /
// 5.8 / 6.8 against 5.7 / 5.9 / 6.9).
inline bool launch_nv4_stream(GemvLaunch p, hipStream_t st) {
  const bool on = switches().nv4_stream;
  const int64_t tiles = (p.N + 15) / 16;
  if (p.M > 5 && tiles >= 4 * (int64_t)device_cus() && launch_dense_stream<StreamNV4, 4, 2, 2>(p, 1, on, st))
    return true;
  return launch_dense_stream<StreamNV4, 2, 2, 2>(p, 1, on, st);
}
// Matrices of 1 to 2 tiles per CU that the few-rows kernel does not take
// (M >= 5, or past its limits): one tile slot per workgroup, two waves, two
// workgroups per CU.  Us at M = 1 / 3 / 4 / 8 against the path these shapes
// take without it: NVFP4 [4096 x 2560] 5.0 / 5.5 / 5.8 / 6.3 against 4.1 /
// 5.4 / 6.0 / 7.9 (the few-rows kernel at M <= 4, then the core); [6144 x
// 2560] 6.5 / 6.9 / 7.2 / 7.7 against 5.1 / 7.3 / 8.4 / 9.9; W6 [4096 x
// 2560] 6.2 / 6.7 / 7.0 / 7.5 against 4.8 / 6.1 / 6.6 / 9.3; [6144 x 2560]
// 8.7 / 9.1 / 9.3 / 9.8 against 6.4 / 9.8 / 10.5 / 12.3.
inline bool launch_nv4_stream_one(GemvLaunch p, hipStream_t st) {
  return launch_dense_stream<StreamNV4, 1, 2, 2>(p, 1, switches().nv4_stream, st);
}
inline bool launch_w6_stream_one(GemvLaunch p, hipStream_t st) {
  return launch_dense_stream<StreamW6, 1, 2, 2>(p, 1, switches().w6_stream, st);
}
// Matrices of half a tile to one tile per CU that the few-rows kernel does
// not take (M >= 5): one tile per workgroup, its K over 8 waves (K a multiple
// of 8 units: 6144) or 5 (2560), two units of ring each.  Us at M = 5 / 8
// (/ 16) against the MFMA core: W6 [2560 x 6144] 8.6 / 9.0 against 16.5 /
// 16.7 (12 waves: 9.2 / -, the activations of 8 rows then overflow LDS; 6:
// 9.0 / 9.7); NVFP4 [2560 x 6144] 6.8 / 7.3 against 12.9 / 13.5; MXFP8 [2560
// x 6144] 7.5 / 8.0 against 13.9 / 15.3; W6 [2048 x 2560] 5.5 / 5.5 / 5.9
// against 8.3 / 8.9 / 10.9 (10 waves: 5.8 / 5.9 / 6.2; 2: 6.7 / 7.2 / 8.3);
// NVFP4 [2048 x 2560] 4.5 / 4.6 / 4.9 against 6.9 / 7.6 / 9.7; MXFP8 [2048 x
// 2560] 4.8 / 4.9 / 5.2 against 7.0 / 7.4 / 8.5.
template <class U>
inline bool launch_stream_tile_per_wg(const GemvLaunch& p, bool on, hipStream_t st) {
  const int64_t tiles = (p.N + 15) / 16, cus = device_cus();
  if (2 * tiles < cus) return false;
  const int units = p.pa.K / U::UK;
  if (units % 8 == 0 && launch_dense_stream<U, 1, 8, 2>(p, 1, on, st, cus / 2)) return true;
  if (units % 5 == 0 && launch_dense_stream<U, 1, 5, 2>(p, 1, on, st, cus / 2)) return true;
  return false;
}
// MXFP8 4096 x 2560 (256 tiles, one per CU; 10 waves of 2 units put a tile's
// 46 KB in flight at once): (1, 10, 2) 5.1 / 5.8 / 6.6; (1, 5, 3) 5.2 / 6.0 /
// 7.0; (1, 5, 4) 5.2 / 5.6 / 6.9; (1, 4, 5) 5.3 / 5.6 / 7.0 (the core: 6.5 /
// 6.8 / 8.7).  Since the K = 2560 instantiation and two workgroups per CU,
// 5 waves of 4 units are faster up to one tile per CU and at M <= 3: 4096 x
// 2560 at M = 3 / 16 5.0 / 5.5 against 5.4 / 5.9; 16384 x 2560 at M = 1 / 3
// 9.7 / 9.9 against 10.0 / 10.2, but at M = 16 13.3 against 11.7.
inline bool launch_mx8_stream(GemvLaunch p, hipStream_t st) {
  const bool on = switches().mx8_stream;
  if ((p.M <= 3 || (p.N + 15) / 16 <= device_cus()) && launch_dense_stream<StreamMX8, 1, 5, 2>(p, 1, on, st))
    return true;
  return launch_dense_stream<StreamMX8, 1, 10, 2>(p, 1, on, st);
}
// W6 8192 x 2560 (512 tiles, two per CU), 256-K units: (2, 2, 2) 7.9 / 8.2 /
// 9.5; (2, 2, 3) 8.1 / 8.3 / 9.6; (2, 2, 4) 8.5 / 8.8 / 10.0; (2, 5, 2) 8.9 /
// 9.5 / 10.6; (2, 2, 5) 8.9 / 9.2 / 10.5; (2, 1, 3) 11.0 / 11.4 / 14.3.  With
// 128-K units (four loads each, three of them 4-byte): (2, 4, 3) 8.6 / 8.8 /
// 9.9; (2, 5, 2) 8.4 / 9.0 / 9.8; (1, 10, 2) 9.0 / 9.3 / 10.2.  The core: 9.8
// / 10.2 / 12.4.  Rechecked with the K = 2560 instantiation: 8192 x 2560 at M =
// 16 8.3 against (1, 5, 2) 8.9, (2, 5, 2) 9.4; 16384 x 2560 at M = 1 / 3 / 16
// (2, 2, 2) 10.6-11.3 / 10.8-10.9 / 12.5 against (1, 5, 2) 11.7-12.0 / 12.1 /
// 14.7, (2, 5, 2) 14.0 / 12.2 / 13.3.
inline bool launch_w6_stream(GemvLaunch p, hipStream_t st) {
  return launch_dense_stream<StreamW6, 2, 2, 2>(p, 1, switches().w6_stream, st);
}
// Single W8 matrices without split-K (fp16 or fp32 scales), as the NVFP4, W6
// and MXFP8 kernels by tiles per CU: 4 slots x 2 waves, 2 x 2, and one tile
// per workgroup (down to half a tile per CU) with its K over KW waves of two
// 256-K units each (K = 2560: 5 waves; K = 6144, the MTP attention output:
// 12).  Other shapes take the MFMA core.
template <class U>
inline bool launch_w8_single_stream(const GemvLaunch& p, hipStream_t st) {
  const bool on = switches().w8_stream;
  const int64_t tiles = (p.N + 15) / 16, cus = device_cus();
  const int units = p.pa.K / 256;
  if (tiles >= 4 * cus) return launch_dense_stream<U, 4, 2, 2>(p, 1, on, st);
  if (tiles >= 2 * cus) return launch_dense_stream<U, 2, 2, 2>(p, 1, on, st);
  if (2 * tiles < cus) return false;
  if (units % 12 == 0) {
    // K = 6144: 12 waves while the activations leave LDS room for their
    // rings (M <= 3), then 8 and 4 (us at M = 5 / 8, fp32 scales: 8.9 / - and
    // - / 10.6 against the MFMA core's 14.6 / 15.2; 6 waves at M = 8: 11.3)
    if (launch_dense_stream<U, 1, 12, 2>(p, 1, on, st, cus / 2)) return true;
    if (launch_dense_stream<U, 1, 8, 2>(p, 1, on, st, cus / 2)) return true;
    return launch_dense_stream<U, 1, 4, 2>(p, 1, on, st, cus / 2);
  }
  if (units % 10 == 0) return launch_dense_stream<U, 1, 5, 2>(p, 1, on, st, cus / 2);
  if (units % 8 == 0) return launch_dense_stream<U, 1, 4, 2>(p, 1, on, st, cus / 2);
  return false;
}

}  // namespace fp4x
