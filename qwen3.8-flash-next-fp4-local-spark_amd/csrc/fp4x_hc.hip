// Hyper-connection mixer kernels (decode, M <= 16, W8 weights).
//
// Fused path (x/fp4x_kernels.py:429-526):
//   hc_down: split-K W8 GEMV; the last-arriving workgroup of each row tile
//            sums the slice partials, writes di = bf16(sum) and the
//            bottleneck bot = bf16(silu(bf16(di / hc))) for rows < lr, and
//            re-arms the tile ticket.
//   hc_up:   W8 GEMV over stream-interleaved rows; a tile of hc*bj stored rows
//            holds the hc stream rows of bj output columns, so the sigmoid
//            gate and the stream mean run in the same workgroup.
// Unfused path (the plugin's 6-kernel mixer, x/fp4patch.py:231-247): W8 GEMV
// with the same split, scaled-SiLU kernel, W8 GEMV, gate-mean kernel.  Both
// paths share the GEMV core, the K split and every epilogue function, so they
// agree bit for bit.
#include <type_traits>

#include "fp4x_mfma.h"
#include "fp4x_stream.h"
#include "../../include/fp4x.h"

namespace fp4x {

// out[m, j] = bf16(sum_s bf16(nrm_s * bf16(sigmoid(g_s))) / hc), s = 0..hc-1
// in order; g_s are bf16-valued gate logits (x/fp4x_kernels.py:486-493).
template <class GF, class NF>
__device__ __forceinline__ uint16_t hc_gate_mean(GF g, NF nrm, int hc) {
  float tot = 0.0f;
  for (int s = 0; s < hc; ++s) {
    const float gate = round_bf16(sigmoid_f32(g(s)));
    tot += round_bf16(nrm(s) * gate);
  }
  return f32_to_bf16(tot / (float)hc);
}

// The same mean with the hc terms made by a quad of lanes: lane s of each
// quad passes stream s's term bf16(nrm_s * bf16(sigmoid(g_s))) (any value
// for s >= hc); lane 0 of the quad gets the bf16 mean, which equals
// hc_gate_mean's bit for bit (the terms added in stream order from 0.0f).
// Every lane of the wave must call it (DPP quad broadcasts).
__device__ __forceinline__ uint16_t hc_quad_mean(float term, int hc) {
  const float t1 = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(term), 0x55, 0xF, 0xF, false));
  const float t2 = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(term), 0xAA, 0xF, 0xF, false));
  const float t3 = __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(term), 0xFF, 0xF, 0xF, false));
  float tot = 0.0f;
  tot += term;
  if (hc > 1) tot += t1;
  if (hc > 2) tot += t2;
  if (hc > 3) tot += t3;
  return f32_to_bf16(tot / (float)hc);
}
__device__ __forceinline__ float hc_gate_term(float nrm, float g) { return round_bf16(nrm * round_bf16(sigmoid_f32(g))); }

struct HcUpArgs {
  const uint16_t* bot; int64_t bot_stride;
  PlaneArgs pa;          // interleaved q [hc*H, K], s [hc*H, K/64]
  const uint16_t* nrm; int64_t nrm_stride;
  uint16_t* out;         // [M, H]
  int M, K, H, hc, bj, lpr, cpl;
};

// The interleaved tile of T = hc*bj stored rows is T/16 MFMA row groups of
// KW waves each; every group runs the same K mapping, batches, MFMA order and
// wave-order reduction as gemv_mfma_kernel<F, KW, CPS, FULL, ...>, so each row's
// sum equals the one w8_linear gives for that row.
template <class F, int KW, int CPS, bool FULL>
__global__ __launch_bounds__(1024) void hc_up_mfma_kernel(HcUpArgs p) {
  constexpr int DP = 4 * KW;
  constexpr int NJ = kNJ;
  extern __shared__ __align__(16) uint16_t lds[];
  const int T = p.hc * p.bj;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int grp = wave / KW, wv = wave - grp * KW;
  const int n = lane & 15, g = lane >> 4;
  const size_t xbytes = ((size_t)p.M * p.K * 2 + 15) & ~(size_t)15;
  float* red = reinterpret_cast<float*>(reinterpret_cast<char*>(lds) + xbytes);
  float* gl = red + (size_t)(T / 16) * (KW > 1 ? KW - 1 : 0) * 256;
  const int nch = p.K / F::KPC, cw = wv * 4 + g;
  const int J = ((nch + CPS - 1) / CPS + DP - 1) / DP, nb = (J + NJ - 1) / NJ;
  const int64_t row = (int64_t)blockIdx.x * T + grp * 16 + n;
  const bool xon = n < p.M;
  const uint16_t* xl0 = lds + (xon ? n : 0) * p.K + CPS * cw * F::KPC;
  f32x4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
  {
    // the bottleneck activations' first staging round goes out ahead of the
    // first weight batch and is written to LDS while the weights are in flight
    XStage<4> xr;
    mfma_xfirst_load(xr, p.bot, p.bot_stride, p.M, 0, p.K, false);
    asm volatile("" ::: "memory");                    // keep the issue order: activations, then weights
    MfmaBatch<F, CPS> cb;
    if constexpr (FULL) mfma_load_full<F, DP, CPS>(cb, F::lane(p.pa, row, CPS * cw));
    else mfma_load_general<F, DP, CPS>(cb, p.pa, row, 0, cw, 0, J, nch);
    mfma_xrest(xr, lds, p.bot, p.bot_stride, p.M, 0, p.K, p.K, false);
    __syncthreads();
    mfma_compute<F, DP, CPS, FULL, false>(cb, xl0, 0, J, cw, nch, acc);
  }
  for (int bi = 1; bi < nb; ++bi) {
    MfmaBatch<F, CPS> cb;
    if constexpr (FULL) mfma_load_full<F, DP, CPS>(cb, F::lane(p.pa, row, CPS * (cw + bi * NJ * DP)));
    else mfma_load_general<F, DP, CPS>(cb, p.pa, row, 0, cw, bi * NJ, J, nch);
    mfma_compute<F, DP, CPS, FULL, false>(cb, xl0 + bi * NJ * CPS * DP * F::KPC, bi * NJ, J, cw, nch, acc);
  }
  // wave-order reduction within each row group
  float* gred = red + (size_t)grp * (KW > 1 ? KW - 1 : 0) * 256;
  if constexpr (KW > 1) {                          // (one wave per row group: nothing to add)
    if (wv > 0) reinterpret_cast<f32x4_t*>(gred)[(wv - 1) * 64 + lane] = acc;
    __syncthreads();
  }
  if (wv == 0) {
#pragma unroll
    for (int w = 1; w < KW; ++w) {
      const f32x4_t o = reinterpret_cast<const f32x4_t*>(gred)[(w - 1) * 64 + lane];
      acc[0] += o[0]; acc[1] += o[1]; acc[2] += o[2]; acc[3] += o[3];
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (g * 4 + i < p.M) gl[(g * 4 + i) * T + grp * 16 + n] = round_bf16(acc[i]);
  }
  __syncthreads();
  // the epilogue on quads of lanes (hc_quad_mean): lane s of a quad takes
  // stream s of one output, blockDim / 4 outputs per pass
  const int qs = (int)threadIdx.x & 3, qsc = qs < p.hc ? qs : p.hc - 1, opp = (int)blockDim.x >> 2;
  for (int t0 = 0; t0 < p.M * p.bj; t0 += opp) {
    const int t = t0 + ((int)threadIdx.x >> 2), tc = t < p.M * p.bj ? t : 0;
    const int m = tc / p.bj, jj = tc - m * p.bj;
    const int64_t j = (int64_t)blockIdx.x * p.bj + jj;
    const float term = hc_gate_term(bf16_to_f32(p.nrm[m * p.nrm_stride + (int64_t)qsc * p.H + j]),
                                    gl[m * T + qsc * p.bj + jj]);
    const uint16_t v = hc_quad_mean(term, p.hc);
    if (qs == 0 && t < p.M * p.bj) p.out[(int64_t)m * p.H + j] = v;
  }
}

template <class F, int CPS>
static void launch_hc_up_full(const HcUpArgs& p, int KW, dim3 grid, dim3 block, size_t lds, hipStream_t st) {
  switch (KW) {
    case 1: hipLaunchKernelGGL((hc_up_mfma_kernel<F, 1, CPS, true>), grid, block, lds, st, p); break;
    case 2: hipLaunchKernelGGL((hc_up_mfma_kernel<F, 2, CPS, true>), grid, block, lds, st, p); break;
    case 4: hipLaunchKernelGGL((hc_up_mfma_kernel<F, 4, CPS, true>), grid, block, lds, st, p); break;
    default: hipLaunchKernelGGL((hc_up_mfma_kernel<F, 8, CPS, true>), grid, block, lds, st, p); break;
  }
}

template <class F>
static void launch_hc_up(const HcUpArgs& p, int KW, int cps, bool full, dim3 grid, size_t lds, hipStream_t st) {
  const int T = p.hc * p.bj;
  const dim3 block((T / 16) * KW * 64);
  if (!full) hipLaunchKernelGGL((hc_up_mfma_kernel<F, kMaxKW, 1, false>), grid, block, lds, st, p);
  else if (cps == 2) launch_hc_up_full<F, 2>(p, KW, grid, block, lds, st);
  else launch_hc_up_full<F, 1>(p, KW, grid, block, lds, st);
}

__global__ __launch_bounds__(256) void hc_scaled_silu_kernel(const uint16_t* d, int64_t d_stride, uint16_t* bot,
                                                             int M, int lr, int hc) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= (int64_t)M * lr) return;
  const int m = (int)(t / lr), n = (int)(t - (int64_t)m * lr);
  bot[t] = hc_scaled_silu(bf16_to_f32(d[m * d_stride + n]), hc);
}

__global__ __launch_bounds__(256) void hc_gate_mean_kernel(const uint16_t* nrm, int64_t nrm_stride, const uint16_t* g,
                                                           int64_t g_stride, uint16_t* out, int M, int H, int hc) {
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= (int64_t)M * H) return;
  const int m = (int)(t / H);
  const int64_t j = t - (int64_t)m * H;
  const uint16_t* gm = g + m * g_stride + j;
  const uint16_t* nm = nrm + m * nrm_stride + j;
  out[t] = hc_gate_mean([&](int s) { return bf16_to_f32(gm[(int64_t)s * H]); },
                        [&](int s) { return bf16_to_f32(nm[(int64_t)s * H]); }, hc);
}

static int hc_fail(const char* msg) {
  set_error(msg);
  return FP4X_ERR_ARG;
}

static bool al(const void* p, int n) { return (reinterpret_cast<uintptr_t>(p) & (n - 1)) == 0; }


// ---------------------------------------------------------------------------
// Single-launch mixer: the down projection (split over C workgroups per tile,
// exactly w8_splitk_kernel's decomposition) and the up projection with its
// gate/stream-mean epilogue (exactly hc_up_mfma_kernel's per-row sums) in one
// launch, so a mixer pays one launch and the up weights stream while the down
// projection runs.
//   * Workgroups 0..D-1 (D = down tiles x C) run one down item each.  The
//     closer of a down tile (the last arriver, or with XCD-local partials its
//     last part) stores di and, device-coherently, the bottleneck, waits for
//     those stores and then advances every workgroup's flag by one (a
//     fetch-add per 128-byte flag line).  (A
//     shared tile count whose last increment advanced the flags cost one more
//     device round trip per mixer: the served mixer 9.9 -> 9.5 us without it.)
//   * Every workgroup (8 waves) then issues the weight loads of its R up
//     tiles (R = 8 / waves per up tile), which stream while it waits.
//     (Issued first, they would share each CU's bandwidth with the down
//     loads and lengthen the critical path.)
//   * One lane of each workgroup waits until its flag reaches the call's
//     generation (s_sleep between reads, at most spin_limit reads); the
//     workgroup then stages the bottleneck with device-coherent loads and
//     runs its up tiles.  (200 workgroups polling one shared counter instead
//     made a hot spot that cost about 13 us per mixer.)
//   * Generations: beside its flag, on the same line, workgroup w keeps the
//     number of tile advances of the calls whose grid held a workgroup w
//     (its ack word).  Every such call advances flag w once per down tile
//     (every down item always runs, so every tile has a closer), and its
//     workgroup w adds the call's tile count to ack w when it starts, so
//     flag w == ack w between calls.  A workgroup therefore waits for flag ==
//     ack + tiles (the ack read at its start): the target does not depend on
//     when the workgroup starts.  A workgroup that only gets a CU after the
//     advances (another kernel holding CUs) finds its flag there already;
//     one whose wait gave up still counts its call, so the late advances
//     cannot satisfy the next call.  (The words wrap modulo 2^32 and are
//     only compared for equality.)
//   * The down items sit in the lowest workgroup indices, which each XCD
//     dispatches in order, so every down item was dispatched before any
//     workgroup that waits on the same XCD, and a wait never depends on a
//     workgroup that waits behind it for a CU; the grid is at most one
//     workgroup per CU.
//   * A wait that reaches spin_limit (which would need another kernel
//     holding the CUs for about a second) writes NaN to that workgroup's
//     outputs and sets bit 0 of the status word sync[1].
constexpr int kMixFlagStride = 32;               // int32 between flags: one 128-byte line each
constexpr int kMixAckAt = 16;                    // a workgroup's ack word, 64 bytes after its flag
constexpr int kMixCountAt = 24;                  // a workgroup slot's call count (every call counts in every slot)

struct HcMixArgs {
  GemvLaunch d;          // down: x, q, s, di (out), bot (out2), lr, hc, split-K slots and tickets
  HcUpArgs u;            // up: bot [M, lr] contiguous, interleaved q/s, normalized, out
  int* sync;             // [0] unused (zero), [1] status (bit 0: a wait gave up,
                         // bit 1: a down tile's partials were not all on its closer's XCD),
                         // [kMixFlagStride * (w + 1)] generation flag of workgroup w,
                         // [kMixFlagStride * (w + 1) + kMixAckAt] its ack word (tile advances of the
                         // calls it has started),
                         // [kMixFlagStride * (w + 1) + kMixCountAt] slot w's call count (the pairs' tags)
  SplitLocal loc;        // XCD-local slots: pairs, status
  int C, D, tiles_d, R, spin_limit;
  int P;                 // workgroups with work; the grid has one per CU, the rest only count the call
};

constexpr int kMixMaxHc = 4;                     // streams the single-launch mixer takes
constexpr int kMixPasses = 8;                    // epilogue passes of 128 outputs (a quad of lanes each)

// SPLIT: the up tiles have workgroups of their own (grid = D + up
// workgroups).  LOCAL: the down items of a tile are the workgroups i < D with
// one residue i mod 8, so they run on one XCD and keep their partials in its
// L2 (w8_splitk_item's LOCAL form); tile counts per residue differ by at most
// one, and the workgroups past a residue's items hold no down item.
template <bool F16S, int KW, int CPS, bool SPLIT, bool LOCAL>
__global__ __launch_bounds__(512) void hc_mix_kernel(HcMixArgs a) {
  using F = FmtW8<F16S>;
  constexpr int DP = 4 * KW;
  extern __shared__ __align__(16) uint16_t lds[];
  __shared__ int s_ok, s_count;
  char* base = reinterpret_cast<char*>(lds);
  const HcUpArgs& u = a.u;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n = lane & 15, g = lane >> 4;
  const int T = u.hc * u.bj, WT = (T / 16) * KW;
  const int slot = wave / WT, ws = wave - slot * WT, grp = ws / KW, wv = ws - grp * KW;
  // up tiles fill the workgroups from the last one down, so that workgroups
  // without a down item take them first (they issue the loads at once)
  const int ntu = u.H / u.bj, tu = (a.P - 1 - (int)blockIdx.x) * a.R + slot;
  const int tuc = tu < ntu ? tu : ntu - 1;          // padding slots recompute the last tile, store nothing
  const int cw = wv * 4 + g;
  const int64_t urow = (int64_t)tuc * T + grp * 16 + n;
  int* flag = a.sync + kMixFlagStride * (blockIdx.x + 1);
  int gen = 0;                                      // the value this call's advances give the flag
  if (threadIdx.x == 0) {
    // the call's count: every call's grid holds every workgroup slot and each
    // slot counts every call in its own word, so all slots agree on it
    // whenever they start (it tags the XCD-local partials)
    const int count = __hip_atomic_load(flag + kMixCountAt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) + 1;
    __hip_atomic_store(flag + kMixCountAt, count, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_count = count;
    if ((int)blockIdx.x < a.P) {
      gen = (int)((uint32_t)__hip_atomic_load(flag + kMixAckAt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) +
                  (uint32_t)a.tiles_d);
      __hip_atomic_store(flag + kMixAckAt, gen, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  if ((int)blockIdx.x >= a.P) return;               // a slot without work: it only counts the call

  // 1. one down item in each of the first D workgroups (the critical path:
  //    its loads go out first)
  int t = -1, c = 0;
  if ((int)blockIdx.x < a.D) {
    if constexpr (LOCAL) {
      const int r = blockIdx.x & 7, k = blockIdx.x >> 3, q = a.tiles_d >> 3, rem = a.tiles_d & 7;
      if (k < (q + (r < rem ? 1 : 0)) * a.C) {
        t = r * q + (r < rem ? r : rem) + k / a.C;
        c = k % a.C;
      }
    } else {
      t = blockIdx.x / a.C;
      c = blockIdx.x - t * a.C;
    }
  }
  if (t >= 0) {
    if (w8_splitk_item<F16S, 8, 2, EpiHcDownShared, LOCAL>(a.d, a.C, t, c, base, a.loc, &s_count)) {
      wait_vmcnt<0>();                              // the tile's bottleneck stores have completed
      // this tile's advance of every workgroup's flag (the flags reach the
      // call's generation when every tile has advanced them)
      for (int w = lane; w < a.P; w += 64)
        __hip_atomic_fetch_add(a.sync + kMixFlagStride * (w + 1), 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }

  // SPLIT: a down item's workgroup is done here; it would only recompute the
  // last up tile as padding, and wait and read the bottleneck for it
  // (measured: the served mixer 11.4 -> 11.1 us).  Its flag still advances,
  // unread.  (With up tiles in the down items' workgroups, the same exit for
  // the workgroups past the up tiles made the synthetic mixer slower, 12.6 ->
  // 12.8 us, also as an instance of its own.)
  if constexpr (SPLIT)
    if ((int)blockIdx.x < a.D) return;

  // 2. the up tiles' weights (one batch per lane) stream during the wait (at
  //    once in a workgroup without a down item)
  MfmaBatch<F, CPS> cb;
  mfma_load_full<F, DP, CPS>(cb, F::lane(u.pa, urow, CPS * cw));
  // ... and the normalized inputs of this lane's epilogue terms, into
  // registers, so that the epilogue waits for no load: each output has a
  // quad of lanes, lane s of the quad taking stream s, and a pass covers
  // blockDim / 4 outputs (outputs past the workgroup's read a valid element
  // and are not stored)
  const int per_slot = u.M * u.bj, nout = a.R * per_slot, opp = (int)blockDim.x >> 2;
  const int qs = (int)threadIdx.x & 3, qsc = qs < u.hc ? qs : u.hc - 1;
  uint16_t nrv[kMixPasses];
#pragma unroll
  for (int q = 0; q < kMixPasses; ++q) {
    const int e = ((int)threadIdx.x >> 2) + q * opp, ec = e < nout ? e : 0;
    const int sl = ec / per_slot, r = ec - sl * per_slot, m = r / u.bj, jj = r - m * u.bj;
    const int tsl = (a.P - 1 - (int)blockIdx.x) * a.R + sl;
    const int64_t j = (int64_t)(tsl < ntu ? tsl : ntu - 1) * u.bj + jj;
    nrv[q] = q * opp < nout ? u.nrm[m * u.nrm_stride + (int64_t)qsc * u.H + j] : (uint16_t)0;
  }
  // the up weights' bf16 operands, made while the bottleneck is outstanding
  // (the plan gives every lane one full batch of kNJ single chunks), so that
  // only the MFMAs follow the flag
  static_assert(CPS == 1 && F::SUB == 1, "one 16-weight chunk per batch slot");
  uint32_t wq[kNJ][8];
#pragma unroll
  for (int j = 0; j < kNJ; ++j) F::deq16(cb.ch[j][0], 0, wq[j]);
  __syncthreads();

  // 3. wait for this workgroup's flag to reach the call's generation
  if (threadIdx.x == 0) {
    int f = __hip_atomic_load(flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    for (int it = 0; f != gen && it < a.spin_limit; ++it) {
      __builtin_amdgcn_s_sleep(4);
      f = __hip_atomic_load(flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    s_ok = f == gen;
    if (!s_ok) __hip_atomic_fetch_or(a.sync + 1, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  const bool ok = s_ok != 0;

  // 4. the bottleneck [M, K] (K = lr), device-coherent loads, into LDS rows of K
  const int K = u.K;
  if (ok) {
    const uint32_t* bg = reinterpret_cast<const uint32_t*>(u.bot);
    uint32_t* bl = reinterpret_cast<uint32_t*>(lds);
    for (int i = threadIdx.x; i < u.M * K / 2; i += blockDim.x)
      bl[i] = __hip_atomic_load(bg + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();

  // 5. up tiles: the MFMA order and wave-order reduction of hc_up_mfma_kernel
  const size_t xbytes = ((size_t)u.M * K * 2 + 15) & ~(size_t)15;
  float* red = reinterpret_cast<float*>(base + xbytes);
  float* gl = red + (size_t)a.R * (T / 16) * (KW > 1 ? KW - 1 : 0) * 256;
  const bool xon = n < u.M;
  const uint16_t* xl0 = lds + (xon ? n : 0) * K + CPS * cw * F::KPC;
  f32x4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
  // the MFMA order of mfma_compute's full path (hc_up_mfma_kernel), on the
  // operands made above
#pragma unroll
  for (int j = 0; j < kNJ; ++j) {
    const uint4* xp = reinterpret_cast<const uint4*>(xl0 + j * DP * F::KPC);
    acc = mfma16(xp[0], make_uint4(wq[j][0], wq[j][1], wq[j][2], wq[j][3]), acc);
    acc = mfma16(xp[1], make_uint4(wq[j][4], wq[j][5], wq[j][6], wq[j][7]), acc);
  }
  float* gred = red + ((size_t)slot * (T / 16) + grp) * (KW > 1 ? KW - 1 : 0) * 256;
  if constexpr (KW > 1) {                          // (one wave per row group: nothing to add)
    if (wv > 0) reinterpret_cast<f32x4_t*>(gred)[(wv - 1) * 64 + lane] = acc;
    __syncthreads();
  }
  if (wv == 0) {
#pragma unroll
    for (int w = 1; w < KW; ++w) {
      const f32x4_t o = reinterpret_cast<const f32x4_t*>(gred)[(w - 1) * 64 + lane];
      acc[0] += o[0]; acc[1] += o[1]; acc[2] += o[2]; acc[3] += o[3];
    }
    float* gls = gl + (size_t)slot * u.M * T;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (g * 4 + i < u.M) gls[(g * 4 + i) * T + grp * 16 + n] = round_bf16(acc[i]);
  }
  __syncthreads();
  // the epilogue of x/fp4x_kernels.py:486-493 on quads of lanes
  // (hc_quad_mean: one sigmoid per lane instead of hc in a row, the terms
  // added in stream order, so every output equals hc_gate_mean's bit for bit)
#pragma unroll
  for (int q = 0; q < kMixPasses; ++q) {
    if (q * opp >= nout) break;                    // (uniform: the same in every thread)
    const int e = ((int)threadIdx.x >> 2) + q * opp, ec = e < nout ? e : 0;
    const int sl = ec / per_slot, r = ec - sl * per_slot, m = r / u.bj, jj = r - m * u.bj;
    const int tsl = (a.P - 1 - (int)blockIdx.x) * a.R + sl;
    const uint16_t v = hc_quad_mean(hc_gate_term(bf16_to_f32(nrv[q]), gl[(size_t)sl * u.M * T + m * T + qsc * u.bj + jj]),
                                     u.hc);
    if (qs == 0 && e < nout && tsl < ntu) u.out[(int64_t)m * u.H + (int64_t)tsl * u.bj + jj] = ok ? v : (uint16_t)0x7fc0u;
  }
}


// The plan keeps the dynamic LDS within 150 KB (the kernel also has a few
// bytes of static LDS); a failed attribute call is cleared so that the
// two-launch fallback does not report it.
template <bool F16S, int KW, bool SPLIT, bool LOCAL>
static bool launch_hc_mix(const HcMixArgs& a, int P, size_t lds, hipStream_t st) {
  auto kern = hc_mix_kernel<F16S, KW, 1, SPLIT, LOCAL>;
  static bool attr_set = false;
  if (!attr_set) {
    if (hipFuncSetAttribute(reinterpret_cast<const void*>(kern), hipFuncAttributeMaxDynamicSharedMemorySize,
                            150 * 1024) != hipSuccess) {
      (void)hipGetLastError();
      return false;
    }
    attr_set = true;
  }
  hipLaunchKernelGGL(kern, dim3(device_cus()), dim3(512), lds, st, a);   // P of them have work
  return true;
}

}  // namespace fp4x

using namespace fp4x;

extern "C" {

int fp4x_hc_down(const void* x, int64_t x_stride, const void* q, const void* s, int s_dtype, void* di, void* bot,
                 int M, int N, int K, int lr, int hc, int ksplit, float* part, int* tickets, void* stream) {
  if (s_dtype != FP4X_DT_F32 && s_dtype != FP4X_DT_F16) return hc_fail("hc_down: scale dtype must be fp32 or fp16");
  if (M < 0 || M > 16 || N <= 0 || K <= 0 || K % 64) return hc_fail("hc_down: bad shape (M <= 16, K % 64 == 0)");
  if (lr < 0 || lr > N || hc <= 0) return hc_fail("hc_down: need 0 <= lr <= N and hc > 0");
  if (ksplit < 1 || ksplit > 64 || K % ksplit || (K / ksplit) % 16) return hc_fail("hc_down: ksplit must divide K into multiples of 16");
  if (ksplit > 1 && (!part || !tickets)) return hc_fail("hc_down: split-K needs scratch");
  if (M > 0 && (!al(x, 16) || x_stride % 8 || x_stride < K)) return hc_fail("hc_down: x must be 16-byte aligned, stride % 8 == 0");
  if (!al(q, 16) || !al(s, s_dtype == FP4X_DT_F16 ? 2 : 4)) return hc_fail("hc_down: misaligned weights");
  if (M == 0) return FP4X_OK;
  GemvLaunch p{};
  p.x = static_cast<const uint16_t*>(x);
  p.x_stride = x_stride;
  p.pa.w0 = static_cast<const uint8_t*>(q);
  p.pa.s = static_cast<const uint8_t*>(s);
  p.pa.K = K;
  p.out = di;
  p.out_dtype = FP4X_DT_BF16;
  p.out_stride = N;
  p.out2 = bot;
  p.lr = lr;
  p.hc = hc;
  p.gs = 1.0f;
  p.M = M;
  p.N = N;
  p.ksplit = ksplit;
  p.part = part;
  p.tickets = tickets;
  hipStream_t st = (hipStream_t)stream;
  // the split-K decomposition fp4x_w8_linear takes for the same (M, N, K, ksplit)
  if (s_dtype == FP4X_DT_F16) {
    if (launch_w8_ktile<true, EpiHcDown>(p, st)) return check_launch("hc_down");
    return launch_gemv_mfma<FmtW8<true>, EpiHcDown>(p, 1, st);
  }
  if (launch_w8_ktile<false, EpiHcDown>(p, st)) return check_launch("hc_down");
  return launch_gemv_mfma<FmtW8<false>, EpiHcDown>(p, 1, st);
}

int fp4x_hc_up(const void* bot, int64_t bot_stride, const void* qi, const void* si, int s_dtype, const void* nrm,
               int64_t nrm_stride, void* out, int M, int K, int H, int hc, int bj, void* stream) {
  if (s_dtype != FP4X_DT_F32 && s_dtype != FP4X_DT_F16) return hc_fail("hc_up: scale dtype must be fp32 or fp16");
  if (M < 0 || M > 16 || K <= 0 || K % 64 || H <= 0 || hc <= 0 || bj <= 0 || H % bj)
    return hc_fail("hc_up: bad shape (M <= 16, K % 64 == 0, H % bj == 0)");
  const int chunks = K / 16;
  // the same slot shape, wave count and path as launch_gemv_mfma picks for W8
  GemvLaunch q{};
  q.pa.w0 = static_cast<const uint8_t*>(qi);
  q.pa.s = static_cast<const uint8_t*>(si);
  const bool pal = s_dtype == FP4X_DT_F16 ? mfma_pair_aligned<FmtW8<true>>(q, 1) : mfma_pair_aligned<FmtW8<false>>(q, 1);
  const int cps = mfma_cps<FmtW8<false>>(chunks) == 2 && pal ? 2 : 1;
  int KW = mfma_kw(chunks, cps);
  const bool full = mfma_full(chunks, KW, cps);
  if (!full) KW = kMaxKW;                       // the GEMV core's general path
  const int T = hc * bj;
  if (T % 16 || (T / 16) * KW > 16) return hc_fail("hc_up: hc*bj must be a multiple of 16 with at most 16 waves per tile");
  const size_t lds = (((size_t)(M < 1 ? 1 : M) * K * 2 + 15) & ~(size_t)15) + (size_t)(T / 16) * (KW - 1) * 256 * 4 +
                     (size_t)16 * T * 4;
  if (lds > 96 * 1024) return hc_fail("hc_up: K too large for the LDS activation stage");
  if (M > 0 && (!al(bot, 16) || bot_stride % 8 || bot_stride < K)) return hc_fail("hc_up: bot must be 16-byte aligned, stride % 8 == 0");
  if (!al(qi, 16) || !al(si, s_dtype == FP4X_DT_F16 ? 2 : 4)) return hc_fail("hc_up: misaligned weights");
  if (M == 0) return FP4X_OK;
  HcUpArgs p{};
  p.bot = static_cast<const uint16_t*>(bot);
  p.bot_stride = bot_stride;
  p.pa.w0 = static_cast<const uint8_t*>(qi);
  p.pa.s = static_cast<const uint8_t*>(si);
  p.pa.K = K;
  p.nrm = static_cast<const uint16_t*>(nrm);
  p.nrm_stride = nrm_stride;
  p.out = static_cast<uint16_t*>(out);
  p.M = M; p.K = K; p.H = H; p.hc = hc; p.bj = bj;
  dim3 grid(H / bj);
  hipStream_t st = (hipStream_t)stream;
  if (s_dtype == FP4X_DT_F16) launch_hc_up<FmtW8<true>>(p, KW, cps, full, grid, lds, st);
  else launch_hc_up<FmtW8<false>>(p, KW, cps, full, grid, lds, st);
  return check_launch("hc_up");
}

int fp4x_hc_mix(const void* x, int64_t x_stride, const void* q, const void* s, int s_dtype, void* di, void* bot,
                int M, int N, int K, int lr, int hc, int ksplit, float* part, int* tickets, int n_tickets,
                const void* qi, const void* si, const void* nrm, int64_t nrm_stride, void* out, int H, int bj,
                void* stream) {
  // one launch when both halves take the planned decompositions; else the two entry points
  auto two = [&]() {
    int rc = fp4x_hc_down(x, x_stride, q, s, s_dtype, di, bot, M, N, K, lr, hc, ksplit, part, tickets, stream);
    if (rc != FP4X_OK) return rc;
    return fp4x_hc_up(bot, lr, qi, si, s_dtype, nrm, nrm_stride, out, M, lr, H, hc, bj, stream);
  };
  if (!switches().hc_mix || M < 1 || M > 16 || N <= 0 || K <= 0 || K % 64 || lr <= 0 || lr > N || lr % 64 ||
      hc <= 0 || bj <= 0 || H <= 0 || H % bj || ksplit < 2 || ksplit > 64 || K % ksplit || (K / ksplit) % 16 ||
      !part || !tickets || (s_dtype != FP4X_DT_F32 && s_dtype != FP4X_DT_F16))
    return two();
  if (!al(x, 16) || x_stride % 8 || x_stride < K || !al(q, 16) || !al(s, 4) || !al(qi, 16) || !al(si, 4) ||
      !al(bot, 4))
    return two();
  GemvLaunch d{};
  d.x = static_cast<const uint16_t*>(x);
  d.x_stride = x_stride;
  d.pa.w0 = static_cast<const uint8_t*>(q);
  d.pa.s = static_cast<const uint8_t*>(s);
  d.pa.K = K;
  d.out = di;
  d.out_dtype = FP4X_DT_BF16;
  d.out_stride = N;
  d.out2 = bot;
  d.lr = lr;
  d.hc = hc;
  d.gs = 1.0f;
  d.M = M;
  d.N = N;
  d.ksplit = ksplit;
  d.part = part;
  d.tickets = tickets;
  d.batch = 1;
  d.per_wg = 1;
  d.xbufs = 1;
  int C = 0;
  size_t lds_d = 0;
  const int tiles_d = (N + 15) / 16;
  // tile tickets one 128-byte line apart from the start of the buffer (the
  // 200 items' ticket atomics of a mixer would otherwise queue on two lines);
  // the status word and the flags in its last 32 * (cus + 1) ints,
  // at the same place for every shape the buffer serves
  d.tstride = kMixFlagStride;
  const int64_t sync_at =
      ((int64_t)n_tickets - (int64_t)kMixFlagStride * (device_cus() + 1)) & ~(int64_t)(kMixFlagStride - 1);
  if (sync_at < (int64_t)tiles_d * kMixFlagStride) return two();
  if (!w8_splitk_plan(d, C, lds_d)) return two();
  // the up projection's shape, as fp4x_hc_up plans it
  const int chunks = lr / 16;
  GemvLaunch qq{};
  qq.pa.w0 = static_cast<const uint8_t*>(qi);
  qq.pa.s = static_cast<const uint8_t*>(si);
  const bool pal = s_dtype == FP4X_DT_F16 ? mfma_pair_aligned<FmtW8<true>>(qq, 1) : mfma_pair_aligned<FmtW8<false>>(qq, 1);
  const int cps = mfma_cps<FmtW8<false>>(chunks) == 2 && pal ? 2 : 1;
  const int KW = mfma_kw(chunks, cps);
  const int T = hc * bj;
  if (cps != 1 || !mfma_full(chunks, KW, cps) || (chunks + 4 * KW - 1) / (4 * KW) > kNJ || T % 16) return two();
  const int WT = (T / 16) * KW;
  if (WT > 8 || 8 % WT || (KW != 1 && KW != 2 && KW != 4)) return two();
  // grid: when the CUs allow, the down items and then separate workgroups for
  // all up tiles (which load them at once); otherwise max(D, up workgroups),
  // the up tiles sharing workgroups with down items (measured: spreading only
  // part of the up tiles to extra workgroups is slower than not at all)
  const int cus = device_cus();
  // XCD-local down partials (w8_splitk_item's LOCAL form): at most 8 parts per
  // tile, a generation word per tile on the flag lines, and the parts' 64-bit
  // (partial, generation) pairs in the caller's slot buffer; the down items
  // then span 8 residues x the most tiles a residue holds x C workgroups
  const bool local = switches().hc_xcd && C <= 8 && tiles_d <= cus && al(part, 8) &&
                     (int64_t)tiles_d * C * M * 16 * 3 + 2 <= (int64_t)ksplit * 16 * N;
  const int R = 8 / WT, ntu = H / bj, D = local ? 8 * ((tiles_d + 7) / 8) * C : tiles_d * C;
  if (hc > kMixMaxHc || R * M * bj > kMixPasses * 128) return two();
  const int need_u = (ntu + R - 1) / R;
  const bool split = D + need_u <= cus;
  const int P = split ? D + need_u : (D > need_u ? D : need_u);
  if (P > cus) return two();
  const size_t lds_u = (((size_t)M * lr * 2 + 15) & ~(size_t)15) + (size_t)R * (T / 16) * (KW - 1) * 1024 +
                       (size_t)R * M * T * 4;
  const size_t lds = lds_d > lds_u ? lds_d : lds_u;
  if (lds > 150 * 1024) return two();
  HcMixArgs a{};
  a.d = d;
  a.u.bot = static_cast<const uint16_t*>(bot);
  a.u.bot_stride = lr;
  a.u.pa.w0 = static_cast<const uint8_t*>(qi);
  a.u.pa.s = static_cast<const uint8_t*>(si);
  a.u.pa.K = lr;
  a.u.nrm = static_cast<const uint16_t*>(nrm);
  a.u.nrm_stride = nrm_stride;
  a.u.out = static_cast<uint16_t*>(out);
  a.u.M = M; a.u.K = lr; a.u.H = H; a.u.hc = hc; a.u.bj = bj;
  a.sync = tickets + sync_at;
  // part: the two-launch path's slots of this shape, then the pairs (zero
  // before the first call: no zero word carries a tag)
  a.loc.pairs = reinterpret_cast<uint64_t*>(part + (((int64_t)tiles_d * C * M * 16 + 1) & ~(int64_t)1));
  a.loc.status = a.sync + 1;
  // the closer waits only for parts of its tile that were dispatched before it
  // and wait on nothing, so its reads keep a floor whatever the flag limit
  a.loc.spin_limit = switches().hc_spin_limit > (1 << 16) ? switches().hc_spin_limit : 1 << 16;
  a.C = C;
  a.D = D;
  a.tiles_d = tiles_d;
  a.R = R;
  a.P = P;
  a.spin_limit = switches().hc_spin_limit;
  hipStream_t st = (hipStream_t)stream;
  auto go = [&](auto f16s, auto loc) {
    constexpr bool F = decltype(f16s)::value, L = decltype(loc)::value;
    if (split) return KW == 1 ? launch_hc_mix<F, 1, true, L>(a, P, lds, st)
                      : KW == 2 ? launch_hc_mix<F, 2, true, L>(a, P, lds, st)
                                : launch_hc_mix<F, 4, true, L>(a, P, lds, st);
    return KW == 1 ? launch_hc_mix<F, 1, false, L>(a, P, lds, st)
           : KW == 2 ? launch_hc_mix<F, 2, false, L>(a, P, lds, st)
                     : launch_hc_mix<F, 4, false, L>(a, P, lds, st);
  };
  using T_ = std::true_type;
  using F_ = std::false_type;
  const bool launched = s_dtype == FP4X_DT_F16 ? (local ? go(T_{}, T_{}) : go(T_{}, F_{}))
                                               : (local ? go(F_{}, T_{}) : go(F_{}, F_{}));
  if (!launched) return two();
  return check_launch("hc_mix");
}

int fp4x_hc_scaled_silu(const void* d, int64_t d_stride, void* bot, int M, int lr, int hc, void* stream) {
  if (M < 0 || lr < 0 || hc <= 0 || d_stride < lr) return hc_fail("hc_scaled_silu: bad shape");
  const int64_t n = (int64_t)M * lr;
  if (n == 0) return FP4X_OK;
  hipLaunchKernelGGL(hc_scaled_silu_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                     static_cast<const uint16_t*>(d), d_stride, static_cast<uint16_t*>(bot), M, lr, hc);
  return check_launch("hc_scaled_silu");
}

int fp4x_hc_gate_mean(const void* nrm, int64_t nrm_stride, const void* g, int64_t g_stride, void* out, int M, int H,
                      int hc, void* stream) {
  if (M < 0 || H < 0 || hc <= 0 || nrm_stride < (int64_t)hc * H || g_stride < (int64_t)hc * H)
    return hc_fail("hc_gate_mean: bad shape");
  const int64_t n = (int64_t)M * H;
  if (n == 0) return FP4X_OK;
  hipLaunchKernelGGL(hc_gate_mean_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream,
                     static_cast<const uint16_t*>(nrm), nrm_stride, static_cast<const uint16_t*>(g), g_stride,
                     static_cast<uint16_t*>(out), M, H, hc);
  return check_launch("hc_gate_mean");
}

}  // extern "C"
