// LM-head kernels of the fast target head (x/fp4patch.py:337-393):
//   refine_mx8: exact MXFP8 logits of C candidate rows per token, scattered in
//               place into the [M, V] coarse logits (x/fp4x_kernels.py:367-388).
//   topk_rows:  top-C row selection under (value desc, index asc), replacing
//               torch.topk(coarse, C) (x/fp4patch.py:377).
#include "fp4x_kernels.h"
#include "../../include/fp4x.h"

namespace fp4x {

// ------------------------------------------------------------------ refine
struct RefineArgs {
  void* out; int out_dtype; int64_t out_stride;
  const uint16_t* x;           // [M, K] contiguous
  const int64_t* idx;          // [M, C]
  PlaneArgs pa;                // candidate rows [V, K] (MXFP8 or NVFP4)
  float gs;                    // NVFP4 global scale
  int M, C, K, V, lpr, cpl;
};

// The candidate rows go through the chunk layout and lane butterfly of
// mx8_linear, accumulated with IEEE fp32 fma (AccFma) so every rounding is
// specified.  MXFP8: e4m3 * 2^(e-127) is exact in bf16 and in fp32, and its
// product with a bf16 activation is exact, as in the reference's fp32 dot;
// the sum goes in place to out[m, idx[m, c]] (x/fp4x_kernels.py:367-388).
// NVFP4 (DENSE): e2m1 * e4m3 is exact in bf16; out[m, c] = sum * gs in fp32,
// NaN for an index outside [0, V) (x/fp4x_kernels.py:391-417).
// Every chunk load of the batch goes out unconditionally, at an in-bounds
// address (row 0 for an invalid candidate, chunk 0 past the row's chunks):
// loads under a branch would each be waited for at the branch's join, one
// memory round trip per chunk.  compute_batch skips the dead chunks, and an
// invalid candidate's sum is never stored.
template <class F>
__device__ __forceinline__ void load_batch_inbounds(ChunkBatch<F, 1>& b, const PlaneArgs& a, int64_t row, int cend,
                                                    int lrow, int lpr, int jb, int cpl) {
  const int64_t r = row >= 0 ? row : 0;
#pragma unroll
  for (int j = 0; j < kCplBatch; ++j) {
    const int jj = jb + j, c = lrow + jj * lpr;
    b.ch[0][j] = F::load(a, r, jj < cpl && c < cend ? c : 0);
  }
}

template <class F, bool DENSE>
__global__ __launch_bounds__(kThreads) void refine_kernel(RefineArgs p) {
  asm volatile("" ::"s"(p.out), "s"(p.out_dtype), "s"(p.out_stride), "s"(p.x), "s"(p.idx), "s"(p.pa.w0),
               "s"(p.pa.s), "s"(p.pa.K), "s"(p.gs), "s"(p.M), "s"(p.C), "s"(p.K), "s"(p.V), "s"(p.lpr), "s"(p.cpl));
  extern __shared__ __align__(16) uint16_t lds_x[];
  const int m = blockIdx.y;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int lpr = p.lpr, lrow = lane & (lpr - 1), slot = lane / lpr, spw = 64 / lpr;
  const int cand = blockIdx.x * (kWaves * spw) + wave * spw + slot;
  int64_t rows[1] = {-1};
  if (cand < p.C) {
    const int64_t r = p.idx[(int64_t)m * p.C + cand];
    rows[0] = (r >= 0 && r < p.V) ? r : -1;
  }
  float acc[1][1] = {{0.0f}};
  for (int jb = 0; jb < p.cpl; jb += kCplBatch) {
    ChunkBatch<F, 1> cb;
    load_batch_inbounds<F>(cb, p.pa, rows[0], p.K / F::KPC, lrow, lpr, jb, p.cpl);
    if (jb == 0) {
      stage_x<1>(lds_x, p.x + (int64_t)m * p.K, p.K, 1, 0, p.K);
      __syncthreads();
    }
    compute_batch<F, 1, 1, const uint16_t*, AccFma>(cb, (const uint16_t*)lds_x, p.K, 0, 1, 0, p.K / F::KPC, lrow,
                                                    lpr, jb, p.cpl, acc);
  }
  const float v = group_allreduce(acc[0][0], lpr);
  if constexpr (DENSE) {
    if (lrow == 0 && cand < p.C)
      reinterpret_cast<float*>(p.out)[(int64_t)m * p.C + cand] = rows[0] >= 0 ? v * p.gs : __builtin_nanf("");
  } else {
    if (lrow == 0 && rows[0] >= 0) store_out(p.out, (int64_t)m * p.out_stride + rows[0], p.out_dtype, v);
  }
}

// ------------------------------------------------------------------ top-k
// Two launches per call, which exchange data only across the launch boundary
// (no grid-wide waits, no cross-workgroup fences):
//   A  slice maxima: smax[m][s] = largest order key of slice s of row m, the
//      elements [S*s, S*s + S) (S = 16 for rows up to 2^19 elements, else the
//      next power of two keeping at most 32768 slices).  The streaming INT2
//      head writes them from its epilogue (fp4x_int2_topk), so A is then free.
//   B  one workgroup per row: T0 = the C-th largest slice maximum (a lower
//      bound of the C-th largest element: C slices each hold an element
//      >= T0); the slices whose maximum reaches T0 (about C of them) are the
//      only ones read back; their elements with key >= T0 are sorted by the
//      total order (value desc, index asc) and the first C indices written.
//      More than 4096 such slices or candidates (massive ties), or fewer than
//      C slices, take the exact threshold path over the whole row instead;
//      rows of at most 4096 elements sort the whole row.
constexpr int kTkCap = 4096;      // candidates (and candidate slices) per row
constexpr int kTkMaxSlices = 32768;

// Composite order key: larger = larger value, then smaller index.
__device__ __forceinline__ uint64_t tk_comp(uint32_t key, uint32_t i) {
  return ((uint64_t)key << 32) | (uint64_t)(0xffffffffu - i);
}

// Slice length for a row of V elements (a power of two >= 16).
__host__ __device__ inline int tk_slice(int V) {
  int S = 16;
  while ((V + S - 1) / S > kTkMaxSlices) S <<= 1;
  return S;
}
__host__ __device__ inline int64_t tk_smax_stride(int V) {
  const int ns = (V + tk_slice(V) - 1) / tk_slice(V);
  return (ns + 7) & ~7;
}

struct TkHist {
  uint32_t hist[256];
  int sel_bin, sel_above;
};

// Walk a 256-bin histogram from the top: the bin holding the k-th largest
// element (k >= 1) and the count of elements in higher bins (bin 0 if the
// count never reaches k).  Wave 0 holds four bins per lane, top bins first,
// scans the lane sums and picks the first lane whose running count reaches k.
__device__ void tk_walk(TkHist& h, int k) {
  if (threadIdx.x < 64) {
    const int l = threadIdx.x;
    uint32_t c[4], sum = 0;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      c[r] = h.hist[255 - 4 * l - r];
      sum += c[r];
    }
    uint32_t incl = sum;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const uint32_t v = __shfl_up(incl, d, 64);
      if (l >= d) incl += v;
    }
    const uint64_t hit = __ballot(incl >= (uint32_t)k);
    const int L = hit ? __ffsll((unsigned long long)hit) - 1 : 63;
    if (l == L) {
      uint32_t above = incl - sum;
      int b = 0;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int bin = 255 - 4 * l - r;
        if (above + c[r] >= (uint32_t)k || bin == 0) { b = bin; break; }
        above += c[r];
      }
      h.sel_bin = b;
      h.sel_above = (int)above;
    }
  }
  __syncthreads();
}

// hist[bin] += 1 for every lane with valid set: lanes holding the same bin
// add together (one LDS atomic per distinct bin per wave), so the high bytes
// of a skewed key set (the slice maxima, logits) do not serialize on one
// address.
__device__ __forceinline__ void tk_hist_add(uint32_t* hist, uint32_t bin, bool valid) {
  const int lane = threadIdx.x & 63;
  uint64_t active = __ballot(valid);
  while (active) {
    const int leader = __ffsll((unsigned long long)active) - 1;
    const uint32_t lb = __shfl(bin, leader, 64);
    const uint64_t same = __ballot(valid && bin == lb) & active;
    if (lane == leader) atomicAdd(&hist[lb], (uint32_t)__popcll(same));
    active &= ~same;
  }
}

// Exact k-th largest key among n keys get(i) of BITS bits (16 or 32; one
// 8-bit radix round per byte); *n_above receives the number of keys strictly
// above it.  The first round's bins are the keys' high bytes, skewed for
// logits, so its adds are wave-aggregated; later rounds' bins are spread out.
template <int BITS, class Get>
__device__ uint32_t tk_kth(TkHist& h, Get get, int n, int k, int* n_above) {
  uint32_t prefix = 0;
  int above = 0;
#pragma unroll
  for (int r = 0; r < BITS / 8; ++r) {
    const int sh = BITS - 8 * (r + 1);
    for (int i = threadIdx.x; i < 256; i += blockDim.x) h.hist[i] = 0;
    __syncthreads();
    if (r == 0) {
      for (int i0 = 0; i0 < n; i0 += blockDim.x) {
        const int i = i0 + threadIdx.x;
        tk_hist_add(h.hist, i < n ? get(i) >> sh : 0u, i < n);
      }
    } else {
      for (int i = threadIdx.x; i < n; i += blockDim.x) {
        const uint32_t kk = get(i);
        if ((kk >> (sh + 8)) == prefix) atomicAdd(&h.hist[(kk >> sh) & 255u], 1u);
      }
    }
    __syncthreads();
    tk_walk(h, k - above);
    prefix = (prefix << 8) | (uint32_t)h.sel_bin;
    above += h.sel_above;
    __syncthreads();
  }
  *n_above = above;
  return prefix;
}

// Wave-aggregated append of v (when flag) to list[*count]; positions past
// cap are counted but not written.
template <class T>
__device__ __forceinline__ void tk_append(T* list, int* count, int cap, bool flag, T v) {
  const uint64_t mask = __ballot(flag);
  if (!mask) return;
  const int lane = threadIdx.x & 63;
  const int leader = __ffsll((unsigned long long)mask) - 1;
  int base = 0;
  if (lane == leader) base = atomicAdd(count, __popcll(mask));
  base = __shfl(base, leader, 64);
  if (flag) {
    const int pos = base + __popcll(mask & ((1ull << lane) - 1ull));
    if (pos < cap) list[pos] = v;
  }
}

// Row elements as order keys: Elem16 (bf16 rows) and Elem32 (fp32 rows).
// key() is the full order key, key16() the key of the element rounded to
// bf16 (round to nearest even, a monotone map), which the slice maxima and
// the candidate threshold use for both: every element whose full key is among
// the row's C largest has a key16 at least the threshold derived from them.
struct Elem16 {
  using T = uint16_t;
  static constexpr int BITS = 16, PER16 = 8;      // key bits, elements per 16 bytes
  __device__ static uint32_t key(T v) { return tk_key(v); }
  __device__ static uint32_t key16(T v) { return tk_key(v); }
  __device__ static uint32_t at(const uint4& q, int i) {   // element i of a 16-byte item
    const uint32_t d = i < 4 ? (i < 2 ? q.x : q.y) : (i < 6 ? q.z : q.w);
    return i & 1 ? d >> 16 : d & 0xffffu;
  }
};
struct Elem32 {
  using T = uint32_t;
  static constexpr int BITS = 32, PER16 = 4;
  __device__ static uint32_t key(T v) { return tk_key32(v); }
  __device__ static uint32_t key16(T v) { return tk_key(f32_to_bf16(__uint_as_float(v))); }
  __device__ static uint32_t at(const uint4& q, int i) { return i == 0 ? q.x : i == 1 ? q.y : i == 2 ? q.z : q.w; }
};

// A: slice maxima (key16) of rows whose slices are S elements (S a multiple of 16).
template <class E>
__global__ __launch_bounds__(256) void topk_slicemax_kernel(const typename E::T* logits, int64_t stride, int V,
                                                            uint16_t* smax, int64_t sstride) {
  const int m = blockIdx.y;
  const typename E::T* row = logits + (int64_t)m * stride;
  const int S = tk_slice(V), ns = (V + S - 1) / S;
  const int sl = blockIdx.x * blockDim.x + threadIdx.x;
  if (sl >= ns) return;
  uint32_t mx = 0;
  const int e0 = sl * S;
  for (int e = e0; e < e0 + S; e += E::PER16) {
    if (e + E::PER16 <= V) {
      const uint4 v = *reinterpret_cast<const uint4*>(row + e);
#pragma unroll
      for (int q = 0; q < E::PER16; ++q) mx = max(mx, E::key16((typename E::T)E::at(v, q)));
    } else {
      for (int i = e; i < V; ++i) mx = max(mx, E::key16(row[i]));
    }
  }
  smax[(int64_t)m * sstride + sl] = (uint16_t)mx;
}

// Descending bitonic sort of a[0, n2), n2 a power of two.
__device__ void tk_sort(uint64_t* a, int n2) {
  for (int size = 2; size <= n2; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int t = threadIdx.x; t < n2 / 2; t += blockDim.x) {
        const int i = 2 * t - (t & (stride - 1));
        const int j = i + stride;
        const bool desc = (i & size) == 0;
        const uint64_t x = a[i], y = a[j];
        if ((x < y) == desc) { a[i] = y; a[j] = x; }
      }
      __syncthreads();
    }
  }
}

// The exact path: T = the C-th largest key of the row, the elements above
// it, then ties at T in index order; n = C on return in cand[0, C).
template <class E>
__device__ void tk_exact(const typename E::T* row, int V, int C, uint64_t* cand, TkHist& h, int* n_sh) {
  if (threadIdx.x == 0) *n_sh = 0;
  __syncthreads();
  int above;
  const uint32_t T = tk_kth<E::BITS>(h, [&](int i) { return E::key(row[i]); }, V, C, &above);
  for (int i0 = 0; i0 < V; i0 += blockDim.x) {
    const int i = i0 + threadIdx.x;
    const uint32_t key = i < V ? E::key(row[i]) : 0u;
    tk_append<uint64_t>(cand, n_sh, kTkCap, i < V && key > T, tk_comp(key, i));
  }
  __syncthreads();
  const int need = C - above;
  if (threadIdx.x < 64) {
    int taken = 0;
    for (int i0 = 0; i0 < V && taken < need; i0 += 64) {
      const int i = i0 + threadIdx.x;
      const bool eq = i < V && E::key(row[i]) == T;
      const uint64_t mask = __ballot(eq);
      const int pos = taken + __popcll(mask & ((1ull << threadIdx.x) - 1ull));
      if (eq && pos < need) cand[above + pos] = tk_comp(T, i);
      taken += __popcll(mask);
    }
  }
  __syncthreads();
}

// Descending bitonic sort of n2 <= blockDim.x keys (n2 a power of two), one
// per thread in a register: stages with partners in the same wave exchange by
// shuffles, the others (stride >= 64) through xch[] in LDS.  Thread t < n2
// holds element t and ends with the t-th largest; threads past n2 sort their
// own values among themselves.  Every thread of the workgroup must call it.
__device__ uint64_t tk_sort_regs(uint64_t a, int n2, uint64_t* xch) {
  const int t = threadIdx.x;
  for (int size = 2; size <= n2; size <<= 1) {
    const bool desc = (t & size) == 0;
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      uint64_t b;
      if (stride >= 64) {
        xch[t] = a;
        __syncthreads();
        b = xch[t ^ stride];
        __syncthreads();
      } else {
        b = __shfl_xor(a, stride, 64);
      }
      const bool lower = (t & stride) == 0;        // t is the first of the pair
      const bool keep_max = lower == desc;
      a = keep_max ? (a > b ? a : b) : (a < b ? a : b);
    }
  }
  return a;
}

// Sort cand[0, n) descending and write the first C indices.
__device__ void tk_finish(uint64_t* cand, int n, int C, int64_t* out) {
  int n2 = 1;
  while (n2 < n) n2 <<= 1;
  if (n2 <= (int)blockDim.x && n2 >= 64) {
    const int t = threadIdx.x;
    const uint64_t a = t < n ? cand[t] : 0ull;
    __syncthreads();                                // cand doubles as the exchange buffer
    const uint64_t r = tk_sort_regs(a, n2, cand);   // every thread takes part in the barriers
    if (t < C) out[t] = (int64_t)(0xffffffffu - (uint32_t)(r & 0xffffffffu));
    return;
  }
  for (int i = n + threadIdx.x; i < n2; i += blockDim.x) cand[i] = 0;
  __syncthreads();
  tk_sort(cand, n2);
  for (int i = threadIdx.x; i < C; i += blockDim.x) out[i] = (int64_t)(0xffffffffu - (uint32_t)(cand[i] & 0xffffffffu));
}

// ---- B: one workgroup of 16 waves per row, no cross-wave atomics ----------
constexpr int kRsThreads = 1024;
constexpr int kRsWaves = kRsThreads / 64;
constexpr int kRsVptMax = kTkMaxSlices / 8 / kRsThreads;   // 8-slice vectors per thread (registers)
constexpr int kRsIpt = 2;                                // candidate 8-element items per thread per round
constexpr int kRsSortThreads = 256;                      // the sort runs on the first 4 waves

// Inclusive prefix sum over the 64 lanes of a wave, by DPP: row shifts build
// the prefix within each row of 16 lanes, row broadcasts carry rows 0-1 and
// 2 into rows 1-3.
__device__ __forceinline__ int rs_wave_scan(int v) {
  int x = v;
  x += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xF, 0xF, true);   // row_shr:1
  x += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xF, 0xF, true);   // row_shr:2
  x += __builtin_amdgcn_update_dpp(0, v, 0x113, 0xF, 0xF, true);   // row_shr:3  (sums of 4)
  x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xF, 0xE, false);  // row_shr:4 into lanes 4-15 of a row
  x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xF, 0xC, false);  // row_shr:8 into lanes 8-15
  x += __builtin_amdgcn_update_dpp(0, x, 0x142, 0xA, 0xF, false);  // row_bcast:15 into rows 1, 3
  x += __builtin_amdgcn_update_dpp(0, x, 0x143, 0xC, 0xF, false);  // row_bcast:31 into rows 2, 3
  return x;
}

// Exclusive prefix of v over the workgroup in thread order; *total = sum.
// Two barriers; slots: kRsWaves ints.
__device__ __forceinline__ int rs_scan(int v, int* slots, int* total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int incl = rs_wave_scan(v);
  if (lane == 63) slots[wave] = incl;
  __syncthreads();
  int before = 0, tot = 0;
#pragma unroll
  for (int w = 0; w < kRsWaves; ++w) {
    const int sw = slots[w];
    before += w < wave ? sw : 0;
    tot += sw;
  }
  __syncthreads();
  *total = tot;
  return before + incl - v;
}

// The bin holding the k-th largest element of a 256-bin histogram (k >= 1)
// and the count in higher bins (bin 0 if the count never reaches k): wave 0,
// four bins per lane, top bins first, DPP scan of the lane sums.
__device__ void rs_walk(TkHist& h, int k) {
  if (threadIdx.x < 64) {
    const int l = threadIdx.x;
    uint32_t c[4], sum = 0;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      c[r] = h.hist[255 - 4 * l - r];
      sum += c[r];
    }
    const uint32_t incl = (uint32_t)rs_wave_scan((int)sum);
    const uint64_t hit = __ballot(incl >= (uint32_t)k);
    const int L = hit ? __ffsll((unsigned long long)hit) - 1 : 63;
    if (l == L) {
      uint32_t above = incl - sum;
      int b = 0;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int bin = 255 - 4 * l - r;
        if (above + c[r] >= (uint32_t)k || bin == 0) { b = bin; break; }
        above += c[r];
      }
      h.sel_bin = b;
      h.sel_above = (int)above;
    }
  }
  __syncthreads();
}

// Value of lane (lane ^ s) of the wave, s = 1 .. 32 (a constant after unrolling).
__device__ __forceinline__ uint32_t rs_xor_lane(uint32_t v, int s) {
  if (s == 1) return __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, false);    // quad_perm [1,0,3,2]
  if (s == 2) return __builtin_amdgcn_mov_dpp(v, 0x4E, 0xF, 0xF, false);    // quad_perm [2,3,0,1]
  if (s == 4) {
    // lane i of an 8-group: half mirror gives 7 - i, a quad reversal then (7 - i) ^ 3 = i ^ 4
    const uint32_t h = __builtin_amdgcn_mov_dpp(v, 0x141, 0xF, 0xF, false);
    return __builtin_amdgcn_mov_dpp(h, 0x1B, 0xF, 0xF, false);
  }
  if (s == 8) return __builtin_amdgcn_mov_dpp(v, 0x128, 0xF, 0xF, false);   // row_ror:8 = xor 8 within 16
  if (s == 16) return __builtin_amdgcn_ds_swizzle(v, 0x401F);               // xor 16 within 32 lanes
  return __shfl_xor(v, 32, 64);
}

// Descending bitonic sort of 1024 32-bit keys, 4 per thread on threads
// t < kRsSortThreads (element 4t + r in a[r]): strides 1 and 2 in registers,
// 4 .. 128 across lanes of a wave, 256 and 512 through xch[1024] in LDS.  Every
// thread of the workgroup calls it (the barriers); the others only wait.
__device__ __forceinline__ void rs_sort1024(uint32_t (&a)[4], uint32_t* xch) {
  const int t = threadIdx.x;
  const bool on = t < kRsSortThreads;
#pragma unroll
  for (int size = 2; size <= 1024; size <<= 1) {
#pragma unroll
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      if (stride <= 2) {
        if (!on) continue;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          if (r & stride) continue;
          const int e = 4 * t + r;
          const bool desc = (e & size) == 0;
          const uint32_t x = a[r], y = a[r + stride];
          const uint32_t hi = max(x, y), lo = min(x, y);
          a[r] = desc ? hi : lo;
          a[r + stride] = desc ? lo : hi;
        }
      } else {
        uint32_t b[4];
        if (stride <= 128) {
          if (!on) continue;
#pragma unroll
          for (int r = 0; r < 4; ++r) b[r] = rs_xor_lane(a[r], stride >> 2);
        } else {
          if (on) {
#pragma unroll
            for (int r = 0; r < 4; ++r) xch[4 * t + r] = a[r];
          }
          __syncthreads();
          if (on) {
#pragma unroll
            for (int r = 0; r < 4; ++r) b[r] = xch[4 * (t ^ (stride >> 2)) + r];
          }
          __syncthreads();
          if (!on) continue;
        }
        const bool keep_max = ((4 * t & stride) == 0) == ((4 * t & size) == 0);
#pragma unroll
        for (int r = 0; r < 4; ++r) a[r] = keep_max ? max(a[r], b[r]) : min(a[r], b[r]);
      }
    }
  }
}

// Descending bitonic sort of a[0, n2) of 32-bit keys in LDS.
__device__ void tk_sort32(uint32_t* a, int n2) {
  for (int size = 2; size <= n2; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int t = threadIdx.x; t < n2 / 2; t += blockDim.x) {
        const int i = 2 * t - (t & (stride - 1));
        const int j = i + stride;
        const bool desc = (i & size) == 0;
        const uint32_t x = a[i], y = a[j];
        if ((x < y) == desc) { a[i] = y; a[j] = x; }
      }
      __syncthreads();
    }
  }
}

// k-th largest (k >= 1) of the keys held N per thread (0 = none; at least k
// nonzero keys), a radix select over per-wave histograms (no atomics across
// waves) whose bins are offsets from the smallest key: one 8-bit round when
// the keys span fewer than 256 values (logit maxima of one row usually do),
// else a round on the offset's high bits and one on its low sh bits.  Spread
// bins also keep the LDS atomics of a wave off one address.
template <int N>
__device__ uint32_t rs_kth(const uint32_t (&key)[N], int k, uint32_t* wh, TkHist& h, uint32_t* ext) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  uint32_t hi = 0, lo = 0xffffu;
#pragma unroll
  for (int j = 0; j < N; ++j)
    if (key[j]) {
      hi = max(hi, key[j]);
      lo = min(lo, key[j]);
    }
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    hi = max(hi, rs_xor_lane(hi, d));
    lo = min(lo, rs_xor_lane(lo, d));
  }
  if (lane == 0) {
    ext[wave] = hi;
    ext[kRsWaves + wave] = lo;
  }
  __syncthreads();
  hi = 0;
  lo = 0xffffu;
#pragma unroll
  for (int w = 0; w < kRsWaves; ++w) {
    hi = max(hi, ext[w]);
    lo = min(lo, ext[kRsWaves + w]);
  }
  int sh = 0;
  while (((hi - lo) >> sh) > 255u) ++sh;           // 0 .. 8
  uint32_t* mine = wh + wave * 256;
  uint32_t sel = 0;
  int kk = k;
  for (int round = 0; round < (sh ? 2 : 1); ++round) {
#pragma unroll
    for (int j = 0; j < 4; ++j) mine[lane * 4 + j] = 0;
    // (LDS operations of one wave complete in order: the zeros land before the adds)
#pragma unroll
    for (int j = 0; j < N; ++j) {
      const uint32_t off = key[j] - lo;
      const bool in = key[j] != 0 && (round == 0 || (off >> sh) == sel);
      if (in) atomicAdd(&mine[round == 0 ? off >> sh : off & ((1u << sh) - 1u)], 1u);
    }
    __syncthreads();
    if (threadIdx.x < 256) {
      const int b = threadIdx.x;
      uint32_t tot = 0;
#pragma unroll
      for (int w = 0; w < kRsWaves; ++w) tot += wh[w * 256 + b];
      h.hist[b] = tot;
    }
    __syncthreads();
    rs_walk(h, kk);
    const uint32_t bin = h.sel_bin;
    kk -= h.sel_above;
    __syncthreads();
    sel = round == 0 ? bin : (sel << sh) | bin;
  }
  return lo + sel;
}

// k-th largest (k >= 1) of the keys held N per thread (0 = none) in one
// histogram round over the kRsThreads key values at and below the largest key
// hi: thread b's bin counts the keys equal to hi - b, and one workgroup scan
// over the bins finds the key.  Returns 0 when fewer than k keys lie in that
// window (the caller then takes rs_kth); else the key, with *hi_out = hi and
// *above_out = the number of keys strictly above it.  hist (kRsThreads words)
// must be zero and visible on entry.  Logit maxima span far fewer than 1024
// bf16 key values above their C-th largest, so one round decides.  A caller
// that knows the largest key passes it as hi_known (0: computed here).
template <int N>
__device__ uint32_t rs_kth_window(const uint32_t (&key)[N], int k, uint32_t* hist, int* slots, uint32_t* ext,
                                  uint32_t* hi_out, int* above_out, uint32_t hi_known = 0) {
  uint32_t hi = hi_known;
  if (hi == 0) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
    for (int j = 0; j < N; ++j) hi = max(hi, key[j]);
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) hi = max(hi, rs_xor_lane(hi, d));
    if (lane == 0) ext[wave] = hi;
    __syncthreads();
    hi = 0;
#pragma unroll
    for (int w = 0; w < kRsWaves; ++w) hi = max(hi, ext[w]);
  }
#pragma unroll
  for (int j = 0; j < N; ++j) {
    const uint32_t off = hi - key[j];
    if (key[j] != 0 && off < (uint32_t)kRsThreads) atomicAdd(&hist[off], 1u);
  }
  __syncthreads();
  const int c = (int)hist[threadIdx.x];
  int tot;
  const int pre = rs_scan(c, slots, &tot);
  if (pre < k && pre + c >= k) {
    ext[2 * kRsWaves] = hi - threadIdx.x;
    ext[2 * kRsWaves + 1] = (uint32_t)pre;
  }
  __syncthreads();
  if (tot < k) return 0;                           // (the same in every thread)
  *hi_out = hi;
  *above_out = (int)ext[2 * kRsWaves + 1];
  return ext[2 * kRsWaves];
}

// The C largest of n_c (C <= n_c <= kRsThreads) bf16 candidates, for callers
// that need the set only: T, the C-th largest key16, by one window round (the
// candidates' keys lie within the window of the row's maxima, so it always
// decides), then every candidate above T and the first C - (count above T) at
// T in candidate (index) order, ranked by ballots and per-wave counts, and
// placed the same way, so the set comes out in increasing index order.
// hist must be zero and visible on entry.  Candidate t's key16 is ck[t] >> 16;
// row_hi is the row's largest key16, which the largest candidate holds.
__device__ void tk_select_set_window(const uint32_t* ck, const int* cidx, int n_c, int C, uint32_t* hist, int* slots,
                                     uint32_t* ext, int64_t* out, uint32_t row_hi) {
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const uint32_t key[1] = {t < n_c ? ck[t] >> 16 : 0u};
  uint32_t hi;
  int above;
  const uint32_t T = rs_kth_window<1>(key, C, hist, slots, ext, &hi, &above, row_hi);
  const bool up = key[0] > T, tie = key[0] != 0 && key[0] == T;
  const uint64_t below = (1ull << lane) - 1ull;
  const uint64_t bt = __ballot(tie);
  if (lane == 0) slots[wave] = __popcll(bt);
  __syncthreads();
  int before = 0;                                   // (all 16 counts read at once, masked)
#pragma unroll
  for (int w = 0; w < kRsWaves; ++w) before += w < wave ? slots[w] : 0;
  const bool in = up || (tie && before + (int)__popcll(bt & below) < C - above);
  const uint64_t bi = __ballot(in);
  if (lane == 0) ext[wave] = __popcll(bi);          // (the window round's reads of ext[0, kRsWaves) are done)
  __syncthreads();
  int pos = 0;
#pragma unroll
  for (int w = 0; w < kRsWaves; ++w) pos += w < wave ? (int)ext[w] : 0;
  if (in) out[pos + __popcll(bi & below)] = (int64_t)cidx[t];
}

// Descending ranks of n <= 256 distinct keys a[0, n) in LDS (32-bit bf16
// composites or 64-bit fp32 ones): thread (t, q)
// counts the keys above a[t] among a quarter (n2 = 256), an eighth (128) or a
// sixteenth (<= 64) of them; the partial counts meet in part[1024].  Returns
// the rank on threads t < n of the first part (threadIdx.x < n), else -1.
template <class K>
__device__ int rs_rank256(const K* a, int n, int* part) {
  int n2 = 64;
  while (n2 < n) n2 <<= 1;
  const int parts = kRsThreads / n2, span = n2 / parts;
  const int t = threadIdx.x % n2, q = threadIdx.x / n2;
  const K mine = t < n ? a[t] : ~K(0);
  int r = 0;
  const int j0 = q * span, j1 = min(j0 + span, n);
  int j = j0;
  for (; j + 4 <= j1; j += 4) {                     // four reads in flight per step
    const K a0 = a[j], a1 = a[j + 1], a2 = a[j + 2], a3 = a[j + 3];
    r += (a0 > mine ? 1 : 0) + (a1 > mine ? 1 : 0) + (a2 > mine ? 1 : 0) + (a3 > mine ? 1 : 0);
  }
  for (; j < j1; ++j) r += a[j] > mine ? 1 : 0;
  part[threadIdx.x] = r;
  __syncthreads();
  if ((int)threadIdx.x >= n) return -1;
  int rank = 0;
  for (int p = 0; p < parts; p += 4)                // parts is 4, 8 or 16
    rank += part[p * n2 + threadIdx.x] + part[(p + 1) * n2 + threadIdx.x] + part[(p + 2) * n2 + threadIdx.x] +
            part[(p + 3) * n2 + threadIdx.x];
  return rank;
}

// The C largest of n_c (C <= n_c <= kRsThreads) bf16 candidates, for callers
// that need the set only, in candidate (index) order: the C-th largest key16
// T by radix select (one key per thread), then every candidate above T and
// the first C - (count above T) at T, placed by two workgroup scans (the
// first packs the counts above T and at T into one word).  Candidate t's
// key16 is ck[t] >> 16; every thread of the workgroup calls it.
__device__ void tk_select_set(const uint32_t* ck, const int* cidx, int n_c, int C, uint32_t* wh, TkHist& h,
                              uint32_t* ext, int* slots, int64_t* out) {
  const int t = threadIdx.x;
  const uint32_t key[1] = {t < n_c ? ck[t] >> 16 : 0u};   // candidates' keys are >= T0 >= 1
  const uint32_t T = rs_kth<1>(key, C, wh, h, ext);
  const int above = key[0] > T ? 1 : 0, tie = key[0] != 0 && key[0] == T ? 1 : 0;
  int tot;
  const int pre = rs_scan(above | (tie << 16), slots, &tot);
  const bool in = above || (tie && (pre >> 16) < C - (tot & 0xffff));
  int n_in;
  const int pos = rs_scan(in ? 1 : 0, slots, &n_in);
  if (in) out[pos] = (int64_t)cidx[t];
}

// The C largest of n_c (kRsThreads < n_c <= 4 kRsThreads) bf16 candidates,
// for callers that need the set only (a top-1024 leaves more candidates than
// threads): thread t holds candidates 4t .. 4t + 3; T, the C-th largest key16,
// by the window round where the row's T0 round was windowed (the candidates'
// keys then lie within its window), else by rs_kth; then every candidate above
// T and the first C - (count above T) at T in candidate (index) order, placed
// by two workgroup scans, so the set comes out in increasing index order, as
// tk_select_set's.  hist must be zero and visible on entry; every thread of the
// workgroup calls it.
__device__ void tk_select_set4(const uint32_t* ck, const int* cidx, int n_c, int C, uint32_t* hist, uint32_t* wh,
                               TkHist& h, int* slots, uint32_t* ext, int64_t* out, bool windowed, uint32_t row_hi) {
  const int t = threadIdx.x;
  uint32_t key[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) key[j] = 4 * t + j < n_c ? ck[4 * t + j] >> 16 : 0u;   // keys >= T0 >= 1
  uint32_t T = 0;
  if (windowed) {
    uint32_t hi;
    int above;
    T = rs_kth_window<4>(key, C, hist, slots, ext, &hi, &above, row_hi);
  }
  if (T == 0) T = rs_kth<4>(key, C, wh, h, ext);
  int na = 0, nt = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    na += key[j] > T ? 1 : 0;
    nt += key[j] != 0 && key[j] == T ? 1 : 0;
  }
  int tot;
  const int pre = rs_scan(na | (nt << 16), slots, &tot);
  const int quota = C - (tot & 0xffff);              // ties at T that make the set
  int tb = pre >> 16, nin = 0;
  bool in[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const bool tie = key[j] != 0 && key[j] == T;
    in[j] = key[j] > T || (tie && tb < quota);
    tb += tie ? 1 : 0;
    nin += in[j] ? 1 : 0;
  }
  int n_in;
  int pos = rs_scan(nin, slots, &n_in);
#pragma unroll
  for (int j = 0; j < 4; ++j)
    if (in[j]) out[pos++] = (int64_t)cidx[4 * t + j];
}

// VPT: 8-slice vectors of the row's slice maxima per thread (1, 2 or 4, the
// fewest that cover the row), so short rows run fewer register slots.  E:
// the row's element type (Elem16 for bf16 logits, Elem32 for fp32).  The
// slice maxima and the threshold T0 are keys of the bf16-rounded elements
// for both; fp32 candidates are then ordered by their full 32-bit keys.
template <int VPT, class E>
__global__ __launch_bounds__(kRsThreads) void topk_rowsel_kernel(const typename E::T* logits, int64_t stride, int V,
                                                                 int C, const uint16_t* smax, int64_t sstride,
                                                                 int64_t* idx_out, int set_only) {
  constexpr bool F32 = E::BITS == 32;
  constexpr int EPI = E::PER16;         // elements per 16-byte item
  // (the 64 entries past kTkCap of cand, ck, cidx and slist take the writes
  // of lanes with nothing to write, so the compactions run without branches)
  __shared__ uint64_t cand[kTkCap + 64];  // exact and short-row paths; fp32 candidates: key << 32 | ~index
  __shared__ uint32_t ck[kTkCap + 64];    // bf16 candidate sort keys: key << 16 | (0xffff - position)
  __shared__ int cidx[kTkCap + 64];       // bf16 candidate element indices, increasing
  __shared__ int slist[kTkCap + 64];      // candidate slices, increasing
  __shared__ uint32_t wh[kRsWaves * 256];
  __shared__ uint32_t hist[kRsThreads];   // the window round's bins (zero before each use)
  __shared__ TkHist h;
  __shared__ int slots[kRsWaves];
  __shared__ uint32_t ext[2 * kRsWaves + 2];
  __shared__ int n_x;
  const int m = blockIdx.x;
  const typename E::T* row = logits + (int64_t)m * stride;
  int64_t* out = idx_out + (int64_t)m * C;
  if (V <= kTkCap) {
    for (int i = threadIdx.x; i < V; i += blockDim.x) cand[i] = tk_comp(E::key(row[i]), i);
    __syncthreads();
    tk_finish(cand, V, C, out);
    return;
  }
  const int S = tk_slice(V), ns = (V + S - 1) / S;
  int n_c = 0;
  bool exact = ns < C, windowed = false;
  uint32_t row_hi = 0;                              // the row's largest key16, from the window round
  if (!exact) {
    hist[threadIdx.x] = 0;                          // (visible after the first barrier of the T0 round)
    // thread t holds the 8-slice vectors [t * VPT, t * VPT + VPT) of the row's
    // slice maxima (the padding past ns is never written: masked)
    const int nv = (ns + 7) / 8;
    const uint4* src = reinterpret_cast<const uint4*>(smax + (int64_t)m * sstride);
    uint32_t sk[VPT * 8];
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
      const int vi = threadIdx.x * VPT + j;
      uint4 v = make_uint4(0, 0, 0, 0);
      if (vi < nv) v = src[vi];
      const uint32_t d[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const uint32_t kq = q & 1 ? d[q >> 1] >> 16 : d[q >> 1] & 0xffffu;
        sk[j * 8 + q] = vi * 8 + q < ns ? kq : 0u;
      }
    }
    // T0: the C-th largest maximum of 4-slice groups (a lower bound of the
    // C-th largest element: C groups each hold an element >= T0), in one
    // window round when the groups' top C lie within 1024 key values of the
    // largest (then every candidate's key does too), else by rs_kth
    uint32_t key[VPT * 2];
#pragma unroll
    for (int j = 0; j < VPT * 2; ++j)
      key[j] = max(max(sk[4 * j], sk[4 * j + 1]), max(sk[4 * j + 2], sk[4 * j + 3]));
    const int ng = (ns + 3) / 4;
    uint32_t T0 = 1u;
    if (ng >= C) {
      uint32_t hi;
      int above;
      T0 = rs_kth_window(key, C, hist, slots, ext, &hi, &above);
      windowed = T0 != 0;
      row_hi = hi;
      if (!windowed) T0 = rs_kth(key, C, wh, h, ext);
    }
    hist[threadIdx.x] = 0;                          // for the final round (the T0 round has read its bin)
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    {
      // candidate slices in increasing order: one scan.  Waves past the row's
      // vectors (short rows) hold no slices and skip the work.
      const bool live = wv * 64 * VPT < nv;
      int cc = 0;
      if (live) {
#pragma unroll
        for (int j = 0; j < VPT * 8; ++j) cc += sk[j] >= T0 ? 1 : 0;
      }
      int nsl;
      int pos = rs_scan(cc, slots, &nsl);
      nsl = __builtin_amdgcn_readfirstlane(nsl);
      if (live) {
        const int dummy = kTkCap + (threadIdx.x & 63);
#pragma unroll
        for (int j = 0; j < VPT * 8; ++j) {
          const bool in = sk[j] >= T0;
          slist[in && pos < kTkCap ? pos : dummy] = (threadIdx.x * VPT + (j >> 3)) * 8 + (j & 7);
          pos += in ? 1 : 0;
        }
      }
      __syncthreads();
      exact = nsl > kTkCap;
      if (!exact) {
        // their elements whose key16 >= T0, in increasing index order: thread t
        // takes contiguous 16-byte items (8 bf16 or 4 fp32 elements) of a round,
        // one scan per round; waves holding no item of the round skip to the
        // scan, and the second item slot is skipped when the round has at most
        // one item per thread
        const int per = S / EPI, tot = nsl * per;
        for (int r0 = 0; r0 < tot; r0 += kRsThreads * kRsIpt) {
          const int nr = min(tot - r0, kRsThreads * kRsIpt);
          const int ipt = (nr + kRsThreads - 1) / kRsThreads;
          const bool wlive = wv * 64 * ipt < nr;
          uint32_t k8[kRsIpt * EPI];        // key16 (0: no element)
          uint32_t raw[kRsIpt * EPI];       // the elements (fp32 rows: for the full key)
          int e[kRsIpt];
          int cnt = 0;
          if (wlive) {
            uint4 v[kRsIpt];
#pragma unroll
            for (int j = 0; j < kRsIpt; ++j) {
              // every slot loads (a dead one, or an item starting past V, reads
              // the row's first item), so no load waits at a branch's join; the
              // item holding element V - 1 is read whole (rows are readable to
              // the 16-byte boundary after V), its elements past V masked below
              const int it = r0 + threadIdx.x * ipt + j;
              const bool ok = j < ipt && it < r0 + nr;
              e[j] = ok ? slist[it / per] * S + (it % per) * EPI : -1;
              v[j] = *reinterpret_cast<const uint4*>(row + (ok && e[j] < V ? e[j] : 0));
            }
#pragma unroll
            for (int j = 0; j < kRsIpt; ++j) {
#pragma unroll
              for (int q = 0; q < EPI; ++q) {
                raw[j * EPI + q] = E::at(v[j], q);
                const uint32_t kq = E::key16((typename E::T)raw[j * EPI + q]);
                k8[j * EPI + q] = e[j] >= 0 && e[j] + q < V ? kq : 0u;
                cnt += k8[j * EPI + q] >= T0 ? 1 : 0;
              }
            }
          }
          int step;
          int p2 = n_c + rs_scan(cnt, slots, &step);
          if (wlive) {
            const int dummy = kTkCap + (threadIdx.x & 63);
#pragma unroll
            for (int j = 0; j < kRsIpt * EPI; ++j) {
              const bool in = k8[j] >= T0;
              const int at = in && p2 < kTkCap ? p2 : dummy;
              const int ei = e[j / EPI] + (j % EPI);
              if constexpr (F32) {
                cand[at] = tk_comp(E::key((typename E::T)raw[j]), (uint32_t)ei);
              } else {
                ck[at] = (k8[j] << 16) | (uint32_t)(0xffff - p2);
                cidx[at] = ei;
              }
              p2 += in ? 1 : 0;
            }
          }
          n_c += __builtin_amdgcn_readfirstlane(step);
        }
        __syncthreads();
        exact = n_c > kTkCap;
      }
    }
  }
  if (exact) {
    tk_exact<E>(row, V, C, cand, h, &n_x);
    tk_finish(cand, C, C, out);
    return;
  }
  if constexpr (F32) {
    // (full key, index) composites: up to 256 (the draft head's top-64) are
    // ranked directly, each counting the composites above it; more are sorted
    if (n_c <= 256) {
      const int r = rs_rank256(cand, n_c, reinterpret_cast<int*>(wh));
      if (r >= 0 && r < C) out[r] = (int64_t)(0xffffffffu - (uint32_t)(cand[threadIdx.x] & 0xffffffffu));
    } else {
      tk_finish(cand, n_c, C, out);
    }
    return;
  }
  if (set_only && n_c <= kRsThreads) {             // the set only: no sort
    if (windowed) tk_select_set_window(ck, cidx, n_c, C, hist, slots, ext, out, row_hi);
    else tk_select_set(ck, cidx, n_c, C, wh, h, ext, slots, out);
    return;
  }
  if (set_only) {                                  // n_c <= kTkCap = 4 kRsThreads here
    tk_select_set4(ck, cidx, n_c, C, hist, wh, h, slots, ext, out, windowed, row_hi);
    return;
  }
  // sort the candidates (positions follow the index order, so ties sort by index)
  if (n_c <= 256) {
    const int r = rs_rank256(ck, n_c, reinterpret_cast<int*>(wh));
    if (r >= 0 && r < C) out[r] = (int64_t)cidx[threadIdx.x];
  } else if (n_c <= 1024) {
    uint32_t a[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int e = 4 * (int)threadIdx.x + r;
      a[r] = threadIdx.x < kRsSortThreads && e < n_c ? ck[e] : 0u;
    }
    __syncthreads();
    rs_sort1024(a, ck);
    if (threadIdx.x < kRsSortThreads) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int e = 4 * threadIdx.x + r;
        if (e < C) out[e] = (int64_t)cidx[0xffff - (a[r] & 0xffffu)];
      }
    }
  } else {
    int n2 = 2048;
    while (n2 < n_c) n2 <<= 1;
    for (int i = n_c + threadIdx.x; i < n2; i += blockDim.x) ck[i] = 0;
    __syncthreads();
    tk_sort32(ck, n2);
    for (int i = threadIdx.x; i < C; i += blockDim.x) out[i] = (int64_t)cidx[0xffff - (ck[i] & 0xffffu)];
  }
}

static bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// ---- Draft logits: -inf rows with the rescored candidates scattered in ----
// (x/fp4patch.py:316-320: torch.full(-inf) + ids[cand] + (vals * inv_t).to(bf16)
// + scatter_, one launch).  Workgroup (b, m) owns columns [b * 2048, b * 2048 +
// 2048) of row m: it fills them with -inf, then, after the barrier, writes the
// candidates that land in them, so every element is written by one workgroup
// and the candidate store follows the fill in that workgroup's order.
// Candidates whose cand or ids entry is out of range are not written.
constexpr int kScatterCols = 2048;

__global__ __launch_bounds__(256) void scatter_draft_kernel(uint16_t* out, int64_t out_stride, const float* vals,
                                                            const int64_t* cand, const int64_t* ids, int64_t n_ids,
                                                            const float* inv_t, int C, int64_t vocab) {
  const int m = blockIdx.y;
  const int64_t c0 = (int64_t)blockIdx.x * kScatterCols;
  uint16_t* row = out + (int64_t)m * out_stride;
  // the first 256 candidates' columns and values load before the fill, so
  // their two dependent round trips overlap its stores
  auto fetch = [&](int c, int64_t& col, float& v) {
    col = -1;
    v = 0.0f;
    if (c >= C) return;
    const int64_t j = cand[(int64_t)m * C + c];
    if (j < 0 || j >= n_ids) return;
    col = ids[j];
    v = vals[(int64_t)m * C + c];
  };
  int64_t col;
  float v;
  fetch(threadIdx.x, col, v);
  const float t = inv_t ? *inv_t : 1.0f;
  const int64_t e = c0 + (int64_t)threadIdx.x * 8;
  if (e + 8 <= vocab && ((reinterpret_cast<uintptr_t>(row + e) & 15) == 0)) {
    const uint32_t w = 0xFF80FF80u;
    *reinterpret_cast<uint4*>(row + e) = make_uint4(w, w, w, w);
  } else {
    for (int i = 0; i < 8; ++i)
      if (e + i < vocab) row[e + i] = 0xFF80;
  }
  __syncthreads();
  for (int c = threadIdx.x;;) {
    if (col >= c0 && col < c0 + kScatterCols && col < vocab) row[col] = f32_to_bf16(inv_t ? v * t : v);
    c += blockDim.x;
    if (c >= C) break;
    fetch(c, col, v);
  }
}

// The draft head's rescore and scatter in one launch (refine_nv4 followed by
// scatter_draft, x/fp4x_kernels.py:391-416 and x/fp4patch.py:316-320), with
// two kinds of workgroups that write disjoint elements, so neither waits for
// the other:
//   * rescore workgroups (blockIdx.x < nr): refine_kernel's candidate slots,
//     loads, fma order and lane reduction; each writes its candidate's
//     bf16((sum * gs) * inv_t) (bf16(sum * gs) without inv_t) at column
//     ids[cand[m, c]], whose load goes out beside the weight loads;
//   * fill workgroups (b, m): -inf over columns [b * 2048, b * 2048 + 2048)
//     of row m except the candidates' columns (an LDS bitmap of them).
// Every element has one writer (a repeated candidate writes the same value
// twice), and the output equals refine_nv4 + scatter_draft bit for bit.  A
// candidate outside [0, n_ids), or whose column lies outside [0, vocab), is
// not written.
constexpr int kDraftMaxC = 2048;

__global__ __launch_bounds__(kThreads) void draft_nv4_kernel(RefineArgs p, uint16_t* out, const int64_t* ids,
                                                            const float* inv_t, int64_t vocab, int nr) {
  extern __shared__ __align__(16) uint16_t lds_x[];
  __shared__ uint32_t mark[kScatterCols / 32];    // the block's candidate columns
  const int m = blockIdx.y;
  uint16_t* row = out + (int64_t)m * p.out_stride;
  if ((int)blockIdx.x < nr) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int lpr = p.lpr, lrow = lane & (lpr - 1), slot = lane / lpr, spw = 64 / lpr;
    const int cand = blockIdx.x * (kWaves * spw) + wave * spw + slot;
    int64_t rows[1] = {-1};
    if (cand < p.C) {
      const int64_t r = p.idx[(int64_t)m * p.C + cand];
      rows[0] = (r >= 0 && r < p.V) ? r : -1;
    }
    const int64_t col = rows[0] >= 0 ? ids[rows[0]] : -1;
    float acc[1][1] = {{0.0f}};
    for (int jb = 0; jb < p.cpl; jb += kCplBatch) {
      ChunkBatch<FmtNV4, 1> cb;
      load_batch_inbounds<FmtNV4>(cb, p.pa, rows[0], p.K / FmtNV4::KPC, lrow, lpr, jb, p.cpl);
      if (jb == 0) {
        stage_x<1>(lds_x, p.x + (int64_t)m * p.K, p.K, 1, 0, p.K);
        __syncthreads();
      }
      compute_batch<FmtNV4, 1, 1, const uint16_t*, AccFma>(cb, (const uint16_t*)lds_x, p.K, 0, 1, 0,
                                                           p.K / FmtNV4::KPC, lrow, lpr, jb, p.cpl, acc);
    }
    const float v = group_allreduce(acc[0][0], lpr) * p.gs;
    if (lrow == 0 && col >= 0 && col < vocab) {
      const float t = inv_t ? *inv_t : 1.0f;
      row[col] = f32_to_bf16(inv_t ? v * t : v);
    }
    return;
  }
  const int64_t c0 = (int64_t)(blockIdx.x - nr) * kScatterCols;
  if (threadIdx.x < kScatterCols / 32) mark[threadIdx.x] = 0u;
  __syncthreads();
  for (int c = threadIdx.x; c < p.C; c += blockDim.x) {
    const int64_t j = p.idx[(int64_t)m * p.C + c];
    if (j < 0 || j >= p.V) continue;
    const int64_t col = ids[j];
    if (col >= c0 && col < c0 + kScatterCols && col < vocab) {
      const int o = (int)(col - c0);
      atomicOr(&mark[o >> 5], 1u << (o & 31));
    }
  }
  __syncthreads();
  const int o = (int)threadIdx.x * 8;
  const int64_t e = c0 + o;
  const uint32_t mk = (mark[o >> 5] >> (o & 31)) & 0xffu;
  if (mk == 0 && e + 8 <= vocab && ((reinterpret_cast<uintptr_t>(row + e) & 15) == 0)) {
    const uint32_t w = 0xFF80FF80u;
    *reinterpret_cast<uint4*>(row + e) = make_uint4(w, w, w, w);
  } else {
    for (int i = 0; i < 8; ++i)
      if (e + i < vocab && !((mk >> i) & 1u)) row[e + i] = 0xFF80;
  }
}

}  // namespace fp4x

using namespace fp4x;

extern "C" {

int64_t fp4x_topk_workspace_size(int M, int V) {
  if (M <= 0 || V <= 0) return 0;
  return (int64_t)M * tk_smax_stride(V) * 2;
}

}  // extern "C"

namespace fp4x {
int topk_slice_len(int V) { return tk_slice(V); }
int64_t topk_smax_stride(int V) { return tk_smax_stride(V); }

int topk_check(const void* logits, int dtype, int64_t stride, int M, int V, int C, void* workspace,
               int64_t ws_bytes) {
  if (dtype != FP4X_DT_BF16 && dtype != FP4X_DT_F32) { set_error("topk: logits must be bf16 or fp32"); return FP4X_ERR_ARG; }
  if (M < 0 || V < 1 || C < 1 || C > V || C > 2048) { set_error("topk: need 1 <= C <= min(V, 2048)"); return FP4X_ERR_ARG; }
  const int per16 = dtype == FP4X_DT_F32 ? 4 : 8;
  if (stride < V || stride % per16 || !al16(logits)) {
    set_error("topk: logits must be 16-byte aligned with 16-byte aligned rows (stride >= V)");
    return FP4X_ERR_ARG;
  }
  if (ws_bytes < fp4x_topk_workspace_size(M, V) || (M > 0 && !al16(workspace))) {
    set_error("topk: workspace smaller than fp4x_topk_workspace_size(M, V) or misaligned");
    return FP4X_ERR_ARG;
  }
  return FP4X_OK;
}

// B (and A unless the slice maxima are already in the workspace).
template <class E>
static int topk_launch_t(const typename E::T* lg, int64_t stride, int M, int V, int C, int64_t* idx_out,
                         uint16_t* smax, bool have_smax, bool set_only, hipStream_t st) {
  const int S = tk_slice(V), ns = (V + S - 1) / S;
  const int64_t ss = tk_smax_stride(V);
  if (V > kTkCap && ns >= C && !have_smax)
    hipLaunchKernelGGL(topk_slicemax_kernel<E>, dim3((ns + 255) / 256, M), dim3(256), 0, st, lg, stride, V, smax, ss);
  const int nv = (ns + 7) / 8;
  auto kern = nv <= kRsThreads ? topk_rowsel_kernel<1, E> : nv <= 2 * kRsThreads ? topk_rowsel_kernel<2, E>
                                                                               : topk_rowsel_kernel<kRsVptMax, E>;
  hipLaunchKernelGGL(kern, dim3(M), dim3(kRsThreads), 0, st, lg, stride, V, C, smax, ss, idx_out, set_only ? 1 : 0);
  return check_launch("topk");
}

int topk_launch(const void* lg, int dtype, int64_t stride, int M, int V, int C, int64_t* idx_out, uint16_t* smax,
                bool have_smax, bool set_only, hipStream_t st) {
  if (dtype == FP4X_DT_F32)
    return topk_launch_t<Elem32>(static_cast<const uint32_t*>(lg), stride, M, V, C, idx_out, smax, have_smax,
                                 set_only, st);
  return topk_launch_t<Elem16>(static_cast<const uint16_t*>(lg), stride, M, V, C, idx_out, smax, have_smax,
                               set_only, st);
}
}  // namespace fp4x

extern "C" {

int fp4x_topk_rows(const void* logits, int dtype, int64_t stride, int M, int V, int C, int64_t* idx_out,
                   void* workspace, int64_t ws_bytes, void* stream) {
  int rc = topk_check(logits, dtype, stride, M, V, C, workspace, ws_bytes);
  if (rc || M == 0) return rc;
  return topk_launch(logits, dtype, stride, M, V, C, idx_out, static_cast<uint16_t*>(workspace), false, false,
                     (hipStream_t)stream);
}

int fp4x_refine_mx8(void* out, int out_dtype, int64_t out_stride, const void* x, const int64_t* idx, int M, int C,
                    const void* w, const void* s, int K, int V, void* stream) {
  if (M < 0 || C < 0 || K <= 0 || K % 32 || V < 0 || out_stride < V || (V == 0 && M > 0 && C > 0)) {
    set_error("refine_mx8: bad shape (K % 32 == 0, out_stride >= V, V > 0)");
    return FP4X_ERR_ARG;
  }
  if (!al16(x) || !al16(w)) { set_error("refine_mx8: x and w must be 16-byte aligned"); return FP4X_ERR_ARG; }
  if (M == 0 || C == 0) return FP4X_OK;
  RefineArgs p{};
  p.out = out; p.out_dtype = out_dtype; p.out_stride = out_stride;
  p.x = static_cast<const uint16_t*>(x);
  p.idx = idx;
  p.pa.w0 = static_cast<const uint8_t*>(w);
  p.pa.s = static_cast<const uint8_t*>(s);
  p.pa.K = K;
  p.M = M; p.C = C; p.K = K; p.V = V;
  const int chunks = K / 16;
  p.lpr = layout_lpr(chunks);
  p.cpl = (chunks + p.lpr - 1) / p.lpr;
  const int per_wg = kWaves * (64 / p.lpr);
  dim3 grid((C + per_wg - 1) / per_wg, M);
  hipLaunchKernelGGL((refine_kernel<FmtMX8, false>), grid, dim3(kThreads), (size_t)K * 2, (hipStream_t)stream, p);
  return check_launch("refine_mx8");
}

int fp4x_scatter_draft(void* out, int64_t out_stride, const float* vals, const int64_t* cand, const int64_t* ids,
                       int64_t n_ids, const float* inv_t, int M, int C, int64_t vocab, void* stream) {
  if (M < 0 || C < 0 || vocab < 1 || n_ids < 0 || out_stride < vocab) {
    set_error("scatter_draft: bad shape (vocab >= 1, out_stride >= vocab)");
    return FP4X_ERR_ARG;
  }
  if (M == 0) return FP4X_OK;
  dim3 grid((unsigned)((vocab + kScatterCols - 1) / kScatterCols), M);
  hipLaunchKernelGGL(scatter_draft_kernel, grid, dim3(256), 0, (hipStream_t)stream, static_cast<uint16_t*>(out),
                     out_stride, vals, cand, ids, n_ids, inv_t, C, vocab);
  return check_launch("scatter_draft");
}

int fp4x_draft_nv4(void* out, int64_t out_stride, const void* x, const int64_t* cand, const int64_t* ids,
                   int64_t n_ids, const void* wp, const void* s, float gs, const float* inv_t, int M, int C, int K,
                   int64_t vocab, void* stream) {
  if (M < 0 || C < 0 || C > kDraftMaxC || K <= 0 || K % 32 || vocab < 1 || out_stride < vocab || n_ids < 0 ||
      n_ids > INT32_MAX || (n_ids == 0 && M > 0 && C > 0)) {
    set_error("draft_nv4: bad shape (C <= 2048, K % 32 == 0, vocab >= 1, out_stride >= vocab, n_ids > 0)");
    return FP4X_ERR_ARG;
  }
  if (!al16(x) || !al16(wp) || (reinterpret_cast<uintptr_t>(s) & 1)) {
    set_error("draft_nv4: x and wp must be 16-byte aligned, s 2-byte aligned");
    return FP4X_ERR_ARG;
  }
  if (M == 0) return FP4X_OK;
  RefineArgs p{};
  p.out = out; p.out_dtype = FP4X_DT_BF16; p.out_stride = out_stride;
  p.x = static_cast<const uint16_t*>(x);
  p.idx = cand;
  p.pa.w0 = static_cast<const uint8_t*>(wp);
  p.pa.s = static_cast<const uint8_t*>(s);
  p.pa.K = K;
  p.gs = gs;
  p.M = M; p.C = C; p.K = K; p.V = (int)n_ids;
  const int chunks = K / FmtNV4::KPC;
  p.lpr = layout_lpr(chunks);
  p.cpl = (chunks + p.lpr - 1) / p.lpr;
  const int nr = (C + kWaves * (64 / p.lpr) - 1) / (kWaves * (64 / p.lpr));   // rescore workgroups per row
  dim3 grid((unsigned)(nr + (vocab + kScatterCols - 1) / kScatterCols), M);
  hipLaunchKernelGGL(draft_nv4_kernel, grid, dim3(kThreads), (size_t)K * 2, (hipStream_t)stream, p,
                     static_cast<uint16_t*>(out), ids, inv_t, vocab, nr);
  return check_launch("draft_nv4");
}

int fp4x_refine_nv4(float* out, const void* x, const int64_t* idx, int M, int C, const void* wp, const void* s, float gs,
                    int K, int V, void* stream) {
  if (M < 0 || C < 0 || K <= 0 || K % 32 || V < 0 || (V == 0 && M > 0 && C > 0)) {
    set_error("refine_nv4: bad shape (K % 32 == 0, V > 0)");
    return FP4X_ERR_ARG;
  }
  if (!al16(x) || !al16(wp) || (reinterpret_cast<uintptr_t>(s) & 1)) {
    set_error("refine_nv4: x and wp must be 16-byte aligned, s 2-byte aligned");
    return FP4X_ERR_ARG;
  }
  if (M == 0 || C == 0) return FP4X_OK;
  RefineArgs p{};
  p.out = out; p.out_dtype = FP4X_DT_F32; p.out_stride = C;
  p.x = static_cast<const uint16_t*>(x);
  p.idx = idx;
  p.pa.w0 = static_cast<const uint8_t*>(wp);
  p.pa.s = static_cast<const uint8_t*>(s);
  p.pa.K = K;
  p.gs = gs;
  p.M = M; p.C = C; p.K = K; p.V = V;
  const int chunks = K / FmtNV4::KPC;
  p.lpr = layout_lpr(chunks);
  p.cpl = (chunks + p.lpr - 1) / p.lpr;
  const int per_wg = kWaves * (64 / p.lpr);
  dim3 grid((C + per_wg - 1) / per_wg, M);
  hipLaunchKernelGGL((refine_kernel<FmtNV4, true>), grid, dim3(kThreads), (size_t)K * 2, (hipStream_t)stream, p);
  return check_launch("refine_nv4");
}

}  // extern "C"
