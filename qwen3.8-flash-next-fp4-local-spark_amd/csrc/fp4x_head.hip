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
  PlaneArgs pa;                // MXFP8 rows [V, K]
  int M, C, K, V, lpr, cpl;
};

// The candidate rows go through the chunk layout and lane butterfly of
// mx8_linear, accumulated with IEEE fp32 fma (AccFma) so every rounding is
// specified; e4m3 * 2^(e-127) is exact in bf16 and in fp32, and its product
// with a bf16 activation is exact, as in the reference's fp32 dot.
__global__ __launch_bounds__(kThreads) void refine_mx8_kernel(RefineArgs p) {
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
    ChunkBatch<FmtMX8, 1> cb;
    load_batch<FmtMX8, 1>(cb, p.pa, rows, 0, p.K / 16, lrow, lpr, jb, p.cpl);
    if (jb == 0) {
      stage_x<1>(lds_x, p.x + (int64_t)m * p.K, p.K, 1, 0, p.K);
      __syncthreads();
    }
    compute_batch<FmtMX8, 1, 1, const uint16_t*, AccFma>(cb, (const uint16_t*)lds_x, p.K, 0, 1, 0, p.K / 16, lrow,
                                                         lpr, jb, p.cpl, acc);
  }
  const float v = group_allreduce(acc[0][0], lpr);
  if (lrow == 0 && rows[0] >= 0) store_out(p.out, (int64_t)m * p.out_stride + rows[0], p.out_dtype, v);
}

// ------------------------------------------------------------------ top-k
// Three launches per call, which exchange data only across launch
// boundaries (no grid-wide waits, no cross-workgroup fences):
//   A  slice maxima: the row is cut into <= 4096 slices of S elements (S a
//      multiple of 8); smax[m][i] = largest order key of slice i.  Also zeroes
//      the row's candidate counter.
//   B  every workgroup of a row derives T0 = the C-th largest slice maximum
//      (a lower bound of the C-th largest element: C slices each hold an
//      element >= T0), gathers its elements with key >= T0 in LDS and
//      appends them to the row's candidate list with one global atomic.
//   C  one workgroup per row sorts the candidates (at most 4096) by the
//      total order and writes the first C indices.  Rows with fewer than C
//      slices, or more than 4096 candidates (massive ties), take the exact
//      threshold path in C instead.  Rows of at most 4096 elements skip A and
//      B: C sorts the whole row.
constexpr int kTkThreads = 1024;
constexpr int kTkCap = 4096;     // candidates per row
constexpr int kTkSlices = 4096;  // slice maxima per row
constexpr int kTkB = 16;         // collecting workgroups per row (kTkThreads each)

// bf16 bits -> 16-bit key increasing with the value; -0 counts as +0 and
// every NaN as the largest value.
__device__ __forceinline__ uint32_t tk_key(uint32_t b) {
  b &= 0xffffu;
  if ((b & 0x7fffu) == 0) b = 0;
  else if ((b & 0x7f80u) == 0x7f80u && (b & 0x7fu)) b = 0x7fc0u;
  return (b & 0x8000u) ? (~b & 0xffffu) : (b | 0x8000u);
}
// Composite order key: larger = larger value, then smaller index.
__device__ __forceinline__ uint64_t tk_comp(uint32_t key, uint32_t i) {
  return ((uint64_t)key << 32) | (uint64_t)(0xffffffffu - i);
}

__host__ __device__ inline int tk_slice(int V) { return 8 * ((V + 8 * kTkSlices - 1) / (8 * kTkSlices)); }

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

// Exact k-th largest key among n keys get(i) (two 8-bit rounds); *n_above
// receives the number of keys strictly above it.
template <class Get>
__device__ uint32_t tk_kth(TkHist& h, Get get, int n, int k, int* n_above) {
  for (int i = threadIdx.x; i < 256; i += blockDim.x) h.hist[i] = 0;
  __syncthreads();
  for (int i0 = 0; i0 < n; i0 += blockDim.x) {
    const int i = i0 + threadIdx.x;
    tk_hist_add(h.hist, i < n ? get(i) >> 8 : 0u, i < n);
  }
  __syncthreads();
  tk_walk(h, k);
  const uint32_t b1 = h.sel_bin;
  const int above1 = h.sel_above;
  __syncthreads();
  for (int i = threadIdx.x; i < 256; i += blockDim.x) h.hist[i] = 0;
  __syncthreads();
  for (int i = threadIdx.x; i < n; i += blockDim.x) {
    // low bytes within one high-byte bin are spread out: plain atomics
    const uint32_t kk = get(i);
    if ((kk >> 8) == b1) atomicAdd(&h.hist[kk & 255u], 1u);
  }
  __syncthreads();
  tk_walk(h, k - above1);
  const uint32_t t = (b1 << 8) | (uint32_t)h.sel_bin;
  *n_above = above1 + h.sel_above;
  __syncthreads();
  return t;
}

// Wave-aggregated append of comp (when flag) to list[*count]; positions past
// cap are counted but not written.
__device__ __forceinline__ void tk_append(uint64_t* list, int* count, int cap, bool flag, uint64_t comp) {
  const uint64_t mask = __ballot(flag);
  if (!mask) return;
  const int lane = threadIdx.x & 63;
  const int leader = __ffsll((unsigned long long)mask) - 1;
  int base = 0;
  if (lane == leader) base = atomicAdd(count, __popcll(mask));
  base = __shfl(base, leader, 64);
  if (flag) {
    const int pos = base + __popcll(mask & ((1ull << lane) - 1ull));
    if (pos < cap) list[pos] = comp;
  }
}

struct TkWork {              // per row, in the caller's workspace
  uint64_t cand[kTkCap];
  uint16_t smax[kTkSlices];
  int count;                 // candidates appended (beyond kTkCap: exact path)
  int pad[3];
};

__global__ __launch_bounds__(256) void topk_slicemax_kernel(const uint16_t* logits, int64_t stride, int V,
                                                            TkWork* work) {
  const int m = blockIdx.y;
  const uint16_t* row = logits + (int64_t)m * stride;
  TkWork& w = work[m];
  const int S = tk_slice(V), ns = (V + S - 1) / S;
  if (blockIdx.x == 0 && threadIdx.x == 0) w.count = 0;
  const int sl = blockIdx.x * blockDim.x + threadIdx.x;
  if (sl >= ns) return;
  uint32_t mx = 0;
  const int e0 = sl * S;
  for (int e = e0; e < e0 + S; e += 8) {
    if (e + 8 <= V) {
      const uint4 v = *reinterpret_cast<const uint4*>(row + e);
      const uint32_t d[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int q = 0; q < 4; ++q) mx = max(mx, max(tk_key(d[q] & 0xffffu), tk_key(d[q] >> 16)));
    } else {
      for (int i = e; i < V; ++i) mx = max(mx, tk_key(row[i]));
    }
  }
  w.smax[sl] = (uint16_t)mx;
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
__device__ void tk_exact(const uint16_t* row, int V, int C, uint64_t* cand, TkHist& h, int* n_sh) {
  if (threadIdx.x == 0) *n_sh = 0;
  __syncthreads();
  int above;
  const uint32_t T = tk_kth(h, [&](int i) { return tk_key(row[i]); }, V, C, &above);
  for (int i0 = 0; i0 < V; i0 += blockDim.x) {
    const int i = i0 + threadIdx.x;
    const uint32_t key = i < V ? tk_key(row[i]) : 0u;
    tk_append(cand, n_sh, kTkCap, i < V && key > T, tk_comp(key, i));
  }
  __syncthreads();
  const int need = C - above;
  if (threadIdx.x < 64) {
    int taken = 0;
    for (int i0 = 0; i0 < V && taken < need; i0 += 64) {
      const int i = i0 + threadIdx.x;
      const bool eq = i < V && tk_key(row[i]) == T;
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

// Elements per collecting thread, held in registers while T0 is derived.
constexpr int kTkVecs = 2;   // 8-element vectors per thread per round

__global__ __launch_bounds__(kTkThreads) void topk_collect_kernel(const uint16_t* logits, int64_t stride, int V, int C,
                                                                  TkWork* work) {
  __shared__ uint64_t buf[kTkCap];     // this workgroup's candidates
  __shared__ uint16_t smax[kTkSlices];
  __shared__ TkHist h;
  __shared__ int n_loc, base_sh;
  const int m = blockIdx.y;
  const uint16_t* row = logits + (int64_t)m * stride;
  TkWork& w = work[m];
  const int S = tk_slice(V), ns = (V + S - 1) / S;
  // this workgroup's share of the row, in whole 8-element vectors
  const int nvec = (V + 7) / 8;
  const int per = (nvec + gridDim.x - 1) / gridDim.x;
  const int v0 = blockIdx.x * per, v1 = min(nvec, v0 + per);
  // first round of row vectors: loads issued before the slice maxima
  uint4 d[kTkVecs];
#pragma unroll
  for (int r = 0; r < kTkVecs; ++r) {
    const int vi = v0 + r * blockDim.x + threadIdx.x;
    d[r] = vi < v1 && vi * 8 + 8 <= V ? *reinterpret_cast<const uint4*>(row + (int64_t)vi * 8) : make_uint4(0, 0, 0, 0);
  }
  if (threadIdx.x == 0) n_loc = 0;
  for (int i = threadIdx.x; i < ns; i += blockDim.x) smax[i] = w.smax[i];
  __syncthreads();
  int above;
  const uint32_t T0 = tk_kth(h, [&](int i) { return (uint32_t)smax[i]; }, ns, C, &above);
  for (int base = v0; base < v1; base += kTkVecs * blockDim.x) {
    if (base != v0) {
#pragma unroll
      for (int r = 0; r < kTkVecs; ++r) {
        const int vi = base + r * blockDim.x + threadIdx.x;
        d[r] = vi < v1 && vi * 8 + 8 <= V ? *reinterpret_cast<const uint4*>(row + (int64_t)vi * 8)
                                          : make_uint4(0, 0, 0, 0);
      }
    }
#pragma unroll
    for (int r = 0; r < kTkVecs; ++r) {
      const int vi = base + r * blockDim.x + threadIdx.x;
      const bool full = vi < v1 && vi * 8 + 8 <= V;
      const uint32_t dd[4] = {d[r].x, d[r].y, d[r].z, d[r].w};
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const int i = vi * 8 + q;
        const bool ok = vi < v1 && i < V;
        uint32_t key = 0;
        if (ok) key = full ? tk_key(q & 1 ? dd[q >> 1] >> 16 : dd[q >> 1] & 0xffffu) : tk_key(row[i]);
        tk_append(buf, &n_loc, kTkCap, ok && key >= T0, tk_comp(key, i));
      }
    }
  }
  __syncthreads();
  const int nl = n_loc;
  if (threadIdx.x == 0) base_sh = nl ? atomicAdd(&w.count, nl) : 0;   // nl > kTkCap pushes count past it
  __syncthreads();
  for (int i = threadIdx.x; i < nl && i < kTkCap; i += blockDim.x)
    if (base_sh + i < kTkCap) w.cand[base_sh + i] = buf[i];
}

__global__ __launch_bounds__(kTkThreads) void topk_select_kernel(const uint16_t* logits, int64_t stride, int V, int C,
                                                                 const TkWork* work, int64_t* idx_out) {
  __shared__ uint64_t cand[kTkCap];
  __shared__ TkHist h;
  __shared__ int n_sh;
  const int m = blockIdx.x;
  const uint16_t* row = logits + (int64_t)m * stride;
  int64_t* out = idx_out + (int64_t)m * C;
  if (V <= kTkCap) {
    for (int i = threadIdx.x; i < V; i += blockDim.x) cand[i] = tk_comp(tk_key(row[i]), i);
    __syncthreads();
    tk_finish(cand, V, C, out);
    return;
  }
  const int S = tk_slice(V), ns = (V + S - 1) / S;
  const int n = ns >= C ? work[m].count : kTkCap + 1;
  if (n <= kTkCap) {
    for (int i = threadIdx.x; i < n; i += blockDim.x) cand[i] = work[m].cand[i];
    __syncthreads();
    tk_finish(cand, n, C, out);
  } else {
    tk_exact(row, V, C, cand, h, &n_sh);
    tk_finish(cand, C, C, out);
  }
}

static bool al16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace fp4x

using namespace fp4x;

extern "C" {

int64_t fp4x_topk_workspace_size(int M) { return (int64_t)(M < 0 ? 0 : M) * (int64_t)sizeof(TkWork); }

int fp4x_topk_rows(const void* logits, int64_t stride, int M, int V, int C, int64_t* idx_out, void* workspace,
                   int64_t ws_bytes, void* stream) {
  if (M < 0 || V < 1 || C < 1 || C > V || C > 2048) { set_error("topk_rows: need 1 <= C <= min(V, 2048)"); return FP4X_ERR_ARG; }
  if (stride < V || stride % 8 || !al16(logits)) {
    set_error("topk_rows: logits must be 16-byte aligned with a row stride that is a multiple of 8");
    return FP4X_ERR_ARG;
  }
  if (ws_bytes < fp4x_topk_workspace_size(M) || (M > 0 && !al16(workspace))) {
    set_error("topk_rows: workspace smaller than fp4x_topk_workspace_size(M) or misaligned");
    return FP4X_ERR_ARG;
  }
  if (M == 0) return FP4X_OK;
  hipStream_t st = (hipStream_t)stream;
  TkWork* w = static_cast<TkWork*>(workspace);
  const uint16_t* lg = static_cast<const uint16_t*>(logits);
  if (V > kTkCap) {
    const int S = tk_slice(V), ns = (V + S - 1) / S;
    hipLaunchKernelGGL(topk_slicemax_kernel, dim3((ns + 255) / 256, M), dim3(256), 0, st, lg, stride, V, w);
    if (ns >= C) hipLaunchKernelGGL(topk_collect_kernel, dim3(kTkB, M), dim3(kTkThreads), 0, st, lg, stride, V, C, w);
  }
  hipLaunchKernelGGL(topk_select_kernel, dim3(M), dim3(kTkThreads), 0, st, lg, stride, V, C, w, idx_out);
  return check_launch("topk_rows");
}

int fp4x_refine_mx8(void* out, int out_dtype, int64_t out_stride, const void* x, const int64_t* idx, int M, int C,
                    const void* w, const void* s, int K, int V, void* stream) {
  if (M < 0 || C < 0 || K <= 0 || K % 32 || V < 0 || out_stride < V) {
    set_error("refine_mx8: bad shape (K % 32 == 0, out_stride >= V)");
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
  hipLaunchKernelGGL(refine_mx8_kernel, grid, dim3(kThreads), (size_t)K * 2, (hipStream_t)stream, p);
  return check_launch("refine_mx8");
}

}  // extern "C"
