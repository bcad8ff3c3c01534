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
// Three launches per call (no grid-wide waits):
//   A  slice maxima: the row is cut into <= 4096 slices of S elements (S a
//      multiple of 8); smax[m][i] = largest order key of slice i.  Also zeroes
//      the row's candidate counter.
//   B  every workgroup of a row derives T0 = the C-th largest slice maximum
//      (a lower bound of the C-th largest element: C slices each hold an
//      element >= T0) and appends its elements with key >= T0 to the row's
//      candidate list (composite keys, wave-aggregated atomics).
//   C  one workgroup per row sorts the candidates (at most 4096) by the
//      total order and writes the first C indices.  Rows with fewer than C
//      slices, or more than 4096 candidates (massive ties), take the exact
//      threshold path in C instead.
constexpr int kTkThreads = 1024;
constexpr int kTkCap = 4096;     // candidates per row
constexpr int kTkSlices = 4096;  // slice maxima per row
constexpr int kTkB = 32;         // collecting workgroups per row

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
// element (k >= 1) and the count of elements in higher bins.
__device__ void tk_walk(TkHist& h, int k) {
  if (threadIdx.x == 0) {
    int above = 0, b = 255;
    for (; b > 0; --b) {
      if (above + (int)h.hist[b] >= k) break;
      above += h.hist[b];
    }
    h.sel_bin = b;
    h.sel_above = above;
  }
  __syncthreads();
}

// Exact k-th largest key among n keys get(i) (two 8-bit rounds); *n_above
// receives the number of keys strictly above it.
template <class Get>
__device__ uint32_t tk_kth(TkHist& h, Get get, int n, int k, int* n_above) {
  for (int i = threadIdx.x; i < 256; i += blockDim.x) h.hist[i] = 0;
  __syncthreads();
  for (int i = threadIdx.x; i < n; i += blockDim.x) atomicAdd(&h.hist[get(i) >> 8], 1u);
  __syncthreads();
  tk_walk(h, k);
  const uint32_t b1 = h.sel_bin;
  const int above1 = h.sel_above;
  __syncthreads();
  for (int i = threadIdx.x; i < 256; i += blockDim.x) h.hist[i] = 0;
  __syncthreads();
  for (int i = threadIdx.x; i < n; i += blockDim.x) {
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
  int count;
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

__global__ __launch_bounds__(256) void topk_collect_kernel(const uint16_t* logits, int64_t stride, int V, int C,
                                                           TkWork* work) {
  __shared__ uint16_t smax[kTkSlices];
  __shared__ TkHist h;
  const int m = blockIdx.y;
  const uint16_t* row = logits + (int64_t)m * stride;
  TkWork& w = work[m];
  const int S = tk_slice(V), ns = (V + S - 1) / S;
  for (int i = threadIdx.x; i < ns; i += blockDim.x) smax[i] = w.smax[i];
  __syncthreads();
  int above;
  const uint32_t T0 = tk_kth(h, [&](int i) { return (uint32_t)smax[i]; }, ns, C, &above);
  // this workgroup's share of the row, in whole 8-element vectors
  const int nvec = (V + 7) / 8;
  const int per = (nvec + gridDim.x - 1) / gridDim.x;
  const int v0 = blockIdx.x * per, v1 = min(nvec, v0 + per);
  for (int base = v0; base < v1; base += blockDim.x) {
    const int vi = base + threadIdx.x;
    uint32_t d[4] = {0, 0, 0, 0};
    const bool full = vi < v1 && vi * 8 + 8 <= V;
    if (full) {
      const uint4 v = *reinterpret_cast<const uint4*>(row + (int64_t)vi * 8);
      d[0] = v.x; d[1] = v.y; d[2] = v.z; d[3] = v.w;
    }
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const int i = vi * 8 + q;
      bool ok = vi < v1 && i < V;
      uint32_t key = 0;
      if (ok) key = full ? tk_key(q & 1 ? d[q >> 1] >> 16 : d[q >> 1] & 0xffffu) : tk_key(row[i]);
      tk_append(w.cand, &w.count, kTkCap, ok && key >= T0, tk_comp(key, i));
    }
  }
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

__global__ __launch_bounds__(kTkThreads) void topk_select_kernel(const uint16_t* logits, int64_t stride, int V, int C,
                                                                 TkWork* work, int64_t* idx_out) {
  __shared__ uint64_t cand[kTkCap];
  __shared__ TkHist h;
  __shared__ int n_sh;
  const int m = blockIdx.x;
  const uint16_t* row = logits + (int64_t)m * stride;
  int64_t* out = idx_out + (int64_t)m * C;
  const int S = tk_slice(V), ns = (V + S - 1) / S;
  int n;
  if (V <= kTkCap) {
    for (int i = threadIdx.x; i < V; i += blockDim.x) cand[i] = tk_comp(tk_key(row[i]), i);
    n = V;
  } else if (ns >= C && work[m].count <= kTkCap) {
    n = work[m].count;
    for (int i = threadIdx.x; i < n; i += blockDim.x) cand[i] = work[m].cand[i];
  } else {
    // exact threshold T, the elements above it, and ties at T in index order
    if (threadIdx.x == 0) n_sh = 0;
    __syncthreads();
    int above;
    const uint32_t T = tk_kth(h, [&](int i) { return tk_key(row[i]); }, V, C, &above);
    for (int i0 = 0; i0 < V; i0 += blockDim.x) {
      const int i = i0 + threadIdx.x;
      const uint32_t key = i < V ? tk_key(row[i]) : 0u;
      tk_append(cand, &n_sh, kTkCap, i < V && key > T, tk_comp(key, i));
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
    n = C;
  }
  int n2 = 1;
  while (n2 < n) n2 <<= 1;
  __syncthreads();
  for (int i = n + threadIdx.x; i < n2; i += blockDim.x) cand[i] = 0;
  __syncthreads();
  tk_sort(cand, n2);
  for (int i = threadIdx.x; i < C; i += blockDim.x) out[i] = (int64_t)(0xffffffffu - (uint32_t)(cand[i] & 0xffffffffu));
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
    if (ns >= C) hipLaunchKernelGGL(topk_collect_kernel, dim3(kTkB, M), dim3(256), 0, st, lg, stride, V, C, w);
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
