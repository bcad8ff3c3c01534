/* Order-exact replica of the rescore sums (oracle; test infrastructure only).
 *
 * The reference's refine kernels (x/fp4x_kernels.py:367-381, :391-409) sum
 * exact fp32 products of a bf16 activation and an exactly representable
 * weight (MXFP8 e4m3 * 2^k, NVFP4 e2m1 * e4m3) with fp32 accumulation whose
 * order Triton leaves open.  The HIP rescore kernels fix that order, and this
 * file restates the same sums in it, so the refined logits can be compared
 * bit for bit:
 *   - a candidate row is cut into chunks of `kpc` weights;
 *   - lane l of `lpr` lanes owns chunks l, l + lpr, l + 2 lpr, ... ;
 *   - each lane starts from 0 and folds its chunks in increasing k, one
 *     IEEE fp32 fma per element: acc = fma(w_k, x_k, acc);
 *   - the lpr partials meet in a butterfly: for s = 1, 2, 4, ...,
 *     v[l] = v[l] + v[l ^ s];
 *   - ksplit equal K slices (1 for the rescore) are scaled by gs and added in
 *     slice order.
 * The GEMV kernels accumulate on MFMA, whose internal rounding is not IEEE;
 * their sums are compared against float64 exact sums within an error bound
 * instead (oracle/ordered.py mfma_bound), not replayed here.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

static inline float bf16f(uint16_t b) {
  uint32_t u = (uint32_t)b << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* One row slice: x and w point at the slice start, `chunks` chunks of kpc. */
static float slice_sum(const uint16_t* x, const uint16_t* w, int chunks, int kpc, int lpr) {
  float v[64];
  const int cpl = (chunks + lpr - 1) / lpr;
  for (int l = 0; l < lpr; ++l) {
    float acc = 0.0f;
    for (int j = 0; j < cpl; ++j) {
      const int c = l + j * lpr;
      if (c >= chunks) continue;
      const uint16_t* xc = x + (int64_t)c * kpc;
      const uint16_t* wc = w + (int64_t)c * kpc;
      for (int k = 0; k < kpc; ++k) acc = fmaf(bf16f(wc[k]), bf16f(xc[k]), acc);
    }
    v[l] = acc;
  }
  for (int s = 1; s < lpr; s <<= 1) {
    float t[64];
    for (int l = 0; l < lpr; ++l) t[l] = v[l] + v[l ^ s];
    memcpy(v, t, sizeof(float) * lpr);
  }
  return v[0];
}

/* out[m * N + i] = ordered sum of x[m] . w[rows ? rows[m * N + i] : i]
 * (bf16 x [M, K], bf16 operand w [*, K]), slices multiplied by gs and summed
 * in slice order.  Rows < 0 give 0. */
void oracle_ordered_gemv(const uint16_t* x, const uint16_t* w, const int64_t* rows, int M, int N, int K, int kpc,
                         int ksplit, int lpr, float gs, float* out) {
  const int ks = K / ksplit, chunks = ks / kpc;
#pragma omp parallel for collapse(2) schedule(static)
  for (int m = 0; m < M; ++m) {
    for (int i = 0; i < N; ++i) {
      const int64_t r = rows ? rows[(int64_t)m * N + i] : i;
      if (r < 0) { out[(int64_t)m * N + i] = 0.0f; continue; }
      float tot = 0.0f;
      for (int s = 0; s < ksplit; ++s) {
        const float p = slice_sum(x + (int64_t)m * K + (int64_t)s * ks, w + r * (int64_t)K + (int64_t)s * ks,
                                  chunks, kpc, lpr) * gs;
        tot = s == 0 ? p : tot + p;
      }
      out[(int64_t)m * N + i] = tot;
    }
  }
}

/* INT2 bf16 operand bits: bf16((code - 1.5) * s), fp16 group scales (raw
 * bits) [N, K/G], codes with element j of a 4-group in bit pair (0,2,1,3)[j].
 * (x/fp4x_kernels.py:318-322, :353-357) */
static float f16_bits_to_f32(uint16_t h) {
  const uint32_t s = (uint32_t)(h >> 15) << 31, e = (h >> 10) & 31, m = h & 1023;
  uint32_t u;
  if (e == 0) {
    if (m == 0) u = s;
    else { float f = (float)m * 0x1p-24f; memcpy(&u, &f, 4); u |= s; }
  } else if (e == 31) u = s | 0x7f800000u | (m << 13);
  else u = s | ((e + 112) << 23) | (m << 13);
  float f;
  memcpy(&f, &u, 4);
  return f;
}

static uint16_t f32_to_bf16_bits(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);
  return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1)) >> 16);
}

void oracle_int2_operand(const uint8_t* P, const uint16_t* S, int64_t N, int K, int G, uint16_t* out) {
  static const int order[4] = {0, 2, 1, 3};
#pragma omp parallel for schedule(static)
  for (int64_t n = 0; n < N; ++n) {
    for (int k = 0; k < K; ++k) {
      const int code = (P[n * (K / 4) + k / 4] >> (2 * order[k & 3])) & 3;
      const float s = f16_bits_to_f32(S[n * (K / G) + k / G]);
      out[n * K + k] = f32_to_bf16_bits(((float)code - 1.5f) * s);
    }
  }
}
