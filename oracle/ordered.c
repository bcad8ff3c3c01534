/* Order-exact replica of the fp4x GEMV sums (oracle; test infrastructure only).
 *
 * The HIP kernels fix every fp32 rounding of a dot product: a row slice is cut
 * into chunks of `kpc` weights; lane l of `lpr` lanes owns chunks
 * l, l + lpr, ... of the slice; each lane runs a chain of v_dot2_f32_bf16
 * steps over its chunks in increasing k, starting from 0; the lpr partials
 * meet in a butterfly (step s = 1, 2, 4, ...: v[l] += v[l ^ s]); split-K
 * slices are summed in slice order.  The reference leaves this order open
 * (fp32 accumulation in tl.dot, x/fp4x_kernels.py:24, :322, :380), so this
 * file restates the reference sums in the order the kernels use; with the same
 * order the sums agree bit for bit, which is what makes the INT2 coarse
 * top-C set and the refined logits comparable exactly.
 *
 * dot2 models (pinned against the hardware by tests/test_gpu_dot2.py):
 *   0  RN(a0*b0 + a1*b1 + c)          single rounding of the exact sum
 *   1  RN(RN(a0*b0 + a1*b1) + c)
 *   2  RN(RN(c + a0*b0) + a1*b1)      two chained fma
 *   3  RN(RN(c + a1*b1) + a0*b0)
 * bf16 x bf16 products are exact in fp32 and in double.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

static inline float bf16f(uint32_t b) {
  uint32_t u = (b & 0xffffu) << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* RN to float of the exact value t + e, where t = RN_double(exact) and e is
 * the exact double error of that rounding (|e| <= ulp(t)/2). */
static float rn_f32_of(double t, double e) {
  float f = (float)t;
  if (e == 0.0) return f;
  double df = (double)f;
  if (df == t) return f;            /* t on the float grid; e far below half a float ulp */
  double d = t - df;                /* exact */
  float g = nextafterf(f, d > 0 ? INFINITY : -INFINITY);
  double half = fabs((double)g - df) * 0.5;
  if (fabs(d) != half) return f;    /* not a tie: RN(t) is RN(t + e) */
  /* tie at t: the exact value t + e lies on the side of e */
  if ((d > 0) == (e > 0)) return g;
  return f;
}

static inline void two_sum(double a, double b, double* s, double* e) {
  double ss = a + b;
  double bb = ss - a;
  *e = (a - (ss - bb)) + (b - bb);
  *s = ss;
}

static float rn3_exact(double p0, double p1, double c) {
  double s, e1, t, e2;
  two_sum(p0, p1, &s, &e1);
  if (e1 == 0.0) {
    two_sum(s, c, &t, &e2);
    return rn_f32_of(t, e2);
  }
  __float128 q = (__float128)p0 + (__float128)p1;
  q += (__float128)c;
  return (float)q;
}

static inline float dot2_model(uint32_t a, uint32_t b, float c, int mode) {
  const float a0 = bf16f(a), a1 = bf16f(a >> 16), b0 = bf16f(b), b1 = bf16f(b >> 16);
  switch (mode) {
    case 0: return rn3_exact((double)a0 * b0, (double)a1 * b1, (double)c);
    case 1: { float p1 = a1 * b1; float s = fmaf(a0, b0, p1); return s + c; }
    case 2: return fmaf(a1, b1, fmaf(a0, b0, c));
    default: return fmaf(a0, b0, fmaf(a1, b1, c));
  }
}

void oracle_dot2_batch(const uint32_t* a, const uint32_t* b, const float* c, float* out, int64_t n, int mode) {
  for (int64_t i = 0; i < n; ++i) out[i] = dot2_model(a[i], b[i], c[i], mode);
}

/* One row slice: x and w point at the slice start, `chunks` chunks of kpc. */
static float slice_sum(const uint16_t* x, const uint16_t* w, int chunks, int kpc, int lpr, int mode) {
  float v[64];
  const int cpl = (chunks + lpr - 1) / lpr;
  for (int l = 0; l < lpr; ++l) {
    float acc = 0.0f;
    for (int j = 0; j < cpl; ++j) {
      const int c = l + j * lpr;
      if (c >= chunks) continue;
      const uint16_t* xc = x + (int64_t)c * kpc;
      const uint16_t* wc = w + (int64_t)c * kpc;
      for (int k = 0; k < kpc; k += 2) {
        const uint32_t wp = (uint32_t)wc[k] | ((uint32_t)wc[k + 1] << 16);
        const uint32_t xp = (uint32_t)xc[k] | ((uint32_t)xc[k + 1] << 16);
        acc = dot2_model(wp, xp, acc, mode);
      }
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
                         int ksplit, int lpr, float gs, int mode, float* out) {
  const int ks = K / ksplit, chunks = ks / kpc;
#pragma omp parallel for collapse(2) schedule(static)
  for (int m = 0; m < M; ++m) {
    for (int i = 0; i < N; ++i) {
      const int64_t r = rows ? rows[(int64_t)m * N + i] : i;
      if (r < 0) { out[(int64_t)m * N + i] = 0.0f; continue; }
      float tot = 0.0f;
      for (int s = 0; s < ksplit; ++s) {
        const float p = slice_sum(x + (int64_t)m * K + (int64_t)s * ks, w + r * (int64_t)K + (int64_t)s * ks,
                                  chunks, kpc, lpr, mode) * gs;
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
