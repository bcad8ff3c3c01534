// Weight preparation on the device: the reference's pure-torch quantizers
// (x/fp4x_kernels.py: quantize_w8 :138-144, quantize_w6 :179-202 with or
// without the clip search, quantize_nv4 :277-300, quantize_int2 :330-351 with fp16 scales,
// or e4m3 scales under an fp32 row scale) as one thread per quantization group.
//
// The source rows are fp32, bf16, or packed MXFP8 / NVFP4 rows decoded in
// registers with the exact dequant of mx8_dequant (:261-267) or dequant_nv4
// (:420-426), so a packed head is requantized without its fp32 copy.
//
// Arithmetic follows the reference's formulas with IEEE fp32 division, the
// semantics of its torch ops on CPU tensors (where its golden vectors were
// taken): torch's GPU division by a Python scalar multiplies by the
// reciprocal instead, which can move a result by one fp32 ulp.
#include <cmath>

#include "fp4x_kernels.h"
#include "../../include/fp4x.h"

namespace fp4x {

int device_cus();

// ------------------------------------------------------------------ sources
// load<G>(row, k0, f): the G fp32 weights [k0, k0 + G) of a row (k0 % 16 == 0).
struct SrcF32 {
  const float* w;
  int64_t ld;
  template <int G>
  __device__ void load(int64_t row, int k0, float (&f)[G]) const {
    const float4* p = reinterpret_cast<const float4*>(w + row * ld + k0);
#pragma unroll
    for (int i = 0; i < G / 4; ++i) {
      const float4 v = p[i];
      f[4 * i] = v.x; f[4 * i + 1] = v.y; f[4 * i + 2] = v.z; f[4 * i + 3] = v.w;
    }
  }
};

struct SrcBF16 {
  const uint16_t* w;
  int64_t ld;
  template <int G>
  __device__ void load(int64_t row, int k0, float (&f)[G]) const {
    const uint4* p = reinterpret_cast<const uint4*>(w + row * ld + k0);
#pragma unroll
    for (int i = 0; i < G / 8; ++i) {
      const uint4 v = p[i];
      const uint32_t d[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        f[8 * i + 2 * j] = bf16_lo(d[j]);
        f[8 * i + 2 * j + 1] = bf16_hi(d[j]);
      }
    }
  }
};

// MXFP8: e4m3fn [N, K] and e8m0 [N, K/32]; e4m3 * 2^(s - 127) is exact.
struct SrcMX8 {
  const uint8_t* w;
  const uint8_t* s;
  int K;
  template <int G>
  __device__ void load(int64_t row, int k0, float (&f)[G]) const {
#pragma unroll
    for (int c = 0; c < G / 16; ++c) {
      const int k = k0 + 16 * c;
      const uint4 q = *reinterpret_cast<const uint4*>(w + row * K + k);
      const uint32_t e = s[row * (K / 32) + k / 32];
      const float sc = e8m0_to_f32(e);
      const uint32_t d[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const f32x2_t a = fp8x2_to_f32x2<false>(d[i], sc), b = fp8x2_to_f32x2<true>(d[i], sc);
        f[16 * c + 4 * i] = a.x; f[16 * c + 4 * i + 1] = a.y;
        f[16 * c + 4 * i + 2] = b.x; f[16 * c + 4 * i + 3] = b.y;
      }
      if (e == 255u) {                                    // exp2(128) = +inf, as mx8_dequant (FmtMX8)
#pragma unroll
        for (int j = 0; j < 16; ++j)
          f[16 * c + j] = __uint_as_float(FmtMX8::inf_bf16((d[j / 4] >> (8 * (j % 4))) & 0xffu) << 16);
      }
    }
  }
};

// NVFP4: e2m1 pairs [N, K/2] (low nibble = even k), e4m3 [N, K/16], gs:
// (e2m1 * e4m3) * gs in fp32, the product exact and one rounding by gs.
struct SrcNV4 {
  const uint8_t* P;
  const uint8_t* S;
  float gs;
  int K;
  template <int G>
  __device__ void load(int64_t row, int k0, float (&f)[G]) const {
#pragma unroll
    for (int c = 0; c < G / 16; ++c) {
      const int k = k0 + 16 * c;
      const uint2 q = *reinterpret_cast<const uint2*>(P + row * (K / 2) + k / 2);
      const float sc = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8((uint32_t)S[row * (K / 16) + k / 16], 1.0f,
                                                                false)[0];
      const uint32_t d[2] = {q.x, q.y};
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const f32x2_t v0 = fp4x2_to_f32x2<0>(d[h]), v1 = fp4x2_to_f32x2<1>(d[h]);
        const f32x2_t v2 = fp4x2_to_f32x2<2>(d[h]), v3 = fp4x2_to_f32x2<3>(d[h]);
        const float v[8] = {v0.x, v0.y, v1.x, v1.y, v2.x, v2.y, v3.x, v3.y};
#pragma unroll
        for (int j = 0; j < 8; ++j) f[16 * c + 8 * h + j] = (v[j] * sc) * gs;
      }
    }
  }
};

__device__ __forceinline__ float f16_round(float v) { return (float)(_Float16)v; }

// Non-negative fp32 v < 464 -> e4m3fn code, round to nearest even (below
// 2^-6 the subnormal step 2^-9; below 2^-10, and at it, code 0).
__device__ __forceinline__ uint32_t e4m3_code(float v) {
  int e = (int)((__float_as_uint(v) >> 23) & 0xff) - 127;
  if (e < -6) e = -6;                                  // subnormal step 2^-9
  float q = rintf(v * __uint_as_float((uint32_t)(127 + 3 - e) << 23));   // v * 2^(3 - e)
  if (q >= 16.0f) { q = 8.0f; ++e; }
  const uint32_t m = (uint32_t)q;
  return m < 8 ? m : ((uint32_t)(e + 7) << 3) | (m - 8);
}
__device__ __forceinline__ float e4m3_value(uint32_t code) {
  const uint32_t e = code >> 3, m = code & 7;
  return e ? (float)(8 + m) * __uint_as_float((uint32_t)(127 + (int)e - 10) << 23) : (float)m * 0x1p-9f;
}

template <int G>
__device__ __forceinline__ float group_amax(const float (&f)[G]) {
  float a = 0.0f;
#pragma unroll
  for (int i = 0; i < G; ++i) a = fmaxf(a, fabsf(f[i]));
  return a;
}

// ------------------------------------------------------------------ targets
// W8 g64: s = max(amax, 1e-12) / 127, q = clamp(rint(w / s), -127, 127).
struct QW8 {
  static constexpr int G = 64;
  int8_t* q;
  float* s;
  __device__ void put(int64_t row, int gi, int K, const float (&f)[G]) const {
    const float sc = fmaxf(group_amax(f), 1e-12f) / 127.0f;
    uint32_t w[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      uint32_t b = 0;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float r = fminf(fmaxf(rintf(f[4 * i + j] / sc), -127.0f), 127.0f);
        b |= ((uint32_t)(int)r & 0xffu) << (8 * j);
      }
      w[i] = b;
    }
    uint4* o = reinterpret_cast<uint4*>(q + row * K + gi * G);
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = make_uint4(w[4 * i], w[4 * i + 1], w[4 * i + 2], w[4 * i + 3]);
    s[row * (K / G) + gi] = sc;
  }
};

// W6 g32: s = max(fp16(amax / qmax), 6.2e-5), c = clamp(rint(w / s), -qmax-1,
// qmax) + 32, split into the nibble plane L and the bit-pair plane H.
struct QW6 {
  static constexpr int G = 32;
  uint8_t* L;
  uint8_t* H;
  uint16_t* S;
  int qmax;
  __device__ static float base_scale(const float (&f)[G], int qmax) {
    return fmaxf(f16_round(group_amax(f) / (float)qmax), 6.2e-5f);
  }
  // codes clamp(rint(w / sc), -qmax - 1, qmax) + 32 into the two planes, fp16(sc) into S
  __device__ void put_scaled(int64_t row, int gi, int K, const float (&f)[G], float sc) const {
    uint32_t c[G];
#pragma unroll
    for (int i = 0; i < G; ++i)
      c[i] = (uint32_t)((int)fminf(fmaxf(rintf(f[i] / sc), (float)(-qmax - 1)), (float)qmax) + 32);
    uint32_t l[4] = {0, 0, 0, 0}, h[2] = {0, 0};
#pragma unroll
    for (int j = 0; j < 16; ++j) l[j >> 2] |= ((c[2 * j] & 15) | ((c[2 * j + 1] & 15) << 4)) << (8 * (j & 3));
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint32_t b = (c[4 * j] >> 4) | ((c[4 * j + 2] >> 4) << 2) | ((c[4 * j + 1] >> 4) << 4) |
                         ((c[4 * j + 3] >> 4) << 6);
      h[j >> 2] |= b << (8 * (j & 3));
    }
    *reinterpret_cast<uint4*>(L + row * (K / 2) + gi * 16) = make_uint4(l[0], l[1], l[2], l[3]);
    *reinterpret_cast<uint2*>(H + row * (K / 4) + gi * 8) = make_uint2(h[0], h[1]);
    S[row * (K / G) + gi] = __builtin_bit_cast(uint16_t, (_Float16)sc);
  }
  __device__ void put(int64_t row, int gi, int K, const float (&f)[G]) const {
    put_scaled(row, gi, K, f, base_scale(f, qmax));
  }
};

// W6 with the clip search: the group's scale is the first of s, sc_1 .. sc_n
// (sc_i = max(fp16(s * c_i), 6.2e-5), c_i the fp32 factors of the clip grid)
// whose squared error sum((clamp(rint(w / sc), -qmax - 1, qmax) * sc - w)^2)
// is strictly the smallest.  Every operation is rounded to fp32 on its own
// (no fused multiply-add); the 32 squares are summed as 8 lanes of 4
// (lane j: elements j, j + 8, j + 16, j + 24 in turn), then lanes 0..7 in
// turn: the order of torch's CPU sum over a 32-element row.
constexpr int kW6MaxClip = 64;
struct W6Clip {
  int n;
  float c[kW6MaxClip];
};
__device__ __forceinline__ float w6_sq_err(const float (&f)[32], float sc, int qmax) {
#pragma clang fp contract(off)
  float lane[8];
#pragma unroll
  for (int i = 0; i < 32; ++i) {
    const float d = fminf(fmaxf(rintf(f[i] / sc), (float)(-qmax - 1)), (float)qmax) * sc - f[i];
    const float d2 = d * d;
    if (i < 8) lane[i] = d2;
    else lane[i & 7] = lane[i & 7] + d2;
  }
  float e = lane[0];
#pragma unroll
  for (int j = 1; j < 8; ++j) e = e + lane[j];
  return e;
}
struct QW6Clip : QW6 {
  W6Clip clip;
  __device__ void put(int64_t row, int gi, int K, const float (&f)[G]) const {
#pragma clang fp contract(off)
    const float s = base_scale(f, qmax);
    float best = w6_sq_err(f, s, qmax), bs = s;
    for (int i = 0; i < clip.n; ++i) {
      // the fp32 product is rounded before its fp16 rounding: without the
      // register barrier the compiler fuses both into one v_fma_mixlo_f16,
      // a single rounding that differs at fp16 midpoints of the fp32 product
      float p = s * clip.c[i];
      asm volatile("" : "+v"(p));
      const float sc = fmaxf(f16_round(p), 6.2e-5f);
      const float e = w6_sq_err(f, sc, qmax);
      if (e < best) {
        best = e;
        bs = sc;
      }
    }
    put_scaled(row, gi, K, f, bs);
  }
};

// NVFP4 g16: sc = e4m3(clamp(amax / 6 / gs, 2^-9, 448)), v = clamp(w / (sc * gs),
// -6, 6), magnitude = the number of e2m1 midpoints below |v| (ties go down),
// sign bit 3 for v < 0.
struct QNV4 {
  static constexpr int G = 16;
  uint8_t* P;
  uint8_t* S;
  float gs;
  __device__ void put(int64_t row, int gi, int K, const float (&f)[G]) const {
    const float sc = fminf(fmaxf(group_amax(f) / 6.0f / gs, 0x1p-9f), 448.0f);
    const uint32_t code = e4m3_code(sc);
    const float sf = e4m3_value(code) * gs;
    uint32_t p[2] = {0, 0};
#pragma unroll
    for (int i = 0; i < G; ++i) {
      const float v = fminf(fmaxf(f[i] / sf, -6.0f), 6.0f), a = fabsf(v);
      const uint32_t mag = (a > 0.25f) + (a > 0.75f) + (a > 1.25f) + (a > 1.75f) + (a > 2.5f) + (a > 3.5f) +
                           (a > 5.0f);
      p[i >> 3] |= (mag | (v < 0.0f ? 8u : 0u)) << (4 * (i & 7));
    }
    *reinterpret_cast<uint2*>(P + row * (K / 2) + gi * 8) = make_uint2(p[0], p[1]);
    S[row * (K / G) + gi] = (uint8_t)code;
  }
};

// The G 2-bit codes clamp(floor(w / sf) + 2, 0, 3) of one INT2 group (0 where
// w / sf is NaN: a zero element of a group whose scale underflows), element j
// of a 4-group in bit pair (0, 2, 1, 3)[j], stored at o (G / 4 bytes).
template <int G>
__device__ __forceinline__ void put_int2_codes(const float (&f)[G], float sf, uint8_t* o) {
  uint32_t b[G / 16];
#pragma unroll
  for (int i = 0; i < G / 16; ++i) b[i] = 0;
#pragma unroll
  for (int i = 0; i < G; ++i) {
    const uint32_t c = (uint32_t)fminf(fmaxf(floorf(f[i] / sf) + 2.0f, 0.0f), 3.0f);
    const int pair = (i & 3) == 1 ? 2 : (i & 3) == 2 ? 1 : (i & 3);
    b[i >> 4] |= c << (2 * pair + 8 * ((i >> 2) & 3));
  }
  uint32_t* o32 = reinterpret_cast<uint32_t*>(o);
#pragma unroll
  for (int i = 0; i < G / 16; ++i) o32[i] = b[i];
}

// INT2 with fp16 group scales: s = fp16(max(amax, 1e-8) / 1.5) (a zero group's
// scale underflows fp16 to 0, and its codes are 0).
template <int GG>
struct QInt2 {
  static constexpr int G = GG;
  uint8_t* P;
  uint16_t* S;
  __device__ void put(int64_t row, int gi, int K, const float (&f)[G]) const {
    const _Float16 s16 = (_Float16)(fmaxf(group_amax(f), 1e-8f) / 1.5f);
    put_int2_codes(f, (float)s16, P + row * (K / 4) + gi * (G / 4));
    S[row * (K / G) + gi] = __builtin_bit_cast(uint16_t, s16);
  }
};

// INT2 with e4m3fn group scales under an fp32 row scale rs (R[row], written by
// int2e_kernel): S = e4m3(s / rs) for s = max(amax, 1e-8) / 1.5,
// codes against sf = float(S) * rs.  A group whose s / rs rounds to e4m3 0
// (amax below about 2^-10 / 448 of the row's largest) has sf = 0: its codes
// are 3, 0 and 0 for positive, negative and zero elements.
template <int GG>
struct QInt2E {
  static constexpr int G = GG;
  uint8_t* P;
  uint8_t* S;
  float* R;
  __device__ void put(int64_t row, int gi, int K, const float (&f)[G]) const { put_rs(row, gi, K, f, R[row]); }
  __device__ void put_rs(int64_t row, int gi, int K, const float (&f)[G], float rs) const {
    const uint32_t code = e4m3_code((fmaxf(group_amax(f), 1e-8f) / 1.5f) / rs);
    put_int2_codes(f, e4m3_value(code) * rs, P + row * (K / 4) + gi * (G / 4));
    S[row * (K / G) + gi] = (uint8_t)code;
  }
};

template <class Src, class Q>
__global__ __launch_bounds__(256) void quant_kernel(Src src, Q q, int64_t N, int K) {
  const int gpr = K / Q::G;
  const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= N * gpr) return;
  const int64_t row = t / gpr;
  const int gi = (int)(t - row * gpr);
  float f[Q::G];
  src.template load<Q::G>(row, gi * Q::G, f);
  q.put(row, gi, K, f);
}

// max |w| over the whole matrix into *out (zeroed by the caller): per-thread
// maxima over 16-groups, a wave maximum, one atomic max of the fp32 bits
// (ordered as unsigned for non-negative values) per wave.
template <class Src>
__global__ __launch_bounds__(256) void absmax_kernel(Src src, int64_t N, int K, uint32_t* out) {
  const int64_t groups = N * (K / 16);
  float m = 0.0f;
  for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < groups; t += (int64_t)gridDim.x * blockDim.x) {
    const int64_t row = t / (K / 16);
    float f[16];
    src.template load<16>(row, (int)(t - row * (K / 16)) * 16, f);
    m = fmaxf(m, group_amax(f));
  }
#pragma unroll
  for (int d = 32; d > 0; d >>= 1) m = fmaxf(m, __shfl_xor(m, d, 64));
  if ((threadIdx.x & 63) == 0) atomicMax(out, __float_as_uint(m));
}

// The e4m3 INT2 target, one wave per row: the row scale R[row] =
// (max(row amax, 1e-8) / 1.5) / 448, the largest group scale of the row over
// 448 (the rounded quotient max(a, 1e-8) / 1.5 is monotonic in a, so the row
// maximum of the group scales is the scale of the row's amax), then the
// row's groups against it.  The second read of the row comes from the caches
// the first one filled.
template <class Src, int G>
__global__ __launch_bounds__(256) void int2e_kernel(Src src, QInt2E<G> q, int64_t N, int K) {
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= N) return;                                  // uniform over the wave
  const int lane = threadIdx.x & 63;
  float m = 0.0f;
  for (int g = lane; g < K / 16; g += 64) {
    float f[16];
    src.template load<16>(row, g * 16, f);
    m = fmaxf(m, group_amax(f));
  }
#pragma unroll
  for (int d = 32; d > 0; d >>= 1) m = fmaxf(m, __shfl_xor(m, d, 64));
  const float rs = (fmaxf(m, 1e-8f) / 1.5f) / 448.0f;
  if (lane == 0) q.R[row] = rs;
  for (int gi = lane; gi < K / G; gi += 64) {
    float f[G];
    src.template load<G>(row, gi * G, f);
    q.put_rs(row, gi, K, f, rs);
  }
}

static bool al(const void* p, int a) { return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0; }

template <class Src, class Q>
static int launch_q(const Src& src, const Q& q, int64_t N, int K, hipStream_t st) {
  const int64_t groups = N * (K / Q::G);
  if (groups == 0) return FP4X_OK;
  hipLaunchKernelGGL((quant_kernel<Src, Q>), dim3((unsigned)((groups + 255) / 256)), dim3(256), 0, st, src, q, N, K);
  return check_launch("quantize");
}

template <class Src>
static int dispatch_q(const Src& src, int64_t N, int K, int dst, int G, int qmax, float gs, void* o0, void* o1,
                      void* o2, hipStream_t st) {
  switch (dst) {
    case FP4X_Q_W8:
      return launch_q(src, QW8{static_cast<int8_t*>(o0), static_cast<float*>(o1)}, N, K, st);
    case FP4X_Q_W6:
      return launch_q(src, QW6{static_cast<uint8_t*>(o0), static_cast<uint8_t*>(o1), static_cast<uint16_t*>(o2), qmax},
                      N, K, st);
    case FP4X_Q_NV4:
      return launch_q(src, QNV4{static_cast<uint8_t*>(o0), static_cast<uint8_t*>(o1), gs}, N, K, st);
    case FP4X_Q_INT2_E4M3: {
      uint8_t* P = static_cast<uint8_t*>(o0);
      uint8_t* S = static_cast<uint8_t*>(o1);
      float* R = static_cast<float*>(o2);
      if (N == 0) return FP4X_OK;
      const dim3 grid((unsigned)((N + 3) / 4));
      if (G == 16) hipLaunchKernelGGL((int2e_kernel<Src, 16>), grid, dim3(256), 0, st, src, QInt2E<16>{P, S, R}, N, K);
      else if (G == 32) hipLaunchKernelGGL((int2e_kernel<Src, 32>), grid, dim3(256), 0, st, src, QInt2E<32>{P, S, R}, N, K);
      else hipLaunchKernelGGL((int2e_kernel<Src, 64>), grid, dim3(256), 0, st, src, QInt2E<64>{P, S, R}, N, K);
      return check_launch("quantize (INT2 e4m3)");
    }
    default:
      if (G == 16) return launch_q(src, QInt2<16>{static_cast<uint8_t*>(o0), static_cast<uint16_t*>(o1)}, N, K, st);
      if (G == 32) return launch_q(src, QInt2<32>{static_cast<uint8_t*>(o0), static_cast<uint16_t*>(o1)}, N, K, st);
      return launch_q(src, QInt2<64>{static_cast<uint8_t*>(o0), static_cast<uint16_t*>(o1)}, N, K, st);
  }
}

static int src_check(int src, const void* a, const void* b, int64_t N, int K) {
  if (N < 0 || K <= 0 || K % 64) { set_error("quantize: need N >= 0 and K % 64 == 0"); return FP4X_ERR_ARG; }
  if (src < FP4X_SRC_F32 || src > FP4X_SRC_NV4) { set_error("quantize: unknown source kind"); return FP4X_ERR_ARG; }
  if (!al(a, 16) || ((src == FP4X_SRC_MX8 || src == FP4X_SRC_NV4) && !b)) {
    set_error("quantize: source rows must be 16-byte aligned (and packed sources need their scales)");
    return FP4X_ERR_ARG;
  }
  return FP4X_OK;
}

}  // namespace fp4x

using namespace fp4x;

extern "C" {

int fp4x_quantize(int src, const void* src_a, const void* src_b, float src_gs, int64_t N, int K, int dst, int G,
                  int qmax, float dst_gs, void* out0, void* out1, void* out2, void* stream) {
  int rc = src_check(src, src_a, src_b, N, K);
  if (rc) return rc;
  const bool int2 = dst == FP4X_Q_INT2 || dst == FP4X_Q_INT2_E4M3;
  if (dst < FP4X_Q_W8 || dst > FP4X_Q_INT2_E4M3 || (int2 && G != 16 && G != 32 && G != 64) ||
      (dst == FP4X_Q_W6 && (qmax < 1 || qmax > 31)) || (dst == FP4X_Q_NV4 && !(dst_gs > 0.0f))) {
    set_error("quantize: bad target (INT2 group 16, 32 or 64; W6 qmax 1..31; NVFP4 gs > 0)");
    return FP4X_ERR_ARG;
  }
  if (!al(out0, 16) || !out1 || ((dst == FP4X_Q_W6 || dst == FP4X_Q_INT2_E4M3) && !out2) ||
      (dst == FP4X_Q_INT2_E4M3 && !al(out2, 4))) {
    set_error("quantize: the packed output must be 16-byte aligned, and every output plane given");
    return FP4X_ERR_ARG;
  }
  hipStream_t st = (hipStream_t)stream;
  switch (src) {
    case FP4X_SRC_F32:
      return dispatch_q(SrcF32{static_cast<const float*>(src_a), K}, N, K, dst, G, qmax, dst_gs, out0, out1, out2, st);
    case FP4X_SRC_BF16:
      return dispatch_q(SrcBF16{static_cast<const uint16_t*>(src_a), K}, N, K, dst, G, qmax, dst_gs, out0, out1, out2,
                        st);
    case FP4X_SRC_MX8:
      return dispatch_q(SrcMX8{static_cast<const uint8_t*>(src_a), static_cast<const uint8_t*>(src_b), K}, N, K, dst,
                        G, qmax, dst_gs, out0, out1, out2, st);
    default:
      return dispatch_q(SrcNV4{static_cast<const uint8_t*>(src_a), static_cast<const uint8_t*>(src_b), src_gs, K}, N,
                        K, dst, G, qmax, dst_gs, out0, out1, out2, st);
  }
}

int fp4x_quantize_w6_clip(int src, const void* src_a, const void* src_b, float src_gs, int64_t N, int K, int qmax,
                          int clip_search, void* L, void* H, void* S, void* stream) {
  int rc = src_check(src, src_a, src_b, N, K);
  if (rc) return rc;
  if (qmax < 1 || qmax > 31 || clip_search < 0 || clip_search > kW6MaxClip) {
    set_error("quantize_w6_clip: need qmax 1..31 and clip_search 0..64");
    return FP4X_ERR_ARG;
  }
  if (!al(L, 16) || !al(H, 8) || !S) {
    set_error("quantize_w6_clip: L must be 16-byte and H 8-byte aligned, and S given");
    return FP4X_ERR_ARG;
  }
  // the clip grid as torch.linspace(0.70, 0.98, n) in fp32: step = (0.98f - 0.70f) / (n - 1),
  // c_i = fma(step, i, 0.70f) below n / 2, else fma(-step, n - 1 - i, 0.98f)
  QW6Clip q;
  q.L = static_cast<uint8_t*>(L);
  q.H = static_cast<uint8_t*>(H);
  q.S = static_cast<uint16_t*>(S);
  q.qmax = qmax;
  q.clip.n = clip_search;
  const float c0 = 0.70f, c1 = 0.98f;
  const float step = clip_search > 1 ? (c1 - c0) / (float)(clip_search - 1) : 0.0f;
  for (int i = 0; i < clip_search; ++i)
    q.clip.c[i] = i < clip_search / 2 || clip_search == 1 ? std::fma(step, (float)i, c0)
                                                          : std::fma(-step, (float)(clip_search - 1 - i), c1);
  for (int i = clip_search; i < kW6MaxClip; ++i) q.clip.c[i] = 0.0f;
  hipStream_t st = (hipStream_t)stream;
  switch (src) {
    case FP4X_SRC_F32:
      return launch_q(SrcF32{static_cast<const float*>(src_a), K}, q, N, K, st);
    case FP4X_SRC_BF16:
      return launch_q(SrcBF16{static_cast<const uint16_t*>(src_a), K}, q, N, K, st);
    case FP4X_SRC_MX8:
      return launch_q(SrcMX8{static_cast<const uint8_t*>(src_a), static_cast<const uint8_t*>(src_b), K}, q, N, K, st);
    default:
      return launch_q(SrcNV4{static_cast<const uint8_t*>(src_a), static_cast<const uint8_t*>(src_b), src_gs, K}, q, N,
                      K, st);
  }
}

int fp4x_absmax(int src, const void* src_a, const void* src_b, float src_gs, int64_t N, int K, float* out,
                void* stream) {
  int rc = src_check(src, src_a, src_b, N, K);
  if (rc) return rc;
  if (!out) { set_error("absmax: no output"); return FP4X_ERR_ARG; }
  if (N == 0) return FP4X_OK;
  hipStream_t st = (hipStream_t)stream;
  const int64_t groups = N * (K / 16);
  const unsigned grid = (unsigned)std::min<int64_t>((groups + 255) / 256, (int64_t)device_cus() * 8);
  uint32_t* o = reinterpret_cast<uint32_t*>(out);
  switch (src) {
    case FP4X_SRC_F32:
      hipLaunchKernelGGL(absmax_kernel<SrcF32>, dim3(grid), dim3(256), 0, st, SrcF32{static_cast<const float*>(src_a), K},
                         N, K, o);
      break;
    case FP4X_SRC_BF16:
      hipLaunchKernelGGL(absmax_kernel<SrcBF16>, dim3(grid), dim3(256), 0, st,
                         SrcBF16{static_cast<const uint16_t*>(src_a), K}, N, K, o);
      break;
    case FP4X_SRC_MX8:
      hipLaunchKernelGGL(absmax_kernel<SrcMX8>, dim3(grid), dim3(256), 0, st,
                         SrcMX8{static_cast<const uint8_t*>(src_a), static_cast<const uint8_t*>(src_b), K}, N, K, o);
      break;
    default:
      hipLaunchKernelGGL(absmax_kernel<SrcNV4>, dim3(grid), dim3(256), 0, st,
                         SrcNV4{static_cast<const uint8_t*>(src_a), static_cast<const uint8_t*>(src_b), src_gs, K}, N,
                         K, o);
  }
  return check_launch("absmax");
}

}  // extern "C"
