// Device helpers shared by every fp4x kernel (gfx950 / CDNA4, wave64).
//
// Number formats follow the packed layouts of the fp4patch plugin's kernels
// (x/fp4x_kernels.py): bf16 activations, fp8 e4m3fn + e8m0 (MXFP8 rows),
// int8 + fp32/fp16 group scales (W8 g64), 6-bit two-plane codes + fp16 scale
// (W6 g32), e2m1 + e4m3 block scale (NVFP4), 2-bit codes + fp16/e4m3 group
// scale (INT2 coarse head).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fp4x {

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

enum DType : int { DT_BF16 = 0, DT_F32 = 1, DT_F16 = 2 };

// ---------------------------------------------------------------- bf16 / f16
__device__ __forceinline__ float bf16_lo(uint32_t v) { return __uint_as_float(v << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t v) { return __uint_as_float(v & 0xffff0000u); }
__device__ __forceinline__ float bf16_to_f32(uint16_t b) { return __uint_as_float(uint32_t(b) << 16); }

// fp32 -> bf16, round to nearest even (v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  __bf16 h = (__bf16)f;
  return __builtin_bit_cast(uint16_t, h);
}
__device__ __forceinline__ float round_bf16(float f) { return bf16_to_f32(f32_to_bf16(f)); }

// Two fp32 -> packed bf16x2 {lo, hi}, round to nearest even.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  bf16x2_t v;
  v.x = (__bf16)lo;
  v.y = (__bf16)hi;
  return __builtin_bit_cast(uint32_t, v);
}

__device__ __forceinline__ float f16_to_f32(uint16_t h) {
  return (float)__builtin_bit_cast(_Float16, h);
}

// ---------------------------------------------------------------- order keys
// bf16 bits -> 16-bit key increasing with the value; -0 counts as +0 and
// every NaN as the largest value.  Key 0 lies below every value (the key of
// -inf is 0x7f), so it marks "no element".
__device__ __forceinline__ uint32_t tk_key(uint32_t b) {
  b &= 0xffffu;
  if ((b & 0x7fffu) == 0) b = 0;
  else if ((b & 0x7f80u) == 0x7f80u && (b & 0x7fu)) b = 0x7fc0u;
  return (b & 0x8000u) ? (~b & 0xffffu) : (b | 0x8000u);
}
// fp32 bits -> 32-bit key with the same order rules (-0 as +0, every NaN
// as the largest value).  No value maps to key 0 (-inf has 0x007fffff), so
// it marks "no element" here too.
__device__ __forceinline__ uint32_t tk_key32(uint32_t b) {
  if ((b & 0x7fffffffu) == 0) b = 0;
  else if ((b & 0x7fffffffu) > 0x7f800000u) b = 0x7fc00000u;
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

// ---------------------------------------------------------------- fp8 / fp4
// e8m0 shared exponent -> fp32 2^(e-127).  e = 0 gives the fp32 denormal
// 2^-127, e = 255 gives +inf (the value exp2(255 - 127) rounds to).
__device__ __forceinline__ float e8m0_to_f32(uint32_t e) {
  return __uint_as_float(e ? (e << 23) : 0x00400000u);
}

// Two OCP e4m3fn bytes (16-bit half `HI` of v) -> bf16x2, each multiplied by
// `scale` (v_cvt_scalef32_pk_bf16_fp8).
template <bool HI>
__device__ __forceinline__ uint32_t fp8x2_to_bf16x2(uint32_t v, float scale) {
  return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(v, scale, HI));
}
template <bool HI>
__device__ __forceinline__ f32x2_t fp8x2_to_f32x2(uint32_t v, float scale) {
  return __builtin_amdgcn_cvt_scalef32_pk_f32_fp8(v, scale, HI);
}
// Two OCP e2m1 nibbles (byte `B` of v; low nibble first) -> fp32 pair.  The
// scalef32 converts apply only the exponent of their scale operand (they are
// built for e8m0 scales), so a general scale is multiplied separately.
template <int B>
__device__ __forceinline__ f32x2_t fp4x2_to_f32x2(uint32_t v) {
  return __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(v, 1.0f, B);
}

// ---------------------------------------------------------------- byte ops
__device__ __forceinline__ uint32_t perm_b32(uint32_t hi, uint32_t lo, uint32_t sel) {
  return __builtin_amdgcn_perm(hi, lo, sel);
}
// Byte B of v as fp32 (selected as v_cvt_f32_ubyteB).
template <int B>
__device__ __forceinline__ float ubyte_to_f32(uint32_t v) {
  return (float)((v >> (8 * B)) & 0xffu);
}

// ---------------------------------------------------------------- lanes
// Butterfly all-reduce over groups of `n` consecutive lanes (n a power of
// two <= 64): step s = 1, 2, 4, ... adds the partner lane (lane ^ s).  Each
// lane pair forms the same sum (fp32 addition is commutative), so after the
// last step every lane of the group holds the identical total.
__device__ __forceinline__ float group_allreduce(float v, int n) {
  for (int s = 1; s < n; s <<= 1) v += __shfl_xor(v, s, 64);
  return v;
}

// Logistic sigmoid 1 / (1 + e^-x) rounded to fp32: evaluated in fp64 (the
// fp64 exp and an IEEE fp64 divide, within two fp64 ulps of the exact value)
// and rounded once to fp32, so the result is the correctly rounded fp32
// sigmoid unless the exact value lies within 2^-51 relative of an fp32
// rounding boundary.  One implementation serves the fused and unfused mixer
// epilogues; they evaluate a few hundred sigmoids per workgroup, where fp64
// costs nothing measurable.
__device__ __forceinline__ float sigmoid_f32(float x) {
  const double t = exp(-(double)x);
  return (float)(1.0 / (1.0 + t));
}

// ---------------------------------------------------------------- memory
__device__ __forceinline__ uint4 ld_u128(const void* p) { return *reinterpret_cast<const uint4*>(p); }
__device__ __forceinline__ uint2 ld_u64(const void* p) { return *reinterpret_cast<const uint2*>(p); }
__device__ __forceinline__ uint32_t ld_u32(const void* p) { return *reinterpret_cast<const uint32_t*>(p); }
__device__ __forceinline__ uint32_t ld_u16(const void* p) { return *reinterpret_cast<const uint16_t*>(p); }
__device__ __forceinline__ uint32_t ld_u8(const void* p) { return *reinterpret_cast<const uint8_t*>(p); }

// Store one output value in the requested dtype.
__device__ __forceinline__ void store_out(void* base, int64_t idx, int dt, float v) {
  if (dt == DT_F32) reinterpret_cast<float*>(base)[idx] = v;
  else if (dt == DT_BF16) reinterpret_cast<uint16_t*>(base)[idx] = f32_to_bf16(v);
  else reinterpret_cast<_Float16*>(base)[idx] = (_Float16)v;
}

// Agent-scope ticket for the last-arriving-workgroup split-K protocol.
__device__ __forceinline__ int ticket_acq_rel(int* p) {
  return __hip_atomic_fetch_add(p, 1, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void ticket_reset(int* p) {
  __hip_atomic_store(p, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_coherent(const float* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace fp4x
