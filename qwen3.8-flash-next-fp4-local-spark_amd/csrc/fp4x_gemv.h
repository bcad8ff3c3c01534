// Format decoders and the chunk layout shared by the fp4x kernels (gfx950).
//
// y[m, n] = sum_k x[m, k] * w[n, k] with x bf16 and w dequantized to the
// bf16 operand the plugin's kernels feed to their dot (x/fp4x_kernels.py:23,
// :92, :129, :170, :322), fp32 accumulation.
//
// This header holds what the GEMV engines have in common:
//   * the per-format decoders Fmt* (one 16-byte "chunk" of the main packed
//     plane: 16 fp8/int8 weights, 32 W6/NVFP4 weights, 64 INT2 weights, and
//     its scales, decoded in registers to bf16 operand pairs);
//   * the chunk layout of the rescore kernels: `lpr` lanes (a power of two)
//     share one row, lane l owns chunks l, l + lpr, ... and folds them in
//     increasing k with IEEE fma (AccFma), the partials meeting in the
//     butterfly of group_allreduce;
//   * the split-K slot protocol (splitk_arrive): slice s of ksplit equal K
//     slices writes its fp32 partial to slot s; the last-arriving workgroup of
//     a row tile sums slots 0..ks-1 in order (((p0 + p1) + p2) + ...), runs the
//     epilogue and re-arms the tile's ticket.  No fp32 atomics: results are
//     deterministic.
// The GEMVs themselves accumulate on MFMA (fp4x_mfma.h, fp4x_stream.h).
#pragma once
#include "fp4x_device.h"

namespace fp4x {

constexpr int kWaves = 4;           // waves per workgroup
constexpr int kThreads = kWaves * 64;
constexpr int kCplBatch = 8;        // chunks per lane loaded in one batch
constexpr int kLdsXBytes = 64 * 1024;

// Lanes per row for a row (slice) of `chunks` 16-byte chunks: the smallest
// power of two giving at most 8 chunks per lane, capped at 64.
__host__ __device__ inline int layout_lpr(int chunks) {
  int want = (chunks + 7) / 8;
  int lpr = 1;
  while (lpr < want && lpr < 64) lpr <<= 1;
  return lpr;
}

// ------------------------------------------------------------------ formats
struct PlaneArgs {
  const uint8_t* w0;   // main packed plane
  const uint8_t* w1;   // auxiliary plane (W6 high bits)
  const uint8_t* s;    // scales
  int K;               // full row length in weights
  int G;               // INT2 group size
};

// MXFP8: fp8 e4m3fn [N, K] + e8m0 [N, K/32]  (x/fp4x_kernels.py:9-29)
struct FmtMX8 {
  static constexpr int KPC = 16, SUB = 1;
  struct Chunk { uint4 q; uint32_t e; };
  // Lane: pointers at chunk c of row r; at<DC>(L, j) reads chunk c + j*DC
  // (DC even) at constant offsets.
  struct Lane { const uint8_t* w; const uint8_t* s; };
  __device__ static Lane lane(const PlaneArgs& a, int64_t r, int c) {
    return {a.w0 + r * a.K + c * 16, a.s + r * (a.K / 32) + (c >> 1)};
  }
  __device__ static Lane step(const Lane& L, int dc) { return {L.w + dc * 16, L.s + (dc >> 1)}; }
  template <int DC>
  __device__ static Chunk at(const Lane& L, int j) {
    Chunk ch;
    ch.q = ld_u128(L.w + j * DC * 16);
    ch.e = ld_u8(L.s + j * (DC / 2));
    return ch;
  }
  // Chunks c, c + 1 (c = lane chunk + j*DC, even): 32 contiguous bytes and
  // their shared e8m0 scale.
  static constexpr int AUX_ALIGN = 1;
  template <int DC>
  __device__ static void pair(const Lane& L, int j, Chunk& a, Chunk& b) {
    a.q = ld_u128(L.w + j * DC * 16);
    b.q = ld_u128(L.w + j * DC * 16 + 16);
    a.e = b.e = ld_u8(L.s + j * (DC / 2));
  }
  __device__ static Chunk load(const PlaneArgs& a, int64_t row, int c) {
    Chunk ch;
    ch.q = ld_u128(a.w0 + row * a.K + c * 16);
    ch.e = ld_u8(a.s + row * (a.K / 32) + (c >> 1));
    return ch;
  }
  __device__ static Chunk zero() { Chunk ch; ch.q = make_uint4(0, 0, 0, 0); ch.e = 127; return ch; }
  __device__ static void deq16(const Chunk& ch, int, uint32_t (&w)[8]) {
    const float sc = e8m0_to_f32(ch.e);
    w[0] = fp8x2_to_bf16x2<false>(ch.q.x, sc); w[1] = fp8x2_to_bf16x2<true>(ch.q.x, sc);
    w[2] = fp8x2_to_bf16x2<false>(ch.q.y, sc); w[3] = fp8x2_to_bf16x2<true>(ch.q.y, sc);
    w[4] = fp8x2_to_bf16x2<false>(ch.q.z, sc); w[5] = fp8x2_to_bf16x2<true>(ch.q.z, sc);
    w[6] = fp8x2_to_bf16x2<false>(ch.q.w, sc); w[7] = fp8x2_to_bf16x2<true>(ch.q.w, sc);
    if (__builtin_expect(ch.e == 255u, 0)) inf_scale(ch.q, w);
  }
  // Exponent 255: the reference's scale exp2(255 - 127) is +inf in fp32, so
  // each weight is +-inf, or NaN for a zero or NaN code; the scaled convert
  // treats that exponent as a NaN scale instead (OCP MX's e8m0 NaN) and gives
  // NaN for every code.
  __device__ static uint32_t inf_bf16(uint32_t c) {
    const uint32_t mag = c & 0x7fu;
    return mag == 0u || mag == 0x7fu ? 0x7fc0u : 0x7f80u | ((c & 0x80u) << 8);
  }
  __device__ static void inf_scale(const uint4& q, uint32_t (&w)[8]) {
    const uint32_t d[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      w[2 * i] = inf_bf16(d[i] & 0xffu) | (inf_bf16((d[i] >> 8) & 0xffu) << 16);
      w[2 * i + 1] = inf_bf16((d[i] >> 16) & 0xffu) | (inf_bf16(d[i] >> 24) << 16);
    }
  }
};

// W8 g64: int8 [N, K] + fp32 (or fp16) [N, K/64]  (x/fp4x_kernels.py:116-135)
// bf16(q*s): fma(q + 128, s, -128*s) is the single rounding of the exact q*s,
// i.e. the fp32 product the reference forms, then rounded to bf16.
template <bool F16S>
struct FmtW8 {
  static constexpr int KPC = 16, SUB = 1;
  struct Chunk { uint4 q; uint32_t s; };
  static constexpr int SB = F16S ? 2 : 4;
  // Lane: pointers at chunk c of row r; at<DC>(L, j) reads chunk c + j*DC
  // (DC a multiple of 4, so the g64 scale index moves by DC/4).
  struct Lane { const uint8_t* w; const uint8_t* s; };
  __device__ static Lane lane(const PlaneArgs& a, int64_t r, int c) {
    return {a.w0 + r * a.K + c * 16, a.s + (r * (a.K / 64) + (c >> 2)) * SB};
  }
  __device__ static Lane step(const Lane& L, int dc) { return {L.w + dc * 16, L.s + (dc >> 2) * SB}; }
  template <int DC>
  __device__ static Chunk at(const Lane& L, int j) {
    Chunk ch;
    ch.q = ld_u128(L.w + j * DC * 16);
    if constexpr (F16S) ch.s = ld_u16(L.s + j * (DC / 4) * 2);
    else ch.s = ld_u32(L.s + j * (DC / 4) * 4);
    return ch;
  }
  // Chunks c, c + 1 (c even): one g64 group, one scale.
  static constexpr int AUX_ALIGN = SB;
  template <int DC>
  __device__ static void pair(const Lane& L, int j, Chunk& a, Chunk& b) {
    a.q = ld_u128(L.w + j * DC * 16);
    b.q = ld_u128(L.w + j * DC * 16 + 16);
    if constexpr (F16S) a.s = b.s = ld_u16(L.s + j * (DC / 4) * 2);
    else a.s = b.s = ld_u32(L.s + j * (DC / 4) * 4);
  }
  __device__ static Chunk load(const PlaneArgs& a, int64_t row, int c) {
    Chunk ch;
    ch.q = ld_u128(a.w0 + row * a.K + c * 16);
    if constexpr (F16S) ch.s = ld_u16(a.s + (row * (a.K / 64) + (c >> 2)) * 2);
    else ch.s = ld_u32(a.s + (row * (a.K / 64) + (c >> 2)) * 4);
    return ch;
  }
  __device__ static Chunk zero() { Chunk ch; ch.q = make_uint4(0, 0, 0, 0); ch.s = 0; return ch; }
  __device__ static float scale(uint32_t s) {
    if constexpr (F16S) return f16_to_f32((uint16_t)s);
    else return __uint_as_float(s);
  }
  __device__ static uint32_t pair4(uint32_t d, float s, float ms, uint32_t& hi) {
    const uint32_t u = d ^ 0x80808080u;   // q + 128 per byte
    float f0 = __builtin_fmaf(ubyte_to_f32<0>(u), s, ms);
    float f1 = __builtin_fmaf(ubyte_to_f32<1>(u), s, ms);
    float f2 = __builtin_fmaf(ubyte_to_f32<2>(u), s, ms);
    float f3 = __builtin_fmaf(ubyte_to_f32<3>(u), s, ms);
    hi = pack_bf16x2(f2, f3);
    return pack_bf16x2(f0, f1);
  }
  __device__ static void deq16(const Chunk& ch, int, uint32_t (&w)[8]) {
    const float s = scale(ch.s);
    const float ms = -128.0f * s;
    w[0] = pair4(ch.q.x, s, ms, w[1]);
    w[2] = pair4(ch.q.y, s, ms, w[3]);
    w[4] = pair4(ch.q.z, s, ms, w[5]);
    w[6] = pair4(ch.q.w, s, ms, w[7]);
  }
};

// W6 g32: lo-nibble plane L [N, K/2], hi-2-bit plane H [N, K/4], fp16 [N, K/32]
// (x/fp4x_kernels.py:151-176, packing :197-200).  Code c = lo | hi << 4 in
// [0, 63], q = c - 32; in an H byte the hi bits of k%4 = 0, 2, 1, 3 sit in
// bit pairs 0, 1, 2, 3.
struct FmtW6 {
  static constexpr int KPC = 32, SUB = 2;
  struct Chunk { uint4 lo; uint2 hi; uint32_t s; };
  struct Lane { const uint8_t* l; const uint8_t* h; const uint8_t* s; };
  __device__ static Lane lane(const PlaneArgs& a, int64_t r, int c) {
    return {a.w0 + r * (a.K / 2) + c * 16, a.w1 + r * (a.K / 4) + c * 8, a.s + (r * (a.K / 32) + c) * 2};
  }
  __device__ static Lane step(const Lane& L, int dc) { return {L.l + dc * 16, L.h + dc * 8, L.s + dc * 2}; }
  template <int DC>
  __device__ static Chunk at(const Lane& L, int j) {
    Chunk ch;
    ch.lo = ld_u128(L.l + j * DC * 16);
    ch.hi = ld_u64(L.h + j * DC * 8);
    ch.s = ld_u16(L.s + j * DC * 2);
    return ch;
  }
  // Chunks c, c + 1 (c even): 32 bytes of L, 16 of H, two scales in a dword.
  static constexpr int AUX_ALIGN = 4;
  template <int DC>
  __device__ static void pair(const Lane& L, int j, Chunk& a, Chunk& b) {
    a.lo = ld_u128(L.l + j * DC * 16);
    b.lo = ld_u128(L.l + j * DC * 16 + 16);
    const uint4 h = ld_u128(L.h + j * DC * 8);
    a.hi = make_uint2(h.x, h.y);
    b.hi = make_uint2(h.z, h.w);
    const uint32_t sc = ld_u32(L.s + j * DC * 2);
    a.s = sc & 0xffffu;
    b.s = sc >> 16;
  }
  __device__ static Chunk load(const PlaneArgs& a, int64_t row, int c) {
    Chunk ch;
    ch.lo = ld_u128(a.w0 + row * (a.K / 2) + c * 16);
    ch.hi = ld_u64(a.w1 + row * (a.K / 4) + c * 8);
    ch.s = ld_u16(a.s + (row * (a.K / 32) + c) * 2);
    return ch;
  }
  // Half h of chunk c (16 weights) in the sub-0 position of a chunk.
  __device__ static Chunk load_half(const PlaneArgs& a, int64_t row, int c, int h) {
    Chunk ch;
    const uint2 l = ld_u64(a.w0 + row * (a.K / 2) + c * 16 + h * 8);
    ch.lo = make_uint4(l.x, l.y, 0, 0);
    ch.hi = make_uint2(ld_u32(a.w1 + row * (a.K / 4) + c * 8 + h * 4), 0);
    ch.s = ld_u16(a.s + (row * (a.K / 32) + c) * 2);
    return ch;
  }
  __device__ static Chunk zero() {
    Chunk ch; ch.lo = make_uint4(0, 0, 0, 0); ch.hi = make_uint2(0, 0); ch.s = 0; return ch;
  }
  // The 6-bit codes of 8 weights k = 0..7: low nibbles from dword L (nibble
  // k = weight k), high bit pairs from H bytes 2 * half and 2 * half + 1 of hd
  // (weights 0-3 and 4-7; an H byte holds k%4 = 0, 2 in its low nibble, bits
  // 1:0 and 3:2, and k%4 = 1, 3 in its high nibble, bits 5:4 and 7:6).  Even k
  // go to ce (byte j: weight 2j), odd k to co (byte j: weight 2j + 1), so the
  // nibble split needs no byte shuffle: about 1.4 instructions per weight.
  __device__ static void codes8(uint32_t L, uint32_t hd, int half, uint32_t& ce, uint32_t& co) {
    const uint32_t ev = L & 0x0F0F0F0Fu;             // nibbles 0, 2, 4, 6
    const uint32_t od = (L >> 4) & 0x0F0F0F0Fu;      // nibbles 1, 3, 5, 7
    const uint32_t u = perm_b32(hd, hd, half ? 0x03030202u : 0x01010000u);   // [Hb, Hb, Hb+1, Hb+1]
    ce = ev | ((u << 4) & 0x00300030u) | ((u << 2) & 0x30003000u);
    co = od | (u & 0x00300030u) | ((u >> 2) & 0x30003000u);
  }
  // bf16 pairs (weights 2j, 2j + 1) of the codes in ce / co: (code - 32) * s
  // exactly in fp32, rounded to bf16.
  template <int J>
  __device__ static uint32_t deq2(uint32_t ce, uint32_t co, float s, float ms) {
    return pack_bf16x2(__builtin_fmaf(ubyte_to_f32<J>(ce), s, ms), __builtin_fmaf(ubyte_to_f32<J>(co), s, ms));
  }
  __device__ static void deq16(const Chunk& ch, int sub, uint32_t (&w)[8]) {
    const float s = f16_to_f32((uint16_t)ch.s);
    const float ms = -32.0f * s;
    const uint32_t L0 = sub ? ch.lo.z : ch.lo.x;
    const uint32_t L1 = sub ? ch.lo.w : ch.lo.y;
    const uint32_t hd = sub ? ch.hi.y : ch.hi.x;
    uint32_t e0, o0, e1, o1;
    codes8(L0, hd, 0, e0, o0);
    codes8(L1, hd, 1, e1, o1);
    w[0] = deq2<0>(e0, o0, s, ms); w[1] = deq2<1>(e0, o0, s, ms);
    w[2] = deq2<2>(e0, o0, s, ms); w[3] = deq2<3>(e0, o0, s, ms);
    w[4] = deq2<0>(e1, o1, s, ms); w[5] = deq2<1>(e1, o1, s, ms);
    w[6] = deq2<2>(e1, o1, s, ms); w[7] = deq2<3>(e1, o1, s, ms);
  }
};

// NVFP4: e2m1 pairs P [N, K/2] (low nibble = even k), e4m3 S [N, K/16]
// (x/fp4x_kernels.py:73-99).  Values e2m1 * e4m3 are exact in bf16.  The fp32
// global scale multiplies the accumulated sum (x/fp4x_kernels.py:94).
struct FmtNV4 {
  static constexpr int KPC = 32, SUB = 2;
  struct Chunk { uint4 q; uint32_t s; };
  struct Lane { const uint8_t* w; const uint8_t* s; };
  __device__ static Lane lane(const PlaneArgs& a, int64_t r, int c) {
    return {a.w0 + r * (a.K / 2) + c * 16, a.s + r * (a.K / 16) + c * 2};
  }
  __device__ static Lane step(const Lane& L, int dc) { return {L.w + dc * 16, L.s + dc * 2}; }
  template <int DC>
  __device__ static Chunk at(const Lane& L, int j) {
    Chunk ch;
    ch.q = ld_u128(L.w + j * DC * 16);
    ch.s = ld_u16(L.s + j * DC * 2);
    return ch;
  }
  // Chunks c, c + 1 (c even): 32 bytes of codes, four e4m3 scales in a dword.
  static constexpr int AUX_ALIGN = 4;
  template <int DC>
  __device__ static void pair(const Lane& L, int j, Chunk& a, Chunk& b) {
    a.q = ld_u128(L.w + j * DC * 16);
    b.q = ld_u128(L.w + j * DC * 16 + 16);
    const uint32_t sc = ld_u32(L.s + j * DC * 2);
    a.s = sc & 0xffffu;
    b.s = sc >> 16;
  }
  __device__ static Chunk load(const PlaneArgs& a, int64_t row, int c) {
    Chunk ch;
    ch.q = ld_u128(a.w0 + row * (a.K / 2) + c * 16);
    ch.s = ld_u16(a.s + row * (a.K / 16) + c * 2);
    return ch;
  }
  // Half h of chunk c (16 weights) in the sub-0 position of a chunk.
  __device__ static Chunk load_half(const PlaneArgs& a, int64_t row, int c, int h) {
    Chunk ch;
    const uint2 q = ld_u64(a.w0 + row * (a.K / 2) + c * 16 + h * 8);
    ch.q = make_uint4(q.x, q.y, 0, 0);
    ch.s = ld_u8(a.s + row * (a.K / 16) + c * 2 + h);
    return ch;
  }
  __device__ static Chunk zero() { Chunk ch; ch.q = make_uint4(0, 0, 0, 0); ch.s = 0; return ch; }
  __device__ static void deq16(const Chunk& ch, int sub, uint32_t (&w)[8]) {
    const f32x2_t sc2 = fp8x2_to_f32x2<false>(ch.s, 1.0f);
    const float sc = sub ? sc2.y : sc2.x;
    const uint32_t d0 = sub ? ch.q.z : ch.q.x;
    const uint32_t d1 = sub ? ch.q.w : ch.q.y;
    w[0] = pair(fp4x2_to_f32x2<0>(d0), sc); w[1] = pair(fp4x2_to_f32x2<1>(d0), sc);
    w[2] = pair(fp4x2_to_f32x2<2>(d0), sc); w[3] = pair(fp4x2_to_f32x2<3>(d0), sc);
    w[4] = pair(fp4x2_to_f32x2<0>(d1), sc); w[5] = pair(fp4x2_to_f32x2<1>(d1), sc);
    w[6] = pair(fp4x2_to_f32x2<2>(d1), sc); w[7] = pair(fp4x2_to_f32x2<3>(d1), sc);
  }
  // e2m1 * e4m3 has at most 6 significant bits: the fp32 product and its
  // bf16 rounding are exact.
  __device__ static uint32_t pair(f32x2_t v, float sc) { return pack_bf16x2(v.x * sc, v.y * sc); }
};

// INT2 coarse head: codes P [N, K/4] (element j of each 4-group in bit pair
// ORDER[j], ORDER = (0, 2, 1, 3)), group scales S [N, K/G] fp16 or e4m3
// (x/fp4x_kernels.py:304-357).  Weight = bf16((code - 1.5) * s).
// GC: 16 or 32 (group size known at compile time) or 0 (any G >= 64).
template <bool E4M3, int GC>
struct FmtInt2 {
  static constexpr int KPC = 64, SUB = 4;
  struct Chunk { uint4 q; uint2 s; };
  // Lane: pointers at chunk c of row r.  GC = 16 / 32: the chunk's group
  // scales sit at a fixed stride, read at constant offsets.  GC = 0 (G >= 64):
  // the lane keeps its row's scale base and first chunk, and at() computes
  // the group index (c * 64) / G.
  static constexpr int SB = E4M3 ? 1 : 2;
  struct Lane { const uint8_t* w; const uint8_t* s; int c, G; };
  __device__ static Lane lane(const PlaneArgs& a, int64_t r, int c) {
    const uint8_t* srow = a.s + r * (a.K / a.G) * SB;
    if constexpr (GC == 0) return {a.w0 + r * (a.K / 4) + c * 16, srow, c, a.G};
    else return {a.w0 + r * (a.K / 4) + c * 16, srow + c * (64 / GC) * SB, c, a.G};
  }
  __device__ static Lane step(const Lane& L, int dc) {
    if constexpr (GC == 0) return {L.w + dc * 16, L.s, L.c + dc, L.G};
    else return {L.w + dc * 16, L.s + dc * (64 / GC) * SB, L.c + dc, L.G};
  }
  template <int DC>
  __device__ static Chunk at(const Lane& L, int j) {
    Chunk ch;
    ch.q = ld_u128(L.w + j * DC * 16);
    if constexpr (GC == 16) {
      if constexpr (E4M3) { ch.s.x = ld_u32(L.s + j * DC * 4); ch.s.y = 0; }
      else ch.s = ld_u64(L.s + j * DC * 8);
    } else if constexpr (GC == 32) {
      if constexpr (E4M3) ch.s.x = ld_u16(L.s + j * DC * 2);
      else ch.s.x = ld_u32(L.s + j * DC * 4);
      ch.s.y = 0;
    } else {
      const int g = ((L.c + j * DC) * 64) / L.G;
      ch.s.x = E4M3 ? ld_u8(L.s + g) : ld_u16(L.s + g * 2);
      ch.s.y = 0;
    }
    return ch;
  }
  // Chunks c, c + 1 (c even): 32 bytes of codes; with G = 16 / 32 the group
  // scales of both chunks in one load.
  static constexpr int AUX_ALIGN = GC == 16 ? (E4M3 ? 8 : 16) : GC == 32 ? (E4M3 ? 4 : 8) : SB;
  template <int DC>
  __device__ static void pair(const Lane& L, int j, Chunk& a, Chunk& b) {
    a.q = ld_u128(L.w + j * DC * 16);
    b.q = ld_u128(L.w + j * DC * 16 + 16);
    if constexpr (GC == 16) {
      if constexpr (E4M3) {
        const uint2 v = ld_u64(L.s + j * DC * 4);
        a.s = make_uint2(v.x, 0);
        b.s = make_uint2(v.y, 0);
      } else {
        const uint4 v = ld_u128(L.s + j * DC * 8);
        a.s = make_uint2(v.x, v.y);
        b.s = make_uint2(v.z, v.w);
      }
    } else if constexpr (GC == 32) {
      if constexpr (E4M3) {
        const uint32_t v = ld_u32(L.s + j * DC * 2);
        a.s = make_uint2(v & 0xffffu, 0);
        b.s = make_uint2(v >> 16, 0);
      } else {
        const uint2 v = ld_u64(L.s + j * DC * 4);
        a.s = make_uint2(v.x, 0);
        b.s = make_uint2(v.y, 0);
      }
    } else {
      const int g0 = ((L.c + j * DC) * 64) / L.G, g1 = ((L.c + j * DC + 1) * 64) / L.G;
      a.s = make_uint2(E4M3 ? ld_u8(L.s + g0) : ld_u16(L.s + g0 * 2), 0);
      b.s = make_uint2(E4M3 ? ld_u8(L.s + g1) : ld_u16(L.s + g1 * 2), 0);
    }
  }
  __device__ static Chunk load(const PlaneArgs& a, int64_t row, int c) {
    Chunk ch;
    ch.q = ld_u128(a.w0 + row * (a.K / 4) + c * 16);
    const int ng = a.K / a.G;                     // groups per row
    constexpr int B = E4M3 ? 1 : 2;               // scale bytes
    const uint8_t* sp = a.s + (row * ng) * B;
    if constexpr (GC == 16) {
      if constexpr (E4M3) { ch.s.x = ld_u32(sp + c * 4); ch.s.y = 0; }
      else ch.s = ld_u64(sp + c * 8);
    } else if constexpr (GC == 32) {
      if constexpr (E4M3) ch.s.x = ld_u16(sp + c * 2);
      else ch.s.x = ld_u32(sp + c * 4);
      ch.s.y = 0;
    } else {
      const int g = (c * 64) / a.G;
      ch.s.x = E4M3 ? ld_u8(sp + g) : ld_u16(sp + g * 2);
      ch.s.y = 0;
    }
    return ch;
  }
  __device__ static Chunk zero() { Chunk ch; ch.q = make_uint4(0, 0, 0, 0); ch.s = make_uint2(0, 0); return ch; }
  __device__ static float group_scale(const Chunk& ch, int sub) {
    int idx;
    if constexpr (GC == 16) idx = sub;
    else if constexpr (GC == 32) idx = sub >> 1;
    else idx = 0;
    if constexpr (E4M3) {
      const uint32_t b = (idx < 4) ? (ch.s.x >> (8 * idx)) & 0xffu : 0u;
      return fp8x2_to_f32x2<false>(b, 1.0f).x;
    } else {
      const uint32_t h = (idx < 2) ? (ch.s.x >> (16 * idx)) : (ch.s.y >> (16 * (idx - 2)));
      return f16_to_f32((uint16_t)(h & 0xffffu));
    }
  }
  // Transposed dequant for the MFMA core: the 16 weights of sub-block `sub`
  // in k order [0,4,8,12, 1,5,9,13, 2,6,10,14, 3,7,11,15] (a 4x4 transpose
  // within the block), matching activations staged in the same order.  Each
  // code word W_t (element t of every 4-group) selects the low and the high
  // bytes of four values at once; two more byte permutes interleave them.
  static constexpr bool XPERM = true;
  __device__ static void deq16t(const Chunk& ch, int sub, uint32_t (&w)[8]) {
    const float s = group_scale(ch, sub);
    const float p = 0.5f * s, q = 1.5f * s;       // exact in fp32
    const uint32_t B = pack_bf16x2(p, q);         // [lo p, hi p, lo q, hi q]
    // value of code c: -q, -p, p, q; negation flips the sign bit of the high byte
    const uint32_t lut_lo = perm_b32(B, B, 0x02000002u);
    const uint32_t lut_hi = perm_b32(B, B, 0x03010103u) ^ 0x00008080u;
    const uint32_t cw = sub == 0 ? ch.q.x : sub == 1 ? ch.q.y : sub == 2 ? ch.q.z : ch.q.w;
    const uint32_t W[4] = {cw & 0x03030303u, (cw >> 4) & 0x03030303u, (cw >> 2) & 0x03030303u,
                           (cw >> 6) & 0x03030303u};
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const uint32_t lo = perm_b32(lut_lo, lut_lo, W[t]);
      const uint32_t hi = perm_b32(lut_hi, lut_hi, W[t]);
      w[2 * t] = perm_b32(hi, lo, 0x05010400u);       // k = t, 4 + t
      w[2 * t + 1] = perm_b32(hi, lo, 0x07030602u);   // k = 8 + t, 12 + t
    }
  }
  __device__ static void deq16(const Chunk& ch, int sub, uint32_t (&w)[8]) {
    const float s = group_scale(ch, sub);
    const float p = 0.5f * s, q = 1.5f * s;       // exact in fp32
    const uint32_t d0 = pack_bf16x2(-q, -p);      // codes 0, 1
    const uint32_t d1 = pack_bf16x2(p, q);        // codes 2, 3
    const uint32_t lut_lo = perm_b32(d1, d0, 0x06040200u);  // low bytes of v0..v3
    const uint32_t lut_hi = perm_b32(d1, d0, 0x07050301u);  // high bytes of v0..v3
    const uint32_t cw = sub == 0 ? ch.q.x : sub == 1 ? ch.q.y : sub == 2 ? ch.q.z : ch.q.w;
    const uint32_t e0 = cw & 0x03030303u;          // element 0 of each 4-group
    const uint32_t e1 = (cw >> 4) & 0x03030303u;   // element 1 (bit pair 2)
    const uint32_t e2 = (cw >> 2) & 0x03030303u;   // element 2 (bit pair 1)
    const uint32_t e3 = (cw >> 6) & 0x03030303u;   // element 3 (bit pair 3)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      // selector [c, c+4, c', c'+4] picks (lo, hi) bytes of v_c and v_c'
      const uint32_t sp = 0x04040000u | (uint32_t(j) * 0x0101u) | (uint32_t(j) * 0x01010000u);
      const uint32_t s01 = perm_b32(e1, e0, sp) | 0x04000400u;
      const uint32_t s23 = perm_b32(e3, e2, sp) | 0x04000400u;
      w[2 * j] = perm_b32(lut_hi, lut_lo, s01);
      w[2 * j + 1] = perm_b32(lut_hi, lut_lo, s23);
    }
  }
};

// BF16 weights [N, K] (x/fp4x_kernels.py:32-47): a chunk is 32 bytes (16
// weights) already in the dot operand format.
struct FmtBF16 {
  static constexpr int KPC = 16, SUB = 1;
  struct Chunk { uint4 a, b; };
  struct Lane { const uint8_t* w; };
  __device__ static Lane lane(const PlaneArgs& p, int64_t r, int c) { return {p.w0 + r * p.K * 2 + c * 32}; }
  __device__ static Lane step(const Lane& L, int dc) { return {L.w + dc * 32}; }
  template <int DC>
  __device__ static Chunk at(const Lane& L, int j) {
    Chunk ch;
    ch.a = ld_u128(L.w + j * DC * 32);
    ch.b = ld_u128(L.w + j * DC * 32 + 16);
    return ch;
  }
  static constexpr int AUX_ALIGN = 1;
  template <int DC>
  __device__ static void pair(const Lane& L, int j, Chunk& a, Chunk& b) {
    a = at<DC>(L, j);
    b.a = ld_u128(L.w + j * DC * 32 + 32);
    b.b = ld_u128(L.w + j * DC * 32 + 48);
  }
  __device__ static Chunk load(const PlaneArgs& p, int64_t row, int c) {
    Chunk ch;
    const uint8_t* base = p.w0 + row * p.K * 2 + c * 32;
    ch.a = ld_u128(base);
    ch.b = ld_u128(base + 16);
    return ch;
  }
  __device__ static Chunk zero() { Chunk ch; ch.a = make_uint4(0, 0, 0, 0); ch.b = ch.a; return ch; }
  __device__ static void deq16(const Chunk& ch, int, uint32_t (&w)[8]) {
    w[0] = ch.a.x; w[1] = ch.a.y; w[2] = ch.a.z; w[3] = ch.a.w;
    w[4] = ch.b.x; w[5] = ch.b.y; w[6] = ch.b.z; w[7] = ch.b.w;
  }
};

// ------------------------------------------------------------------ core
// Accumulation step of one (weight pair, activation pair) in the rescore
// kernels: two IEEE fp32 fma, low element first.  Every rounding is
// specified, so the sum can be replayed bit for bit on a CPU.
struct AccFma {
  __device__ static float step(uint32_t w, uint32_t x, float acc) {
    acc = __builtin_fmaf(bf16_lo(w), bf16_lo(x), acc);
    return __builtin_fmaf(bf16_hi(w), bf16_hi(x), acc);
  }
};

// Load one batch of chunks for RPL rows.  Row r of this lane is rows[r]
// (negative = no row); chunk j is c0 + lrow + (jb + j) * lpr, and chunks at
// or past cend (the end of the K slice) are neither loaded nor used.
template <class F, int RPL>
struct ChunkBatch {
  typename F::Chunk ch[RPL][kCplBatch];
};

template <class F, int RPL>
__device__ __forceinline__ void load_batch(ChunkBatch<F, RPL>& b, const PlaneArgs& a, const int64_t (&rows)[RPL],
                                           int c0, int cend, int lrow, int lpr, int jb, int cpl) {
#pragma unroll
  for (int j = 0; j < kCplBatch; ++j) {
    const int jj = jb + j;
    const int c = c0 + lrow + jj * lpr;
#pragma unroll
    for (int r = 0; r < RPL; ++r) {
      if (jj < cpl && rows[r] >= 0 && c < cend) b.ch[r][j] = F::load(a, rows[r], c);
      else b.ch[r][j] = F::zero();
    }
  }
}

// x[m][k] lives at xs[m * xstride + k - kx0] (LDS or global, bf16).
// Rows m >= M of x are not read (their accumulators stay 0).
template <class F, int MT, int RPL, class XPtr, class Acc = AccFma>
__device__ __forceinline__ void compute_batch(const ChunkBatch<F, RPL>& b, XPtr xs, int xstride, int kx0, int M,
                                              int c0, int cend, int lrow, int lpr, int jb, int cpl,
                                              float (&acc)[RPL][MT]) {
#pragma unroll
  for (int j = 0; j < kCplBatch; ++j) {
    const int jj = jb + j;
    if (jj >= cpl) break;
    const int c = c0 + lrow + jj * lpr;
    if (c >= cend) continue;
#pragma unroll
    for (int sub = 0; sub < F::SUB; ++sub) {
      const int k = c * F::KPC + sub * 16;
      uint32_t w[RPL][8];
#pragma unroll
      for (int r = 0; r < RPL; ++r) F::deq16(b.ch[r][j], sub, w[r]);
#pragma unroll
      for (int m = 0; m < MT; ++m) {
        if (m >= M) break;
        const uint4* xp = reinterpret_cast<const uint4*>(xs + (int64_t)m * xstride + (k - kx0));
        const uint4 xa = xp[0], xb = xp[1];
        const uint32_t xv[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
#pragma unroll
        for (int r = 0; r < RPL; ++r) {
          float t = acc[r][m];
#pragma unroll
          for (int i = 0; i < 8; ++i) t = Acc::step(w[r][i], xv[i], t);
          acc[r][m] = t;
        }
      }
    }
  }
}

// Stage x[0:M, k0:k0+ks] (bf16, row stride xstride elements) into LDS as
// [MT][ks], zero rows m >= M.  ks is a multiple of 16.
template <int MT>
__device__ __forceinline__ void stage_x(uint16_t* lds, const uint16_t* x, int64_t xstride, int M, int k0, int ks) {
  const int per_row = ks / 8;  // uint4 per row
  const int total = MT * per_row;
  for (int i = threadIdx.x; i < total; i += blockDim.x) {
    const int m = i / per_row, q = i - m * per_row;
    uint4 v = make_uint4(0, 0, 0, 0);
    if (m < M) v = *reinterpret_cast<const uint4*>(x + m * xstride + k0 + q * 8);
    reinterpret_cast<uint4*>(lds + m * ks)[q] = v;
  }
}

// Split-K slot protocol.  Partial sums travel through LDS to wave 0, which
// stores the tile's slot with device-coherent (agent-scope atomic) stores,
// waits for them to complete and takes the tile ticket.  splitk_arrive
// returns true in the (single) last-arriving workgroup of the tile, whose
// threads then read the slots with device-coherent loads (ld_coherent): the
// loads follow the ticket's return through the barrier, and no cache-wide
// write-back or invalidate (an agent-scope fence on a multi-XCD GPU) is needed.
__device__ __forceinline__ bool splitk_arrive(int* ticket, int ksplit) {
  __shared__ int last;
  if (threadIdx.x < 64) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // wave 0's slot stores have completed
    if (threadIdx.x == 0) last = (__hip_atomic_fetch_add(ticket, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                                  ksplit - 1);
  }
  __syncthreads();
  return last != 0;
}

}  // namespace fp4x
