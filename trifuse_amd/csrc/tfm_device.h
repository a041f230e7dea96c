// Device-side helpers shared by the MoE kernels (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tfm {

constexpr int kWave = 64;

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float bf2f(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }

// Round to nearest even, NaN kept quiet with its sign. Integer arithmetic, so
// the result does not depend on the hardware denormal mode.
__device__ __forceinline__ uint16_t f2bf(float f) {
  const uint32_t u = __float_as_uint(f);
  const uint32_t rounded = (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
  const uint32_t quiet = (u >> 16) | 0x0040u;  // NaN: keep sign and payload, set the quiet bit
  return (uint16_t)((u & 0x7fffffffu) > 0x7f800000u ? quiet : rounded);
}

// Two floats to packed bf16 (low = a), hardware round-to-nearest-even.
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  bf16x2_t v;
  v[0] = (__bf16)a;
  v[1] = (__bf16)b;
  return __builtin_bit_cast(uint32_t, v);
}

// IEEE half bits to float (exact).
__device__ __forceinline__ float h2f(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }

// Float to IEEE half bits, round to nearest even (subnormal results included,
// overflow to infinity, NaN kept quiet with its sign): one v_cvt_f16_f32.
// Every kernel of the library runs with round-to-nearest-even and f32 and
// f16 denormals preserved (the code object's default float mode), so the
// conversion is the IEEE one. It has no branches: a branchy integer version
// in the GEMV epilogues kept the compiler from moving loads and dot products
// across it.
__device__ __forceinline__ uint16_t f2h(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }

// Activation storage of the block: bf16 (F16 = false) or IEEE half, as bits.
template <bool F16>
__device__ __forceinline__ float st2f(uint16_t h) { return F16 ? h2f(h) : bf2f(h); }
template <bool F16>
__device__ __forceinline__ uint16_t f2st(float f) { return F16 ? f2h(f) : f2bf(f); }

// Two floats to packed half (low = a), hardware round-to-nearest-even.
__device__ __forceinline__ uint32_t pack_f16x2(float a, float b) {
  typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
  f16x2_t v;
  v[0] = (_Float16)a;
  v[1] = (_Float16)b;
  return __builtin_bit_cast(uint32_t, v);
}

// Low/high 16-bit half of a word in the storage dtype, to float.
template <bool F16>
__device__ __forceinline__ float lo_st(uint32_t w) { return F16 ? h2f((uint16_t)(w & 0xffffu)) : __uint_as_float(w << 16); }
template <bool F16>
__device__ __forceinline__ float hi_st(uint32_t w) { return F16 ? h2f((uint16_t)(w >> 16)) : __uint_as_float(w & 0xffff0000u); }

template <bool F16>
__device__ __forceinline__ uint32_t pack_st2(float a, float b) {
  return F16 ? pack_f16x2(a, b) : pack_bf16x2(a, b);
}

// Word k (0..3) of a 16-byte vector.
__device__ __forceinline__ uint32_t word_of(const uint4& v, int k) {
  return k == 0 ? v.x : k == 1 ? v.y : k == 2 ? v.z : v.w;
}

// Unpack the low/high bf16 of a 32-bit word to float.
__device__ __forceinline__ float lo_bf(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float hi_bf(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// exp for the routing softmax. Cody-Waite reduction x = n*ln2 + r with
// ln2 = 0x1.62e4p-1 + 0x1.7f7d1cp-20, then the degree-7 Taylor polynomial of
// e^r (coefficients fl(1/k!)) by Horner with fused multiply-adds, scaled by
// 2^n. x < -80 gives 0 so that softmax terms never become subnormal.
__device__ __forceinline__ float route_expf(float x) {
  if (x != x) return x;
  if (x < -80.0f) return 0.0f;
  if (x > 88.0f) return __builtin_inff();
  const float n = __builtin_rintf(x * 0x1.715476p+0f);
  float r = __builtin_fmaf(-n, 0x1.62e4p-1f, x);
  r = __builtin_fmaf(-n, 0x1.7f7d1cp-20f, r);
  float p = 0x1.a01a02p-13f;
  p = __builtin_fmaf(p, r, 0x1.6c16c2p-10f);
  p = __builtin_fmaf(p, r, 0x1.111112p-7f);
  p = __builtin_fmaf(p, r, 0x1.555556p-5f);
  p = __builtin_fmaf(p, r, 0x1.555556p-3f);
  p = __builtin_fmaf(p, r, 0.5f);
  p = __builtin_fmaf(p, r, 1.0f);
  p = __builtin_fmaf(p, r, 1.0f);
  return __builtin_ldexpf(p, (int)n);
}

__device__ __forceinline__ float shfl_xor_f(float v, int m) { return __shfl_xor(v, m, kWave); }
__device__ __forceinline__ float shfl_f(float v, int src) { return __shfl(v, src, kWave); }

// Sum over aligned groups of G lanes (G a power of two <= 64). The tree is
// the natural pairwise one: lanes l and l^1 first, then pairs of pairs.
template <int G>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
  for (int m = 1; m < G; m <<= 1) v = v + shfl_xor_f(v, m);
  return v;
}

// The same pairwise tree as group_sum<64> (lanes l and l^1 first, then pairs
// of pairs), computed with DPP instead of LDS shuffles; the root lands in lane
// 63. Each level adds the two operands group_sum<64> adds (after level 2 the
// lanes of a quad, after level 3 of a half-row, hold equal values, so the
// mirror patterns pick the same partner sums as xor 4 and xor 8, and row_bcast
// 15/31 deliver the xor 16/32 partners to the last row), and IEEE addition is
// commutative, so the result is bit-identical.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_plus(float v) {
  const int s = __builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROW_MASK, 0xf, false);
  return v + __int_as_float(s);
}

__device__ __forceinline__ float wave_tree_sum64(float v) {
  v = dpp_plus<0xb1, 0xf>(v);   // quad_perm [1,0,3,2]  (xor 1)
  v = dpp_plus<0x4e, 0xf>(v);   // quad_perm [2,3,0,1]  (xor 2)
  v = dpp_plus<0x141, 0xf>(v);  // row_half_mirror      (xor 4)
  v = dpp_plus<0x140, 0xf>(v);  // row_mirror           (xor 8)
  v = dpp_plus<0x142, 0xa>(v);  // row_bcast:15         (xor 16, rows 1 and 3)
  v = dpp_plus<0x143, 0xc>(v);  // row_bcast:31         (xor 32, rows 2 and 3)
  return v;                     // lane 63: the tree root
}

// The same tree for four values at once: every lane of row t (lanes
// 16t..16t+15) returns the root of value t (a, b, c, d for t = 0..3). Levels
// 1-4 run per value (afterwards every lane of a row holds that row's sum);
// levels 5 and 6 exchange rows between the values with v_permlane16_swap
// (rows [a0,a1,a2,a3], [b0..b3] -> [a0,b0,a2,b2], [a1,b1,a3,b3]) and
// v_permlane32_swap (lane halves), so each of their adds sums the same two
// operands as the single-value tree: (row 0 + row 1), (row 2 + row 3), then
// (rows 0-1 + rows 2-3). Six DPP or permute adds serve four values.
__device__ __forceinline__ float row_tree_sum16(float v) {
  v = dpp_plus<0xb1, 0xf>(v);   // quad_perm [1,0,3,2]  (xor 1)
  v = dpp_plus<0x4e, 0xf>(v);   // quad_perm [2,3,0,1]  (xor 2)
  v = dpp_plus<0x141, 0xf>(v);  // row_half_mirror      (xor 4)
  v = dpp_plus<0x140, 0xf>(v);  // row_mirror           (xor 8)
  return v;
}

__device__ __forceinline__ float wave_tree_sum64x4(float a, float b, float c, float d) {
  a = row_tree_sum16(a);
  b = row_tree_sum16(b);
  c = row_tree_sum16(c);
  d = row_tree_sum16(d);
  const auto ab = __builtin_amdgcn_permlane16_swap(__float_as_uint(a), __float_as_uint(b), false, false);
  const auto cd = __builtin_amdgcn_permlane16_swap(__float_as_uint(c), __float_as_uint(d), false, false);
  const float sab = __uint_as_float(ab[0]) + __uint_as_float(ab[1]);  // rows: a01 b01 a23 b23
  const float scd = __uint_as_float(cd[0]) + __uint_as_float(cd[1]);  // rows: c01 d01 c23 d23
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(sab), __float_as_uint(scd), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);               // rows: a b c d
}

__device__ __forceinline__ float silu_mul(float g, float u) {
  return g / (1.0f + __expf(-g)) * u;
}

// 8 nibbles of a packed word (LSB first) dequantised as s*q+b, as floats.
// q order: element i is bits [4i, 4i+4).
__device__ __forceinline__ void dequant8(uint32_t w, float s, float b, float* out) {
  uint32_t lo = w & 0x0f0f0f0fu, hi = (w >> 4) & 0x0f0f0f0fu;
  // Opaque to the optimiser, so that the byte extractions below are not
  // folded into 4-bit field extracts: each converts with one v_cvt_f32_ubyteN.
  asm("" : "+v"(lo));
  asm("" : "+v"(hi));
  out[0] = __builtin_fmaf(s, (float)(lo & 0xffu), b);
  out[1] = __builtin_fmaf(s, (float)(hi & 0xffu), b);
  out[2] = __builtin_fmaf(s, (float)((lo >> 8) & 0xffu), b);
  out[3] = __builtin_fmaf(s, (float)((hi >> 8) & 0xffu), b);
  out[4] = __builtin_fmaf(s, (float)((lo >> 16) & 0xffu), b);
  out[5] = __builtin_fmaf(s, (float)((hi >> 16) & 0xffu), b);
  out[6] = __builtin_fmaf(s, (float)(lo >> 24), b);
  out[7] = __builtin_fmaf(s, (float)(hi >> 24), b);
}

// 4 bytes (one 32-bit word of an 8-bit weight row, LSB first) -> 4 values
// s*q+b; each byte converts with one v_cvt_f32_ubyteN.
__device__ __forceinline__ void dequant4_u8(uint32_t w, float s, float b, float* out) {
  out[0] = __builtin_fmaf(s, (float)(w & 0xffu), b);
  out[1] = __builtin_fmaf(s, (float)((w >> 8) & 0xffu), b);
  out[2] = __builtin_fmaf(s, (float)((w >> 16) & 0xffu), b);
  out[3] = __builtin_fmaf(s, (float)(w >> 24), b);
}

// Sum_i q_i * x_i over the 8 nibbles of a packed word (x in element order).
__device__ __forceinline__ float qdot8(uint32_t w, const float* x, float acc) {
  const uint32_t lo = w & 0x0f0f0f0fu, hi = (w >> 4) & 0x0f0f0f0fu;
  acc = __builtin_fmaf((float)(lo & 0xffu), x[0], acc);
  acc = __builtin_fmaf((float)(hi & 0xffu), x[1], acc);
  acc = __builtin_fmaf((float)((lo >> 8) & 0xffu), x[2], acc);
  acc = __builtin_fmaf((float)((hi >> 8) & 0xffu), x[3], acc);
  acc = __builtin_fmaf((float)((lo >> 16) & 0xffu), x[4], acc);
  acc = __builtin_fmaf((float)((hi >> 16) & 0xffu), x[5], acc);
  acc = __builtin_fmaf((float)(lo >> 24), x[6], acc);
  acc = __builtin_fmaf((float)(hi >> 24), x[7], acc);
  return acc;
}

}  // namespace tfm
