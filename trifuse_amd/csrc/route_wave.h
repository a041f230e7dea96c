// Per-token routing inside one wave (lane = expert id, E <= 64): the OLMoE and
// Granite rules with the reference's rounding points, slot order and tie rules.
//
//  * OLMoE (MLXOLMoERouter.h:19-84, native_affine_ops.py:128-146): fp32
//    softmax over E, probabilities rounded to bf16, then the K largest in
//    descending order; equal values go to the lower expert id; NaN after every
//    number. Gates are the bf16 probabilities (no renormalisation).
//  * Granite (MLXNativeGraniteMoEPrefill.h:77-150, native_affine_lowering.py:61-74):
//    a stable ascending rank (NaN last, equal values by increasing id); the K
//    highest ranks fill slots rank-(E-K) in ascending order; gates are the fp32
//    softmax over the K selected logits.
//
// Selection is K rounds of "largest remaining key". A lane's key is unique: the
// value's 16-bit storage pattern mapped to an order-preserving integer (NaN
// placed by the rule), then the tie rule's id order in the low 6 bits; absent
// and taken lanes hold 0. A round is one DPP maximum, and the winner's id is
// the maximum's low bits.
#pragma once

#include "tfm_device.h"

namespace tfm {

// Softmax over 64 lanes (absent lanes hold -inf): returns e_l and writes the
// normaliser 1/sum. Order of arithmetic: max by compare-select from -FLT_MAX
// (NaN skipped), e = exp(l - max) with route_expf, the sum as four-value
// chunks (each summed in order) combined by the natural pairwise tree, and
// p = e * (1/sum) (MLXOLMoERouter.h:26-61). The cross-lane steps are DPP
// moves: the maximum is exact in any order, and each tree level adds the two
// operands the xor-partner tree adds (the quads, then half-rows, then rows
// hold equal values), so the result is that tree's bit for bit.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_max_f(float v) {
  const int s = __builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), CTRL, ROW_MASK, 0xf, false);
  return fmaxf(v, __int_as_float(s));
}

template <int CTRL>
__device__ __forceinline__ float dpp_mov_f(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}

__device__ __forceinline__ float wave_softmax_exp(float ld, float* norm) {
  float m = -3.40282347e38f;
  m = m < ld ? ld : m;
  m = dpp_max_f<0xb1, 0xf>(m);   // quad_perm [1,0,3,2]
  m = dpp_max_f<0x4e, 0xf>(m);   // quad_perm [2,3,0,1]
  m = dpp_max_f<0x141, 0xf>(m);  // row_half_mirror
  m = dpp_max_f<0x140, 0xf>(m);  // row_mirror
  m = dpp_max_f<0x142, 0xa>(m);  // row_bcast:15
  m = dpp_max_f<0x143, 0xc>(m);  // row_bcast:31
  m = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(m), 63));
  const float ex = route_expf(ld - m);
  // Lane values of the quad: quad_perm [0,0,0,0] .. [3,3,3,3].
  const float a0 = dpp_mov_f<0x00>(ex), a1 = dpp_mov_f<0x55>(ex), a2 = dpp_mov_f<0xaa>(ex),
              a3 = dpp_mov_f<0xff>(ex);
  float s = a0 + a1;
  s = s + a2;
  s = s + a3;
  s = dpp_plus<0x141, 0xf>(s);  // + quad l ^ 1 (xor 4)
  s = dpp_plus<0x140, 0xf>(s);  // + half-row l ^ 1 (xor 8)
  s = dpp_plus<0x142, 0xa>(s);  // + row l ^ 1 (xor 16), rows 1 and 3
  s = dpp_plus<0x143, 0xc>(s);  // + rows 0-1 (xor 32), rows 2 and 3
  s = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(s), 63));
  *norm = 1.0f / s;
  return ex;
}

// Order-preserving map of a non-NaN float to uint32 (-0 and +0 map alike).
__device__ __forceinline__ uint32_t sortable_key(float f) {
  uint32_t u = __float_as_uint(f == 0.0f ? 0.0f : f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// The same map for a non-NaN bf16 or half storage pattern: 16-bit keys whose
// order is the values' order (-0 and +0 map alike). Both formats are sign and
// magnitude, so equal keys mean equal values.
__device__ __forceinline__ uint32_t sortable_key16(uint32_t u) {
  u = u == 0x8000u ? 0u : u;
  return (u & 0x8000u) ? (~u & 0xffffu) : (u | 0x8000u);
}

template <int CTRL, int ROW_MASK>
__device__ __forceinline__ uint32_t dpp_max_u32(uint32_t v) {
  const uint32_t s = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, ROW_MASK, 0xf, false);
  return v > s ? v : s;
}

// Wave-uniform maximum of v over all 64 lanes (exec must be full).
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  v = dpp_max_u32<0xb1, 0xf>(v);   // quad_perm [1,0,3,2]
  v = dpp_max_u32<0x4e, 0xf>(v);   // quad_perm [2,3,0,1]
  v = dpp_max_u32<0x141, 0xf>(v);  // row_half_mirror
  v = dpp_max_u32<0x140, 0xf>(v);  // row_mirror
  v = dpp_max_u32<0x142, 0xa>(v);  // row_bcast:15
  v = dpp_max_u32<0x143, 0xc>(v);  // row_bcast:31
  return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}

// OLMoE routing of one token. row: E logits in the storage dtype (bf16, or
// half when F16). Lane s < K of the wave returns slot s's expert id and gate
// (others return -1 / 0); the gate's storage bits come back in *gate_bits and,
// when `selected` is given, the mask of the K chosen ids in *selected.
template <bool F16 = false>
__device__ __forceinline__ int olmoe_route_wave(const uint16_t* __restrict__ row, int E, int K,
                                                float* gate, uint16_t* gate_bits,
                                                uint64_t* selected = nullptr) {
  const int lane = threadIdx.x & 63;
  const bool valid = lane < E;
  const float ld = valid ? st2f<F16>(row[lane]) : -__builtin_inff();
  float norm;
  const float ex = wave_softmax_exp(ld, &norm);
  const uint16_t pb = f2st<F16>(ex * norm);
  const float p = st2f<F16>(pb);
  // Larger probabilities first, NaN after every number (key 1, below the key
  // of -inf), equal values by increasing id (63 - id in the low bits). Every
  // present lane's key is at least 64.
  const uint32_t k16 = p != p ? 1u : sortable_key16(pb) + 2u;
  uint32_t key = valid ? (k16 << 6) | (uint32_t)(63 - lane) : 0u;
  int my_idx = -1;
  for (int slot = 0; slot < K; ++slot) {
    const int sel = 63 - (int)(wave_max_u32(key) & 63u);
    if (lane == slot) my_idx = sel;  // slot s goes to lane s of the result
    if (lane == sel) key = 0u;
  }
  const int src = my_idx < 0 ? lane : my_idx;
  const float g = __int_as_float(__shfl(__float_as_int(p), src, 64));
  const int gb = __shfl((int)pb, src, 64);
  *gate = my_idx < 0 ? 0.0f : g;
  *gate_bits = my_idx < 0 ? (uint16_t)0 : (uint16_t)gb;
  if (selected) *selected = __ballot(valid && key == 0u);
  return my_idx;
}

// Granite routing of one token. Lane s < K returns slot s's expert id and fp32
// gate; other lanes return -1. With `selected`, *selected gets the mask of the
// K chosen ids.
template <bool F16 = false>
__device__ __forceinline__ int granite_route_wave(const uint16_t* __restrict__ row, int E, int K,
                                                  float* gate, uint64_t* selected = nullptr) {
  const int lane = threadIdx.x & 63;
  const bool valid = lane < E;
  const uint32_t vb = valid ? row[lane] : 0u;
  const float v = st2f<F16>((uint16_t)vb);
  // NaN ranks above every number (key 0x10001, above the key of +inf); equal
  // values: the higher id ranks higher (id in the low bits). Every present
  // lane's key is at least 64.
  const uint32_t k16 = v != v ? 0x10001u : sortable_key16(vb) + 1u;
  uint32_t key = valid ? (k16 << 6) | (uint32_t)lane : 0u;
  int my_idx = -1;
  for (int r = 0; r < K; ++r) {
    const int sel = (int)(wave_max_u32(key) & 63u);
    if (lane == K - 1 - r) my_idx = sel;
    if (lane == sel) key = 0u;
  }
  const float sv = __int_as_float(__shfl(__float_as_int(v), my_idx < 0 ? lane : my_idx, 64));
  const float ld = lane < K ? sv : -__builtin_inff();
  float norm;
  const float ex = wave_softmax_exp(ld, &norm);
  *gate = ex * norm;
  if (selected) *selected = __ballot(valid && key == 0u);
  return my_idx;
}

}  // namespace tfm
