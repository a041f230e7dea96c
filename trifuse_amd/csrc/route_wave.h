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
// Selection is K rounds of "largest remaining key": keys are the values mapped
// to order-preserving unsigned integers, the maximum is a DPP wave reduction,
// and a ballot of the lanes holding it resolves ties by id.
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
// (others return -1 / 0); the gate's storage bits come back in *gate_bits.
template <bool F16 = false>
__device__ __forceinline__ int olmoe_route_wave(const uint16_t* __restrict__ row, int E, int K,
                                                float* gate, uint16_t* gate_bits) {
  const int lane = threadIdx.x & 63;
  const bool valid = lane < E;
  const float ld = valid ? st2f<F16>(row[lane]) : -__builtin_inff();
  float norm;
  const float ex = wave_softmax_exp(ld, &norm);
  const uint16_t pb = f2st<F16>(ex * norm);
  const float p = st2f<F16>(pb);
  // NaN ranks after every number: key 0, below sortable(-inf) = 0x007fffff.
  uint32_t key = p != p ? 0u : sortable_key(p);
  bool removed = !valid;
  int my_idx = -1;
  float my_gate = 0.0f;
  uint16_t my_bits = 0;
  for (int slot = 0; slot < K; ++slot) {
    const uint32_t kmax = wave_max_u32(removed ? 0u : key);
    const uint64_t m = __ballot(!removed && key == kmax);
    const int sel = __ffsll((unsigned long long)m) - 1;  // ties: lowest id
    // Slot `slot` goes to lane `slot` of the result.
    const float g = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(p), sel));
    const int gb = __builtin_amdgcn_readlane((int)pb, sel);
    if (lane == slot) {
      my_idx = sel;
      my_gate = g;
      my_bits = (uint16_t)gb;
    }
    if (lane == sel) removed = true;
  }
  *gate = my_gate;
  *gate_bits = my_bits;
  return my_idx;
}

// Granite routing of one token. Lane s < K returns slot s's expert id and fp32
// gate; other lanes return -1.
template <bool F16 = false>
__device__ __forceinline__ int granite_route_wave(const uint16_t* __restrict__ row, int E, int K,
                                                  float* gate) {
  const int lane = threadIdx.x & 63;
  const bool valid = lane < E;
  const float v = valid ? st2f<F16>(row[lane]) : 0.0f;
  // NaN ranks above every number: key ~0u.
  const uint32_t key = v != v ? 0xffffffffu : sortable_key(v);
  bool removed = !valid;
  int my_idx = -1;
  float my_val = 0.0f;
  for (int r = 0; r < K; ++r) {
    const uint32_t kmax = wave_max_u32(removed ? 0u : key);
    const uint64_t m = __ballot(!removed && key == kmax);
    const int sel = 63 - __clzll((long long)m);  // ties: the higher id ranks higher
    const int slot = K - 1 - r;
    const float sv = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), sel));
    if (lane == slot) {
      my_idx = sel;
      my_val = sv;
    }
    if (lane == sel) removed = true;
  }
  const float ld = lane < K ? my_val : -__builtin_inff();
  float norm;
  const float ex = wave_softmax_exp(ld, &norm);
  *gate = ex * norm;
  return my_idx;
}

}  // namespace tfm
