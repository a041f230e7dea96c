// Router linear, OLMoE/Granite routing and the OLMoE softmax.
//
// Bit-defined arithmetic (the routing must reproduce exactly):
//  * logits[t,e] = bf16(tree64(s_0..s_63) [+ bias[e]]), lane l summing
//    x*w over h in [l*c, l*c+c) (c = H/64) with sequential fmaf from 0, and
//    tree64 the natural pairwise tree over lanes (l^1 first, then l^2, ...).
//  * softmax: max by compare-select from -FLT_MAX (NaN skipped), e = exp(l-max)
//    with route_expf, normaliser = 1/(tree over four-value chunks, each chunk
//    summed in order), p = e * normaliser (MLXOLMoERouter.h:26-61).
//  * ranks as in MLXOLMoERouter.h:65-83 (OLMoE) and
//    MLXNativeGraniteMoEPrefill.h:92-109 (Granite).
#include "route_wave.h"
#include "tfm_device.h"
#include "tfm_internal.h"

#pragma clang fp contract(off)

namespace tfm {

// One wave per (token tile of TW tokens, expert tile of EPW experts).
template <int C, int TW, bool F16>
__global__ __launch_bounds__(256) void router_logits_kernel(const uint16_t* __restrict__ x,
                                                            const uint16_t* __restrict__ w,
                                                            const float* __restrict__ bias,
                                                            int T, int H, int E, int EPW,
                                                            uint16_t* __restrict__ logits) {
  const int lane = threadIdx.x & 63;
  const int wave = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int n_tt = (T + TW - 1) / TW;
  const int n_et = (E + EPW - 1) / EPW;
  if (wave >= n_tt * n_et) return;
  const int tt = wave % n_tt, et = wave / n_tt;
  float xv[TW][C];
#pragma unroll
  for (int t = 0; t < TW; ++t) {
    const int tok = tt * TW + t;
    if (tok < T) {
      const uint4* src = reinterpret_cast<const uint4*>(x + (int64_t)tok * H + lane * C);
#pragma unroll
      for (int i = 0; i < C / 8; ++i) {
        const uint4 v = src[i];
        xv[t][8 * i + 0] = lo_st<F16>(v.x); xv[t][8 * i + 1] = hi_st<F16>(v.x);
        xv[t][8 * i + 2] = lo_st<F16>(v.y); xv[t][8 * i + 3] = hi_st<F16>(v.y);
        xv[t][8 * i + 4] = lo_st<F16>(v.z); xv[t][8 * i + 5] = hi_st<F16>(v.z);
        xv[t][8 * i + 6] = lo_st<F16>(v.w); xv[t][8 * i + 7] = hi_st<F16>(v.w);
      }
    } else {
#pragma unroll
      for (int j = 0; j < C; ++j) xv[t][j] = 0.0f;
    }
  }
  const int e_end = min(E, (et + 1) * EPW);
  for (int e = et * EPW; e < e_end; ++e) {
    float wv[C];
    const uint4* src = reinterpret_cast<const uint4*>(w + (int64_t)e * H + lane * C);
#pragma unroll
    for (int i = 0; i < C / 8; ++i) {
      const uint4 v = src[i];
      wv[8 * i + 0] = lo_st<F16>(v.x); wv[8 * i + 1] = hi_st<F16>(v.x);
      wv[8 * i + 2] = lo_st<F16>(v.y); wv[8 * i + 3] = hi_st<F16>(v.y);
      wv[8 * i + 4] = lo_st<F16>(v.z); wv[8 * i + 5] = hi_st<F16>(v.z);
      wv[8 * i + 6] = lo_st<F16>(v.w); wv[8 * i + 7] = hi_st<F16>(v.w);
    }
    const float be = bias ? bias[e] : 0.0f;
    if constexpr (TW == 4) {
      float s[4];
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        s[t] = 0.0f;
#pragma unroll
        for (int j = 0; j < C; ++j) s[t] = __builtin_fmaf(xv[t][j], wv[j], s[t]);
      }
      // Row t of the wave holds token t's logit.
      const float r = wave_tree_sum64x4(s[0], s[1], s[2], s[3]);
      const int tok = tt * 4 + (lane >> 4);
      if ((lane & 15) == 0 && tok < T) logits[(int64_t)tok * E + e] = f2st<F16>(bias ? r + be : r);
    } else {
#pragma unroll
      for (int t = 0; t < TW; ++t) {
        float s = 0.0f;
#pragma unroll
        for (int j = 0; j < C; ++j) s = __builtin_fmaf(xv[t][j], wv[j], s);
        s = wave_tree_sum64(s);
        const int tok = tt * TW + t;
        if (lane == 63 && tok < T) {
          const float v = bias ? s + be : s;
          logits[(int64_t)tok * E + e] = f2st<F16>(v);
        }
      }
    }
  }
}

// Prefill routing in one pass: router linear, top-k and the chunk histogram
// for the grouping. A workgroup takes kTopkTokensPerBlock (4) tokens with W
// waves: every wave keeps their x rows in registers and computes the logits
// of 1/W of the experts, streaming those router rows (the next one loading
// while the current one is used), each logit exactly as router_logits_kernel
// computes it. Then wave t < 4 ranks token t from the logits in LDS with the
// same wave-level ranking as topk_kernel. Few tokens take W = 8 (each wave
// waits on a chain of E/8 router-row loads instead of E/4: 512 tokens
// 21 -> 16 us); many take W = 4, two workgroups per compute unit.
template <int C, int ROUTE, bool F16, int W>
__global__ __launch_bounds__(W * 64) void router_topk_kernel(const uint16_t* __restrict__ x,
                                                          const uint16_t* __restrict__ w,
                                                          const float* __restrict__ bias, int T,
                                                          int H, int E, int K,
                                                          int32_t* __restrict__ idx,
                                                          float* __restrict__ gates_f32,
                                                          int32_t* __restrict__ hist,
                                                          uint16_t* __restrict__ logits_out) {
  constexpr int TB = kTopkTokensPerBlock;
  static_assert(TB == 4, "one ranking wave per token");
  __shared__ uint16_t s_logit[TB][64];
  __shared__ int h[65];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  if (tid <= E) h[tid] = 0;
  const int t0 = blockIdx.x * TB;
  float xv[TB][C];
#pragma unroll
  for (int t = 0; t < TB; ++t) {
    if (t0 + t < T) {
      const uint4* src = reinterpret_cast<const uint4*>(x + (int64_t)(t0 + t) * H + lane * C);
#pragma unroll
      for (int i = 0; i < C / 8; ++i) {
        const uint4 v = src[i];
        xv[t][8 * i + 0] = lo_st<F16>(v.x); xv[t][8 * i + 1] = hi_st<F16>(v.x);
        xv[t][8 * i + 2] = lo_st<F16>(v.y); xv[t][8 * i + 3] = hi_st<F16>(v.y);
        xv[t][8 * i + 4] = lo_st<F16>(v.z); xv[t][8 * i + 5] = hi_st<F16>(v.z);
        xv[t][8 * i + 6] = lo_st<F16>(v.w); xv[t][8 * i + 7] = hi_st<F16>(v.w);
      }
    } else {
#pragma unroll
      for (int j = 0; j < C; ++j) xv[t][j] = 0.0f;
    }
  }
  auto wrow = [&](uint4 (&r)[C / 8], int e) {
    const uint4* src = reinterpret_cast<const uint4*>(w + (int64_t)e * H + lane * C);
#pragma unroll
    for (int i = 0; i < C / 8; ++i) r[i] = src[i];
  };
  auto logits_of = [&](const uint4 (&r)[C / 8], int e) {
    float wv[C];
#pragma unroll
    for (int i = 0; i < C / 8; ++i) {
      wv[8 * i + 0] = lo_st<F16>(r[i].x); wv[8 * i + 1] = hi_st<F16>(r[i].x);
      wv[8 * i + 2] = lo_st<F16>(r[i].y); wv[8 * i + 3] = hi_st<F16>(r[i].y);
      wv[8 * i + 4] = lo_st<F16>(r[i].z); wv[8 * i + 5] = hi_st<F16>(r[i].z);
      wv[8 * i + 6] = lo_st<F16>(r[i].w); wv[8 * i + 7] = hi_st<F16>(r[i].w);
    }
    const float be = bias ? bias[e] : 0.0f;
    float s[TB];
#pragma unroll
    for (int t = 0; t < TB; ++t) {
      s[t] = 0.0f;
#pragma unroll
      for (int j = 0; j < C; ++j) s[t] = __builtin_fmaf(xv[t][j], wv[j], s[t]);
    }
    // Row t of the wave holds token t's logit.
    const float lg = wave_tree_sum64x4(s[0], s[1], s[2], s[3]);
    if ((lane & 15) == 0) s_logit[lane >> 4][e] = f2st<F16>(bias ? lg + be : lg);
  };
  const int epw = (E + W - 1) / W;
  const int e0 = wave * epw, e1 = min(E, e0 + epw);
  if (e0 < e1) {  // wave-uniform
    uint4 ra[C / 8], rb[C / 8];
    wrow(ra, e0);
    for (int e = e0; e < e1; e += 2) {
      if (e + 1 < e1) wrow(rb, e + 1);
      logits_of(ra, e);
      if (e + 1 >= e1) break;
      if (e + 2 < e1) wrow(ra, e + 2);
      logits_of(rb, e + 1);
    }
  }
  __syncthreads();  // every expert's logits of the block's tokens are in LDS
  const int tok = t0 + wave;
  if (wave < TB && tok < T) {  // wave-uniform
    const uint16_t* row = &s_logit[wave][0];
    if (logits_out && lane < E) logits_out[(int64_t)tok * E + lane] = row[lane];
    float g;
    int id;
    if (ROUTE == TFM_ROUTE_OLMOE) {
      uint16_t gb;
      id = olmoe_route_wave<F16>(row, E, K, &g, &gb);
    } else {
      id = granite_route_wave<F16>(row, E, K, &g);
    }
    if (lane < K) {
      idx[(int64_t)tok * K + lane] = id;
      gates_f32[(int64_t)tok * K + lane] = g;
      atomicAdd(&h[id], 1);
    }
  }
  __syncthreads();
  if (tid <= E) hist[(int64_t)blockIdx.x * (E + 1) + tid] = h[tid];
}

template <int C, bool F16>
static void launch_router_topk_c(int route_kind, const uint16_t* x, const uint16_t* w,
                                 const float* bias, int T, int H, int E, int K, int32_t* idx,
                                 float* gates_f32, int32_t* hist, uint16_t* logits_out,
                                 hipStream_t s) {
  const unsigned blocks = (unsigned)((T + kTopkTokensPerBlock - 1) / kTopkTokensPerBlock);
  const bool few = blocks < 512;  // under 2048 tokens: eight waves per workgroup
  if (route_kind == TFM_ROUTE_OLMOE) {
    if (few)
      tfm_launch(router_topk_kernel<C, TFM_ROUTE_OLMOE, F16, 8>, blocks, 512, 0, s, x, w, bias, T, H, E, K, idx, gates_f32,
                 hist, logits_out);
    else
      tfm_launch(router_topk_kernel<C, TFM_ROUTE_OLMOE, F16, 4>, blocks, 256, 0, s, x, w, bias, T, H, E, K, idx, gates_f32,
                 hist, logits_out);
  } else {
    if (few)
      tfm_launch(router_topk_kernel<C, TFM_ROUTE_GRANITE, F16, 8>, blocks, 512, 0, s, x, w, bias, T, H, E, K, idx, gates_f32,
                 hist, logits_out);
    else
      tfm_launch(router_topk_kernel<C, TFM_ROUTE_GRANITE, F16, 4>, blocks, 256, 0, s, x, w, bias, T, H, E, K, idx, gates_f32,
                 hist, logits_out);
  }
}

template <bool F16>
static bool router_topk_dt(int route_kind, const uint16_t* x, const uint16_t* w, const float* bias,
                           int T, int H, int E, int K, int32_t* idx, float* gates_f32, int32_t* hist,
                           uint16_t* logits_out, hipStream_t s) {
  switch (H) {
    case 512: launch_router_topk_c<8, F16>(route_kind, x, w, bias, T, H, E, K, idx, gates_f32, hist, logits_out, s); break;
    case 1024: launch_router_topk_c<16, F16>(route_kind, x, w, bias, T, H, E, K, idx, gates_f32, hist, logits_out, s); break;
    case 1536: launch_router_topk_c<24, F16>(route_kind, x, w, bias, T, H, E, K, idx, gates_f32, hist, logits_out, s); break;
    case 2048: launch_router_topk_c<32, F16>(route_kind, x, w, bias, T, H, E, K, idx, gates_f32, hist, logits_out, s); break;
    default: return false;
  }
  return true;
}

bool launch_router_topk(int route_kind, bool f16, const uint16_t* x, const uint16_t* w, const float* bias,
                        int T, int H, int E, int K, int32_t* idx, float* gates_f32, int32_t* hist,
                        uint16_t* logits_out, hipStream_t s) {
  if (T <= 0) return true;
  const bool ok = f16 ? router_topk_dt<true>(route_kind, x, w, bias, T, H, E, K, idx, gates_f32, hist, logits_out, s)
                      : router_topk_dt<false>(route_kind, x, w, bias, T, H, E, K, idx, gates_f32, hist, logits_out, s);
  if (ok) check_hip(hipGetLastError(), "router_topk launch");
  return ok;
}

// Any H % 64 == 0: the same arithmetic with scalar loads.
template <bool F16>
__global__ __launch_bounds__(256) void router_logits_generic(const uint16_t* __restrict__ x,
                                                             const uint16_t* __restrict__ w,
                                                             const float* __restrict__ bias,
                                                             int T, int H, int E,
                                                             uint16_t* __restrict__ logits) {
  const int lane = threadIdx.x & 63;
  const int wave = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (wave >= T * E) return;
  const int tok = wave / E, e = wave % E;
  const int c = H / 64;
  float s = 0.0f;
  for (int j = 0; j < c; ++j)
    s = __builtin_fmaf(st2f<F16>(x[(int64_t)tok * H + lane * c + j]), st2f<F16>(w[(int64_t)e * H + lane * c + j]), s);
  s = wave_tree_sum64(s);
  if (lane == 63) logits[(int64_t)tok * E + e] = f2st<F16>(bias ? s + bias[e] : s);
}

template <int C, bool F16>
static void launch_router_c(const uint16_t* x, const uint16_t* w, const float* bias, int T,
                            int H, int E, uint16_t* logits, hipStream_t s) {
  if (T <= 64) {
    // Few tokens: one wave per (token, expert), so the router rows stream in
    // parallel across the chip.
    const int waves = T * E;
    tfm_launch(router_logits_kernel<C, 1, F16>, (waves + 3) / 4, 256, 0, s, x, w, bias, T, H, E, 1, logits);
  } else {
    // Many tokens: a wave keeps 4 token rows in registers and walks EPW
    // experts, reading router rows from L2: as few experts per wave as keep
    // about 2048 waves (EPW 1 to 16, a power of two).
    constexpr int TW = 4;
    const int64_t tiles = (T + TW - 1) / TW;
    int EPW = 1;
    while (EPW < 16 && tiles * ((E + 2 * EPW - 1) / (2 * EPW)) >= 2048) EPW *= 2;
    const int waves = (int)(tiles * ((E + EPW - 1) / EPW));
    tfm_launch(router_logits_kernel<C, TW, F16>, (waves + 3) / 4, 256, 0, s, x, w, bias, T, H, E, EPW, logits);
  }
}

template <bool F16>
static void router_logits_dt(const uint16_t* x, const uint16_t* w, const float* bias, int T,
                             int H, int E, uint16_t* logits, hipStream_t s) {
  switch (H) {
    case 512: launch_router_c<8, F16>(x, w, bias, T, H, E, logits, s); break;
    case 1024: launch_router_c<16, F16>(x, w, bias, T, H, E, logits, s); break;
    case 1536: launch_router_c<24, F16>(x, w, bias, T, H, E, logits, s); break;
    case 2048: launch_router_c<32, F16>(x, w, bias, T, H, E, logits, s); break;
    default: {
      const int64_t waves = (int64_t)T * E;
      router_logits_generic<F16><<<(unsigned)((waves + 3) / 4), 256, 0, s>>>(x, w, bias, T, H, E, logits);
    }
  }
}

void launch_router_logits(bool f16, const uint16_t* x, const uint16_t* w, const float* bias, int T,
                          int H, int E, uint16_t* logits, hipStream_t s) {
  if (T <= 0) return;
  if (f16)
    router_logits_dt<true>(x, w, bias, T, H, E, logits, s);
  else
    router_logits_dt<false>(x, w, bias, T, H, E, logits, s);
  check_hip(hipGetLastError(), "router_logits launch");
}

// Affine-quantised router (native_affine_qmm of the router weight,
// export_native_olmoe_target.py:194-200) dequantised once per call into a
// dense [E, H] matrix in the storage dtype: w[e,h] = st(fmaf(s, q, b)), the
// value native_affine_ops.py:29-36 rounds to the scales' dtype. The dense
// router kernels then compute the logits in their bit-defined order. One
// thread per packed word (8 or 4 codes); group size 64.
template <bool F16, int BITS>
__global__ __launch_bounds__(256) void dequant_router_kernel(const uint32_t* __restrict__ q,
                                                             const uint16_t* __restrict__ sc,
                                                             const uint16_t* __restrict__ bi,
                                                             int64_t words, uint16_t* __restrict__ w) {
  constexpr int PER = 32 / BITS;
  constexpr uint32_t MASK = (1u << BITS) - 1u;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= words) return;
  const int64_t k0 = i * PER;               // first element: row k0 / H, column k0 % H
  const int64_t g = k0 / 64;                // rows are whole groups (H % 64 == 0)
  const float s = st2f<F16>(sc[g]), b = st2f<F16>(bi[g]);
  const uint32_t word = q[i];
  uint16_t out[PER];
#pragma unroll
  for (int j = 0; j < PER; ++j)
    out[j] = f2st<F16>(__builtin_fmaf(s, (float)((word >> (BITS * j)) & MASK), b));
  if constexpr (PER == 8) {
    uint4 v;
    v.x = out[0] | ((uint32_t)out[1] << 16);
    v.y = out[2] | ((uint32_t)out[3] << 16);
    v.z = out[4] | ((uint32_t)out[5] << 16);
    v.w = out[6] | ((uint32_t)out[7] << 16);
    *reinterpret_cast<uint4*>(w + k0) = v;
  } else {
    uint2 v;
    v.x = out[0] | ((uint32_t)out[1] << 16);
    v.y = out[2] | ((uint32_t)out[3] << 16);
    *reinterpret_cast<uint2*>(w + k0) = v;
  }
}

void launch_dequant_router(bool f16, int bits, const tfm_affine& r, int E, int H, uint16_t* w,
                           hipStream_t s) {
  const int64_t words = (int64_t)E * H * bits / 32;
  if (words <= 0) return;
  const unsigned blocks = (unsigned)((words + 255) / 256);
  const uint32_t* q = static_cast<const uint32_t*>(r.q);
  const uint16_t* sc = static_cast<const uint16_t*>(r.scales);
  const uint16_t* bi = static_cast<const uint16_t*>(r.biases);
  if (f16 && bits == 8)
    dequant_router_kernel<true, 8><<<blocks, 256, 0, s>>>(q, sc, bi, words, w);
  else if (f16)
    dequant_router_kernel<true, 4><<<blocks, 256, 0, s>>>(q, sc, bi, words, w);
  else if (bits == 8)
    dequant_router_kernel<false, 8><<<blocks, 256, 0, s>>>(q, sc, bi, words, w);
  else
    dequant_router_kernel<false, 4><<<blocks, 256, 0, s>>>(q, sc, bi, words, w);
  check_hip(hipGetLastError(), "router dequant launch");
}

__device__ __forceinline__ float readlane_f(float v, int j) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), j));
}

// One wave per token. gates_native: bf16 probabilities (OLMoE) or fp32
// (Granite); gates_f32: fp32 copy. Either may be null.
template <int ROUTE, bool F16>
__global__ __launch_bounds__(256) void topk_kernel(const uint16_t* __restrict__ logits, int T,
                                                   int E, int K, int32_t* __restrict__ idx,
                                                   void* __restrict__ gates_native,
                                                   float* __restrict__ gates_f32) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;  // whole wave exits together
  const uint16_t* row = logits + (int64_t)t * E;
  float g;
  int id;
  if (ROUTE == TFM_ROUTE_OLMOE) {
    uint16_t gb;
    id = olmoe_route_wave<F16>(row, E, K, &g, &gb);
    if (lane < K && gates_native) static_cast<uint16_t*>(gates_native)[(int64_t)t * K + lane] = gb;
  } else {
    id = granite_route_wave<F16>(row, E, K, &g);
    if (lane < K && gates_native) static_cast<float*>(gates_native)[(int64_t)t * K + lane] = g;
  }
  if (lane < K) {
    idx[(int64_t)t * K + lane] = id;
    if (gates_f32) gates_f32[(int64_t)t * K + lane] = g;
  }
}

// Top-k of kTopkTokensPerBlock tokens per workgroup (one wave per token at a
// time), plus the histogram of the workgroup's routes over the E experts for
// the grouping pass (its chunk is kTopkTokensPerBlock * K flat routes).
template <int ROUTE, bool F16>
__global__ __launch_bounds__(256) void topk_hist_kernel(const uint16_t* __restrict__ logits, int T,
                                                        int E, int K, int32_t* __restrict__ idx,
                                                        float* __restrict__ gates_f32,
                                                        int32_t* __restrict__ hist) {
  __shared__ int h[65];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  if (tid <= E) h[tid] = 0;
  __syncthreads();
  constexpr int kPerWave = kTopkTokensPerBlock / 4;
  for (int i = 0; i < kPerWave; ++i) {
    const int t = blockIdx.x * kTopkTokensPerBlock + wave * kPerWave + i;
    if (t >= T) break;  // wave-uniform
    const uint16_t* row = logits + (int64_t)t * E;
    float g;
    int id;
    if (ROUTE == TFM_ROUTE_OLMOE) {
      uint16_t gb;
      id = olmoe_route_wave<F16>(row, E, K, &g, &gb);
    } else {
      id = granite_route_wave<F16>(row, E, K, &g);
    }
    if (lane < K) {
      idx[(int64_t)t * K + lane] = id;
      gates_f32[(int64_t)t * K + lane] = g;
      atomicAdd(&h[id], 1);
    }
  }
  __syncthreads();
  if (tid <= E) hist[(int64_t)blockIdx.x * (E + 1) + tid] = h[tid];
}

template <bool F16>
static void topk_hist_dt(int route_kind, const uint16_t* logits, int T, int E, int K, int32_t* idx,
                         float* gates_f32, int32_t* hist, hipStream_t s) {
  const unsigned blocks = (unsigned)((T + kTopkTokensPerBlock - 1) / kTopkTokensPerBlock);
  if (route_kind == TFM_ROUTE_OLMOE)
    tfm_launch(topk_hist_kernel<TFM_ROUTE_OLMOE, F16>, blocks, 256, 0, s, logits, T, E, K, idx, gates_f32, hist);
  else
    tfm_launch(topk_hist_kernel<TFM_ROUTE_GRANITE, F16>, blocks, 256, 0, s, logits, T, E, K, idx, gates_f32, hist);
}

void launch_topk_hist(int route_kind, bool f16, const uint16_t* logits, int T, int E, int K, int32_t* idx,
                      float* gates_f32, int32_t* hist, hipStream_t s) {
  if (T <= 0) return;
  if (f16)
    topk_hist_dt<true>(route_kind, logits, T, E, K, idx, gates_f32, hist, s);
  else
    topk_hist_dt<false>(route_kind, logits, T, E, K, idx, gates_f32, hist, s);
  check_hip(hipGetLastError(), "topk_hist launch");
}

template <bool F16>
static void topk_dt(int route_kind, const uint16_t* logits, int T, int E, int K, int32_t* idx,
                    void* gates_native, float* gates_f32, hipStream_t s) {
  const unsigned blocks = (unsigned)((T + 3) / 4);
  if (route_kind == TFM_ROUTE_OLMOE)
    topk_kernel<TFM_ROUTE_OLMOE, F16><<<blocks, 256, 0, s>>>(logits, T, E, K, idx, gates_native, gates_f32);
  else
    topk_kernel<TFM_ROUTE_GRANITE, F16><<<blocks, 256, 0, s>>>(logits, T, E, K, idx, gates_native, gates_f32);
}

void launch_topk(int route_kind, bool f16, const uint16_t* logits, int T, int E, int K, int32_t* idx,
                 void* gates_native, float* gates_f32, hipStream_t s) {
  if (T <= 0) return;
  if (f16)
    topk_dt<true>(route_kind, logits, T, E, K, idx, gates_native, gates_f32, s);
  else
    topk_dt<false>(route_kind, logits, T, E, K, idx, gates_native, gates_f32, s);
  check_hip(hipGetLastError(), "topk launch");
}

// Ranking only (values given): one wave per row.
template <int RULE, bool F16>
__global__ __launch_bounds__(256) void rank_topk_kernel(const uint16_t* __restrict__ values, int T,
                                                        int n, int K, int32_t* __restrict__ idx) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;  // whole wave exits together
  const bool valid = lane < n;
  const float v = valid ? st2f<F16>(values[(int64_t)t * n + lane]) : 0.0f;
  const bool vn = v != v;
  int rank = 0;
  for (int j = 0; j < n; ++j) {
    const float o = readlane_f(v, j);
    const bool on = o != o;
    const bool equal = (on && vn) || (!on && !vn && o == v);
    const bool ahead = RULE == TFM_ROUTE_OLMOE ? (!on && (vn || o > v)) : (!on && (vn || o < v));
    rank += (ahead || (equal && j < lane)) ? 1 : 0;
  }
  if (!valid) return;
  if (RULE == TFM_ROUTE_OLMOE) {
    if (rank < K) idx[(int64_t)t * K + rank] = lane;
  } else {
    if (rank >= n - K) idx[(int64_t)t * K + rank - (n - K)] = lane;
  }
}

void launch_rank_topk(int rule, bool f16, const uint16_t* values, int T, int n, int K, int32_t* idx,
                      hipStream_t s) {
  if (T <= 0) return;
  const unsigned blocks = (unsigned)((T + 3) / 4);
  if (rule == TFM_ROUTE_OLMOE && f16)
    rank_topk_kernel<TFM_ROUTE_OLMOE, true><<<blocks, 256, 0, s>>>(values, T, n, K, idx);
  else if (rule == TFM_ROUTE_OLMOE)
    rank_topk_kernel<TFM_ROUTE_OLMOE, false><<<blocks, 256, 0, s>>>(values, T, n, K, idx);
  else if (f16)
    rank_topk_kernel<TFM_ROUTE_GRANITE, true><<<blocks, 256, 0, s>>>(values, T, n, K, idx);
  else
    rank_topk_kernel<TFM_ROUTE_GRANITE, false><<<blocks, 256, 0, s>>>(values, T, n, K, idx);
  check_hip(hipGetLastError(), "rank_topk launch");
}

template <bool F16>
__global__ __launch_bounds__(256) void olmoe_softmax_kernel(const uint16_t* __restrict__ logits,
                                                            int T, int E,
                                                            uint16_t* __restrict__ probs) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;  // whole wave exits together
  const bool valid = lane < E;
  const float ld = valid ? st2f<F16>(logits[(int64_t)t * E + lane]) : -__builtin_inff();
  float norm;
  const float ex = wave_softmax_exp(ld, &norm);
  if (valid) probs[(int64_t)t * E + lane] = f2st<F16>(ex * norm);
}

void launch_olmoe_softmax(bool f16, const uint16_t* logits, int T, int E, uint16_t* probs, hipStream_t s) {
  if (T <= 0) return;
  if (f16)
    olmoe_softmax_kernel<true><<<(unsigned)((T + 3) / 4), 256, 0, s>>>(logits, T, E, probs);
  else
    olmoe_softmax_kernel<false><<<(unsigned)((T + 3) / 4), 256, 0, s>>>(logits, T, E, probs);
  check_hip(hipGetLastError(), "olmoe_softmax launch");
}

}  // namespace tfm
