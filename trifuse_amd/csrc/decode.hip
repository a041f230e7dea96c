// Decode path of the MoE block (few routes: T*K <= 256).
//
// The block that NativeGraniteMoEPrefill::moe runs per layer
// (MLXNativeGraniteMoEPrefill.h:627-702) as four kernels:
//   1. decode_route_kernel: one workgroup per token computes the token's E
//      router logits (same arithmetic as the router kernel) and its top-k,
//   2. decode_gateup_kernel: every workgroup first groups the T*K routes by
//      expert (stable, in LDS; a few hundred VALU ops) and then streams a few
//      gate/up row units of one active expert through the dequant GEMV with
//      the SwiGLU epilogue; workgroup (0, 0) also publishes the grouping for
//      the next kernels,
//   3. the down dequant GEMV scaled by each route's gate (gemv.hip),
//   4. the ordered K reduction + residual (combine.hip).
// Each kernel boundary is the only synchronisation: on MI355X a launch costs
// ~2.4 us, while a cross-workgroup hand-off inside a kernel needs an L2
// write-back per workgroup, which costs more at these grid sizes.
#include "gemv_body.h"
#include "route_wave.h"
#include "tfm_device.h"
#include "tfm_internal.h"

namespace tfm {

constexpr int kDecodeMaxRoutes = 256;  // one thread per route in the grouping

struct DecodeGateUpArgs {
  const uint16_t* x;       // [T, H]
  const int32_t* idx;      // [R] route -> expert (from decode_route_kernel)
  int T, E, K, H, I;
  tfm_affine gate, up;
  int32_t* order;          // [R] sorted position -> flat route
  int32_t* inverse;        // [R]
  int32_t* offsets;        // [E+1]
  int32_t* active;         // [E+1]
  uint16_t* h;             // [R, I] SwiGLU output, expert-sorted rows
  uint32_t* status;        // the call's status word, cleared here
};

__device__ __forceinline__ uint64_t lanemask_lt64() {
  const int lane = threadIdx.x & 63;
  return lane == 0 ? 0ull : (~0ull >> (64 - lane));
}

template <int LG>
__global__ __launch_bounds__(256) void decode_gateup_kernel(DecodeGateUpArgs A) {
  __shared__ GemvLds L;
  __shared__ int s_order[kDecodeMaxRoutes];
  __shared__ int s_off[65];
  __shared__ int s_act[65];
  __shared__ int wcnt[4][64];
  __shared__ int wpre[4][64];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int E = A.E, K = A.K;
  const int R = A.T * K;

  // Stable grouping of the R routes: route f's position is the number of
  // routes to lower experts plus routes to its expert with a lower index.
  (&wcnt[0][0])[tid] = 0;
  const bool live = tid < R;
  const int e = live ? A.idx[tid] : 0;
  __syncthreads();
  uint64_t match = __ballot(live);
#pragma unroll
  for (int bit = 0; bit < 6; ++bit) {
    const bool b = (e >> bit) & 1;
    const uint64_t ones = __ballot(live && b);
    match &= b ? ones : ~ones;
  }
  const int rank_w = __popcll(match & lanemask_lt64());
  if (live && rank_w == 0) wcnt[wave][e] = __popcll(match);
  __syncthreads();
  if (wave == 0) {
    const int c0 = wcnt[0][lane], c1 = wcnt[1][lane], c2 = wcnt[2][lane], c3 = wcnt[3][lane];
    const int cnt = c0 + c1 + c2 + c3;
    int incl = cnt;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int o = __shfl_up(incl, d, 64);
      if (lane >= d) incl += o;
    }
    const int excl = incl - cnt;
    if (lane < E) {
      s_off[lane] = excl;
      wpre[0][lane] = excl;
      wpre[1][lane] = excl + c0;
      wpre[2][lane] = excl + c0 + c1;
      wpre[3][lane] = excl + c0 + c1 + c2;
    }
    if (lane == 63) s_off[E] = incl;
    const uint64_t act = __ballot(lane < E && cnt > 0);
    if (lane < E && cnt > 0) s_act[__popcll(act & lanemask_lt64())] = lane;
    if (lane == 0) s_act[E] = __popcll(act);
  }
  __syncthreads();
  int pos = 0;
  if (live) {
    pos = wpre[wave][e] + rank_w;
    s_order[pos] = tid;
  }
  __syncthreads();

  // Workgroup (0, 0) publishes the grouping for the down GEMV and the combine.
  if (blockIdx.x == 0 && blockIdx.y == 0) {
    if (live) {
      A.order[pos] = tid;
      A.inverse[tid] = pos;
    }
    if (tid <= E) {
      A.offsets[tid] = s_off[tid];
      if (tid == E || tid < s_act[E]) A.active[tid] = s_act[tid];
    }
    if (tid == 0) *A.status = 0u;
  }

  // Gate/up rows: kGemvUnits row units of active expert blockIdx.y.
  const int N = A.I;
  if ((int)blockIdx.y >= s_act[E]) return;
  const int ex = s_act[blockIdx.y];
  uint16_t* h = A.h;
  auto xrow = [&](int j) -> int64_t { return (int64_t)(s_order[j] / K); };
  auto stage = [&](int, int) {};
  auto emit = [&](int j, int, int n, float gt, float up) {
    const float hv = gt * __builtin_amdgcn_rcpf(1.0f + __expf(-gt)) * up;
    h[(int64_t)j * N + n] = f2bf(hv);
  };
  gemv_units<LG, 2, kGemvUnits>(L, A.x, A.H, N, A.gate, A.up, ex, s_off[ex], s_off[ex + 1],
                                blockIdx.x * kGemvUnits, xrow, stage, emit);
}

// Router logits and top-k of one token per workgroup (16 waves). Logit e is
// computed by one wave exactly as the router kernel does (lane l sums x*w
// over its H/64 contiguous elements with sequential fused multiply-adds, then
// the xor-shuffle tree across lanes, then + bias, rounded to bf16); wave 0
// then ranks the E logits of the token.
template <int C, int ROUTE>
__global__ __launch_bounds__(1024) void decode_route_kernel(const uint16_t* __restrict__ x,
                                                            const uint16_t* __restrict__ w,
                                                            const float* __restrict__ bias,
                                                            int H, int E, int K,
                                                            uint16_t* __restrict__ logits,
                                                            int32_t* __restrict__ idx,
                                                            float* __restrict__ gates) {
  __shared__ uint16_t s_logit[64];
  const int t = blockIdx.x;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  float xv[C];
  const uint4* xs = reinterpret_cast<const uint4*>(x + (int64_t)t * H + lane * C);
#pragma unroll
  for (int i = 0; i < C / 8; ++i) {
    const uint4 v = xs[i];
    xv[8 * i + 0] = lo_bf(v.x); xv[8 * i + 1] = hi_bf(v.x);
    xv[8 * i + 2] = lo_bf(v.y); xv[8 * i + 3] = hi_bf(v.y);
    xv[8 * i + 4] = lo_bf(v.z); xv[8 * i + 5] = hi_bf(v.z);
    xv[8 * i + 6] = lo_bf(v.w); xv[8 * i + 7] = hi_bf(v.w);
  }
  for (int e = wave; e < E; e += 16) {
    const uint4* ws = reinterpret_cast<const uint4*>(w + (int64_t)e * H + lane * C);
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < C / 8; ++i) {
      const uint4 v = ws[i];
      s = __builtin_fmaf(xv[8 * i + 0], lo_bf(v.x), s);
      s = __builtin_fmaf(xv[8 * i + 1], hi_bf(v.x), s);
      s = __builtin_fmaf(xv[8 * i + 2], lo_bf(v.y), s);
      s = __builtin_fmaf(xv[8 * i + 3], hi_bf(v.y), s);
      s = __builtin_fmaf(xv[8 * i + 4], lo_bf(v.z), s);
      s = __builtin_fmaf(xv[8 * i + 5], hi_bf(v.z), s);
      s = __builtin_fmaf(xv[8 * i + 6], lo_bf(v.w), s);
      s = __builtin_fmaf(xv[8 * i + 7], hi_bf(v.w), s);
    }
    s = wave_tree_sum64(s);
    if (lane == 63) {
      const uint16_t lb = f2bf(bias ? s + bias[e] : s);
      s_logit[e] = lb;
      if (logits) logits[(int64_t)t * E + e] = lb;
    }
  }
  __syncthreads();
  if (wave != 0) return;
  float g;
  int id;
  if (ROUTE == TFM_ROUTE_OLMOE) {
    uint16_t gb;
    id = olmoe_route_wave(s_logit, E, K, &g, &gb);
  } else {
    id = granite_route_wave(s_logit, E, K, &g);
  }
  if (lane < K) {
    idx[(int64_t)t * K + lane] = id;
    gates[(int64_t)t * K + lane] = g;
  }
}

// Any H % 64 == 0: the same arithmetic as decode_route_kernel with scalar loads.
template <int ROUTE>
__global__ __launch_bounds__(1024) void decode_route_generic(const uint16_t* __restrict__ x,
                                                             const uint16_t* __restrict__ w,
                                                             const float* __restrict__ bias,
                                                             int H, int E, int K,
                                                             uint16_t* __restrict__ logits,
                                                             int32_t* __restrict__ idx,
                                                             float* __restrict__ gates) {
  __shared__ uint16_t s_logit[64];
  const int t = blockIdx.x;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int c = H / 64;
  for (int e = wave; e < E; e += 16) {
    float s = 0.0f;
    for (int j = 0; j < c; ++j)
      s = __builtin_fmaf(bf2f(x[(int64_t)t * H + lane * c + j]), bf2f(w[(int64_t)e * H + lane * c + j]), s);
    s = wave_tree_sum64(s);
    if (lane == 63) {
      const uint16_t lb = f2bf(bias ? s + bias[e] : s);
      s_logit[e] = lb;
      if (logits) logits[(int64_t)t * E + e] = lb;
    }
  }
  __syncthreads();
  if (wave != 0) return;
  float g;
  int id;
  if (ROUTE == TFM_ROUTE_OLMOE) {
    uint16_t gb;
    id = olmoe_route_wave(s_logit, E, K, &g, &gb);
  } else {
    id = granite_route_wave(s_logit, E, K, &g);
  }
  if (lane < K) {
    idx[(int64_t)t * K + lane] = id;
    gates[(int64_t)t * K + lane] = g;
  }
}

static int lg_for(int kin) {
  const int nch = kin / 32;
  return nch <= 4 ? 4 : nch <= 8 ? 8 : nch <= 16 ? 16 : nch <= 32 ? 32 : 64;
}

void launch_decode_route(int route_kind, const uint16_t* x, const uint16_t* router, const float* bias,
                         int T, int H, int E, int K, uint16_t* logits, int32_t* idx, float* gates,
                         hipStream_t s) {
  if (T <= 0) return;
  if (E > 64) fail(TFM_E_UNSUPPORTED, "decode routing: more than 64 experts");
#define TFM_DR(CV)                                                                            \
  {                                                                                         \
    if (route_kind == TFM_ROUTE_OLMOE)                                                       \
      decode_route_kernel<CV, TFM_ROUTE_OLMOE><<<T, 1024, 0, s>>>(x, router, bias, H, E, K,   \
                                                                  logits, idx, gates);        \
    else                                                                                    \
      decode_route_kernel<CV, TFM_ROUTE_GRANITE><<<T, 1024, 0, s>>>(x, router, bias, H, E, K, \
                                                                    logits, idx, gates);      \
  }
  switch (H) {
    case 512: TFM_DR(8) break;
    case 1024: TFM_DR(16) break;
    case 1536: TFM_DR(24) break;
    case 2048: TFM_DR(32) break;
    case 3072: TFM_DR(48) break;
    case 4096: TFM_DR(64) break;
    default:
      if (route_kind == TFM_ROUTE_OLMOE)
        decode_route_generic<TFM_ROUTE_OLMOE><<<T, 1024, 0, s>>>(x, router, bias, H, E, K, logits,
                                                                 idx, gates);
      else
        decode_route_generic<TFM_ROUTE_GRANITE><<<T, 1024, 0, s>>>(x, router, bias, H, E, K,
                                                                   logits, idx, gates);
  }
#undef TFM_DR
  check_hip(hipGetLastError(), "decode route launch");
}

void launch_decode_gateup(const uint16_t* x, const int32_t* idx, int T, int E, int K, int H, int I,
                          const tfm_affine& gate, const tfm_affine& up, const Grouping& g,
                          uint16_t* h, uint32_t* status, hipStream_t s) {
  if (T * K > kDecodeMaxRoutes) fail(TFM_E_INVALID, "decode gate/up: more than 256 routes");
  if (H % 64 != 0 || H > 2048) fail(TFM_E_UNSUPPORTED, "decode gate/up: hidden width above 2048");
  DecodeGateUpArgs A{};
  A.x = x; A.idx = idx; A.T = T; A.E = E; A.K = K; A.H = H; A.I = I;
  A.gate = gate; A.up = up; A.order = g.order; A.inverse = g.inverse; A.offsets = g.offsets;
  A.active = g.active; A.h = h; A.status = status;
  const int lg = lg_for(H);
  const int ur = 4 * (64 / lg), upe = (I + ur - 1) / ur;
  const int max_active = T * K < E ? T * K : E;
  const dim3 grid((unsigned)((upe + kGemvUnits - 1) / kGemvUnits), (unsigned)max_active);
  switch (lg) {
    case 4: decode_gateup_kernel<4><<<grid, 256, 0, s>>>(A); break;
    case 8: decode_gateup_kernel<8><<<grid, 256, 0, s>>>(A); break;
    case 16: decode_gateup_kernel<16><<<grid, 256, 0, s>>>(A); break;
    case 32: decode_gateup_kernel<32><<<grid, 256, 0, s>>>(A); break;
    default: decode_gateup_kernel<64><<<grid, 256, 0, s>>>(A); break;
  }
  check_hip(hipGetLastError(), "decode gate/up launch");
}

}  // namespace tfm
