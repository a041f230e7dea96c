// Decode path of the MoE block (few routes: T*K <= 256).
//
// The block that NativeGraniteMoEPrefill::moe runs per layer
// (MLXNativeGraniteMoEPrefill.h:627-702) as five kernels:
//   1. decode_logits_kernel: one workgroup per expert computes that expert's
//      router logit for every token (same arithmetic as the router kernel),
//      then topk_kernel ranks each token's E logits,
//   2. decode_gateup_kernel: every workgroup first groups the T*K routes by
//      expert (stable, in LDS; a few hundred VALU ops) and then streams a few
//      gate/up row units of one active expert through the dequant GEMV with
//      the SwiGLU epilogue; workgroup (0, 0) also publishes the grouping for
//      the next kernels. (With many gate/up workgroups the block instead runs
//      one route-and-group workgroup after the logits and the slot-reading
//      GEMV of gemv.hip: capi.hip, decode_slot_grouping.)
//   3. the down dequant GEMV scaled by each route's gate (gemv.hip),
//   4. the ordered K reduction + residual (combine.hip).
// Each kernel boundary is the only synchronisation: on MI355X a launch costs
// ~2.4 us, while a cross-workgroup hand-off inside a kernel needs an L2
// write-back per workgroup, which costs more at these grid sizes.
#include "gemv_body.h"
#include "tfm_device.h"
#include "tfm_internal.h"

namespace tfm {

constexpr int kDecodeMaxRoutes = 256;  // one thread per route in the grouping

struct DecodeGateUpArgs {
  const uint16_t* x;       // [T, H]
  const int32_t* idx;      // [R] route -> expert (from decode_route_kernel)
  const float* gates;      // [R] route gates (fp32, flat order)
  int T, E, K, H, I;
  tfm_affine gate, up;
  int32_t* order;          // [R] sorted position -> flat route
  int32_t* inverse;        // [R]
  int32_t* offsets;        // [E+1]
  int32_t* active;         // [E+1]
  int4* slots;             // [E] per active slot {expert, first route, end route, 0}
  float* gates_sorted;     // [R] gates in sorted order
  uint16_t* h;             // [R, I] SwiGLU output, expert-sorted rows
  uint32_t* status;        // status word (no bits: routes come from the router)
};

__device__ __forceinline__ uint64_t lanemask_lt64() {
  const int lane = threadIdx.x & 63;
  return lane == 0 ? 0ull : (~0ull >> (64 - lane));
}

template <int LG, bool F16>
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
  const float gate = (live && blockIdx.x == 0 && blockIdx.y == 0) ? A.gates[tid] : 0.0f;
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
      A.gates_sorted[pos] = gate;
    }
    if (tid <= E) {
      A.offsets[tid] = s_off[tid];
      if (tid == E || tid < s_act[E]) A.active[tid] = s_act[tid];
    }
    if (tid < E) {
      const int ex = tid < s_act[E] ? s_act[tid] : -1;
      A.slots[tid] = ex < 0 ? make_int4(-1, 0, 0, 0) : make_int4(ex, s_off[ex], s_off[ex + 1], 0);
    }
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
    h[(int64_t)j * N + n] = f2st<F16>(hv);
  };
  gemv_units<LG, 2, kGemvUnits, F16>(L, A.x, A.H, N, A.gate, A.up, ex, s_off[ex], s_off[ex + 1],
                                blockIdx.x * kGemvUnits, xrow, stage, emit);
}

// Router logits of the decode path, one workgroup (4 waves) per expert e:
// logit[t][e] for every token t, each computed exactly as the router kernel
// does (lane l sums x*w over its H/64 contiguous elements with sequential
// fused multiply-adds, then the xor-shuffle tree across lanes, then + bias,
// rounded to bf16). One router row per workgroup spreads the router read
// over E compute units (a single compute unit pulling the whole router is
// limited by its own outstanding misses). Wave w takes tokens w, w + 4, ..,
// two at a time.
//
// BITS = 0: w is the dense router [E, H] in the storage dtype. BITS = 4 or 8:
// the router is affine-quantised (aq: codes [E, H*BITS/32] LSB first, scales
// and biases [E, H/64] in the storage dtype) and each lane dequantises its own
// H/64 elements in place, w = st(s*q + b) as the router dequant pass
// computes it, so one kernel replaces that pass and its boundary.
template <int C, bool F16, int BITS = 0>
__global__ __launch_bounds__(256) void decode_logits_kernel(const uint16_t* __restrict__ x,
                                                            const uint16_t* __restrict__ w,
                                                            tfm_affine aq,
                                                            const float* __restrict__ bias, int T,
                                                            int H, int E,
                                                            uint16_t* __restrict__ logits) {
  const int e = blockIdx.x;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  float wv[C];
  if constexpr (BITS == 0) {
    const uint4* ws = reinterpret_cast<const uint4*>(w + (int64_t)e * H + lane * C);
#pragma unroll
    for (int i = 0; i < C / 8; ++i) {
      const uint4 v = ws[i];
      wv[8 * i + 0] = lo_st<F16>(v.x); wv[8 * i + 1] = hi_st<F16>(v.x);
      wv[8 * i + 2] = lo_st<F16>(v.y); wv[8 * i + 3] = hi_st<F16>(v.y);
      wv[8 * i + 4] = lo_st<F16>(v.z); wv[8 * i + 5] = hi_st<F16>(v.z);
      wv[8 * i + 6] = lo_st<F16>(v.w); wv[8 * i + 7] = hi_st<F16>(v.w);
    }
  } else {
    constexpr int PER = 32 / BITS;                  // codes per word
    constexpr uint32_t MASK = (1u << BITS) - 1u;
    static_assert(C % PER == 0, "a lane's elements are whole words");
    const int64_t k0 = (int64_t)e * H + lane * C;    // first element of this lane
    const uint32_t* qr = static_cast<const uint32_t*>(aq.q) + k0 / PER;
    uint32_t wd[C / PER];
#pragma unroll
    for (int i = 0; i < C / PER; ++i) wd[i] = qr[i];
    // Rows are whole 64-element groups; a lane's elements span at most two.
    const int64_t g0 = k0 / 64, g1 = (k0 + C - 1) / 64;
    const uint16_t* sc = static_cast<const uint16_t*>(aq.scales);
    const uint16_t* bi = static_cast<const uint16_t*>(aq.biases);
    const float s0 = st2f<F16>(sc[g0]), b0 = st2f<F16>(bi[g0]);
    const float s1 = st2f<F16>(sc[g1]), b1 = st2f<F16>(bi[g1]);
    const int split = (int)((g0 + 1) * 64 - k0);     // elements j >= split are in group g1
#pragma unroll
    for (int j = 0; j < C; ++j) {
      const float code = (float)((wd[j / PER] >> (BITS * (j % PER))) & MASK);
      const bool second = j >= split;
      wv[j] = st2f<F16>(f2st<F16>(__builtin_fmaf(second ? s1 : s0, code, second ? b1 : b0)));
    }
  }
  const float be = bias ? bias[e] : 0.0f;
  // Token rows past T read zeros (offset beyond the buffer).
  const __amdgpu_buffer_rsrc_t rx = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(x), (short)0, (int)((uint32_t)T * H * 2), 0x00020000);
  for (int t0 = wave; t0 < T; t0 += 8) {
    uint4 xv[2][C / 8];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int t = t0 + 4 * u;
      const uint32_t off = t < T ? ((uint32_t)t * H + lane * C) * 2u : 0x80000000u;
#pragma unroll
      for (int i = 0; i < C / 8; ++i)
        xv[u][i] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rx, off + 16u * i, 0, 0));
    }
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int t = t0 + 4 * u;
      if (t < T) {  // wave-uniform
        float s = 0.0f;
#pragma unroll
        for (int i = 0; i < C / 8; ++i) {
          const uint4 v = xv[u][i];
          s = __builtin_fmaf(lo_st<F16>(v.x), wv[8 * i + 0], s);
          s = __builtin_fmaf(hi_st<F16>(v.x), wv[8 * i + 1], s);
          s = __builtin_fmaf(lo_st<F16>(v.y), wv[8 * i + 2], s);
          s = __builtin_fmaf(hi_st<F16>(v.y), wv[8 * i + 3], s);
          s = __builtin_fmaf(lo_st<F16>(v.z), wv[8 * i + 4], s);
          s = __builtin_fmaf(hi_st<F16>(v.z), wv[8 * i + 5], s);
          s = __builtin_fmaf(lo_st<F16>(v.w), wv[8 * i + 6], s);
          s = __builtin_fmaf(hi_st<F16>(v.w), wv[8 * i + 7], s);
        }
        s = wave_tree_sum64(s);
        if (lane == 63) logits[(int64_t)t * E + e] = f2st<F16>(bias ? s + be : s);
      }
    }
  }
}

// Any H % 64 == 0: the same arithmetic as decode_logits_kernel with scalar loads.
template <bool F16>
__global__ __launch_bounds__(256) void decode_logits_generic(const uint16_t* __restrict__ x,
                                                             const uint16_t* __restrict__ w,
                                                             const float* __restrict__ bias, int T,
                                                             int H, int E,
                                                             uint16_t* __restrict__ logits) {
  const int e = blockIdx.x;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int c = H / 64;
  for (int t = wave; t < T; t += 4) {
    float s = 0.0f;
    for (int j = 0; j < c; ++j)
      s = __builtin_fmaf(st2f<F16>(x[(int64_t)t * H + lane * c + j]), st2f<F16>(w[(int64_t)e * H + lane * c + j]), s);
    s = wave_tree_sum64(s);
    if (lane == 63) logits[(int64_t)t * E + e] = f2st<F16>(bias ? s + bias[e] : s);
  }
}

static int lg_for(int kin) {
  const int nch = kin / 32;
  return nch <= 4 ? 4 : nch <= 8 ? 8 : nch <= 16 ? 16 : nch <= 32 ? 32 : 64;
}

template <bool F16>
static void decode_logits_dt(const uint16_t* x, const uint16_t* router, const float* bias, int T, int H,
                             int E, uint16_t* logits, hipStream_t s) {
  const tfm_affine none{};
  switch (H) {
    case 512: tfm_launch(decode_logits_kernel<8, F16>, E, 256, 0, s, x, router, none, bias, T, H, E, logits); break;
    case 1024: tfm_launch(decode_logits_kernel<16, F16>, E, 256, 0, s, x, router, none, bias, T, H, E, logits); break;
    case 1536: tfm_launch(decode_logits_kernel<24, F16>, E, 256, 0, s, x, router, none, bias, T, H, E, logits); break;
    case 2048: tfm_launch(decode_logits_kernel<32, F16>, E, 256, 0, s, x, router, none, bias, T, H, E, logits); break;
    default: tfm_launch(decode_logits_generic<F16>, E, 256, 0, s, x, router, bias, T, H, E, logits); break;
  }
}

template <bool F16, int BITS>
static bool decode_logits_affine_dt(const uint16_t* x, const tfm_affine& r, const float* bias, int T, int H,
                                    int E, uint16_t* logits, hipStream_t s) {
  switch (H) {
    case 512: tfm_launch(decode_logits_kernel<8, F16, BITS>, E, 256, 0, s, x, nullptr, r, bias, T, H, E, logits); break;
    case 1024: tfm_launch(decode_logits_kernel<16, F16, BITS>, E, 256, 0, s, x, nullptr, r, bias, T, H, E, logits); break;
    case 1536: tfm_launch(decode_logits_kernel<24, F16, BITS>, E, 256, 0, s, x, nullptr, r, bias, T, H, E, logits); break;
    case 2048: tfm_launch(decode_logits_kernel<32, F16, BITS>, E, 256, 0, s, x, nullptr, r, bias, T, H, E, logits); break;
    default: return false;
  }
  return true;
}

bool launch_decode_logits_affine(bool f16, int bits, const uint16_t* x, const tfm_affine& router, const float* bias,
                                 int T, int H, int E, uint16_t* logits, hipStream_t s) {
  if (T <= 0) return true;
  if (E > 64) fail(TFM_E_UNSUPPORTED, "decode routing: more than 64 experts");
  if (!logits) fail(TFM_E_INVALID, "decode routing: logits buffer missing");
  bool ok;
  if (f16)
    ok = bits == 8 ? decode_logits_affine_dt<true, 8>(x, router, bias, T, H, E, logits, s)
                   : decode_logits_affine_dt<true, 4>(x, router, bias, T, H, E, logits, s);
  else
    ok = bits == 8 ? decode_logits_affine_dt<false, 8>(x, router, bias, T, H, E, logits, s)
                   : decode_logits_affine_dt<false, 4>(x, router, bias, T, H, E, logits, s);
  if (ok) check_hip(hipGetLastError(), "decode logits launch");
  return ok;
}

void launch_decode_logits(bool f16, const uint16_t* x, const uint16_t* router, const float* bias, int T,
                          int H, int E, uint16_t* logits, hipStream_t s) {
  if (T <= 0) return;
  if (E > 64) fail(TFM_E_UNSUPPORTED, "decode routing: more than 64 experts");
  if (!logits) fail(TFM_E_INVALID, "decode routing: logits buffer missing");
  if (f16)
    decode_logits_dt<true>(x, router, bias, T, H, E, logits, s);
  else
    decode_logits_dt<false>(x, router, bias, T, H, E, logits, s);
  check_hip(hipGetLastError(), "decode logits launch");
}

int decode_gateup_workgroups(int T, int K, int E, int H, int I) {
  const int lg = lg_for(H);
  const int ur = 4 * (64 / lg), upe = (I + ur - 1) / ur;
  const int max_active = T * K < E ? T * K : E;
  return ((upe + kGemvUnits - 1) / kGemvUnits) * max_active;
}

void launch_decode_gateup(bool f16, const uint16_t* x, const int32_t* idx, const float* gates, int T, int E,
                          int K, int H, int I, const tfm_affine& gate, const tfm_affine& up,
                          const Grouping& g, uint16_t* h, uint32_t* status, hipStream_t s) {
  if (!g.slots || !g.gates_sorted) fail(TFM_E_INVALID, "decode gate/up: slot table missing");
  if (T * K > kDecodeMaxRoutes) fail(TFM_E_INVALID, "decode gate/up: more than 256 routes");
  if (H % 64 != 0 || H > 2048) fail(TFM_E_UNSUPPORTED, "decode gate/up: hidden width above 2048");
  DecodeGateUpArgs A{};
  A.x = x; A.idx = idx; A.gates = gates; A.T = T; A.E = E; A.K = K; A.H = H; A.I = I;
  A.slots = g.slots; A.gates_sorted = g.gates_sorted;
  A.gate = gate; A.up = up; A.order = g.order; A.inverse = g.inverse; A.offsets = g.offsets;
  A.active = g.active; A.h = h; A.status = status;
  const int lg = lg_for(H);
  const int ur = 4 * (64 / lg), upe = (I + ur - 1) / ur;
  const int max_active = T * K < E ? T * K : E;
  const dim3 grid((unsigned)((upe + kGemvUnits - 1) / kGemvUnits), (unsigned)max_active);
#define TFM_DECODE_GU(LGV)                                                  \
  {                                                                         \
    if (f16)                                                                \
      tfm_launch(decode_gateup_kernel<LGV, true>, grid, 256, 0, s, A);      \
    else                                                                    \
      tfm_launch(decode_gateup_kernel<LGV, false>, grid, 256, 0, s, A);     \
  }
  switch (lg) {
    case 4: TFM_DECODE_GU(4) break;
    case 8: TFM_DECODE_GU(8) break;
    case 16: TFM_DECODE_GU(16) break;
    case 32: TFM_DECODE_GU(32) break;
    default: TFM_DECODE_GU(64) break;
  }
#undef TFM_DECODE_GU
  check_hip(hipGetLastError(), "decode gate/up launch");
}

}  // namespace tfm
