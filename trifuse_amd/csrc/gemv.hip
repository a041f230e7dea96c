// Decode path: fused affine-4bit dequant GEMV over routed experts (no MFMA).
//
// A workgroup owns one routed expert (blockIdx.y indexes the ascending list
// of experts that received routes) and a block of output rows. Each wave
// keeps RW row-loads of packed weights in registers (coalesced 16-byte loads:
// one row of Kin=2048 is exactly 64 lanes x 16 B) and applies them to every
// route of its expert, so each weight byte is read from HBM once per call.
//
// Arithmetic per 32-element chunk (which lies inside one 64-wide group):
//   sum_k x_k (s q_k + b) = s * sum_k x_k (128 + q_k) + (b - 128 s) * sum_k x_k.
// 128 + q is exact in bf16 and is built from a nibble with one byte permute
// (bf16 bits 0x43qq with qq = q), so the products run as v_dot2_f32_bf16 on
// (x_a, x_b) . (128+q_a, 128+q_b) pairs with fp32 accumulation. Row partial sums
// are reduced across lanes with DPP row operations and two lane swizzles.
#include "tfm_device.h"
#include "tfm_internal.h"

namespace tfm {

enum GemvMode { kGateUp = 0, kPlain = 1, kScaled = 2 };

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

// A row of kin inputs is nch = kin/32 chunks of 32 elements. LG lanes share
// one row (chunk c of the row goes to lane c % LG, slot c / LG), so a wave
// covers RPL = 64/LG rows per load instruction and each lane holds CPL chunks.
template <int LG_, int CPL_>
struct GemvShape {
  static constexpr int LG = LG_;
  static constexpr int CPL = CPL_;
  static constexpr int RPL = 64 / LG;
};

__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                         __builtin_bit_cast(bf16x2_t, b), c, false);
}

template <int CTRL>
__device__ __forceinline__ float dpp_add(float v) {
  const int s = __builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false);
  return v + __int_as_float(s);
}

// Sum over aligned groups of G lanes; every lane of a group gets the sum.
template <int G>
__device__ __forceinline__ float lane_group_sum(float v) {
  if (G >= 2) v = dpp_add<0xb1>(v);    // quad_perm [1,0,3,2]
  if (G >= 4) v = dpp_add<0x4e>(v);    // quad_perm [2,3,0,1]
  if (G >= 8) v = dpp_add<0x141>(v);   // row_half_mirror
  if (G >= 16) v = dpp_add<0x140>(v);  // row_mirror
  if (G >= 32) v = v + __shfl_xor(v, 16, 64);
  if (G >= 64) v = v + __shfl_xor(v, 32, 64);
  return v;
}

// One row-chunk of packed weights with its folded scale/offset.
struct ChunkW {
  uint4 q;
  float s;  // scale
  float c;  // bias - 128 * scale
};

// x chunk of one route in the pair order of the unpacked nibbles:
// for each packed word i (elements 8i..8i+7) pairs (0,2) (4,6) (1,3) (5,7).
struct ChunkX {
  uint32_t p[16];
  float sum;
};

__device__ __forceinline__ void load_x(const uint16_t* __restrict__ src, ChunkX& cx) {
  const uint4* p4 = reinterpret_cast<const uint4*>(src);
  const uint32_t ones = 0x3f803f80u;  // (1.0, 1.0) in bf16
  float sum = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint4 v = p4[i];  // (x0,x1) (x2,x3) (x4,x5) (x6,x7) of word i
    cx.p[4 * i + 0] = __builtin_amdgcn_perm(v.y, v.x, 0x05040100u);  // (x0, x2)
    cx.p[4 * i + 1] = __builtin_amdgcn_perm(v.w, v.z, 0x05040100u);  // (x4, x6)
    cx.p[4 * i + 2] = __builtin_amdgcn_perm(v.y, v.x, 0x07060302u);  // (x1, x3)
    cx.p[4 * i + 3] = __builtin_amdgcn_perm(v.w, v.z, 0x07060302u);  // (x5, x7)
    sum = dot2(v.x, ones, sum);
    sum = dot2(v.y, ones, sum);
    sum = dot2(v.z, ones, sum);
    sum = dot2(v.w, ones, sum);
  }
  cx.sum = sum;
}

__device__ __forceinline__ void zero_x(ChunkX& cx) {
#pragma unroll
  for (int i = 0; i < 16; ++i) cx.p[i] = 0u;
  cx.sum = 0.0f;
}

// (128+q) pairs of one packed word: (n0,n2) (n4,n6) (n1,n3) (n5,n7).
// v_perm_b32 picks the nibble bytes of lo/hi and the 0x43 exponent bytes.
__device__ __forceinline__ void unpack_word(uint32_t w, uint32_t* q) {
  const uint32_t magic = 0x43434343u;
  const uint32_t lo = w & 0x0f0f0f0fu, hi = (w >> 4) & 0x0f0f0f0fu;
  q[0] = __builtin_amdgcn_perm(magic, lo, 0x04010400u);
  q[1] = __builtin_amdgcn_perm(magic, lo, 0x04030402u);
  q[2] = __builtin_amdgcn_perm(magic, hi, 0x04010400u);
  q[3] = __builtin_amdgcn_perm(magic, hi, 0x04030402u);
}

__device__ __forceinline__ ChunkW load_chunk(const tfm_affine& m, int64_t row, int kin, int c) {
  ChunkW w;
  w.q = reinterpret_cast<const uint4*>(m.q + row * (kin / 8))[c];
  const int64_t gi = row * (kin / 64) + (c >> 1);
  w.s = bf2f(static_cast<const uint16_t*>(m.scales)[gi]);
  const float b = bf2f(static_cast<const uint16_t*>(m.biases)[gi]);
  w.c = __builtin_fmaf(-128.0f, w.s, b);
  return w;
}

template <int LG, int CPL, int MODE, int RW, int TB>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2, 8)))
void gemv_kernel(const uint16_t* __restrict__ x, RowMap rm, Grouping g, tfm_affine wa,
                 tfm_affine wb, int N, int kin, const float* __restrict__ gates,
                 void* __restrict__ out) {
  using S = GemvShape<LG, CPL>;
  const int nch = kin / 32;
  constexpr int NM = MODE == kGateUp ? 2 : 1;
  const int a = blockIdx.y;
  const int E = g.E;
  if (a >= g.active[E]) return;
  const int e = g.active[a];
  const int j0 = g.offsets[e], j1 = g.offsets[e + 1];
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int sub = lane / S::LG, ll = lane % S::LG;
  const int row0 = (blockIdx.x * 4 + wave) * RW * S::RPL;
  if (row0 >= N) return;

  ChunkW w[NM][RW][S::CPL];
#pragma unroll
  for (int r = 0; r < RW; ++r) {
    const int n = row0 + r * S::RPL + sub;
#pragma unroll
    for (int i = 0; i < S::CPL; ++i) {
      const int c = ll + S::LG * i;
      const bool ok = n < N && c < nch;
#pragma unroll
      for (int m = 0; m < NM; ++m) {
        if (ok) {
          w[m][r][i] = load_chunk(m == 0 ? wa : wb, (int64_t)e * N + n, kin, c);
        } else {
          w[m][r][i].q = make_uint4(0, 0, 0, 0);
          w[m][r][i].s = 0.0f;
          w[m][r][i].c = 0.0f;
        }
      }
    }
  }

  for (int jb = j0; jb < j1; jb += TB) {
    ChunkX cx[TB][S::CPL];
#pragma unroll
    for (int t = 0; t < TB; ++t) {
      const int j = jb + t;
      const int64_t xrow = j < j1 ? (MODE == kScaled ? (int64_t)j : route_row(rm, j)) : -1;
#pragma unroll
      for (int i = 0; i < S::CPL; ++i) {
        const int c = ll + S::LG * i;
        if (xrow >= 0 && c < nch)
          load_x(x + xrow * kin + 32 * c, cx[t][i]);
        else
          zero_x(cx[t][i]);
      }
    }
#pragma unroll
    for (int r = 0; r < RW; ++r) {
      const int n = row0 + r * S::RPL + sub;
      float acc[NM][TB];
#pragma unroll
      for (int m = 0; m < NM; ++m) {
#pragma unroll
        for (int t = 0; t < TB; ++t) acc[m][t] = 0.0f;
#pragma unroll
        for (int i = 0; i < S::CPL; ++i) {
          const ChunkW& cw = w[m][r][i];
          const uint32_t words[4] = {cw.q.x, cw.q.y, cw.q.z, cw.q.w};
          float d[TB];
#pragma unroll
          for (int t = 0; t < TB; ++t) d[t] = 0.0f;
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            uint32_t q[4];
            unpack_word(words[k], q);
#pragma unroll
            for (int t = 0; t < TB; ++t) {
              d[t] = dot2(q[0], cx[t][i].p[4 * k + 0], d[t]);
              d[t] = dot2(q[1], cx[t][i].p[4 * k + 1], d[t]);
              d[t] = dot2(q[2], cx[t][i].p[4 * k + 2], d[t]);
              d[t] = dot2(q[3], cx[t][i].p[4 * k + 3], d[t]);
            }
          }
#pragma unroll
          for (int t = 0; t < TB; ++t) acc[m][t] += __builtin_fmaf(cw.s, d[t], cw.c * cx[t][i].sum);
        }
#pragma unroll
        for (int t = 0; t < TB; ++t) acc[m][t] = lane_group_sum<S::LG>(acc[m][t]);
      }
      if (ll == 0 && n < N) {
#pragma unroll
        for (int t = 0; t < TB; ++t) {
          const int j = jb + t;
          if (j >= j1) continue;
          if (MODE == kGateUp) {
            static_cast<uint16_t*>(out)[(int64_t)j * N + n] = f2bf(silu_mul(acc[0][t], acc[1][t]));
          } else if (MODE == kPlain) {
            static_cast<uint16_t*>(out)[(int64_t)rm.order[j] * N + n] = f2bf(acc[0][t]);
          } else {
            const float gw = gates ? gates[rm.order[j]] : 1.0f;
            static_cast<float*>(out)[(int64_t)j * N + n] = acc[0][t] * gw;
          }
        }
      }
    }
  }
}

template <int LG, int CPL, int MODE, int RW, int TB>
static void launch_gemv_k(const uint16_t* x, RowMap rm, const Grouping& g, int max_active,
                          const tfm_affine& wa, const tfm_affine& wb, int N, int kin,
                          const float* gates, void* out, hipStream_t s) {
  using S = GemvShape<LG, CPL>;
  const int rows_per_block = 4 * RW * S::RPL;
  dim3 grid((unsigned)((N + rows_per_block - 1) / rows_per_block), (unsigned)max_active);
  gemv_kernel<LG, CPL, MODE, RW, TB><<<grid, 256, 0, s>>>(x, rm, g, wa, wb, N, kin, gates, out);
}

template <int LG, int CPL, int MODE, int RW>
static void launch_gemv_tb(bool pair, const uint16_t* x, RowMap rm, const Grouping& g,
                           int max_active, const tfm_affine& wa, const tfm_affine& wb, int N,
                           int kin, const float* gates, void* out, hipStream_t s) {
  if (pair)
    launch_gemv_k<LG, CPL, MODE, RW, 2>(x, rm, g, max_active, wa, wb, N, kin, gates, out, s);
  else
    launch_gemv_k<LG, CPL, MODE, RW, 1>(x, rm, g, max_active, wa, wb, N, kin, gates, out, s);
}

template <int MODE, int RW>
static void dispatch_gemv(int Kin, int64_t routes, const uint16_t* x, RowMap rm, const Grouping& g,
                          int max_active, const tfm_affine& wa, const tfm_affine& wb, int N,
                          const float* gates, void* out, hipStream_t s) {
  if (max_active <= 0 || N <= 0) return;
  if (Kin % 64 != 0 || Kin <= 0) fail(TFM_E_UNSUPPORTED, "affine GEMV: input width must be a multiple of 64");
  const int nch = Kin / 32;
  // Two routes per pass over the unpacked weights once experts see several routes.
  const bool pair = routes > 2 * (int64_t)max_active;
  if (nch <= 4)
    launch_gemv_tb<4, 1, MODE, RW>(pair, x, rm, g, max_active, wa, wb, N, Kin, gates, out, s);
  else if (nch <= 8)
    launch_gemv_tb<8, 1, MODE, RW>(pair, x, rm, g, max_active, wa, wb, N, Kin, gates, out, s);
  else if (nch <= 16)
    launch_gemv_tb<16, 1, MODE, RW>(pair, x, rm, g, max_active, wa, wb, N, Kin, gates, out, s);
  else if (nch <= 32)
    launch_gemv_tb<32, 1, MODE, RW>(pair, x, rm, g, max_active, wa, wb, N, Kin, gates, out, s);
  else if (nch <= 64)
    launch_gemv_tb<64, 1, MODE, RW>(pair, x, rm, g, max_active, wa, wb, N, Kin, gates, out, s);
  else if (nch <= 128)
    launch_gemv_tb<64, 2, MODE, RW>(pair, x, rm, g, max_active, wa, wb, N, Kin, gates, out, s);
  else if (nch <= 256)
    launch_gemv_tb<64, 4, MODE, RW>(pair, x, rm, g, max_active, wa, wb, N, Kin, gates, out, s);
  else
    fail(TFM_E_UNSUPPORTED, "affine GEMV: input width " + std::to_string(Kin) + " above 8192 not built");
  check_hip(hipGetLastError(), "gemv launch");
}

void launch_gemv_gateup(const uint16_t* x, RowMap rm, const Grouping& g, int max_active,
                        int64_t routes, const tfm_affine& gate, const tfm_affine& up, int N,
                        int Kin, uint16_t* h, hipStream_t s) {
  dispatch_gemv<kGateUp, 4>(Kin, routes, x, rm, g, max_active, gate, up, N, nullptr, h, s);
}

void launch_gemv_plain(const uint16_t* x, RowMap rm, const Grouping& g, int max_active,
                       int64_t routes, const tfm_affine& w, int N, int Kin, uint16_t* out,
                       hipStream_t s) {
  dispatch_gemv<kPlain, 4>(Kin, routes, x, rm, g, max_active, w, w, N, nullptr, out, s);
}

void launch_gemv_scaled(const uint16_t* hsorted, const Grouping& g, int max_active,
                        int64_t routes, const tfm_affine& w, int N, int Kin, const float* gates,
                        float* P, hipStream_t s) {
  RowMap rm{g.order, nullptr, 1, 0, nullptr};
  dispatch_gemv<kScaled, 4>(Kin, routes, hsorted, rm, g, max_active, w, w, N, gates, P, s);
}

}  // namespace tfm
